# Particles and a grid, the transfer steps of a particle-in-cell solver: each particle splats
# its mass and momentum onto the 3 x 3 grid nodes around it with quadratic B-spline weights
# (scatter-adds at vector indices base + offset, Taichi's atomic adds), the grid turns momentum
# into velocity and applies gravity and the walls, and each particle gathers its new velocity
# back from the same nodes.  Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/splat.py --frames 3
import taichi as ti

ti.init(arch=ti.gpu)

N, G = 8192, 128
inv_dx = float(G)
dt, gravity = 2e-4, 9.8
x = ti.Vector.field(2, dtype=float, shape=N)
v = ti.Vector.field(2, dtype=float, shape=N)
grid_m = ti.field(dtype=float, shape=(G, G))
grid_v = ti.Vector.field(2, dtype=float, shape=(G, G))


@ti.kernel
def seed():
    for p in x:
        x[p] = [0.3 + (p * 37 % 1009) / 1009.0 * 0.4, 0.3 + (p * 59 % 997) / 997.0 * 0.4]
        v[p] = [((p * 13 % 17) - 8) * 0.05, -1.0]


@ti.kernel
def clear():
    for i, j in grid_m:
        grid_m[i, j] = 0.0
        grid_v[i, j] = [0.0, 0.0]


@ti.kernel
def p2g():
    for p in x:
        base = (x[p] * inv_dx - 0.5).cast(int)
        fx = x[p] * inv_dx - base.cast(float)
        w = [0.5 * (1.5 - fx) ** 2, 0.75 - (fx - 1.0) ** 2, 0.5 * (fx - 0.5) ** 2]
        for i, j in ti.static(ti.ndrange(3, 3)):
            weight = w[i][0] * w[j][1]
            grid_m[base + ti.Vector([i, j])] += weight
            grid_v[base + ti.Vector([i, j])] += weight * v[p]


@ti.kernel
def grid_update():
    for i, j in grid_m:
        m = grid_m[i, j]
        if m > 0.0:
            vel = grid_v[i, j] / m
            vel[1] -= dt * gravity
            if (i < 3 and vel[0] < 0.0) or (i > G - 3 and vel[0] > 0.0):
                vel[0] = 0.0
            if (j < 3 and vel[1] < 0.0) or (j > G - 3 and vel[1] > 0.0):
                vel[1] = 0.0
            grid_v[i, j] = vel


@ti.kernel
def g2p():
    for p in x:
        base = (x[p] * inv_dx - 0.5).cast(int)
        fx = x[p] * inv_dx - base.cast(float)
        w = [0.5 * (1.5 - fx) ** 2, 0.75 - (fx - 1.0) ** 2, 0.5 * (fx - 0.5) ** 2]
        new_v = ti.Vector([0.0, 0.0])
        for i, j in ti.static(ti.ndrange(3, 3)):
            new_v += w[i][0] * w[j][1] * grid_v[base + ti.Vector([i, j])]
        v[p] = new_v
        x[p] = x[p] + dt * new_v


gui = ti.GUI("splat", res=(512, 512))
seed()
while gui.running:
    for _ in range(4):
        clear()
        p2g()
        grid_update()
        g2p()
    gui.circles(x.to_numpy(), radius=1.5)
    gui.show()
