# A 2-D material-point (MLS-MPM) fluid of 8192 particles on a 128 x 128 grid, the shape of
# Taichi's classic 88-line demo: each substep clears the grid, splats every particle's mass and
# its momentum plus the affine velocity field (a 2 x 2 matrix per particle, and a pressure
# term from its volume ratio J) onto 3 x 3 nodes (scatter-adds), turns node momentum into
# velocity with gravity and walls, and gathers velocity and the affine field back (outer
# products).  Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/mpm88.py --frames 3
import taichi as ti

ti.init(arch=ti.gpu)

n_particles, n_grid = 8192, 128
dx = 1.0 / n_grid
dt = 2e-4
p_rho = 1.0
p_vol = (dx * 0.5) ** 2
p_mass = p_vol * p_rho
gravity = 9.8
bound = 3
E = 400.0

x = ti.Vector.field(2, dtype=float, shape=n_particles)
v = ti.Vector.field(2, dtype=float, shape=n_particles)
C = ti.Matrix.field(2, 2, dtype=float, shape=n_particles)
J = ti.field(dtype=float, shape=n_particles)
grid_v = ti.Vector.field(2, dtype=float, shape=(n_grid, n_grid))
grid_m = ti.field(dtype=float, shape=(n_grid, n_grid))


@ti.kernel
def substep():
    for i, j in grid_m:
        grid_v[i, j] = [0.0, 0.0]
        grid_m[i, j] = 0.0
    for p in x:
        Xp = x[p] / dx
        base = int(Xp - 0.5)
        fx = Xp - base
        w = [0.5 * (1.5 - fx) ** 2, 0.75 - (fx - 1.0) ** 2, 0.5 * (fx - 0.5) ** 2]
        stress = -dt * 4.0 * E * p_vol * (J[p] - 1.0) / dx ** 2
        affine = ti.Matrix([[stress, 0.0], [0.0, stress]]) + p_mass * C[p]
        for i, j in ti.static(ti.ndrange(3, 3)):
            offset = ti.Vector([i, j])
            dpos = (offset - fx) * dx
            weight = w[i].x * w[j].y
            grid_v[base + offset] += weight * (p_mass * v[p] + affine @ dpos)
            grid_m[base + offset] += weight * p_mass
    for i, j in grid_m:
        if grid_m[i, j] > 0.0:
            grid_v[i, j] /= grid_m[i, j]
        grid_v[i, j].y -= dt * gravity
        if i < bound and grid_v[i, j].x < 0.0:
            grid_v[i, j].x = 0.0
        if i > n_grid - bound and grid_v[i, j].x > 0.0:
            grid_v[i, j].x = 0.0
        if j < bound and grid_v[i, j].y < 0.0:
            grid_v[i, j].y = 0.0
        if j > n_grid - bound and grid_v[i, j].y > 0.0:
            grid_v[i, j].y = 0.0
    for p in x:
        Xp = x[p] / dx
        base = int(Xp - 0.5)
        fx = Xp - base
        w = [0.5 * (1.5 - fx) ** 2, 0.75 - (fx - 1.0) ** 2, 0.5 * (fx - 0.5) ** 2]
        new_v = ti.Vector.zero(float, 2)
        new_C = ti.Matrix.zero(float, 2, 2)
        for i, j in ti.static(ti.ndrange(3, 3)):
            offset = ti.Vector([i, j])
            dpos = (offset - fx) * dx
            weight = w[i].x * w[j].y
            g_v = grid_v[base + offset]
            new_v += weight * g_v
            new_C += 4.0 * weight * g_v.outer_product(dpos) / dx ** 2
        v[p] = new_v
        x[p] += dt * v[p]
        J[p] *= 1.0 + dt * new_C.trace()
        C[p] = new_C


@ti.kernel
def init():
    for p in x:
        x[p] = [(p * 37 % 1009) / 1009.0 * 0.4 + 0.2, (p * 59 % 997) / 997.0 * 0.4 + 0.2]
        v[p] = [0.0, -1.0]
        J[p] = 1.0


gui = ti.GUI("mpm88", res=(512, 512))
init()
while gui.running:
    for _ in range(50):
        substep()
    gui.circles(x.to_numpy(), radius=1.5)
    gui.show()
