# Particles falling in a box: 1-D fields of 2-vectors (positions and velocities) iterated by
# 1-D struct-fors, a body storing both fields (one program per stored field), bounces written as
# conditional component assignments on local vectors, and an augmented store (age[i] += dt).
# Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/particles.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

N = 16384
x = ti.Vector.field(2, dtype=float, shape=N)
v = ti.Vector.field(2, dtype=float, shape=N)
age = ti.field(dtype=float, shape=N)
gravity, dt, damping = -9.8, 0.002, 0.8


@ti.kernel
def seed():
    for i in range(N):
        x[i] = [(i * 37 % 1009) / 1009.0, 0.5 + (i * 59 % 997) / 1994.0]
        v[i] = [((i * 13 % 17) - 8) * 0.25, 0.0]


@ti.kernel
def step():
    for i in x:
        vel = v[i]
        vel[1] += gravity * dt
        pos = x[i] + vel * dt
        if pos[1] < 0.0:
            pos[1] = -pos[1]
            vel[1] = -vel[1] * damping
        if pos[0] < 0.0 or pos[0] > 1.0:
            pos[0] = ti.min(ti.max(pos[0], 0.0), 1.0)
            vel[0] = -vel[0] * damping
        x[i] = pos
        v[i] = vel
    for i in age:
        age[i] += dt


gui = ti.GUI("particles", res=(512, 512))
seed()
while gui.running:
    for _ in range(10):
        step()
    gui.circles(x.to_numpy(), radius=1.5)
    gui.show()
