# Gray-Scott reaction-diffusion on a torus: two chemicals u and v, each struct-for storing both
# (one program per stored field), and a step kernel of two struct-fors run one after the other
# (the update into nu, nv, then the copy back).  Written against Taichi's API; run headless on the
# HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/reaction.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

N = 256
u = ti.field(dtype=float, shape=(N, N))
v = ti.field(dtype=float, shape=(N, N))
nu = ti.field(dtype=float, shape=(N, N))
nv = ti.field(dtype=float, shape=(N, N))
Du, Dv, feed, kill = 0.16, 0.08, 0.035, 0.065


@ti.kernel
def seed():
    for i, j in u:
        inside = abs(i - N // 2) < 12 and abs(j - N // 2) < 12
        u[i, j] = 0.5 if inside else 1.0
        v[i, j] = 0.25 + 0.01 * ((i * 7 + j * 3) % 5) if inside else 0.0


@ti.kernel
def step(dt: float):
    for i, j in nu:
        a = u[i, j]
        b = v[i, j]
        lu = (u[(i + 1) % N, j] + u[(i + N - 1) % N, j] + u[i, (j + 1) % N] + u[i, (j + N - 1) % N]) - 4.0 * a
        lv = (v[(i + 1) % N, j] + v[(i + N - 1) % N, j] + v[i, (j + 1) % N] + v[i, (j + N - 1) % N]) - 4.0 * b
        r = a * b * b
        nu[i, j] = a + dt * (Du * lu - r + feed * (1.0 - a))
        nv[i, j] = b + dt * (Dv * lv + r - (feed + kill) * b)
    for i, j in u:
        u[i, j] = nu[i, j]
        v[i, j] = nv[i, j]


gui = ti.GUI("reaction", res=(N, N))
seed()
while gui.running:
    for _ in range(8):
        step(1.0)
    gui.set_image(v)
    gui.show()
