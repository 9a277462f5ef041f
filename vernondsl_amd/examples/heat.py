# Explicit heat diffusion on a plate with a hot spot: a five-point stencil whose indices are
# clamped at the border with ti.max / ti.min (an insulated edge), ping-ponged between two fields.
# Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/heat.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

W, H = 384, 256
u = ti.field(dtype=float, shape=(W, H))
v = ti.field(dtype=float, shape=(W, H))


@ti.kernel
def init():
    for x, y in u:
        d2 = (x - W * 0.3) ** 2 + (y - H * 0.6) ** 2
        u[x, y] = 1.0 if d2 < 400.0 else 0.0


@ti.kernel
def diffuse(k: float):
    for x, y in v:
        c = u[x, y]
        lap = (u[ti.max(x - 1, 0), y] + u[ti.min(x + 1, W - 1), y] + u[x, ti.max(y - 1, 0)]
               + u[x, ti.min(y + 1, H - 1)] - 4.0 * c)
        v[x, y] = c + k * lap


@ti.kernel
def swap():
    for x, y in u:
        u[x, y] = v[x, y]


gui = ti.GUI("heat", res=(W, H))
init()
while gui.running:
    for _ in range(10):
        diffuse(0.2)
        swap()
    gui.set_image(u)
    gui.show()
