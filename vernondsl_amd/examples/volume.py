# Heat diffusion in a 3-D volume: a 3-D field iterated by a 3-D struct-for with a clamped
# seven-point stencil, ping-ponged between two fields; the shown image is the middle slice.
# Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/volume.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

A, B, C = 96, 96, 96
u = ti.field(dtype=float, shape=(A, B, C))
v = ti.field(dtype=float, shape=(A, B, C))


@ti.kernel
def init():
    for i, j, k in u:
        d2 = (i - A * 0.5) ** 2 + (j - B * 0.4) ** 2 + (k - C * 0.5) ** 2
        u[i, j, k] = 1.0 if d2 < 100.0 else 0.0


@ti.kernel
def diffuse(c: float):
    for i, j, k in v:
        s = (u[ti.max(i - 1, 0), j, k] + u[ti.min(i + 1, A - 1), j, k] + u[i, ti.max(j - 1, 0), k]
             + u[i, ti.min(j + 1, B - 1), k] + u[i, j, ti.max(k - 1, 0)] + u[i, j, ti.min(k + 1, C - 1)])
        v[i, j, k] = u[i, j, k] + c * (s - 6.0 * u[i, j, k])


@ti.kernel
def swap():
    for i, j, k in u:
        u[i, j, k] = v[i, j, k]


gui = ti.GUI("volume", res=(A, B))
init()
while gui.running:
    for _ in range(5):
        diffuse(0.15)
        swap()
    gui.set_image(u.to_numpy()[:, :, C // 2])
    gui.show()
