# Two-source wave interference over a plate: a plain per-pixel expression with transcendentals
# and a second field read at each pixel (a damping mask), no loop.  Written against Taichi's API;
# run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/interference.py --frames 3
import taichi as ti

ti.init(arch=ti.gpu)

N = 768
plate = ti.field(dtype=float, shape=(N, N))
mask = ti.field(dtype=float, shape=(N, N))


@ti.kernel
def waves(phase: float):
    for r, s in plate:
        d1 = ti.sqrt((r - 200.0) ** 2 + (s - 300.0) ** 2)
        d2 = ti.sqrt((r - 560.0) ** 2 + (s - 420.0) ** 2)
        amp = ti.sin(d1 * 0.08 - phase) + ti.sin(d2 * 0.08 - phase)
        plate[r, s] = 0.5 + 0.25 * amp * mask[r, s]


@ti.kernel
def make_mask():
    for r, s in mask:
        mask[r, s] = ti.exp(-((r - 384.0) ** 2 + (s - 384.0) ** 2) * 0.00001)


gui = ti.GUI("interference", res=(N, N))
make_mask()
phase = 0.0
while gui.running:
    waves(phase)
    gui.set_image(plate)
    gui.show()
    phase += 0.5
