# Escape-time histogram: each pixel runs its escape loop, stores its count and adds one to the
# histogram bin of that count (a scatter-add into a 1-D int field of another shape, Taichi's
# atomic add) and its count to a 0-D total (`total[None] += k`).  The histogram then colours
# the image by the share of pixels that escaped no later (histogram equalisation).  Written
# against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/histogram.py --frames 2
import taichi as ti

ti.init(arch=ti.gpu)

W, H, MAX = 640, 480, 200
counts = ti.field(dtype=int, shape=(W, H))
hist = ti.field(dtype=int, shape=MAX + 1)
cdf = ti.field(dtype=float, shape=MAX + 1)
total = ti.field(dtype=int, shape=())
img = ti.field(dtype=float, shape=(W, H))


@ti.kernel
def escape(cx: float, cy: float, scale: float):
    for i, j in counts:
        x0 = cx + (i - W / 2) * scale
        y0 = cy + (j - H / 2) * scale
        x, y = 0.0, 0.0
        k = 0
        while x * x + y * y <= 4.0 and k < MAX:
            x, y = x * x - y * y + x0, 2.0 * x * y + y0
            k += 1
        counts[i, j] = k
        hist[k] += 1
        total[None] += k


@ti.kernel
def clear():
    for b in hist:
        hist[b] = 0


@ti.kernel
def shade():
    for i, j in img:
        img[i, j] = cdf[counts[i, j]]


gui = ti.GUI("histogram", res=(W, H))
frame = 0
while gui.running:
    clear()
    total[None] = 0
    escape(-0.745, 0.11 + 0.002 * frame, 0.004 / (1.0 + frame))
    h = hist.to_numpy()
    cdf.from_numpy((h.cumsum() / max(h.sum(), 1)).astype("float32"))
    shade()
    gui.set_image(img)
    gui.show()
    frame += 1
