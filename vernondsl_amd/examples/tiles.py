# Tiles and rings: a per-pixel pattern made of conditionals (if/else, a conditional expression,
# ti.select, `and` / `or`, % and //), and a second field that keeps a fading trail of the first,
# updated in place where a condition holds.  Written against Taichi's API; run headless on the
# HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/tiles.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

N = 640
canvas = ti.field(dtype=float, shape=(N, N))
trail = ti.field(dtype=float, shape=(N, N))


@ti.kernel
def paint(t: float):
    for r, c in canvas:
        cell = (r // 40 + c // 40) % 2
        dr = r - N / 2
        dc = c - N / 2
        ring = ti.sqrt(dr * dr + dc * dc) % 64.0
        shade = 0.2 if cell == 0 else 0.8
        if ring < 8.0 + 4.0 * ti.sin(t):
            shade = 1.0 - shade
        canvas[r, c] = ti.select(abs(dr) < 3 or abs(dc) < 3, 0.5, shade)


@ti.kernel
def fade():
    for r, c in trail:
        if canvas[r, c] > trail[r, c]:
            trail[r, c] = canvas[r, c]
        else:
            trail[r, c] = trail[r, c] * 0.9


gui = ti.GUI("tiles", res=(N, N))
t = 0.0
while gui.running:
    paint(t)
    fade()
    gui.set_image(trail)
    gui.show()
    t += 0.25
