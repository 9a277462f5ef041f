# The "Burning Ship" escape-time fractal: like Mandelbrot, but the real and imaginary parts are
# folded to their absolute values before each squaring, so the update is not a complex
# polynomial and does not have the escape-time op's form; the kernel body is lowered to a
# per-pixel program compiled for it at run time.  Written against Taichi's API; run headless on
# the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/burning_ship.py --frames 1
import taichi as ti

ti.init(arch=ti.gpu)

W, H = 1024, 1024
LIMIT = 256
hits = ti.field(dtype=ti.i32, shape=(W, H))


@ti.kernel
def ship(zoom: float):
    for px, py in hits:
        cx = (px / W - 0.5) * zoom - 0.45
        cy = (py / H - 0.5) * zoom - 0.5
        x = 0.0
        y = 0.0
        n = 0
        while x * x + y * y <= 4.0 and n < LIMIT:
            ax = abs(x)
            ay = abs(y)
            x, y = ax * ax - ay * ay + cx, 2.0 * ax * ay + cy
            n += 1
        hits[px, py] = n


gui = ti.GUI("burning ship", res=(W, H))
while gui.running:
    ship(3.2)
    gui.set_image(hits)
    gui.show()
