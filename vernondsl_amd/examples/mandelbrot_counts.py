# Escape-time counts of the Mandelbrot set over re in [-2, 1), im in [-1.5, 1.5), written
# against Taichi's API; run on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/mandelbrot_counts.py --frames 1
import taichi as ti

ti.init(arch=ti.gpu)

N = 1024
counts = ti.field(dtype=ti.i32, shape=(N, N))


@ti.func
def csquare(w):
    return ti.Vector([w[0] * w[0] - w[1] * w[1], w[0] * w[1] * 2])


@ti.kernel
def render(limit: int):
    for x, y in counts:
        z = ti.Vector([0.0, 0.0])
        c = ti.Vector([x / N * 3 - 2, y / N * 3 - 1.5])
        k = 0
        while k < limit and z.norm_sqr() <= 4:
            z = csquare(z) + c
            k += 1
        counts[x, y] = k


view = ti.GUI("Mandelbrot counts", res=(N, N))
while view.running:
    render(256)
    view.set_image(counts)
    view.show()
