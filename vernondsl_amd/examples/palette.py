# An escape-time image of z -> z^3 + c in colour: a field of RGB vectors (ti.Vector.field) filled
# from a cosine palette of the escape count, then a second kernel that reads that field (vector
# reads, component access) and writes a vignetted copy into another.  Written against Taichi's
# API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/palette.py --frames 2
import taichi as ti

ti.init(arch=ti.gpu)

W, H = 800, 600
LIMIT = 120
rgb = ti.Vector.field(3, dtype=float, shape=(W, H))
shaded = ti.Vector.field(3, dtype=float, shape=(W, H))


@ti.func
def palette(t):
    return ti.Vector([0.5 + 0.5 * ti.cos(6.2831 * t),
                      0.5 + 0.5 * ti.cos(6.2831 * (t + 0.33)),
                      0.5 + 0.5 * ti.cos(6.2831 * (t + 0.67))])


@ti.kernel
def render(shift: float):
    for x, y in rgb:
        c = ti.Vector([x / W * 3.0 - 1.5, y / H * 2.4 - 1.2])
        z = ti.Vector([0.0, 0.0])
        n = 0
        while z.dot(z) < 16.0 and n < LIMIT:
            re2 = z[0] * z[0] - z[1] * z[1]
            im2 = 2.0 * z[0] * z[1]
            z = ti.Vector([z[0] * re2 - z[1] * im2, z[0] * im2 + z[1] * re2]) + c
            n += 1
        if n == LIMIT:
            rgb[x, y] = ti.Vector([0.0, 0.0, 0.0])
        else:
            rgb[x, y] = palette(n / LIMIT + shift)


@ti.kernel
def vignette():
    for x, y in shaded:
        d = ti.Vector([x / W - 0.5, y / H - 0.5])
        k = 1.0 - 1.2 * d.dot(d)
        px = rgb[x, y]
        shaded[x, y] = ti.Vector([px.x * k, px[1] * k, ti.min(px.z * k + 0.05, 1.0)])


gui = ti.GUI("palette", res=(W, H))
shift = 0.0
while gui.running:
    render(shift)
    vignette()
    gui.set_image(shaded)
    gui.show()
    shift += 0.05
