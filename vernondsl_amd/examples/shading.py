# Shading with taichi.math over ti.ndrange: vec2/vec3 constructors, normalize, dot, cross, clamp,
# mix, smoothstep, fract, step and sign, a ti.static loop over the colour channels that sets
# components of a local vector, and a mask field read per pixel.  Written against Taichi's API;
# run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/shading.py --frames 3
import taichi as ti
import taichi.math as tm

ti.init(arch=ti.gpu)

W, H = 480, 400
img = ti.Vector.field(3, dtype=float, shape=(W, H))
mask = ti.field(dtype=float, shape=(W, H))


@ti.func
def shade(p):
    light = tm.normalize(tm.vec3(0.3, 0.5, 1.0))
    n = tm.normalize(tm.vec3(p.x, p.y, 1.0))
    return tm.clamp(tm.dot(n, light), 0.0, 1.0)


@ti.kernel
def make_mask():
    for x, y in mask:
        mask[x, y] = 1.0 - 0.5 * tm.step(0.7, ti.sqrt((x / W - 0.5) ** 2 + (y / H - 0.5) ** 2) * 2.0)


@ti.kernel
def draw(t: float):
    for x, y in ti.ndrange(W, H):
        p = tm.vec2(x / W - 0.5, y / H - 0.5) * 2.0
        base = tm.vec3(tm.fract(p.x * 3.0 + t), tm.smoothstep(0.2, 0.8, tm.length(p)), tm.step(0.0, p.y))
        acc = tm.vec3(0.0)
        for k in ti.static(range(3)):
            acc[k] = base[k] * shade(p) + tm.sign(p.x) * 0.1 * k
        c = tm.cross(acc, tm.vec3(0.0, 0.0, 1.0))
        img[x, y] = tm.mix(acc, c, 0.25) * mask[x, y]


gui = ti.GUI("shading", res=(W, H))
make_mask()
t = 0.0
while gui.running:
    draw(t)
    gui.set_image(img)
    gui.show()
    t += 0.25
