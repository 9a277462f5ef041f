# An animated Julia set whose constant circles with the frame phase, written against Taichi's API;
# run on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/julia_orbit.py --frames 4
import taichi as ti

ti.init(arch=ti.vulkan)

W, H = 400, 300
img = ti.field(dtype=float, shape=(W, H))


@ti.func
def sq(p):
    return ti.Vector([p[0] ** 2 - p[1] ** 2, p[1] * p[0] * 2])


@ti.kernel
def frame(phase: float):
    for u, v in img:
        k0 = ti.Vector([-0.70176, ti.sin(phase) * 0.3842])
        p = ti.Vector([u / H - 0.6667, v / H - 0.5]) * 3
        n = 0
        while p.norm() < 8 and n < 96:
            p = sq(p) + k0
            n += 1
        img[u, v] = n * 0.01 + 0.05


gui = ti.GUI("julia orbit", res=(W, H))
for f in range(100000):
    frame(f * 0.05)
    gui.set_image(img)
    gui.show()
