# Julia sets whose constant drifts on a small circle around the "Douady rabbit" parameter
# c = -0.1226 + 0.7449i, shaded from white (fast escape) to black (never escapes within STEPS).
# Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/rabbit_drift.py --frames 4
import taichi as ti

ti.init(arch=ti.amdgpu)

SIDE = 512
STEPS = 128
ESCAPE_R2 = 16.0
shade = ti.field(dtype=ti.f32, shape=(SIDE, SIDE))


@ti.func
def square(w):
    re = w[0] * w[0] - w[1] * w[1]
    im = 2 * (w[0] * w[1])
    return ti.Vector([re, im])


@ti.kernel
def draw(angle: ti.f32):
    for a, b in shade:
        c = ti.Vector([-0.1226 + 0.05 * ti.cos(angle), 0.7449 + 0.05 * ti.sin(angle)])
        w = ti.Vector([a / SIDE * 3.2 - 1.6, b / SIDE * 3.2 - 1.6])
        steps = 0
        while steps < STEPS and w.dot(w) <= ESCAPE_R2:
            w = square(w) + c
            steps += 1
        shade[a, b] = 1.0 - steps * (1.0 / STEPS)


window = ti.GUI("rabbit drift", res=(SIDE, SIDE))
angle = 0.0
while window.running:
    draw(angle)
    window.set_image(shade)
    window.show()
    angle += 0.1
