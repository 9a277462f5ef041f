# Gravitational N-body in 2-D: every particle sums the pull of all N (an O(N^2) loop whose
# variable indexes another field, `x[j]`: a runtime loop reading its trip), then a kick-drift
# update storing velocities and positions.  Written against Taichi's API; run headless on the HIP
# device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/nbody.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

N = 4096
x = ti.Vector.field(2, dtype=float, shape=N)
v = ti.Vector.field(2, dtype=float, shape=N)
a = ti.Vector.field(2, dtype=float, shape=N)
dt, soft = 0.0005, 0.001


@ti.kernel
def seed():
    for i in x:
        ang = i * 2.399963
        rad = ti.sqrt((i + 0.5) / N)
        x[i] = [rad * ti.cos(ang), rad * ti.sin(ang)]
        v[i] = [-ti.sin(ang) * rad * 0.5, ti.cos(ang) * rad * 0.5]


@ti.kernel
def forces():
    for i in a:
        acc = ti.Vector([0.0, 0.0])
        p = x[i]
        for j in range(N):
            d = x[j] - p
            r2 = d.dot(d) + soft
            acc += d / (r2 * ti.sqrt(r2))
        a[i] = acc / N


@ti.kernel
def advance():
    for i in x:
        v[i] += a[i] * dt
        x[i] += v[i] * dt


gui = ti.GUI("nbody", res=(512, 512))
seed()
while gui.running:
    for _ in range(2):
        forces()
        advance()
    gui.circles(x.to_numpy() * 0.4 + 0.5, radius=1)
    gui.show()
