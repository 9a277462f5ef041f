# Metaballs: a 2-D image kernel sums the field of every ball, read from a 1-D field of positions
# (a field of another shape than the loop's, gathered at the loop's trip), while the balls move
# in a 1-D kernel of their own.  Written against Taichi's API; run headless on the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/metaballs.py --frames 4
import taichi as ti

ti.init(arch=ti.gpu)

W, H, N = 640, 480, 48
img = ti.field(dtype=float, shape=(W, H))
pos = ti.Vector.field(2, dtype=float, shape=N)
vel = ti.Vector.field(2, dtype=float, shape=N)


@ti.kernel
def seed():
    for k in pos:
        pos[k] = [(k * 97 % 613) + 10.0, (k * 53 % 457) + 10.0]
        vel[k] = [((k * 7 % 11) - 5) * 0.9, ((k * 5 % 13) - 6) * 0.7]


@ti.kernel
def move():
    for k in pos:
        p = pos[k] + vel[k]
        v = vel[k]
        if p[0] < 0.0 or p[0] > W:
            v[0] = -v[0]
        if p[1] < 0.0 or p[1] > H:
            v[1] = -v[1]
        pos[k] = p
        vel[k] = v


@ti.kernel
def render():
    for i, j in img:
        s = 0.0
        for k in range(N):
            d = pos[k] - ti.Vector([i * 1.0, j * 1.0])
            s += 300.0 / (d.dot(d) + 1.0)
        img[i, j] = ti.min(s, 1.0)


gui = ti.GUI("metaballs", res=(W, H))
seed()
while gui.running:
    move()
    render()
    gui.set_image(img)
    gui.show()
