# Conway's game of life on a torus: int32 fields, the eight neighbours read at offset indices
# (wrapped with %), ti.static loops over the offsets, a conditional expression for the rule, and
# a second kernel copying the new generation back.  Written against Taichi's API; run headless on
# the HIP device with
#     python -m vernondsl_amd.run vernondsl_amd/examples/life.py --frames 8
import taichi as ti

ti.init(arch=ti.gpu)

N = 320
state = ti.field(ti.i32, shape=(N, N))
nxt = ti.field(ti.i32, shape=(N, N))


@ti.kernel
def seed():
    for i, j in state:
        state[i, j] = 1 if (i * 37 + j * 91 + i * j) % 7 < 2 else 0


@ti.kernel
def step():
    for i, j in nxt:
        count = 0
        for di in ti.static(range(-1, 2)):
            for dj in ti.static(range(-1, 2)):
                if di != 0 or dj != 0:
                    count += state[(i + di + N) % N, (j + dj + N) % N]
        nxt[i, j] = 1 if count == 3 or (state[i, j] == 1 and count == 2) else 0


@ti.kernel
def copy_back():
    for i, j in state:
        state[i, j] = nxt[i, j]


gui = ti.GUI("life", res=(N, N))
seed()
while gui.running:
    step()
    copy_back()
    gui.set_image(state)
    gui.show()
