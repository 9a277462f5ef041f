"""The five workloads of the tensor-op path: shapes, constants, seeds and seeded inputs.

Decisions the workload descriptions leave open are fixed here once, and both the HIP device
and the CPU oracle consume the same host bytes produced below.

config 1  Mandelbrot escape time (the per-pixel iterative map of fractal.py:16-25, in
          Mandelbrot form): 1024 x 1024, c = (-2 + 3 i/1024, -1.5 + 3 j/1024), z0 = 0,
          max_iter = 256, stop when |z|^2 > 4, int32 counts, layout [i = re][j = im].
          Rounding: fused form (ESC_ROUND_FMA); the separately-rounded form of complex_sqr
          is also supported and tested.
config 2  y = tanh(a x + b) * exp(-x^2) + bias[col], x ~ N(0,1) f32 [8192][8192],
          a = 0.75, b = -0.25 (each product/sum rounded separately), bias ~ U(-1,1) [8192].
config 3  rows of x ~ N(0, sigma = 2) [16384][4096] (the "4" read as variance), 1% of rows
          (164, a seeded choice) get +20 in one seeded column; f32 and bf16 (RNE of the f32
          values).  Outputs: row sum, row max (f32), softmax (input dtype).
config 4  2-layer MLP, in = hidden = out = 4096, batch 2048, no biases, exact-erf GELU, MSE
          mean loss; X ~ N(0,1) -> bf16, W1, W2 Xavier-uniform U(+-sqrt(6/8192)) -> bf16 with
          the PyTorch Linear layout [out][in], T ~ N(0,1) f32.
config 5  4-layer int8 MLP 8192 -> 8192 -> 8192 -> 8192 -> 1024, batch 512, X ~ N(0,1) -> bf16,
          W int8 uniform on [-127, 127] stored [out][in], per-output-channel scales
          U(0.005, 0.02); dynamic per-row activation quantisation; ReLU between layers, none
          after the last; bf16 activations out of every layer.
"""
from __future__ import annotations

import numpy as np

from . import _lib, rng

SEEDS = {1: 0x5EED0001, 2: 0x5EED0002, 3: 0x5EED0003, 4: 0x5EED0004, 5: 0x5EED0005}


# ---- config 1 -------------------------------------------------------------------------------
def mandelbrot_params(n: int = 1024, max_iter: int = 256, rounding: int = _lib.ESC_ROUND_FMA) -> dict:
    """Window re in [-2, 1), im in [-1.5, 1.5): re = (i / n) * 3 + (-2), every step exact in f32
    for n a power of two."""
    return dict(ni=n, nj=n, family=_lib.ESC_MANDELBROT, escape_test=_lib.ESC_MAG2_GT, rounding=rounding,
                out_kind=_lib.ESC_OUT_I32_COUNT, max_iter=max_iter, bound=4.0,
                re_den=float(n), re_off=0.0, re_scale=3.0, re_post=-2.0,
                im_den=float(n), im_off=0.0, im_scale=3.0, im_post=-1.5)


def julia_paint_params(t: float, n: int = 320) -> dict:
    """The program of fractal.py:7-25 for frame time t: pixels f32 [2n][n],
    z0 = (i/n - 1, j/n - 0.5) * 2, c = (-0.8, cos(t) * 0.2), `while |z| < 20 and it < 50`,
    store 1 - it * 0.02.  c is evaluated in f32 as Taichi's default float type would."""
    c_im = np.float32(np.cos(np.float32(t), dtype=np.float32) * np.float32(0.2))
    return dict(ni=2 * n, nj=n, family=_lib.ESC_JULIA, escape_test=_lib.ESC_NORM_GE,
                rounding=_lib.ESC_ROUND_SEPARATE, out_kind=_lib.ESC_OUT_F32_AFFINE, max_iter=50, bound=20.0,
                re_den=float(n), re_off=-1.0, re_scale=2.0, re_post=0.0,
                im_den=float(n), im_off=-0.5, im_scale=2.0, im_post=0.0,
                c_re=-0.8, c_im=float(c_im), out_base=1.0, out_scale=-0.02)


# ---- config 2 -------------------------------------------------------------------------------
MAP_A, MAP_B = 0.75, -0.25


def map_chain_inputs(rows: int = 8192, cols: int = 8192, seed: int = SEEDS[2]):
    x = rng.normal(seed, rows * cols).reshape(rows, cols)
    bias = rng.uniform(seed ^ 0xB1A5, cols, -1.0, 1.0)
    return x, bias


def map_chain_expr():
    from . import mapchain as mc
    x = mc.Input(0)
    bias = mc.Input(1, bcast="row")
    return mc.tanh(x * MAP_A + MAP_B) * mc.exp(-(x * x)) + bias


def map_chain_bytes(rows: int, cols: int) -> int:
    """Algorithmic HBM bytes of one call: read x, write y, read bias once."""
    return rows * cols * 4 * 2 + cols * 4


# ---- config 3 -------------------------------------------------------------------------------
def softmax_inputs(rows: int = 16384, cols: int = 4096, seed: int = SEEDS[3]):
    x = rng.normal(seed, rows * cols, 0.0, 2.0).reshape(rows, cols)
    n_out = max(1, round(rows * 0.01))
    perm_keys = rng.u64(seed ^ 0x0071, rows)
    out_rows = np.sort(np.argsort(perm_keys, kind="stable")[:n_out])
    out_cols = (rng.u64(seed ^ 0xC01, n_out) % np.uint64(cols)).astype(np.int64)
    x[out_rows, out_cols] += np.float32(20.0)
    return x, out_rows, out_cols


def softmax_bytes(rows: int, cols: int, dtype: int) -> int:
    """Algorithmic HBM bytes: read x, write softmax, write row sum and row max."""
    es = 4 if dtype == _lib.F32 else 2
    return rows * cols * es * 2 + rows * 4 * 2


# ---- config 4 -------------------------------------------------------------------------------
def mlp_inputs(batch: int = 2048, d_in: int = 4096, hidden: int = 4096, d_out: int = 4096, seed: int = SEEDS[4]):
    x = rng.f32_to_bf16(rng.normal(seed, batch * d_in)).reshape(batch, d_in)
    b1 = float(np.sqrt(6.0 / (d_in + hidden)))
    b2 = float(np.sqrt(6.0 / (hidden + d_out)))
    w1 = rng.f32_to_bf16(rng.uniform(seed ^ 0x1, hidden * d_in, -b1, b1)).reshape(hidden, d_in)
    w2 = rng.f32_to_bf16(rng.uniform(seed ^ 0x2, d_out * hidden, -b2, b2)).reshape(d_out, hidden)
    t = rng.normal(seed ^ 0x3, batch * d_out).reshape(batch, d_out)
    return x, w1, w2, t


def mlp_flops(batch: int, d_in: int, hidden: int, d_out: int) -> int:
    """Five GEMMs: H = X W1^T, Y = H W2^T, dW2 = dY^T H, dH = dY W2, dW1 = dA^T X."""
    return 2 * batch * (d_in * hidden * 2 + hidden * d_out * 3)


# ---- config 5 -------------------------------------------------------------------------------
W8A8_WIDTHS = (8192, 8192, 8192, 8192, 1024)


def w8a8_inputs(batch: int = 512, widths=W8A8_WIDTHS, seed: int = SEEDS[5]):
    x = rng.f32_to_bf16(rng.normal(seed, batch * widths[0])).reshape(batch, widths[0])
    layers = []
    for li in range(len(widths) - 1):
        n_in, n_out = widths[li], widths[li + 1]
        w = rng.int_uniform(seed ^ (0x100 + li), n_out * n_in, -127, 127).astype(np.int8).reshape(n_out, n_in)
        s = rng.uniform(seed ^ (0x200 + li), n_out, 0.005, 0.02)
        layers.append((w, s))
    return x, layers


def w8a8_ops(batch: int, widths=W8A8_WIDTHS) -> int:
    return sum(2 * batch * widths[i] * widths[i + 1] for i in range(len(widths) - 1))
