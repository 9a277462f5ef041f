#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ (run from the repository root:
`python tests/golden/make_golden.py`).

The reference ships no golden vectors, known-answer tests or fixtures for this path (its only
program, fractal.py, has no test and runs on Taichi, which is not importable here), so every
fixture below is produced by the CPU oracle on a small seeded input and cross-checked, before it
is written, against an independent computation (numpy in f32/f64/int64) that shares no code with
the oracle.  The fixtures are data only: inputs and expected outputs, as .npz (no pickles) plus
known_answers.json.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle  # noqa: E402
from vernondsl_amd import _lib, mapchain as mc, rng, spec  # noqa: E402
from test_oracle_escape_time import numpy_escape  # noqa: E402  (independent numpy restatement)


def save(name, **arrays):
    np.savez(os.path.join(HERE, name), **arrays)


def main():
    known = {}
    # ---- escape time ------------------------------------------------------------------------
    for rnd, tag in ((_lib.ESC_ROUND_SEPARATE, "separate"), (_lib.ESC_ROUND_FMA, "fma")):
        p = spec.mandelbrot_params(n=64, rounding=rnd)
        c = oracle.escape_time(p)
        assert np.array_equal(c, numpy_escape(p))
        save(f"mandelbrot_64_{tag}.npz", counts=c)
        full = oracle.escape_time(spec.mandelbrot_params(rounding=rnd))
        assert np.array_equal(full, numpy_escape(spec.mandelbrot_params(rounding=rnd)))
        known[f"mandelbrot_1024_{tag}"] = {
            "sum": int(full.sum()), "pixels_at_max_iter": int((full == 256).sum()),
            "sha256_int32_le": hashlib.sha256(np.ascontiguousarray(full, "<i4").tobytes()).hexdigest(),
            "corner_00": int(full[0, 0]), "corner_last": int(full[-1, -1]), "c_minus2": int(full[0, 512])}
    p = spec.julia_paint_params(0.0, n=40)
    j = oracle.escape_time(p)
    assert np.array_equal(j, numpy_escape(p))
    save("julia_paint_n40_t0.npz", pixels=j)

    # ---- map chain ------------------------------------------------------------------------------
    x, bias = spec.map_chain_inputs(32, 64)
    prog = mc.compile(spec.map_chain_expr())
    y = oracle.map_chain(prog, [x, bias], 32, 64)
    u = ((np.float32(spec.MAP_A) * x) + np.float32(spec.MAP_B)).astype(np.float64)
    te = np.tanh(u) * np.exp(-(x.astype(np.float64) ** 2))
    assert np.all(np.abs(y - (te + bias)) <= 1e-6 * (np.abs(te) + np.abs(bias)))
    save("map_chain_32x64.npz", x=x, bias=bias, y=y)

    # ---- softmax ----------------------------------------------------------------------------------
    xs, _, _ = spec.softmax_inputs(16, 256)
    for tag, xh in (("f32", xs), ("bf16", rng.f32_to_bf16(xs))):
        s, m, sm = oracle.row_reduce_softmax(xh)
        xf = rng.bf16_to_f32(xh) if tag == "bf16" else xh
        x64 = xf.astype(np.float64)
        ref = np.exp(x64 - x64.max(1, keepdims=True))
        ref /= ref.sum(1, keepdims=True)
        smf = rng.bf16_to_f32(sm) if tag == "bf16" else sm
        # f32: exp's argument x - max is itself rounded (error |x - max| 2^-24, |x - max| < 40 here)
        assert np.all(np.abs(smf - ref) <= (2 ** -8 if tag == "bf16" else 5e-6) * ref + 1e-30)
        assert np.array_equal(m, xf.max(1))
        save(f"softmax_16x256_{tag}.npz", x=xh, row_sum=s, row_max=m, softmax=sm)

    # ---- bf16 GEMM ----------------------------------------------------------------------------------
    A = rng.f32_to_bf16(rng.uniform(11, 48 * 64, -1, 1)).reshape(48, 64)
    B = rng.f32_to_bf16(rng.uniform(12, 40 * 64, -1, 1)).reshape(40, 64)
    Cm, pre = oracle.gemm_bf16(A, B, False, True, c_dtype=1, epilogue=1, want_pre=True)
    ref = rng.bf16_to_f32(A).astype(np.float64) @ rng.bf16_to_f32(B).astype(np.float64).T
    assert np.allclose(pre, ref, rtol=1e-6, atol=1e-6)
    save("gemm_bf16_48x40x64_gelu.npz", A=A, B=B, pre=pre, C=Cm)

    # ---- int8 --------------------------------------------------------------------------------------
    xq8, layers = spec.w8a8_inputs(batch=16, widths=(128, 96, 64))
    y8 = oracle.w8a8_forward(xq8, layers)
    h = xq8
    for li, (w, s) in enumerate(layers):  # independent numpy restatement, bit for bit
        hf = rng.bf16_to_f32(h)
        sc = (np.abs(hf).max(1) / np.float32(127)).astype(np.float32)
        q = np.where(sc[:, None] > 0, np.clip(np.rint(hf / np.where(sc > 0, sc, 1)[:, None]), -127, 127), 0).astype(np.int8)
        acc = (q.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
        v = (acc.astype(np.float32) * sc[:, None]).astype(np.float32) * s[None, :]
        if li < len(layers) - 1:
            v = np.where(v > 0, v, np.float32(0))
        h = rng.f32_to_bf16(v.astype(np.float32))
    assert np.array_equal(h, y8)
    save("w8a8_16_128_96_64.npz", x=xq8, w0=layers[0][0], s0=layers[0][1], w1=layers[1][0], s1=layers[1][1], y=y8)

    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known, f, indent=1, sort_keys=True)
    print("golden fixtures written:", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
