"""Runs a Taichi-style program on the HIP device:  python -m vernondsl_amd.run PROG.py [--frames N]

`import taichi as ti` inside PROG resolves to vernondsl_amd.taichi_compat for the duration of the
run, so the program text is unchanged.  GUI windows are headless; an endless frame loop such as
the reference's `for i in range(1000000)` (fractal.py:30) stops after --frames frames (default 8)
and the runner prints one JSON line: frames rendered and a checksum of the last image.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import runpy
import sys

import numpy as np

from . import taichi_compat


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m vernondsl_amd.run")
    ap.add_argument("program")
    ap.add_argument("--frames", type=int, default=8)
    args = ap.parse_args(argv)
    saved = {name: sys.modules.get(name) for name in ("taichi", "taichi.math")}
    sys.modules["taichi"] = taichi_compat
    sys.modules["taichi.math"] = taichi_compat.math
    taichi_compat.GUI.frame_limit = args.frames
    result = {"program": args.program, "frames": 0, "last_image_sha256": None}
    try:
        runpy.run_path(args.program, run_name="__main__")
    except taichi_compat.FrameLimitReached:
        pass
    finally:
        for name, mod in saved.items():
            if mod is None:
                sys.modules.pop(name, None)
            else:
                sys.modules[name] = mod
    gui = taichi_compat._state.get("last_gui")
    if gui is not None and gui.last_image is not None:
        img = np.ascontiguousarray(gui.last_image)
        result.update(frames=gui.frames, shape=list(img.shape), dtype=str(img.dtype),
                      last_image_sha256=hashlib.sha256(img.tobytes()).hexdigest())
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
