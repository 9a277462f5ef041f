"""ctypes binding of libvdsl.so, the C ABI declared in include/vdsl.h.

The library is the HIP device: there is no CPU fallback.  If libvdsl.so has not been built,
importing this module raises ImportError naming the build step.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvdsl.so")

# ---- enums (include/vdsl.h) ----------------------------------------------------------------
VDSL_OK = 0
STATUS_NAMES = {
    0: "VDSL_OK",
    -1: "VDSL_ERR_INVALID_ARG",
    -2: "VDSL_ERR_INVALID_HANDLE",
    -3: "VDSL_ERR_OUT_OF_MEMORY",
    -4: "VDSL_ERR_DEVICE",
    -5: "VDSL_ERR_UNSUPPORTED",
    -6: "VDSL_ERR_CAPTURE",
    -7: "VDSL_ERR_SHAPE",
    -8: "VDSL_ERR_NO_DEVICE",
}
DEVICE_HIP = 1

BIND_STORAGE_BUFFER, BIND_INPUT, BIND_OUTPUT, BIND_UNIFORM, BIND_UNIFORM_CONSTANT, BIND_IMAGE, BIND_VARYING = range(7)
# `vernon.semantic` strings (VernonToSpirv.cpp:44-55, color.mlir:4-9) -> binding kinds.
SEMANTIC_TO_BINDING = {
    "storage_buffer": BIND_STORAGE_BUFFER,
    "input": BIND_INPUT,
    "output": BIND_OUTPUT,
    "uniform": BIND_UNIFORM,
    "uniform_constant": BIND_UNIFORM_CONSTANT,
    "image": BIND_IMAGE,
    "varying": BIND_VARYING,
}

F32, BF16, I8, I32 = 0, 1, 2, 3

ESC_MANDELBROT, ESC_JULIA = 0, 1
ESC_MAG2_GT, ESC_NORM_GE = 0, 1
ESC_ROUND_SEPARATE, ESC_ROUND_FMA = 0, 1
ESC_OUT_I32_COUNT, ESC_OUT_F32_AFFINE = 0, 1

MAP_MAX_INSTR, MAP_MAX_REGS, MAP_MAX_INPUTS = 32, 8, 4
MAP_OPS = {
    "load": 1, "const": 2, "mov": 3, "neg": 4, "abs": 5, "square": 6, "exp": 7, "log": 8,
    "tanh": 9, "sigmoid": 10, "relu": 11, "sqrt": 12, "recip": 13, "add": 14, "sub": 15,
    "mul": 16, "div": 17, "max": 18, "min": 19, "fma": 20, "mul_imm": 21, "add_imm": 22,
    "matvec": 23, "vecmat": 24,
}
BCAST_FULL, BCAST_ROW, BCAST_COL, BCAST_SCALAR = 0, 1, 2, 3

EPI_NONE, EPI_GELU, EPI_RELU, EPI_GELU_DERIV = 0, 1, 2, 3


# ---- structs -------------------------------------------------------------------------------
class DeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 64),
        ("arch", C.c_char * 32),
        ("compute_units", C.c_int32),
        ("clock_khz", C.c_int32),
        ("wavefront_size", C.c_int32),
        ("lds_bytes_per_block", C.c_int32),
        ("hbm_bytes", C.c_uint64),
    ]


class EscapeTimeParams(C.Structure):
    _fields_ = [
        ("ni", C.c_int32), ("nj", C.c_int32), ("family", C.c_int32), ("escape_test", C.c_int32),
        ("rounding", C.c_int32), ("out_kind", C.c_int32), ("max_iter", C.c_int32), ("bound", C.c_float),
        ("re_den", C.c_float), ("re_off", C.c_float), ("re_scale", C.c_float), ("re_post", C.c_float),
        ("im_den", C.c_float), ("im_off", C.c_float), ("im_scale", C.c_float), ("im_post", C.c_float),
        ("c_re", C.c_float), ("c_im", C.c_float), ("out_base", C.c_float), ("out_scale", C.c_float),
    ]


class MapInstr(C.Structure):
    _fields_ = [
        ("op", C.c_uint8), ("dst", C.c_uint8), ("a", C.c_uint8), ("b", C.c_uint8), ("c", C.c_uint8),
        ("ext", C.c_uint8 * 3), ("imm", C.c_float),
    ]


class MapInput(C.Structure):
    _fields_ = [("buf", C.c_void_p), ("bcast", C.c_int32), ("dtype", C.c_int32)]


class MapVInput(C.Structure):
    _fields_ = [("buf", C.c_void_p), ("bcast", C.c_int32), ("dtype", C.c_int32), ("width", C.c_int32),
                ("mat_dim", C.c_int32)]


_vp = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_sz = C.c_size_t

# name -> (restype, argtypes).  Every symbol of include/vdsl.h appears here.
PROTOTYPES = {
    "vdsl_last_error": (C.c_char_p, []),
    "vdsl_abi_version": (C.c_int, []),
    "vdsl_device_count": (C.c_int, [C.c_int, C.POINTER(C.c_int)]),
    "vdsl_device_open": (C.c_int, [C.c_int, C.c_int, C.POINTER(_vp)]),
    "vdsl_device_close": (C.c_int, [_vp]),
    "vdsl_device_get_info": (C.c_int, [_vp, C.POINTER(DeviceInfo)]),
    "vdsl_buffer_alloc": (C.c_int, [_vp, _sz, C.c_int, C.POINTER(_vp)]),
    "vdsl_buffer_free": (C.c_int, [_vp]),
    "vdsl_buffer_size": (C.c_int, [_vp, C.POINTER(_sz)]),
    "vdsl_buffer_binding": (C.c_int, [_vp, C.POINTER(C.c_int)]),
    "vdsl_buffer_device_address": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "vdsl_buffer_write": (C.c_int, [_vp, _vp, _sz, _vp, _sz]),
    "vdsl_buffer_read": (C.c_int, [_vp, _vp, _sz, _vp, _sz]),
    "vdsl_buffer_fill_u32": (C.c_int, [_vp, _vp, _sz, _sz, C.c_uint32]),
    "vdsl_buffer_copy": (C.c_int, [_vp, _vp, _sz, _vp, _sz, _sz]),
    "vdsl_queue_create": (C.c_int, [_vp, C.POINTER(_vp)]),
    "vdsl_queue_destroy": (C.c_int, [_vp]),
    "vdsl_queue_sync": (C.c_int, [_vp]),
    "vdsl_graph_begin": (C.c_int, [_vp]),
    "vdsl_graph_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "vdsl_graph_launch": (C.c_int, [_vp, _vp]),
    "vdsl_graph_destroy": (C.c_int, [_vp]),
    "vdsl_event_create": (C.c_int, [_vp, C.POINTER(_vp)]),
    "vdsl_event_record": (C.c_int, [_vp, _vp]),
    "vdsl_event_elapsed_ms": (C.c_int, [_vp, _vp, C.POINTER(C.c_float)]),
    "vdsl_event_destroy": (C.c_int, [_vp]),
    "vdsl_op_escape_time": (C.c_int, [_vp, C.POINTER(EscapeTimeParams), _vp]),
    "vdsl_op_map_chain": (C.c_int, [_vp, _i64, _i64, C.POINTER(MapInstr), _i32, C.POINTER(MapInput), _i32, _i32, _vp]),
    "vdsl_op_map_chain_v": (C.c_int, [_vp, _i64, _i64, C.POINTER(MapInstr), _i32, C.POINTER(MapVInput), _i32,
                                      C.POINTER(_i32), _i32, _vp]),
    "vdsl_op_vec_transform": (C.c_int, [_vp, _i64, _i32, _vp, _i32, _vp, _vp, _vp]),
    "vdsl_op_mat_transform": (C.c_int, [_vp, _i64, _i32, _i32, _vp, _i32, _vp, _vp, _vp]),
    "vdsl_op_gemm_bf16_mse_packed": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vdsl_debug_map_chain_mode": (C.c_int, [_i32]),
    "vdsl_debug_map_chain_stats": (C.c_int, [C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)]),
    "vdsl_op_row_reduce_softmax": (C.c_int, [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "vdsl_op_col_reduce": (C.c_int, [_vp, _i64, _i64, _i32, _vp, _vp, _vp]),
    "vdsl_gemm_bf16_workspace_bytes": (C.c_int, [_i32, _i32, _i64, _i64, _i64, C.POINTER(_sz)]),
    "vdsl_op_gemm_bf16": (C.c_int, [_vp, _i32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "vdsl_op_pack_bf16_weights": (C.c_int, [_vp, _i64, _i64, _vp, _vp]),
    "vdsl_op_gemm_bf16_packed": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _vp]),
    "vdsl_op_transpose": (C.c_int, [_vp, _i64, _i64, _i32, _vp, _vp]),
    "vdsl_op_cast": (C.c_int, [_vp, _i64, _i32, _vp, _i32, _vp]),
    "vdsl_op_gelu_fwd": (C.c_int, [_vp, _i64, _i32, _vp, _i32, _vp]),
    "vdsl_op_gelu_bwd": (C.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "vdsl_op_relu_bwd": (C.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "vdsl_op_add": (C.c_int, [_vp, _i64, C.c_int32, _vp, C.c_int32, _vp, C.c_int32, _vp]),
    "vdsl_op_gemm_bf16_gelu_bwd": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "vdsl_op_gemm_bf16_gelu_bwd_packed": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "vdsl_op_gemm_bf16_mul_packed": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "vdsl_op_pixel_program": (C.c_int, [_vp, C.c_int32, C.c_int32, _vp, C.POINTER(_vp), C.c_int32, _vp]),
    "vdsl_mse_partials_count": (C.c_int64, [_i64, _i64]),
    "vdsl_op_mse_fwd_bwd": (C.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vdsl_op_quantize_rows_i8": (C.c_int, [_vp, _i64, _i64, _i32, _vp, _vp, _vp]),
    "vdsl_op_gemm_w8a8_packed_noalloc": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "vdsl_gemm_w8a8_workspace_bytes": (C.c_int, [_i64, _i64, _i64, C.POINTER(_sz)]),
    "vdsl_op_gemm_w8a8": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "vdsl_op_pack_w8a8_weights": (C.c_int, [_vp, _i64, _i64, _vp, _vp]),
    "vdsl_gemm_w8a8_packed_workspace_bytes": (C.c_int, [_i64, _i64, _i64, C.POINTER(_sz)]),
    "vdsl_op_gemm_w8a8_packed": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "vdsl_debug_fail_alloc_after": (C.c_int, [_i64]),
    "vdsl_debug_gemm_config": (C.c_int, [_i32]),
    "vdsl_debug_w8a8_packed_plan": (C.c_int, [_i32, _i32]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `make -C vernondsl_amd/csrc`).  There is no CPU fallback."
        )
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name, None)
        if fn is None:  # reported by missing_symbols(); calling it raises AttributeError
            continue
        fn.restype = res
        fn.argtypes = args
    return lib


def missing_symbols() -> list:
    """Symbols of include/vdsl.h that the loaded library does not export."""
    return [n for n in PROTOTYPES if getattr(lib, n, None) is None]


lib = _load()


class VdslError(RuntimeError):
    """A C-ABI call returned a negative vdsl_status."""

    def __init__(self, status: int, func: str, message: str):
        self.status = status
        self.func = func
        self.message = message
        super().__init__(f"{func} -> {STATUS_NAMES.get(status, status)}: {message}")


def call(name: str, *args) -> int:
    st = getattr(lib, name)(*args)
    if st != VDSL_OK:
        msg = lib.vdsl_last_error()
        raise VdslError(st, name, msg.decode() if msg else "")
    return st
