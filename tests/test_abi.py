"""The C ABI (include/vdsl.h) on a host without a GPU: the library loads, exports every declared
symbol, its struct layouts match the ctypes mirrors, and host-side error paths return statuses
with messages instead of crashing.  No op is executed here."""
import ctypes as C
import os
import re
import subprocess
import threading

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vdsl.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(vdsl_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    from vernondsl_amd import _lib
    names = header_functions()
    assert len(names) >= 40
    assert _lib.missing_symbols() == []
    assert sorted(_lib.PROTOTYPES) == names
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (vdsl_\w+)", nm))
    assert set(names) <= exported


def test_abi_version():
    from vernondsl_amd import _lib
    assert _lib.lib.vdsl_abi_version() == 7


def test_struct_layouts_match_header(tmp_path):
    from vernondsl_amd import _lib
    src = tmp_path / "probe.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "vdsl.h"\n'
                   "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(vdsl_escape_time_params),"
                   " sizeof(vdsl_map_instr), offsetof(vdsl_map_instr, imm), sizeof(vdsl_map_input),"
                   " sizeof(vdsl_device_info), offsetof(vdsl_escape_time_params, out_scale),"
                   " offsetof(vdsl_map_instr, ext), sizeof(vdsl_map_vinput), offsetof(vdsl_map_vinput, mat_dim));"
                   "printf(\"%zu %zu\\n\", sizeof(vdsl_pixel_program), offsetof(vdsl_pixel_program, code));"
                   "return 0;}\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [C.sizeof(_lib.EscapeTimeParams), C.sizeof(_lib.MapInstr), _lib.MapInstr.imm.offset,
            C.sizeof(_lib.MapInput), C.sizeof(_lib.DeviceInfo), _lib.EscapeTimeParams.out_scale.offset,
            _lib.MapInstr.ext.offset, C.sizeof(_lib.MapVInput), _lib.MapVInput.mat_dim.offset]
    from vernondsl_amd import pixprog
    want += [C.sizeof(pixprog.PixelProgram), pixprog.PixelProgram.code.offset]
    assert got == want


def test_null_handles_are_rejected_with_messages():
    from vernondsl_amd import _lib
    L = _lib.lib
    assert L.vdsl_queue_sync(None) == -2
    assert b"queue" in L.vdsl_last_error()
    assert L.vdsl_buffer_free(None) == -2
    assert L.vdsl_device_close(None) == -2
    assert L.vdsl_graph_launch(None, None) == -2
    assert L.vdsl_event_destroy(None) == -2
    assert L.vdsl_op_escape_time(None, None, None) == -2
    assert L.vdsl_op_gemm_bf16(None, 0, 1, 1, 1, 1, None, None, None, 0, 0, None, None) == -2
    out = C.c_void_p()
    assert L.vdsl_buffer_alloc(None, 16, 0, C.byref(out)) == -2 and out.value is None
    # a pointer that was never a handle is not dereferenced
    bogus = C.create_string_buffer(64)
    assert L.vdsl_queue_sync(C.cast(bogus, C.c_void_p)) == -2


def test_bad_arguments_without_device():
    from vernondsl_amd import _lib
    L = _lib.lib
    n = C.c_int(-1)
    assert L.vdsl_device_count(99, C.byref(n)) == -1
    assert L.vdsl_device_count(_lib.DEVICE_HIP, None) == -1
    st = L.vdsl_device_count(_lib.DEVICE_HIP, C.byref(n))
    assert st == 0 and n.value >= 0
    h = C.c_void_p()
    assert L.vdsl_device_open(_lib.DEVICE_HIP, 4096, C.byref(h)) == -8
    assert b"no HIP device" in L.vdsl_last_error()


def test_workspace_queries_are_pure_host():
    from vernondsl_amd import _lib
    L = _lib.lib
    n = C.c_size_t(123)
    assert L.vdsl_gemm_bf16_workspace_bytes(0, 1, 256, 256, 256, C.byref(n)) == 0 and n.value == 0
    assert L.vdsl_gemm_bf16_workspace_bytes(0, 0, 256, 512, 128, C.byref(n)) == 0 and n.value == 512 * 128 * 2
    assert L.vdsl_gemm_bf16_workspace_bytes(1, 0, 256, 512, 128, C.byref(n)) == 0
    assert n.value == (256 * 128 + 512 * 128) * 2
    assert L.vdsl_gemm_bf16_workspace_bytes(0, 1, -1, 2, 2, C.byref(n)) == -1
    assert L.vdsl_mse_partials_count(2048, 4096) > 0
    # sizes that wrap size_t are errors, not small numbers
    n.value = 123
    assert L.vdsl_gemm_bf16_workspace_bytes(1, 0, 1 << 40, 1 << 40, 1 << 40, C.byref(n)) == -7
    assert b"overflows" in L.vdsl_last_error() and n.value == 123
    # a narrow output splits K into M x N int32 partials
    assert L.vdsl_gemm_w8a8_workspace_bytes(64, 64, 4096, C.byref(n)) == 0 and n.value == 64 * 64 * 4


def test_last_error_is_thread_local():
    from vernondsl_amd import _lib
    L = _lib.lib
    L.vdsl_queue_sync(None)
    mine = L.vdsl_last_error()
    seen = {}

    def other():
        seen["before"] = L.vdsl_last_error()
        h = C.c_void_p()
        L.vdsl_device_open(_lib.DEVICE_HIP, 4096, C.byref(h))
        seen["after"] = L.vdsl_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == b""
    assert b"no HIP device" in seen["after"]
    assert L.vdsl_last_error() == mine


def test_python_wrapper_raises():
    from vernondsl_amd import _lib, rhi
    with pytest.raises(_lib.VdslError) as ei:
        rhi.Device(4096)
    assert ei.value.status == -8


def test_semantic_vocabulary_covers_pass_table():
    # VernonToSpirv.cpp:44-55 maps these `vernon.semantic` strings; color.mlir adds "varying".
    from vernondsl_amd import _lib
    for s in ("input", "output", "uniform", "uniform_constant", "storage_buffer", "image", "varying"):
        assert s in _lib.SEMANTIC_TO_BINDING
    assert len(set(_lib.SEMANTIC_TO_BINDING.values())) == 7


def test_opcode_tables_match_the_header():
    """pixprog.OP and the map-chain opcodes name the values include/vdsl.h gives them."""
    from vernondsl_amd import pixprog
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    enum = {m.group(1).lower(): int(m.group(2)) for m in re.finditer(r"VDSL_(?:MAP|PIX)_(\w+)\s*=\s*(\d+)", text)}
    for name, code in pixprog.OP.items():
        assert enum.get(name) == code, name
    assert enum["trip"] == 43 and pixprog.OP["trip"] == 43
