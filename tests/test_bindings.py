"""vernon.semantic binding-model reader (vernondsl_amd.bindings) on the CPU."""
import os

import pytest

from vernondsl_amd import _lib, bindings

REF = "/root/reference/source/tests/integration/color.mlir"

OWN = '''
module {
  func.func @shade(%uv: tensor<2xf32> {vernon.semantic = "varying"},
                   %lut: tensor<256x4xf32> {vernon.semantic = "uniform_constant"},
                   %scratch: tensor<64x64xbf16> {vernon.semantic = "storage_buffer"},
                   %plain: tensor<4xi32>)
                  -> (tensor<4xf32> {vernon.semantic="output"}, tensor<8xi8> {vernon.semantic = "image"}) {
    return
  }
}
'''


def test_own_signature():
    bs = bindings.read_bindings(OWN, "shade")
    assert [(b.name, b.shape, b.dtype, b.semantic) for b in bs] == [
        ("%uv", (2,), "f32", "varying"), ("%lut", (256, 4), "f32", "uniform_constant"),
        ("%scratch", (64, 64), "bf16", "storage_buffer"), ("result0", (4,), "f32", "output"),
        ("result1", (8,), "i8", "image")]
    assert [b.binding for b in bs] == [_lib.BIND_VARYING, _lib.BIND_UNIFORM_CONSTANT, _lib.BIND_STORAGE_BUFFER,
                                       _lib.BIND_OUTPUT, _lib.BIND_IMAGE]


def test_errors_are_reported_not_crashes():
    with pytest.raises(bindings.BindingError, match="no func.func @vertex_main"):
        bindings.read_bindings(OWN, "vertex_main")  # the pass dereferences a null FuncOp here
    bad = OWN.replace('"varying"', '"texture"')
    with pytest.raises(bindings.BindingError, match="unknown vernon.semantic"):
        bindings.read_bindings(bad, "shade")  # the pass prints an uninitialised storage class here


@pytest.mark.skipif(not os.path.exists(REF), reason="the reference tree is only mounted in the build container")
def test_reference_color_mlir():
    """The reference's test input (color.mlir:4-9, 43-45), read as text."""
    text = open(REF).read()
    vs = bindings.read_bindings(text, "vertex_main")
    assert [(b.name, b.shape, b.semantic) for b in vs] == [
        ("%pos", (3,), "input"), ("%model", (4, 4), "uniform"), ("%view", (4, 4), "uniform"),
        ("%proj", (4, 4), "uniform"), ("result0", (4,), "output"), ("result1", (3,), "varying")]
    fs = bindings.read_bindings(text, "frag_main")
    assert [(b.name, b.semantic, b.binding) for b in fs] == [
        ("%color", "uniform", _lib.BIND_UNIFORM), ("%frag_pos", "varying", _lib.BIND_VARYING),
        ("result0", "output", _lib.BIND_OUTPUT)]
