"""The C ABI library: loads, exports every symbol include/vaayu_amd.h declares, and rejects
bad arguments before touching a GPU (no compute calls here)."""
import ctypes
import os
import re

import pytest

from vaayu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    inc = os.path.join(ROOT, "include")
    for f in sorted(os.listdir(inc)):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(vaayu_\w+)\s*\(", text, re.M)
    return names


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 8
    assert set(_lib.EXPORTS) <= set(declared)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.vaayu_abi_version() == _lib.ABI_VERSION


def test_bad_arguments_are_rejected_without_a_launch():
    lib = _lib.load()
    g = _lib.geom_struct((4, 32, (("gate", 512, 2048), ("down", 2048, 512), ("up", 512, 2048))))
    rc = lib.vaayu_decode_gate_up(None, None, None, 1, ctypes.byref(g), 0, 0, None)
    assert rc == -1 and b"null" in lib.vaayu_last_error()
    rc = lib.vaayu_decode_gate_up(8, 256, 256, 1, ctypes.byref(g), 0, 0, None)
    assert rc == -1 and b"aligned" in lib.vaayu_last_error()
    rc = lib.vaayu_decode_down(1, 1, 1, 2, 1, 0, ctypes.byref(g), 0, 0, 0, None)
    assert rc == -1
    bad = _lib.geom_struct((3, 32, (("gate", 512, 2048), ("down", 2048, 512), ("up", 512, 2048))))
    rc = lib.vaayu_decode_gate_up(256, 256, 256, 1, ctypes.byref(bad), 0, 0, None)
    assert rc == -2 and b"bit width" in lib.vaayu_last_error()
    rc = lib.vaayu_prefill_gate_up(1, 1, 1, 1, 0, 1, 1, 1, 1, ctypes.byref(g), 2, 0, None)
    assert rc == -2 and b"activation" in lib.vaayu_last_error()
    small = _lib.geom_struct((4, 32, (("gate", 64, 64), ("down", 64, 64), ("up", 64, 64))))
    rc = lib.vaayu_prefill_gate_up(1, 1, 1, 1, 0, 1, 1, 1, 1, ctypes.byref(small), 0, 0, None)
    assert rc == -2 and b"K tile" in lib.vaayu_last_error()
    rc = lib.vaayu_dequant_blob(1, 1, 0, 1, 0, 0, 4, 32, None)
    assert rc == -1
    rc = lib.vaayu_prefill_reduce(None, None, None, 1, 1, 1, None)
    assert rc == -1


def test_the_geometry_struct_follows_the_layout():
    g = _lib.geom_struct((4, 128, (("gate", 768, 2048), ("down", 2048, 768), ("up", 768, 2048))))
    assert (g.bits, g.group, g.hidden, g.inter) == (4, 128, 2048, 768)
    assert (g.gate_w, g.gate_s) == (0, 0)
    assert (g.down_w, g.down_s) == (768 * 2048 // 8, 768 * 2048 // 128)
    assert (g.up_w, g.up_s) == (2 * 768 * 2048 // 8, 2 * 768 * 2048 // 128)


def test_the_kernel_module_refuses_without_the_library(monkeypatch):
    import vaayu_amd.packed_expert_kernels as pk
    monkeypatch.setattr(pk, "triton", None)
    with pytest.raises(ImportError):
        pk._require_backend()
