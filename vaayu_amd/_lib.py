"""ctypes binding of libvaayu_amd.so (the C ABI in include/vaayu_amd.h).

The library is built in-tree by `vaayu_amd.build`. There is no fallback: if it is missing
or fails to load, every kernel entry raises, naming the file.
"""
import ctypes
import os

import torch  # noqa: F401  -- loads the HIP runtime the library binds to

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvaayu_amd.so")
ABI_VERSION = 12

# The reference's `_DTYPE_CODE` (vaayu/packed_expert_kernels.py:70).
DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

EXPORTS = ("vaayu_abi_version", "vaayu_last_error", "vaayu_decode_gate_up", "vaayu_decode_down",
           "vaayu_prefill_gate_up", "vaayu_prefill_down", "vaayu_prefill_reduce",
           "vaayu_dequant_blob", "vaayu_dequant_fp8_block", "vaayu_upcast_mx",
           "vaayu_route_topk", "vaayu_gdn_rule", "vaayu_gdn_conv_update", "vaayu_gdn_gated_norm",
           "vaayu_fused3d_gate_up", "vaayu_fused3d_down", "vaayu_router_logits",
           "vaayu_decode_noalloc", "vaayu_decode_noalloc_scratch_bytes", "vaayu_probe_mfma",
           "vaayu_decode_fused", "vaayu_decode_fused_sync_words", "vaayu_probe_mfma_sum",
           "vaayu_prefill_run_blocks")


class Geom(ctypes.Structure):
    """`vaayu_geom` of include/vaayu_amd.h."""
    _fields_ = [("bits", ctypes.c_int32), ("group", ctypes.c_int32),
                ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
                ("gate_w", ctypes.c_int64), ("gate_s", ctypes.c_int64),
                ("up_w", ctypes.c_int64), ("up_s", ctypes.c_int64),
                ("down_w", ctypes.c_int64), ("down_s", ctypes.c_int64),
                ("format", ctypes.c_int32), ("block_rows", ctypes.c_int32)]


class KernelError(RuntimeError):
    """A rejected or failed kernel call (the library's nonzero return code)."""


_LIB = None
_LOAD_ERROR = None


def _bind(lib):
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    gp = ctypes.POINTER(Geom)
    sig = {
        "vaayu_abi_version": (ctypes.c_int, []),
        "vaayu_last_error": (ctypes.c_char_p, []),
        "vaayu_decode_gate_up": (ctypes.c_int, [vp, vp, vp, i32, gp, i32, i32, vp]),
        "vaayu_decode_down": (ctypes.c_int, [vp, vp, vp, i32, vp, i32, gp, i32, i32, i32, vp]),
        "vaayu_prefill_gate_up": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, vp, i32, i32, gp,
                                                 i32, i32, vp]),
        "vaayu_prefill_down": (ctypes.c_int,
                               [vp, vp, vp, vp, i32, i32, vp, i32, vp, i32, gp, i32, i32, i32,
                                vp]),
        "vaayu_prefill_run_blocks": (ctypes.c_int32, [i32]),
        "vaayu_prefill_reduce": (ctypes.c_int, [vp, vp, vp, i32, i32, i32, vp]),
        "vaayu_dequant_blob": (ctypes.c_int, [vp, vp, i32, vp, i32, i64, i32, i32, vp]),
        "vaayu_dequant_fp8_block": (ctypes.c_int, [vp, vp, i32, vp, i32, i64, i64, i64, i64, vp]),
        "vaayu_upcast_mx": (ctypes.c_int, [vp, i32, vp, vp, i32, i64, i64, vp]),
        "vaayu_route_topk": (ctypes.c_int, [vp, i32, i32, i32, i32, i32, ctypes.c_float, i32,
                                             vp, vp, vp, vp, vp]),
        "vaayu_gdn_rule": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                          i32, ctypes.c_float, i32, i32, i32, i32, i32, vp]),
        "vaayu_gdn_conv_update": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                                 i32, i32, i32, vp]),
        "vaayu_gdn_gated_norm": (ctypes.c_int, [vp, vp, vp, vp, vp, i64, i32, ctypes.c_float,
                                                i32, i32, i32, i32, vp]),
        "vaayu_fused3d_gate_up": (ctypes.c_int, [vp, vp, vp, vp, vp, i32, i32, vp, i32, i32,
                                                 i32, i32, i32, i32, vp, vp, ctypes.c_float,
                                                 ctypes.c_float, vp]),
        "vaayu_fused3d_down": (ctypes.c_int, [vp, vp, vp, vp, vp, i32, i32, vp, vp, i32, i32,
                                              i32, i32, i32, vp, vp, vp]),
        "vaayu_router_logits": (ctypes.c_int, [vp, vp, i32, vp, i32, i32, i32, i32, vp]),
        "vaayu_decode_noalloc": (ctypes.c_int, [vp, vp, vp, i32, vp, i32, gp, i32, i32, i32,
                                                vp]),
        "vaayu_decode_noalloc_scratch_bytes": (ctypes.c_int64, []),
        "vaayu_probe_mfma": (ctypes.c_int, [vp, i32, i32, vp]),
        "vaayu_probe_mfma_sum": (ctypes.c_int, [vp, vp, vp, i32, i32, i32, vp]),
        "vaayu_decode_fused": (ctypes.c_int, [vp, vp, vp, i32, vp, vp, vp, i32, gp, i32, i32,
                                              i32, i32, vp]),
        "vaayu_decode_fused_sync_words": (ctypes.c_int32, [i32, gp, i32, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args


def load(path: str = LIB_PATH):
    """The loaded library; raises (with the path) if it is absent or stale."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise ImportError(f"vaayu_amd: {path} is not built; run `python -m vaayu_amd.build`")
    lib = ctypes.CDLL(path)
    _bind(lib)
    if lib.vaayu_abi_version() != ABI_VERSION:
        raise ImportError(f"vaayu_amd: {path} has ABI {lib.vaayu_abi_version()}, "
                          f"this package expects {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except Exception:
        return False


def check(rc: int, what: str) -> None:
    if rc:
        msg = (_LIB.vaayu_last_error() or b"").decode(errors="replace")
        raise KernelError(f"{what} failed (code {rc}): {msg}")


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def geom_struct(geom) -> Geom:
    """`vaayu_geom` for a blob geometry `(bits or format, gs, roles)`: the role offsets of
    `_layout`, the code format and its scale blocking."""
    from .block_formats import blob_layout, geom_format
    fmt, bits, group, brows = geom_format(geom)
    lay = blob_layout(geom)
    inter, hidden = lay["gate"][2], lay["gate"][3]
    return Geom(bits, group, hidden, inter, lay["gate"][0], lay["gate"][1], lay["up"][0],
                lay["up"][1], lay["down"][0], lay["down"][1], fmt, brows)
