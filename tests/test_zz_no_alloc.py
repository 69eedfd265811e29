"""`vaayu_decode_noalloc`: the one-token decode with its intermediate h in the library's
static device scratch, held to the two decode entries that take a caller buffer
(`vaayu_decode_gate_up` + `vaayu_decode_down`, through `_launch`) bit for bit, on two
calls in a row -- the second smaller -- so the second reads only what it wrote."""
import pytest
import torch

import vaayu_amd.packed_expert_kernels as pk
from tests.helpers import decode_case, format_case
from vaayu_amd import _lib

pytestmark = pytest.mark.gpu


def noalloc(x, pairs, routing_weights, out):
    """The no-alloc entry through the C ABI, over the same pointer table `_launch` builds."""
    lib = pk._require_backend()
    blob = pairs[0][0]
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    rw = routing_weights.reshape(-1).contiguous()
    w_round = int(rw.dtype == x.dtype and x.dtype != torch.float32)
    rc = lib.vaayu_decode_noalloc(x.data_ptr(), tbl.data_ptr(), rw.data_ptr(),
                                  pk._DTYPE_CODE[rw.dtype], out.data_ptr(), len(pairs),
                                  _lib.geom_struct(blob["geom"]), pk._DTYPE_CODE[x.dtype],
                                  pk._SCALE_CODE[blob["flat"]["scale"].dtype], w_round,
                                  _lib.stream_ptr(x.device))
    _lib.check(rc, "vaayu_decode_noalloc")


def _both(case):
    x, pairs, w, _cpu = case
    want = torch.full((1, x.shape[1]), float("nan"), device="cuda")
    pk._launch(x, pairs, w, want)
    got = torch.full((1, x.shape[1]), float("nan"), device="cuda")
    noalloc(x, pairs, w, got)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16], ids=["fp32-w", "bf16-w"])
def test_two_calls_in_a_row_the_second_smaller(w_dtype):
    """Qwen3-30B-A3B shape (8 pairs x 768), then the toy shape (4 pairs x 512)."""
    for case in (decode_case(2048, 768, 4, 128, 8, seed=1, w_dtype=w_dtype),
                 decode_case(1024, 512, 4, 128, 4, seed=2, w_dtype=w_dtype)):
        got, want = _both(case)
        assert torch.equal(got, want)


def test_fp8_then_mxfp4_blobs():
    for case in (format_case("e4m3", 2048, 768, 8, seed=3),
                 format_case("mxfp4", 1024, 512, 2, seed=4)):
        got, want = _both(case)
        assert torch.equal(got, want)


def test_the_call_allocates_nothing():
    x, pairs, w, _cpu = decode_case(2048, 768, 4, 128, 8, seed=5)
    out = torch.empty(1, 2048, device="cuda")
    for _ in range(len(pk._TABLES._slots)):      # the table lanes' lazy state first
        noalloc(x, pairs, w, out)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    for _ in range(3):
        noalloc(x, pairs, w, out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before


def test_an_intermediate_over_the_scratch_is_refused():
    """n_pairs * inter * 2 bytes past 4 MiB: -3 before any pointer is read."""
    lib = pk._require_backend()
    assert lib.vaayu_decode_noalloc_scratch_bytes() == 4 << 20
    geom = (4, 128, (("gate", 14336, 4096), ("down", 4096, 14336), ("up", 14336, 4096)))
    buf = torch.zeros(64, dtype=torch.int64, device="cuda")
    n_pairs = (4 << 20) // (14336 * 2) + 1
    rc = lib.vaayu_decode_noalloc(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), 2,
                                  buf.data_ptr(), n_pairs, _lib.geom_struct(geom), 0, 1, 0,
                                  _lib.stream_ptr(buf.device))
    assert rc == -3 and b"4 MiB" in lib.vaayu_last_error()
