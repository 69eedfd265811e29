"""The one-launch decode layer (`vaayu_decode_fused`) against the two-launch decode
(`vaayu_decode_gate_up` + `vaayu_decode_down` through `_launch`): the same arithmetic, so
the same bits, at every geometry the decode tests use, over consecutive calls on one sync
buffer; and the bounded wait reporting a sync buffer whose counters cannot be met."""
import pytest
import torch

import vaayu_amd.packed_expert_kernels as pk
from tests.helpers import decode_case, format_case

pytestmark = pytest.mark.gpu

CASES = [
    pytest.param((2048, 768, 4, 128, 8), id="qwen3-30b-a3b-int4-g128"),
    pytest.param((1024, 512, 4, 128, 4), id="toy-int4-g128"),
    pytest.param((2048, 512, 4, 32, 10), id="qwen3next-int4-g32"),
    pytest.param((3072, 1536, 8, 128, 6), id="minimax-dims-int8-g128"),
    pytest.param((7168, 2048, 4, 128, 8), id="dsv3-int4-g128"),
]


def _buffers(x, pairs):
    blob = pairs[0][0]
    words = pk._fused_sync_words(len(pairs), blob["geom"], x.dtype, blob["flat"]["scale"].dtype)
    assert words is not None
    inter = pk._layout(blob["geom"])["gate"][2]
    h = torch.empty(len(pairs), inter, dtype=x.dtype, device=x.device)
    return h, torch.zeros(words, dtype=torch.int32, device=x.device)


def _fused(x, pairs, w, h, sync, max_polls=0):
    blob = pairs[0][0]
    out = torch.full((1, x.shape[1]), float("nan"), device=x.device)
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    pk._fused(x, tbl, len(pairs), blob["geom"], pk._scale_code(blob), w, out, h, sync, max_polls)
    return out


def _eager(x, pairs, w):
    out = torch.full((1, x.shape[1]), float("nan"), device=x.device)
    pk._launch(x, pairs, w, out)
    return out


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16], ids=["fp32-w", "bf16-w"])
def test_one_launch_gives_the_two_launch_bits(case, w_dtype):
    hid, inter, bits, gs, k = case
    print(f"fused decode {case} {w_dtype}", flush=True)
    x, pairs, w, _cpu = decode_case(hid, inter, bits, gs, k, seed=3, w_dtype=w_dtype)
    h, sync = _buffers(x, pairs)
    for call in range(3):               # the counters advance call by call
        got = _fused(x * (call + 1), pairs, w, h, sync)
        want = _eager(x * (call + 1), pairs, w)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}"
    assert int(sync[-1]) == 0
    assert torch.all(sync[:-1] == 3)


@pytest.mark.parametrize("fmt", ["e4m3", "mxfp4"])
def test_fp8_and_mxfp4_blobs(fmt):
    x, pairs, w, _cpu = format_case(fmt, 2048, 768, 8, seed=4)
    h, sync = _buffers(x, pairs)
    for call in range(2):
        got, want = _fused(x, pairs, w, h, sync), _eager(x, pairs, w)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_a_wait_that_cannot_be_met_ends_and_reports():
    """Down workgroups whose own call count is far ahead wait for producer counters that
    never reach it: after the given number of polls they set the sync buffer's last word
    and end."""
    x, pairs, w, _cpu = decode_case(2048, 768, 4, 128, 8, seed=5)
    h, sync = _buffers(x, pairs)
    blob = pairs[0][0]
    producers = (768 // 16) * len(pairs)
    sync[producers:-1] = 100
    _fused(x, pairs, w, h, sync, max_polls=4)
    torch.cuda.synchronize()
    assert int(sync[-1]) == 1
    assert torch.all(sync[:producers] == 1)


def test_unsupported_configurations_say_so():
    lib = pk._require_backend()
    from vaayu_amd import _lib
    geom = (4, 128, (("gate", 768, 2048), ("down", 2048, 768), ("up", 768, 2048)))
    assert lib.vaayu_decode_fused_sync_words(8, _lib.geom_struct(geom), 2, 1) < 0   # fp32 act
    assert lib.vaayu_decode_fused_sync_words(8, _lib.geom_struct(geom), 0, 1) == \
        (768 // 16) * 8 + 2048 // 8 + 1
