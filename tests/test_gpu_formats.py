"""The decode kernels on FP8 (e4m3, 128 x 128 fp32 block scales) and MXFP4 (e2m1, E8M0 per
32) expert blobs, held to the oracle: the dequantized weights are the reference's
(`dequantize_block_scaled`, `upcast_from_mxfp_torch`), every stage rounds where the stock
loop rounds, the sum over pairs is exact in table order, and the layer output is within
the stated tolerance (relL2 5e-3, max-abs 2e-2)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.packed_expert_kernels as pk
from oracle import oracle as O
from tests.helpers import format_case, frac_equal, rel

pytestmark = pytest.mark.gpu
FORMATS = ["e4m3", "mxfp4"]
SHAPES = [pytest.param(2048, 768, 8, id="qwen3-30b-a3b"), pytest.param(1024, 512, 4, id="toy"),
          pytest.param(4096, 1536, 2, id="h4096-i1536-top2")]


def _sc(blob):
    return pk._SCALE_CODE[blob["flat"]["scale"].dtype]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("hid,inter,k", SHAPES)
def test_each_rounding_point_matches_the_oracle(fmt, hid, inter, k):
    x, pairs, w, cpairs = format_case(fmt, hid, inter, k)
    geom, sc = pairs[0][0]["geom"], _sc(pairs[0][0])
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    h = pk._gate_up(x, tbl, len(pairs), geom, sc)
    torch.cuda.synchronize()
    stages = [O.expert_stages(O.to_np(x), blob, "bf16") for blob, _s in cpairs]
    assert frac_equal(h, np.concatenate([s[0] for s in stages])) >= 0.99
    one = torch.ones(1, device="cuda")
    for (blob, _s), (sh, sy) in zip(pairs, stages):
        t1 = pk._TABLES.put(pk._table_values([(blob, 0)]), x.device)
        out = torch.empty(1, hid, device="cuda")
        pk._down(torch.from_numpy(sh).to(torch.bfloat16).cuda(), t1, one, out, 1, geom, sc)
        torch.cuda.synchronize()
        assert frac_equal(out, sy) >= 0.99


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16], ids=["fp32-w", "bf16-w"])
def test_layer_within_tolerance_and_summed_in_table_order(fmt, w_dtype):
    x, pairs, w, cpairs = format_case(fmt, 2048, 768, 8, w_dtype=w_dtype)
    out = torch.full((1, 2048), float("nan"), device="cuda")
    pk._launch(x, pairs, w, out)
    torch.cuda.synchronize()
    ref = O.stock_decode(x, cpairs, w)
    got = out.cpu().numpy()
    assert O.rel_l2(got, ref) <= 5e-3 and np.abs(got - ref).max() <= 2e-2
    # exact table-order sum of the kernel's own per-pair contributions
    geom, sc = pairs[0][0]["geom"], _sc(pairs[0][0])
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    h = pk._gate_up(x, tbl, len(pairs), geom, sc)
    exp = torch.zeros(1, 2048, device="cuda")
    for i, (blob, slot) in enumerate(pairs):
        t1 = pk._TABLES.put(pk._table_values([(blob, 0)]), x.device)
        o = torch.empty(1, 2048, device="cuda")
        pk._down(h[i:i + 1], t1, torch.ones(1, device="cuda"), o, 1, geom, sc)
        exp += (o.to(torch.bfloat16) * w.reshape(-1)[slot:slot + 1]).float()
    torch.cuda.synchronize()
    assert torch.equal(out, exp)


@pytest.mark.parametrize("fmt", FORMATS)
def test_fp16_activations(fmt):
    x, pairs, w, cpairs = format_case(fmt, 1024, 512, 4, act=torch.float16)
    out = torch.empty(1, 1024, device="cuda")
    pk._launch(x, pairs, w, out)
    torch.cuda.synchronize()
    ref = O.stock_decode(x, cpairs, w, act="fp16")
    assert rel(out, ref) <= 5e-3


@pytest.mark.parametrize("fmt", FORMATS)
def test_the_public_entry_and_its_graph_use_the_kernels(fmt):
    x, pairs, w, cpairs = format_case(fmt, 2048, 768, 8)
    out = torch.empty(1, 2048, device="cuda")
    pk.packed_experts_decode(x, pairs, w, out, F.silu)
    key = (pairs[0][0]["geom"], x.dtype, w.dtype, pairs[0][0]["flat"]["scale"].dtype)
    assert pk._VERDICTS.get(key) is True
    ref = O.stock_decode(x, cpairs, w)
    assert O.rel_l2(out.cpu().numpy(), ref) <= 5e-3
    layer = 900 + len(fmt)
    results = [pk.packed_experts_decode_graphed(layer, x, pairs, w, None, F.silu, tail=False)
               for _ in range(3)]
    torch.cuda.synchronize()
    for r in results:
        assert r is not None and torch.equal(r, out)


def test_unsupported_format_blobs_fall_back_loudly(capsys):
    x, pairs, w, _c = format_case("e4m3", 1024, 512, 4)
    bad = [({"flat": b["flat"], "geom": ("e5m2", (128, 128), b["geom"][2])}, s) for b, s in pairs]
    assert pk._unsupported(bad[0][0]["geom"], x.dtype, torch.float32, w.dtype) is not None
