"""The grouped prefill kernels on FP8 (e4m3, 128 x 128 fp32 block scales) and MXFP4 (e2m1,
E8M0 per 32) expert blobs, held to the oracle like the integer blobs: each stage rounds
where the stock loop rounds (>= 99 % of h and of the down output bit-equal to the oracle's
correctly rounded replay), each contribution is the rounded down output times its weight,
the token sum runs in expert-id order, and the layer is within relL2 5e-3 / max-abs 2e-2."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.packed_expert_kernels as pk
from oracle import oracle as O
from tests.helpers import format_blobs, frac_equal, rel

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
FORMATS = ["e4m3", "mxfp4"]
SHAPES = [pytest.param(2048, 768, id="qwen3-30b-a3b"), pytest.param(1024, 512, id="toy"),
          pytest.param(4096, 1536, id="h4096-i1536")]


def _case(fmt, hid, inter, *, n_exp=4, tokens=40, top_k=3, seed=0, w_dtype=torch.float32,
          act=BF, std=0.05):
    """(x, eidx, w, blobs_gpu, blobs_cpu): tokens each routed to top_k distinct experts of
    n_exp distinct blobs of N(0, std) weights, ids 3i+1 (so ids are not table positions)."""
    base = format_blobs(fmt, hid, inter, n_exp, "cuda", std)
    cbase = format_blobs(fmt, hid, inter, n_exp, "cpu", std)
    ids = [3 * i + 1 for i in range(n_exp)]
    blobs = {e: base[i] for i, e in enumerate(ids)}
    cblobs = {e: cbase[i] for i, e in enumerate(ids)}
    g = torch.Generator().manual_seed(seed)
    eidx = torch.stack([torch.tensor(ids)[torch.randperm(n_exp, generator=g)[:top_k]]
                        for _ in range(tokens)])
    x = (torch.randn(tokens, hid, generator=g) * 0.5).to(act)
    w = torch.rand(eidx.shape, generator=g) + 0.05
    w = (w / w.sum(-1, keepdim=True)).to(w_dtype)
    return x.cuda(), eidx, w.cuda(), blobs, cblobs


def _stages(x, eidx, w, blobs):
    plan = pk._prefill_plan(eidx)
    blob = blobs[int(plan[1][0])]
    geom, sc = blob["geom"], pk._SCALE_CODE[blob["flat"]["scale"].dtype]
    tbl, rows, order, n_blocks = pk._prefill_tables(eidx, plan, blobs, x.device)
    h = pk._gate_up_g(x, tbl, rows, n_blocks, eidx.shape[1], geom, sc)
    y = pk._down_g(h, tbl, rows, n_blocks, w, geom, sc)
    torch.cuda.synchronize()
    return h, y, order


def _launch(x, eidx, w, blobs):
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk._prefill_launch(x, eidx, w, blobs, out)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("hid,inter", SHAPES)
def test_each_stage_is_correctly_rounded(fmt, hid, inter):
    x, eidx, w, blobs, cblobs = _case(fmt, hid, inter)
    h, y, _order = _stages(x, eidx, torch.ones_like(w), blobs)
    want_h, _y = O.prefill_stages(x, eidx, cblobs)
    assert frac_equal(h, want_h) >= 0.99, "gate/up/SiLU/product stage"
    hv = O.to_np(h)
    e = eidx.reshape(-1).numpy()
    want_y = np.empty((e.size, hid), np.float32)
    for ex in np.unique(e):
        rows = np.nonzero(e == ex)[0]
        _wg, wd, _wu = O.expert_weights(cblobs[int(ex)], "bf16")
        want_y[rows] = O._linear(hv[rows], wd, "bf16")
    assert frac_equal(y, want_y) >= 0.99, "down stage"


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("w_dtype", [torch.float32, BF], ids=["fp32-w", "bf16-w"])
def test_contributions_and_the_expert_id_order_sum(fmt, w_dtype):
    x, eidx, w, blobs, _c = _case(fmt, 2048, 768, w_dtype=w_dtype)
    _h, down, _o = _stages(x, eidx, torch.ones_like(w), blobs)
    _h, y, order = _stages(x, eidx, w, blobs)
    assert torch.equal(y, (down.to(BF) * w.reshape(-1, 1)).float())
    out = _launch(x, eidx, w, blobs)
    o = order.cpu().reshape(eidx.shape)
    want = torch.zeros_like(out)
    for k in range(eidx.shape[1]):
        want += y[o[:, k]]
    assert torch.equal(out, want)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("hid,inter", SHAPES)
def test_layer_within_tolerance(fmt, hid, inter):
    """The stated tolerance at realistic magnitudes: weights N(0, 0.02), as in models of these
    widths, so the outputs are O(1) and a one-ulp bf16 flip of an intermediate (the only
    difference fp32 accumulation leaves) stays under the 2e-2 absolute bound."""
    x, eidx, w, blobs, cblobs = _case(fmt, hid, inter, tokens=56, std=0.02)
    got = _launch(x, eidx, w, blobs)
    ref = O.stock_prefill(x, eidx, w, cblobs)
    assert O.rel_l2(O.to_np(got), ref) <= 5e-3
    assert np.abs(O.to_np(got) - ref).max() <= 2e-2


@pytest.mark.parametrize("fmt", FORMATS)
def test_fp16_activations(fmt):
    x, eidx, w, blobs, cblobs = _case(fmt, 1024, 512, act=torch.float16)
    got = _launch(x, eidx, w, blobs)
    ref = O.stock_prefill(x, eidx, w, cblobs, act="fp16")
    assert rel(got, ref) <= 5e-3


@pytest.mark.parametrize("fmt", FORMATS)
def test_rows_are_batch_invariant(fmt):
    """A token's output does not depend on which other tokens share its blocks."""
    x, eidx, w, blobs, _c = _case(fmt, 1024, 512, tokens=48)
    full = _launch(x, eidx, w, blobs)
    half = _launch(x[:17].contiguous(), eidx[:17], w[:17].contiguous(), blobs)
    assert torch.equal(full[:17], half)


@pytest.mark.parametrize("fmt", FORMATS)
def test_the_public_entry_uses_the_kernels(fmt):
    x, eidx, w, blobs, _c = _case(fmt, 2048, 768)
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk.packed_experts_prefill(x, eidx, w, blobs, out, F.silu)
    torch.cuda.synchronize()
    blob = next(iter(blobs.values()))
    key = (blob["geom"], x.dtype, w.dtype, blob["flat"]["scale"].dtype)
    assert pk._PF_VERDICTS[key] is True
    assert torch.equal(out, _launch(x, eidx, w, blobs))
