"""The one-token decode kernels (HIP, gfx950) against the oracle and the stock loop.

Ports the reference's kernel tests (tests/test_packed_expert_kernels.py) with the CPU
oracle as the stock arithmetic: per-stage rounding agreement, the exact table-order sum,
accuracy against fp64 truth, independence from blob addresses, zero-weight duplicates,
NaN propagation, verdicts and fallbacks, plus the BASELINE tolerance (max-abs 2e-2,
relL2 5e-3) at the Qwen3-30B-A3B shape.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.packed_expert_kernels as pk
from oracle import oracle as O
from tests.helpers import decode_case, gpu_blobs, frac_equal, rel

pytestmark = pytest.mark.gpu

# (hidden, intermediate, bits, group, top_k)
GEOMS = [
    pytest.param(2048, 512, 4, 32, 10, id="qwen3next-int4-g32"),
    pytest.param(3072, 1536, 4, 128, 8, id="minimax-like-int4-g128"),
    pytest.param(1024, 512, 8, 64, 4, id="int8-g64"),
    pytest.param(2048, 768, 4, 128, 8, id="qwen3-30b-a3b-int4-g128"),
    pytest.param(1024, 512, 4, 128, 4, id="toy-int4-g128"),
]
QWEN = (2048, 512, 4, 32, 10)


def _run(fn, x, pairs, w):
    out = torch.full((1, x.shape[1]), float("nan"), device="cuda")   # must be overwritten
    fn(x, pairs, w, out)
    torch.cuda.synchronize()
    return out


def _stock(x, pairs, w, out):
    pk.stock_experts_decode(x, pairs, w, out, F.silu)


def _decode(x, pairs, w, out):
    pk.packed_experts_decode(x, pairs, w, out, F.silu)


def _one_pair_down(h, blob, w):
    geom, sc = blob["geom"], pk._DTYPE_CODE[blob["flat"]["scale"].dtype]
    tbl = pk._TABLES.put(pk._table_values([(blob, 0)]), h.device)
    out = torch.empty(1, pk._layout(geom)["gate"][3], device="cuda")
    pk._down(h, tbl, w, out, 1, geom, sc)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hid,inter,bits,gs,k", GEOMS)
def test_each_rounding_point_matches_the_oracle(hid, inter, bits, gs, k):
    """Stage by stage: h = round(round(SiLU(round(g))) * round(u)) and the rounded down
    output, >= 99 % bit-equal with the correctly rounded oracle (the reference's bar)."""
    x, pairs, w, cpairs = decode_case(hid, inter, bits, gs, k)
    geom, sc = pairs[0][0]["geom"], pk._DTYPE_CODE[pairs[0][0]["flat"]["scale"].dtype]
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    h = pk._gate_up(x, tbl, len(pairs), geom, sc)
    torch.cuda.synchronize()
    xv = O.to_np(x)
    stages = [O.expert_stages(xv, blob, "bf16") for blob, _s in cpairs]
    want_h = np.concatenate([s[0] for s in stages])
    h_equal = frac_equal(h, want_h)
    assert h_equal >= 0.99, f"gate/up/SiLU/product stage: {h_equal:.4%} bit-equal"
    one = torch.ones(1, device="cuda")
    for (blob, _s), (sh, sy) in zip(pairs, stages):
        got = _one_pair_down(torch.from_numpy(sh).to(torch.bfloat16).cuda(), blob, one)
        assert frac_equal(got, sy) >= 0.99, "down stage"


@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16], ids=["fp32-w", "bf16-w"])
def test_the_expert_sum_runs_in_table_order(w_dtype):
    """EXACT: the output is the fp32 sum, in table order, of each pair's contribution."""
    x, pairs, w, _c = decode_case(*QWEN, w_dtype=w_dtype)
    geom, sc = pairs[0][0]["geom"], pk._DTYPE_CODE[pairs[0][0]["flat"]["scale"].dtype]
    tbl = pk._TABLES.put(pk._table_values(pairs), x.device)
    h = pk._gate_up(x, tbl, len(pairs), geom, sc)
    full = torch.empty(1, x.shape[1], device="cuda")
    pk._down(h, tbl, w, full, len(pairs), geom, sc)
    expected = torch.zeros(1, x.shape[1], device="cuda")
    for i, (blob, slot) in enumerate(pairs):
        weight = w.reshape(-1)[slot:slot + 1]
        o = _one_pair_down(h[i:i + 1], blob, torch.ones(1, device="cuda"))
        expected += (o.to(torch.bfloat16) * weight).float()
    torch.cuda.synchronize()
    assert torch.equal(full, expected)


@pytest.mark.parametrize("hid,inter,bits,gs,k", GEOMS)
def test_kernel_output_is_as_accurate_as_the_stock_arithmetic(hid, inter, bits, gs, k):
    x, pairs, w, cpairs = decode_case(hid, inter, bits, gs, k)
    got = _run(pk._launch, x, pairs, w)
    ref = O.stock_decode(x, cpairs, w)
    truth = O.fp64_truth_decode(x, cpairs, w)
    assert rel(got, ref) <= 1e-3, f"relL2 vs oracle {rel(got, ref):.2e}"
    e_got, e_ref = O.rel_l2(O.to_np(got)[0], truth), O.rel_l2(ref[0], truth)
    assert e_got <= 1.25 * e_ref + 1e-12, f"fp64 error {e_got:.3e} vs stock's {e_ref:.3e}"
    # the stated layer tolerance: max-abs 2e-2, relL2 5e-3 at fp32 accumulate
    assert np.abs(O.to_np(got) - ref).max() <= 2e-2 and rel(got, ref) <= 5e-3
    # and the product's own stock loop on the GPU (hipBLASLt GEMVs) agrees too
    assert rel(got, _run(_stock, x, pairs, w)) <= 1e-3


@pytest.mark.parametrize("act", [torch.float16, torch.float32], ids=["fp16", "fp32"])
def test_other_activation_dtypes(act):
    x, pairs, w, cpairs = decode_case(1024, 512, 4, 32, 4, act=act,
                                      scale_dtype=torch.float16)
    got = _run(pk._launch, x, pairs, w)
    ref = O.stock_decode(x, cpairs, w, act=act)
    assert rel(got, ref) <= 1e-3


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32], ids=["fp16-scale", "fp32-scale"])
def test_scale_dtypes(sdt):
    x, pairs, w, cpairs = decode_case(2048, 768, 4, 128, 8, scale_dtype=sdt)
    got = _run(pk._launch, x, pairs, w)
    assert rel(got, O.stock_decode(x, cpairs, w)) <= 1e-3


def test_bf16_routing_weights_round_like_the_stock_arithmetic():
    x, pairs, w, cpairs = decode_case(*QWEN, w_dtype=torch.bfloat16)
    got = _run(pk._launch, x, pairs, w)
    ref = O.stock_decode(x, cpairs, w)
    assert frac_equal(O.round_to(O.to_np(got), "bf16"), O.round_to(ref, "bf16")) >= 0.99
    assert rel(got, ref) <= 1e-3


def test_the_output_does_not_depend_on_where_the_blobs_live():
    x, pairs, w, _c = decode_case(*QWEN)
    clones = [({"flat": {n: t.clone() for n, t in b["flat"].items()}, "geom": b["geom"]}, s)
              for b, s in pairs]
    assert torch.equal(_run(pk._launch, x, pairs, w), _run(pk._launch, x, clones, w))


def test_a_zero_weight_duplicate_slot_changes_nothing():
    x, pairs, w, _c = decode_case(*QWEN)
    k = w.shape[1]
    w2 = torch.cat([w, torch.zeros(1, 1, dtype=w.dtype, device=w.device)], dim=1)
    dup = pairs[:1] + [(pairs[0][0], k)] + pairs[1:]
    assert torch.equal(_run(pk._launch, x, pairs, w), _run(pk._launch, x, dup, w2))


def test_back_to_back_calls_do_not_share_a_table():
    cases = [decode_case(*QWEN, seed=s) for s in range(3 * len(pk._TABLES._slots))]
    outs = []
    for x, pairs, w, _c in cases:
        out = torch.empty(1, x.shape[1], device="cuda")
        pk._launch(x, pairs, w, out)
        outs.append(out)
    torch.cuda.synchronize()
    for (x, pairs, w, _c), out in zip(cases, outs):
        assert torch.equal(out, _run(pk._launch, x, pairs, w))


def test_decode_uses_the_kernel_when_it_agrees(monkeypatch):
    monkeypatch.setattr(pk, "_VERDICTS", {})
    x, pairs, w, _c = decode_case(*QWEN)
    assert torch.equal(_run(_decode, x, pairs, w), _run(pk._launch, x, pairs, w))
    assert list(pk._VERDICTS.values()) == [True]


def test_the_verdict_is_taken_once_per_geometry(monkeypatch):
    monkeypatch.setattr(pk, "_VERDICTS", {})
    calls = []
    real = pk._verdict
    monkeypatch.setattr(pk, "_verdict", lambda *a: calls.append(1) or real(*a))
    x, pairs, w, _c = decode_case(*QWEN)
    for _ in range(3):
        _run(_decode, x, pairs, w)
    assert len(calls) == 1


def test_two_geometries_get_two_verdicts(monkeypatch):
    monkeypatch.setattr(pk, "_VERDICTS", {})
    for geom in ((2048, 512, 4, 32, 10), (1024, 512, 8, 64, 4)):
        x, pairs, w, cpairs = decode_case(*geom)
        assert rel(_run(_decode, x, pairs, w), O.stock_decode(x, cpairs, w)) <= 1e-3
    assert len(pk._VERDICTS) == 2 and all(pk._VERDICTS.values())


def test_an_unsupported_group_size_stays_on_the_stock_loop(monkeypatch, capsys):
    """Group 48 packs whole int4 words but is not a power of two."""
    monkeypatch.setattr(pk, "_VERDICTS", {})
    x, pairs, w, _c = decode_case(192, 96, 4, 48, 2)
    got = _run(_decode, x, pairs, w)
    assert "WARNING" in capsys.readouterr().out
    assert torch.equal(got, _run(_stock, x, pairs, w))


def test_a_wrong_kernel_is_refused_loudly(monkeypatch, capsys):
    monkeypatch.setattr(pk, "_VERDICTS", {})
    monkeypatch.setattr(pk, "_launch", lambda x, pairs, w, out: out.zero_())
    x, pairs, w, _c = decode_case(*QWEN)
    got = _run(_decode, x, pairs, w)
    assert "WARNING" in capsys.readouterr().out
    assert torch.equal(got, _run(_stock, x, pairs, w))


def test_a_call_that_is_not_all_one_geometry_runs_the_stock_arithmetic(monkeypatch, capsys):
    from vaayu_amd.moe_patch import expert_weights_from_entry
    monkeypatch.setattr(pk, "_VERDICTS", {})
    x, pairs, w, _c = decode_case(*QWEN)
    blob0 = pairs[0][0]
    dense = {"dense": dict(zip(("gate", "down", "up"),
                               expert_weights_from_entry(blob0, x.dtype)))}
    for mixed in ([(dense, pairs[0][1])] + pairs[1:],
                  pairs[:9] + [(gpu_blobs(2048, 512, 4, 64, 1)[0], pairs[9][1])]):
        got = _run(_decode, x, mixed, w)
        assert torch.equal(got, _run(_stock, x, mixed, w))
    assert "WARNING" not in capsys.readouterr().out


def test_a_nan_inside_the_experts_is_not_masked():
    x, pairs, w, _c = decode_case(*QWEN)
    x = x.clone()
    x[0, 5] = float("nan")
    got, ref = _run(pk._launch, x, pairs, w), _run(_stock, x, pairs, w)
    assert torch.isnan(ref).all(), "premise: a NaN input poisons every stock output"
    assert torch.isnan(got).all()


def test_many_pairs_and_repeated_experts():
    """More pairs than the down kernel's waves: 22 slots over 5 experts (duplicates)."""
    blobs = gpu_blobs(2048, 768, 4, 128, 5)
    from tests.helpers import cpu_blobs
    cb = cpu_blobs(2048, 768, 4, 128, 5)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1, 2048, generator=g) * 0.5).to(torch.bfloat16).cuda()
    w = (torch.rand(1, 22, generator=g) + 0.05).cuda()
    idx = sorted([(i % 5, i) for i in range(22)])
    pairs = [(blobs[e], s) for e, s in idx]
    cpairs = [(cb[e], s) for e, s in idx]
    got = _run(pk._launch, x, pairs, w)
    assert rel(got, O.stock_decode(x, cpairs, w)) <= 1e-3
