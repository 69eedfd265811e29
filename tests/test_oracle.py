"""Pins the oracle (oracle/oracle.py) before anything is held to it.

Each check is chosen so a plausible mistake in the oracle -- a dropped rounding point, a
wrong offset or shift, a transposed block scale, a tie broken the wrong way -- fails:
  * library routines it must agree with (torch's bf16 / fp16 / fp8 conversions);
  * a second, independently written C restatement (oracle/cref.c);
  * the reference's own literal expectations and known-answer fixtures;
  * closed forms and brute force on tiny inputs.
"""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import oracle as O
from tests.helpers import cpu_blobs


# ── rounding ────────────────────────────────────────────────────────────────────────────

def _specials():
    v = [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.3895313892515355e38, 3.4e38, -3.4e38,
         1e-40, -1e-40, 1.1754944e-38, 5.877472e-39]
    # exact ties between consecutive bf16 values: 1 + k/256 for odd k
    v += [1.0 + k / 256 for k in range(1, 256, 2)] + [-(2.0 + k / 128) for k in range(1, 64, 2)]
    return np.array(v, dtype=np.float32)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10 ** rng.uniform(
        -30, 30, 100000).astype(np.float32), _specials()])
    a = a.astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_bits(a), want)
    nan = np.array([np.nan], np.float32)
    assert np.isnan(O.bf16_value(O.bf16_bits(nan)))


def test_bf16_rounding_matches_the_c_restatement():
    a = np.concatenate([np.random.default_rng(1).standard_normal(5000).astype(np.float32),
                        _specials()])
    c = np.array([cref.lib().cref_bf16_bits(float(v)) for v in a], np.uint16)
    assert np.array_equal(O.bf16_bits(a), c)


def test_float64_to_bf16_is_correctly_rounded():
    """No double rounding: values just off a bf16 tie in float64 (where float32 would
    first round onto the tie) must go to the nearer bf16 value."""
    rng = np.random.default_rng(2)
    base = rng.standard_normal(20000) * 10 ** rng.uniform(-20, 20, 20000)
    # exact midpoints of bf16 neighbours, nudged by far less than a float32 ulp
    bits = O.bf16_bits(base.astype(np.float32))
    lo = O.bf16_value(bits).astype(np.float64)
    hi = O.bf16_value((bits + 1).astype(np.uint16)).astype(np.float64)
    ok = np.isfinite(lo) & np.isfinite(hi) & (np.abs(lo) > 1e-30)
    mids = ((lo + hi) / 2)[ok]
    nudged = np.concatenate([mids * (1 + 2.0 ** -40), mids * (1 - 2.0 ** -40), base])
    got = O.round_to(nudged, "bf16")
    want = cref.round_act(nudged, "bf16")
    assert np.array_equal(got, want)
    # and the double-rounding trap is real: float32 first would differ somewhere
    assert not np.array_equal(got, O.round_to(nudged.astype(np.float32), "bf16"))


def test_fp16_fp32_rounding_match_the_c_restatement():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(5000) * 10 ** rng.uniform(-8, 5, 5000)
    for act in ("fp16", "fp32"):
        assert np.array_equal(O.round_to(a, act), cref.round_act(a, act)), act


# ── packing ─────────────────────────────────────────────────────────────────────────────

def _python_codes(words, bits, cols):
    """Brute force from the documented layout: a row is a little-endian bit stream."""
    out = []
    for row in words:
        stream = 0
        for i, w in enumerate(row):
            stream |= (int(w) & 0xFFFFFFFF) << (32 * i)
        out.append([((stream >> (j * bits)) & ((1 << bits) - 1)) - (1 << (bits - 1))
                    for j in range(cols)])
    return np.array(out, dtype=np.int64)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_pack_unpack_round_trip_and_bit_layout(bits):
    rng = np.random.default_rng(bits)
    cols = 96
    q = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), (3, cols))
    words = O.pack_to_int32(q, bits)
    assert words.shape == (3, -(-cols * bits // 32))
    assert np.array_equal(O.unpack_int32(words, bits, cols), q)
    assert np.array_equal(_python_codes(words, bits, cols), q)
    u = (q + (1 << (bits - 1))).astype(np.uint64)
    assert np.array_equal(O._pack_bitstream(u, bits, words.shape[1]), words)


def test_the_product_unpack_agrees_with_the_oracle():
    from vaayu_amd.moe_patch import unpack_int32_to_int8
    for bits in (2, 3, 4, 5, 8):
        q = np.random.default_rng(bits).integers(-(1 << (bits - 1)), 1 << (bits - 1), (4, 64))
        words = torch.from_numpy(O.pack_to_int32(q, bits))
        assert torch.equal(unpack_int32_to_int8(words, bits, 64), torch.from_numpy(q).to(torch.int8))


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64), (8, 128)])
def test_quantizer_properties(bits, gs):
    """The repo's quantizer (tests/test_packed_expert_dequant.py:44-57): every code in
    range, each group's largest |w| maps to +-qmax, every unclamped code within half a
    step of w/scale, and the reference test's reconstruction bar."""
    rng = np.random.default_rng(gs + bits)
    w = torch.from_numpy(rng.standard_normal((16, 4 * gs), dtype=np.float32)).to(torch.bfloat16)
    q, s = O.quantize_symmetric(w, bits, gs)
    qmax = 2 ** (bits - 1) - 1
    wf = w.float().numpy().reshape(16, 4, gs)
    qq = q.astype(np.float64).reshape(16, 4, gs)
    assert q.min() >= -qmax - 1 and q.max() <= qmax
    arg = np.abs(wf).argmax(-1)
    top = np.take_along_axis(qq, arg[..., None], -1)[..., 0]
    assert np.array_equal(np.abs(top), np.full_like(top, qmax))
    err = np.abs(wf / s[..., None] - qq)
    assert err.max() <= 0.5 + 1e-6
    recon = (qq * s[..., None]).reshape(16, -1)
    rel = np.linalg.norm(recon - w.float().numpy()) / np.linalg.norm(w.float().numpy())
    assert rel < 0.15


# ── dequant ─────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64), (2, 64)])
@pytest.mark.parametrize("act", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_matches_c_restatement(bits, gs, act, sdt):
    rng = np.random.default_rng(7)
    q = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), (8, 256))
    packed = O.pack_to_int32(q, bits).reshape(-1)
    scale = torch.from_numpy(rng.uniform(1e-3, 3e-2, 8 * 256 // gs).astype(np.float32)).to(sdt)
    got = O.dequant_flat(packed, scale, bits, gs, act)
    want = cref.dequant(packed, O.to_np(scale), bits, gs, act)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64)])
def test_dequant_matches_the_per_role_torch_arithmetic(bits, gs):
    """`dequantize_packed_weight`'s int8 hop (vaayu/moe_patch.py:713-744) on torch CPU --
    a different formulation -- gives the same bf16 bits (the reference asserts this
    bitwise, tests/test_packed_expert_dequant.py:368-381)."""
    (blob,) = cpu_blobs(256, 128, bits, gs, 1)
    flat = O.dequant_flat(blob["flat"]["packed"], blob["flat"]["scale"], bits, gs, "bf16")
    lay = O.layout(blob["geom"])
    for role, (w_at, s_at, rows, cols) in lay.items():
        words = blob["flat"]["packed"][w_at:w_at + rows * cols * bits // 32].reshape(rows, -1)
        sc = blob["flat"]["scale"][s_at:s_at + rows * cols // gs].reshape(rows, -1)
        codes = torch.from_numpy(O.unpack_int32(words.numpy(), bits, cols))
        groups = cols // gs
        dense = (codes.view(rows, groups, gs).to(torch.bfloat16)
                 * sc.view(rows, groups, 1).to(torch.bfloat16)).view(rows, cols)
        start = lay[role][0] * 32 // bits
        assert np.array_equal(flat[start:start + rows * cols], dense.float().numpy().reshape(-1))


def test_the_product_eager_dequant_agrees_with_the_oracle():
    from vaayu_amd.moe_patch import dequantize_expert_blob
    (blob,) = cpu_blobs(256, 128, 4, 32, 1)
    dense = dequantize_expert_blob(blob, torch.bfloat16)
    wg, wd, wu = O.expert_weights(blob, "bf16")
    for t, o in ((dense["gate"], wg), (dense["down"], wd), (dense["up"], wu)):
        assert np.array_equal(t.float().numpy(), o)


def test_layout_literal():
    """tests/test_packed_expert_kernels.py:265-270, verbatim expectations."""
    geom = (4, 32, (("gate", 512, 2048), ("down", 2048, 512), ("up", 512, 2048)))
    lay = O.layout(geom)
    assert lay["gate"] == (0, 0, 512, 2048)
    assert lay["down"] == (512 * 2048 * 4 // 32, 512 * 2048 // 32, 2048, 512)
    assert lay["up"] == (2 * 512 * 2048 * 4 // 32, 2 * 512 * 2048 // 32, 512, 2048)


# ── the stock stages ────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("act", ["bf16", "fp16", "fp32"])
def test_expert_stages_match_the_c_restatement(act):
    (blob,) = cpu_blobs(256, 128, 4, 32, 1)
    x = O.round_to(np.random.default_rng(5).standard_normal((1, 256)) * 0.5, act)
    h, y = O.expert_stages(x, blob, act)
    wg, wd, wu = O.expert_weights(blob, act)
    ch, cy = cref.expert(x, wg, wd, wu, act)
    if act == "fp32":
        # no rounding to hide it: numpy's and libm's expf may differ by an ulp
        assert np.allclose(h[0], ch, rtol=4e-7, atol=0) and np.allclose(y[0], cy, rtol=1e-5)
        return
    assert np.array_equal(h[0], ch)
    assert np.array_equal(y[0], cy)


def test_stock_decode_agrees_with_the_torch_cpu_stock_loop():
    """The reference's own bar for a faithful restatement of the stock loop
    (tests/test_packed_expert_kernels.py:118-168): per stage >= 99 % bit-equal, relL2
    <= 1e-3 overall. With the stage rounding removed the same comparison collapses."""
    hid, inter, k = 512, 256, 6
    blobs = cpu_blobs(hid, inter, 4, 32, k)
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(1, hid, generator=g) * 0.5).to(torch.bfloat16)
    w = torch.rand(1, k, generator=g) + 0.05
    w = w / w.sum(-1, keepdim=True)
    pairs = [(blobs[i], (i * 5) % k) for i in range(k)]
    out = torch.empty(1, hid)
    O.stock_decode_torch(x, pairs, w, out)
    got = O.stock_decode(x, pairs, w)
    assert O.rel_l2(got, out.numpy()) <= 1e-3
    import torch.nn.functional as F
    xv = O.to_np(x)
    for blob, _slot in pairs:
        h, y = O.expert_stages(xv, blob, "bf16")
        wg, wd, wu = O._dequant_torch(blob, torch.bfloat16)
        th = F.silu(F.linear(x, wg)) * F.linear(x, wu)
        ty = F.linear(th, wd)
        assert O.isclose_frac(h, th.float().numpy()) >= 0.99
        assert O.isclose_frac(y, F.linear(torch.from_numpy(h).to(torch.bfloat16), wd)
                              .float().numpy()) >= 0.99
        # premise: a missing rounding point (h left in fp32) is caught by the same bar
        h_unrounded = (O.silu_round(O._linear(xv, O.expert_weights(blob, "bf16")[0], "bf16"),
                                    "fp32") * O._linear(xv, O.expert_weights(blob, "bf16")[2],
                                                        "bf16"))
        assert O.isclose_frac(h_unrounded, th.float().numpy()) < 0.5
        del ty


def test_stock_decode_is_the_table_order_sum_and_close_to_fp64_truth():
    hid, inter, k = 512, 256, 6
    blobs = cpu_blobs(hid, inter, 4, 32, k)
    x = torch.from_numpy(O.round_to(np.random.default_rng(9).standard_normal((1, hid)) * .5,
                                    "bf16")).to(torch.bfloat16)
    w = torch.from_numpy(np.random.default_rng(10).uniform(0.05, 1, (1, k)).astype(np.float32))
    pairs = [(blobs[i], i) for i in range(k)]
    got = O.stock_decode(x, pairs, w)
    acc = np.zeros((1, hid), np.float32)
    for blob, slot in pairs:
        _h, y = O.expert_stages(O.to_np(x), blob, "bf16")
        acc = (acc + (y * w[0, slot].item()).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, acc)
    truth = O.fp64_truth_decode(x, pairs, w)
    assert O.rel_l2(got[0], truth) < 2e-2


def test_bf16_routing_weight_rounds_the_product():
    y = np.array([[1.0 + 2 ** -7]], np.float32)
    w = np.float32(1.0 + 2 ** -7)
    assert O.contribution(y, w, "fp32", "bf16")[0, 0] == np.float32(y[0, 0] * w)
    assert O.contribution(y, w, "bf16", "bf16")[0, 0] == O.round_to(np.float32(y[0, 0] * w), "bf16")


# ── accumulation order (tests/test_expert_accumulation_order.py:24-92) ──────────────────

def test_accumulation_known_answer():
    """{1e8, -1e8, 1.0} from experts 7, 2, 5: in expert-id order the 1.0 is absorbed by
    -1e8 (fp32 spacing 8), so the sum is exactly 0.0; arrival order would give 1.0."""
    c = [(7, [0], [[1e8]]), (2, [0], [[-1e8]]), (5, [0], [[1.0]])]
    results = {float(O.accumulate(np.zeros((1, 1)), list(p))[0, 0]) for p in itertools.permutations(c)}
    assert results == {0.0}
    naive = np.float32(0)
    for _e, _r, v in c:
        naive = np.float32(naive + np.float32(v[0][0]))
    assert naive == 1.0


# ── prefill tables (tests/test_packed_prefill_kernels.py:404-411) ───────────────────────

def test_prefill_plan_literal():
    eidx = np.array([[5, 2], [2, 9], [9, 5]])
    order, live, counts = O.prefill_plan(eidx)
    assert live.tolist() == [2, 5, 9] and counts.tolist() == [2, 2, 2]
    assert order.tolist() == [1, 2, 0, 5, 3, 4]
    _tbl, _rows, slot_order, _n = O.prefill_tables(eidx, (order, live, counts),
                                                   {e: (e, -e) for e in (2, 5, 9)})
    assert slot_order.reshape(3, 2).tolist() == [[1, 0], [2, 3], [5, 4]]


def test_prefill_tables_block_structure():
    counts = {1: 1, 4: 16, 7: 17, 10: 40}
    slots = [e for e, c in counts.items() for _ in range(c)]
    filler = [13, 16, 19, 22]
    eidx = np.array([[e, filler[i % 4]] for i, e in enumerate(slots)])
    plan = O.prefill_plan(eidx)
    assert plan[2][:4].tolist() == [1, 16, 17, 40]
    tbl, rows, _o, n_blocks = O.prefill_tables(eidx, plan, {e: (e, 0) for e in plan[1]})
    assert n_blocks == 1 + 1 + 2 + 3 + sum(-(-int(c) // 16) for c in plan[2][4:])
    rows = rows.reshape(n_blocks, 16)
    for b in range(n_blocks):
        live = rows[b][rows[b] >= 0]
        assert live.size and (np.diff(np.nonzero(rows[b] >= 0)[0]) == 1).all()
        assert len({int(eidx.reshape(-1)[r]) for r in live}) == 1          # one expert
        assert {int(eidx.reshape(-1)[r]) for r in live} == {int(tbl[b][0])}
    assert sorted(rows[rows >= 0].tolist()) == list(range(eidx.size))


def test_stock_prefill_is_the_expert_order_reduce_of_its_stages():
    hid, inter = 256, 128
    blobs = {e: b for e, b in zip((1, 4, 7, 10, 13), cpu_blobs(hid, inter, 4, 32, 5))}
    rng = np.random.default_rng(3)
    eidx = np.stack([rng.permutation([1, 4, 7, 10, 13])[:2] for _ in range(9)])
    x = O.round_to(rng.standard_normal((9, hid)) * 0.5, "bf16")
    w = rng.uniform(0.05, 1, (9, 2)).astype(np.float32)
    got = O.stock_prefill(x, eidx, w, blobs, w_dtype="fp32")
    _h, y = O.prefill_stages(x, eidx, blobs)
    contrib = (y * w.reshape(-1, 1)).astype(np.float32)
    plan = O.prefill_plan(eidx)
    _t, _r, slot_order, _n = O.prefill_tables(eidx, plan, {e: (0, 0) for e in plan[1]})
    assert np.array_equal(got, O.reduce_in_order(contrib, slot_order, 9, 2))


def test_stock_prefill_agrees_with_the_torch_cpu_loop():
    hid, inter = 256, 128
    blobs = {e: b for e, b in zip((1, 4, 7, 10, 13), cpu_blobs(hid, inter, 4, 32, 5))}
    g = torch.Generator().manual_seed(4)
    eidx = torch.stack([torch.tensor([1, 4, 7, 10, 13])[torch.randperm(5, generator=g)[:3]]
                        for _ in range(12)])
    x = (torch.randn(12, hid, generator=g) * 0.5).to(torch.bfloat16)
    w = torch.rand(12, 3, generator=g) + 0.05
    out = torch.empty(12, hid)
    O.stock_prefill_torch(x, eidx, w, blobs, out)
    assert O.rel_l2(O.stock_prefill(x, eidx, w, blobs), out.numpy()) <= 1e-3


# ── routing ─────────────────────────────────────────────────────────────────────────────

def test_softmax_topk_renorm_brute_force_and_ties():
    logits = np.array([[0.5, 2.0, 2.0, -1.0, 0.25], [1.0, 1.0, 1.0, 1.0, 1.0]], np.float32)
    w, idx = O.route_softmax_topk(logits, 3)
    assert idx.tolist() == [[1, 2, 0], [0, 1, 2]]              # ties -> lower expert id
    for r in range(2):
        e = [math.exp(v - max(logits[r])) for v in logits[r]]
        p = [v / sum(e) for v in e]
        top = [p[i] for i in idx[r]]
        assert np.allclose(w[r], [t / sum(top) for t in top], rtol=1e-6)


# truncate_top_k: the reference's known answers (tests/test_decode_top_k.py:393-433) and
# what the definition fixes by brute force over every kept subset.

def test_truncate_cutoff_repoints_dropped_slots_at_the_top1():
    w, i = O.truncate_top_k([[0.5, 0.3, 0.15, 0.05]], [[7, 3, 9, 1]], None, p=0.9)
    assert i.tolist() == [[7, 3, 9, 7]] and w[0, 3] == 0.0
    assert abs(float(w.sum()) - 1.0) < 1e-6


def test_truncate_cutoff_finds_the_top1_by_weight_on_unsorted_routing():
    w, i = O.truncate_top_k([[0.05, 0.5, 0.15, 0.3]], [[1, 7, 9, 3]], None, p=0.9)
    assert i.tolist() == [[7, 7, 9, 3]] and w[0, 0] == 0.0


def test_truncate_cutoff_always_keeps_the_top1():
    w, i = O.truncate_top_k([[0.4, 0.3, 0.2, 0.1]], [[5, 6, 7, 8]], None, p=0.01)
    assert set(i.flatten().tolist()) == {5} and abs(float(w[0, 0]) - 1.0) < 1e-6


def test_truncate_off_path_is_unchanged():
    w = np.random.default_rng(0).random((3, 8)).astype(np.float32)
    w /= w.sum(-1, keepdims=True)
    i = np.arange(24).reshape(3, 8)
    a, b = O.truncate_top_k(w, i, 8, None)
    assert np.array_equal(a, w) and np.array_equal(b, i)


@pytest.mark.parametrize("experts,top_k", [(128, 8), (256, 8), (512, 10)])
def test_truncate_keeps_the_k_largest_renormalised(experts, top_k):
    """tests/test_decode_top_k.py:36-70: the kept experts are the k largest weights, and
    the kept weights sum to the original (unit) sum."""
    rng = np.random.default_rng(experts)
    w, idx = O.route_softmax_topk(rng.standard_normal((7, experts)).astype(np.float32), top_k)
    k = top_k - 2
    wt, it = O.truncate_top_k(w, idx, k)
    assert wt.shape == it.shape == (7, k)
    for r in range(7):
        assert set(it[r].tolist()) == set(idx[r][np.argsort(-w[r], kind="stable")[:k]].tolist())
    assert np.allclose(wt.sum(-1), 1.0, atol=1e-5)


def test_truncate_p_is_the_fewest_slots_reaching_p_brute_force():
    """p keeps the smallest prefix of the weight-sorted slots whose mass reaches p: checked
    against every prefix length, on rows whose cumulative sums are far from p."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        w = rng.random(6).astype(np.float32)
        w /= w.sum()
        idx = rng.permutation(64)[:6]
        p = float(rng.uniform(0.05, 0.95))
        srt = np.sort(w)[::-1]
        if np.min(np.abs(np.cumsum(srt) - p)) < 1e-4:
            continue
        n_keep = next(n for n in range(1, 7) if srt[:n].sum() >= p)
        wt, it = O.truncate_top_k(w[None], idx[None], None, p)
        kept = wt[0] > 0
        assert kept.sum() == n_keep
        assert set(it[0][kept].tolist()) == set(idx[np.argsort(-w)[:n_keep]].tolist())
        assert (it[0][~kept] == idx[np.argmax(w)]).all()
        assert np.isclose(wt[0].sum(), 1.0, atol=1e-6)
        assert np.allclose(wt[0][kept], w[kept] / w[kept].sum(), rtol=1e-5)


def test_truncate_rescales_to_the_original_sum():
    """A row that does not sum to 1 (a scaled router) keeps its sum; one within 1e-2 of 1
    snaps to exactly 1."""
    w = np.array([[0.8, 0.6, 0.4, 0.2]], np.float32)            # sums to 2
    wt, _ = O.truncate_top_k(w, [[0, 1, 2, 3]], 2)
    assert np.allclose(wt, [[0.8 / 1.4 * 2, 0.6 / 1.4 * 2]], rtol=1e-6)
    w = np.array([[0.5, 0.3, 0.1, 0.095]], np.float32)           # sums to 0.995
    wt, _ = O.truncate_top_k(w, [[0, 1, 2, 3]], 2)
    assert np.allclose(wt.sum(), 1.0, atol=1e-7)


def test_host_truncate_matches_the_oracle():
    """The package's host `truncate_top_k` (torch) against the oracle on routed rows."""
    from vaayu_amd.moe_patch import truncate_top_k as host
    rng = np.random.default_rng(5)
    w, idx = O.route_softmax_topk(rng.standard_normal((32, 128)).astype(np.float32), 8)
    for k, p in [(6, None), (None, 0.7), (5, 0.6), (8, 0.5)]:
        hw, hi = host(torch.from_numpy(w), torch.from_numpy(idx), k, p)
        ow, oi = O.truncate_top_k(w, idx, k, p)
        assert np.array_equal(hi.numpy(), oi)
        np.testing.assert_allclose(hw.numpy(), ow, rtol=1e-6, atol=1e-7)


# ── FP8 block-scaled and MXFP4 ──────────────────────────────────────────────────────────

def test_e4m3_exhaustive():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.e4m3_value(codes)
    lib = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    c = np.array([cref.e4m3(int(b)) for b in codes], np.float32)
    same = (ours == lib) | (np.isnan(ours) & np.isnan(lib))
    assert same.all()
    assert ((ours == c) | (np.isnan(ours) & np.isnan(c))).all()


@pytest.mark.parametrize("shape,block", [((256, 512), (128, 128)), ((64, 128), (32, 64))])
def test_block_scaled_dequant_reference_test(shape, block):
    """tests/test_deepseek_v4_linear.py:306-323: scale[i, j] covers the (bo, bi) tile;
    the block shape is read from the two shapes."""
    torch.manual_seed(0)
    weight = torch.randn(*shape).to(torch.float8_e4m3fn)
    scale = torch.randn(shape[0] // block[0], shape[1] // block[1]).exp().to(torch.float8_e8m0fnu)
    got = O.dequant_block_scaled(weight.view(torch.uint8).numpy(), scale.float(), "bf16")
    expanded = scale.float().repeat_interleave(block[0], 0).repeat_interleave(block[1], 1)
    want = (weight.float() * expanded).bfloat16().float().numpy()
    assert np.array_equal(got, want)


def test_e2m1_table_and_mxfp4_upcast_known_answers():
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for n in range(16):
        want = table[n & 7] * (-1 if n & 8 else 1)
        assert O.e2m1_value(n) == want == cref.e2m1(n)
    packed = np.array([[0x21, 0xF7] + [0] * 14], np.uint8)          # 32 elements, one block
    for s, f in ((127, 1.0), (128, 2.0), (120, 2.0 ** -7)):
        v = O.upcast_mxfp4(packed, np.array([[s]], np.uint8), "fp32")
        assert v[0, :4].tolist() == [0.5 * f, 1.0 * f, 6.0 * f, -6.0 * f]
    assert np.isnan(O.upcast_mxfp4(packed, np.array([[255]], np.uint8), "fp32")).all()
    assert not O.upcast_mxfp4(packed, np.array([[0]], np.uint8), "fp32").any()   # s << 23 = 0.0


def test_mx_e4m3_upcast_known_answers():
    codes = np.zeros((1, 32), np.uint8)
    codes[0, :5] = [0x38, 0x40, 0x01, 0xB8, 0x7F]        # 1, 2, 2^-9, -1, NaN
    v = O.upcast_mx_e4m3(codes, np.array([[130]], np.uint8), "fp32")   # x 8
    assert v[0, :4].tolist() == [8.0, 16.0, 2.0 ** -6, -8.0] and np.isnan(v[0, 4])
    assert np.isnan(O.upcast_mx_e4m3(codes, np.array([[255]], np.uint8), "fp32")).all()
    # a bf16 cast that rounds: 1.125 * 2^0 in e4m3 (0x39) is exact in bf16; 0x3F = 1.875
    codes[0, :2] = [0x39, 0x3F]
    assert O.upcast_mx_e4m3(codes, np.array([[127]], np.uint8), "bf16")[0, :2].tolist() == [1.125, 1.875]


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64)])
def test_the_torch_quantizer_matches_the_oracle(bits, gs):
    """vaayu_amd.synth (used to build benchmark experts in HBM) packs the same words and
    scales as the oracle's restatement of the repo's quantizer."""
    from vaayu_amd.synth import quantize_pack
    w = torch.from_numpy(np.random.default_rng(bits * gs).standard_normal((32, 512)).astype(
        np.float32) * 0.02).to(torch.bfloat16)
    words, scale = quantize_pack(w, bits, gs, torch.float16)
    q, s = O.quantize_symmetric(w, bits, gs)
    assert np.array_equal(words.numpy(), O.pack_to_int32(q, bits))
    assert torch.equal(scale, torch.from_numpy(s).to(torch.float16))
