"""The grouped prefill kernels (HIP MFMA, gfx950) against the oracle.

Ports the reference's tests/test_packed_prefill_kernels.py with the CPU oracle's
correctly rounded replay as the truth: per-stage rounding, the exact contribution and
expert-id-order sum, batch invariance, block boundaries, padding, strided views, NaN
isolation, freed blobs, verdicts.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.packed_expert_kernels as pk
from oracle import oracle as O
from tests.helpers import frac_equal, gpu_blobs, prefill_case, rel

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
GEOMS = [
    pytest.param(2048, 512, 4, 32, id="qwen3next-int4-g32"),
    pytest.param(3072, 1536, 8, 128, id="minimax-dims-int8-g128"),
    pytest.param(1024, 512, 8, 64, id="int8-g64"),
    pytest.param(2048, 768, 4, 128, id="qwen3-30b-a3b-int4-g128"),
]
QWEN = (2048, 512, 4, 32)


def _launch(x, eidx, w, blobs):
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk._prefill_launch(x, eidx, w, blobs, out)
    torch.cuda.synchronize()
    return out


def _stock(x, eidx, w, blobs, linear=F.linear):
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk.stock_experts_prefill(x, eidx, w, blobs, out, F.silu, linear=linear)
    return out


def _prefill(x, eidx, w, blobs):
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk.packed_experts_prefill(x, eidx, w, blobs, out, F.silu)
    torch.cuda.synchronize()
    return out


def _stages(x, eidx, w, blobs, h=None, y=None):
    plan = pk._prefill_plan(eidx)
    blob = blobs[int(plan[1][0])]
    geom, sc = blob["geom"], pk._DTYPE_CODE[blob["flat"]["scale"].dtype]
    top_k = eidx.shape[1]
    tbl, rows, order, n_blocks = pk._prefill_tables(eidx, plan, blobs, x.device)
    h = pk._gate_up_g(x, tbl, rows, n_blocks, top_k, geom, sc, h=h)
    y = pk._down_g(h, tbl, rows, n_blocks, w, geom, sc, y=y)
    torch.cuda.synchronize()
    return h, y, order, plan


@pytest.mark.parametrize("hid,inter,bits,gs", GEOMS)
def test_each_stage_is_correctly_rounded(hid, inter, bits, gs):
    """h vs the oracle's correctly rounded stages; y (weight 1) vs the oracle's rounded
    down output of the kernel's own h: >= 99 % bit-equal each."""
    x, eidx, w, blobs, cblobs = prefill_case(hid, inter, bits, gs)
    h, y, _order, _plan = _stages(x, eidx, torch.ones_like(w), blobs)
    want_h, _y = O.prefill_stages(x, eidx, cblobs)
    assert frac_equal(h, want_h) >= 0.99, "gate/up/SiLU/product stage"
    # down of the kernel's own h, correctly rounded
    hv = O.to_np(h)
    e = eidx.reshape(-1).numpy()
    want_y = np.empty((e.size, hid), np.float32)
    for ex in np.unique(e):
        rows = np.nonzero(e == ex)[0]
        _wg, wd, _wu = O.expert_weights(cblobs[int(ex)], "bf16")
        want_y[rows] = O._linear(hv[rows], wd, "bf16")
    assert frac_equal(y, want_y) >= 0.99, "down stage"


@pytest.mark.parametrize("w_dtype", [torch.float32, BF], ids=["fp32-w", "bf16-w"])
def test_the_contribution_is_the_rounded_down_output_times_its_weight(w_dtype):
    x, eidx, w, blobs, _c = prefill_case(*QWEN, w_dtype=w_dtype)
    _h, down, _o, _p = _stages(x, eidx, torch.ones_like(w), blobs)
    _h, y, _o, _p = _stages(x, eidx, w, blobs)
    assert torch.equal(y, (down.to(BF) * w.reshape(-1, 1)).float())


@pytest.mark.parametrize("hid,inter,bits,gs", GEOMS)
def test_the_token_sum_runs_in_expert_id_order(hid, inter, bits, gs):
    x, eidx, w, blobs, _c = prefill_case(hid, inter, bits, gs)
    _h, y, order, plan = _stages(x, eidx, w, blobs)
    out = torch.full(x.shape, float("nan"), device="cuda")
    pk._reduce(y, order, out, eidx.shape[1])
    torch.cuda.synchronize()
    want = O.reduce_in_order(O.to_np(y), O.to_np(order), x.shape[0], eidx.shape[1])
    assert np.array_equal(O.to_np(out), want)


@pytest.mark.parametrize("tokens,top_k", [(3, 10), (8, 8), (5, 17), (600, 10)],
                         ids=["few-tokens-k10", "b8-k8", "few-tokens-k17", "many-tokens-k10"])
def test_the_token_sum_is_exact_for_any_slot_count(tokens, top_k):
    """The reduce alone, on small and large grids and top_k above eight: bit-equal to the
    sequential sum in `ord` order, values spread over many binades so order matters."""
    hid = 1024
    g = torch.Generator().manual_seed(tokens * 31 + top_k)
    y = (torch.randn(tokens * top_k, hid, generator=g)
         * torch.exp2(torch.randint(-20, 20, (tokens * top_k, 1), generator=g).float()))
    order = torch.stack([torch.randperm(tokens * top_k, generator=g)[:top_k]
                         for _ in range(tokens)])
    out = torch.full((tokens, hid), float("nan"), device="cuda")
    pk._reduce(y.cuda(), order.cuda(), out, top_k)
    torch.cuda.synchronize()
    want = O.reduce_in_order(y.numpy(), order.numpy(), tokens, top_k)
    assert np.array_equal(O.to_np(out), want)


@pytest.mark.parametrize("hid,inter,bits,gs", GEOMS)
def test_kernel_output_is_as_accurate_as_the_stock_arithmetic(hid, inter, bits, gs):
    x, eidx, w, blobs, cblobs = prefill_case(hid, inter, bits, gs)
    got = _launch(x, eidx, w, blobs)
    precise = O.stock_prefill(x, eidx, w, cblobs)
    assert rel(got, precise) <= 2e-3, f"relL2 vs the oracle {rel(got, precise):.2e}"
    assert np.abs(O.to_np(got) - precise).max() <= 2e-2
    assert rel(got, _stock(x, eidx, w, blobs)) <= 1e-2


def test_a_token_does_not_depend_on_the_tokens_it_shares_a_call_with():
    x, eidx, w, blobs, _c = prefill_case(*QWEN, tokens=40)
    full = _launch(x, eidx, w, blobs)
    for t in (0, 17, 39):
        alone = _launch(x[t:t + 1], eidx[t:t + 1], w[t:t + 1], blobs)
        assert torch.equal(alone[0], full[t]), f"token {t}"


def test_every_run_length_gives_the_same_bits(monkeypatch):
    """h and y do not depend on how an expert's blocks are cut into runs (runs of 1 to 16
    blocks for gate/up; down's kernel for runs of up to 8 and the one for up to 16): every
    row takes the same MFMAs in the same order."""
    x, eidx, w, blobs, _c = prefill_case(*QWEN, n_exp=3, tokens=300, top_k=2)
    assert int(pk._prefill_plan(eidx)[2].max()) > 12 * 16, "premise: experts of > 12 blocks"
    outs = {}
    for r_gu, r_dn in ((8, 8), (16, 16), (16, 1), (4, 16), (1, 2), (3, 11)):
        monkeypatch.setattr(pk, "_run_length",
                            lambda blocks, run, n_tiles, n_cus, r=r_gu: min(run, r))
        monkeypatch.setattr(pk, "_down_run",
                            lambda blocks, n_tiles, n_cus, k=0, r=r_dn: min(r, max(blocks)))
        h, y, _o, _p = _stages(x, eidx, w, blobs)
        outs[(r_gu, r_dn)] = (h.clone(), y.clone())
    h0, y0 = outs[(8, 8)]
    for key, (h, y) in outs.items():
        assert torch.equal(h, h0), f"h, runs {key}"
        assert torch.equal(y, y0), f"y, runs {key}"


def test_block_boundaries():
    counts = {1: 1, 4: 16, 7: 17, 10: 40}
    slots = [e for e, c in counts.items() for _ in range(c)]
    filler = [13, 16, 19, 22]
    eidx = torch.tensor([[e, filler[i % 4]] for i, e in enumerate(slots)])
    x, eidx, w, blobs, cblobs = prefill_case(*QWEN, top_k=2, eidx=eidx)
    plan = pk._prefill_plan(eidx)
    assert [int(c) for c in plan[2][:4]] == [1, 16, 17, 40]
    full = _launch(x, eidx, w, blobs)
    assert not torch.isnan(full).any()
    for t in (0, 1, 16, 17, 33, 34, 73):
        alone = _launch(x[t:t + 1], eidx[t:t + 1], w[t:t + 1], blobs)
        assert torch.equal(alone[0], full[t]), f"token {t}"
    assert rel(full, O.stock_prefill(x, eidx, w, cblobs)) <= 2e-3


def test_padding_rows_are_never_written():
    x, eidx, w, blobs, _c = prefill_case(*QWEN, tokens=5, top_k=3)
    n, inter, hid = eidx.numel(), QWEN[1], QWEN[0]
    h_big = torch.full((n + 2, inter), 7.0, dtype=BF, device="cuda")
    y_big = torch.full((n + 2, hid), 7.0, device="cuda")
    _stages(x, eidx, w, blobs, h=h_big[1:n + 1], y=y_big[1:n + 1])
    for big in (h_big, y_big):
        assert (big[0] == 7.0).all() and (big[-1] == 7.0).all(), "a guard row was written"
        assert not (big[1:n + 1] == 7.0).all(dim=1).any(), "a live row was not written"


def test_the_output_does_not_depend_on_where_the_blobs_live_or_their_order():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    moved = {e: {"flat": {n: t.clone() for n, t in b["flat"].items()}, "geom": b["geom"]}
             for e, b in reversed(list(blobs.items()))}
    assert torch.equal(_launch(x, eidx, w, blobs), _launch(x, eidx, w, moved))


def test_a_zero_weight_duplicate_slot_changes_nothing():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    eidx2 = torch.cat([eidx, eidx[:, :1]], dim=1)
    w2 = torch.cat([w, torch.zeros_like(w[:, :1])], dim=1)
    assert torch.equal(_launch(x, eidx, w, blobs), _launch(x, eidx2, w2, blobs))


def test_one_token():
    x, eidx, w, blobs, cblobs = prefill_case(*QWEN, tokens=1)
    assert rel(_launch(x, eidx, w, blobs), O.stock_prefill(x, eidx, w, cblobs)) <= 2e-3


def test_a_nan_token_poisons_its_own_row_and_no_other():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    clean = _launch(x, eidx, w, blobs)
    x = x.clone()
    x[0, 5] = float("nan")
    got = _launch(x, eidx, w, blobs)
    assert torch.isnan(got[0]).all()
    assert torch.equal(got[1:], clean[1:])


def test_a_strided_view_of_the_activations_is_read_as_what_it_holds():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    wide = torch.zeros(2 * x.shape[0], x.shape[1], dtype=BF, device="cuda")
    wide[::2] = x
    view = wide[::2]
    assert not view.is_contiguous()
    assert torch.equal(_launch(view, eidx, w, blobs), _launch(x, eidx, w, blobs))


def test_the_blobs_may_be_freed_as_soon_as_the_launch_returns():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    expected = _launch(x, eidx, w, blobs)
    mine = {e: {"flat": {n: t.clone() for n, t in b["flat"].items()}, "geom": b["geom"]}
            for e, b in blobs.items()}
    sizes = [(t.shape, t.dtype) for b in mine.values() for t in b["flat"].values()]
    out = torch.empty(x.shape, device="cuda")
    pk._prefill_launch(x, eidx, w, mine, out)
    del mine
    junk = [torch.zeros(shape, dtype=dtype, device="cuda") for shape, dtype in sizes]
    torch.cuda.synchronize()
    assert torch.equal(out, expected)
    assert len(junk) == len(sizes)


def test_two_geometries_get_two_verdicts(monkeypatch):
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})
    for geom in (QWEN, (1024, 512, 8, 64)):
        x, eidx, w, blobs, cblobs = prefill_case(*geom)
        assert rel(_prefill(x, eidx, w, blobs), O.stock_prefill(x, eidx, w, cblobs)) <= 2e-3
    assert len(pk._PF_VERDICTS) == 2 and all(pk._PF_VERDICTS.values())


def test_back_to_back_calls_do_not_share_a_table():
    cases = [prefill_case(*QWEN, tokens=5 + 3 * s, seed=s)
             for s in range(3 * len(pk._PF_TABLES._slots))]
    outs = []
    for x, eidx, w, blobs, _c in cases:
        out = torch.empty(x.shape, device="cuda")
        pk._prefill_launch(x, eidx, w, blobs, out)
        outs.append(out)
    torch.cuda.synchronize()
    for (x, eidx, w, blobs, _c), out in zip(cases, outs):
        assert torch.equal(out, _launch(x, eidx, w, blobs))


def test_prefill_uses_the_kernels_when_they_agree(monkeypatch):
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    assert torch.equal(_prefill(x, eidx, w, blobs), _launch(x, eidx, w, blobs))
    assert list(pk._PF_VERDICTS.values()) == [True]


def test_a_wrong_kernel_is_refused_loudly(monkeypatch, capsys):
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})
    monkeypatch.setattr(pk, "_prefill_launch", lambda x, e, w, b, out, plan=None: out.zero_())
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    got = _prefill(x, eidx, w, blobs)
    assert "WARNING" in capsys.readouterr().out
    assert torch.equal(got, _stock(x, eidx, w, blobs))


def test_a_geometry_with_no_matrix_core_tile_stays_on_the_stock_loop(monkeypatch, capsys):
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})
    x, eidx, w, blobs, _c = prefill_case(64, 64, 4, 32, n_exp=8, top_k=2)
    got = _prefill(x, eidx, w, blobs)
    out = capsys.readouterr().out
    assert "WARNING" in out and "K tile" in out
    assert torch.equal(got, _stock(x, eidx, w, blobs))


def test_a_call_the_kernels_cannot_take_runs_the_stock_arithmetic(monkeypatch, capsys):
    from vaayu_amd.moe_patch import expert_weights_from_entry
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    first = int(eidx[0, 0])
    dense = {"dense": dict(zip(("gate", "down", "up"),
                               expert_weights_from_entry(blobs[first], BF)))}
    other = gpu_blobs(2048, 512, 4, 64, 1)[0]
    missing = {e: b for e, b in blobs.items() if e != first}
    for mixed in ({**blobs, first: dense}, {**blobs, first: other}, missing):
        assert torch.equal(_prefill(x, eidx, w, mixed), _stock(x, eidx, w, mixed))
    assert "WARNING" not in capsys.readouterr().out
    assert pk._PF_VERDICTS == {}


def test_a_strided_view_of_the_output_is_written_as_what_it_holds():
    x, eidx, w, blobs, _c = prefill_case(*QWEN)
    dense = _launch(x, eidx, w, blobs)
    wide = torch.full((2 * x.shape[0], x.shape[1]), 7.0, device="cuda")
    view = wide[::2]
    pk._prefill_launch(x, eidx, w, blobs, view)
    torch.cuda.synchronize()
    assert torch.equal(view, dense)
    assert (wide[1::2] == 7.0).all()


def test_a_strided_view_of_the_routing_weights_is_read_as_what_it_holds():
    x, eidx, w, blobs, _c = prefill_case(*QWEN, top_k=1, tokens=20)
    wide = torch.zeros(w.shape[0], 3, device="cuda")
    wide[:, 1:2] = w
    view = wide[:, 1:2]
    assert not view.reshape(-1).is_contiguous()
    assert torch.equal(_launch(x, eidx, view, blobs), _launch(x, eidx, w, blobs))


def test_fp16_activations():
    x, eidx, w, blobs, cblobs = prefill_case(1024, 512, 4, 32, act=torch.float16,
                                             scale_dtype=torch.float16)
    got = _launch(x, eidx, w, blobs)
    assert rel(got, O.stock_prefill(x, eidx, w, cblobs, act="fp16")) <= 2e-3


def test_a_call_split_into_token_chunks_gives_the_same_bits(monkeypatch):
    """With the offset limit lowered to 512 KiB `_prefill_launch` runs the call in token
    chunks (25 tokens each); each token's output equals the one-launch call's bit for bit (batch
    invariance), and the chunks cover the call in order."""
    x, eidx, w, blobs, _c = prefill_case(*QWEN, tokens=300, top_k=6)
    whole = _launch(x, eidx, w, blobs)
    monkeypatch.setattr(pk, "_OFFSET_LIMIT", 512 << 10)
    step = pk._tokens_per_launch(QWEN[0], QWEN[1], 6, len(set(eidx.reshape(-1).tolist())))
    assert step * 3 < 300, "premise: the lowered limit splits the call"
    parts = []
    real = pk._prefill_call
    monkeypatch.setattr(pk, "_prefill_call",
                        lambda x_, e_, w_, b_, o_, p_: (parts.append(x_.shape[0]),
                                                        real(x_, e_, w_, b_, o_, p_)))
    split = _launch(x, eidx, w, blobs)
    assert len(parts) == -(-300 // step) and sum(parts) == 300
    assert torch.equal(split, whole)


def test_the_library_refuses_a_launch_past_its_offset_range():
    """A launch whose tables could hold rows past the 32-bit offset range returns an error
    before anything is launched (the check reads only the sizes)."""
    lib = pk._require_backend()
    from vaayu_amd import _lib
    blob = gpu_blobs(*QWEN, 1)[0]
    g = _lib.geom_struct(blob["geom"])
    buf = torch.zeros(64, dtype=torch.int64, device="cuda")
    huge = (0xF0000000 // (2 * QWEN[1])) // 16 + 1                 # h rows one block past
    rc = lib.vaayu_prefill_down(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                                0, 8, buf.data_ptr(), 2, buf.data_ptr(), huge, g, 0, 0, 0,
                                _lib.stream_ptr(buf.device))
    assert rc != 0 and b"32-bit offset" in lib.vaayu_last_error()
    tokens_over = (0xF0000000 // (2 * QWEN[0])) + 1                 # x rows one token past
    rc = lib.vaayu_prefill_gate_up(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                                   buf.data_ptr(), 0, 16, buf.data_ptr(), -(-tokens_over // 16), 1,
                                   g, 0, 0, _lib.stream_ptr(buf.device))
    assert rc != 0 and b"32-bit offset" in lib.vaayu_last_error()
    torch.cuda.synchronize()


def test_work_entries_that_do_not_fit_the_table_compute_nothing():
    """The kernels check each work-list entry against the table: a run that reaches past
    the table's last block, one longer than the launched kernel's run length, and a
    negative entry compute nothing, while the valid entries' rows come out as from the
    host's own list."""
    from vaayu_amd import _lib
    lib = pk._require_backend()
    x, eidx, w, blobs, _c = prefill_case(*QWEN, n_exp=3, tokens=200, top_k=2)
    plan = pk._prefill_plan(eidx)
    blob = blobs[int(plan[1][0])]
    geom, sc = blob["geom"], pk._DTYPE_CODE[blob["flat"]["scale"].dtype]
    tbl, rows, _order, n_blocks = pk._prefill_tables(eidx, plan, blobs, x.device)
    ref = pk._gate_up_g(x, tbl, rows, n_blocks, 2, geom, sc).clone()
    first_blocks = int((plan[2][0] + 15) // 16)        # the first expert's blocks: 0 ..
    assert 4 < first_blocks < n_blocks
    entries = [f * 32 + min(4, first_blocks - f) for f in range(0, first_blocks, 4)]
    entries += [(n_blocks - 2) * 32 + 3,                # reaches past the last block
                first_blocks * 32 + 9,                  # longer than the kernel's 4
                -7]
    n_slots = -(-len(entries) // 8)
    bad = torch.full((n_slots * 8,), -1, dtype=torch.int64)
    bad[:len(entries)] = torch.tensor(entries, dtype=torch.int64)
    bad = bad.to(x.device)
    sentinel = torch.tensor(1234.0, dtype=torch.bfloat16)
    h = torch.full_like(ref, float(sentinel))
    g = _lib.geom_struct(geom)
    rc = lib.vaayu_prefill_gate_up(x.data_ptr(), rows.data_ptr(), tbl.data_ptr(),
                                   bad.data_ptr(), n_slots, 4, h.data_ptr(), n_blocks, 2, g,
                                   pk._DTYPE_CODE[x.dtype], sc, _lib.stream_ptr(x.device))
    assert rc == 0, lib.vaayu_last_error()
    torch.cuda.synchronize()
    mine = rows[:first_blocks * 16]
    mine = mine[mine >= 0]
    assert torch.equal(h[mine], ref[mine])
    others = torch.ones(h.shape[0], dtype=torch.bool, device=h.device)
    others[mine] = False
    assert (h[others] == sentinel.to(h.device)).all()


def test_a_table_without_its_work_lists_gets_them_rebuilt():
    """The reference's call sequence (`_prefill_tables`, then `_gate_up_g` / `_down_g` on
    its tables) finds the work lists on the table; a copy of the table, which does not
    carry them, has them rebuilt from its entries, with the same bits (here with experts
    that share one blob, so consecutive experts have equal table entries)."""
    x, eidx, w, blobs, _c = prefill_case(*QWEN, n_exp=5, tokens=150, top_k=3)
    ids = sorted(blobs)
    blobs = {e: blobs[ids[2 * (i // 2)]] for i, e in enumerate(ids)}   # pairs share a blob
    plan = pk._prefill_plan(eidx)
    blob = blobs[int(plan[1][0])]
    geom, sc = blob["geom"], pk._DTYPE_CODE[blob["flat"]["scale"].dtype]
    tbl, rows, _order, n_blocks = pk._prefill_tables(eidx, plan, blobs, x.device)
    assert getattr(tbl, "vaayu_work", None) is not None
    h = pk._gate_up_g(x, tbl, rows, n_blocks, 3, geom, sc).clone()
    y = pk._down_g(h, tbl, rows, n_blocks, w, geom, sc).clone()
    copy = tbl.clone()
    assert getattr(copy, "vaayu_work", None) is None
    h2 = pk._gate_up_g(x, copy, rows, n_blocks, 3, geom, sc)
    y2 = pk._down_g(h2, copy, rows, n_blocks, w, geom, sc)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(y, y2)
