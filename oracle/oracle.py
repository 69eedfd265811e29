"""CPU restatement of Vaayu's packed-expert routed-MoE arithmetic -- the oracle.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the checker the HIP path is held to,
never a product path.

Every function cites the reference file:line whose arithmetic it restates. The float
stages are computed the way the reference's stock loop defines them -- every value that
the stock path stores in the activation dtype is rounded (nearest-even) to it, once --
with each GEMV/GEMM summed in float64 and rounded ONCE (a correctly-rounded replay, the
reference's own test truth: tests/test_packed_prefill_kernels.py:115-134). Integer and
byte work (pack, unpack, tables, routing order) is exact numpy.

Pinning (what checks this file, so a plausible mistake fails a test): tests/test_oracle.py.
"""
from __future__ import annotations

import math

import numpy as np
import torch

ACTS = ("bf16", "fp16", "fp32")
_TORCH_ACT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
_ACT_OF = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}
ROLES = ("gate", "down", "up")


def act_name(dtype) -> str:
    return dtype if isinstance(dtype, str) else _ACT_OF[dtype]


# ── rounding ────────────────────────────────────────────────────────────────────────────

def bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even; NaN -> 0x7FC0.

    Restates `_round` CODE 0 (vaayu/packed_expert_kernels.py:78-84): add 0x7FFF plus the
    kept lsb, drop the low 16 bits; a NaN is passed through (here: the canonical quiet
    NaN torch stores)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = r.astype(np.uint16)
    return np.where(np.isnan(a), np.uint16(0x7FC0), r)


def bf16_value(bits) -> np.ndarray:
    """bfloat16 bit patterns -> float32 values (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def _f64_to_bf16(a: np.ndarray) -> np.ndarray:
    """float64 -> bf16 values (as float32), correctly rounded from the float64 value
    (no double rounding through float32). Normal range by mantissa arithmetic on the
    float64 bits; the bf16 subnormal range by rint at the fixed 2^-133 quantum."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    u = a.view(np.uint64)
    drop = np.uint64(45)                                    # 52 - 7 mantissa bits
    bias = np.uint64((1 << 44) - 1) + ((u >> drop) & np.uint64(1))
    r = ((u + bias) >> drop) << drop
    out = r.view(np.float64)
    tiny = np.abs(a) < 2.0 ** -126
    if tiny.any():
        q = 2.0 ** -133
        out = np.where(tiny, np.rint(a / q) * q, out)
    with np.errstate(over="ignore"):
        out32 = out.astype(np.float32)                      # exact, or +-inf past bf16 max
    return np.where(np.isnan(a), np.float32(np.nan), out32)


def round_to(a, act: str) -> np.ndarray:
    """Round `a` (float32 or float64 values) ONCE, nearest-even, to the activation dtype
    `act`; returned as float32 values exactly representable in it. This is what storing
    into that dtype does at every stock-path rounding point
    (vaayu/packed_expert_kernels.py:75-88)."""
    a = np.asarray(a)
    if act == "fp32":
        return a.astype(np.float32)
    if act == "fp16":
        with np.errstate(over="ignore"):
            return a.astype(np.float16).astype(np.float32)  # numpy: correctly rounded
    if a.dtype == np.float64:
        return _f64_to_bf16(a)
    return bf16_value(bf16_bits(a.astype(np.float32)))


def to_np(t) -> np.ndarray:
    """A torch tensor (any float dtype, any device) or array -> float32 numpy values."""
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.is_floating_point():
            return t.float().numpy()
        return t.numpy()
    return np.asarray(t)


# ── the repo's quantizer and compressed-tensors packing ──────────────────────────────────

def quantize_symmetric(weight, num_bits: int, group_size: int):
    """(q int8 [rows, cols], scale fp32 [rows, groups]) of `weight`.

    Restates `_reference_pack` (tests/test_packed_expert_dequant.py:44-57): per group,
    scale = max(|w|).clamp(1e-6) / qmax in fp32; q = round-half-even(w / scale) clamped to
    [-qmax-1, qmax]."""
    w = to_np(weight).astype(np.float32)
    rows, cols = w.shape
    g = w.reshape(rows, cols // group_size, group_size)
    qmax = np.float32(2 ** (num_bits - 1) - 1)
    scale = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-6)) / qmax
    q = np.clip(np.rint(g / scale[..., None]), -qmax - 1, qmax)
    return q.reshape(rows, cols).astype(np.int8), scale.astype(np.float32)


def pack_to_int32(q, num_bits: int) -> np.ndarray:
    """Signed codes [rows, cols] -> int32 words [rows, ceil(cols*bits/32)].

    The layout `unpack_int32_to_int8` inverts (vaayu/moe_patch.py:668-710): each code is
    stored unsigned with offset 2^(bits-1); a row is one dense little-endian bit stream,
    code i at bits [i*bits, (i+1)*bits). (compressed-tensors' own `pack_to_int32` is not
    installed here; this restates the layout the reference's unpack documents.)"""
    q = np.asarray(q).astype(np.int64)
    rows, cols = q.shape
    u = (q + (1 << (num_bits - 1))).astype(np.uint64)
    if np.any(u >> np.uint64(num_bits)):
        raise ValueError("code out of range")
    n_words = -(-cols * num_bits // 32)
    per = 32 // num_bits
    if 32 % num_bits == 0 and cols % per == 0:          # no code straddles a word
        sh = np.arange(per, dtype=np.uint64) * np.uint64(num_bits)
        w = (u.reshape(rows, n_words, per) << sh).sum(axis=-1, dtype=np.uint64)
        return w.astype(np.uint32).view(np.int32)
    return _pack_bitstream(u, num_bits, n_words)


def _pack_bitstream(u, num_bits: int, n_words: int) -> np.ndarray:
    """Unsigned codes -> words, one code at a time (any bit width): the brute-force
    form of the layout, also what the vectorised path is checked against."""
    rows, cols = u.shape
    out = np.zeros((rows, n_words), dtype=np.uint64)
    for i in range(cols):                       # vectorised over rows
        bit = i * num_bits
        w, o = divmod(bit, 32)
        out[:, w] |= (u[:, i] << np.uint64(o)) & np.uint64(0xFFFFFFFF)
        if o + num_bits > 32:
            out[:, w + 1] |= u[:, i] >> np.uint64(32 - o)
    return out.astype(np.uint32).view(np.int32)


def unpack_int32(packed, num_bits: int, cols: int) -> np.ndarray:
    """int32 words -> signed int8 codes: vaayu/moe_patch.py:668-710 (both branches: the
    per-word shift for 32 % bits == 0 and the straddling bit stream otherwise)."""
    p = np.asarray(packed).view(np.uint32).astype(np.uint64)
    rows = p.shape[0]
    if 32 % num_bits == 0:
        per = 32 // num_bits
        sh = np.arange(per, dtype=np.uint64) * np.uint64(num_bits)
        c = ((p[:, :, None] >> sh) & np.uint64((1 << num_bits) - 1)).reshape(rows, -1)[:, :cols]
        return (c.astype(np.int64) - (1 << (num_bits - 1))).astype(np.int8)
    return _unpack_bitstream(p, num_bits, cols)


def _unpack_bitstream(p, num_bits: int, cols: int) -> np.ndarray:
    """Words -> signed codes one code at a time (any bit width, straddling allowed)."""
    rows = p.shape[0]
    out = np.zeros((rows, cols), dtype=np.int64)
    for i in range(cols):
        bit = i * num_bits
        w, o = divmod(bit, 32)
        v = p[:, w] >> np.uint64(o)
        if o + num_bits > 32:
            v |= p[:, w + 1] << np.uint64(32 - o)
        out[:, i] = (v & np.uint64((1 << num_bits) - 1)).astype(np.int64)
    return (out - (1 << (num_bits - 1))).astype(np.int8)


# ── blobs ───────────────────────────────────────────────────────────────────────────────

def make_expert(hidden: int, inter: int, num_bits: int, group_size: int, *, rng,
                std: float = 0.02, scale_dtype=torch.float16) -> dict:
    """One synthetic expert: bf16 N(0, std) weights quantized per role, as the
    `{role: {weight_packed, weight_scale, weight_shape}}` dict a pack-quantized
    checkpoint stores (role order gate, down, up: vaayu/moe_patch.py:532-551)."""
    by_role = {}
    for role, shape in (("gate", (inter, hidden)), ("down", (hidden, inter)),
                        ("up", (inter, hidden))):
        w = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * std)
        w = w.to(torch.bfloat16)
        q, s = quantize_symmetric(w, num_bits, group_size)
        by_role[role] = {
            "weight_packed": torch.from_numpy(pack_to_int32(q, num_bits)),
            "weight_scale": torch.from_numpy(s).to(scale_dtype),
            "weight_shape": torch.tensor(list(shape)),
        }
    return by_role


def build_blob(by_role: dict) -> dict:
    """`build_expert_blob` (vaayu/moe_patch.py:794-846) for symmetric packed roles:
    flat streams concatenated in the dict's role order, geometry derived from tensors."""
    geom, packed, scale = [], [], []
    for role, comps in by_role.items():
        rows, cols = (int(v) for v in comps["weight_shape"].tolist())
        bits = comps["weight_packed"].numel() * 32 // (rows * cols)
        gs = cols // comps["weight_scale"].shape[-1]
        geom.append((role, rows, cols, bits, gs))
        packed.append(comps["weight_packed"].reshape(-1))
        scale.append(comps["weight_scale"].reshape(-1))
    bits, gs = geom[0][3], geom[0][4]
    return {"flat": {"packed": torch.cat(packed), "scale": torch.cat(scale)},
            "geom": (bits, gs, tuple((g[0], g[1], g[2]) for g in geom))}


def layout(geom) -> dict:
    """{role: (word offset, scale offset, rows, cols)}: vaayu/packed_expert_kernels.py:301-309."""
    bits, gs, roles = geom
    out, w_at, s_at = {}, 0, 0
    for role, rows, cols in roles:
        out[role] = (w_at, s_at, rows, cols)
        w_at += rows * cols * bits // 32
        s_at += rows * cols // gs
    return out


def dequant_flat(flat_packed, flat_scale, num_bits: int, group_size: int, act) -> np.ndarray:
    """Whole-blob dequant, float32 values of dtype `act`.

    Restates `_fused_dequant_kernel` (vaayu/moe_patch.py:750-769): codes
    `(word >> j*bits) & mask` for j in 0..32/bits-1, offset 2^(bits-1) subtracted in the
    target dtype (exact), times the group's scale converted to the target dtype, the
    product rounded to it."""
    act = act_name(act)
    p = to_np(flat_packed).astype(np.int32).view(np.uint32)
    per = 32 // num_bits
    shifts = (np.arange(per, dtype=np.uint32) * np.uint32(num_bits))
    codes = (p[:, None] >> shifts[None, :]) & np.uint32((1 << num_bits) - 1)
    # The product (c - off) * s is exact in float32 when s has at most 11 significant bits
    # (a bf16 / fp16 scale) and |c - off| at most 8: then float32 and float64 agree, and
    # float32 takes a quarter of the memory traffic. An fp32 scale needs float64.
    wide = np.float32 if act in ("bf16", "fp16") else np.float64
    codes = codes.reshape(-1, group_size).astype(wide) - wide(1 << (num_bits - 1))
    s = round_to(to_np(flat_scale).astype(np.float32), act).astype(wide)
    return round_to(codes * s.reshape(-1, 1), act).reshape(-1)


def expert_weights(blob: dict, act) -> tuple:
    """(w_gate, w_down, w_up) float32 values: `expert_weights_from_entry`
    (vaayu/moe_patch.py:849-877, 880-891) for a packed blob or a dense entry."""
    if "dense" in blob:
        d = blob["dense"]
        return tuple(round_to(to_np(d[r]), act_name(act)) for r in ("gate", "down", "up"))
    if isinstance(blob["geom"][0], str):
        return format_expert_weights(blob, act)
    bits, gs, roles = blob["geom"]
    flat = dequant_flat(blob["flat"]["packed"], blob["flat"]["scale"], bits, gs, act)
    out, at = {}, 0
    for role, rows, cols in roles:
        out[role] = flat[at:at + rows * cols].reshape(rows, cols)
        at += rows * cols
    return out["gate"], out["down"], out["up"]


def format_expert_weights(blob: dict, act) -> tuple:
    """(w_gate, w_down, w_up) of an FP8 ("e4m3", (bo, bi)) or MXFP4 ("mxfp4", 32) blob:
    roles gate, down, up concatenated, codes along the last dim; each role through
    `dequant_block_scaled` / `upcast_mxfp4` (the weights the reference's dequant of that
    format gives: vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240, vendor
    …/numerics_details/mxfp.py:256-299)."""
    act = act_name(act)
    kind, gs, roles = blob["geom"]
    codes = to_np(blob["flat"]["packed"]).astype(np.int32).view(np.uint8)
    scale = to_np(blob["flat"]["scale"])
    out, c_at, s_at = {}, 0, 0
    for role, rows, cols in roles:
        if kind == "e4m3":
            bo, bi = gs
            n_c, n_s = rows * cols, (rows // bo) * (cols // bi)
            q = codes[c_at:c_at + n_c].reshape(rows, cols)
            sc = scale[s_at:s_at + n_s].astype(np.float32).reshape(rows // bo, cols // bi)
            out[role] = dequant_block_scaled(q, sc, act)
        elif kind == "mxfp4":
            n_c, n_s = rows * cols // 2, rows * cols // 32
            q = codes[c_at:c_at + n_c].reshape(rows, cols // 2)
            sc = scale[s_at:s_at + n_s].astype(np.uint8).reshape(rows, cols // 32)
            out[role] = upcast_mxfp4(q, sc, act)
        else:
            raise ValueError(f"format {kind!r}")
        c_at += n_c
        s_at += n_s
    return out["gate"], out["down"], out["up"]


# ── the stock arithmetic (correctly rounded replay) ──────────────────────────────────────

def _linear(a, w, act):
    """F.linear(a, w) summed in float64 and rounded ONCE to `act`."""
    return round_to(a.astype(np.float64) @ w.astype(np.float64).T, act)


def silu_round(g, act):
    """`act_fn` = SiLU on a tensor of dtype `act`: g / (1 + exp(-g)) in fp32, rounded
    (vaayu/packed_expert_kernels.py:149 for the kernels' own form)."""
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return round_to(g / (np.float32(1.0) + np.exp(-g)), act)


def expert_stages(x, blob, act, weights=None):
    """One expert's stock stages for rows `x` [n, hidden] (float32 values of `act`):
    (h, y) with h = act(x Wg^T) * (x Wu^T) and y = h Wd^T, each rounded to `act`
    (vaayu/packed_expert_kernels.py:408-409). `weights`: the expert's dequantized
    (gate, down, up), when the caller already holds them."""
    wg, wd, wu = weights if weights is not None else expert_weights(blob, act)
    g = _linear(x, wg, act)
    u = _linear(x, wu, act)
    h = round_to(silu_round(g, act).astype(np.float64) * u.astype(np.float64), act)
    y = _linear(h, wd, act)
    return h, y


def truth_stages(x, exact_weights):
    """The fp64 truth of one expert (tests/test_packed_prefill_kernels.py:100-116): the
    checkpoint's exact weights (gate, down, up) as float64, no rounding anywhere.
    Returns y = (silu(x Wg^T) * (x Wu^T)) Wd^T, float64."""
    wg, wd, wu = (np.asarray(w, dtype=np.float64) for w in exact_weights)
    xv = np.asarray(x, dtype=np.float64)
    g, u = xv @ wg.T, xv @ wu.T
    return (g / (1.0 + np.exp(-g)) * u) @ wd.T


def contribution(y, w, w_dtype, act):
    """`(y * rw).to(fp32)` with torch's promotion (vaayu/packed_expert_kernels.py:410):
    an fp32 weight gives an fp32 product; a weight already in the activation dtype makes
    the product round to it."""
    w = np.asarray(w, dtype=np.float32)
    if act_name(w_dtype) == act and act != "fp32":
        return round_to(y.astype(np.float64) * w.astype(np.float64), act)
    return (y.astype(np.float32) * w.astype(np.float32)).astype(np.float32)


def stock_decode(x, pairs, routing_weights, w_dtype=None, act="bf16") -> np.ndarray:
    """`stock_experts_decode` (vaayu/packed_expert_kernels.py:399-410): per pair, in pair
    order, the expert's rounded stages and contribution, summed in fp32 from zero.

    x [1, hidden] (float32 values of `act`); pairs [(blob, slot)]; returns fp32 [1, hidden]."""
    act = act_name(act)
    xv = to_np(x).reshape(1, -1)
    if w_dtype is None:
        w_dtype = routing_weights.dtype if isinstance(routing_weights, torch.Tensor) else "fp32"
    rw = to_np(routing_weights).reshape(-1)
    out = np.zeros(xv.shape, dtype=np.float32)
    for blob, slot in pairs:
        _h, y = expert_stages(xv, blob, act)
        out = (out + contribution(y, rw[slot], w_dtype, act)).astype(np.float32)
    return out


def decode_table_values(pairs, ptr_of=id) -> list:
    """`_table_values` (vaayu/packed_expert_kernels.py:349-352) with a caller-given
    address function: (packed address, scale address, slot) per pair."""
    return [v for blob, slot in pairs
            for v in (ptr_of(blob["flat"]["packed"]), ptr_of(blob["flat"]["scale"]), slot)]


# ── prefill ─────────────────────────────────────────────────────────────────────────────

BLOCK_M = 16   # rows per block in the prefill tables (vaayu/packed_expert_kernels.py:63)


def prefill_plan(eidx):
    """(order, live, counts): vaayu/packed_expert_kernels.py:676-688 -- row ids
    (token*top_k + slot) stable-sorted by expert id, routed ids ascending, rows each."""
    e = np.asarray(to_np(eidx), dtype=np.int64).reshape(-1)
    order = np.argsort(e, kind="stable")
    per = np.bincount(e)
    live = np.nonzero(per)[0]
    return order, live, per[live]


def prefill_tables(eidx, plan, ptrs) -> tuple:
    """Host half of `_prefill_tables` (vaayu/packed_expert_kernels.py:691-717):
    (tbl [n_blocks, 2], rows [n_blocks*16] with -1 padding, slot_order [T*top_k], n_blocks).
    `ptrs[e]` is expert e's (packed address, scale address)."""
    order, live, counts = plan
    e = np.asarray(to_np(eidx), dtype=np.int64)
    n, top_k = e.shape
    nblk = (counts + BLOCK_M - 1) // BLOCK_M
    blk_end = np.cumsum(nblk)
    n_blocks = int(blk_end[-1])
    which = np.repeat(np.arange(live.size), counts)
    src_start = np.cumsum(counts) - counts
    dest = ((blk_end - nblk) * BLOCK_M)[which] + np.arange(order.size) - src_start[which]
    rows = np.full(n_blocks * BLOCK_M, -1, dtype=np.int64)
    rows[dest] = order
    p = np.asarray([ptrs[int(x)] for x in live], dtype=np.int64).reshape(-1, 2)
    tbl = p[np.repeat(np.arange(live.size), nblk)]
    slot_order = (np.argsort(e, axis=1, kind="stable") + (np.arange(n) * top_k)[:, None])
    return tbl, rows, slot_order.reshape(-1), n_blocks


def prefill_stages(x, eidx, blobs, act="bf16"):
    """The grouped kernels' intermediates, stock-rounded: (h [T*k, inter], y_down [T*k, hidden])
    with y_down the rounded down output BEFORE the routing weight."""
    act = act_name(act)
    xv = to_np(x)
    e = np.asarray(to_np(eidx), dtype=np.int64)
    top_k = e.shape[1]
    order, live, counts = prefill_plan(e)
    h = y = None
    at = 0
    for ex, c in zip(live.tolist(), counts.tolist()):
        rows = order[at:at + c]
        at += c
        hs, ys = expert_stages(xv[rows // top_k], blobs[ex], act)
        if h is None:
            h = np.full((e.size, hs.shape[1]), np.nan, np.float32)
            y = np.full((e.size, ys.shape[1]), np.nan, np.float32)
        h[rows], y[rows] = hs, ys
    return h, y


def stock_prefill(x, eidx, routing_weights, blobs, w_dtype=None, act="bf16",
                  weights_of=None) -> np.ndarray:
    """`stock_experts_prefill(linear=_linear_fp32)` (vaayu/packed_expert_kernels.py:780-814),
    correctly rounded: per live expert in id order, its rows' rounded stages times their
    weights, added into each token's fp32 row in expert-id order (the order
    `accumulate_expert_outputs` sums in, vaayu/moe_patch.py:914-940). A routed expert
    with no entry is skipped. `weights_of(expert id)`: its dequantized (gate, down, up),
    when the caller holds them (otherwise dequantized here)."""
    act = act_name(act)
    xv = to_np(x)
    e = np.asarray(to_np(eidx), dtype=np.int64)
    top_k = e.shape[1]
    if w_dtype is None:
        w_dtype = routing_weights.dtype if isinstance(routing_weights, torch.Tensor) else "fp32"
    rw = to_np(routing_weights).reshape(-1)
    order, live, counts = prefill_plan(e)
    out = np.zeros(xv.shape, dtype=np.float32)
    at = 0
    for ex, c in zip(live.tolist(), counts.tolist()):
        rows = order[at:at + c]
        at += c
        if ex not in blobs:
            continue
        wts = weights_of(ex) if weights_of is not None else None
        _h, y = expert_stages(xv[rows // top_k], blobs[ex], act, weights=wts)
        contrib = contribution(y, rw[rows][:, None], w_dtype, act)
        for i, r in enumerate(rows.tolist()):          # sequential: a token may repeat
            t = r // top_k
            out[t] = (out[t] + contrib[i]).astype(np.float32)
    return out


def reduce_in_order(y, slot_order, tokens: int, top_k: int) -> np.ndarray:
    """`_reduce_kernel` (vaayu/packed_expert_kernels.py:250-260): out[t] = sum over k of
    y[ord[t, k]], sequentially from 0 in fp32."""
    y = np.asarray(y, dtype=np.float32)
    o = np.asarray(slot_order).reshape(tokens, top_k)
    out = np.zeros((tokens, y.shape[1]), dtype=np.float32)
    for k in range(top_k):
        out = (out + y[o[:, k]]).astype(np.float32)
    return out


def accumulate(final, contributions) -> np.ndarray:
    """`accumulate_expert_outputs` (vaayu/moe_patch.py:914-940): contributions
    (expert id, token rows, values) added into an fp32 accumulator in expert-id order."""
    out = np.array(final, dtype=np.float32, copy=True)
    for _e, rows, vals in sorted(contributions, key=lambda c: c[0]):
        vals = np.asarray(vals, dtype=np.float32)
        for i, r in enumerate(np.asarray(rows).reshape(-1).tolist()):
            out[r] = (out[r] + vals[i]).astype(np.float32)
    return out


# ── routing ─────────────────────────────────────────────────────────────────────────────

def route_softmax_topk(logits, top_k: int):
    """The bare-logits branch of `_route` (vaayu/moe_patch.py:2330-2334): softmax of the
    fp32 logits, top-k, renormalised (fp32 weights). Ties break to the LOWER expert id
    (stable), a rule the reference leaves to torch.topk."""
    lg = to_np(logits).astype(np.float32)
    m = lg.max(axis=-1, keepdims=True)
    p = np.exp(lg - m)
    p = (p / p.sum(axis=-1, keepdims=True)).astype(np.float32)
    idx = np.argsort(-p, axis=-1, kind="stable")[..., :top_k]
    w = np.take_along_axis(p, idx, axis=-1)
    return (w / w.sum(axis=-1, keepdims=True)).astype(np.float32), idx.astype(np.int64)


def truncate_top_k(weights, indices, k=None, p=None):
    """The decode-time expert budget `truncate_top_k` (vaayu/moe_patch.py:170-215) on
    routed (weights, indices) [..., K]: keep the k largest weights (rescaled to the row's
    original sum), then with p keep per row the fewest slots whose normalised weight
    reaches p (the mass BEFORE a slot < p keeps it), re-pointing each dropped slot at the
    row's top-1 expert with weight 0. The original sum snaps to 1.0 within 1e-2. Equal
    weights order by slot (stable); sums run in slot order, in fp32."""
    w = np.array(to_np(weights), dtype=np.float32)
    idx = np.array(to_np(indices), dtype=np.int64)
    n = w.shape[-1]
    if (k is None or k >= n) and p is None:
        return w, idx

    def ssum(a):                                   # slot-order fp32 sum over the last axis
        acc = np.zeros(a.shape[:-1] + (1,), dtype=np.float32)
        for j in range(a.shape[-1]):
            acc = (acc + a[..., j:j + 1]).astype(np.float32)
        return acc

    total = ssum(w)
    total = np.where(np.abs(total - np.float32(1)) < np.float32(1e-2), np.float32(1), total)
    if k is not None and k < n:
        pos = np.argsort(-w, axis=-1, kind="stable")[..., :k]
        wk = np.take_along_axis(w, pos, -1)
        w = (wk / ssum(wk) * total).astype(np.float32)
        idx = np.take_along_axis(idx, pos, -1)
    if p is None:
        return w, idx
    wn = (w / ssum(w)).astype(np.float32)
    order = np.argsort(-wn, axis=-1, kind="stable")
    ws = np.take_along_axis(wn, order, -1)
    cs = np.cumsum(ws, axis=-1, dtype=np.float32)
    keep_sorted = (cs - ws).astype(np.float32) < np.float32(p)
    keep = np.zeros_like(keep_sorted)
    np.put_along_axis(keep, order, keep_sorted, -1)
    top1 = np.broadcast_to(np.take_along_axis(idx, order[..., :1], -1), idx.shape)
    wk = np.where(keep, wn, np.float32(0)).astype(np.float32)
    w = (wk / ssum(wk) * total).astype(np.float32)
    return w, np.where(keep, idx, top1)


# ── FP8 block-scaled and MXFP4 formats ──────────────────────────────────────────────────

def e4m3_value(byte) -> np.ndarray:
    """float8 e4m3fn bit patterns -> float32 (bias 7, no infinities, S.1111.111 = NaN)."""
    b = np.asarray(byte, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (s * val).astype(np.float32)


def dequant_block_scaled(w_bytes, scale, act="bf16") -> np.ndarray:
    """`dequantize_block_scaled` (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240):
    W[i, j] = round_act(fp32(e4m3) * fp32(scale[i // bo, j // bi])), the fp32 product
    itself rounded (torch's fp32 multiply), block sizes derived from the two shapes."""
    w = e4m3_value(w_bytes)
    s = to_np(scale).astype(np.float32)
    bo = w.shape[0] // s.shape[0]
    bi = w.shape[1] // s.shape[1]
    full = np.repeat(np.repeat(s, bo, axis=0), bi, axis=1)
    return round_to((w * full).astype(np.float32), act_name(act))


E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def e2m1_value(nibble) -> np.ndarray:
    """`cvt_e2m1_to_fp32` (vendor …/numerics_details/mxfp.py:238-253): nibble -> value,
    bit 3 the sign."""
    n = np.asarray(nibble, dtype=np.int64) & 0xF
    v = np.asarray(E2M1, dtype=np.float32)[n & 7]
    return np.where(n & 8, -v, v).astype(np.float32)


def upcast_mxfp4(packed_u8, scale_e8m0, act="bf16") -> np.ndarray:
    """`upcast_from_mxfp_torch` for e2m1 along the last axis (vendor
    …/numerics_details/mxfp.py:256-299): even element in the low nibble, scale
    2^(s-127) per 32 elements (the fp32 built by `s << 23`), product in fp32 then cast.
    Scale 0xFF is NaN (the Triton twin's rule, …/mxfp_details/_upcast_from_mxfp.py)."""
    p = np.asarray(packed_u8, dtype=np.uint8)
    lo = e2m1_value(p & 0xF)
    hi = e2m1_value(p >> 4)
    vals = np.stack([lo, hi], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    s = np.asarray(scale_e8m0, dtype=np.uint8).astype(np.uint32)
    sf = (s << np.uint32(23)).view(np.float32)
    sf = np.where(s == 0xFF, np.float32(np.nan), sf)
    full = np.repeat(sf, 32, axis=-1)[..., :vals.shape[-1]]
    return round_to((vals * full).astype(np.float32), act_name(act))


def upcast_mx_e4m3(codes_u8, scale_e8m0, act="bf16") -> np.ndarray:
    """`upcast_from_mxfp_torch` for float8_e4m3fn codes (vendor …/numerics_details/mxfp.py:
    276-279: `tensor.to(float32)`), otherwise as `upcast_mxfp4`: 2^(s-127) per 32 elements
    along the last axis, fp32 product, one cast; scale 0xFF is NaN."""
    vals = e4m3_value(codes_u8)
    s = np.asarray(scale_e8m0, dtype=np.uint8).astype(np.uint32)
    sf = (s << np.uint32(23)).view(np.float32)
    sf = np.where(s == 0xFF, np.float32(np.nan), sf)
    full = np.repeat(sf, 32, axis=-1)[..., :vals.shape[-1]]
    return round_to((vals * full).astype(np.float32), act_name(act))


# ── the CPU baseline: the stock loop itself on torch CPU ─────────────────────────────────

def _dequant_format_torch(blob, dtype):
    """FP8 / MXFP4 blob roles on torch CPU, as the reference's dequant functions compute
    them (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240; vendor
    …/numerics_details/mxfp.py:238-299)."""
    kind, gs, roles = blob["geom"]
    codes = blob["flat"]["packed"].contiguous().view(torch.uint8)
    scale = blob["flat"]["scale"]
    out, c_at, s_at = {}, 0, 0
    for role, rows, cols in roles:
        if kind == "e4m3":
            bo, bi = gs
            n_c, n_s = rows * cols, (rows // bo) * (cols // bi)
            w = codes[c_at:c_at + n_c].view(torch.float8_e4m3fn).view(rows, cols)
            sc = scale[s_at:s_at + n_s].view(rows // bo, cols // bi)
            t = w.unflatten(0, (-1, bo)).unflatten(-1, (-1, bi)).float() * sc[:, None, :, None].float()
            out[role] = t.flatten(2, 3).flatten(0, 1).to(dtype)
        else:
            n_c, n_s = rows * cols // 2, rows * cols // 32
            q = codes[c_at:c_at + n_c].view(rows, cols // 2).to(torch.int32)
            lut = torch.tensor(E2M1 + tuple(-v for v in E2M1), dtype=torch.float32)
            vals = torch.stack([lut[q & 0xF], lut[(q >> 4) & 0xF]], -1).view(rows, cols)
            s8 = scale[s_at:s_at + n_s].view(rows, cols // 32).to(torch.int32)
            f = torch.where(s8 == 0xFF, torch.tensor(float("nan")), (s8 << 23).view(torch.float32))
            out[role] = (vals * f.repeat_interleave(32, dim=-1)).to(dtype)
        c_at += n_c
        s_at += n_s
    return out["gate"], out["down"], out["up"]


def _dequant_torch(blob, dtype):
    """`_fused_dequant_kernel` eager on torch CPU (vaayu/moe_patch.py:750-769)."""
    if isinstance(blob["geom"][0], str):
        return _dequant_format_torch(blob, dtype)
    bits, gs, roles = blob["geom"]
    packed, scale = blob["flat"]["packed"], blob["flat"]["scale"]
    per = 32 // bits
    shifts = torch.arange(per, dtype=torch.int32) * bits
    codes = (packed.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    codes = codes.view(-1, gs).to(dtype) - (1 << (bits - 1))
    flat = (codes * scale.reshape(-1, 1).to(dtype)).view(-1)
    out, at = {}, 0
    for role, rows, cols in roles:
        out[role] = flat[at:at + rows * cols].view(rows, cols)
        at += rows * cols
    return out["gate"], out["down"], out["up"]


def stock_decode_torch(x, pairs, routing_weights, out) -> None:
    """The reference's stock decode loop (vaayu/packed_expert_kernels.py:399-410) run as
    written on torch CPU: dequant every routed expert, three `F.linear`, SiLU, product,
    routing-weight product, fp32 add in pair order. This is what the CPU baseline times."""
    import torch.nn.functional as F
    rw = routing_weights.reshape(-1)
    out.zero_()
    for blob, slot in pairs:
        w_gate, w_down, w_up = _dequant_torch(blob, x.dtype)
        y = F.linear(F.silu(F.linear(x, w_gate)) * F.linear(x, w_up), w_down)
        out += (y * rw[slot:slot + 1]).to(out.dtype)


def stock_prefill_torch(x, eidx, routing_weights, blobs, out) -> None:
    """The reference's stock prefill loop (vaayu/packed_expert_kernels.py:785-814) on
    torch CPU: per live expert in id order, gather, three `F.linear`, `index_add_`."""
    import torch.nn.functional as F
    e = eidx.reshape(-1)
    order = torch.argsort(e, stable=True)
    per = torch.bincount(e)
    live = per.nonzero().reshape(-1)
    top_k = eidx.shape[1]
    rw = routing_weights.reshape(-1)
    out.zero_()
    at = 0
    for ex, c in zip(live.tolist(), per[live].tolist()):
        rows = order[at:at + c]
        at += c
        if ex not in blobs:
            continue
        w_gate, w_down, w_up = _dequant_torch(blobs[ex], x.dtype)
        tok = rows // top_k
        xs = x[tok]
        y = F.linear(F.silu(F.linear(xs, w_gate)) * F.linear(xs, w_up), w_down)
        out.index_add_(0, tok, (y * rw[rows, None]).to(out.dtype))


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def fp64_truth_decode(x, pairs, routing_weights) -> np.ndarray:
    """The reference's fp64 truth (tests/test_packed_expert_kernels.py:75-89): the
    checkpoint's exact weights, no rounding anywhere."""
    xv = to_np(x).reshape(-1).astype(np.float64)
    rw = to_np(routing_weights).reshape(-1).astype(np.float64)
    out = np.zeros(xv.shape, np.float64)
    for blob, slot in pairs:
        bits, gs, roles = blob["geom"]
        p = to_np(blob["flat"]["packed"]).astype(np.int32).view(np.uint32)
        per = 32 // bits
        shifts = np.arange(per, dtype=np.uint32) * np.uint32(bits)
        codes = ((p[:, None] >> shifts) & np.uint32((1 << bits) - 1)).reshape(-1, gs)
        flat = ((codes.astype(np.float64) - (1 << (bits - 1)))
                * to_np(blob["flat"]["scale"]).astype(np.float64).reshape(-1, 1)).reshape(-1)
        mats, at = {}, 0
        for role, rows, cols in roles:
            mats[role] = flat[at:at + rows * cols].reshape(rows, cols)
            at += rows * cols
        g, u = mats["gate"] @ xv, mats["up"] @ xv
        out += (mats["down"] @ (g / (1 + np.exp(-g)) * u)) * rw[slot]
    return out


def isclose_frac(a, b) -> float:
    """Fraction of positions where a and b are bit-equal (NaN == NaN)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return float(np.mean((a == b) | (np.isnan(a) & np.isnan(b))))


def ulp_bf16(v) -> float:
    return math.ldexp(1.0, math.frexp(abs(v))[1] - 8) if v else 0.0
