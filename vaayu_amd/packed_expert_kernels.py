"""Packed-expert routed-MoE kernels for MI355X: the drop-in for Vaayu's
`vaayu/packed_expert_kernels.py`.

The public entries, their arguments and results, the pointer tables, the verdict and
fallback rules, the per-layer decode graph and the installer behave as the reference's
(file:line cited per function), so the engine's fused forward (vaayu/moe_patch.py:2394-2401,
2608-2624) and installer call (vaayu/vaayu_base.py:3560) need no change. The arithmetic
runs in hand-written HIP kernels for gfx950 (vaayu_amd/csrc, C ABI in include/vaayu_amd.h):

  decode  (one token)  `vaayu_decode_gate_up` + `vaayu_decode_down`: GEMVs on the VALU,
                       codes unpacked in registers, the fp32 sum over pairs in table order.
  prefill (a call of   `vaayu_prefill_gate_up` + `vaayu_prefill_down` + `vaayu_prefill_reduce`:
   any length)         grouped GEMMs on MFMA over 16-row blocks of one expert each, then
                       each token's contributions summed in ascending expert id.

Every value the stock path stores in the activation dtype is rounded to it at the same
point, and nothing is accumulated atomically: the output is a function of (x, routing,
weights) alone, whatever the blobs' addresses or arrival order.

Without the built library (vaayu_amd/libvaayu_amd.so) the kernels raise ImportError,
naming the file; there is no silent substitute.
"""
import collections
import gc
from pathlib import Path

import torch
import torch.nn.functional as F

from . import _lib
from .block_formats import blob_layout, geom_format, FMT_E4M3, FMT_MXFP4

try:
    _lib.load()
    _BACKEND = _lib
except ImportError as _exc:              # reported at the first kernel call / install
    _BACKEND = None
    _LOAD_ERROR = str(_exc)

# Truthiness of the kernel backend, under the name the engine's installer and its tests
# use for it (they set it to None to simulate a machine without the kernels).
triton = _BACKEND

# relL2 of a layer's output against its reference above which a kernel is refused.
_CHECK_TOL = 1e-2
_BK_MAX = 512
# Prefill tables group each expert's (token, slot) rows into blocks of this many rows.
_PF_BLOCK_M = 16
_PF_MIN_TILE = 16
_PF_GU_BK_MAX, _PF_DN_BK_MAX = 256, 256
_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
# Scale dtypes the kernels read: the activation dtypes, and E8M0 bytes (MXFP4 blobs).
_SCALE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.uint8: 3}
_ROLES = ("gate", "down", "up")


def _require_backend():
    if triton is None:
        raise ImportError(globals().get("_LOAD_ERROR", "vaayu_amd kernels unavailable"))
    return _lib.load()


class _TableRing:
    """Pinned host staging for the per-call pointer tables, reused round-robin
    (vaayu/packed_expert_kernels.py:263-292). A slot's host buffer is rewritten only after
    the copy that last read it has completed (its event); each slot has its own device
    table, so no queued kernel's table is overwritten."""

    def __init__(self, n_slots: int = 4):
        self._slots: list = [None] * n_slots
        self._next = 0

    def put(self, values, device) -> torch.Tensor:
        i = self._next
        self._next = (i + 1) % len(self._slots)
        n = len(values)
        slot = self._slots[i]
        if slot is None or slot[0].numel() < n or slot[1].device != torch.device(device):
            cap = max(64, 1 << (n - 1).bit_length())
            host = torch.empty(cap, dtype=torch.int64, pin_memory=True)
            slot = self._slots[i] = [host, torch.empty(cap, dtype=torch.int64, device=device),
                                     torch.cuda.Event(), False]
        host, dev, done, used = slot
        if used:
            done.synchronize()
        host[:n] = torch.as_tensor(values, dtype=torch.int64)
        dev[:n].copy_(host[:n], non_blocking=True)
        done.record()
        slot[3] = True
        return dev


_TABLES = _TableRing()
_VERDICTS: dict = {}
_PF_TABLES = _TableRing()
_PF_VERDICTS: dict = {}


def _layout(geom) -> dict:
    """{role: (word offset, scale offset, rows, cols)} inside a blob's flat streams
    (vaayu/packed_expert_kernels.py:301-309); FP8 / MXFP4 blobs by their own scale blocking
    (vaayu_amd.block_formats)."""
    if isinstance(geom[0], str):
        return blob_layout(geom)
    bits, gs, roles = geom
    out, w_at, s_at = {}, 0, 0
    for role, rows, cols in roles:
        out[role] = (w_at, s_at, rows, cols)
        w_at += rows * cols * bits // 32
        s_at += rows * cols // gs
    return out


def _block_k(k: int, gs: int, cap: int = _BK_MAX):
    """Largest power-of-two multiple of the group size, at most max(cap, gs), dividing k
    (vaayu/packed_expert_kernels.py:312-319); None if there is none."""
    best, b = None, gs
    while b <= max(cap, gs):
        if k % b == 0:
            best = b
        b *= 2
    return best


def _pow2_divisor(n: int, cap: int) -> int:
    b = cap
    while n % b:
        b //= 2
    return b


def _unsupported(geom, act_dtype, scale_dtype, w_dtype):
    """Why the decode kernels cannot run this geometry / these dtypes, or None.

    The reference's rules (vaayu/packed_expert_kernels.py:329-346), plus what the HIP
    GEMV needs: a row is whole 16-byte units of codes, and a unit lies in one group."""
    shapes = {r: (rows, cols) for r, rows, cols in geom[2]}
    if set(shapes) != set(_ROLES):
        return f"expert roles {sorted(shapes)} are not gate/up/down"
    inter, hid = shapes["gate"]
    if shapes["up"] != (inter, hid) or shapes["down"] != (hid, inter):
        return f"projection shapes {shapes} are not a gated MLP"
    if isinstance(geom[0], str):
        return _format_unsupported(geom, act_dtype, scale_dtype, w_dtype, inter, hid)
    bits, gs, roles = geom
    if gs & (gs - 1) or gs % (32 // bits):
        return f"group size {gs} is not a power of two holding whole {bits}-bit words"
    if _block_k(hid, gs) is None or _block_k(inter, gs) is None:
        return f"no tile divides hidden {hid} / intermediate {inter} at group size {gs}"
    for what, dt in (("activation", act_dtype), ("scale", scale_dtype),
                     ("routing-weight", w_dtype)):
        if dt not in _DTYPE_CODE:
            return f"{what} dtype {dt}"
    unit = 128 // bits                      # codes per 16-byte unit
    if gs % unit:
        return f"group size {gs} holds less than one 16-byte unit of {bits}-bit codes"
    if hid % (2 * unit) or inter % unit:
        return (f"hidden {hid} / intermediate {inter} is not whole (hidden: an even number "
                f"of) 16-byte units of codes")
    return None


def _format_unsupported(geom, act_dtype, scale_dtype, w_dtype, inter, hid):
    """Why the decode kernels cannot run an FP8 / MXFP4 blob, or None."""
    try:
        fmt, bits, group, brows = geom_format(geom)
    except (TypeError, ValueError):
        return f"code format {geom[0]!r}"
    if fmt == FMT_E4M3:
        if scale_dtype not in _DTYPE_CODE:
            return f"e4m3 scale dtype {scale_dtype}"
        if group & (group - 1) or group % 16 or brows & (brows - 1) or inter % brows or hid % brows:
            return f"e4m3 scale blocks {brows} x {group} do not tile {inter} x {hid}"
    elif fmt == FMT_MXFP4:
        if scale_dtype != torch.uint8:
            return f"mxfp4 scales are E8M0 bytes, not {scale_dtype}"
    else:
        return f"code format {geom[0]!r}"
    for what, dt in (("activation", act_dtype), ("routing-weight", w_dtype)):
        if dt not in _DTYPE_CODE:
            return f"{what} dtype {dt}"
    unit = 128 // bits
    if hid % (2 * unit) or inter % unit or hid % group or inter % group:
        return f"hidden {hid} / intermediate {inter} is not whole 16-byte units and scale groups"
    return None


def _table_values(pairs) -> list:
    """The pointer table, flattened: (packed address, scale address, slot) per pair
    (vaayu/packed_expert_kernels.py:349-352)."""
    return [v for blob, slot in pairs
            for v in (blob["flat"]["packed"].data_ptr(), blob["flat"]["scale"].data_ptr(), slot)]


def _aligned(pairs_or_blobs) -> bool:
    """The kernels read codes with 16-byte loads: every packed stream must start on 16 B."""
    return all(b["flat"]["packed"].data_ptr() % 16 == 0 for b in pairs_or_blobs)


def _gate_up(x, tbl, n, geom, sc, h=None):
    """h [n, intermediate] in the activation dtype: SiLU(gate) * up per table row
    (vaayu/packed_expert_kernels.py:355-371). `h` given: written in place (a graph
    capture must allocate nothing)."""
    lib = _require_backend()
    g = _lib.geom_struct(geom)
    if h is None:
        h = torch.empty(n, g.inter, dtype=x.dtype, device=x.device)
    rc = lib.vaayu_decode_gate_up(x.data_ptr(), tbl.data_ptr(), h.data_ptr(), n, g,
                                  _DTYPE_CODE[x.dtype], sc, _lib.stream_ptr(x.device))
    _lib.check(rc, "vaayu_decode_gate_up")
    return h


def _down(h, tbl, routing_weights, out, n, geom, sc) -> None:
    """`out` = the fp32 sum, in table order, of each row's down projection times its
    weight (vaayu/packed_expert_kernels.py:374-387). torch promotes `y * w` to fp32 unless
    the weight is already the activation dtype; only then does the product round."""
    lib = _require_backend()
    g = _lib.geom_struct(geom)
    rw = routing_weights.reshape(-1)
    if not rw.is_contiguous():
        rw = rw.contiguous()
    w_round = rw.dtype == h.dtype and h.dtype != torch.float32
    rc = lib.vaayu_decode_down(h.data_ptr(), tbl.data_ptr(), rw.data_ptr(), _DTYPE_CODE[rw.dtype],
                               out.data_ptr(), n, g, _DTYPE_CODE[h.dtype], sc, int(w_round),
                               _lib.stream_ptr(h.device))
    _lib.check(rc, "vaayu_decode_down")


def _launch(x, pairs, routing_weights, out) -> None:
    """The two decode kernels over `pairs`, into `out`. No checks: `_checked` gates this
    (vaayu/packed_expert_kernels.py:390-396)."""
    geom = pairs[0][0]["geom"]
    sc = _SCALE_CODE[pairs[0][0]["flat"]["scale"].dtype]
    tbl = _TABLES.put(_table_values(pairs), x.device)
    h = _gate_up(x, tbl, len(pairs), geom, sc)
    _down(h, tbl, routing_weights, out, len(pairs), geom, sc)


def stock_experts_decode(x, pairs, routing_weights, out, act_fn) -> None:
    """The per-slot loop's arithmetic for one token, pair by pair, into `out`: the
    reference the kernels are held to and their fallback (vaayu/packed_expert_kernels.py:
    399-410) -- dense weights, three `F.linear`, `act_fn`, the routing-weight product with
    torch's promotion, an fp32 add in pair order."""
    from .moe_patch import expert_weights_from_entry
    rw = routing_weights.reshape(-1)
    out.zero_()
    for blob, slot in pairs:
        w_gate, w_down, w_up = expert_weights_from_entry(blob, x.dtype)
        y = F.linear(act_fn(F.linear(x, w_gate)) * F.linear(x, w_up), w_down)
        out += (y * rw[slot:slot + 1]).to(out.dtype)


_REFERENCE = {"decode": "the stock per-expert loop",
              "prefill": "the per-expert loop with fp32-summed GEMMs"}


def _agrees(why, x, run_stock, run_kernel, what) -> bool:
    """True if the kernel agrees (relL2 <= _CHECK_TOL) with its reference on this call's
    data (vaayu/packed_expert_kernels.py:413-433). A refusal prints one WARNING naming
    `what`. A missing kernel library is not a disagreement: it raises."""
    if why is None:
        _require_backend()
        try:
            ref = torch.empty(x.shape, dtype=torch.float32, device=x.device)
            got = torch.empty_like(ref)
            run_stock(ref)
            run_kernel(got)
            err = ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()
            if not err <= _CHECK_TOL:
                why = (f"relL2 {err:.2e} vs {_REFERENCE[what]}, "
                       f"tolerance {_CHECK_TOL:.0e}")
        except Exception as exc:  # a rejected or failed launch
            why = f"{type(exc).__name__}: {exc}"
    if why is None:
        return True
    print(f"[Vaayu] WARNING: fused packed-expert {what} kernel refused ({why}); "
          f"these experts stay on the stock per-expert path")
    return False


def _verdict(x, pairs, routing_weights, act_fn) -> bool:
    """Run the kernels AND the stock arithmetic on this call's data; True if they agree
    (vaayu/packed_expert_kernels.py:440-447)."""
    blob = pairs[0][0]
    why = _unsupported(blob["geom"], x.dtype, blob["flat"]["scale"].dtype, routing_weights.dtype)
    return _agrees(why, x,
                   lambda ref: stock_experts_decode(x, pairs, routing_weights, ref, act_fn),
                   lambda got: _launch(x, pairs, routing_weights, got), "decode")


def _checked(x, pairs, routing_weights, act_fn) -> bool:
    """The cached verdict for this call's (geometry, dtypes) key, taken on first sight
    (vaayu/packed_expert_kernels.py:450-456)."""
    blob = pairs[0][0]
    key = (blob["geom"], x.dtype, routing_weights.dtype, blob["flat"]["scale"].dtype)
    if key not in _VERDICTS:
        _VERDICTS[key] = _verdict(x, pairs, routing_weights, act_fn)
    return _VERDICTS[key]


def packed_experts_decode(x, pairs, routing_weights, out, act_fn) -> None:
    """One token's routed-expert sum for one MoE layer, written into `out`
    (vaayu/packed_expert_kernels.py:459-480).

    x               [1, hidden], activation dtype, contiguous, on the current device
    pairs           [(blob, slot), ...] sorted by (expert id, slot): the fp32 sum's order
    routing_weights this token's [1, top_k] (or [top_k]) weights; `slot` indexes them
    out             [1, hidden] float32, overwritten
    act_fn          the experts' activation; only the stock fallback calls it

    Entries that are not all blobs of ONE geometry run the stock arithmetic."""
    geoms = {blob.get("geom") for blob, _slot in pairs}
    if len(geoms) != 1 or None in geoms or not _aligned(b for b, _s in pairs):
        stock_experts_decode(x, pairs, routing_weights, out, act_fn)
    elif _checked(x, pairs, routing_weights, act_fn):
        _launch(x, pairs, routing_weights, out)
    else:
        stock_experts_decode(x, pairs, routing_weights, out, act_fn)


# ── the decode kernels of one MoE layer as ONE graph (vaayu/packed_expert_kernels.py:483-654)
# A decode visit's inputs (x, the routing weights, the shared expert's output) are the same
# tensors every token under the engine's decode graphs, so the table upload, both launches
# and the epilogue are recorded once per layer and replayed with only the table's contents
# rewritten. Each capture is held bitwise to the eager launch.
_GRAPHS: dict = {}              # layer -> _LayerGraph
_GRAPH_REFUSED: dict = {}       # layer -> why
_GRAPH_WARNED: set = set()
_GRAPH_STREAMS: dict = {}       # device -> the capture stream
GRAPH_STATS: collections.Counter = collections.Counter()


class _LayerGraph:
    __slots__ = ("key", "graph", "host", "host_np", "tbl", "h", "out", "tmp", "result",
                 "done", "replays")


def _tail(out, dtype, shared):
    """The fused forward's epilogue: the fp32 sum cast back, plus the shared expert."""
    result = out.to(dtype)
    if shared is not None:
        result = result + shared.to(result.dtype)
    return result


def _refuse_graph(layer, why) -> None:
    _GRAPH_REFUSED[layer] = why
    _GRAPHS.pop(layer, None)
    GRAPH_STATS["refused"] += 1
    if why not in _GRAPH_WARNED:
        _GRAPH_WARNED.add(why)
        print(f"[Vaayu] WARNING: packed-expert decode graph refused for MoE layer {layer} "
              f"({why}); it launches eagerly. Later layers refused for the same reason are "
              f"not listed.")


def _warn_skip(why) -> None:
    """A call the graph cannot take launches eagerly; said once per reason."""
    if why not in _GRAPH_WARNED:
        _GRAPH_WARNED.add(why)
        print(f"[Vaayu] WARNING: packed-expert decode graph not used ({why}); those calls "
              f"launch the kernels eagerly. Shown once per reason.")


def packed_experts_decode_graphed(layer, x, pairs, routing_weights, shared, act_fn, tail):
    """`packed_experts_decode` (and, `tail` True, the forward's epilogue) through one graph
    per MoE layer -- or None: not the graph's call, run the eager path
    (vaayu/packed_expert_kernels.py:531-575). Returns a STATIC tensor the layer's next
    call overwrites: the fp32 sum [1, hidden], or `_tail(sum, x.dtype, shared)`."""
    if layer in _GRAPH_REFUSED:
        return None
    blob0 = pairs[0][0]
    geom = blob0.get("geom")
    if geom is None or any(blob.get("geom") != geom for blob, _slot in pairs[1:]):
        return None
    if not _aligned(b for b, _s in pairs):
        return None
    if not (x.is_contiguous() and routing_weights.is_contiguous()):
        _warn_skip("a non-contiguous expert input or routing-weight tensor")
        return None
    if tail and shared is not None and shared.dtype != x.dtype:
        _warn_skip(f"the shared expert's output is {shared.dtype}, the activations {x.dtype}")
        return None
    if not _checked(x, pairs, routing_weights, act_fn):
        return None
    vals = _table_values(pairs)
    key = (len(pairs), x.data_ptr(), routing_weights.data_ptr(), routing_weights.dtype,
           0 if shared is None else shared.data_ptr(), tail, geom, x.dtype,
           blob0["flat"]["scale"].dtype)
    g = _GRAPHS.get(layer)
    if g is not None and g.key == key:
        g.done.synchronize()            # the last replay has read the table
        g.host_np[:] = vals
        g.graph.replay()
        g.done.record()
        g.replays += 1
        GRAPH_STATS["replays"] += 1
        return g.result if tail else g.out
    if g is not None:
        del _GRAPHS[layer]
        if g.replays == 0:
            GRAPH_STATS["replaced_unreplayed"] += 1
        del g
    return _capture(layer, key, x, pairs, routing_weights, shared, tail, vals, act_fn)


def _cleanup_pool(pool) -> None:
    """Release a graph pool whose capture failed to end: torch's allocator otherwise
    keeps believing a capture records into it."""
    dev = torch.cuda.current_device()
    try:
        torch._C._cuda_endAllocateToPool(dev, pool)
    except Exception:
        pass
    try:
        torch._C._cuda_releasePool(dev, pool)
    except Exception:
        pass


def _capture(layer, key, x, pairs, rw, shared, tail, vals, act_fn):
    """Record the layer's graph, replay it once and hold it bitwise to the eager launch
    (vaayu/packed_expert_kernels.py:578-654). Nothing here raises into the request."""
    geom = pairs[0][0]["geom"]
    sc = _SCALE_CODE[pairs[0][0]["flat"]["scale"].dtype]
    n = len(pairs)
    inter = _layout(geom)["gate"][2]
    dev = x.device
    ref_out = torch.empty(x.shape, dtype=torch.float32, device=dev)
    _launch(x, pairs, rw, ref_out)
    ref = _tail(ref_out, x.dtype, shared) if tail else ref_out
    g = _LayerGraph()
    graph = torch.cuda.CUDAGraph()
    pool = torch.cuda.graph_pool_handle()
    was = gc.isenabled()
    gc.disable()
    try:
        g.key, g.replays = key, 0
        g.host = torch.empty(len(vals), dtype=torch.int64, pin_memory=True)
        g.host_np = g.host.numpy()
        g.host_np[:] = vals
        g.tbl = torch.empty(len(vals), dtype=torch.int64, device=dev)
        g.h = torch.empty(n, inter, dtype=x.dtype, device=dev)
        g.out = torch.empty(x.shape, dtype=torch.float32, device=dev)
        g.tmp = torch.empty(x.shape, dtype=x.dtype, device=dev) if tail else None
        g.result = (torch.empty(x.shape, dtype=x.dtype, device=dev)
                    if tail and shared is not None else g.tmp)
        g.done = torch.cuda.Event()
        side = _GRAPH_STREAMS.get(dev)
        if side is None:
            side = _GRAPH_STREAMS[dev] = torch.cuda.Stream(device=dev)
        cur = torch.cuda.current_stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side), torch.no_grad():
            graph.capture_begin(pool=pool, capture_error_mode="thread_local")
            try:
                g.tbl.copy_(g.host, non_blocking=True)
                _gate_up(x, g.tbl, n, geom, sc, h=g.h)
                _down(g.h, g.tbl, rw, g.out, n, geom, sc)
                if tail:
                    g.tmp.copy_(g.out)
                    if shared is not None:
                        torch.add(g.tmp, shared, out=g.result)
            finally:
                try:
                    graph.capture_end()
                except Exception:
                    _cleanup_pool(pool)
                    raise
        cur.wait_stream(side)
        g.graph = graph
        graph.replay()
        got = g.result if tail else g.out
        same = torch.equal(got, ref)
    except Exception as exc:
        first = (str(exc).splitlines() or [""])[0][:200]
        _refuse_graph(layer, f"capture failed: {type(exc).__name__}: {first}")
        return ref
    finally:
        if was:
            gc.enable()
    if not same:
        _refuse_graph(layer, "its replay disagrees bitwise with the eager launch")
        return ref
    g.done.record()
    _GRAPHS[layer] = g
    GRAPH_STATS["captures"] += 1
    return got


# ── prefill ─────────────────────────────────────────────────────────────────────────────

def _prefill_unsupported(geom, act_dtype, scale_dtype, w_dtype):
    """Why the grouped prefill kernels cannot run this geometry, or None
    (vaayu/packed_expert_kernels.py:657-673): the decode rules, no fp32 activations, and
    an MFMA K step -- 4 lanes' 16-byte units -- that divides hidden and intermediate."""
    why = _unsupported(geom, act_dtype, scale_dtype, w_dtype)
    if why is not None:
        return why
    if isinstance(geom[0], str):                 # FP8 e4m3 / MXFP4 blobs
        if act_dtype == torch.float32:
            return "fp32 activations (the matrix cores would run them at reduced precision)"
        _fmt, bits, _group, _brows = geom_format(geom)
        lay = _layout(geom)
        step = 4 * (128 // bits)
        for what, k in (("hidden", lay["gate"][3]), ("intermediate", lay["gate"][2])):
            if k % step:
                return f"{what} {k} is not a multiple of the {step}-code K tile"
        return None
    bits, gs, _roles = geom
    lay = _layout(geom)
    inter, hid = lay["gate"][2], lay["gate"][3]
    if act_dtype == torch.float32:
        return "fp32 activations (the matrix cores would run them at reduced precision)"
    if bits not in (4, 8):
        return f"{bits}-bit codes (the grouped kernels take 4 and 8)"
    step = 4 * (128 // bits)
    for what, k in (("hidden", hid), ("intermediate", inter)):
        if _block_k(k, gs, min(_PF_GU_BK_MAX, _PF_DN_BK_MAX)) // (32 // bits) < _PF_MIN_TILE:
            return f"{what} {k} at group size {gs} leaves a K tile under {_PF_MIN_TILE} words"
        if k % step:
            return f"{what} {k} is not a multiple of the {step}-code K tile"
    return None


def _prefill_plan(eidx_cpu):
    """(order, live, counts) of one call's routing (vaayu/packed_expert_kernels.py:676-688):
    row ids (token*top_k + slot) stable-sorted by expert id, the routed ids ascending,
    and rows per routed expert."""
    eids = eidx_cpu.reshape(-1)
    order = torch.argsort(eids, stable=True)
    per_expert = torch.bincount(eids)
    live = per_expert.nonzero().reshape(-1)
    return order, live, per_expert[live]


def _prefill_tables(eidx_cpu, plan, blobs, device):
    """The call's three tables on the device from ONE pinned copy
    (vaayu/packed_expert_kernels.py:691-717): (tbl, rows, ord, n_blocks).

    tbl   [n_blocks, 2] (packed address, scale address) of each block's expert
    rows  [n_blocks, _PF_BLOCK_M] row ids, each expert's run padded to whole blocks with -1
    ord   [tokens, top_k] row ids of each token's slots in ascending expert id"""
    order, live, counts = plan
    n, top_k = eidx_cpu.shape
    nblk = (counts + _PF_BLOCK_M - 1) // _PF_BLOCK_M
    blk_end = nblk.cumsum(0)
    n_blocks = int(blk_end[-1])
    owner = torch.repeat_interleave(torch.arange(live.numel()), counts)
    first_row = counts.cumsum(0) - counts
    dest = (((blk_end - nblk) * _PF_BLOCK_M)[owner] + torch.arange(order.numel())
            - first_row[owner])
    rows = torch.full((n_blocks * _PF_BLOCK_M,), -1, dtype=torch.int64)
    rows[dest] = order
    ptrs = torch.tensor([(blobs[e]["flat"]["packed"].data_ptr(),
                          blobs[e]["flat"]["scale"].data_ptr()) for e in live.tolist()],
                        dtype=torch.int64)
    tbl = ptrs[torch.repeat_interleave(torch.arange(live.numel()), nblk)].reshape(-1)
    slot_order = (torch.argsort(eidx_cpu, dim=1, stable=True)
                  + (torch.arange(n) * top_k)[:, None]).reshape(-1)
    dev = _PF_TABLES.put(torch.cat([tbl, rows, slot_order]), device)
    a, b = tbl.numel(), tbl.numel() + rows.numel()
    return dev[:a], dev[a:b], dev[b:b + slot_order.numel()], n_blocks


def _gate_up_g(x, tbl, rows, n_blocks, top_k, geom, sc, h=None):
    """h [tokens * top_k, intermediate], activation dtype: SiLU(gate) * up per live row
    (vaayu/packed_expert_kernels.py:720-732)."""
    lib = _require_backend()
    g = _lib.geom_struct(geom)
    if h is None:
        h = torch.empty(x.shape[0] * top_k, g.inter, dtype=x.dtype, device=x.device)
    rc = lib.vaayu_prefill_gate_up(x.data_ptr(), rows.data_ptr(), tbl.data_ptr(), h.data_ptr(),
                                   n_blocks, top_k, g, _DTYPE_CODE[x.dtype], sc,
                                   _lib.stream_ptr(x.device))
    _lib.check(rc, "vaayu_prefill_gate_up")
    return h


def _down_g(h, tbl, rows, n_blocks, routing_weights, geom, sc, y=None):
    """y [tokens * top_k, hidden] fp32: each live row's down projection times its weight
    (vaayu/packed_expert_kernels.py:735-749)."""
    lib = _require_backend()
    g = _lib.geom_struct(geom)
    rw = routing_weights.reshape(-1).contiguous()
    if y is None:
        y = torch.empty(h.shape[0], g.hidden, dtype=torch.float32, device=h.device)
    w_round = rw.dtype == h.dtype and h.dtype != torch.float32
    rc = lib.vaayu_prefill_down(h.data_ptr(), rows.data_ptr(), tbl.data_ptr(), rw.data_ptr(),
                                _DTYPE_CODE[rw.dtype], y.data_ptr(), n_blocks, g,
                                _DTYPE_CODE[h.dtype], sc, int(w_round), _lib.stream_ptr(h.device))
    _lib.check(rc, "vaayu_prefill_down")
    return y


def _reduce(y, order, out, top_k) -> None:
    """`out` [tokens, hidden] fp32 = each token's contributions summed in `order`
    (vaayu/packed_expert_kernels.py:752-757)."""
    lib = _require_backend()
    rc = lib.vaayu_prefill_reduce(y.data_ptr(), order.data_ptr(), out.data_ptr(), out.shape[0],
                                  top_k, y.shape[1], _lib.stream_ptr(y.device))
    _lib.check(rc, "vaayu_prefill_reduce")


def _prefill_launch(x, eidx_cpu, routing_weights, blobs, out, plan=None) -> None:
    """The three prefill kernels over one call. No checks: `_prefill_checked` gates this
    (vaayu/packed_expert_kernels.py:760-777). A strided `x` is made dense first; a
    strided `out` is written through a dense temporary."""
    plan = plan or _prefill_plan(eidx_cpu)
    blob = blobs[int(plan[1][0])]
    geom, sc = blob["geom"], _SCALE_CODE[blob["flat"]["scale"].dtype]
    top_k = eidx_cpu.shape[1]
    x = x.contiguous()
    tbl, rows, order, n_blocks = _prefill_tables(eidx_cpu, plan, blobs, x.device)
    h = _gate_up_g(x, tbl, rows, n_blocks, top_k, geom, sc)
    y = _down_g(h, tbl, rows, n_blocks, routing_weights, geom, sc)
    if out.is_contiguous():
        _reduce(y, order, out, top_k)
    else:
        dense = torch.empty(out.shape, dtype=torch.float32, device=out.device)
        _reduce(y, order, dense, top_k)
        out.copy_(dense)


def _linear_fp32(a, w):
    """`F.linear` with the product summed in fp32 and rounded ONCE to the activation dtype."""
    return F.linear(a.float(), w.float()).to(a.dtype)


def stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn,
                          linear=F.linear) -> None:
    """The per-slot loop's arithmetic for a multi-token call, into `out`
    (vaayu/packed_expert_kernels.py:785-814): per expert in id order, gather its rows,
    dense weights, three `linear`s, `act_fn`, the routing-weight product, `index_add_`.
    A routed expert with no entry is skipped. `linear=_linear_fp32` is the reference the
    kernels are checked against."""
    from .moe_patch import expert_weights_from_entry
    order, live, counts = _prefill_plan(eidx_cpu)
    top_k = eidx_cpu.shape[1]
    rw = routing_weights.reshape(-1)
    order = order.to(x.device)
    out.zero_()
    at = 0
    for e, c in zip(live.tolist(), counts.tolist()):
        rows = order[at:at + c]
        at += c
        entry = blobs.get(e)
        if entry is None:
            continue
        w_gate, w_down, w_up = expert_weights_from_entry(entry, x.dtype)
        tok = rows // top_k
        xs = x[tok]
        y = linear(act_fn(linear(xs, w_gate)) * linear(xs, w_up), w_down)
        out.index_add_(0, tok, (y * rw[rows, None]).to(out.dtype))


def _prefill_verdict(x, eidx_cpu, routing_weights, blobs, act_fn, plan) -> bool:
    """Run the grouped kernels AND the fp32-GEMM stock arithmetic on this call's data
    (vaayu/packed_expert_kernels.py:817-826)."""
    blob = blobs[int(plan[1][0])]
    why = _prefill_unsupported(blob["geom"], x.dtype, blob["flat"]["scale"].dtype,
                               routing_weights.dtype)
    return _agrees(
        why, x,
        lambda ref: stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, ref, act_fn,
                                          linear=_linear_fp32),
        lambda got: _prefill_launch(x, eidx_cpu, routing_weights, blobs, got, plan), "prefill")


def _prefill_checked(x, eidx_cpu, routing_weights, blobs, act_fn, plan) -> bool:
    """The cached verdict for this call's (geometry, dtypes) key
    (vaayu/packed_expert_kernels.py:829-835)."""
    blob = blobs[int(plan[1][0])]
    key = (blob["geom"], x.dtype, routing_weights.dtype, blob["flat"]["scale"].dtype)
    if key not in _PF_VERDICTS:
        _PF_VERDICTS[key] = _prefill_verdict(x, eidx_cpu, routing_weights, blobs, act_fn, plan)
    return _PF_VERDICTS[key]


def packed_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn) -> None:
    """A multi-token call's routed-expert sum for one MoE layer, written into `out`
    (vaayu/packed_expert_kernels.py:838-861).

    x               [tokens, hidden], activation dtype (a strided view is fine)
    eidx_cpu        [tokens, top_k] int64 on the CPU: the routed expert ids
    routing_weights [tokens, top_k] on x's device; row t*top_k + s weighs slot s of token t
    blobs           {expert id: entry}; anything but blobs of one geometry for every
                    routed expert sends the whole call to the stock arithmetic
    out             [tokens, hidden] float32, overwritten (a strided view is fine)"""
    plan = _prefill_plan(eidx_cpu)
    geoms = {blobs[e].get("geom") if e in blobs else None for e in plan[1].tolist()}
    if (len(geoms) != 1 or None in geoms
            or not _aligned(blobs[e] for e in plan[1].tolist())):
        stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn)
    elif _prefill_checked(x, eidx_cpu, routing_weights, blobs, act_fn, plan):
        _prefill_launch(x, eidx_cpu, routing_weights, blobs, out, plan)
    else:
        stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn)


# ── load-time install ─────────────────────────────────────────────────────────────────────

def _is_silu(act_fn, device, dtype) -> bool:
    """Behavioural: does the experts' activation compute SiLU? (the kernels hardcode it)"""
    if act_fn is None:
        return False
    t = torch.linspace(-8.0, 8.0, 257, device=device).to(dtype)
    try:
        return torch.equal(act_fn(t), F.silu(t))
    except Exception:
        return False


_ST_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32,
              "I32": torch.int32, "I64": torch.int64, "U8": torch.uint8, "I8": torch.int8}


def _read_expert_tensors(path: str, metas: dict) -> dict:
    """{key: cpu tensor} for one expert's tensors of a safetensors shard, read at the byte
    ranges the engine's offset index records (file_offset, byte_length, shape, dtype)."""
    out = {}
    with open(path, "rb") as f:
        for key, m in metas.items():
            f.seek(m.file_offset)
            buf = bytearray(f.read(m.byte_length))
            t = torch.frombuffer(buf, dtype=_ST_DTYPES[m.dtype]) if buf else torch.empty(0)
            out[key] = t.reshape(m.shape).clone()
    return out


def _one_real_blob(vaayu_ref, block, device, quiet=False):
    """The blob of `block`'s lowest-numbered expert read off the checkpoint, or None when
    its experts are not pack-quantized (vaayu/packed_expert_kernels.py:875-899)."""
    from .moe_patch import (_group_packed_tensors_by_weight, _packed_roles_complete,
                            _upload_packed_expert, build_expert_blob)
    metas = vaayu_ref._expert_offset_index.index.get(block.layer_name, {})
    if not metas:
        return None
    path = str(Path(vaayu_ref.checkpoint_path) / f"{block.layer_name}.safetensors")
    try:     # inside the engine, its own reader (io_uring, pinned buffers)
        from vaayu.persist.safetensor_model_persister import load_expert_sparse
    except ImportError:
        load_expert_sparse = _read_expert_tensors
    raw = load_expert_sparse(path, metas[min(metas)])
    packed = _group_packed_tensors_by_weight(raw)
    if not packed["gate"] or not _packed_roles_complete(packed):
        return None
    why = "its projections are packed at different bit widths or group sizes"
    try:
        blob = build_expert_blob(_upload_packed_expert(packed, device))
    except NotImplementedError as exc:
        blob, why = None, str(exc)
    if blob is None and not quiet:
        print(f"[Vaayu] WARNING: fused packed-expert decode kernel not installed: {why}")
    return blob


_PREFILL_VRAM_HEADROOM = 4 << 30


def install_packed_expert_kernels(vaayu_ref) -> bool:
    """Route the fused pack-quantized MoE blocks through the kernels if they agree with
    the stock arithmetic on one real expert of this model on this device
    (vaayu/packed_expert_kernels.py:902-1012). Sets `vaayu_ref._packed_moe_kernel` (decode)
    and `vaayu_ref._packed_moe_prefill_kernel` (the eligible prefill layers); returns
    whether the decode kernel was installed."""
    device = str(vaayu_ref.running_device)
    if torch.device(device).type != "cuda":
        return False
    if triton is None:
        if torch.cuda.is_available():
            print(f"[Vaayu] WARNING: fused packed-expert kernels not installed: "
                  f"{globals().get('_LOAD_ERROR', 'the kernel library is absent')}")
        return False
    blocks = [b for b in (getattr(vaayu_ref, "_moe_blocks", None) or [])
              if getattr(b, "forward_name", None) == "_make_fused_sparse_forward"]
    if not blocks or getattr(vaayu_ref, "_expert_offset_index", None) is None:
        return False
    dev_index = torch.device(device).index
    if dev_index is not None and dev_index != torch.cuda.current_device():
        print(f"[Vaayu] WARNING: fused packed-expert decode kernel not installed: model "
              f"device {device} is not the current GPU ({torch.cuda.current_device()}); "
              f"decode keeps the stock per-expert path")
        return False
    block, dtype = blocks[0], vaayu_ref.running_dtype
    act_fn = getattr(getattr(block.moe_module, block.experts_attr, None), "act_fn", None)
    if not _is_silu(act_fn, device, dtype):
        print("[Vaayu] fused packed-expert decode kernel not used: the experts' activation "
              "is not SiLU")
        return False
    blob = _one_real_blob(vaayu_ref, block, device)
    if blob is None:
        return False
    k = int(getattr(vaayu_ref, "moe_top_k", 0) or 1)
    gen = torch.Generator(device=device).manual_seed(0)
    x = (torch.randn(1, _layout(blob["geom"])["gate"][3], generator=gen, device=device)
         * 0.5).to(dtype)
    w = torch.rand(1, k, generator=gen, device=device) + 0.1
    w = w / w.sum(-1, keepdim=True)
    pairs = [(blob, s) for s in range(k)]
    if not all(_checked(x, pairs, rw, act_fn) for rw in (w, w.to(dtype))):
        return False
    vaayu_ref._packed_moe_kernel = blob["geom"]
    bits, gs, _roles = blob["geom"]
    print(f"[Vaayu] fused packed-expert decode kernel on {len(blocks)} MoE layers "
          f"({bits}-bit, group {gs})")
    try:
        from vaayu.moe_patch import _PREFILL_VRAM_HEADROOM as headroom
    except ImportError:
        headroom = _PREFILL_VRAM_HEADROOM
    checked = (blob["geom"], blob["flat"]["scale"].dtype)
    eligible, skipped = [], {}
    for b in blocks:
        one = blob if b is block else _one_real_blob(vaayu_ref, b, device, quiet=True)
        if one is None:
            why = "experts not pack-quantized, or packed with no fused pass"
        elif (one["geom"], one["flat"]["scale"].dtype) != checked:
            why = "a different geometry or scale dtype than the checked layer"
        else:
            n_experts = int(getattr(getattr(b.moe_module, b.experts_attr), "num_experts", 0))
            held = n_experts * sum(t.numel() * t.element_size() for t in one["flat"].values())
            if n_experts and held <= headroom // 2:
                eligible.append(b.layer_idx)
                continue
            why = (f"one call can hold a layer's {n_experts} experts on the GPU at once "
                   f"({held / 2**30:.2f} GiB), over half the "
                   f"{headroom / 2**30:.2f} GiB prefill headroom")
        skipped.setdefault(why, []).append(b.layer_idx)
    if not eligible:
        print(f"[Vaayu] WARNING: fused packed-expert prefill kernel not installed: "
              f"{'; '.join(skipped)}; prefill keeps the per-expert path")
        return True
    tokens = _PF_BLOCK_M + _PF_BLOCK_M // 2
    eidx = torch.stack([torch.roll(torch.arange(k), t) for t in range(tokens)])
    xs = (torch.randn(tokens, x.shape[1], generator=gen, device=device) * 0.5).to(dtype)
    ws = torch.rand(tokens, k, generator=gen, device=device) + 0.1
    ws = ws / ws.sum(-1, keepdim=True)
    blobs = {e: blob for e in range(k)}
    plan = _prefill_plan(eidx)
    if all(_prefill_checked(xs, eidx, rw, blobs, act_fn, plan) for rw in (ws, ws.to(dtype))):
        vaayu_ref._packed_moe_prefill_kernel = frozenset(eligible)
        print(f"[Vaayu] fused packed-expert prefill kernel on {len(eligible)} MoE layers "
              f"({bits}-bit, group {gs})")
        if skipped:
            left_out = sorted(i for idxs in skipped.values() for i in idxs)
            whys = "; ".join(
                why if len(skipped) == 1 else f"{why} (layers {', '.join(map(str, idxs))})"
                for why, idxs in skipped.items())
            print(f"[Vaayu] WARNING: fused packed-expert prefill kernel not used on "
                  f"{len(left_out)} of {len(blocks)} MoE layers (layer indices "
                  f"{', '.join(map(str, left_out))}): {whys}; prefill keeps the per-expert "
                  f"path there")
    return True
