"""Packed-expert routed-MoE kernels for MI355X: the drop-in for Vaayu's
`vaayu/packed_expert_kernels.py`.

The engine's fused forward (vaayu/moe_patch.py:2394-2401, 2608-2624) and its installer call
(vaayu/vaayu_base.py:3560) reach this module through the reference's names, arguments,
results, table formats and WARNING lines; the arithmetic runs in hand-written gfx950 HIP
kernels behind a C ABI (vaayu_amd/csrc, include/vaayu_amd.h):

  decode  (one token)  `vaayu_decode_gate_up` + `vaayu_decode_down`: GEMVs over (blob, slot)
                       pairs, codes dequantized in registers, the fp32 sum over pairs in
                       table order.
  prefill (a call of   `vaayu_prefill_gate_up` + `vaayu_prefill_down` + `vaayu_prefill_reduce`:
   any length)         grouped GEMMs on MFMA over 16-row blocks of one expert each, then each
                       token's contributions summed in ascending expert id.

How the host side is organised here:

  * `_UploadPool` stages each call's int64 tables through pinned lanes that are reused only
    after the copy that last read them has completed.
  * Support rules are small reason-returning checks (`_unsupported`, `_prefill_unsupported`);
    a call's first sight of a (geometry, dtypes) key runs kernels and stock arithmetic side
    by side once, and the answer is kept in `_VERDICTS` / `_PF_VERDICTS`.
  * `_LayerGraph` owns one MoE layer's recorded decode launches and their static buffers.
  * `_prefill_launch` splits a call whose activation or intermediate rows would not fit the
    kernels' 32-bit row offsets into token chunks (bit-identical: a row's arithmetic does not
    depend on the rows it shares a launch with).
  * `install_packed_expert_kernels` is a sequence of stages (preconditions, the decode
    verdict, per-layer prefill eligibility, the prefill verdict).

Every value the stock path stores in the activation dtype is rounded to it at the same
point, and nothing is accumulated atomically. Without the built library
(vaayu_amd/libvaayu_amd.so) every kernel entry raises ImportError naming the file.
"""
import collections
import gc
import itertools
from typing import NamedTuple
from pathlib import Path

import torch
import torch.nn.functional as F

from . import _lib
from .block_formats import FMT_E4M3, FMT_MXFP4, blob_layout, geom_format

try:
    _lib.load()
    _BACKEND, _LOAD_ERROR = _lib, None
except ImportError as _exc:              # reported at the first kernel call / install
    _BACKEND, _LOAD_ERROR = None, str(_exc)

# The kernel backend's truthiness under the name the engine's installer and its tests use
# (they set it to None to stand for a machine without the kernels).
triton = _BACKEND

_CHECK_TOL = 1e-2            # relL2 of a call's output vs its reference above which: refused
_BK_MAX = 512
_PF_BLOCK_M = 16             # rows per block of the prefill tables
_XCDS = 8                    # MI355X's accelerator dies: workgroup L runs on XCD L % 8
_PF_MIN_TILE = 16
_PF_GU_BK_MAX, _PF_DN_BK_MAX = 256, 256
_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
# Scale dtypes the kernels read: the activation dtypes, and E8M0 bytes (MXFP4 blobs).
_SCALE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.uint8: 3}
_ROLES = ("gate", "down", "up")
# Byte span the grouped kernels address with 32-bit row offsets (activation rows x, and
# intermediate rows h); a prefill call past it is launched in token chunks. Read at call
# time, so a test can lower it.
_OFFSET_LIMIT = 0xF0000000


def _require_backend():
    if triton is None:
        raise ImportError(_LOAD_ERROR or "vaayu_amd kernels unavailable")
    return _lib.load()


# ── pinned staging of the per-call tables ───────────────────────────────────────────────

def _pow2_at_least(n: int, floor: int = 64) -> int:
    return max(floor, 1 << max(n - 1, 0).bit_length())


def _same_device(a: torch.device, b) -> bool:
    b = torch.device(b)
    if b.type == "cuda" and b.index is None:
        b = torch.device("cuda", torch.cuda.current_device())
    return a == b


class _UploadLane:
    """One pinned int64 host buffer, its device twin, and the event recorded after the last
    copy out of the host buffer (which must not be rewritten before that copy is done)."""
    __slots__ = ("host", "dev", "copied", "in_flight")

    def __init__(self, capacity: int, device):
        self.host = torch.empty(capacity, dtype=torch.int64, pin_memory=True)
        self.dev = torch.empty(capacity, dtype=torch.int64, device=device)
        self.copied = torch.cuda.Event()
        self.in_flight = False

    def fits(self, n: int, device) -> bool:
        return self.host.numel() >= n and _same_device(self.dev.device, device)

    def upload(self, values) -> torch.Tensor:
        n = len(values)
        if self.in_flight:
            self.copied.synchronize()
        self.host[:n] = torch.as_tensor(values, dtype=torch.int64)
        self.dev[:n].copy_(self.host[:n], non_blocking=True)
        self.copied.record()
        self.in_flight = True
        return self.dev


class _UploadPool:
    """Round-robin lanes (vaayu/packed_expert_kernels.py:263-292 stages the same way): each
    call's table gets its own device buffer, so a table still queued for a kernel is never
    overwritten, and a lane's pinned buffer is reused only after its copy completed. Lanes
    grow to the next power of two (prefill tables change length call to call)."""

    def __init__(self, depth: int = 4):
        self._slots: list = [None] * depth
        self._turn = itertools.cycle(range(depth))

    def put(self, values, device) -> torch.Tensor:
        """A device int64 tensor whose first len(values) entries hold `values` once the
        stream reaches this point."""
        i = next(self._turn)
        lane = self._slots[i]
        if lane is None or not lane.fits(len(values), device):
            lane = self._slots[i] = _UploadLane(_pow2_at_least(len(values)), device)
        return lane.upload(values)


_TABLES = _UploadPool()
_PF_TABLES = _UploadPool()
_VERDICTS: dict = {}
_PF_VERDICTS: dict = {}


# ── geometry and support rules ──────────────────────────────────────────────────────────

def _layout(geom) -> dict:
    """{role: (word offset, scale offset, rows, cols)} inside a blob's flat streams
    (vaayu/packed_expert_kernels.py:301-309); FP8 / MXFP4 blobs by their own scale
    blocking (vaayu_amd.block_formats)."""
    if isinstance(geom[0], str):
        return blob_layout(geom)
    bits, gs, roles = geom
    out, words, scales = {}, 0, 0
    for role, rows, cols in roles:
        out[role] = (words, scales, rows, cols)
        words += rows * cols * bits // 32
        scales += rows * cols // gs
    return out


def _block_k(k: int, gs: int, cap: int = _BK_MAX):
    """The largest power-of-two multiple of the group size, at most max(cap, gs), that
    divides k (vaayu/packed_expert_kernels.py:312-319); None if none does."""
    fitting = [b for b in (gs << s for s in range(32)) if b <= max(cap, gs) and k % b == 0]
    return fitting[-1] if fitting else None


def _pow2_divisor(n: int, cap: int) -> int:
    """The largest power of two at most `cap` dividing n."""
    while n % cap:
        cap //= 2
    return cap


def _gated_mlp(geom):
    """(intermediate, hidden) of a gate/up/down geometry, or the reason it is not one."""
    shapes = {role: (rows, cols) for role, rows, cols in geom[2]}
    if set(shapes) != set(_ROLES):
        return f"expert roles {sorted(shapes)} are not gate/up/down"
    inter, hid = shapes["gate"]
    if shapes["up"] != (inter, hid) or shapes["down"] != (hid, inter):
        return f"projection shapes {shapes} are not a gated MLP"
    return inter, hid


def _first(*checks):
    """The first reason (a non-empty string) the checks give, or None; each check is a
    zero-argument callable, called only if every earlier one passed."""
    for check in checks:
        why = check()
        if why:
            return why
    return None


def _dtype_reason(**dtypes):
    for what, dt in dtypes.items():
        if dt not in _DTYPE_CODE:
            return f"{what.replace('_', '-')} dtype {dt}"
    return None


def _unsupported(geom, act_dtype, scale_dtype, w_dtype):
    """Why the decode kernels cannot run this geometry with these dtypes, or None.

    The reference's rules (vaayu/packed_expert_kernels.py:329-346) -- a gated MLP, a
    power-of-two group of whole words, a K tile dividing both dims, dtypes among
    bf16/fp16/fp32 -- plus what the HIP GEMV reads: whole 16-byte units of codes, each
    within one group."""
    mlp = _gated_mlp(geom)
    if isinstance(mlp, str):
        return mlp
    inter, hid = mlp
    if isinstance(geom[0], str):
        return _format_unsupported(geom, act_dtype, scale_dtype, w_dtype, inter, hid)
    bits, gs, _roles = geom
    unit = 128 // bits                                  # codes per 16-byte unit
    return _first(
        lambda: (gs & (gs - 1) or gs % (32 // bits))
        and f"group size {gs} is not a power of two holding whole {bits}-bit words",
        lambda: (_block_k(hid, gs) is None or _block_k(inter, gs) is None)
        and f"no tile divides hidden {hid} / intermediate {inter} at group size {gs}",
        lambda: _dtype_reason(activation=act_dtype, scale=scale_dtype,
                              routing_weight=w_dtype),
        lambda: gs % unit
        and f"group size {gs} holds less than one 16-byte unit of {bits}-bit codes",
        lambda: (hid % (2 * unit) or inter % unit)
        and (f"hidden {hid} / intermediate {inter} is not whole (hidden: an even number "
             f"of) 16-byte units of codes"))


def _format_unsupported(geom, act_dtype, scale_dtype, w_dtype, inter, hid):
    """Why the decode kernels cannot run an FP8 / MXFP4 blob, or None."""
    try:
        fmt, bits, group, brows = geom_format(geom)
    except (TypeError, ValueError):
        return f"code format {geom[0]!r}"
    if fmt == FMT_E4M3:
        scale_rule = lambda: (  # noqa: E731
            (scale_dtype not in _DTYPE_CODE and f"e4m3 scale dtype {scale_dtype}")
            or ((group & (group - 1) or group % 16 or brows & (brows - 1) or inter % brows
                 or hid % brows)
                and f"e4m3 scale blocks {brows} x {group} do not tile {inter} x {hid}"))
    elif fmt == FMT_MXFP4:
        scale_rule = lambda: (scale_dtype != torch.uint8  # noqa: E731
                              and f"mxfp4 scales are E8M0 bytes, not {scale_dtype}")
    else:
        return f"code format {geom[0]!r}"
    unit = 128 // bits
    return _first(
        scale_rule,
        lambda: _dtype_reason(activation=act_dtype, routing_weight=w_dtype),
        lambda: (hid % (2 * unit) or inter % unit or hid % group or inter % group)
        and f"hidden {hid} / intermediate {inter} is not whole 16-byte units and scale groups")


def _prefill_unsupported(geom, act_dtype, scale_dtype, w_dtype):
    """Why the grouped prefill kernels cannot run this geometry, or None
    (vaayu/packed_expert_kernels.py:657-673): the decode rules, no fp32 activations, and
    an MFMA K step -- 4 lanes' 16-byte units -- that divides hidden and intermediate."""
    why = _unsupported(geom, act_dtype, scale_dtype, w_dtype)
    if why:
        return why
    if act_dtype == torch.float32:
        return "fp32 activations (the matrix cores would run them at reduced precision)"
    lay = _layout(geom)
    dims = (("hidden", lay["gate"][3]), ("intermediate", lay["gate"][2]))
    if isinstance(geom[0], str):                 # FP8 e4m3 / MXFP4 blobs
        step = 4 * (128 // geom_format(geom)[1])
        return _first(*(lambda what=what, k=k: k % step
                        and f"{what} {k} is not a multiple of the {step}-code K tile"
                        for what, k in dims))
    bits, gs, _roles = geom
    if bits not in (4, 8):
        return f"{bits}-bit codes (the grouped kernels take 4 and 8)"
    step = 4 * (128 // bits)
    tile_cap = min(_PF_GU_BK_MAX, _PF_DN_BK_MAX)

    def k_rules(what, k):
        return (lambda: _block_k(k, gs, tile_cap) // (32 // bits) < _PF_MIN_TILE
                and f"{what} {k} at group size {gs} leaves a K tile under {_PF_MIN_TILE} words",
                lambda: k % step and f"{what} {k} is not a multiple of the {step}-code K tile")
    return _first(*(rule for what, k in dims for rule in k_rules(what, k)))


def _aligned(blobs) -> bool:
    """The kernels read codes with 16-byte loads: every packed stream must start on 16 B."""
    return all(b["flat"]["packed"].data_ptr() % 16 == 0 for b in blobs)


def _kernel_ready(blobs) -> bool:
    """The entries are blobs of ONE geometry, each aligned for the kernels' loads."""
    blobs = list(blobs)
    geoms = {b.get("geom") for b in blobs}
    return len(geoms) == 1 and None not in geoms and _aligned(blobs)


def _scale_code(blob) -> int:
    return _SCALE_CODE[blob["flat"]["scale"].dtype]


# ── verdicts: kernels against the stock arithmetic, once per key ─────────────────────────

_REFERENCE = {"decode": "the stock per-expert loop",
              "prefill": "the per-expert loop with fp32-summed GEMMs"}


def _disagreement(x, fill_reference, fill_candidate, kind):
    """Why the candidate's fp32 output (relL2) does not match the reference's on this call,
    or None. A failed launch is a disagreement too."""
    try:
        want = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        got = torch.empty_like(want)
        fill_reference(want)
        fill_candidate(got)
        err = ((got - want).norm() / want.norm().clamp_min(1e-30)).item()
    except Exception as exc:  # a rejected or failed launch
        return f"{type(exc).__name__}: {exc}"
    if err <= _CHECK_TOL:                 # False for NaN: a NaN output is refused
        return None
    return f"relL2 {err:.2e} vs {_REFERENCE[kind]}, tolerance {_CHECK_TOL:.0e}"


def _judge(kind, x, why, fill_reference, fill_candidate) -> bool:
    """The verdict on one call (vaayu/packed_expert_kernels.py:413-433): True if the
    kernels may run it. A refusal prints one WARNING naming `kind`; a missing kernel
    library is not a refusal, it raises."""
    if why is None:
        _require_backend()
        why = _disagreement(x, fill_reference, fill_candidate, kind)
    if why is not None:
        print(f"[Vaayu] WARNING: fused packed-expert {kind} kernel refused ({why}); "
              f"these experts stay on the stock per-expert path")
    return why is None


def _remembered(book_name: str, key, decide) -> bool:
    """The verdict kept in the module dict `book_name` for `key`, decided on first sight.
    The dict is looked up by name at call time (tests swap in fresh ones)."""
    book = globals()[book_name]
    if key not in book:
        book[key] = decide()
    return book[key]


def _verdict_key(blob, x, routing_weights):
    return (blob["geom"], x.dtype, routing_weights.dtype, blob["flat"]["scale"].dtype)


# ── decode ──────────────────────────────────────────────────────────────────────────────

def _table_values(pairs) -> list:
    """The decode pointer table, flattened: (packed address, scale address, slot) per pair
    (vaayu/packed_expert_kernels.py:349-352)."""
    return [v for blob, slot in pairs
            for v in (blob["flat"]["packed"].data_ptr(), blob["flat"]["scale"].data_ptr(), slot)]


def _gate_up(x, tbl, n, geom, sc, h=None):
    """h [n, intermediate] in the activation dtype: SiLU(gate) * up per table row
    (vaayu/packed_expert_kernels.py:355-371). `h` given: written in place (a graph
    capture must allocate nothing)."""
    lib = _require_backend()
    g = _lib.geom_struct(geom)
    if h is None:
        h = torch.empty(n, g.inter, dtype=x.dtype, device=x.device)
    _lib.check(lib.vaayu_decode_gate_up(x.data_ptr(), tbl.data_ptr(), h.data_ptr(), n, g,
                                        _DTYPE_CODE[x.dtype], sc, _lib.stream_ptr(x.device)),
               "vaayu_decode_gate_up")
    return h


def _rounds_weighted(weight_dtype, act_dtype) -> bool:
    """torch promotes `y * w` to fp32 unless the weight is already the (half-precision)
    activation dtype; only then does the product round."""
    return weight_dtype == act_dtype and act_dtype != torch.float32


def _down(h, tbl, routing_weights, out, n, geom, sc) -> None:
    """`out` = the fp32 sum, in table order, of each row's down projection times its weight
    (vaayu/packed_expert_kernels.py:374-387)."""
    lib = _require_backend()
    rw = routing_weights.reshape(-1).contiguous()
    _lib.check(lib.vaayu_decode_down(h.data_ptr(), tbl.data_ptr(), rw.data_ptr(),
                                     _DTYPE_CODE[rw.dtype], out.data_ptr(), n,
                                     _lib.geom_struct(geom), _DTYPE_CODE[h.dtype], sc,
                                     int(_rounds_weighted(rw.dtype, h.dtype)),
                                     _lib.stream_ptr(h.device)),
               "vaayu_decode_down")


def _launch(x, pairs, routing_weights, out) -> None:
    """Both decode kernels over `pairs`, into `out`, unchecked (`_checked` gates this;
    vaayu/packed_expert_kernels.py:390-396)."""
    blob = pairs[0][0]
    tbl = _TABLES.put(_table_values(pairs), x.device)
    h = _gate_up(x, tbl, len(pairs), blob["geom"], _scale_code(blob))
    _down(h, tbl, routing_weights, out, len(pairs), blob["geom"], _scale_code(blob))


def _fused_sync_words(n_pairs, geom, act_dtype, scale_dtype):
    """int32 words of the one-launch decode's sync buffer for this configuration, or None
    when the one-launch kernel does not take it."""
    lib = _require_backend()
    words = lib.vaayu_decode_fused_sync_words(n_pairs, _lib.geom_struct(geom),
                                              _DTYPE_CODE[act_dtype], _SCALE_CODE[scale_dtype])
    return words if words > 0 else None


def _fused(x, tbl, n, geom, sc, routing_weights, out, h, sync, max_polls=0) -> None:
    """Both decode stages in one launch (`vaayu_decode_fused`): the arithmetic of `_gate_up`
    then `_down`, with the down workgroups streaming their codes while gate/up runs. `sync`
    is the configuration's zero-initialised int32 counter buffer (`_fused_sync_words`)."""
    lib = _require_backend()
    rw = routing_weights.reshape(-1).contiguous()
    _lib.check(lib.vaayu_decode_fused(x.data_ptr(), tbl.data_ptr(), rw.data_ptr(),
                                      _DTYPE_CODE[rw.dtype], out.data_ptr(), h.data_ptr(),
                                      sync.data_ptr(), n, _lib.geom_struct(geom),
                                      _DTYPE_CODE[x.dtype], sc,
                                      int(_rounds_weighted(rw.dtype, x.dtype)), max_polls,
                                      _lib.stream_ptr(x.device)),
               "vaayu_decode_fused")


def stock_experts_decode(x, pairs, routing_weights, out, act_fn) -> None:
    """One token through the per-slot loop's arithmetic, into `out`: the reference the
    kernels are held to and their fallback (vaayu/packed_expert_kernels.py:399-410) --
    dense weights, three `F.linear`, `act_fn`, the routing-weight product with torch's
    promotion, an fp32 add in pair order."""
    from .moe_patch import expert_weights_from_entry
    rw = routing_weights.reshape(-1)
    out.zero_()
    for blob, slot in pairs:
        gate_w, down_w, up_w = expert_weights_from_entry(blob, x.dtype)
        hidden = act_fn(F.linear(x, gate_w)) * F.linear(x, up_w)
        out += (F.linear(hidden, down_w) * rw[slot:slot + 1]).to(out.dtype)


def _verdict(x, pairs, routing_weights, act_fn) -> bool:
    """Kernels AND stock arithmetic on this call's data; True if they agree
    (vaayu/packed_expert_kernels.py:440-447)."""
    blob = pairs[0][0]
    return _judge("decode", x,
                  _unsupported(blob["geom"], x.dtype, blob["flat"]["scale"].dtype,
                               routing_weights.dtype),
                  lambda want: stock_experts_decode(x, pairs, routing_weights, want, act_fn),
                  lambda got: _launch(x, pairs, routing_weights, got))


def _checked(x, pairs, routing_weights, act_fn) -> bool:
    """The verdict of this call's (geometry, dtypes) key (vaayu/packed_expert_kernels.py:
    450-456)."""
    return _remembered("_VERDICTS", _verdict_key(pairs[0][0], x, routing_weights),
                       lambda: _verdict(x, pairs, routing_weights, act_fn))


def packed_experts_decode(x, pairs, routing_weights, out, act_fn) -> None:
    """One token's routed-expert sum for one MoE layer, written into `out`
    (vaayu/packed_expert_kernels.py:459-480).

    x               [1, hidden], activation dtype, contiguous, on the current device
    pairs           [(blob, slot), ...] sorted by (expert id, slot): the fp32 sum's order
    routing_weights this token's [1, top_k] (or [top_k]) weights; `slot` indexes them
    out             [1, hidden] float32, overwritten
    act_fn          the experts' activation; only the stock fallback calls it

    Entries that are not all blobs of ONE geometry run the stock arithmetic."""
    on_kernels = (_kernel_ready(b for b, _slot in pairs)
                  and _checked(x, pairs, routing_weights, act_fn))
    if on_kernels:
        _launch(x, pairs, routing_weights, out)
    else:
        stock_experts_decode(x, pairs, routing_weights, out, act_fn)


# ── one MoE layer's decode launches as ONE graph (vaayu/packed_expert_kernels.py:483-654) ──
# Under the engine's decode graphs a layer's inputs (x, the routing weights, the shared
# expert's output) are the same tensors every token, so the table upload, both launches
# and the epilogue are recorded once per layer and replayed with only the pinned table
# rewritten. Each recording is held bitwise to the eager launch before it is kept.
_GRAPHS: dict = {}              # layer -> _LayerGraph
_GRAPH_REFUSED: dict = {}       # layer -> why
_GRAPH_WARNED: set = set()
_GRAPH_STREAMS: dict = {}       # device -> the recording stream
GRAPH_STATS: collections.Counter = collections.Counter()


def _tail(out, dtype, shared):
    """The fused forward's epilogue: the fp32 sum cast back, plus the shared expert."""
    result = out.to(dtype)
    return result + shared.to(result.dtype) if shared is not None else result


def _warn_once(why, message) -> None:
    if why not in _GRAPH_WARNED:
        _GRAPH_WARNED.add(why)
        print(message)


def _refuse_graph(layer, why) -> None:
    _GRAPH_REFUSED[layer] = why
    _GRAPHS.pop(layer, None)
    GRAPH_STATS["refused"] += 1
    _warn_once(why, f"[Vaayu] WARNING: packed-expert decode graph refused for MoE layer "
                    f"{layer} ({why}); it launches eagerly. Later layers refused for the same "
                    f"reason are not listed.")


def _warn_skip(why) -> None:
    """A call the graph cannot take launches eagerly; said once per reason."""
    _warn_once(why, f"[Vaayu] WARNING: packed-expert decode graph not used ({why}); those "
                    f"calls launch the kernels eagerly. Shown once per reason.")


def _release_pool(pool) -> None:
    """Return a graph pool whose recording failed to end: torch's allocator otherwise keeps
    believing a capture records into it."""
    dev = torch.cuda.current_device()
    for release in (torch._C._cuda_endAllocateToPool, torch._C._cuda_releasePool):
        try:
            release(dev, pool)
        except Exception:
            pass


class _LayerGraph:
    """One MoE layer's recorded decode: the pinned table it replays from (`host`), its
    device copy (`tbl`), the static intermediates (`h`, `out`, `tmp`) and the returned
    tensor (`result`, or `out` without the epilogue)."""
    __slots__ = ("key", "graph", "host", "host_np", "tbl", "h", "out", "tmp", "result",
                 "done", "replays")

    def __init__(self, key, n_values, n_pairs, inter, x, tail, shared):
        dev = x.device
        self.key, self.replays, self.graph = key, 0, None
        self.host = torch.empty(n_values, dtype=torch.int64, pin_memory=True)
        self.host_np = self.host.numpy()
        self.tbl = torch.empty(n_values, dtype=torch.int64, device=dev)
        self.h = torch.empty(n_pairs, inter, dtype=x.dtype, device=dev)
        self.out = torch.empty(x.shape, dtype=torch.float32, device=dev)
        self.tmp = torch.empty(x.shape, dtype=x.dtype, device=dev) if tail else None
        self.result = (torch.empty(x.shape, dtype=x.dtype, device=dev)
                       if tail and shared is not None else self.tmp)
        self.done = torch.cuda.Event()

    def returned(self, tail):
        return self.result if tail else self.out

    def record(self, x, routing_weights, shared, tail, geom, sc) -> None:
        """Capture the launches on the device's recording stream (no allocation inside)."""
        n = self.h.shape[0]
        graph, pool = torch.cuda.CUDAGraph(), torch.cuda.graph_pool_handle()
        dev = x.device
        side = _GRAPH_STREAMS.get(dev)
        if side is None:
            side = _GRAPH_STREAMS[dev] = torch.cuda.Stream(device=dev)
        here = torch.cuda.current_stream(dev)
        side.wait_stream(here)
        with torch.cuda.stream(side), torch.no_grad():
            graph.capture_begin(pool=pool, capture_error_mode="thread_local")
            try:
                self.tbl.copy_(self.host, non_blocking=True)
                _gate_up(x, self.tbl, n, geom, sc, h=self.h)
                _down(self.h, self.tbl, routing_weights, self.out, n, geom, sc)
                if tail:
                    self.tmp.copy_(self.out)
                    if shared is not None:
                        torch.add(self.tmp, shared, out=self.result)
            finally:
                try:
                    graph.capture_end()
                except Exception:
                    _release_pool(pool)
                    raise
        here.wait_stream(side)
        self.graph = graph

    def replay(self, values) -> None:
        self.done.synchronize()             # the previous replay has read the table
        self.host_np[:] = values
        self.graph.replay()
        self.done.record()
        self.replays += 1


def _graph_obstacle(x, pairs, routing_weights, shared, tail):
    """(reason, say_it) when the graph cannot take this call: say_it is False for calls that
    are simply not the graph's (mixed or unaligned entries), True for inputs it cannot bind."""
    if not _kernel_ready(b for b, _s in pairs):
        return "not one geometry of aligned blobs", False
    if not (x.is_contiguous() and routing_weights.is_contiguous()):
        return "a non-contiguous expert input or routing-weight tensor", True
    if tail and shared is not None and shared.dtype != x.dtype:
        return f"the shared expert's output is {shared.dtype}, the activations {x.dtype}", True
    return None, False


def packed_experts_decode_graphed(layer, x, pairs, routing_weights, shared, act_fn, tail):
    """`packed_experts_decode` (and, `tail` True, the forward's epilogue) through one graph
    per MoE layer -- or None: not the graph's call, run the eager path
    (vaayu/packed_expert_kernels.py:531-575). Returns a STATIC tensor the layer's next call
    overwrites: the fp32 sum [1, hidden], or `_tail(sum, x.dtype, shared)`."""
    if layer in _GRAPH_REFUSED:
        return None
    why, say_it = _graph_obstacle(x, pairs, routing_weights, shared, tail)
    if why is not None:
        if say_it:
            _warn_skip(why)
        return None
    if not _checked(x, pairs, routing_weights, act_fn):
        return None
    blob = pairs[0][0]
    values = _table_values(pairs)
    key = (len(pairs), x.data_ptr(), routing_weights.data_ptr(), routing_weights.dtype,
           0 if shared is None else shared.data_ptr(), tail, blob["geom"], x.dtype,
           blob["flat"]["scale"].dtype)
    kept = _GRAPHS.get(layer)
    if kept is not None and kept.key == key:
        kept.replay(values)
        GRAPH_STATS["replays"] += 1
        return kept.returned(tail)
    if kept is not None:                    # inputs moved: this layer records again
        del _GRAPHS[layer]
        if kept.replays == 0:
            GRAPH_STATS["replaced_unreplayed"] += 1
        del kept
    return _record_layer(layer, key, x, pairs, routing_weights, shared, tail, values)


def _record_layer(layer, key, x, pairs, routing_weights, shared, tail, values):
    """Launch eagerly, record the layer's graph, replay it once and keep it only if the
    replay equals the eager result bit for bit (vaayu/packed_expert_kernels.py:578-654).
    The eager result is what this call returns unless the graph's equals it; nothing here
    raises into the request."""
    blob = pairs[0][0]
    eager_out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _launch(x, pairs, routing_weights, eager_out)
    eager = _tail(eager_out, x.dtype, shared) if tail else eager_out
    collecting = gc.isenabled()
    gc.disable()            # a collection inside the capture could free a tensor mid-record
    try:
        g = _LayerGraph(key, len(values), len(pairs), _layout(blob["geom"])["gate"][2], x,
                        tail, shared)
        g.host_np[:] = values
        g.record(x, routing_weights, shared, tail, blob["geom"], _scale_code(blob))
        g.graph.replay()
        agrees = torch.equal(g.returned(tail), eager)
    except Exception as exc:
        first = (str(exc).splitlines() or [""])[0][:200]
        _refuse_graph(layer, f"capture failed: {type(exc).__name__}: {first}")
        return eager
    finally:
        if collecting:
            gc.enable()
    if not agrees:
        _refuse_graph(layer, "its replay disagrees bitwise with the eager launch")
        return eager
    g.done.record()
    _GRAPHS[layer] = g
    GRAPH_STATS["captures"] += 1
    return g.returned(tail)


# ── prefill ─────────────────────────────────────────────────────────────────────────────

def _prefill_plan(eidx_cpu):
    """(order, live, counts) of one call's routing (vaayu/packed_expert_kernels.py:676-688):
    row ids (token*top_k + slot) stable-sorted by expert id, the routed ids ascending, and
    the rows of each."""
    flat = eidx_cpu.reshape(-1)
    rows_per_expert = torch.bincount(flat)
    live = torch.nonzero(rows_per_expert).reshape(-1)
    return torch.argsort(flat, stable=True), live, rows_per_expert[live]


def _run_cost(blocks: int) -> float:
    """Relative time of one work item of a run of `blocks` blocks in the grouped kernels: a
    fixed part per K step (every run streams all its N tile's weight codes) and a part per
    16-row block. Fitted to per-item times on MI355X (DeepSeek-V3 gate/up, K 7168: 1 block
    67.5 us, 2 blocks 77.8, 4 blocks 95.0, 8 blocks 141.1; down in about the same ratio)."""
    return 5.5 + blocks


class PrefillWork(NamedTuple):
    """The work lists of one call's grouped launches (int64 on the device, `_prefill_work`),
    their slots per XCD, and the longest run of each."""
    gate_up: torch.Tensor
    gate_up_slots: int
    down: torch.Tensor
    down_slots: int
    down_run: int
    gate_up_run: int

    def clone(self) -> "PrefillWork":
        return self._replace(gate_up=self.gate_up.clone(), down=self.down.clone())


_RUN_BLOCKS = {}
_CUS = {}


def _cu_count(device) -> int:
    """Compute units of the device (256 on MI355X)."""
    d = torch.device(device)
    key = d.index if d.index is not None else torch.cuda.current_device()
    if key not in _CUS:
        _CUS[key] = int(torch.cuda.get_device_properties(key).multi_processor_count)
    return _CUS[key]


def _run_blocks(which: int) -> int:
    """Longest run (16-row blocks) a work item of the library's grouped kernel may take:
    which = 0 gate/up (packed and fused-3D), 1 down."""
    if which not in _RUN_BLOCKS:
        _RUN_BLOCKS[which] = int(_require_backend().vaayu_prefill_run_blocks(which))
    return _RUN_BLOCKS[which]


def _run_length(blocks, run: int, n_tiles: int, n_cus: int) -> int:
    """The run length (at most `run` blocks, halving) with the shortest estimated launch:
    the larger of the work spread over the CUs and the longest item, by `_run_cost`. Long
    runs share each K step's dequant among more rows; a call of few long runs (one
    expert's 2048 rows) leaves CUs idle unless they are split (runs of 16 blocks give 128
    work items for 256 CUs there, runs of 8 fill them)."""
    best, best_t, r = run, None, run
    while r >= 1:
        n = [min(r, int(b) - f) for b in blocks for f in range(0, int(b), r)]
        t = max(sum(_run_cost(x) for x in n) * n_tiles / n_cus,
                _run_cost(max(n, default=0)))
        if best_t is None or t < best_t:
            best, best_t = r, t
        r //= 2
    return best


def _down_run(blocks, n_tiles: int, n_cus: int, k: int = 0) -> int:
    """The down launch's run length (k: the down GEMM's K, the intermediate size). The
    library's down kernel for runs of up to 16 blocks holds twice the accumulators and
    twice the LDS of the one for runs of up to 8, so one workgroup runs per CU instead of
    two. It pays only where the longer runs halve the run count over a long K (Mixtral's
    512-token layer, experts of 8-9 blocks, K 14336: down 185 -> 172 us); not over a short
    one (gpt-oss-20b, experts of 16 blocks, K 2880: layer 569-576 us with runs of 8 against
    596-608 us with runs of 16, alternating in one process), nor where they save few runs
    (DeepSeek-V3's Zipf routing: down 1086 -> 1219 us)."""
    longest = _run_blocks(1)
    runs = {r: sum(-(-int(b) // r) for b in blocks) for r in (8, longest)}
    run = longest if runs[longest] <= 0.75 * runs[8] and k >= 8192 else 8
    return min(_run_length(blocks, run, n_tiles, n_cus), max(int(b) for b in blocks))


def _prefill_work(blocks, run: int, n_tiles: int = 0, n_cus: int = 0):
    """(work, n_slots, run): the work list of one grouped launch over tables whose experts
    hold `blocks` 16-row blocks each, in table order. Each expert's blocks form runs of up to
    `run` blocks (or the `_run_length` for `n_tiles` N tiles on `n_cus` CUs, when given)
    from its first block on; a run is one work item per N tile, all on one XCD (so they
    share the run's activation rows in its L2). The runs go to the eight XCDs longest
    first, each to the XCD with the least work so far (`_run_cost`) among those holding
    fewer than ceil(runs / 8), and each XCD takes its runs in that order.
    work[k * 8 + x] = first_block * 32 + length of XCD x's k-th run, or -1; n_slots is the
    most runs an XCD holds, run the longest run. A row's arithmetic does not depend on its
    run's place or length, so every choice gives the same bits."""
    if n_tiles and n_cus:
        run = _run_length(blocks, run, n_tiles, n_cus)
    run = min(run, max((int(b) for b in blocks), default=1))
    runs, pos = [], 0
    for b in blocks:
        b = int(b)
        for first in range(0, b, run):
            runs.append((pos + first, min(run, b - first)))
        pos += b
    cap = -(-len(runs) // _XCDS)
    load, per = [0.0] * _XCDS, [[] for _ in range(_XCDS)]
    for first, n in sorted(runs, key=lambda r: (-r[1], r[0])):
        x = min((t for t in range(_XCDS) if len(per[t]) < cap), key=lambda t: (load[t], t))
        per[x].append(first * 32 + n)
        load[x] += _run_cost(n)
    work = torch.full((max(cap, 0), _XCDS), -1, dtype=torch.int64)
    for x, entries in enumerate(per):
        if entries:
            work[:len(entries), x] = torch.tensor(entries, dtype=torch.int64)
    return work.reshape(-1), cap, run


def _prefill_layout(plan):
    """Host tables of one call's blocks: (lay, blocks, rows). `lay` the live experts (as
    indices into `live`) in table order (ascending id, as the reference lays them out),
    `blocks` each live expert's block count, `rows` [n_blocks * _PF_BLOCK_M] row ids: each
    expert's rows in ascending order over its blocks, padded with -1 to whole blocks."""
    order, live, counts = plan
    blocks = (counts + _PF_BLOCK_M - 1) // _PF_BLOCK_M          # per live expert
    n_blocks = int(blocks.sum())
    lay = torch.arange(live.numel(), dtype=torch.int64)
    first_block = torch.empty_like(blocks)
    first_block[lay] = torch.cumsum(blocks[lay], 0) - blocks[lay]
    expert_of_row = torch.repeat_interleave(torch.arange(live.numel()), counts)
    # a row's place: its expert's first padded slot plus its rank among that expert's rows
    padded_start = first_block * _PF_BLOCK_M
    rank = torch.arange(order.numel()) - (torch.cumsum(counts, 0) - counts)[expert_of_row]
    rows = torch.full((n_blocks * _PF_BLOCK_M,), -1, dtype=torch.int64)
    rows[padded_start[expert_of_row] + rank] = order
    return lay, blocks, rows


def _prefill_tables(eidx_cpu, plan, blobs, device):
    """The call's tables on the device from ONE pinned copy
    (vaayu/packed_expert_kernels.py:691-717): (tbl, rows, ord, n_blocks).

    tbl   [n_blocks, 2] (packed address, scale address) of each block's expert
    rows  [n_blocks, _PF_BLOCK_M] row ids, each expert's rows padded to whole blocks with -1
    ord   [tokens, top_k] row ids of each token's slots in ascending expert id

    The gate/up and down launches' work lists (`PrefillWork`, `_prefill_work`) come in the
    same copy and ride on the returned `tbl` object (`tbl.vaayu_work`), where `_gate_up_g`
    and `_down_g` find them; a copy of `tbl` does not carry them (see `_work_of`)."""
    _order, live, _counts = plan
    tokens, top_k = eidx_cpu.shape
    lay, blocks, rows = _prefill_layout(plan)
    n_blocks = int(blocks.sum())
    addresses = torch.tensor([[blobs[e]["flat"]["packed"].data_ptr(),
                               blobs[e]["flat"]["scale"].data_ptr()] for e in live.tolist()],
                             dtype=torch.int64)
    tbl = torch.repeat_interleave(addresses[lay], blocks[lay], dim=0).reshape(-1)
    by_expert = torch.argsort(eidx_cpu, dim=1, stable=True)
    ord_ = (by_expert + top_k * torch.arange(tokens)[:, None]).reshape(-1)
    lay_geom = _layout(blobs[int(live[0])]["geom"])
    hidden, inter = lay_geom["gate"][3], lay_geom["gate"][2]
    n_cus = _cu_count(device)
    blk = blocks[lay].tolist()
    w_gu, s_gu, r_gu = _prefill_work(blk, _run_blocks(0), -(-inter // 128), n_cus)
    w_dn, s_dn, r_dn = _prefill_work(blk, _down_run(blk, -(-hidden // 128), n_cus, inter))
    parts = [tbl, rows, ord_, w_gu, w_dn]
    dev = _PF_TABLES.put(torch.cat(parts), device)
    at = [0]
    for t in parts:
        at.append(at[-1] + t.numel())
    sl = [dev[at[i]:at[i + 1]] for i in range(len(parts))]
    sl[0].vaayu_work = PrefillWork(sl[3], s_gu, sl[4], s_dn, r_dn, r_gu)
    return sl[0], sl[1], sl[2], n_blocks


def _work_of(tbl, n_blocks: int, geom) -> PrefillWork:
    """The work lists of a launch over `tbl`: those `_prefill_tables` attached to it, or,
    for a table from elsewhere (a copy, a caller's own), lists rebuilt from the table
    itself (one device-to-host copy): a run only needs its blocks to share one expert's
    address, which consecutive equal entries give."""
    work = getattr(tbl, "vaayu_work", None)
    if work is not None:
        return work
    addr = tbl.reshape(-1, 2)[:n_blocks, 0].cpu()
    change = torch.nonzero(addr[1:] != addr[:-1]).reshape(-1) + 1
    edges = torch.cat([torch.tensor([0]), change, torch.tensor([n_blocks])])
    blk = (edges[1:] - edges[:-1]).tolist()
    lay = _layout(geom)
    hidden, inter = lay["gate"][3], lay["gate"][2]
    n_cus = _cu_count(tbl.device)
    w_gu, s_gu, r_gu = _prefill_work(blk, _run_blocks(0), -(-inter // 128), n_cus)
    w_dn, s_dn, r_dn = _prefill_work(blk, _down_run(blk, -(-hidden // 128), n_cus, inter))
    dev = torch.cat([w_gu, w_dn]).to(tbl.device)
    work = PrefillWork(dev[:w_gu.numel()], s_gu, dev[w_gu.numel():], s_dn, r_dn, r_gu)
    tbl.vaayu_work = work
    return work


def _gate_up_g(x, tbl, rows, n_blocks, top_k, geom, sc, h=None, work=None):
    """h [tokens * top_k, intermediate], activation dtype: SiLU(gate) * up per live row
    (vaayu/packed_expert_kernels.py:720-732); `work` the call's `PrefillWork` (by default
    `_work_of(tbl)`)."""
    lib = _require_backend()
    work = work if work is not None else _work_of(tbl, n_blocks, geom)
    g = _lib.geom_struct(geom)
    if h is None:
        h = torch.empty(x.shape[0] * top_k, g.inter, dtype=x.dtype, device=x.device)
    _lib.check(lib.vaayu_prefill_gate_up(x.data_ptr(), rows.data_ptr(), tbl.data_ptr(),
                                         work.gate_up.data_ptr(), work.gate_up_slots,
                                         work.gate_up_run, h.data_ptr(), n_blocks, top_k, g,
                                         _DTYPE_CODE[x.dtype], sc, _lib.stream_ptr(x.device)),
               "vaayu_prefill_gate_up")
    return h


def _down_g(h, tbl, rows, n_blocks, routing_weights, geom, sc, y=None, work=None):
    """y [tokens * top_k, hidden] fp32: each live row's down projection times its weight
    (vaayu/packed_expert_kernels.py:735-749); `work` the call's `PrefillWork` (by default
    `_work_of(tbl)`)."""
    lib = _require_backend()
    work = work if work is not None else _work_of(tbl, n_blocks, geom)
    g = _lib.geom_struct(geom)
    rw = routing_weights.reshape(-1).contiguous()
    if y is None:
        y = torch.empty(h.shape[0], g.hidden, dtype=torch.float32, device=h.device)
    _lib.check(lib.vaayu_prefill_down(h.data_ptr(), rows.data_ptr(), tbl.data_ptr(),
                                      work.down.data_ptr(), work.down_slots, work.down_run,
                                      rw.data_ptr(), _DTYPE_CODE[rw.dtype], y.data_ptr(),
                                      n_blocks, g, _DTYPE_CODE[h.dtype], sc,
                                      int(_rounds_weighted(rw.dtype, h.dtype)),
                                      _lib.stream_ptr(h.device)),
               "vaayu_prefill_down")
    return y


def _reduce(y, order, out, top_k) -> None:
    """`out` [tokens, hidden] fp32 = each token's contributions summed in `order`
    (vaayu/packed_expert_kernels.py:752-757)."""
    lib = _require_backend()
    _lib.check(lib.vaayu_prefill_reduce(y.data_ptr(), order.data_ptr(), out.data_ptr(),
                                        out.shape[0], top_k, y.shape[1],
                                        _lib.stream_ptr(y.device)),
               "vaayu_prefill_reduce")


def _tokens_per_launch(hidden: int, inter: int, top_k: int, n_live: int) -> int:
    """The most tokens one launch of the grouped kernels may take. They address activation
    rows (x: hidden bf16 values per token) and intermediate rows (h: inter values per table
    row) with 32-bit byte offsets, and the library refuses a launch whose tables could hold
    rows past `_OFFSET_LIMIT`: at most n_blocks * 16 rows, i.e. the call's tokens * top_k
    plus up to 15 padding rows per routed expert."""
    rows = min(_OFFSET_LIMIT // (2 * inter), (_OFFSET_LIMIT // (2 * hidden)) * top_k)
    return max((rows - (_PF_BLOCK_M - 1) * n_live) // top_k, 1)


def _prefill_call(x, eidx_cpu, routing_weights, blobs, out, plan) -> None:
    """The three kernels over one launch's tokens."""
    blob = blobs[int(plan[1][0])]
    geom, sc, top_k = blob["geom"], _scale_code(blob), eidx_cpu.shape[1]
    x = x.contiguous()
    tbl, rows, order, n_blocks = _prefill_tables(eidx_cpu, plan, blobs, x.device)
    h = _gate_up_g(x, tbl, rows, n_blocks, top_k, geom, sc)
    y = _down_g(h, tbl, rows, n_blocks, routing_weights, geom, sc)
    dense = out if out.is_contiguous() else torch.empty(out.shape, dtype=torch.float32,
                                                        device=out.device)
    _reduce(y, order, dense, top_k)
    if dense is not out:
        out.copy_(dense)


def _prefill_launch(x, eidx_cpu, routing_weights, blobs, out, plan=None) -> None:
    """The three prefill kernels over one call, unchecked (`_prefill_checked` gates this;
    vaayu/packed_expert_kernels.py:760-777). A strided `x` is made dense; a strided `out` is
    written through a dense temporary. A call too large for the kernels' 32-bit row offsets
    is launched in token chunks, with the same bits (each row's arithmetic is its own)."""
    plan = plan or _prefill_plan(eidx_cpu)
    lay = _layout(blobs[int(plan[1][0])]["geom"])
    top_k = eidx_cpu.shape[1]
    step = _tokens_per_launch(lay["gate"][3], lay["gate"][2], top_k, plan[1].numel())
    tokens = x.shape[0]
    if tokens <= step:
        _prefill_call(x, eidx_cpu, routing_weights, blobs, out, plan)
        return
    for t0 in range(0, tokens, step):
        part = slice(t0, min(t0 + step, tokens))
        e_part = eidx_cpu[part]
        _prefill_call(x[part], e_part, routing_weights[part], blobs, out[part],
                      _prefill_plan(e_part))


def _linear_fp32(a, w):
    """`F.linear` with the product summed in fp32 and rounded ONCE to the activation dtype."""
    return F.linear(a.float(), w.float()).to(a.dtype)


def stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn,
                          linear=F.linear) -> None:
    """A multi-token call through the per-slot loop's arithmetic, into `out`
    (vaayu/packed_expert_kernels.py:785-814): per expert in id order, its rows gathered,
    dense weights, three `linear`s, `act_fn`, the routing-weight product, `index_add_`. A
    routed expert with no entry is skipped. `linear=_linear_fp32` is the reference the
    kernels are checked against."""
    from .moe_patch import expert_weights_from_entry
    order, live, counts = _prefill_plan(eidx_cpu)
    top_k = eidx_cpu.shape[1]
    rw = routing_weights.reshape(-1)
    order = order.to(x.device)
    out.zero_()
    for e, rows in zip(live.tolist(), torch.split(order, counts.tolist())):
        entry = blobs.get(e)
        if entry is None:
            continue
        gate_w, down_w, up_w = expert_weights_from_entry(entry, x.dtype)
        tokens = rows // top_k
        xs = x[tokens]
        hidden = act_fn(linear(xs, gate_w)) * linear(xs, up_w)
        out.index_add_(0, tokens, (linear(hidden, down_w) * rw[rows, None]).to(out.dtype))


def _prefill_verdict(x, eidx_cpu, routing_weights, blobs, act_fn, plan) -> bool:
    """The grouped kernels AND the fp32-GEMM stock arithmetic on this call's data
    (vaayu/packed_expert_kernels.py:817-826)."""
    blob = blobs[int(plan[1][0])]
    return _judge("prefill", x,
                  _prefill_unsupported(blob["geom"], x.dtype, blob["flat"]["scale"].dtype,
                                       routing_weights.dtype),
                  lambda want: stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, want,
                                                     act_fn, linear=_linear_fp32),
                  lambda got: _prefill_launch(x, eidx_cpu, routing_weights, blobs, got, plan))


def _prefill_checked(x, eidx_cpu, routing_weights, blobs, act_fn, plan) -> bool:
    """The verdict of this call's (geometry, dtypes) key (vaayu/packed_expert_kernels.py:
    829-835)."""
    return _remembered("_PF_VERDICTS",
                       _verdict_key(blobs[int(plan[1][0])], x, routing_weights),
                       lambda: _prefill_verdict(x, eidx_cpu, routing_weights, blobs, act_fn,
                                                plan))


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
    routed = plan[1].tolist()
    on_kernels = (all(e in blobs for e in routed)
                  and _kernel_ready(blobs[e] for e in routed)
                  and _prefill_checked(x, eidx_cpu, routing_weights, blobs, act_fn, plan))
    if on_kernels:
        _prefill_launch(x, eidx_cpu, routing_weights, blobs, out, plan)
    else:
        stock_experts_prefill(x, eidx_cpu, routing_weights, blobs, out, act_fn)


# ── load-time install ─────────────────────────────────────────────────────────────────────

def _is_silu(act_fn, device, dtype) -> bool:
    """Does the experts' activation compute SiLU (which the kernels hardcode)? Judged by
    its values on a grid, since the module may be any callable."""
    if act_fn is None:
        return False
    probe = torch.linspace(-8.0, 8.0, 257, device=device).to(dtype)
    try:
        return torch.equal(act_fn(probe), F.silu(probe))
    except Exception:
        return False


_ST_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32,
              "I32": torch.int32, "I64": torch.int64, "U8": torch.uint8, "I8": torch.int8}


def _read_expert_tensors(path: str, metas: dict) -> dict:
    """{key: cpu tensor} of one expert's tensors in a safetensors shard, read at the byte
    ranges the engine's offset index records (file_offset, byte_length, shape, dtype)."""
    out = {}
    with open(path, "rb") as f:
        for key, m in metas.items():
            f.seek(m.file_offset)
            raw = bytearray(f.read(m.byte_length))
            flat = torch.frombuffer(raw, dtype=_ST_DTYPES[m.dtype]) if raw else torch.empty(0)
            out[key] = flat.reshape(m.shape).clone()
    return out


def _one_real_blob(vaayu_ref, block, device, quiet=False):
    """The blob of `block`'s lowest-numbered expert as the checkpoint stores it, or None when
    its experts are not pack-quantized (vaayu/packed_expert_kernels.py:875-899)."""
    from .moe_patch import (_group_packed_tensors_by_weight, _packed_roles_complete,
                            _upload_packed_expert, build_expert_blob)
    metas = vaayu_ref._expert_offset_index.index.get(block.layer_name, {})
    if not metas:
        return None
    shard = Path(vaayu_ref.checkpoint_path) / f"{block.layer_name}.safetensors"
    try:     # inside the engine, its own reader (io_uring, pinned buffers)
        from vaayu.persist.safetensor_model_persister import load_expert_sparse as read
    except ImportError:
        read = _read_expert_tensors
    roles = _group_packed_tensors_by_weight(read(str(shard), metas[min(metas)]))
    if not roles["gate"] or not _packed_roles_complete(roles):
        return None
    try:
        blob = build_expert_blob(_upload_packed_expert(roles, device))
        why = "its projections are packed at different bit widths or group sizes"
    except NotImplementedError as exc:
        blob, why = None, str(exc)
    if blob is None and not quiet:
        print(f"[Vaayu] WARNING: fused packed-expert decode kernel not installed: {why}")
    return blob


_PREFILL_VRAM_HEADROOM = 4 << 30


def _describe(geom) -> str:
    """"4-bit, group 128" for integer blobs (the reference's wording); the format and its
    scale blocking for FP8 / MXFP4 blobs."""
    if isinstance(geom[0], str):
        return f"{geom[0]}, scale block {geom[1]}"
    return f"{geom[0]}-bit, group {geom[1]}"


def _install_preconditions(vaayu_ref):
    """(device, dtype, fused blocks) when the kernels could be installed, else None (with
    the WARNING the reference prints for a missing library or a non-current device)."""
    device = str(vaayu_ref.running_device)
    if torch.device(device).type != "cuda":
        return None
    if triton is None:
        if torch.cuda.is_available():
            print(f"[Vaayu] WARNING: fused packed-expert kernels not installed: "
                  f"{_LOAD_ERROR or 'the kernel library is absent'}")
        return None
    blocks = [b for b in (getattr(vaayu_ref, "_moe_blocks", None) or [])
              if getattr(b, "forward_name", None) == "_make_fused_sparse_forward"]
    if not blocks or getattr(vaayu_ref, "_expert_offset_index", None) is None:
        return None
    index = torch.device(device).index
    if index is not None and index != torch.cuda.current_device():
        print(f"[Vaayu] WARNING: fused packed-expert decode kernel not installed: model "
              f"device {device} is not the current GPU ({torch.cuda.current_device()}); "
              f"decode keeps the stock per-expert path")
        return None
    return device, vaayu_ref.running_dtype, blocks


def _probe_inputs(blob, tokens, top_k, device, dtype, gen):
    """Seeded activations [tokens, hidden] and routing weights [tokens, top_k] (rows sum to
    one; fp32) for the load-time verdicts."""
    hidden = _layout(blob["geom"])["gate"][3]
    x = (torch.randn(tokens, hidden, generator=gen, device=device) * 0.5).to(dtype)
    w = torch.rand(tokens, top_k, generator=gen, device=device) + 0.1
    return x, w / w.sum(-1, keepdim=True)


def _prefill_eligibility(vaayu_ref, blocks, first, blob, device, headroom):
    """(eligible layer indices, {reason: [layer indices]}) over the fused blocks: a layer
    qualifies when one real expert of it has the checked layer's geometry and scale dtype
    and its whole expert set fits in half the prefill headroom (a call holds every blob it
    uploaded until its launches run)."""
    checked = (blob["geom"], blob["flat"]["scale"].dtype)
    eligible, left_out = [], {}
    for b in blocks:
        one = blob if b is first else _one_real_blob(vaayu_ref, b, device, quiet=True)
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
        left_out.setdefault(why, []).append(b.layer_idx)
    return eligible, left_out


def _prefill_holds(blob, top_k, device, dtype, act_fn, gen) -> bool:
    """The prefill verdict on a call of 1.5 blocks of tokens, every token routed to every
    slot of the one real expert (in rotating slot order), with fp32 and activation-dtype
    routing weights."""
    tokens = _PF_BLOCK_M + _PF_BLOCK_M // 2
    eidx = torch.stack([torch.roll(torch.arange(top_k), t) for t in range(tokens)])
    xs, ws = _probe_inputs(blob, tokens, top_k, device, dtype, gen)
    blobs = dict.fromkeys(range(top_k), blob)
    plan = _prefill_plan(eidx)
    return all(_prefill_checked(xs, eidx, w, blobs, act_fn, plan) for w in (ws, ws.to(dtype)))


def _announce_prefill(eligible, left_out, n_blocks, what) -> None:
    print(f"[Vaayu] fused packed-expert prefill kernel on {len(eligible)} MoE layers ({what})")
    if not left_out:
        return
    skipped = sorted(i for idxs in left_out.values() for i in idxs)
    reasons = "; ".join(
        why if len(left_out) == 1 else f"{why} (layers {', '.join(map(str, idxs))})"
        for why, idxs in left_out.items())
    print(f"[Vaayu] WARNING: fused packed-expert prefill kernel not used on {len(skipped)} of "
          f"{n_blocks} MoE layers (layer indices {', '.join(map(str, skipped))}): {reasons}; "
          f"prefill keeps the per-expert path there")


def install_packed_expert_kernels(vaayu_ref) -> bool:
    """Route the fused pack-quantized MoE blocks through the kernels if they agree with the
    stock arithmetic on one real expert of this model on this device
    (vaayu/packed_expert_kernels.py:902-1012). Sets `vaayu_ref._packed_moe_kernel` (decode)
    and `vaayu_ref._packed_moe_prefill_kernel` (the eligible prefill layers); returns
    whether the decode kernel was installed."""
    ready = _install_preconditions(vaayu_ref)
    if ready is None:
        return False
    device, dtype, blocks = ready
    first = blocks[0]
    act_fn = getattr(getattr(first.moe_module, first.experts_attr, None), "act_fn", None)
    if not _is_silu(act_fn, device, dtype):
        print("[Vaayu] fused packed-expert decode kernel not used: the experts' activation "
              "is not SiLU")
        return False
    blob = _one_real_blob(vaayu_ref, first, device)
    if blob is None:
        return False

    # decode: one token over every slot of the real expert, fp32 and activation-dtype weights
    top_k = int(getattr(vaayu_ref, "moe_top_k", 0) or 1)
    gen = torch.Generator(device=device).manual_seed(0)
    x, w = _probe_inputs(blob, 1, top_k, device, dtype, gen)
    pairs = [(blob, s) for s in range(top_k)]
    if not all(_checked(x, pairs, rw, act_fn) for rw in (w, w.to(dtype))):
        return False
    vaayu_ref._packed_moe_kernel = blob["geom"]
    what = _describe(blob["geom"])
    print(f"[Vaayu] fused packed-expert decode kernel on {len(blocks)} MoE layers ({what})")

    # prefill: the layers that qualify, then the verdict on one real call
    try:
        from vaayu.moe_patch import _PREFILL_VRAM_HEADROOM as headroom
    except ImportError:
        headroom = _PREFILL_VRAM_HEADROOM
    eligible, left_out = _prefill_eligibility(vaayu_ref, blocks, first, blob, device, headroom)
    if not eligible:
        print(f"[Vaayu] WARNING: fused packed-expert prefill kernel not installed: "
              f"{'; '.join(left_out)}; prefill keeps the per-expert path")
        return True
    if _prefill_holds(blob, top_k, device, dtype, act_fn, gen):
        vaayu_ref._packed_moe_prefill_kernel = frozenset(eligible)
        _announce_prefill(eligible, left_out, len(blocks), what)
    return True
