"""Routing on the GPU for a layer whose experts are all resident, and a one-token decode
that runs from the router's logits to the expert sum with no host step, so a whole MoE
decode layer (router, routing, table, both expert kernels) can be captured in one graph.

The reference routes on the GPU (`_route`, vaayu/moe_patch.py:2324-2335), then brings the
ids to the host through one sync (`_routing_to_host`, :232-243) to look up each routed
expert's blob, sorts the slots by expert id (:2386-2389) and uploads the pointer table
(`_table_values`, vaayu/packed_expert_kernels.py:349-352) before its kernels can launch.
With every expert of the layer resident, the blob addresses are known in advance:
`ResidentExperts` keeps them in a device table, `vaayu_route_topk` routes (the reference's
default softmax -> top-k -> renormalise) and writes the decode table straight from it, and
the decode kernels read that table.
"""
import torch

from . import _lib
from . import packed_expert_kernels as pk


def router_logits(x, weight, out=None, out_dtype=None):
    """The model's gate product `F.linear(x, weight)` for decode-sized calls in one HIP
    launch (one wave per token x expert, fp32 sum rounded once): x [tokens, hidden] and
    weight [experts, hidden] bf16 or fp16, contiguous. Returns logits [tokens, experts] in
    `out_dtype` (x's dtype by default, or fp32); `out` given: written in place."""
    lib = pk._require_backend()
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x [tokens, hidden] and weight [experts, hidden] disagree")
    if weight.dtype != x.dtype or not (x.is_contiguous() and weight.is_contiguous()):
        raise ValueError("x and weight must be contiguous and of one dtype")
    tokens, experts = x.shape[0], weight.shape[0]
    if out is None:
        out = torch.empty(tokens, experts, dtype=out_dtype or x.dtype, device=x.device)
    rc = lib.vaayu_router_logits(x.data_ptr(), weight.data_ptr(), pk._DTYPE_CODE[x.dtype],
                                 out.data_ptr(), pk._DTYPE_CODE[out.dtype], tokens, x.shape[1],
                                 experts, _lib.stream_ptr(x.device))
    _lib.check(rc, "vaayu_router_logits")
    return out


def _budget(top_k: int, keep_k, top_p):
    """(n_out, keep_k, top_p) for the C-ABI: `truncate_top_k`'s (k, p), None meaning off."""
    if keep_k is not None and keep_k < 1:
        raise ValueError("keep_k must be at least 1")
    if top_p is not None and not top_p > 0:
        raise ValueError("top_p must be positive")
    keep = top_k if keep_k is None else int(keep_k)
    return min(keep, top_k), keep, 0.0 if top_p is None else float(top_p)


def route_topk(logits, top_k: int, renorm: bool = True, keep_k=None, top_p=None,
               weights=None, ids=None):
    """The reference's default routing on the GPU, `w, idx = torch.topk(logits.float()
    .softmax(-1), top_k)` then `w / w.sum(-1)` (vaayu/moe_patch.py:2329-2334, 159-161), and
    `truncate_top_k(w, idx, keep_k, top_p)` on it (vaayu/moe_patch.py:170-215): (weights
    fp32 [..., n], ids int64 [..., n]), n = min(keep_k, top_k). Equal probabilities go to
    the lower expert id. `weights` / `ids` given (contiguous [tokens, n]): written in place."""
    lib = pk._require_backend()
    if logits.dtype not in pk._DTYPE_CODE:
        raise ValueError(f"logits must be bf16, fp16 or fp32, got {logits.dtype}")
    n_out, keep, p = _budget(top_k, keep_k, top_p)
    experts = logits.shape[-1]
    lead = logits.shape[:-1]
    flat = logits.reshape(-1, experts)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    tokens = flat.shape[0]
    if weights is None:
        weights = torch.empty(tokens, n_out, dtype=torch.float32, device=logits.device)
    if ids is None:
        ids = torch.empty(tokens, n_out, dtype=torch.int64, device=logits.device)
    for what, t, dt in (("weights", weights, torch.float32), ("ids", ids, torch.int64)):
        # the kernel writes tokens x n_out entries through the raw pointer
        if (t.dtype != dt or not t.is_contiguous() or t.device != logits.device
                or t.numel() != tokens * n_out):
            raise ValueError(f"{what} must be a contiguous {dt} tensor of {tokens} x {n_out} "
                             f"on {logits.device}, got {t.dtype} {tuple(t.shape)} on {t.device}")
    rc = lib.vaayu_route_topk(flat.data_ptr(), pk._DTYPE_CODE[flat.dtype], tokens, experts,
                              top_k, keep, p, int(renorm), weights.data_ptr(), ids.data_ptr(),
                              None, None, _lib.stream_ptr(logits.device))
    _lib.check(rc, "vaayu_route_topk")
    return weights.reshape(*lead, n_out), ids.reshape(*lead, n_out)


class DecodeBuffers:
    """The work tensors of `ResidentExperts.decode` for one slot count (`top_k` here is
    the routed slots after the decode budget) and activation dtype: routing weights, ids,
    the pair table and `h`. Held across calls, so a decode with them allocates nothing (a
    graph capture records it as it is)."""

    def __init__(self, top_k: int, inter: int, act_dtype, device):
        self.top_k = top_k
        self.weights = torch.empty(1, top_k, dtype=torch.float32, device=device)
        self.ids = torch.empty(1, top_k, dtype=torch.int64, device=device)
        self.table = torch.empty(top_k * 3, dtype=torch.int64, device=device)
        self.h = torch.empty(top_k, inter, dtype=act_dtype, device=device)


class ResidentExperts:
    """One MoE layer's experts, all resident on one device: `blobs[e]` is expert e's blob
    (`{"flat": {"packed", "scale"}, "geom"}`, vaayu/moe_patch.py:794-846), ids 0..E-1, one
    geometry and scale dtype. Raises ValueError when the decode kernels cannot take them."""

    def __init__(self, blobs):
        blobs = [blobs[e] for e in range(len(blobs))] if isinstance(blobs, dict) else list(blobs)
        if not blobs:
            raise ValueError("no experts")
        b0 = blobs[0]
        self.geom = b0["geom"]
        self.scale_dtype = b0["flat"]["scale"].dtype
        self.device = b0["flat"]["packed"].device
        for e, b in enumerate(blobs):
            if b.get("geom") != self.geom or b["flat"]["scale"].dtype != self.scale_dtype:
                raise ValueError(f"expert {e}: geometry or scale dtype differs from expert 0")
            if b["flat"]["packed"].device != self.device:
                raise ValueError(f"expert {e} is on {b['flat']['packed'].device}, not {self.device}")
        if not pk._aligned(blobs):
            raise ValueError("a packed stream does not start on 16 bytes")
        self.blobs = blobs
        self.sc = pk._SCALE_CODE[self.scale_dtype]
        self.inter = {r: rows for r, rows, _cols in self.geom[2]}["gate"]
        self.hidden = {r: cols for r, _rows, cols in self.geom[2]}["gate"]
        # [E, 2] (packed address, scale address); the blobs must outlive this object
        self.table = torch.tensor([[b["flat"]["packed"].data_ptr(), b["flat"]["scale"].data_ptr()]
                                   for b in blobs], dtype=torch.int64, device=self.device)

    def __len__(self):
        return len(self.blobs)

    def buffers(self, top_k: int, act_dtype, keep_k=None) -> DecodeBuffers:
        """Work tensors for `decode` with this (top_k, keep_k) and activation dtype."""
        n_out, _keep, _p = _budget(top_k, keep_k, None)
        return DecodeBuffers(n_out, self.inter, act_dtype, self.device)

    def decode(self, x, logits, top_k: int, out, renorm: bool = True, keep_k=None,
               top_p=None, bufs=None):
        """One token: route on `logits` [1, E] (with the decode budget `keep_k` / `top_p`
        of `truncate_top_k`), build the pair table, run the decode kernels; `out` fp32
        [1, hidden] <- the expert sum in (expert id, slot) order, as
        `packed_experts_decode` over the same routing (vaayu/packed_expert_kernels.py:459-480).
        Returns (weights fp32 [1, n], ids int64 [1, n]), n = min(keep_k, top_k). With
        `bufs` (from `buffers(top_k, x.dtype, keep_k)`) it allocates nothing."""
        lib = pk._require_backend()
        n_out, keep, p = _budget(top_k, keep_k, top_p)
        why = pk._unsupported(self.geom, x.dtype, self.scale_dtype, torch.float32)
        if why:
            raise ValueError(f"decode kernels do not take this layer: {why}")
        if x.shape != (1, self.hidden) or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous [1, {self.hidden}] tensor")
        if logits.shape != (1, len(self)) or not logits.is_contiguous():
            raise ValueError(f"logits must be a contiguous [1, {len(self)}] tensor")
        if bufs is None:
            bufs = self.buffers(top_k, x.dtype, keep_k)
        elif bufs.top_k != n_out or bufs.h.dtype != x.dtype:
            raise ValueError("buffers made for another slot count or activation dtype")
        rc = lib.vaayu_route_topk(logits.data_ptr(), pk._DTYPE_CODE[logits.dtype], 1, len(self),
                                  top_k, keep, p, int(renorm), bufs.weights.data_ptr(),
                                  bufs.ids.data_ptr(), self.table.data_ptr(),
                                  bufs.table.data_ptr(), _lib.stream_ptr(x.device))
        _lib.check(rc, "vaayu_route_topk")
        pk._gate_up(x, bufs.table, n_out, self.geom, self.sc, h=bufs.h)
        pk._down(bufs.h, bufs.table, bufs.weights, out, n_out, self.geom, self.sc)
        return bufs.weights, bufs.ids
