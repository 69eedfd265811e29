"""Shared test fixtures: synthetic packed experts, routed cases, comparisons."""
import functools

import numpy as np
import torch

from oracle import oracle as O


@functools.lru_cache(maxsize=None)
def cpu_blobs(hid, inter, bits, gs, k, scale_dtype=torch.bfloat16, std=0.05, seed=None):
    """k distinct experts quantized by the repo's quantizer (oracle restatement), as
    blobs with CPU tensors (roles gate, down, up)."""
    rng = np.random.default_rng(seed if seed is not None else hid * 7 + inter + bits + gs)
    return tuple(O.build_blob(O.make_expert(hid, inter, bits, gs, rng=rng, std=std,
                                            scale_dtype=scale_dtype)) for _ in range(k))


def to_device(blob, device="cuda"):
    return {"flat": {n: t.to(device) for n, t in blob["flat"].items()}, "geom": blob["geom"]}


@functools.lru_cache(maxsize=None)
def gpu_blobs(hid, inter, bits, gs, k, scale_dtype=torch.bfloat16, std=0.05, seed=None):
    return tuple(to_device(b) for b in cpu_blobs(hid, inter, bits, gs, k, scale_dtype, std, seed))


def decode_case(hid, inter, bits, gs, k, seed=0, w_dtype=torch.float32, act=torch.bfloat16,
                scale_dtype=torch.bfloat16, device="cuda"):
    """(x, pairs, routing_weights, cpu_pairs): expert i routed in a shuffled slot, pairs
    sorted by expert id (the table order)."""
    blobs = (gpu_blobs if device == "cuda" else cpu_blobs)(hid, inter, bits, gs, k, scale_dtype)
    cb = cpu_blobs(hid, inter, bits, gs, k, scale_dtype)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, hid, generator=g) * 0.5).to(act)
    w = torch.rand(1, k, generator=g) + 0.05
    w = (w / w.sum(-1, keepdim=True)).to(w_dtype)
    slots = torch.randperm(k, generator=torch.Generator().manual_seed(seed)).tolist()
    pairs = [(blobs[i], slots[i]) for i in range(k)]
    cpairs = [(cb[i], slots[i]) for i in range(k)]
    return x.to(device), pairs, w.to(device), cpairs


def prefill_case(hid, inter, bits, gs, *, n_exp=24, tokens=40, top_k=6, seed=0,
                 w_dtype=torch.float32, eidx=None, act=torch.bfloat16,
                 scale_dtype=torch.bfloat16):
    """(x, eidx, w, blobs_gpu, blobs_cpu): tokens each routed to top_k distinct experts of
    n_exp (ids 3i+1, so ids are not table positions)."""
    base = gpu_blobs(hid, inter, bits, gs, 8, scale_dtype)
    cbase = cpu_blobs(hid, inter, bits, gs, 8, scale_dtype)
    ids = [3 * i + 1 for i in range(n_exp)]
    blobs = {e: base[i % len(base)] for i, e in enumerate(ids)}
    cblobs = {e: cbase[i % len(cbase)] for i, e in enumerate(ids)}
    g = torch.Generator().manual_seed(seed)
    if eidx is None:
        eidx = torch.stack([torch.tensor(ids)[torch.randperm(n_exp, generator=g)[:top_k]]
                            for _ in range(tokens)])
    x = (torch.randn(eidx.shape[0], hid, generator=g) * 0.5).to(act)
    w = torch.rand(eidx.shape, generator=g) + 0.05
    w = (w / w.sum(-1, keepdim=True)).to(w_dtype)
    return x.cuda(), eidx, w.cuda(), blobs, cblobs


def rel(a, b):
    return O.rel_l2(O.to_np(a), O.to_np(b))


def frac_equal(a, b):
    return O.isclose_frac(O.to_np(a), O.to_np(b))


@functools.lru_cache(maxsize=None)
def format_blobs(fmt, hid, inter, k, device="cuda", std=0.05):
    """k distinct FP8 ("e4m3", 128 x 128 fp32 block scales) or MXFP4 ("mxfp4", E8M0 per 32)
    expert blobs of N(0, std) weights, built on the CPU and copied to `device`."""
    from vaayu_amd.block_formats import random_format_expert
    g = torch.Generator().manual_seed(hid * 3 + inter + len(fmt))
    blobs = [random_format_expert(fmt, hid, inter, generator=g, device="cpu", std=std)
             for _ in range(k)]
    return tuple(to_device(b, device) for b in blobs)


def format_case(fmt, hid, inter, k, seed=0, w_dtype=torch.float32, act=torch.bfloat16):
    """(x, pairs, routing_weights, cpu_pairs) over `format_blobs`, as `decode_case`."""
    blobs = format_blobs(fmt, hid, inter, k)
    cb = format_blobs(fmt, hid, inter, k, "cpu")
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, hid, generator=g) * 0.5).to(act)
    w = torch.rand(1, k, generator=g) + 0.05
    w = (w / w.sum(-1, keepdim=True)).to(w_dtype)
    slots = torch.randperm(k, generator=torch.Generator().manual_seed(seed)).tolist()
    return (x.cuda(), [(blobs[i], slots[i]) for i in range(k)], w.cuda(),
            [(cb[i], slots[i]) for i in range(k)])
