"""One-token decode at the large expert shapes: Mixtral-8x7B (hidden 4096, intermediate
14336, top-2) and DeepSeek-V3 (hidden 7168, intermediate 2048, top-8 of 256, plus the
always-on shared expert as a one-slot call of weight 1).

int4 group-128 experts with fp16 scales quantized from N(0, 0.02) weights, bf16 N(0, 1)
activations, renormalised softmax routing weights in fp32. The kernels run through the
launch internal (`_launch`, no verdict in between, so a refusal cannot hide behind the
stock loop) and are held to the layer tolerance (max-abs 2e-2, relL2 5e-3) against the
oracle's torch port of the stock loop on the CPU.
"""
import numpy as np
import pytest
import torch

import vaayu_amd.packed_expert_kernels as pk
from oracle import oracle as O
from vaayu_amd.synth import random_expert

pytestmark = pytest.mark.gpu

TOL_REL, TOL_ABS = 5e-3, 2e-2


def _experts(hid, inter, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [random_expert(hid, inter, 4, 128, generator=g, device="cuda", std=0.02,
                          scale_dtype=torch.float16) for _ in range(n)]


def _cpu(blob):
    return {"flat": {n: t.cpu() for n, t in blob["flat"].items()}, "geom": blob["geom"]}


def _routing(n_exp, k, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.randn(1, n_exp, generator=g).softmax(-1)
    w, ids = p.topk(k, dim=-1)
    return w / w.sum(-1, keepdim=True), ids[0].tolist()


def _check(x, pairs, w):
    out = torch.full((1, x.shape[1]), float("nan"), device="cuda")
    pk._launch(x, pairs, w, out)
    torch.cuda.synchronize()
    ref = torch.empty(1, x.shape[1])
    O.stock_decode_torch(x.cpu(), [(_cpu(b), s) for b, s in pairs], w.cpu(), ref)
    got = out.cpu()
    assert torch.isfinite(got).all()
    r, a = O.rel_l2(got.numpy(), ref.numpy()), float((got - ref).abs().max())
    assert r <= TOL_REL and a <= TOL_ABS, (r, a)
    return got


@pytest.mark.parametrize("seed", [0, 1])
def test_mixtral_shape_decode_one_token(seed):
    blobs = _experts(4096, 14336, 8, seed=11 + seed)        # the layer's 8 experts
    w, ids = _routing(8, 2, seed)
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    pairs = [(blobs[ids[s]], s) for s in sorted(range(2), key=ids.__getitem__)]
    _check(x.cuda(), pairs, w.cuda())


def test_deepseek_v3_shape_decode_one_token_with_shared_expert():
    routed = _experts(7168, 2048, 8, seed=21)     # the 8 routed experts of 256
    ids = [3, 41, 77, 120, 160, 199, 230, 255]
    w, _ = _routing(8, 8, 5)
    slots = torch.randperm(8, generator=torch.Generator().manual_seed(3)).tolist()
    by_id = {ids[i]: routed[i] for i in range(8)}
    eid = [ids[slots[s]] for s in range(8)]           # slot s routed to expert eid[s]
    pairs = [(by_id[eid[s]], s) for s in sorted(range(8), key=eid.__getitem__)]
    x = torch.randn(1, 7168, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    _check(x.cuda(), pairs, w.cuda())
    shared = _experts(7168, 2048, 1, seed=22)[0]
    _check(x.cuda(), [(shared, 0)], torch.ones(1, 1, device="cuda"))


def test_large_shape_decode_is_independent_of_pair_order_in_the_blob_heap():
    """Same routing, experts copied to new addresses: identical bits."""
    blobs = _experts(4096, 14336, 2, seed=31)
    w, _ = _routing(2, 2, 4)
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    a = _check(x.cuda(), [(blobs[0], 0), (blobs[1], 1)], w.cuda())
    moved = [{"flat": {n: t.clone() for n, t in b["flat"].items()}, "geom": b["geom"]}
             for b in blobs]
    b = _check(x.cuda(), [(moved[0], 0), (moved[1], 1)], w.cuda())
    assert np.array_equal(a.numpy(), b.numpy())
