"""Writes tests/golden/toy_decode.npz, the toy MoE layer decode evaluated by the oracle.

Workload (the reference's own CPU-runnable case): hidden 1024, 32 experts of intermediate
512 (gate/up/down SwiGLU), a bf16 router Linear(1024 -> 32) with N(0, 0.02) weights,
softmax top-4 renormalised routing, 1 token; activations bf16 N(0, 1); expert weights bf16
N(0, 0.02) quantized to packed int4 group 128 with fp16 scales. numpy default_rng(SEED)
draws, in order: x, the router weight, then the experts 0..31 (gate, down, up each).

Stored: the inputs' bit patterns and digests, the router logits (bf16), the routed ids
and weights, every routed pair's h (bf16 bits) and y, and the layer output (fp32) -- so
the HIP path can be checked against fixed vectors and the oracle against its own past
output. Regenerate with `python tests/golden/make_golden.py`.
"""
import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

SEED = 2024
HIDDEN, EXPERTS, INTER, TOP_K, BITS, GROUP = 1024, 32, 512, 4, 4, 128
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "toy_decode.npz")


def inputs():
    """(x bf16 [1, H] as float32, router weight bf16 [E, H] as float32, 32 blobs)."""
    rng = np.random.default_rng(SEED)
    x = torch.from_numpy(rng.standard_normal((1, HIDDEN), dtype=np.float32)).to(torch.bfloat16)
    wr = torch.from_numpy(rng.standard_normal((EXPERTS, HIDDEN), dtype=np.float32) * 0.02)
    wr = wr.to(torch.bfloat16)
    blobs = [O.build_blob(O.make_expert(HIDDEN, INTER, BITS, GROUP, rng=rng, std=0.02,
                                        scale_dtype=torch.float16)) for _ in range(EXPERTS)]
    return x.float().numpy(), wr.float().numpy(), blobs


def digest(blob) -> str:
    h = hashlib.sha256()
    h.update(blob["flat"]["packed"].numpy().tobytes())
    h.update(blob["flat"]["scale"].view(torch.int16).numpy().tobytes())
    return h.hexdigest()


def evaluate(x, wr, blobs):
    logits = O._linear(x, wr, "bf16")                        # bf16 router output
    w, ids = O.route_softmax_topk(logits, TOP_K)
    ids, w = ids[0], w[0]
    order = sorted(range(TOP_K), key=lambda s: int(ids[s]))  # (expert id, slot) order
    pairs = [(blobs[int(ids[s])], s) for s in order]
    hs, ys = [], []
    for blob, _slot in pairs:
        h, y = O.expert_stages(x, blob, "bf16")
        hs.append(h[0])
        ys.append(y[0])
    out = O.stock_decode(torch.from_numpy(x), pairs, torch.from_numpy(w), "fp32", "bf16")
    return logits, ids, w, np.array(order), np.stack(hs), np.stack(ys), out


def main():
    x, wr, blobs = inputs()
    logits, ids, w, order, hs, ys, out = evaluate(x, wr, blobs)
    np.savez_compressed(
        OUT, seed=np.int64(SEED),
        shape=np.array([HIDDEN, EXPERTS, INTER, TOP_K, BITS, GROUP], dtype=np.int64),
        x_bits=O.bf16_bits(x), router_sha256=np.array(hashlib.sha256(
            O.bf16_bits(wr).tobytes()).hexdigest()),
        expert_sha256=np.array([digest(b) for b in blobs]),
        logits_bits=O.bf16_bits(logits), ids=ids, weights=w, pair_order=order,
        h_bits=O.bf16_bits(hs), y=ys.astype(np.float32), out=out.astype(np.float32))
    print(f"wrote {OUT}: ids {ids.tolist()}, weights {w.tolist()}")


if __name__ == "__main__":
    main()
