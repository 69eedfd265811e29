"""CPU restatement of the routed fused-3D MXFP4 expert layer (gpt-oss) -- part of the oracle.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the checker vaayu_amd/csrc/fused3d.hip
and vaayu_amd/fused3d.py are held to, never a product path.

The computation is the experts module's two vendored `matmul_ogs` calls and their finalize
sum, as transformers' `Mxfp4GptOssExperts.forward` issues them over the buffers that
vaayu/routed_fused3d.py:131-238 fills:
  weights  `upcast_from_mxfp` of the blocks and E8M0 scales (oracle.upcast_mxfp4)
  gate/up  acc + bias (vendor matmul_ogs_details/_matmul_ogs.py:310-338), then the fused
           `swiglu_fn` (vendor swiglu_details/_swiglu.py compute_swiglu / swiglu.py:89-101:
           gate clipped above at limit, linear to [-limit, limit], s = gate / (1 +
           exp(-alpha gate)), out = s * linear + s), stored bf16
  down     (acc + bias) * gamma (_matmul_ogs.py:338-349), stored bf16
  finalize each token's rows summed in fp32 in slot order (matmul_ogs_details/
           _finalize_matmul.py:295-330), the slots being the router's ids sorted ascending
           (transformers' routing sorts them), then stored bf16.
Products and sums run in float64 and are rounded where the kernels store.

Pinning (tests/test_fused3d_oracle.py): with `exact=True` (no storage rounding) it equals
transformers' dense `GptOssExperts.forward` in float64 on the dequantized weights -- an
independent implementation of the same expert math -- and the MXFP4 dequant is the one
pinned by tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np

from .oracle import round_to, to_np, upcast_mxfp4


def dequant_fused3d(blocks, scales) -> np.ndarray:
    """[E, R, C/32, 16] e2m1 blocks + [E, R, C/32] E8M0 scales -> float64 [E, R, C]."""
    b = np.asarray(to_np(blocks), dtype=np.uint8)
    E, R, G, _ = b.shape
    vals = upcast_mxfp4(b.reshape(E, R, G * 16), np.asarray(to_np(scales), dtype=np.uint8), "fp32")
    return vals.astype(np.float64)


def fused3d_experts(x, expert_ids, weights, gu_blocks, gu_scales, gu_bias, dn_blocks,
                    dn_scales, dn_bias, alpha=1.702, limit=7.0, exact=False, w_gu=None,
                    w_dn=None):
    """The layer's output [tokens, H]: float32 values of bf16 (or, `exact`, unrounded).
    `w_gu` / `w_dn`: already dequantized weights (indexable by expert id), to skip the
    dequant; otherwise only the routed experts are dequantized."""
    x64 = np.asarray(to_np(x), dtype=np.float64)
    eids = np.asarray(to_np(expert_ids), dtype=np.int64)
    w = np.asarray(to_np(weights), dtype=np.float64)
    Wgu = {} if w_gu is None else w_gu          # dequantized lazily, routed experts only
    Wdn = {} if w_dn is None else w_dn
    for e in np.unique(eids):
        if w_gu is None:
            Wgu[e] = dequant_fused3d(to_np(gu_blocks[e:e + 1]), to_np(gu_scales[e:e + 1]))[0]
        if w_dn is None:
            Wdn[e] = dequant_fused3d(to_np(dn_blocks[e:e + 1]), to_np(dn_scales[e:e + 1]))[0]
    bgu = np.asarray(to_np(gu_bias), dtype=np.float32).astype(np.float64)
    bdn = np.asarray(to_np(dn_bias), dtype=np.float32).astype(np.float64)
    rnd = (lambda v: v) if exact else (lambda v: round_to(v, "bf16").astype(np.float64))
    T, H = x64.shape
    out = np.zeros((T, H))
    for t in range(T):
        acc = np.zeros(H, dtype=np.float64 if exact else np.float32)
        for s in np.argsort(eids[t], kind="stable"):
            e = eids[t, s]
            a = Wgu[e] @ x64[t] + bgu[e]
            g = np.minimum(a[0::2], limit)
            u = np.clip(a[1::2], -limit, limit)
            sg = g / (1.0 + np.exp(-alpha * g))
            hv = rnd(sg * u + sg)
            yv = rnd((Wdn[e] @ hv + bdn[e]) * w[t, s])
            acc = acc + yv if exact else (acc + yv.astype(np.float32)).astype(np.float32)
        out[t] = acc
    return out if exact else round_to(out, "bf16")
