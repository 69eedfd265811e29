"""CPU restatement of Vaayu's gated-delta decode kernels -- part of the oracle.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): the checker the HIP kernels in
vaayu_amd/csrc/gated_delta.hip are held to, never a product path.

Each function restates one of the reference's fused seams (vaayu/gated_delta_kernels.py)
in float64, rounding to a storage dtype exactly where the reference kernel stores or
converts to one, so the result is the correctly-rounded value of the kernel's algorithm;
the HIP kernels compute in fp32 and may differ from it by the fp32 rounding of their sums.

Pinning (tests/test_gated_delta_oracle.py): against transformers' own torch fallbacks the
reference's seams replace (`torch_recurrent_gated_delta_rule`, `causal_conv1d_update`,
`Qwen3NextRMSNormGated.forward`), against closed forms (a zero-beta rule is pure decay,
a one-row state by hand), and T steps at once against T one-step calls carrying the state.
"""
from __future__ import annotations

import numpy as np

from .oracle import round_to, to_np


def _f64(t):
    return np.asarray(to_np(t), dtype=np.float64)


def gdn_rule(q, k, v, g, beta, h0=None, l2=True, act="bf16"):
    """`_rule_kernel` (vaayu/gated_delta_kernels.py:66-110) for q, k [B, T, HV, K],
    v [B, T, HV, V], g, beta [B, T, HV], h0 [B, HV, K, V] or None. Per step: q, k
    l2-normalised (eps 1e-6) when `l2`, q scaled by K^-1/2; h *= exp(g);
    delta = (v - sum_k h[k] k[k]) * beta; h += k delta; o = sum_k h[k] q[k].
    Returns (o [B, T, HV, V] rounded once to `act`, as float32; the final state, float32)."""
    q, k, v, g, beta = (_f64(x) for x in (q, k, v, g, beta))
    B, T, HV, K = k.shape
    V = v.shape[-1]
    h = np.zeros((B, HV, K, V)) if h0 is None else _f64(h0).copy()
    out = np.zeros((B, T, HV, V))
    for t in range(T):
        bq, bk = q[:, t], k[:, t]
        if l2:
            bq = bq / np.sqrt((bq * bq).sum(-1, keepdims=True) + 1e-6)
            bk = bk / np.sqrt((bk * bk).sum(-1, keepdims=True) + 1e-6)
        bq = bq / np.sqrt(K)
        h = h * np.exp(g[:, t])[..., None, None]
        delta = (v[:, t] - np.einsum("bhkv,bhk->bhv", h, bk)) * beta[:, t][..., None]
        h = h + bk[..., None] * delta[..., None, :]
        out[:, t] = np.einsum("bhkv,bhk->bhv", h, bq)
    return round_to(out, act), h.astype(np.float32)


def gdn_conv_update(x, state, w, bias=None, x_act="bf16", s_act="bf16", w_act="bf16"):
    """`_conv_kernel` (vaayu/gated_delta_kernels.py:148-175) for one token: x [B, D, 1],
    state [B, D, W], w [D, W], bias [D] or None. Every value passes through the weight
    dtype (the fallback's `cat([state, x]).to(weight.dtype)`), the state keeps its own;
    out = silu(round_w(sum_j s_j w_j + bias)) rounded to the weight dtype, then to x's.
    Returns (out [B, D, 1] float32, the new state [B, D, W] float32)."""
    xv = _f64(x)[..., 0]
    s = _f64(state)
    wv = _f64(w)
    taps = np.concatenate([s[..., 1:], xv[..., None]], -1)          # [B, D, W]
    taps = round_to(taps, w_act).astype(np.float64)
    new_state = round_to(taps, s_act)
    acc = (taps * wv[None]).sum(-1)
    if bias is not None:
        acc = acc + _f64(bias)[None]
    acc = round_to(acc, w_act).astype(np.float64)
    y = round_to(acc / (1.0 + np.exp(-acc)), w_act)
    return round_to(y, x_act)[..., None], new_state


def gdn_gated_norm(x, z, w, eps, x_act="bf16", round_mid=True):
    """`_norm_kernel` (vaayu/gated_delta_kernels.py:205-222) per row of N = w.size:
    y = round_x(x / sqrt(mean(x^2) + eps)); y = w * y (rounded to x's dtype when
    `round_mid`, i.e. when the weight does not promote the product); out =
    round_x(y * silu(z)). Returns float32 values of x's dtype."""
    xv, zv, wv = _f64(x), _f64(z), _f64(w)
    n = wv.size
    xr, zr = xv.reshape(-1, n), zv.reshape(-1, n)
    y = round_to(xr / np.sqrt((xr * xr).mean(-1, keepdims=True) + eps), x_act).astype(np.float64)
    y = wv[None] * y
    if round_mid:
        y = round_to(y, x_act).astype(np.float64)
    out = round_to(y * (zr / (1.0 + np.exp(-zr))), x_act)
    return out.reshape(xv.shape)
