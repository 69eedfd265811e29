"""Fused decode kernels for gated-delta-net mixers on MI355X: the drop-in for Vaayu's
`vaayu/gated_delta_kernels.py`.

transformers' gated-delta-net mixers (qwen3_next, qwen3_5, qwen3_5_moe; olmo_hybrid for the
rule only) decode through three swappable seams -- `recurrent_gated_delta_rule`,
`causal_conv1d_update` and the gated `norm` -- whose torch fallbacks cost dozens of small
launches per mixer per token. Each seam here is one hand-written HIP kernel
(vaayu_amd/csrc/gated_delta.hip, C ABI `vaayu_gdn_rule`, `vaayu_gdn_conv_update`,
`vaayu_gdn_gated_norm`):

  rule  one workgroup per (batch, value head, 16 value columns): the fp32 state slice
        [K, 16] lives in registers (16 k-groups of K/16 rows) for every step of the call.
  conv  one thread per (batch, channel): shift, append, depthwise dot, silu, in place.
  norm  one wave per row.

Detection, the self-checks and the installer behave as the reference's (file:line cited per
function): a seam is found by the surface it needs, never by class or architecture name;
each fused seam is checked against the stock one on the device before it goes in, and one
that disagrees stays stock with a WARNING. Without the built library `triton` is None and
nothing is installed (the reference's "no Triton" state); a direct kernel call then raises
ImportError.
"""
import ctypes
import math
import types

import torch

from . import _lib

try:
    _lib.load()
    _BACKEND = _lib
except ImportError as _exc:              # reported at the first kernel call
    _BACKEND = None
    _LOAD_ERROR = str(_exc)

# Truthiness of the kernel backend, under the name the reference's installer and tests use
# for it (they set it to None to simulate a machine without the kernels).
triton = _BACKEND

# Every fused seam carries the stock callable it replaced under this attribute
# (vaayu/gated_delta_kernels.py:31-33).
_MARK = "_vaayu_fused"
# Self-check tolerance on seam outputs, relative L2 against the stock seam (:34-37).
_CHECK_TOL = 5e-2
_ATTR = {"rule": "recurrent_gated_delta_rule", "conv": "causal_conv1d_update"}
_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _require_backend():
    if triton is None:
        raise ImportError(globals().get("_LOAD_ERROR", "vaayu_amd kernels unavailable"))
    return _lib.load()


def _strides(*values):
    """Element strides as the int64 array the C ABI reads (kept alive by the caller)."""
    return (ctypes.c_int64 * len(values))(*values)


def _code(t, what):
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"{what} must be bf16, fp16 or fp32, got {t.dtype}") from None


def gated_delta_seams(model) -> dict:
    """{"rule": [...], "conv": [...], "norm": [...]}: every gated-delta mixer under `model`
    (itself included) exposing each seam (vaayu/gated_delta_kernels.py:43-61). A mixer is a
    module with a callable `recurrent_gated_delta_rule`; its `norm` counts only with a 1-D
    `weight` and a float `variance_epsilon` (the gated RMSNorm's surface)."""
    seams = {"rule": [], "conv": [], "norm": []}
    for module in model.modules():
        if not callable(getattr(module, "recurrent_gated_delta_rule", None)):
            continue
        seams["rule"].append(module)
        if callable(getattr(module, "causal_conv1d_update", None)):
            seams["conv"].append(module)
        norm = getattr(module, "norm", None)
        weight = getattr(norm, "weight", None)
        if (isinstance(weight, torch.Tensor) and weight.dim() == 1
                and isinstance(getattr(norm, "variance_epsilon", None), float)):
            seams["norm"].append(module)
    return seams


def fused_recurrent_rule(query, key, value, g, beta, initial_state, output_final_state,
                         use_qk_l2norm_in_kernel=False):
    """Drop-in for transformers' `torch_recurrent_gated_delta_rule`
    (vaayu/gated_delta_kernels.py:113-133): same arguments, same `(output [B, T, HV, V] in
    query.dtype, fp32 state | None)`, one launch. l2norm runs in fp32; `initial_state` may
    be None, bf16, fp16 or fp32."""
    lib = _require_backend()
    B, T, HV, K = key.shape
    V = value.shape[-1]
    query, key, value = (x if x.stride(-1) == 1 else x.contiguous() for x in (query, key, value))
    if key.dtype != query.dtype or value.dtype != query.dtype:
        key, value = key.to(query.dtype), value.to(query.dtype)
    o = torch.empty(B, T, HV, V, device=value.device, dtype=query.dtype)
    ht = (torch.empty(B, HV, K, V, device=value.device, dtype=torch.float32)
          if output_final_state else None)
    sh = initial_state.stride() if initial_state is not None else (0, 0, 0, 0)
    strides = _strides(*query.stride()[:3], *key.stride()[:3], *value.stride()[:3],
                       *g.stride(), *beta.stride(), *sh)
    rc = lib.vaayu_gdn_rule(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), g.data_ptr(), beta.data_ptr(),
        initial_state.data_ptr() if initial_state is not None else None, o.data_ptr(),
        ht.data_ptr() if ht is not None else None, ctypes.addressof(strides), B, T, HV, K, V,
        1 / (K ** 0.5), _code(query, "query"), _code(g, "g"), _code(beta, "beta"),
        _code(initial_state, "initial_state") if initial_state is not None else 2,
        int(bool(use_qk_l2norm_in_kernel)), _lib.stream_ptr(value.device))
    _lib.check(rc, "vaayu_gdn_rule")
    return o, ht


def fused_conv_update(hidden_states, conv_state, weight, bias=None, activation=None):
    """One-token drop-in for transformers' `causal_conv1d_update`
    (vaayu/gated_delta_kernels.py:178-190): shifts `conv_state` in place (any strides) and
    returns silu(conv) as [B, D, 1]. Like the fallback, it applies silu whatever
    `activation` says."""
    lib = _require_backend()
    B, D, _ = hidden_states.shape
    W = conv_state.shape[-1]
    o = torch.empty(B, D, 1, device=hidden_states.device, dtype=hidden_states.dtype)
    strides = _strides(hidden_states.stride(0), hidden_states.stride(1),
                       *conv_state.stride(), *weight.stride())
    rc = lib.vaayu_gdn_conv_update(
        hidden_states.data_ptr(), conv_state.data_ptr(), weight.data_ptr(),
        bias.data_ptr() if bias is not None else None, o.data_ptr(), ctypes.addressof(strides),
        B, D, W,
        _code(hidden_states, "hidden_states"), _code(conv_state, "conv_state"),
        _code(weight, "weight"), _code(bias, "bias") if bias is not None else 2,
        _lib.stream_ptr(hidden_states.device))
    _lib.check(rc, "vaayu_gdn_conv_update")
    return o


def fused_gated_norm(weight, eps, hidden_states, gate):
    """transformers' `*RMSNormGated.forward(hidden_states, gate)` in one launch, at the
    stock rounding points (vaayu/gated_delta_kernels.py:225-235). Rows are everything but
    the last dim."""
    lib = _require_backend()
    n = weight.numel()
    x = hidden_states.reshape(-1, n)
    z = gate.reshape(-1, n)
    o = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    strides = _strides(*x.stride(), *z.stride(), weight.stride(0))
    round_mid = torch.promote_types(weight.dtype, x.dtype) == x.dtype
    rc = lib.vaayu_gdn_gated_norm(
        x.data_ptr(), z.data_ptr(), weight.data_ptr(), o.data_ptr(), ctypes.addressof(strides),
        x.shape[0], n,
        float(eps), _code(x, "hidden_states"), _code(z, "gate"), _code(weight, "weight"),
        int(round_mid), _lib.stream_ptr(x.device))
    _lib.check(rc, "vaayu_gdn_gated_norm")
    return o.view(hidden_states.shape)


def _patch_norm(norm):
    """Patch the norm's forward IN PLACE, reading `norm.weight` at call time: a streamed
    layer's Parameters are replaced on every load (vaayu/gated_delta_kernels.py:238-249)."""
    stock = norm.forward

    def forward(hidden_states, gate=None):
        if gate is None:
            return stock(hidden_states, gate)
        return fused_gated_norm(norm.weight, norm.variance_epsilon, hidden_states, gate)

    setattr(forward, _MARK, stock)
    norm.forward = forward


def _rule_seam(stock):
    def seam(query, key, value, g, beta, initial_state, output_final_state,
             use_qk_l2norm_in_kernel=False):
        return fused_recurrent_rule(query, key, value, g, beta, initial_state,
                                    output_final_state, use_qk_l2norm_in_kernel)

    setattr(seam, _MARK, stock)
    return seam


def _conv_seam(stock):
    """Multi-token calls go to the stock seam; HF's decode path never sends them
    (vaayu/gated_delta_kernels.py:193-200)."""
    def seam(hidden_states, conv_state, weight, bias=None, activation=None):
        if hidden_states.shape[-1] != 1:
            return stock(hidden_states, conv_state, weight, bias, activation)
        return fused_conv_update(hidden_states, conv_state, weight, bias, activation)

    setattr(seam, _MARK, stock)
    return seam


def _rel(a, b) -> float:
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-12)).item()


def _randn(gen, device, *shape):
    return torch.randn(*shape, generator=gen, device=device)


def _rule_geometry(mixer):
    """(HV, K, V) read off the mixer when it exposes them, else a tiny fallback
    (vaayu/gated_delta_kernels.py:275-280): the self-check runs the geometry decode uses."""
    hv, k, v = (getattr(mixer, "num_v_heads", None), getattr(mixer, "head_k_dim", None),
                getattr(mixer, "head_v_dim", None))
    if isinstance(hv, int) and isinstance(k, int) and isinstance(v, int):
        return hv, k, v
    return 2, 16, 16


def _conv_geometry(mixer):
    """(D, W) from the mixer's conv1d weight [D, 1, W], shape only (:283-288)."""
    weight = getattr(getattr(mixer, "conv1d", None), "weight", None)
    if isinstance(weight, torch.Tensor) and weight.dim() == 3:
        d, _, w = weight.shape
        return d, w
    return 64, 4


def _check_rule(stock, device, dtype, geom) -> float:
    """Stock vs fused at B=1, T=1 on random inputs in the model's dtype (:295-307)."""
    HV, K, V = geom
    gen = torch.Generator(device=device).manual_seed(0)
    q = _randn(gen, device, 1, 1, HV, K).to(dtype)
    k = _randn(gen, device, 1, 1, HV, K).to(dtype)
    v = _randn(gen, device, 1, 1, HV, V).to(dtype)
    g = -torch.rand(1, 1, HV, generator=gen, device=device)
    beta = torch.rand(1, 1, HV, generator=gen, device=device).to(dtype)
    h0 = (_randn(gen, device, 1, HV, K, V) * 0.1).to(dtype)
    kw = dict(g=g, beta=beta, output_final_state=True, use_qk_l2norm_in_kernel=True)
    so, sh = stock(q, k, v, initial_state=h0.clone(), **kw)
    fo, fh = fused_recurrent_rule(q, k, v, initial_state=h0.clone(), **kw)
    return max(_rel(fo, so), _rel(fh, sh))


def _check_conv(stock, device, dtype, geom) -> float:
    """inf unless the conv state is bit-identical to the stock seam's (:310-320)."""
    D, W = geom
    gen = torch.Generator(device=device).manual_seed(0)
    x = _randn(gen, device, 1, 1, D).to(dtype).transpose(1, 2)
    state = _randn(gen, device, 1, W, D).to(dtype).transpose(1, 2)
    w = _randn(gen, device, D, W).to(dtype)
    s_state, f_state = state.clone(), state.clone()
    so = stock(x, s_state, w, None, "silu")
    fo = fused_conv_update(x, f_state, w, None, "silu")
    return _rel(fo, so) if torch.equal(f_state, s_state) else math.inf


def _check_norm(norm, device, dtype) -> float:
    """A stand-in carries the weight: a streamed layer's own may be on the meta device
    (:323-333). It also carries the norm's `activation` name, which newer transformers'
    forward reads (a gate other than silu then fails the check and stays stock)."""
    gen = torch.Generator(device=device).manual_seed(0)
    n = norm.weight.numel()
    stand_in = types.SimpleNamespace(weight=_randn(gen, device, n).to(norm.weight.dtype),
                                     variance_epsilon=norm.variance_epsilon,
                                     activation=getattr(norm, "activation", "silu"))
    x, z = (_randn(gen, device, 4, n).to(dtype) for _ in range(2))
    so = type(norm).forward(stand_in, x, z)
    fo = fused_gated_norm(stand_in.weight, stand_in.variance_epsilon, x, z)
    return _rel(fo, so)


def _passes_self_check(seam, stock, mixer, device, dtype) -> bool:
    """(vaayu/gated_delta_kernels.py:336-354)"""
    try:
        if seam == "norm":
            err = _check_norm(mixer.norm, device, dtype)
        elif seam == "rule":
            err = _check_rule(stock, device, dtype, _rule_geometry(mixer))
        else:
            err = _check_conv(stock, device, dtype, _conv_geometry(mixer))
    except Exception as exc:  # a launch failure, or a stock seam with another contract
        why = f"{type(exc).__name__}: {exc}"
    else:
        if err <= _CHECK_TOL:
            return True
        why = ("its conv state is not bit-identical to the stock seam's" if math.isinf(err)
               else f"relL2 {err:.2e} vs the stock seam, tolerance {_CHECK_TOL:.0e}")
    print(f"[Vaayu] WARNING: fused gated-delta '{seam}' kernel failed its self-check "
          f"({why}); that seam stays on the stock torch path")
    return False


def _install(seam, mixer, stock):
    if seam == "norm":
        _patch_norm(mixer.norm)
    elif seam == "rule":
        mixer.recurrent_gated_delta_rule = _rule_seam(stock)
    else:
        mixer.causal_conv1d_update = _conv_seam(stock)


def install_gated_delta_kernels(hf_model, device, dtype) -> dict:
    """Put a fused kernel on every gated-delta seam under `hf_model` whose on-device
    self-check passes (vaayu/gated_delta_kernels.py:364-410). Returns {"rule": n, "conv": n,
    "norm": n}, already-fused seams included, so a second call is a no-op. Nothing is
    installed off the GPU or without the kernel library, nor -- all-zero counts, nothing
    touched -- when `device` names a GPU index that is not the current one (the kernels
    launch on the current device's stream)."""
    counts = {"rule": 0, "conv": 0, "norm": 0}
    if triton is None or torch.device(device).type != "cuda":
        return counts
    dev_index = torch.device(device).index
    if dev_index is not None and dev_index != torch.cuda.current_device():
        print(f"[Vaayu] WARNING: fused gated-delta kernels not installed: model device {device} "
              f"is not the current CUDA device ({torch.cuda.current_device()}); decode keeps the "
              f"stock torch path")
        return counts
    verdicts = {}
    for seam, mixers in gated_delta_seams(hf_model).items():
        for mixer in mixers:
            current = mixer.norm.forward if seam == "norm" else getattr(mixer, _ATTR[seam])
            if not hasattr(current, _MARK):
                if seam == "norm":
                    key = (seam, type(mixer.norm), mixer.norm.weight.numel(),
                           mixer.norm.weight.dtype, mixer.norm.variance_epsilon)
                elif seam == "rule":
                    key = (seam, current, *_rule_geometry(mixer))
                else:
                    key = (seam, current, *_conv_geometry(mixer))
                if key not in verdicts:
                    verdicts[key] = _passes_self_check(seam, current, mixer, device, dtype)
                if not verdicts[key]:
                    continue
                _install(seam, mixer, current)
            counts[seam] += 1
    return counts
