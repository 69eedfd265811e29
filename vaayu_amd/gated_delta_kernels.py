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

The host side is a table of seam descriptors (`_Seam`): how a mixer exposes the seam (by
its surface, never by class or architecture name), what callable is there now, the key
its verdict is kept under, the on-device self-check against the stock seam, and how the
fused seam is put in. A seam whose check disagrees stays stock with a WARNING; a fused
seam carries the stock callable it replaced under `_MARK`, so installing twice is a
no-op. Without the built library `triton` is None and nothing is installed (the
reference's "no Triton" state); a direct kernel call then raises ImportError.
"""
import ctypes
import math
import types

import torch

from . import _lib

try:
    _lib.load()
    _BACKEND, _LOAD_ERROR = _lib, None
except ImportError as _exc:              # reported at the first kernel call
    _BACKEND, _LOAD_ERROR = None, str(_exc)

# The kernel backend's truthiness under the name the reference's installer and tests use
# (they set it to None to stand for a machine without the kernels).
triton = _BACKEND

# A fused seam carries the stock callable it replaced under this attribute
# (vaayu/gated_delta_kernels.py:31-33).
_MARK = "_vaayu_fused"
# Self-check tolerance on seam outputs, relative L2 against the stock seam (:34-37).
_CHECK_TOL = 5e-2
_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _require_backend():
    if triton is None:
        raise ImportError(_LOAD_ERROR or "vaayu_amd kernels unavailable")
    return _lib.load()


def _strides(*values):
    """Element strides as the int64 array the C ABI reads (kept alive by the caller)."""
    return (ctypes.c_int64 * len(values))(*values)


def _code(t, what):
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"{what} must be bf16, fp16 or fp32, got {t.dtype}") from None


# ── the three kernels ────────────────────────────────────────────────────────────────────

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


# ── fused seams ──────────────────────────────────────────────────────────────────────────

def _marked(fn, stock):
    setattr(fn, _MARK, stock)
    return fn


def _patch_norm(norm):
    """Replace the norm's forward IN PLACE with one that reads `norm.weight` at call time
    (a streamed layer's Parameters are replaced on every load; vaayu/gated_delta_kernels.py:
    238-249). A call without a gate goes to the stock forward."""
    stock = norm.forward

    def forward(hidden_states, gate=None):
        if gate is None:
            return stock(hidden_states, gate)
        return fused_gated_norm(norm.weight, norm.variance_epsilon, hidden_states, gate)

    norm.forward = _marked(forward, stock)


def _rule_seam(stock):
    def seam(query, key, value, g, beta, initial_state, output_final_state,
             use_qk_l2norm_in_kernel=False):
        return fused_recurrent_rule(query, key, value, g, beta, initial_state,
                                    output_final_state, use_qk_l2norm_in_kernel)
    return _marked(seam, stock)


def _conv_seam(stock):
    """Multi-token calls go to the stock seam; transformers' decode path never sends them
    (vaayu/gated_delta_kernels.py:193-200)."""
    def seam(hidden_states, conv_state, weight, bias=None, activation=None):
        if hidden_states.shape[-1] != 1:
            return stock(hidden_states, conv_state, weight, bias, activation)
        return fused_conv_update(hidden_states, conv_state, weight, bias, activation)
    return _marked(seam, stock)


# ── self-checks: stock against fused on the device, at the mixer's decode geometry ──────

def _rel(a, b) -> float:
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-12)).item()


def _rule_geometry(mixer):
    """(HV, K, V) as the mixer declares them, else a tiny stand-in (vaayu/gated_delta_kernels.
    py:275-280): the check should run the geometry decode will."""
    dims = tuple(getattr(mixer, a, None) for a in ("num_v_heads", "head_k_dim", "head_v_dim"))
    return dims if all(isinstance(d, int) for d in dims) else (2, 16, 16)


def _conv_geometry(mixer):
    """(D, W) from the mixer's conv1d weight [D, 1, W], by shape only (safe on the meta
    device; :283-288), else a stand-in."""
    weight = getattr(getattr(mixer, "conv1d", None), "weight", None)
    if isinstance(weight, torch.Tensor) and weight.dim() == 3:
        return weight.shape[0], weight.shape[2]
    return 64, 4


class _Draw:
    """Seeded random tensors on one device, made in the dtype asked for."""

    def __init__(self, device):
        self.device = device
        self.gen = torch.Generator(device=device).manual_seed(0)

    def normal(self, *shape, dtype=torch.float32, scale=1.0):
        return (torch.randn(*shape, generator=self.gen, device=self.device) * scale).to(dtype)

    def uniform(self, *shape, dtype=torch.float32):
        return torch.rand(*shape, generator=self.gen, device=self.device).to(dtype)


def _check_rule(stock, device, dtype, geom) -> float:
    """relL2 of the fused rule against `stock` at one decode step (B = T = 1, l2 norm on),
    output and final state, on random inputs in the model's dtype (:295-307)."""
    heads, k_dim, v_dim = geom
    d = _Draw(device)
    q, k = d.normal(1, 1, heads, k_dim, dtype=dtype), d.normal(1, 1, heads, k_dim, dtype=dtype)
    v = d.normal(1, 1, heads, v_dim, dtype=dtype)
    args = dict(g=-d.uniform(1, 1, heads), beta=d.uniform(1, 1, heads, dtype=dtype),
                output_final_state=True, use_qk_l2norm_in_kernel=True)
    state = d.normal(1, heads, k_dim, v_dim, dtype=dtype, scale=0.1)
    want_o, want_h = stock(q, k, v, initial_state=state.clone(), **args)
    got_o, got_h = fused_recurrent_rule(q, k, v, initial_state=state.clone(), **args)
    return max(_rel(got_o, want_o), _rel(got_h, want_h))


def _check_conv(stock, device, dtype, geom) -> float:
    """relL2 of the fused conv update's output, or inf unless the in-place state update is
    bit-identical to the stock seam's (:310-320). Inputs as transformers passes them:
    x [B, D, 1] and a channels-last state."""
    channels, width = geom
    d = _Draw(device)
    x = d.normal(1, 1, channels, dtype=dtype).transpose(1, 2)
    state = d.normal(1, width, channels, dtype=dtype).transpose(1, 2)
    w = d.normal(channels, width, dtype=dtype)
    stock_state, fused_state = state.clone(), state.clone()
    want = stock(x, stock_state, w, None, "silu")
    got = fused_conv_update(x, fused_state, w, None, "silu")
    return _rel(got, want) if torch.equal(fused_state, stock_state) else math.inf


def _check_norm(norm, device, dtype) -> float:
    """relL2 of the fused gated norm against the norm class's own forward, run on a
    stand-in that carries a fresh weight (a streamed layer's may be on the meta device;
    :323-333) and the norm's `activation` name (newer transformers reads it: a gate other
    than silu then fails the check)."""
    d = _Draw(device)
    n = norm.weight.numel()
    stand_in = types.SimpleNamespace(weight=d.normal(n, dtype=norm.weight.dtype),
                                     variance_epsilon=norm.variance_epsilon,
                                     activation=getattr(norm, "activation", "silu"))
    x, z = d.normal(4, n, dtype=dtype), d.normal(4, n, dtype=dtype)
    want = type(norm).forward(stand_in, x, z)
    return _rel(fused_gated_norm(stand_in.weight, stand_in.variance_epsilon, x, z), want)


# ── the seam table ───────────────────────────────────────────────────────────────────────

class _Seam:
    """One kind of seam: `present(mixer)` (by surface), `current(mixer)` (the callable in
    place now), `key(mixer, current)` (what its verdict depends on), `error(...)` (the
    self-check's relL2, inf for a state mismatch) and `install(mixer, stock)`."""

    def __init__(self, name, present, current, key, error, install):
        self.name, self.present, self.current = name, present, current
        self.key, self.error, self.install = key, error, install


def _has_gated_norm(mixer) -> bool:
    norm = getattr(mixer, "norm", None)
    weight = getattr(norm, "weight", None)
    return (isinstance(weight, torch.Tensor) and weight.dim() == 1
            and isinstance(getattr(norm, "variance_epsilon", None), float))


def _set_attr(attr, wrap):
    def install(mixer, stock):
        setattr(mixer, attr, wrap(stock))
    return install


# Looked up by name at call time, so the module's checks can be swapped (tests do).
_SEAMS = (
    _Seam("rule",
          present=lambda m: True,
          current=lambda m: m.recurrent_gated_delta_rule,
          key=lambda m, cur: ("rule", cur, *_rule_geometry(m)),
          error=lambda m, cur, dev, dt: _check_rule(cur, dev, dt, _rule_geometry(m)),
          install=_set_attr("recurrent_gated_delta_rule", _rule_seam)),
    _Seam("conv",
          present=lambda m: callable(getattr(m, "causal_conv1d_update", None)),
          current=lambda m: m.causal_conv1d_update,
          key=lambda m, cur: ("conv", cur, *_conv_geometry(m)),
          error=lambda m, cur, dev, dt: _check_conv(cur, dev, dt, _conv_geometry(m)),
          install=_set_attr("causal_conv1d_update", _conv_seam)),
    _Seam("norm",
          present=_has_gated_norm,
          current=lambda m: m.norm.forward,
          key=lambda m, cur: ("norm", type(m.norm), m.norm.weight.numel(),
                              m.norm.weight.dtype, m.norm.variance_epsilon),
          error=lambda m, cur, dev, dt: _check_norm(m.norm, dev, dt),
          install=lambda m, stock: _patch_norm(m.norm)),
)


def _is_mixer(module) -> bool:
    return callable(getattr(module, "recurrent_gated_delta_rule", None))


def gated_delta_seams(model) -> dict:
    """{"rule": [...], "conv": [...], "norm": [...]}: every gated-delta mixer under `model`
    (itself included) exposing each seam (vaayu/gated_delta_kernels.py:43-61). A mixer is a
    module with a callable `recurrent_gated_delta_rule`; its `norm` counts only with a 1-D
    `weight` and a float `variance_epsilon` (the gated RMSNorm's surface)."""
    mixers = [m for m in model.modules() if _is_mixer(m)]
    return {s.name: [m for m in mixers if s.present(m)] for s in _SEAMS}


def _self_check(seam, mixer, stock, device, dtype) -> bool:
    """True if the fused seam agrees with `stock` on the device; else one WARNING
    (vaayu/gated_delta_kernels.py:336-354)."""
    try:
        err = seam.error(mixer, stock, device, dtype)
    except Exception as exc:  # a launch failure, or a stock seam with another contract
        why = f"{type(exc).__name__}: {exc}"
    else:
        if err <= _CHECK_TOL:
            return True
        why = ("its conv state is not bit-identical to the stock seam's" if math.isinf(err)
               else f"relL2 {err:.2e} vs the stock seam, tolerance {_CHECK_TOL:.0e}")
    print(f"[Vaayu] WARNING: fused gated-delta '{seam.name}' kernel failed its self-check "
          f"({why}); that seam stays on the stock torch path")
    return False


def install_gated_delta_kernels(hf_model, device, dtype) -> dict:
    """Put a fused kernel on every gated-delta seam under `hf_model` whose on-device
    self-check passes (vaayu/gated_delta_kernels.py:364-410). Returns {"rule": n, "conv": n,
    "norm": n}, already-fused seams included, so a second call is a no-op. Nothing is
    installed off the GPU or without the kernel library, nor -- all-zero counts, nothing
    touched -- when `device` names a GPU index that is not the current one (the kernels
    launch on the current device's stream)."""
    counts = {s.name: 0 for s in _SEAMS}
    dev = torch.device(device)
    if triton is None or dev.type != "cuda":
        return counts
    if dev.index is not None and dev.index != torch.cuda.current_device():
        print(f"[Vaayu] WARNING: fused gated-delta kernels not installed: model device {device} "
              f"is not the current CUDA device ({torch.cuda.current_device()}); decode keeps the "
              f"stock torch path")
        return counts
    verdicts = {}            # one self-check per (seam, stock callable / class, geometry)
    found = gated_delta_seams(hf_model)
    for seam in _SEAMS:
        for mixer in found[seam.name]:
            stock = seam.current(mixer)
            if not hasattr(stock, _MARK):
                key = seam.key(mixer, stock)
                if key not in verdicts:
                    verdicts[key] = _self_check(seam, mixer, stock, device, dtype)
                if not verdicts[key]:
                    continue
                seam.install(mixer, stock)
            counts[seam.name] += 1
    return counts
