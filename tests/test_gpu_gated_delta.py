"""The gated-delta decode kernels on the GPU (vaayu_amd/csrc/gated_delta.hip through
vaayu_amd/gated_delta_kernels.py), held to the oracle (oracle/gated_delta.py: the reference
kernels' algorithm, correctly rounded) and to the reference's own bar
(tests/test_gated_delta_kernels.py: no further from an fp64 truth than the stock torch
seam, conv state bit-exact with the stock seam's).

Tolerances: the kernels sum in fp32, the oracle in fp64, so a value rounded to a 16-bit
dtype may land one unit in the last place away; where an intermediate is rounded too (the
norm's normalised x, the conv's sum) that flip can carry, so 16-bit outputs are held to two
units in the last place and to mostly equal bits; fp32 outputs and the fp32 state to
relL2 1e-5."""
import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.gated_delta_kernels as gdk
from oracle import gated_delta as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

tf = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
stock_rule = tf.torch_recurrent_gated_delta_rule
stock_conv = tf.causal_conv1d_update
StockNorm = tf.Qwen3NextRMSNormGated

DEV = "cuda"
GEOMS = {"qwen3next": dict(HV=32, HK=16, K=128, V=128, W=4),
         "odd": dict(HV=6, HK=3, K=48, V=80, W=3)}
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}
TINY = {torch.bfloat16: 0.0, torch.float16: 2.0 ** -24}     # fp16's subnormal spacing


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _close_to_oracle(got, ref, dtype, equal_frac=0.9):
    got = O.to_np(got)
    if dtype == torch.float32:
        assert O.rel_l2(got, ref) <= 1e-5
        return
    scale = np.abs(ref).max()
    tol = 2 * ULP[dtype] * np.abs(ref) + max(1e-6 * scale, 2 * TINY[dtype])
    assert (np.abs(got - ref) <= tol).all()
    assert (got == ref).mean() >= equal_frac


def _rule_inputs(geom, B, T_, dtype, h0_dtype, strided=False, seed=0):
    torch.manual_seed(seed)
    HV, K, V = geom["HV"], geom["K"], geom["V"]
    q = torch.randn(B, T_, HV, K, device=DEV).to(dtype)
    k = torch.randn(B, T_, HV, K, device=DEV).to(dtype)
    v = torch.randn(B, T_, HV, 2 * V if strided else V, device=DEV).to(dtype)[..., :V]
    g = -F.softplus(torch.randn(B, T_, HV, device=DEV))
    beta = torch.sigmoid(torch.randn(B, T_, HV, device=DEV)).to(dtype)
    h0 = (None if h0_dtype is None
          else (torch.randn(B, HV, K, V, device=DEV) * 0.1).to(h0_dtype))
    return q, k, v, g, beta, h0


def _ref_rule(q, k, v, g, beta, h0):
    """The rule in fp64 with qk-l2norm (tests/test_gated_delta_kernels.py:120-136)."""
    q, k, v, g, beta = (x.double() for x in (q, k, v, g, beta))
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * q.shape[-1] ** -0.5
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    B, T_, HV, K = k.shape
    h = (torch.zeros(B, HV, K, v.shape[-1], dtype=torch.float64, device=q.device)
         if h0 is None else h0.double())
    out = []
    for t in range(T_):
        h = h * g[:, t].exp()[..., None, None]
        delta = (v[:, t] - (h * k[:, t, :, :, None]).sum(-2)) * beta[:, t, :, None]
        h = h + k[:, t, :, :, None] * delta[:, :, None, :]
        out.append((h * q[:, t, :, :, None]).sum(-2))
    return torch.stack(out, 1), h


def _both_rules(q, k, v, g, beta, h0, final=True, l2=True):
    kw = dict(g=g, beta=beta, output_final_state=final, use_qk_l2norm_in_kernel=l2)
    clone = (lambda: None) if h0 is None else h0.clone
    return (stock_rule(q, k, v, initial_state=clone(), **kw),
            gdk.fused_recurrent_rule(q, k, v, initial_state=clone(), **kw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("h0_dtype", [None, torch.bfloat16, torch.float32],
                         ids=["h0none", "h0bf16", "h0fp32"])
@pytest.mark.parametrize("B,T_", [(1, 1), (2, 1), (1, 3)], ids=["decode", "batch2", "T3"])
@pytest.mark.parametrize("geom", GEOMS)
def test_rule_matches_the_oracle_and_beats_stock(geom, B, T_, h0_dtype, dtype):
    print(f"rule {geom} B={B} T={T_} h0={h0_dtype} act={dtype}", flush=True)
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS[geom], B, T_, dtype, h0_dtype)
    (so, sh), (fo, fh) = _both_rules(q, k, v, g, beta, h0)
    torch.cuda.synchronize()
    assert fo.shape == so.shape and fo.dtype == so.dtype
    assert fh.shape == sh.shape and fh.dtype == torch.float32
    ro, rh = G.gdn_rule(q, k, v, g, beta, h0, act=O.act_name(dtype))
    _close_to_oracle(fo, ro, dtype)
    assert O.rel_l2(O.to_np(fh), rh) <= 1e-5
    # the reference's bar; fp32 values carry only fp32 rounding noise on both sides (the
    # reference runs it on 16-bit outputs), hence the 1e-6 floor
    to, th = _ref_rule(q, k, v, g, beta, h0)
    assert _rel(fo, to) <= 1.25 * _rel(so, to) + 1e-6
    assert _rel(fh, th) <= 1.25 * _rel(sh, th) + 1e-6


def test_rule_without_l2norm():
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS["odd"], 1, 2, torch.float32, torch.float32, seed=1)
    q, k = q * 0.2, k * 0.2
    (so, sh), (fo, fh) = _both_rules(q, k, v, g, beta, h0, l2=False)
    ro, rh = G.gdn_rule(q, k, v, g, beta, h0, l2=False, act="fp32")
    assert O.rel_l2(O.to_np(fo), ro) <= 1e-5 and O.rel_l2(O.to_np(fh), rh) <= 1e-5
    assert _rel(fo, so) <= 1e-5


@pytest.mark.parametrize("geom", GEOMS)
def test_rule_reads_strided_inputs(geom):
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS[geom], 1, 1, torch.bfloat16, torch.bfloat16,
                                        strided=True)
    assert not v.is_contiguous()
    _, (fo, fh) = _both_rules(q, k, v, g, beta, h0)
    _, (co, ch) = _both_rules(q, k, v.contiguous(), g, beta, h0)
    assert torch.equal(fo, co) and torch.equal(fh, ch)


def test_rule_reads_a_strided_state():
    """A state view with other strides (a slice of a larger cache) reads the same values."""
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS["odd"], 2, 1, torch.bfloat16, torch.float32)
    big = torch.zeros(2, 6, 48, 2 * 80, device=DEV)
    big[..., ::2] = h0
    view = big[..., ::2]
    assert not view.is_contiguous()
    _, (fo, fh) = _both_rules(q, k, v, g, beta, view)
    _, (co, ch) = _both_rules(q, k, v, g, beta, h0)
    assert torch.equal(fo, co) and torch.equal(fh, ch)


def test_rule_without_final_state_returns_none():
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS["qwen3next"], 1, 1, torch.bfloat16, torch.bfloat16)
    _, (with_state, _) = _both_rules(q, k, v, g, beta, h0, final=True)
    _, (without, state) = _both_rules(q, k, v, g, beta, h0, final=False)
    assert state is None and torch.equal(without, with_state)


def test_rule_rejects_a_key_dim_past_256():
    q, k, v, g, beta, h0 = _rule_inputs(dict(HV=1, K=320, V=16), 1, 1, torch.bfloat16, None)
    with pytest.raises(Exception):
        gdk.fused_recurrent_rule(q, k, v, g, beta, None, True, True)


# ── conv update ─────────────────────────────────────────────────────────────────────────

def _conv_dim(g):
    return 2 * g["HK"] * g["K"] + g["HV"] * g["V"]


def _conv_inputs(D, W, B, dtype, layout, seed=0):
    torch.manual_seed(seed)
    x = torch.randn(B, 1, D, device=DEV).to(dtype).transpose(1, 2)
    state = torch.randn(B, W, D, device=DEV).to(dtype).transpose(1, 2)
    if layout == "contiguous":
        state = state.contiguous()
    w = torch.randn(D, 1, W, device=DEV).to(dtype).squeeze(1)
    return x, state, w


def _ref_conv(x, state, w, bias):
    full = torch.cat([state.double(), x.double()], -1)[..., 1:]
    out = (full * w.double()[None]).sum(-1, keepdim=True)
    if bias is not None:
        out = out + bias.double()[None, :, None]
    return F.silu(out)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("layout", ["channels_last", "contiguous"])
@pytest.mark.parametrize("geom", GEOMS)
def test_conv_update_state_is_bit_exact(geom, layout, B, dtype):
    print(f"conv {geom} {layout} B={B} {dtype}", flush=True)
    D, W = _conv_dim(GEOMS[geom]), GEOMS[geom]["W"]
    x, state, w = _conv_inputs(D, W, B, dtype, layout)
    s_state, f_state = state.clone(), state.clone()
    so = stock_conv(x, s_state, w, None, "silu")
    fo = gdk.fused_conv_update(x, f_state, w, None, "silu")
    torch.cuda.synchronize()
    assert torch.equal(f_state, s_state)
    assert f_state.stride() == state.stride()
    assert fo.shape == so.shape and fo.dtype == so.dtype
    act = O.act_name(dtype)
    ro, rs = G.gdn_conv_update(x, state, w, None, act, act, act)
    assert np.array_equal(O.to_np(f_state), rs)
    _close_to_oracle(fo, ro, dtype)
    ref = _ref_conv(x, state, w, None)
    assert _rel(fo, ref) <= 1.25 * _rel(so, ref) + 1e-7


def test_conv_update_adds_bias():
    D, W = _conv_dim(GEOMS["qwen3next"]), GEOMS["qwen3next"]["W"]
    x, state, w = _conv_inputs(D, W, 1, torch.bfloat16, "contiguous")
    bias = torch.randn(D, device=DEV).bfloat16()
    s_state, f_state = state.clone(), state.clone()
    so = stock_conv(x, s_state, w, bias, "silu")
    fo = gdk.fused_conv_update(x, f_state, w, bias, "silu")
    assert torch.equal(f_state, s_state)
    ro, _ = G.gdn_conv_update(x, state, w, bias)
    _close_to_oracle(fo, ro, torch.bfloat16)
    ref = _ref_conv(x, state, w, bias)
    assert _rel(fo, ref) <= 1.25 * _rel(so, ref)


def test_conv_update_after_a_pinned_round_trip():
    D, W = _conv_dim(GEOMS["qwen3next"]), GEOMS["qwen3next"]["W"]
    x, state, w = _conv_inputs(D, W, 1, torch.bfloat16, "channels_last")
    state = state.to("cpu").pin_memory().to(DEV)
    s_state, f_state = state.clone(), state.clone()
    stock_conv(x, s_state, w, None, "silu")
    gdk.fused_conv_update(x, f_state, w, None, "silu")
    assert torch.equal(f_state, s_state)


# ── gated norm ──────────────────────────────────────────────────────────────────────────

def _ref_norm(x, z, w, eps):
    x, z, w = x.double(), z.double(), w.double()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w * F.silu(z)


def _stock_norm(n, wdtype, seed=0):
    torch.manual_seed(seed)
    norm = StockNorm(n, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(n))
    return norm.to(DEV).to(wdtype)


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["xbf16", "xfp16", "xfp32"])
@pytest.mark.parametrize("rows", [1, 64, 333])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32], ids=["wbf16", "wfp32"])
@pytest.mark.parametrize("geom", GEOMS)
def test_norm_matches_the_oracle_and_beats_stock(geom, wdtype, rows, xdtype):
    n = GEOMS[geom]["V"]
    norm = _stock_norm(n, wdtype)
    x = torch.randn(rows, n, device=DEV).to(xdtype)
    z = torch.randn(rows, n, device=DEV).to(xdtype)
    so = norm(x, z)
    gdk._patch_norm(norm)
    fo = norm(x, z)
    torch.cuda.synchronize()
    assert fo.shape == so.shape and fo.dtype == so.dtype
    round_mid = torch.promote_types(wdtype, xdtype) == xdtype
    ro = G.gdn_gated_norm(x, z, norm.weight, 1e-6, O.act_name(xdtype), round_mid)
    _close_to_oracle(fo, ro, xdtype)
    ref = _ref_norm(x, z, norm.weight, 1e-6)
    assert _rel(fo, ref) <= 1.25 * _rel(so, ref) + 1e-7


def test_norm_of_a_three_dim_strided_input():
    norm = _stock_norm(128, torch.bfloat16)
    x = torch.randn(2, 5, 256, device=DEV).bfloat16()[..., :128]
    z = torch.randn(2, 5, 128, device=DEV).bfloat16()
    want = norm(x, z)
    gdk._patch_norm(norm)
    got = norm(x, z)
    assert got.shape == want.shape
    ro = G.gdn_gated_norm(x, z, norm.weight, 1e-6, "bf16", True)
    _close_to_oracle(got, ro, torch.bfloat16)


def test_patched_norm_reads_a_weight_replaced_after_install():
    norm = _stock_norm(128, torch.bfloat16)
    gdk._patch_norm(norm)
    norm.weight = torch.nn.Parameter(torch.randn(128, device=DEV).bfloat16())
    x = torch.randn(4, 128, device=DEV).bfloat16()
    z = torch.randn(4, 128, device=DEV).bfloat16()
    want = type(norm).forward(norm, x, z)
    assert _rel(norm(x, z), want) < 1e-2


# ── installer ───────────────────────────────────────────────────────────────────────────

class _Mixer(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.recurrent_gated_delta_rule = stock_rule
        self.causal_conv1d_update = stock_conv
        self.norm = StockNorm(128, eps=1e-6)
        self.num_v_heads, self.head_k_dim, self.head_v_dim = 32, 128, 128
        self.conv1d = torch.nn.Conv1d(8192, 8192, 4, groups=8192, bias=False)


def _mixer():
    return _Mixer().to(DEV).bfloat16()


def _seam_fns(m):
    return [m.recurrent_gated_delta_rule, m.causal_conv1d_update, m.norm.forward]


def test_install_covers_every_seam_and_is_idempotent():
    mixer = _mixer()
    want = {"rule": 1, "conv": 1, "norm": 1}
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == want
    first = _seam_fns(mixer)
    assert all(hasattr(f, gdk._MARK) for f in first)
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == want
    assert all(a == b for a, b in zip(first, _seam_fns(mixer)))


def test_self_check_runs_the_mixers_real_rule_geometry(monkeypatch):
    seen = []
    real = gdk._check_rule

    def spy(stock, device, dtype, geom):
        seen.append(geom)
        return real(stock, device, dtype, geom)

    monkeypatch.setattr(gdk, "_check_rule", spy)
    gdk.install_gated_delta_kernels(_mixer(), "cuda", torch.bfloat16)
    assert seen == [(32, 128, 128)]


def test_refuses_a_non_current_device(capsys):
    mixer = _mixer()
    before = _seam_fns(mixer)
    assert gdk.install_gated_delta_kernels(mixer, "cuda:1", torch.bfloat16) == \
        {"rule": 0, "conv": 0, "norm": 0}
    assert all(a == b for a, b in zip(before, _seam_fns(mixer)))
    out = capsys.readouterr().out
    assert "WARNING" in out and "cuda:1" in out and "current CUDA device" in out


def test_a_rule_that_fails_its_self_check_stays_stock_and_warns(monkeypatch, capsys):
    def wrong(q, k, v, g, beta, initial_state, output_final_state,
              use_qk_l2norm_in_kernel=False):
        B, T_, HV, K = k.shape
        return (torch.zeros_like(v),
                torch.zeros(B, HV, K, v.shape[-1], device=v.device, dtype=torch.float32))

    monkeypatch.setattr(gdk, "fused_recurrent_rule", wrong)
    mixer = _mixer()
    stock = mixer.recurrent_gated_delta_rule
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == \
        {"rule": 0, "conv": 1, "norm": 1}
    assert mixer.recurrent_gated_delta_rule is stock
    out = capsys.readouterr().out
    assert "WARNING" in out and "'rule'" in out and "relL2" in out


def test_a_conv_that_does_not_update_the_state_stays_stock(monkeypatch, capsys):
    def no_state_update(hidden_states, conv_state, weight, bias=None, activation=None):
        B, D, _ = hidden_states.shape
        return torch.zeros(B, D, 1, device=hidden_states.device, dtype=hidden_states.dtype)

    monkeypatch.setattr(gdk, "fused_conv_update", no_state_update)
    mixer = _mixer()
    stock = mixer.causal_conv1d_update
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == \
        {"rule": 1, "conv": 0, "norm": 1}
    assert mixer.causal_conv1d_update is stock
    assert "not bit-identical" in capsys.readouterr().out


def test_a_norm_with_different_math_stays_stock_and_warns(capsys):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    mixer = _mixer()
    mixer.norm = LlamaRMSNorm(128).to(DEV)
    stock = mixer.norm.forward
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == \
        {"rule": 1, "conv": 1, "norm": 0}
    assert mixer.norm.forward == stock
    assert "'norm'" in capsys.readouterr().out


def test_one_decode_step_of_a_mixer_through_the_three_seams():
    """conv -> rule -> norm as a mixer's decode step chains them, fused against stock on
    the same inputs, no further from fp64 than stock."""
    torch.manual_seed(3)
    geo = GEOMS["qwen3next"]
    D, W = _conv_dim(geo), geo["W"]
    x, state, w = _conv_inputs(D, W, 1, torch.bfloat16, "channels_last", seed=3)
    s_state, f_state = state.clone(), state.clone()
    HV, HK, K, V = geo["HV"], geo["HK"], geo["K"], geo["V"]
    g = -F.softplus(torch.randn(1, 1, HV, device=DEV))
    beta = torch.sigmoid(torch.randn(1, 1, HV, device=DEV)).bfloat16()
    h0 = (torch.randn(1, HV, K, V, device=DEV) * 0.1)
    zgate = torch.randn(1, 1, HV, V, device=DEV).bfloat16()
    norm = _stock_norm(V, torch.bfloat16)
    fused_norm = copy.deepcopy(norm)
    gdk._patch_norm(fused_norm)

    def step(conv, rule, nrm, st):
        qkv = conv(x, st, w, None, "silu")[..., 0]                        # [1, D]
        q, k, v = torch.split(qkv, [HK * K, HK * K, HV * V], -1)
        q = q.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
        k = k.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
        v = v.reshape(1, 1, HV, V)
        o, h = rule(q, k, v, g=g, beta=beta, initial_state=h0.clone(), output_final_state=True,
                    use_qk_l2norm_in_kernel=True)
        return nrm(o, zgate), h

    so, sh = step(stock_conv, stock_rule, norm, s_state)
    fo, fh = step(gdk.fused_conv_update, gdk.fused_recurrent_rule, fused_norm, f_state)
    assert torch.equal(s_state, f_state)
    assert _rel(fo, so) < 2e-2 and _rel(fh, sh) < 1e-2
