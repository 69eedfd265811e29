"""The gated-delta oracle (oracle/gated_delta.py) pinned on the CPU, and the host logic of
vaayu_amd/gated_delta_kernels.py that needs no GPU.

The oracle restates the reference's three fused seams (vaayu/gated_delta_kernels.py:66-235).
It is held to transformers' own torch fallbacks -- the stock seams those kernels replace and
the reference's tests compare against -- and to closed forms, so a dropped term, a wrong
sign or a transposed state fails here."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gated_delta as G
from oracle import oracle as O

tf = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
stock_rule = tf.torch_recurrent_gated_delta_rule
stock_conv = tf.causal_conv1d_update
StockNorm = tf.Qwen3NextRMSNormGated

GEOMS = {"qwen3next": dict(HV=32, K=128, V=128, W=4), "odd": dict(HV=6, K=48, V=80, W=3)}


def _rule_inputs(geom, B, T, seed, h0=True):
    gen = torch.Generator().manual_seed(seed)
    HV, K, V = geom["HV"], geom["K"], geom["V"]
    q = torch.randn(B, T, HV, K, generator=gen)
    k = torch.randn(B, T, HV, K, generator=gen)
    v = torch.randn(B, T, HV, V, generator=gen)
    g = -F.softplus(torch.randn(B, T, HV, generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, HV, generator=gen))
    h = torch.randn(B, HV, K, V, generator=gen) * 0.1 if h0 else None
    return q, k, v, g, beta, h


@pytest.mark.parametrize("l2", [True, False])
@pytest.mark.parametrize("B,T", [(1, 1), (2, 3)])
@pytest.mark.parametrize("geom", GEOMS)
def test_rule_matches_the_stock_fallback(geom, B, T, l2):
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS[geom], B, T, seed=B * 10 + T)
    so, sh = stock_rule(q, k, v, g, beta, initial_state=h0.clone(), output_final_state=True,
                        use_qk_l2norm_in_kernel=l2)
    oo, oh = G.gdn_rule(q, k, v, g, beta, h0, l2=l2, act="fp32")
    assert O.rel_l2(oo, O.to_np(so)) < 2e-6
    assert O.rel_l2(oh, O.to_np(sh)) < 2e-6


def test_rule_without_initial_state_starts_from_zeros():
    q, k, v, g, beta, _ = _rule_inputs(GEOMS["odd"], 1, 2, seed=3, h0=False)
    so, sh = stock_rule(q, k, v, g, beta, initial_state=None, output_final_state=True,
                        use_qk_l2norm_in_kernel=True)
    oo, oh = G.gdn_rule(q, k, v, g, beta, None, act="fp32")
    assert O.rel_l2(oo, O.to_np(so)) < 2e-6 and O.rel_l2(oh, O.to_np(sh)) < 2e-6


def test_rule_with_zero_beta_is_pure_decay():
    """beta = 0: the state only decays, h_t = h0 exp(g_1 + ... + g_t), o_t = h_t^T q_t."""
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS["odd"], 1, 3, seed=4)
    beta = torch.zeros_like(beta)
    o, h = G.gdn_rule(q, k, v, g, beta, h0, l2=False, act="fp32")
    decay = torch.exp(torch.cumsum(g.double(), 1))                # [1, T, HV]
    for t in range(3):
        ht = h0.double() * decay[:, t, :, None, None]
        want = torch.einsum("bhkv,bhk->bhv", ht, q[:, t].double() / math.sqrt(48))
        assert O.rel_l2(o[:, t], want.numpy()) < 1e-6
    assert O.rel_l2(h, (h0.double() * decay[:, -1, :, None, None]).numpy()) < 1e-6


def test_rule_one_cell_by_hand():
    """K = V = 1, no l2: h' = h e^g + k ((v - h e^g k) beta), o = h' q."""
    h0, q, k, v, g, b = 0.5, 2.0, 3.0, 7.0, -0.25, 0.4
    hd = h0 * math.exp(g)
    h1 = hd + k * ((v - hd * k) * b)
    o, h = G.gdn_rule(*(torch.tensor(x, dtype=torch.float64).reshape(1, 1, 1, 1)
                        for x in (q, k, v)),
                      torch.tensor([[[g]]]), torch.tensor([[[b]]]),
                      torch.tensor(h0).reshape(1, 1, 1, 1), l2=False, act="fp32")
    assert abs(float(o.ravel()[0]) - h1 * q) < 1e-5 and abs(float(h.ravel()[0]) - h1) < 1e-6


def test_rule_steps_compose():
    """T steps in one call = T one-step calls carrying the state."""
    q, k, v, g, beta, h0 = _rule_inputs(GEOMS["odd"], 2, 4, seed=5)
    o_all, h_all = G.gdn_rule(q, k, v, g, beta, h0, act="fp32")
    h = h0
    for t in range(4):
        o_t, h = G.gdn_rule(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1],
                            beta[:, t:t + 1], torch.from_numpy(h) if t else h, act="fp32")
        np.testing.assert_allclose(o_t[:, 0], o_all[:, t], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(h, h_all, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["channels_last", "contiguous"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("geom", GEOMS)
def test_conv_update_matches_the_stock_fallback(geom, layout, bias, dtype):
    D, W = 2 * 16 * GEOMS[geom]["K"] // 8 + GEOMS[geom]["V"], GEOMS[geom]["W"]
    gen = torch.Generator().manual_seed(D + W)
    x = torch.randn(2, 1, D, generator=gen).to(dtype).transpose(1, 2)
    state = torch.randn(2, W, D, generator=gen).to(dtype).transpose(1, 2)
    if layout == "contiguous":
        state = state.contiguous()
    w = torch.randn(D, W, generator=gen).to(dtype)
    b = torch.randn(D, generator=gen).to(dtype) if bias else None
    act = O.act_name(dtype)
    want_out, want_state = G.gdn_conv_update(x, state, w, b, act, act, act)
    s_state = state.clone()
    so = stock_conv(x, s_state, w, b, "silu")
    assert np.array_equal(want_state, O.to_np(s_state))           # pure copies: bit-exact
    got, ref = O.to_np(so), want_out
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    else:                           # the stock conv's own rounding: at most one bf16 ulp
        assert np.abs(got - ref).max() <= 2.0 ** -7 * np.abs(ref).max()
        assert (got == ref).mean() > 0.97


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [128, 80])
def test_gated_norm_matches_the_stock_module(n, wdtype, xdtype):
    gen = torch.Generator().manual_seed(n)
    norm = StockNorm(n, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(n, generator=gen))
    norm = norm.to(wdtype)
    x = torch.randn(16, n, generator=gen).to(xdtype)
    z = torch.randn(16, n, generator=gen).to(xdtype)
    so = O.to_np(norm(x, z))
    round_mid = torch.promote_types(wdtype, xdtype) == xdtype
    ref = G.gdn_gated_norm(x, z, norm.weight, 1e-6, O.act_name(xdtype), round_mid)
    if xdtype == torch.float32:
        np.testing.assert_allclose(so, ref, rtol=1e-5, atol=1e-6)
    else:
        ulp = 2.0 ** (-7 if xdtype == torch.bfloat16 else -10)
        assert (np.abs(so - ref) <= ulp * np.abs(ref) + 1e-6).all()
        assert (so == ref).mean() > 0.97


def test_gated_norm_round_mid_matters():
    """With a bf16 weight and bf16 x the product is rounded before the gate; dropping that
    rounding changes the bits (so the flag is pinned, not a no-op)."""
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(64, 128, generator=gen).bfloat16()
    z = torch.randn(64, 128, generator=gen).bfloat16()
    w = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16()
    a = G.gdn_gated_norm(x, z, w, 1e-6, "bf16", True)
    b = G.gdn_gated_norm(x, z, w, 1e-6, "bf16", False)
    assert not np.array_equal(a, b)


# ── host logic (no GPU) ─────────────────────────────────────────────────────────────────

import vaayu_amd.gated_delta_kernels as gdk            # noqa: E402

NO_SEAMS = {"rule": 0, "conv": 0, "norm": 0}


class _Mixer(torch.nn.Module):
    """A mixer exposing the three seams as attributes, the surface the detection reads
    (tests/test_gated_delta_kernels.py:63-72 builds the same kind of stand-in)."""

    def __init__(self, conv=True, norm=None):
        super().__init__()
        self.recurrent_gated_delta_rule = stock_rule
        if conv:
            self.causal_conv1d_update = stock_conv
        self.norm = norm if norm is not None else StockNorm(16)
        self.num_v_heads, self.head_k_dim, self.head_v_dim = 2, 16, 16
        self.conv1d = torch.nn.Conv1d(64, 64, 4, groups=64, bias=False)


def _counts(model):
    return {s: len(m) for s, m in gdk.gated_delta_seams(model).items()}


def test_seams_found_by_surface():
    model = torch.nn.Sequential(_Mixer(), torch.nn.Linear(4, 4), _Mixer(conv=False))
    assert _counts(model) == {"rule": 2, "conv": 1, "norm": 2}


def test_no_seams_on_a_dense_model():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    model = torch.nn.Sequential(torch.nn.Linear(4, 4), LlamaRMSNorm(4))
    assert hasattr(model[1], "variance_epsilon")
    assert _counts(model) == NO_SEAMS


def test_a_norm_without_the_gated_surface_is_not_a_seam():
    mixer = _Mixer()
    mixer.norm = torch.nn.LayerNorm(16)
    assert _counts(mixer) == {"rule": 1, "conv": 1, "norm": 0}


def test_geometry_read_off_the_mixer():
    mixer = _Mixer()
    assert gdk._rule_geometry(mixer) == (2, 16, 16)
    assert gdk._conv_geometry(mixer) == (64, 4)
    assert gdk._rule_geometry(torch.nn.Module()) == (2, 16, 16)
    assert gdk._conv_geometry(torch.nn.Module()) == (64, 4)


def test_nothing_installed_on_cpu():
    mixer = _Mixer()
    before = mixer.recurrent_gated_delta_rule
    assert gdk.install_gated_delta_kernels(mixer, "cpu", torch.float32) == NO_SEAMS
    assert mixer.recurrent_gated_delta_rule is before


def test_nothing_installed_without_the_kernels(monkeypatch):
    monkeypatch.setattr(gdk, "triton", None)
    mixer = _Mixer()
    before = mixer.causal_conv1d_update
    assert gdk.install_gated_delta_kernels(mixer, "cuda", torch.bfloat16) == NO_SEAMS
    assert mixer.causal_conv1d_update is before


def test_kernels_raise_without_the_library(monkeypatch):
    monkeypatch.setattr(gdk, "triton", None)
    with pytest.raises(ImportError):
        gdk.fused_conv_update(torch.zeros(1, 4, 1), torch.zeros(1, 4, 3), torch.zeros(4, 3))


def test_conv_seam_delegates_multi_token_calls_to_stock():
    calls = []

    def stock(*args):
        calls.append(args)
        return "stock"

    seam = gdk._conv_seam(stock)
    assert seam(torch.zeros(1, 8, 2), torch.zeros(1, 8, 4), torch.zeros(8, 4)) == "stock"
    assert len(calls) == 1 and getattr(seam, gdk._MARK) is stock


def test_patched_norm_hands_gateless_calls_to_stock():
    class Norm(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.ones(4))
            self.variance_epsilon = 1e-6

        def forward(self, hidden_states, gate=None):
            return "stock"

    norm = Norm()
    gdk._patch_norm(norm)
    assert norm(torch.zeros(2, 4)) == "stock"
    assert hasattr(norm.forward, gdk._MARK)
