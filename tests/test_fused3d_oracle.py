"""The fused-3D (gpt-oss MXFP4) expert oracle pinned on the CPU, and the host checks of
vaayu_amd/fused3d.py that need no GPU.

Pin: `oracle.fused3d.fused3d_experts(..., exact=True)` must equal transformers' dense
`GptOssExperts.forward` run in float64 on the dequantized weights -- an independent
implementation of the same expert math (interleaved gate/up, biases, the clipped SwiGLU with
the (up + 1) term, routing weights, the sum over a token's slots). The MXFP4 dequant itself
is pinned in tests/test_oracle.py."""
import numpy as np
import pytest
import torch

from oracle import fused3d as F3
from oracle import oracle as O

M = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")


def random_layer(E, H, I, seed=0, scale_spread=2):
    g = torch.Generator().manual_seed(seed)
    def blocks(r, c):
        return torch.randint(0, 256, (E, r, c // 32, 16), generator=g, dtype=torch.uint8)
    def scales(r, c):
        return torch.randint(124 - scale_spread, 124 + scale_spread + 1, (E, r, c // 32),
                             generator=g).to(torch.uint8)
    return dict(gu_blocks=blocks(2 * I, H), gu_scales=scales(2 * I, H),
                gu_bias=torch.randn(E, 2 * I, generator=g) * 0.1,
                dn_blocks=blocks(H, I), dn_scales=scales(H, I),
                dn_bias=torch.randn(E, H, generator=g) * 0.1)


def routing(T, E, k, seed=1):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    top, idx = torch.topk(logits, k, dim=-1)
    return idx, torch.softmax(top, dim=-1)


def _dense(layer, E, H, I):
    """transformers' eager `GptOssExperts.forward` (the undecorated function: the experts
    interface wrapper would dispatch on a config attribute) in float64."""
    from transformers import GptOssConfig
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E,
                       num_hidden_layers=1, num_attention_heads=2, num_key_value_heads=1,
                       head_dim=32, vocab_size=32)
    ex = M.GptOssExperts(cfg).double()
    eager = getattr(M.GptOssExperts.forward, "__wrapped__", M.GptOssExperts.forward)
    wgu = F3.dequant_fused3d(layer["gu_blocks"], layer["gu_scales"])      # [E, 2I, H]
    wdn = F3.dequant_fused3d(layer["dn_blocks"], layer["dn_scales"])      # [E, H, I]
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.from_numpy(wgu).transpose(1, 2))
        ex.down_proj.copy_(torch.from_numpy(wdn).transpose(1, 2))
        ex.gate_up_proj_bias.copy_(layer["gu_bias"].double())
        ex.down_proj_bias.copy_(layer["dn_bias"].double())
    def run(x, router_indices, routing_weights):
        with torch.no_grad():
            return eager(ex, x, router_indices=router_indices, routing_weights=routing_weights)
    return run


@pytest.mark.parametrize("E,H,I,k,T", [(4, 64, 64, 2, 5), (6, 96, 160, 3, 7)])
def test_exact_oracle_is_transformers_dense_gpt_oss_experts(E, H, I, k, T):
    layer = random_layer(E, H, I)
    idx, w = routing(T, E, k)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(2)).bfloat16()
    want = _dense(layer, E, H, I)(x.double(), router_indices=idx, routing_weights=w.double())
    got = F3.fused3d_experts(x, idx, w, **layer, exact=True)
    assert O.rel_l2(got, want.numpy()) < 1e-12


def test_the_clip_is_exercised_and_matches():
    """Scales large enough that many gate / up values pass +-7: the clipped branches agree."""
    E, H, I = 3, 64, 64
    layer = random_layer(E, H, I, seed=4, scale_spread=0)
    layer["gu_scales"] = torch.full_like(layer["gu_scales"], 128)        # x2: large pre-acts
    idx, w = routing(6, E, 2, seed=5)
    x = (torch.randn(6, H, generator=torch.Generator().manual_seed(6)) * 2).bfloat16()
    wgu = F3.dequant_fused3d(layer["gu_blocks"], layer["gu_scales"])
    pre = np.einsum("eoh,th->teo", wgu, x.double().numpy())
    assert (pre[..., 0::2] > 7).mean() > 0.05 and (np.abs(pre[..., 1::2]) > 7).mean() > 0.05
    want = _dense(layer, E, H, I)(x.double(), router_indices=idx, routing_weights=w.double())
    got = F3.fused3d_experts(x, idx, w, **layer, exact=True)
    assert O.rel_l2(got, want.numpy()) < 1e-12


def test_swiglu_constants_change_the_result():
    """alpha and limit are live inputs (a dropped constant fails the dense comparison)."""
    E, H, I = 2, 64, 64
    layer = random_layer(E, H, I, seed=7)
    idx, w = routing(3, E, 1, seed=8)
    x = torch.randn(3, H, generator=torch.Generator().manual_seed(9)).bfloat16() * 4
    a = F3.fused3d_experts(x, idx, w, **layer, exact=True)
    b = F3.fused3d_experts(x, idx, w, **layer, exact=True, alpha=1.0)
    c = F3.fused3d_experts(x, idx, w, **layer, exact=True, limit=1.0)
    assert not np.allclose(a, b) and not np.allclose(a, c)


def test_rounded_oracle_is_close_to_exact():
    E, H, I = 4, 64, 96
    layer = random_layer(E, H, I, seed=10)
    idx, w = routing(8, E, 2, seed=11)
    x = torch.randn(8, H, generator=torch.Generator().manual_seed(12)).bfloat16()
    a = F3.fused3d_experts(x, idx, w, **layer, exact=True)
    b = F3.fused3d_experts(x, idx, w, **layer)
    assert O.rel_l2(b, a) < 1e-2
    assert np.array_equal(b, O.round_to(b, "bf16"))                      # bf16 values


def test_host_module_validates_shapes():
    from vaayu_amd.fused3d import Fused3DExperts
    layer = random_layer(2, 64, 64)
    args = [layer[k] for k in ("gu_blocks", "gu_scales", "gu_bias", "dn_blocks", "dn_scales",
                               "dn_bias")]
    Fused3DExperts(*args)                                                 # fine on the CPU
    bad = list(args)
    bad[4] = bad[4][:, :, :1]
    with pytest.raises(ValueError):
        Fused3DExperts(*bad)
    bad = list(args)
    bad[0] = bad[0].to(torch.int16)
    with pytest.raises(ValueError):
        Fused3DExperts(*bad)
