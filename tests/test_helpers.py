"""The host helpers of the packed-expert path (vaayu_amd/moe_patch.py) on the CPU, each
against the reference's known answers or the oracle:

  accumulate_expert_outputs  the reference's order fixture {1e8, -1e8, 1}
                             (tests/test_expert_accumulation_order.py:24-92)
  _shared_expert_output      ungated (DeepSeek) and sigmoid-gated (Qwen2 / Qwen3-Next)
                             (vaayu/moe_patch.py:554-580)
  dequantize_packed_weight   bit-equal to the whole-blob dequant's role views and to the
                             oracle (tests/test_packed_expert_dequant.py:368-381)
  route_experts              the softmax-top-k fallback against the oracle, and the
                             model's own `route_tokens_to_experts` in either return order
                             (vaayu/moe_patch.py:130-167)
  _routing_to_host           the routed ids ascending, both branches
                             (vaayu/moe_patch.py:232-243)
"""
import itertools

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import oracle as O
from vaayu_amd.moe_patch import (_routing_to_host, _shared_expert_output,
                                 accumulate_expert_outputs, build_expert_blob,
                                 dequantize_expert_blob, dequantize_packed_weight,
                                 route_experts)
from vaayu_amd.synth import quantize_pack


# ── accumulate_expert_outputs ────────────────────────────────────────────────────────────

def _order_fixture():
    """fp32 spacing at 1e8 is 8: (1e8 + 1) + -1e8 = 0 but (1e8 + -1e8) + 1 = 1. Expert ids
    out of arrival order."""
    idx = torch.tensor([0])
    return [(7, idx, torch.tensor([[1e8]])), (2, idx, torch.tensor([[-1e8]])),
            (5, idx, torch.tensor([[1.0]]))]


def _accumulate(contribs):
    out = torch.zeros(1, 1)
    accumulate_expert_outputs(out, contribs)
    return out


def test_the_order_fixture_is_order_sensitive():
    c = _order_fixture()
    forward, backward = torch.zeros(1, 1), torch.zeros(1, 1)
    for _e, i, v in c:
        forward.index_add_(0, i, v)
    for _e, i, v in reversed(c):
        backward.index_add_(0, i, v)
    assert not torch.equal(forward, backward)


def test_every_arrival_order_gives_the_same_bits():
    results = [_accumulate(list(p)) for p in itertools.permutations(_order_fixture())]
    assert all(torch.equal(results[0], r) for r in results[1:])


def test_the_sum_runs_in_expert_id_order():
    """Ids 2, 5, 7: (-1e8 + 1) + 1e8 = 0 in fp32 (the 1 is lost at 1e8's spacing)."""
    assert _accumulate(list(reversed(_order_fixture()))).item() == 0.0
    want = O.accumulate(np.zeros((1, 1), np.float32),
                        [(e, i.numpy(), v.numpy()) for e, i, v in _order_fixture()])
    assert torch.equal(_accumulate(_order_fixture()), torch.from_numpy(want))


def test_contributions_are_cast_to_the_accumulator_dtype():
    out = torch.zeros(1, 4)
    accumulate_expert_outputs(out, [(0, torch.tensor([0]), torch.full((1, 4), 0.5,
                                                                       dtype=torch.float16))])
    assert out.dtype == torch.float32 and torch.equal(out, torch.full((1, 4), 0.5))


def test_overlapping_token_rows_all_land():
    out = torch.zeros(3, 2)
    accumulate_expert_outputs(out, [(1, torch.tensor([0, 2]), torch.ones(2, 2)),
                                    (0, torch.tensor([0, 1]), torch.ones(2, 2))])
    assert torch.equal(out, torch.tensor([[2.0, 2.0], [1.0, 1.0], [1.0, 1.0]]))


def test_random_contributions_match_the_oracle():
    g = torch.Generator().manual_seed(0)
    contribs = [(int(e), torch.randperm(16, generator=g)[:5], torch.randn(5, 8, generator=g)
                 * 10 ** float(torch.randint(-3, 4, (1,), generator=g)))
                for e in torch.randperm(40, generator=g)[:12]]
    got = torch.zeros(16, 8)
    accumulate_expert_outputs(got, contribs)
    want = O.accumulate(np.zeros((16, 8), np.float32),
                        [(e, i.numpy(), v.numpy()) for e, i, v in contribs])
    assert torch.equal(got, torch.from_numpy(want))


# ── _shared_expert_output ────────────────────────────────────────────────────────────────

class _Block(nn.Module):
    def __init__(self, children):
        super().__init__()
        for name, mod in children:
            self.add_module(name, mod)


def _mlp(hidden, seed):
    torch.manual_seed(seed)
    return nn.Sequential(nn.Linear(hidden, 2 * hidden, bias=False), nn.SiLU(),
                         nn.Linear(2 * hidden, hidden, bias=False)).to(torch.bfloat16)


def test_an_ungated_shared_expert_is_added_as_is():
    shared = _mlp(32, 1)
    block = _Block([("gate", nn.Linear(32, 8)), ("shared_experts", shared)])
    x = torch.randn(5, 32).bfloat16()
    assert torch.equal(_shared_expert_output(block, x), shared(x))


def test_a_gated_shared_expert_is_scaled_by_its_sigmoid_gate():
    shared = _mlp(32, 2)
    torch.manual_seed(3)
    gate = nn.Linear(32, 1, bias=False).to(torch.bfloat16)
    x = torch.randn(5, 32).bfloat16()
    want = torch.sigmoid(gate(x)) * shared(x)
    for order in (("shared_expert", "shared_expert_gate"), ("shared_expert_gate", "shared_expert")):
        block = _Block([(n, shared if n == "shared_expert" else gate) for n in order])
        got = _shared_expert_output(block, x)
        assert torch.equal(got, want), f"children in order {order}"
    assert not torch.equal(want, shared(x)), "premise: the gate changes the output"


def test_no_shared_expert_gives_none():
    block = _Block([("gate", nn.Linear(32, 8)), ("experts", nn.ModuleList())])
    assert _shared_expert_output(block, torch.randn(2, 32)) is None


# ── dequantize_packed_weight ─────────────────────────────────────────────────────────────

def _packed_roles(hidden, inter, bits, gs, scale_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    by_role = {}
    for role, shape in (("gate", (inter, hidden)), ("down", (hidden, inter)),
                        ("up", (inter, hidden))):
        w = (torch.randn(shape, generator=g) * 0.05).bfloat16()
        packed, scale = quantize_pack(w, bits, gs, scale_dtype)
        by_role[role] = {"weight_packed": packed, "weight_scale": scale,
                         "weight_shape": torch.tensor(list(shape))}
    return by_role


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64), (2, 32)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.bfloat16])
def test_per_role_dequant_equals_the_blob_dequant_and_the_oracle(bits, gs, dtype, scale_dtype):
    by_role = _packed_roles(256, 128, bits, gs, scale_dtype, seed=bits * gs)
    blob = build_expert_blob(by_role)
    via_blob = dequantize_expert_blob(blob, dtype)
    flat = O.dequant_flat(blob["flat"]["packed"], blob["flat"]["scale"], bits, gs, dtype)
    at = 0
    for role, comps in by_role.items():
        got = dequantize_packed_weight(comps, dtype)
        rows, cols = comps["weight_shape"].tolist()
        assert got.dtype == dtype and got.shape == (rows, cols)
        assert torch.equal(got, via_blob[role]), role
        assert np.array_equal(got.float().numpy(), flat[at:at + rows * cols].reshape(rows, cols))
        at += rows * cols


def test_per_role_dequant_refuses_asymmetric_and_underivable_widths():
    comps = _packed_roles(64, 64, 4, 32, torch.float16, 0)["gate"]
    with pytest.raises(NotImplementedError):
        dequantize_packed_weight(dict(comps, weight_zero_point=torch.zeros(1)), torch.bfloat16)
    with pytest.raises(ValueError):
        dequantize_packed_weight(dict(comps, weight_shape=torch.tensor([64, 60])),
                                 torch.bfloat16)


# ── routing ──────────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("shape,top_k", [((7, 32), 4), ((2, 3, 128), 8), ((1, 8), 2)])
def test_the_fallback_is_softmax_top_k_renormalised(shape, top_k):
    logits = torch.randn(shape, generator=torch.Generator().manual_seed(top_k))   # no ties
    w, idx = route_experts(object(), logits, top_k)
    assert w.dtype == torch.float32 and idx.dtype == torch.int64
    assert w.shape == idx.shape == (*shape[:-1], top_k)
    ow, oi = O.route_softmax_topk(logits.reshape(-1, shape[-1]), top_k)
    assert np.array_equal(idx.reshape(-1, top_k).numpy(), oi)
    np.testing.assert_allclose(w.reshape(-1, top_k).numpy(), ow, rtol=2e-7, atol=0)
    np.testing.assert_allclose(w.sum(-1).numpy(), 1.0, rtol=1e-6)


@pytest.mark.parametrize("indices_first", [True, False])
def test_the_models_own_router_is_used_in_either_return_order(indices_first):
    """DeepSeek / GLM return (indices, weights), dbrx (weights, indices): told apart by
    dtype; leading dims are flattened for the call and restored."""
    seen = []

    class Router:
        def route_tokens_to_experts(self, logits):
            seen.append(tuple(logits.shape))
            w, idx = torch.topk(torch.sigmoid(logits), 2, dim=-1)
            return (idx, w) if indices_first else (w, idx)

    logits = torch.randn(2, 3, 16, generator=torch.Generator().manual_seed(1))
    w, idx = route_experts(Router(), logits, 2)
    assert seen == [(6, 16)]
    assert w.shape == idx.shape == (2, 3, 2) and not idx.is_floating_point()
    want_w, want_i = torch.topk(torch.sigmoid(logits), 2, dim=-1)
    assert torch.equal(w, want_w) and torch.equal(idx, want_i)


def test_routing_to_host_one_token_and_many():
    one = torch.tensor([[9, 3, 3, 1]])
    cpu, ids = _routing_to_host(one)
    assert torch.equal(cpu, one) and ids == [1, 3, 9]
    many = torch.randint(0, 64, (40, 8), generator=torch.Generator().manual_seed(2))
    cpu, ids = _routing_to_host(many)
    assert torch.equal(cpu, many) and ids == sorted(set(many.reshape(-1).tolist()))
    assert ids == np.unique(many.numpy()).tolist()
