"""The per-layer decode graph (vaayu/packed_expert_kernels.py:483-654 semantics).

Each graph is replayed several times with eager work and synchronisations in between, and
every replay is checked against the eager result."""
import collections

import pytest
import torch
import torch.nn.functional as F

import vaayu_amd.packed_expert_kernels as pk
from tests.helpers import decode_case, gpu_blobs

pytestmark = pytest.mark.gpu

QWEN = (2048, 512, 4, 32, 10)


def fresh_graphs(monkeypatch):
    for name, fresh in (("_GRAPHS", {}), ("_GRAPH_REFUSED", {}), ("_GRAPH_WARNED", set()),
                        ("GRAPH_STATS", collections.Counter())):
        monkeypatch.setattr(pk, name, fresh)


def _eager(x, pairs, w, shared, tail):
    out = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    pk._launch(x, pairs, w, out)
    if not tail:
        return out
    result = out.to(x.dtype)
    return result + shared.to(result.dtype) if shared is not None else result


def _shared_out(hid, seed=5):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(1, hid, generator=g, device="cuda") * 0.1).to(torch.bfloat16)


@pytest.mark.parametrize("geom", [QWEN, (2048, 768, 4, 128, 8), (1024, 512, 8, 64, 4)],
                         ids=["qwen3next", "qwen3-30b", "int8"])
@pytest.mark.parametrize("tail,shared", [(False, False), (True, False), (True, True)],
                         ids=["sum", "tail", "tail+shared"])
def test_the_graph_gives_the_eager_bits(monkeypatch, geom, tail, shared):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*geom)
    sh = _shared_out(geom[0]) if shared else None
    want = _eager(x, pairs, w, sh, tail)
    first = pk.packed_experts_decode_graphed(0, x, pairs, w, sh, F.silu, tail)
    assert torch.equal(first, want)
    for _ in range(3):
        junk = torch.randn(1000, device="cuda").sum()          # eager work between replays
        torch.cuda.synchronize()
        again = pk.packed_experts_decode_graphed(0, x, pairs, w, sh, F.silu, tail)
        torch.cuda.synchronize()
        assert torch.equal(again, want)
        del junk
    assert (pk.GRAPH_STATS["captures"], pk.GRAPH_STATS["replays"]) == (1, 3)


def test_a_rewritten_table_computes_the_new_experts(monkeypatch):
    fresh_graphs(monkeypatch)
    hid, inter, bits, gs, k = QWEN
    blobs = gpu_blobs(hid, inter, bits, gs, 2 * k)
    x, _pairs, w, _c = decode_case(*QWEN)
    a = [(blobs[i], i) for i in range(k)]
    b = [(blobs[k + i], i) for i in range(k)]
    pk.packed_experts_decode_graphed(0, x, a, w, None, F.silu, False)
    for pairs in (b, a, b):
        got = pk.packed_experts_decode_graphed(0, x, pairs, w, None, F.silu, False)
        torch.cuda.synchronize()
        assert torch.equal(got, _eager(x, pairs, w, None, False))
    assert pk.GRAPH_STATS["replays"] == 3


def test_a_new_input_tensor_recaptures(monkeypatch):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*QWEN)
    pk.packed_experts_decode_graphed(0, x, pairs, w, None, F.silu, False)
    x2 = x * 2
    got = pk.packed_experts_decode_graphed(0, x2, pairs, w, None, F.silu, False)
    assert pk.GRAPH_STATS["captures"] == 2
    assert torch.equal(got, _eager(x2, pairs, w, None, False))


def test_a_replay_that_disagrees_refuses_the_layer(monkeypatch, capsys):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*QWEN)
    assert pk._checked(x, pairs, w, F.silu)
    want = _eager(x, pairs, w, None, False)
    real = pk._launch
    monkeypatch.setattr(pk, "_launch", lambda x, p, w, out: (real(x, p, w, out), out.add_(1.0)))
    got = pk.packed_experts_decode_graphed(0, x, pairs, w, None, F.silu, False)
    assert torch.equal(got, want + 1.0)
    assert "disagrees bitwise" in pk._GRAPH_REFUSED.get(0, "")
    assert "WARNING" in capsys.readouterr().out
    assert pk.packed_experts_decode_graphed(0, x, pairs, w, None, F.silu, False) is None


def test_a_call_the_graph_cannot_take_is_left_to_the_caller(monkeypatch):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*QWEN)
    mixed = [({"dense": {}}, pairs[0][1])] + pairs[1:]
    assert pk.packed_experts_decode_graphed(0, x, mixed, w, None, F.silu, False) is None
    assert pk.GRAPH_STATS["captures"] == 0


def test_the_capture_allocates_only_its_static_buffers(monkeypatch):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*QWEN)
    sh = _shared_out(QWEN[0])
    for _ in range(len(pk._TABLES._slots)):
        _eager(x, pairs, w, sh, True)
    assert pk._checked(x, pairs, w, F.silu)
    pk.packed_experts_decode_graphed(99, x * 3, pairs, w, sh, F.silu, True)
    import gc
    gc.collect()
    torch.cuda.synchronize()
    m0 = torch.cuda.memory_allocated()
    pk.packed_experts_decode_graphed(0, x, pairs, w, sh, F.silu, True)
    torch.cuda.synchronize()
    g = pk._GRAPHS[0]
    static = sum(-(-t.numel() * t.element_size() // 512) * 512
                 for t in (g.tbl, g.h, g.out, g.tmp, g.result))
    assert torch.cuda.memory_allocated() - m0 == static
    for _ in range(20):
        pk.packed_experts_decode_graphed(0, x, pairs, w, sh, F.silu, True)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() - m0 == static
    assert pk.GRAPH_STATS["replays"] == 20


def test_an_input_the_graph_cannot_take_warns_once(monkeypatch, capsys):
    fresh_graphs(monkeypatch)
    x, pairs, w, _c = decode_case(*QWEN)
    w_strided = torch.cat([w, w], dim=1)[:, ::2]
    for _ in range(3):
        assert pk.packed_experts_decode_graphed(0, x, pairs, w_strided, None, F.silu, False) is None
    out = capsys.readouterr().out
    assert out.count("WARNING") == 1 and "not used" in out
