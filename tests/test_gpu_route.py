"""Routing on the GPU (`vaayu_route_topk`) and the one-token decode that runs from router
logits to the expert sum with no host step (`ResidentExperts.decode`), held to the oracle's
restatement of the reference's default routing (softmax -> top-k -> renormalise,
vaayu/moe_patch.py:2329-2334; ties to the lower expert id) and decode budget
(`truncate_top_k`, :170-215), and to the host path's table and kernels: ids equal, weights
within a few fp32 ulps (the exp and the sums run in another order than numpy's), the pair
table and the layer output bit-equal to the host path's."""

import numpy as np
import pytest
import torch

import vaayu_amd.packed_expert_kernels as pk
from vaayu_amd import _lib
from vaayu_amd.device_routing import ResidentExperts, route_topk, router_logits
from vaayu_amd.synth import random_expert
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
W_RTOL = 8e-7 * 8          # a few fp32 ulps of the renormalised weights


@pytest.mark.parametrize("experts,top_k,dtype,tokens", [
    (128, 8, torch.bfloat16, 1), (128, 8, torch.bfloat16, 37), (256, 8, torch.float32, 5),
    (32, 4, torch.float16, 9), (8, 2, torch.bfloat16, 64), (64, 6, torch.float32, 3),
    (1024, 16, torch.bfloat16, 2), (5, 5, torch.float32, 4)])
def test_ids_and_weights_match_the_oracle(experts, top_k, dtype, tokens):
    g = torch.Generator().manual_seed(experts * 31 + top_k)
    logits = (torch.randn(tokens, experts, generator=g) * 2).to(dtype)
    w, ids = route_topk(logits.to(DEV), top_k)
    torch.cuda.synchronize()
    want_w, want_ids = O.route_softmax_topk(logits.float(), top_k)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=W_RTOL, atol=0)


def test_ties_go_to_the_lower_expert_id():
    logits = torch.tensor([[0.5, 2.0, 2.0, -1.0, 0.25, 2.0], [1.0] * 6], dtype=torch.float32)
    w, ids = route_topk(logits.to(DEV), 4)
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [[1, 2, 5, 0], [0, 1, 2, 3]]
    want_w, _ = O.route_softmax_topk(logits, 4)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=W_RTOL)


def test_without_renormalisation_the_weights_are_the_probabilities():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(4, 64, generator=g)
    w, ids = route_topk(logits.to(DEV), 6, renorm=False)
    torch.cuda.synchronize()
    p = torch.softmax(logits.double(), -1)
    want = torch.gather(p, 1, ids.cpu()).float()
    np.testing.assert_allclose(w.cpu().numpy(), want.numpy(), rtol=W_RTOL)
    assert float(w.sum(-1).max()) < 1.0


def test_nan_logits_give_nan_weights_and_valid_ids():
    logits = torch.randn(2, 16)
    logits[1, 3] = float("nan")
    w, ids = route_topk(logits.to(DEV), 4)
    torch.cuda.synchronize()
    assert torch.isfinite(w[0]).all() and torch.isnan(w[1]).all()
    assert ((ids >= 0) & (ids < 16)).all()


def test_rejections_raise():
    with pytest.raises(_lib.KernelError):
        route_topk(torch.randn(1, 32, device=DEV), 17)
    with pytest.raises(_lib.KernelError):
        route_topk(torch.randn(1, 2048, device=DEV), 8)
    with pytest.raises(_lib.KernelError):
        route_topk(torch.randn(1, 4, device=DEV), 5)
    with pytest.raises(ValueError):
        route_topk(torch.randn(1, 32, device=DEV), 4, keep_k=0)
    with pytest.raises(ValueError):
        route_topk(torch.randn(1, 32, device=DEV), 4, top_p=0.0)


def test_output_buffers_are_checked_before_the_launch():
    """Caller-given weights / ids must be contiguous fp32 / int64 [tokens, n] on the logits'
    device: the kernel writes through their pointers. Logits of another dtype are refused."""
    logits = torch.randn(3, 32, device=DEV)
    bad = [dict(weights=torch.empty(3, 2, device=DEV)),                       # too small
           dict(weights=torch.empty(3, 4, device=DEV, dtype=torch.bfloat16)),
           dict(weights=torch.empty(4, 3, device=DEV).t()),                   # not contiguous
           dict(ids=torch.empty(3, 4, device=DEV, dtype=torch.int32)),
           dict(ids=torch.empty(3, 4, dtype=torch.int64))]                    # host memory
    for kw in bad:
        with pytest.raises(ValueError):
            route_topk(logits, 4, **kw)
    with pytest.raises(ValueError):
        route_topk(logits.double(), 4)
    w, ids = torch.empty(3, 4, device=DEV), torch.empty(3, 4, device=DEV, dtype=torch.int64)
    got_w, got_ids = route_topk(logits, 4, weights=w, ids=ids)
    torch.cuda.synchronize()
    assert got_w.data_ptr() == w.data_ptr() and got_ids.data_ptr() == ids.data_ptr()
    want_w, want_ids = route_topk(logits, 4)
    assert torch.equal(w, want_w) and torch.equal(ids, want_ids)


@pytest.mark.parametrize("experts,top_k,keep_k,top_p", [
    (128, 8, 6, None), (128, 8, None, 0.7), (256, 8, 5, 0.6), (64, 6, 6, 0.5),
    (512, 10, 4, None), (128, 8, None, 0.01), (128, 8, 1, None), (32, 4, 8, 0.95)])
def test_decode_budget_matches_the_oracle(experts, top_k, keep_k, top_p):
    g = torch.Generator().manual_seed(experts + top_k + (keep_k or 0))
    logits = torch.randn(48, experts, generator=g) * 1.5
    w, ids = route_topk(logits.to(DEV), top_k, keep_k=keep_k, top_p=top_p)
    torch.cuda.synchronize()
    rw, ridx = O.route_softmax_topk(logits, top_k)
    want_w, want_ids = O.truncate_top_k(rw, ridx, keep_k, top_p)
    rows = np.arange(48)
    if top_p is not None:            # rows whose kept set sits within 1e-5 of the cutoff
        n = want_w.shape[-1]
        ws = rw[:, :n] / rw[:, :n].sum(-1, keepdims=True) if keep_k else rw
        margin = np.abs(np.cumsum(ws, -1) - ws - top_p).min(-1)
        rows = rows[margin > 1e-5]
        assert len(rows) > 40
    assert np.array_equal(ids.cpu().numpy()[rows], want_ids[rows])
    np.testing.assert_allclose(w.cpu().numpy()[rows], want_w[rows], rtol=W_RTOL, atol=1e-7)


def test_the_budget_off_is_the_plain_routing():
    logits = torch.randn(16, 128, generator=torch.Generator().manual_seed(4)).to(DEV)
    a = route_topk(logits, 8)
    b = route_topk(logits, 8, keep_k=8)
    c = route_topk(logits, 8, keep_k=12)
    torch.cuda.synchronize()
    for other in (b, c):
        assert torch.equal(a[0], other[0]) and torch.equal(a[1], other[1])


@pytest.mark.parametrize("tokens,hidden,experts,dtype,out_dtype", [
    (1, 2048, 128, torch.bfloat16, None), (3, 7168, 256, torch.bfloat16, torch.float32),
    (2, 1024, 32, torch.float16, None), (5, 4096, 8, torch.bfloat16, None)])
def test_router_logits_are_the_correctly_rounded_product(tokens, hidden, experts, dtype,
                                                         out_dtype):
    """Against the fp64 product rounded once: within one unit in the last place of a 16-bit
    output dtype (fp32 accumulation order) and mostly equal, within 2^-20 relative for fp32
    outputs, and close to torch's own F.linear."""
    g = torch.Generator().manual_seed(hidden + experts)
    x = torch.randn(tokens, hidden, generator=g).to(dtype)
    w = (torch.randn(experts, hidden, generator=g) * 0.02).to(dtype)
    got = router_logits(x.to(DEV), w.to(DEV), out_dtype=out_dtype)
    torch.cuda.synchronize()
    exact = (x.double() @ w.double().T).numpy()
    od = out_dtype or dtype
    ref = O.round_to(exact, O.act_name(od))
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -20}[od]
    gv = O.to_np(got)
    assert got.dtype == od
    assert (np.abs(gv - ref) <= ulp * np.abs(ref) + 1e-6).all()
    if od != torch.float32:                  # fp32 outputs carry the fp32 sum's own error
        assert (gv == ref).mean() > 0.9
    lib = torch.nn.functional.linear(x.to(DEV), w.to(DEV)).to(od)
    assert O.rel_l2(gv, O.to_np(lib)) < 1e-2


def test_router_logits_reject_bad_shapes():
    with pytest.raises(ValueError):
        router_logits(torch.zeros(1, 64, device=DEV, dtype=torch.bfloat16),
                      torch.zeros(8, 32, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(_lib.KernelError):
        router_logits(torch.zeros(1, 60, device=DEV, dtype=torch.bfloat16),
                      torch.zeros(8, 60, device=DEV, dtype=torch.bfloat16))


# ── the resident-expert decode ──────────────────────────────────────────────────────────

H, I, E, K = 1024, 512, 16, 4


@pytest.fixture(scope="module")
def layer():
    gen = torch.Generator(device=DEV).manual_seed(11)
    blobs = [random_expert(H, I, 4, 128, generator=gen, device=DEV, std=0.05,
                           scale_dtype=torch.float16) for _ in range(E)]
    return blobs, ResidentExperts(blobs)


def _host_decode(x, blobs, weights, ids):
    """The reference-shaped host path over the same routing: pairs sorted by expert id."""
    e = ids[0].tolist()
    pairs = [(blobs[e[s]], s) for s in sorted(range(len(e)), key=e.__getitem__)]
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    pk._launch(x, pairs, weights, out)
    return pairs, out


def test_the_device_table_is_the_host_table(layer):
    blobs, rx = layer
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    logits = torch.randn(1, E, generator=g).to(DEV)
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    bufs = rx.buffers(K, x.dtype)
    w, ids = rx.decode(x, logits, K, out, bufs=bufs)
    torch.cuda.synchronize()
    pairs, host_out = _host_decode(x, blobs, w.clone(), ids.cpu())
    torch.cuda.synchronize()
    assert bufs.table.cpu().tolist() == pk._table_values(pairs)
    assert torch.equal(out, host_out)
    want_w, want_ids = O.route_softmax_topk(logits.cpu(), K)
    assert np.array_equal(ids.cpu().numpy(), want_ids)


@pytest.mark.parametrize("keep_k,top_p", [(2, None), (None, 0.3), (3, 0.5), (None, 0.01)])
def test_the_budgeted_table_is_the_host_table(layer, keep_k, top_p):
    """With a budget the table has re-pointed (duplicate) experts: it must still be the
    host path's stable (expert id, slot) order, and the layer the host path's bits."""
    blobs, rx = layer
    g = torch.Generator().manual_seed(21 + (keep_k or 0))
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    logits = torch.randn(1, E, generator=g).to(DEV)
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    bufs = rx.buffers(K, x.dtype, keep_k)
    w, ids = rx.decode(x, logits, K, out, keep_k=keep_k, top_p=top_p, bufs=bufs)
    torch.cuda.synchronize()
    pairs, host_out = _host_decode(x, blobs, w.clone(), ids.cpu())
    torch.cuda.synchronize()
    assert bufs.table.cpu().tolist() == pk._table_values(pairs)
    assert torch.equal(out, host_out)
    rw, ridx = O.route_softmax_topk(logits.cpu(), K)
    want_w, want_ids = O.truncate_top_k(rw, ridx, keep_k, top_p)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=W_RTOL, atol=1e-7)


def test_the_layer_matches_the_stock_loop(layer):
    blobs, rx = layer
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    logits = torch.randn(1, E, generator=g).to(torch.bfloat16).to(DEV)
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    w, ids = rx.decode(x, logits, K, out)
    torch.cuda.synchronize()
    e = ids[0].cpu().tolist()
    pairs = [({"flat": {n: t.cpu() for n, t in blobs[e[s]]["flat"].items()},
               "geom": blobs[0]["geom"]}, s) for s in sorted(range(K), key=e.__getitem__)]
    ref = O.stock_decode(x.cpu(), pairs, w.cpu())
    assert O.rel_l2(O.to_np(out), ref) <= 5e-3
    assert np.abs(O.to_np(out) - ref).max() <= 2e-2


def test_one_graph_from_logits_to_the_sum_replays_exactly(layer):
    blobs, rx = layer
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    # the router's weight stored transposed ([H, E], contiguous): a plain 2-D product
    w_router_t = (torch.randn(H, E, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    bufs = rx.buffers(K, x.dtype)
    logits = torch.empty(1, E, dtype=torch.bfloat16, device=DEV)

    def layer_step():
        torch.matmul(x, w_router_t, out=logits)
        rx.decode(x, logits, K, out, bufs=bufs)

    layer_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer_step()
    for rep in range(3):
        x.copy_((torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got_out, got_ids, got_w = out.clone(), bufs.ids.clone(), bufs.weights.clone()
        layer_step()                     # eager, same inputs
        torch.cuda.synchronize()
        assert torch.equal(got_ids, bufs.ids), rep
        assert torch.equal(got_w, bufs.weights), rep
        assert torch.equal(got_out, out), rep


def test_graph_with_the_router_product_on_the_gpu(layer):
    """router_logits -> routing -> both kernels in one graph, replays equal to eager."""
    blobs, rx = layer
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    w_router = (torch.randn(E, H, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    out = torch.empty(1, H, dtype=torch.float32, device=DEV)
    bufs = rx.buffers(K, x.dtype)
    logits = torch.empty(1, E, dtype=torch.bfloat16, device=DEV)

    def layer_step():
        router_logits(x, w_router, out=logits)
        rx.decode(x, logits, K, out, bufs=bufs)

    layer_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer_step()
    for rep in range(3):
        x.copy_((torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got_out, got_ids = out.clone(), bufs.ids.clone()
        layer_step()
        torch.cuda.synchronize()
        assert torch.equal(got_ids, bufs.ids) and torch.equal(got_out, out), rep


def test_resident_experts_reject_mixed_blobs(layer):
    blobs, _rx = layer
    gen = torch.Generator(device=DEV).manual_seed(12)
    other = random_expert(H, I, 4, 64, generator=gen, device=DEV, std=0.05,
                          scale_dtype=torch.float16)
    with pytest.raises(ValueError):
        ResidentExperts(list(blobs[:3]) + [other])
    rx = ResidentExperts(blobs)
    x = torch.zeros(1, H, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        rx.decode(x, torch.zeros(1, E + 1, device=DEV), K,
                  torch.empty(1, H, dtype=torch.float32, device=DEV))
