"""How far the prefill GEMMs' fp32 MFMA accumulation lands from the exact sum, measured
through `vaayu_probe_mfma_sum` (the prefill K loop's MFMA order on given bf16 operands)
against exact float64 sums on the host.

Data of the benchmark's kind: int4 g128 weights of N(0, 0.02) rounded to bf16 against
N(0, 1) activations (K 7168, the DeepSeek-V3 gate/up loop) and against SwiGLU
intermediates (K 2048 and 14336, the DeepSeek-V3 and Mixtral down loops). With Q the sum
of squares of the partial sums after each 32-product MFMA, the error v - S is unbiased
with rms about 0.7 * 2^-24 sqrt(Q), and it rounds to another bf16 than S in a few outputs
in 10,000; the figures are printed as one JSON line per K."""
import json

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def int4_weights(rows, k, gen):
    w = torch.randn(rows, k // 128, 128, generator=gen) * 0.02
    s = (w.abs().amax(-1, keepdim=True) / 7).half().float().bfloat16().float()
    c = torch.clamp(torch.round(w / s), -8, 7)
    return (c * s).reshape(rows, k).bfloat16()


def swiglu_rows(rows, k, gen):
    g = (torch.randn(rows, k, generator=gen) * 1.69).bfloat16().float()
    u = (torch.randn(rows, k, generator=gen) * 1.69).bfloat16().float()
    return (torch.nn.functional.silu(g).bfloat16().float() * u).bfloat16()


def mfma_order(k):
    """Element indices in the order the K loop's MFMAs take them: per 128-step, MFMA i
    sums elements 32q + 8i + j over quarters q and j < 8."""
    idx = [s + 32 * q + 8 * i + j for s in range(0, k, 128) for i in range(4)
           for q in range(4) for j in range(8)]
    return np.asarray(idx)


@pytest.mark.parametrize("what,k", [("gate/up", 7168), ("down", 2048), ("down", 14336)])
def test_accumulation_error_is_small_and_unbiased(what, k):
    from vaayu_amd import _lib
    lib = _lib.load()
    gen = torch.Generator().manual_seed(k)
    rows, cols = 64, 256
    a = torch.randn(rows, k, generator=gen).bfloat16() if what == "gate/up" \
        else swiglu_rows(rows, k, gen)
    b = int4_weights(cols, k, gen)
    da, db = a.cuda(), b.cuda()
    d = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    print(f"mfma sum probe {what} K={k}", flush=True)
    rc = lib.vaayu_probe_mfma_sum(da.data_ptr(), db.data_ptr(), d.data_ptr(), k, rows // 16,
                                  cols // 16, _lib.stream_ptr(da.device))
    _lib.check(rc, "vaayu_probe_mfma_sum")
    v = d.cpu().numpy().astype(np.float64)
    order = mfma_order(k)
    A = a.float().numpy().astype(np.float64)[:, order]
    B = b.float().numpy().astype(np.float64)[:, order]
    S = A @ B.T
    run = np.zeros_like(S)
    Q = np.zeros_like(S)
    for k0 in range(0, k, 32):
        run += A[:, k0:k0 + 32] @ B[:, k0:k0 + 32].T
        Q += run ** 2
    z = (v - S) / (U * np.sqrt(Q))
    flips = O.round_to(v.astype(np.float32), "bf16") != O.round_to(S, "bf16")
    rep = {"what": what, "K": k, "outputs": int(S.size), "mean_z": float(z.mean()),
           "rms_z": float(np.sqrt((z ** 2).mean())), "max_abs_z": float(np.abs(z).max()),
           "bf16_flips": int(flips.sum()), "flip_rate": float(flips.mean())}
    print("MFMA_ERROR " + json.dumps(rep), flush=True)
    assert abs(rep["mean_z"]) < 0.05                  # unbiased (the mean's own spread ~0.006)
    assert 0.4 < rep["rms_z"] < 1.2
    assert rep["max_abs_z"] < 6.0
    assert rep["flip_rate"] < 2e-3


def test_bad_calls_are_rejected():
    from vaayu_amd import _lib
    lib = _lib.load()
    t = torch.zeros(16, 256, dtype=torch.bfloat16, device="cuda")
    d = torch.zeros(16, 16, device="cuda")
    st = _lib.stream_ptr(t.device)
    assert lib.vaayu_probe_mfma_sum(t.data_ptr(), t.data_ptr(), d.data_ptr(), 200, 1, 1, st) == -2
    assert lib.vaayu_probe_mfma_sum(t.data_ptr(), t.data_ptr(), d.data_ptr(), 256, 0, 1, st) == -2
    assert lib.vaayu_probe_mfma_sum(t.data_ptr() + 2, t.data_ptr(), d.data_ptr(), 256, 1, 1,
                                    st) == -2
    assert lib.vaayu_probe_mfma_sum(None, t.data_ptr(), d.data_ptr(), 256, 1, 1, st) == -1
