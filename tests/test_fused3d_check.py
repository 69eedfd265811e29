"""The fused-3D load-time check's host logic (vaayu_amd/fused3d.py: check_routed_reads,
routed_reads_verdict), on stand-in modules run by torch on the CPU: an honest one that
reads only the routed experts' rows, one that reads every row, one that raises, and a
geometry whose calls route every expert. The reference's check is
vaayu/routed_fused3d.py:241-345; the kernels themselves are held to it on the GPU
(tests/test_gpu_fused3d.py)."""
import torch

from vaayu_amd import fused3d as F


class StandIn:
    """A module with the surface the check uses: E, H, I, alpha, limit, device,
    tensors(), like(), forward()."""

    def __init__(self, E=8, H=16, I=32, bias=None, scales=None, leak=False, boom=False):
        g = torch.Generator().manual_seed(5)
        self.E, self.H, self.I = E, H, I
        self.alpha, self.limit, self.device = 1.702, 7.0, torch.device("cpu")
        self.bias = bias if bias is not None else torch.randn(E, H, generator=g)
        self.scales = scales if scales is not None else torch.full((E, 4), 120, dtype=torch.uint8)
        self.leak, self.boom = leak, boom
        self.calls = 0

    def tensors(self):
        return {"bias": self.bias, "scales": self.scales}

    def like(self, tensors):
        return StandIn(self.E, self.H, self.I, tensors["bias"], tensors["scales"],
                       self.leak, self.boom)

    def forward(self, x, ids, w):
        self.calls += 1
        if self.boom:
            raise RuntimeError("kernel refused the call")
        out = x.float().clone()
        for t in range(ids.shape[0]):
            for s in range(ids.shape[1]):
                e = int(ids[t, s])
                out[t] += w[t, s] * self.bias[e] * self.scales[e, 0].float()
        if self.leak:
            out += self.bias.sum(0)               # every expert's row, routed or not
        return out.to(x.dtype)


def test_a_module_that_reads_only_routed_rows_passes():
    ok, why = F.check_routed_reads(StandIn(), top_k=2)
    assert ok, why
    assert "M=1 and M=2" in why                   # max(2, 8 // (2 * 2))


def test_a_module_that_reads_every_row_fails_at_one_token():
    ok, why = F.check_routed_reads(StandIn(leak=True), top_k=2)
    assert not ok
    assert why.startswith("non-routed expert rows change the output at M=1")


def test_the_multi_token_call_has_e_over_two_k_tokens():
    m = StandIn(E=64)
    ok, why = F.check_routed_reads(m, top_k=4)
    assert ok and "M=8" in why                    # 64 // (2 * 4)


def test_a_raising_module_fails_closed():
    ok, why = F.check_routed_reads(StandIn(boom=True), top_k=2)
    assert not ok and why == "self-check raised RuntimeError: kernel refused the call"


def test_a_call_that_routes_every_expert_is_vacuous():
    ok, why = F.check_routed_reads(StandIn(E=2), top_k=2)
    assert not ok and why.startswith("vacuous at M=1: all 2 experts were routed")


def test_the_original_tensors_are_left_untouched():
    m = StandIn()
    before = {k: v.clone() for k, v in m.tensors().items()}
    F.check_routed_reads(m, top_k=2)
    for k, v in m.tensors().items():
        assert torch.equal(v, before[k])


def test_the_verdict_is_decided_once_per_geometry(capsys, monkeypatch):
    monkeypatch.setattr(F, "_ROUTED_VERDICTS", {})
    good, bad = StandIn(H=16), StandIn(H=24, leak=True)
    assert F.routed_reads_verdict(good, 2, "layers.0.mlp") is True
    assert F.routed_reads_verdict(StandIn(H=16), 2, "layers.1.mlp") is True
    assert F.routed_reads_verdict(bad, 2, "layers.2.mlp") is False
    out = capsys.readouterr().out.splitlines()
    assert len(out) == 2
    assert out[0].startswith("[Vaayu-MoE] fused-3D kernels ON for layers.0.mlp's geometry")
    assert out[1].startswith("[Vaayu-MoE] WARNING: fused-3D kernels OFF for layers.2.mlp's")
    assert F.routed_reads_verdict(bad, 3, "layers.3.mlp") is False   # top_k is in the key
    assert len(capsys.readouterr().out.splitlines()) == 1
