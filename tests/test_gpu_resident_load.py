"""A compressed-tensors checkpoint layer read from its safetensors byte ranges straight into
HBM-resident blobs (vaayu_amd/expert_offset_index.py), then decoded on the GPU with routing
on the device: the blobs are byte-equal to blobs built from the same tensors in memory, and
the layer's output equals the stock loop's (oracle) on the routing the device chose."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from vaayu_amd.device_routing import ResidentExperts
from vaayu_amd.expert_offset_index import ExpertOffsetIndex, load_resident_experts
from vaayu_amd.moe_patch import build_expert_blob
from tests.test_expert_offset_index import _compressed_tensors_layer

pytestmark = pytest.mark.gpu


def test_resident_layer_from_the_checkpoint_bytes(tmp_path):
    E, H, I, K = 8, 256, 128, 2
    by_expert = _compressed_tensors_layer(tmp_path, "model.layers.5", E, H, I, bits=4, gs=32,
                                          seed=9)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build_or_load()
    blobs = load_resident_experts(idx, "model.layers.5", "cuda")
    torch.cuda.synchronize()
    for e, by_role in by_expert.items():
        want = build_expert_blob(by_role)
        assert blobs[e]["flat"]["packed"].is_cuda and blobs[e]["geom"] == want["geom"]
        for k in ("packed", "scale"):
            assert torch.equal(blobs[e]["flat"][k].cpu(), want["flat"][k])
    rx = ResidentExperts([blobs[e] for e in range(E)])
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(1, H, generator=g) * 0.5).bfloat16().cuda()
    logits = torch.randn(1, E, generator=g).cuda()
    out = torch.empty(1, H, dtype=torch.float32, device="cuda")
    w, ids = rx.decode(x, logits, K, out)
    torch.cuda.synchronize()
    e = ids[0].cpu().tolist()
    pairs = [({"flat": {n: t.cpu() for n, t in blobs[e[s]]["flat"].items()},
               "geom": blobs[0]["geom"]}, s) for s in sorted(range(K), key=e.__getitem__)]
    ref = O.stock_decode(x.cpu(), pairs, w.cpu())
    assert O.rel_l2(O.to_np(out), ref) <= 5e-3
    assert np.abs(O.to_np(out) - ref).max() <= 2e-2
