"""The HIP decode on the committed toy-layer fixture (hidden 1024, 32 experts, inter 512,
top-4, int4 g128 fp16 scales, bf16): routed pairs' stages and the layer output."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden import make_golden as G
import vaayu_amd.packed_expert_kernels as pk

pytestmark = pytest.mark.gpu
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_decode.npz")


def test_the_toy_layer_matches_the_fixture():
    gold = dict(np.load(FIXTURE))
    x, _wr, blobs = G.inputs()
    ids, w, order = gold["ids"], gold["weights"], gold["pair_order"]
    dev = [{"flat": {n: t.cuda() for n, t in blobs[int(ids[s])]["flat"].items()},
            "geom": blobs[int(ids[s])]["geom"]} for s in order]
    pairs = [(dev[i], int(s)) for i, s in enumerate(order)]
    xd = torch.from_numpy(x).to(torch.bfloat16).cuda()
    rw = torch.from_numpy(w).reshape(1, -1).cuda()
    out = torch.empty(1, G.HIDDEN, dtype=torch.float32, device="cuda")
    pk._launch(xd, pairs, rw, out)
    tbl = pk._TABLES.put(pk._table_values(pairs), "cuda")
    sc = pk._DTYPE_CODE[torch.float16]
    h = pk._gate_up(xd, tbl, len(pairs), pairs[0][0]["geom"], sc)
    torch.cuda.synchronize()
    got_h = O.bf16_bits(h.float().cpu().numpy())
    assert (got_h == gold["h_bits"]).mean() >= 0.99
    got = out.cpu().numpy()
    ref = gold["out"]
    assert O.rel_l2(got, ref) <= 5e-3
    assert np.abs(got - ref).max() <= 2e-2
