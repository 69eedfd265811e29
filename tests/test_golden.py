"""The committed toy-layer fixture (tests/golden/toy_decode.npz): the oracle still
reproduces it bit for bit, and its routing obeys the closed form."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden import make_golden as G

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_decode.npz")


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(FIXTURE))


@pytest.fixture(scope="module")
def generated():
    return G.inputs()


def test_the_inputs_regenerate_from_the_seed(golden, generated):
    x, wr, blobs = generated
    assert int(golden["seed"]) == G.SEED
    assert np.array_equal(O.bf16_bits(x), golden["x_bits"])
    import hashlib
    assert hashlib.sha256(O.bf16_bits(wr).tobytes()).hexdigest() == str(golden["router_sha256"])
    assert [G.digest(b) for b in blobs] == golden["expert_sha256"].tolist()


def test_the_oracle_reproduces_the_fixture(golden, generated):
    logits, ids, w, order, hs, ys, out = G.evaluate(*generated)
    assert np.array_equal(O.bf16_bits(logits), golden["logits_bits"])
    assert np.array_equal(ids, golden["ids"]) and np.array_equal(w, golden["weights"])
    assert np.array_equal(order, golden["pair_order"])
    assert np.array_equal(O.bf16_bits(hs), golden["h_bits"])
    assert np.array_equal(ys, golden["y"]) and np.array_equal(out, golden["out"])


def test_the_routing_is_the_closed_form(golden):
    lg = O.bf16_value(golden["logits_bits"]).astype(np.float64).reshape(-1)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    top = np.argsort(-p, kind="stable")[:4]
    assert golden["ids"].tolist() == top.tolist()
    assert np.allclose(golden["weights"], p[top] / p[top].sum(), rtol=1e-6)
    assert len(set(golden["ids"].tolist())) == 4


def test_the_output_is_the_ordered_sum_of_the_contributions(golden):
    w = golden["weights"]
    acc = np.zeros(golden["out"].shape[-1], dtype=np.float32)
    for p, slot in enumerate(golden["pair_order"]):
        acc = (acc + (golden["y"][p] * w[slot]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(acc, golden["out"].reshape(-1))
