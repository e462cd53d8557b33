"""The committed tiny-MoE golden fixture (tests/golden/make_tiny_moe.py):
inputs regenerate from the seed, and the oracle reproduces every stored
intermediate bit for bit.  The GPU side of the fixture is in test_gpu_moe.py."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_tiny_moe as G  # noqa: E402

from oracle import moe as OM  # noqa: E402


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(G.PATH))


@pytest.fixture(scope="module")
def inputs():
    return G.make_inputs()


def test_inputs_regenerate_from_seed(golden, inputs):
    assert bytes(golden["weights_sha256"]).decode() == G.weights_digest(inputs)
    np.testing.assert_array_equal((inputs["x"].view(np.uint32) >> 16).astype(np.uint16),
                                  golden["x_bf16_bits"])
    np.testing.assert_array_equal(inputs["logits"].view(np.uint32),
                                  golden["logits"].view(np.uint32))


def test_routing_has_no_near_ties(golden):
    assert OM.topk_margin(golden["logits"], G.K_TOP) > 1e-4


def test_oracle_reproduces_fixture(golden, inputs):
    out = G.compute(inputs)
    for key, val in out.items():
        ref = golden[key]
        assert val.shape == ref.shape, key
        if val.dtype.kind == "f":
            np.testing.assert_array_equal(val.view(np.uint32), ref.view(np.uint32), err_msg=key)
        else:
            np.testing.assert_array_equal(val, ref, err_msg=key)


def test_fixture_invariants(golden):
    """Facts fixed by the math, independent of the oracle's code."""
    ids, counts, offsets = golden["ids"], golden["counts"], golden["offsets"]
    assert ids.shape == (G.T, G.K_TOP) and all(len(set(r)) == G.K_TOP for r in ids.tolist())
    np.testing.assert_array_equal(counts, np.bincount(ids.ravel(), minlength=G.E))
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    ss, sp = golden["sorted_slot"], golden["slot_pos"]
    np.testing.assert_array_equal(np.sort(ss), np.arange(G.T * G.K_TOP))
    np.testing.assert_array_equal(sp[ss], np.arange(G.T * G.K_TOP))
    # softmax top-k weights of 8 experts: each in (0, 1), a row sums to < 1
    w = golden["route_w"]
    assert np.all(w > 0) and np.all(w.sum(axis=1) < 1)
    assert golden["hq"].shape == (G.T * G.K_TOP + G.T, G.I)
