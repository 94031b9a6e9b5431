"""The oracle against the committed golden fixtures (tests/golden/make_golden.py): any change to the oracle's
arithmetic shows up here, on the CPU."""
from pathlib import Path

import numpy as np
import pytest

import oracle as O

G = np.load(Path(__file__).resolve().parent / "golden" / "oracle_vectors.npz")


@pytest.mark.parametrize("cb,k2", sorted(O.COMPILED))
def test_golden_dequant(cb, k2):
    assert np.array_equal(O.dequant(G[f"dequant_cb{cb}_k{k2}_trellis"], k2, cb), G[f"dequant_cb{cb}_k{k2}_w"])


def test_golden_rotate_and_had():
    assert np.array_equal(O.rotate(G["rotate_x_bf16"], "bf16", G["rotate_suh"]), G["rotate_out"])
    assert np.array_equal(O.had(G["had_x"], G["had_pre"], G["had_post"]), G["had_out"])


def test_golden_route_and_group():
    pick, wts, logits, _ = O.route(G["route_x"], G["route_gate"], 8, G["route_sgate"], shared_id=64)
    assert np.array_equal(pick, G["route_pick"])
    assert np.array_equal(logits, G["route_logits"])
    assert np.array_equal(wts, G["route_wts"])
    cnt, uids, members = O.group(G["group_pick"], 5, 9, 10, 45)
    assert np.array_equal(uids, G["group_uids"]) and np.array_equal(members, G["group_members"])
