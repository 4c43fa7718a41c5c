"""The oracle against its committed golden fixtures (tests/golden/*.json,
written by tests/golden/make_golden.py): pins the CPU restatement against
drift.  The oracle is deterministic, so the bar is float round-off."""
import json
import os

import numpy as np
import pytest

from tests.golden.make_golden import CASES, adaptive_threshold, detections, forward
from simdyolo_amd import synth

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(HERE, f"{name}.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(name):
    arch, scale = CASES[name]
    g = load(name)
    cfg = synth.config(scale, arch=arch)
    head = forward(arch, scale, synth.params(cfg, seed=g["weights_seed"]),
                   synth.images(1, g["size"], g["size"], seed=g["image_seed"]))
    assert list(head.shape) == g["shape"]
    flat = head.reshape(-1)
    np.testing.assert_allclose(flat[g["sample_index"]], g["sample_value"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(head[0].astype(np.float64).sum(1), g["channel_sums"], rtol=1e-6, atol=1e-4)
    assert adaptive_threshold(head[0]) == pytest.approx(g["adaptive_threshold"], rel=1e-6)
    got = detections(head[0], g["adaptive_threshold"])
    assert [d[:2] for d in got] == [d[:2] for d in g["detections_adaptive"]]
    assert len(g["detections_adaptive"]) > 50  # the threshold makes NMS decide real cases
