"""CPU: the oracle reproduces the committed golden fixtures (determinism of the
generator and of the oracle across machines and builds)."""
import json
import os

import numpy as np

import oracle as O
from conftest import rel_rmse

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_config1_fixture_reproduces():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    want = json.load(open(os.path.join(HERE, "config1.json")))
    got = mg.config1()
    assert got["x_sha"] == want["x_sha"]
    assert got["topk_idx"] == want["topk_idx"]
    assert np.array_equal(np.float32(got["out"]), np.float32(want["out"]))
    assert np.array_equal(np.float32(got["logits"]), np.float32(want["logits"]))
    # the chosen experts are the 8 largest logits, ties to the lower index
    lg = np.array(want["logits"])
    order = sorted(range(len(lg)), key=lambda e: (-lg[e], e))[:8]
    assert order == want["topk_idx"]
    assert abs(sum(want["topk_w"]) - 1.0) < 1e-6
