"""The oracle's per-layer-embedding functions (oracle/decoder.py ple_inputs,
ple_block) against the reference's own E2B restatement
(bench/tools/run_gemma4_e2b_manifest_shape_execution.py: compute_per_layer_inputs,
execute_layer), run by tests/golden/make_e2b_ple_vectors.py on seeded inputs
that make_inputs() regenerates here.  The two compute the same products in
other orders (numpy matmul against the oracle's left folds), so they agree to
f32 rounding; a dropped term (the sqrt(width) table scale, the 1/sqrt(2)
combine, the hidden^-1/2 projection scale, the post-block norm or the
residual) moves the result by orders of magnitude more."""
import importlib.util
import json

import numpy as np
import pytest

from conftest import ROOT

GOLDEN = ROOT / "tests" / "golden"


def _gen():
    spec = importlib.util.spec_from_file_location("make_e2b_ple_vectors", GOLDEN / "make_e2b_ple_vectors.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def case():
    gen = _gen()
    vec = json.loads((GOLDEN / "e2b_ple_vectors.json").read_text())
    assert vec["seed"] == gen.SEED
    return gen, gen.make_inputs(vec["seed"]), vec


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_ple_inputs_match_the_reference(case):
    from oracle.decoder import ple_inputs

    gen, inp, vec = case
    c = vec["config"]
    got = ple_inputs(inp["table"], inp["proj"], inp["norm_ple_proj"], c["token"], inp["x"], c["layers"], c["width"],
                     c["hidden"], c["eps"], False)
    want = np.asarray(vec["per_layer_inputs"], np.float32)
    assert got.shape == want.shape == (c["layers"], c["width"])
    assert rel(got, want) <= 1e-6


def test_ple_block_matches_the_reference(case):
    from oracle.decoder import ple_block

    gen, inp, vec = case
    c = vec["config"]
    u0 = np.asarray(vec["per_layer_inputs"], np.float32)[0]
    got = ple_block(inp["w_gate"], inp["w_out"], inp["norm_post_ple"], inp["h"], u0, c["width"], c["hidden"],
                    c["eps"], False)
    want = np.asarray(vec["ple_block_out"], np.float32)
    assert rel(got, want) <= 1e-6
    # the block's own contribution is a sizeable part of the output, so the
    # bound above constrains it, not only the residual it is added to
    assert rel(inp["h"], want) > 0.1


def test_a_dropped_scale_is_caught(case):
    # the same check fails for the oracle's inputs without the 1/sqrt(2) combine
    from oracle.decoder import ple_inputs

    gen, inp, vec = case
    c = vec["config"]
    got = ple_inputs(inp["table"], inp["proj"], inp["norm_ple_proj"], c["token"], inp["x"], c["layers"], c["width"],
                     c["hidden"], c["eps"], False) * np.float32(2.0 ** 0.5)
    assert rel(got, vec["per_layer_inputs"]) > 0.1
