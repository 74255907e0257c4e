"""Writes e2b_ple_vectors.json: the reference's Gemma 4 E2B per-layer-input
functions run on small seeded inputs.

The reference restates the E2B text stack in numpy
(bench/tools/run_gemma4_e2b_manifest_shape_execution.py).  Two of its
functions define what the decoder's per-layer-embedding steps compute, and no
known-answer vector of the reference covers them:

  * compute_per_layer_inputs (:383-404): one token's per-layer inputs;
  * execute_layer (:314-380), whose last lines are a layer's per-layer input
    block.  It runs here with o_proj and down_proj zero (the attention and
    MLP add nothing: rms_norm(0) = 0) and layer_scalar 1, so its output is
    the residual stream after the block alone.

This script imports that module from /root/reference (it reads tensors
through a store object; a dict-backed one stands in for its SafeTensors
reader) and records the outputs.  The inputs are not stored: make_inputs()
regenerates them from the seed, and tests/test_oracle_ple.py feeds the same
inputs to the oracle.  Q4_K weights reach the reference as their exact
dequantised values (the oracle's dequant, pinned by the reference's own
Q4_K vectors), f16 tables as their exact f32 values.

Run from the repository root: python tests/golden/make_e2b_ple_vectors.py
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REFERENCE = Path("/root/reference/bench/tools/run_gemma4_e2b_manifest_shape_execution.py")
OUT = HERE / "e2b_ple_vectors.json"

SEED = 20261202
LAYERS, WIDTH, HIDDEN, VOCAB, TOKEN, EPS = 2, 256, 256, 8, 5, 1e-6


def make_inputs(seed: int = SEED) -> dict:
    """The seeded inputs: f16 per-layer table and model projection, f32 norm
    weights used as they are (no 1 + w), the token's input embedding x, the
    residual stream h entering the block, Q4_K gate [WIDTH][HIDDEN] and
    projection [HIDDEN][WIDTH] rows."""
    sys.path.insert(0, str(ROOT))
    from doe_amd import q4k

    rng = np.random.default_rng(seed)
    return {
        "table": (rng.standard_normal((VOCAB, LAYERS * WIDTH)) * 0.05).astype(np.float16),
        "proj": (rng.standard_normal((LAYERS * WIDTH, HIDDEN)) * 0.05).astype(np.float16),
        "norm_ple_proj": (1.0 + 0.1 * rng.standard_normal(WIDTH)).astype(np.float32),
        "x": rng.standard_normal(HIDDEN).astype(np.float32),
        "h": rng.standard_normal(HIDDEN).astype(np.float32),
        "w_gate": q4k.random_q4k(rng, WIDTH, HIDDEN),
        "w_out": q4k.random_q4k(rng, HIDDEN, WIDTH),
        "norm_post_ple": (1.0 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32),
    }


class _Store:
    """The reference runner's tensor store interface (read(name, row=None))."""

    def __init__(self, tensors: dict):
        self.t = tensors

    def read(self, name: str, row: int | None = None) -> np.ndarray:
        a = self.t[name]
        return a[row] if row is not None else a


def main() -> int:
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as ora

    spec = importlib.util.spec_from_file_location("e2b_reference_runner", REFERENCE)
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)

    inp = make_inputs()
    pre = ref.LANG_PREFIX
    lp = f"{pre}.layers.0"
    hd, ffn = HIDDEN, 16
    zeros = np.zeros
    rng = np.random.default_rng(SEED + 1)  # attention / MLP weights: their output is zeroed
    tensors = {
        f"{pre}.embed_tokens_per_layer.weight": inp["table"].astype(np.float32),
        f"{pre}.per_layer_model_projection.weight": inp["proj"].astype(np.float32),
        f"{pre}.per_layer_projection_norm.weight": inp["norm_ple_proj"],
        f"{lp}.input_layernorm.weight": np.ones(HIDDEN, np.float32),
        f"{lp}.self_attn.q_proj.weight": rng.standard_normal((hd, HIDDEN)).astype(np.float32),
        f"{lp}.self_attn.q_norm.weight": np.ones(hd, np.float32),
        f"{lp}.self_attn.k_proj.weight": rng.standard_normal((hd, HIDDEN)).astype(np.float32),
        f"{lp}.self_attn.v_proj.weight": rng.standard_normal((hd, HIDDEN)).astype(np.float32),
        f"{lp}.self_attn.k_norm.weight": np.ones(hd, np.float32),
        f"{lp}.self_attn.o_proj.weight": zeros((HIDDEN, hd), np.float32),
        f"{lp}.post_attention_layernorm.weight": np.ones(HIDDEN, np.float32),
        f"{lp}.pre_feedforward_layernorm.weight": np.ones(HIDDEN, np.float32),
        f"{lp}.mlp.gate_proj.weight": rng.standard_normal((ffn, HIDDEN)).astype(np.float32),
        f"{lp}.mlp.up_proj.weight": rng.standard_normal((ffn, HIDDEN)).astype(np.float32),
        f"{lp}.mlp.down_proj.weight": zeros((HIDDEN, ffn), np.float32),
        f"{lp}.post_feedforward_layernorm.weight": np.ones(HIDDEN, np.float32),
        f"{lp}.per_layer_input_gate.weight": ora.q4k_dequant_rowwise(inp["w_gate"], WIDTH, HIDDEN),
        f"{lp}.per_layer_projection.weight": ora.q4k_dequant_rowwise(inp["w_out"], HIDDEN, WIDTH),
        f"{lp}.post_per_layer_input_norm.weight": inp["norm_post_ple"],
        f"{lp}.layer_scalar": np.ones(1, np.float32),
    }
    store = _Store(tensors)
    config = {
        "num_hidden_layers": LAYERS,
        "hidden_size_per_layer_input": WIDTH,
        "hidden_size": HIDDEN,
        "rms_norm_eps": EPS,
        "num_attention_heads": 1,
        "num_key_value_heads": 1,
        "head_dim": hd,
        "layer_types": ["sliding_attention"] * LAYERS,
        "num_kv_shared_layers": 0,
    }
    per_layer = ref.compute_per_layer_inputs(store, config, TOKEN, inp["x"])
    out, _ = ref.execute_layer(store, config, inp["h"], per_layer[0], 0, {})
    OUT.write_text(json.dumps({
        "source": "bench/tools/run_gemma4_e2b_manifest_shape_execution.py: compute_per_layer_inputs "
                  "(383-404) and execute_layer (314-380; o_proj and down_proj zero, layer_scalar 1)",
        "generator": "tests/golden/make_e2b_ple_vectors.py",
        "seed": SEED,
        "config": {"layers": LAYERS, "width": WIDTH, "hidden": HIDDEN, "vocab": VOCAB, "token": TOKEN, "eps": EPS},
        "per_layer_inputs": np.asarray(per_layer, np.float32).round(9).tolist(),
        "ple_block_out": np.asarray(out, np.float32).round(9).tolist(),
    }, indent=None) + "\n")
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
