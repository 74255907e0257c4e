"""RDRR artifacts (doe_amd/rdrr.py): the span reader over shard files, the
Q4_K_M row checks, dense conversions and the weight-key names -- including
the reference reader's own case (bench/tests/test_doppler_rdrr_q4k.py:
103-143: two 300-column rows of constant-quant blocks in one shard, read
across the row boundary)."""
import json

import numpy as np
import pytest

from doe_amd import q4k, rdrr


def block(qv: int) -> bytes:
    # d = 1, dmin = 0, every scale 1: each weight equals its quant
    return q4k.pack_blocks([1.0], [0.0], [[1] * 8], [[0] * 8], [[qv] * 256]).tobytes()


def write_artifact(root, shards: dict, tensors: dict, with_filenames: bool = True):
    for idx, data in shards.items():
        (root / f"shard_{idx:05d}.bin").write_bytes(data)
    manifest = {"shards": [{"index": i, **({"filename": f"shard_{i:05d}.bin"} if with_filenames else {}),
                            "size": len(d)} for i, d in shards.items()],
                "tensors": tensors}
    (root / "manifest.json").write_text(json.dumps(manifest))
    return rdrr.RdrrArtifact(root)


def test_reference_reader_case(tmp_path, ora):
    data = block(1) + block(2) + block(3) + block(4)
    art = write_artifact(tmp_path, {0: data}, {"tensor.weight": {
        "shard": 0, "offset": 0, "size": len(data), "shape": [2, 300], "dtype": "Q4_K_M", "layout": "row"}})
    rows = art.q4k_rows("tensor.weight")
    assert rows.shape == (2, 288) and rows.tobytes() == data  # byte-identical, tail padding kept
    vals = ora.q4k_dequant_rowwise(rows, 2, 300).reshape(-1)
    # the reference's expectations for the first 320 values
    assert (vals[:256] == 1.0).all() and (vals[256:300] == 2.0).all() and (vals[300:320] == 3.0).all()
    assert (vals[320:556] == 3.0).all() and (vals[556:600] == 4.0).all()


def test_spans_across_shards_and_ranges(tmp_path):
    rng = np.random.default_rng(0)
    mat = q4k.random_q4k(rng, 3, 512)  # 3 rows x 288 bytes
    raw = mat.tobytes()
    pad = bytes(rng.integers(0, 256, 100, dtype=np.uint8))
    # rows split mid-row over two shards; shard 1 has no filename (default name)
    s0, s1 = pad + raw[:400], raw[400:] + pad
    art = write_artifact(tmp_path, {0: s0, 1: s1}, {"w": {
        "spans": [{"shardIndex": 0, "offset": 100, "size": 400}, {"shard": 1, "offset": 0, "size": len(raw) - 400}],
        "size": len(raw), "shape": [3, 512], "dtype": "Q4_K_M", "layout": "row"}}, with_filenames=False)
    assert art.read("w").tobytes() == raw
    assert art.read("w", 350, 100).tobytes() == raw[350:450]  # across the span boundary
    assert art.read("w", 400, 10).tobytes() == raw[400:410]
    assert np.array_equal(art.q4k_rows("w"), mat.reshape(3, 288))
    with pytest.raises(rdrr.RdrrError, match="outside"):
        art.read("w", 800, 100)
    with pytest.raises(KeyError):
        art.read("missing")


def test_malformed_tensors_raise(tmp_path):
    data = block(5) * 2
    base = {"shard": 0, "offset": 0, "size": len(data), "shape": [2, 256], "dtype": "Q4_K_M", "layout": "row"}
    tensors = {
        "ok": base,
        "not_q4k": {**base, "dtype": "F16", "shape": [2, 144]},
        "col_layout": {**base, "layout": "col"},
        "short": {**base, "shape": [3, 256]},
        "past_end": {**base, "offset": 10},
        "no_shard_file": {**base, "shard": 7},
        "vector": {**base, "shape": [288]},
    }
    art = write_artifact(tmp_path, {0: data}, tensors)
    assert art.q4k_rows("ok").shape == (2, 144)
    with pytest.raises(rdrr.RdrrError, match="not Q4_K_M"):
        art.q4k_rows("not_q4k")
    with pytest.raises(rdrr.RdrrError, match="layout"):
        art.q4k_rows("col_layout")
    with pytest.raises(rdrr.RdrrError, match="Q4_K_M matrix has"):
        art.q4k_rows("short")
    with pytest.raises(rdrr.RdrrError, match="runs past"):
        art.q4k_rows("past_end")
    with pytest.raises(FileNotFoundError):
        art.q4k_rows("no_shard_file")
    with pytest.raises(rdrr.RdrrError, match="not a matrix"):
        art.q4k_rows("vector")
    with pytest.raises(rdrr.RdrrError):
        rdrr.RdrrArtifact(tmp_path / "nowhere")


def test_dense_tensors_convert_exactly(tmp_path):
    f32 = np.array([1.5, -2.25, 0.0, 65504.0, 2.0 ** -24, -0.1], np.float32)
    f16 = f32.astype(np.float16)
    bf = (f32.view(np.uint32) >> 16).astype(np.uint16)  # truncation: values chosen exact in bf16 above
    blob = f32.tobytes() + f16.tobytes() + bf.tobytes()
    o1, o2 = f32.nbytes, f32.nbytes + f16.nbytes
    art = write_artifact(tmp_path, {0: blob}, {
        "a": {"shard": 0, "offset": 0, "size": f32.nbytes, "shape": [6], "dtype": "F32"},
        "b": {"shard": 0, "offset": o1, "size": f16.nbytes, "shape": [2, 3], "dtype": "F16"},
        "c": {"shard": 0, "offset": o2, "size": bf.nbytes, "shape": [6], "dtype": "BF16"},
        "d": {"shard": 0, "offset": 0, "size": 8, "shape": [2], "dtype": "Q8_0"},
    })
    assert np.array_equal(art.dense("a", np.float32), f32)
    assert np.array_equal(art.dense("b", np.float32).reshape(-1), f16.astype(np.float32))
    assert art.dense("b", np.float16).shape == (2, 3)
    want_bf = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(art.dense("c", np.float32), want_bf)
    with pytest.raises(rdrr.RdrrError, match="not dense"):
        art.dense("d", np.float32)


def test_weight_keys_resolve_to_tensor_names(tmp_path):
    assert rdrr.weight_key_candidates("layer.3.self_attn.q_proj") == [
        "model.language_model.layers.3.self_attn.q_proj.weight", "model.layers.3.self_attn.q_proj.weight"]
    assert rdrr.weight_key_candidates("layer.0.input_layernorm")[1] == "model.layers.0.input_layernorm.weight"
    # a tied lm_head falls back to the embedding
    assert rdrr.weight_key_candidates("lm_head")[-1] == "embed_tokens.weight"
    with pytest.raises(rdrr.RdrrError):
        rdrr.weight_key_candidates("layer.x.mlp")
    with pytest.raises(rdrr.RdrrError):
        rdrr.weight_key_candidates("something_else")
    art = write_artifact(tmp_path, {0: b"\0" * 16}, {
        "model.embed_tokens.weight": {"shard": 0, "offset": 0, "size": 16, "shape": [2, 4], "dtype": "F16"}})
    assert art.resolve("embed_tokens") == "model.embed_tokens.weight"
    assert art.resolve("lm_head") == "model.embed_tokens.weight"
    with pytest.raises(KeyError, match="norm"):
        art.resolve("norm")


def test_per_layer_embedding_keys_resolve_to_the_reference_names():
    # gemma-4-e2b-smoke.json's per_layer_inputs.* weight keys and the
    # per-layer block's tensors, named as in the reference's E2B artifact
    # (config/gemma-4-e2b-doppler-rdrr-int4ple-fixture.json:34,116-140)
    lp = "model.language_model"
    assert rdrr.weight_key_candidates("per_layer_inputs.embedTokensPerLayer")[0] == \
        f"{lp}.embed_tokens_per_layer.weight"
    assert rdrr.weight_key_candidates("per_layer_inputs.perLayerModelProjection")[0] == \
        f"{lp}.per_layer_model_projection.weight"
    assert rdrr.weight_key_candidates("per_layer_inputs.perLayerProjectionNorm")[0] == \
        f"{lp}.per_layer_projection_norm.weight"
    for tail in ("per_layer_input_gate", "per_layer_projection", "post_per_layer_input_norm"):
        assert rdrr.weight_key_candidates(f"layer.0.{tail}")[0] == f"{lp}.layers.0.{tail}.weight"
