"""Execution-v1 step graphs: parsing both forms of the reference's example
graphs (tests/golden/execution_v1, data files of runtime/zig/examples/
execution-v1), the decode plan, the per-layer attention window rule of
emit_csl_exec_v1.zig:612-641 and the errors the reference's lowering raises."""
import copy
import json
from pathlib import Path

import pytest

from doe_amd import execution as ex
from doe_amd.model import DecoderConfig

GOLD = Path(__file__).parent / "golden" / "execution_v1"


def graph_json(name):
    return json.loads((GOLD / name).read_text())


def test_both_forms_of_the_270m_graph_plan_alike():
    flat = ex.load_step_graph(GOLD / "gemma-3-270m-smoke.json")
    manifest = ex.load_step_graph(GOLD / "gemma-3-270m-manifest-smoke.json")
    assert flat.model_id == manifest.model_id == "gemma-3-270m-it-q4k-ehf16-af32"
    assert flat.eos_token_id == manifest.eos_token_id == 1
    p1, p2 = ex.plan_decode(flat, 18), ex.plan_decode(manifest, 18)
    assert p1.layer == p2.layer
    assert [d.kind for d in p1.layer] == ["qkv_rope_kv", "attention", "attn_out", "gate_up", "down"]
    assert p1.windows == p2.windows == (0,) * 18
    # every decode step is carried out by exactly one dispatch
    for g, p in ((flat, p1), (manifest, p2)):
        covered = [n for d in p.layer + p.post for n in d.steps]
        assert sorted(covered) == sorted(s.name for s in g.phase("decode"))
    assert p2.post[0].steps == ("final_norm", "lm_head", "sample")
    # manifest ops come from the kernel files (gemv -> matmul_gemv_subgroup.wgsl -> matmul_q4k)
    ops = {s.name: s.op for s in manifest.phase("decode")}
    assert ops["q_proj"] == "matmul_q4k" and ops["attention"] == "attention" and ops["activation"] == "gelu"


def test_graphs_this_library_does_not_execute_are_refused_by_step():
    with pytest.raises(ex.UnsupportedStep, match="numKvSharedLayers"):
        ex.plan_decode(ex.load_step_graph(GOLD / "gemma-4-e2b-smoke.json"), 35)
    with pytest.raises(ex.UnsupportedStep, match="conv1d_depthwise"):
        ex.plan_decode(ex.load_step_graph(GOLD / "qwen-3-6-27b-smoke.json"), 64)
    e2b = graph_json("gemma-4-e2b-smoke.json")
    with pytest.raises(ex.UnsupportedStep, match="globalHeadDim"):
        DecoderConfig.from_model_config(e2b["modelConfig"])
    # without the shared-KV layers the per-layer embedding steps are what stops it
    e2b.pop("numKvSharedLayers")
    with pytest.raises(ex.UnsupportedStep, match="ple_"):
        ex.plan_decode(ex.load_step_graph(e2b), 35)


def test_layer_pattern_windows_follow_the_reference_rule():
    g = graph_json("gemma-3-270m-smoke.json")
    g["layerPattern"] = {"type": "every_n", "period": 6, "offset": 5}
    g["slidingWindowSize"] = 512
    plan = ex.plan_decode(ex.load_step_graph(g), 18)
    # emit_csl_exec_v1.zig:612-614: layer i is global iff i % period == offset
    assert plan.windows == tuple(0 if i % 6 == 5 else 512 for i in range(18))
    # a step's attentionType wins over the pattern; attention_sliding is always sliding
    g2 = copy.deepcopy(g)
    for s in g2["steps"]:
        if s["phase"] == "decode" and s["op"] == "attention":
            s["attentionType"] = "global"
    assert ex.plan_decode(ex.load_step_graph(g2), 18).windows == (0,) * 18
    for s in g2["steps"]:
        if s["phase"] == "decode" and s["op"] == "attention":
            s["op"] = "attention_sliding"
            s.pop("attentionType")
            s["slidingWindowSize"] = 64
    assert ex.plan_decode(ex.load_step_graph(g2), 18).windows == (64,) * 18


def test_malformed_graphs_raise():
    g = graph_json("gemma-3-270m-smoke.json")
    bad = copy.deepcopy(g)
    bad["steps"][3]["op"] = "no_such_op"
    with pytest.raises(ex.StepGraphError, match="unknown op"):
        ex.load_step_graph(bad)
    bad = copy.deepcopy(g)
    bad["steps"][7]["phase"] = "prefill"  # attention (decode-only) in prefill
    bad["steps"][7]["op"] = "attention"
    with pytest.raises(ex.StepGraphError, match="not allowed in prefill"):
        ex.load_step_graph(bad)
    bad = copy.deepcopy(g)
    bad["steps"][-1]["kind"] = "compute"  # sample is of kind sample
    with pytest.raises(ex.StepGraphError, match="kind"):
        ex.load_step_graph(bad)
    bad = copy.deepcopy(g)
    bad["layerPattern"] = {"type": "every_n", "period": 2, "offset": 0}  # sliding layers, no window
    with pytest.raises(ex.StepGraphError, match="slidingWindowSize"):
        ex.plan_decode(ex.load_step_graph(bad), 4)
    bad = copy.deepcopy(g)
    bad["layerPattern"] = {"type": "every_other"}
    with pytest.raises(ex.StepGraphError, match="every_n"):
        ex.load_step_graph(bad)
    bad = copy.deepcopy(g)
    del bad["steps"][-1]  # no sample
    with pytest.raises(ex.StepGraphError, match="sample"):
        ex.plan_decode(ex.load_step_graph(bad), 4)
    bad = copy.deepcopy(g)
    bad["steps"] = [s for s in bad["steps"] if not (s["phase"] == "decode" and s["name"] == "v_proj")]
    with pytest.raises(ex.UnsupportedStep, match="matmul_q4k"):
        ex.plan_decode(ex.load_step_graph(bad), 4)
    with pytest.raises(ex.StepGraphError):
        ex.load_step_graph({"modelId": "x"})
    with pytest.raises(ex.StepGraphError):
        ex.load_step_graph("{not json")


def test_model_config_maps_to_decoder_config():
    mc = {"hiddenDim": 640, "numHeads": 4, "headDim": 256, "numKeyValueHeads": 1, "numLayers": 18,
          "vocabSize": 262144, "maxSeqLen": 512, "quantFormat": "q4k", "ffnExpansionFactor": 4}
    c = DecoderConfig.from_model_config(mc, max_seq=64)
    assert (c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim, c.vocab, c.ffn, c.max_seq) == \
        (18, 640, 4, 1, 256, 262144, 2560, 64)
    assert c.weight_format == "q4k"
    q8 = DecoderConfig.from_model_config({**mc, "quantFormat": "q8_0"})
    assert q8.weight_format == "q8_0"
    # 640-wide rows are 20 Q8_0 blocks of 34 bytes, 3 Q4_K blocks of 144; per
    # layer: qkv 1536 and gate/up 2 x 2560 rows of 640, o_proj 640 rows of
    # 1024 (32 blocks), down 640 rows of 2560 (80 blocks)
    assert q8.row_bytes(640) == 680 and c.row_bytes(640) == 432
    assert q8.weight_bytes_per_layer() == (1536 + 2 * 2560) * 680 + 640 * 32 * 34 + 640 * 80 * 34
    for bad in ("q6k", "f16"):
        with pytest.raises(ex.UnsupportedStep, match="quantFormat"):
            DecoderConfig.from_model_config({**mc, "quantFormat": bad})


def test_reference_lowering_known_answers():
    # the cases of runtime/zig/tests/wgsl/emit_csl_exec_v1_test.zig, as data
    with pytest.raises(ex.StepGraphError, match="kind"):  # embed declared as a sample step
        ex.load_step_graph({"grid": {"width": 8, "height": 1}, "steps": [
            {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather", "kind": "sample"}]})
    with pytest.raises(ex.StepGraphError, match="before any prefill"):  # decode before prefill
        ex.load_step_graph({"grid": {"width": 8, "height": 1}, "steps": [
            {"phase": "decode", "op": "attention", "kernelKey": "attn_0"}]})
    with pytest.raises(ex.StepGraphError, match="attentionType"):  # "local" is not an attention type
        ex.load_step_graph({"grid": {"width": 8, "height": 1}, "steps": [
            {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
            {"phase": "decode", "op": "attention", "kernelKey": "attn_0", "attentionType": "local"}]})
    # Gemma 4 routing from layerPattern: decode attention 0 is sliding (512),
    # attention 1 global
    g = ex.load_step_graph({"grid": {"width": 8, "height": 1}, "slidingWindowSize": 512,
                            "layerPattern": {"type": "every_n", "period": 2, "offset": 1}, "steps": [
                                {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
                                {"phase": "decode", "op": "attention", "kernelKey": "attn_local"},
                                {"phase": "decode", "op": "kv_write", "kernelKey": "kv_write"},
                                {"phase": "decode", "op": "attention", "kernelKey": "attn_global"},
                                {"phase": "decode", "op": "sample", "kernelKey": "sampler", "kind": "sample"}]})
    attns = [s for s in g.phase("decode") if s.op == "attention"]
    assert [ex._window(g, a, i) for i, a in enumerate(attns)] == [512, 0]
