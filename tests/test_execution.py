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


def test_qwen_hybrid_graph_plans_and_the_decoder_refuses_it():
    # qwen-3-6-27b-smoke.json: input_norm, the linear-attention body
    # (conv1d_depthwise, l2_normalize q and k, linear_attention, each
    # repeat 48), then the gated attention layer (q/k norms, rope, attention,
    # o_gate, o_proj, SwiGLU FFN): 48 linear and 16 attention layers, a full
    # attention layer closing each group of four
    g = ex.load_step_graph(GOLD / "qwen-3-6-27b-smoke.json")
    plan = ex.plan_decode(g, 64)
    assert [d.kind for d in plan.layer] == ["qkv_norm_rope_kv", "attention", "gated_attn_out", "gate_up", "down"]
    assert plan.linear.steps == ("input_norm", "ssm_conv1d_depthwise", "ssm_q_l2_normalize", "ssm_k_l2_normalize",
                                 "ssm_linear_attention")
    assert plan.layer_types == ("linear_attention",) * 3 + ("attention",) + plan.layer_types[4:]
    assert [i for i, t in enumerate(plan.layer_types) if t == "attention"] == list(range(3, 64, 4))
    assert plan.windows == (0,) * 64
    # every decode step is carried out by one dispatch
    covered = [n for d in plan.layer + plan.post + (plan.linear,) for n in d.steps]
    assert sorted(set(covered)) == sorted({s.name for s in g.phase("decode")})
    # the host plan launches each body op once per linear-attention layer
    # (decode and prefill)
    hp = ex.lower_host_plan(g)
    counts = {k["name"]: k["count"] for k in hp["kernels"]}
    assert counts["ssm_conv1d_depthwise"] == counts["ssm_linear_attention"] == 96
    # a body whose ops repeat unequally is malformed
    q = graph_json("qwen-3-6-27b-smoke.json")
    bad = copy.deepcopy(q)
    next(s for s in bad["steps"] if s["phase"] == "decode" and s["op"] == "l2_normalize")["repeat"] = 47
    with pytest.raises(ex.StepGraphError, match="not equally"):
        ex.plan_decode(ex.load_step_graph(bad), 64)
    # the decoder refuses what the graph does not define: the projections
    # around the linear-attention body
    from doe_amd.model import Decoder

    cfg = DecoderConfig(layers=64, hidden=256, heads=2, kv_heads=1, head_dim=128, ffn=512, vocab=256, max_seq=16)
    with pytest.raises(ex.UnsupportedStep, match="linear-attention"):
        Decoder(cfg, plan=plan)


def test_graphs_this_library_does_not_execute_are_refused_by_step():
    # per-layer embedding steps out of their order
    e2b = graph_json("gemma-4-e2b-smoke.json")
    dec = [s for s in e2b["steps"] if s["phase"] == "decode"]
    dec[0], dec[1] = dec[1], dec[0]
    e2b["steps"] = [s for s in e2b["steps"] if s["phase"] == "prefill"] + dec
    with pytest.raises(ex.UnsupportedStep, match="ple_"):
        ex.plan_decode(ex.load_step_graph(e2b), 35)


def test_gemma4_e2b_graph_plans_per_layer():
    # gemma-4-e2b-smoke.json: 35 layers, layerPattern every 5 offset 4 (global
    # layers 4, 9, ..., 34 at globalHeadDim 512, the others sliding over 512
    # keys at headDim 256), the last 20 layers (15..34) sharing KV: a sliding
    # one reads the cache of layer 13 (the last sliding layer before 15), a
    # global one that of layer 14.
    g = ex.load_step_graph(GOLD / "gemma-4-e2b-smoke.json")
    mc = g.model_config
    plan = ex.plan_decode(g, mc["numLayers"], mc["headDim"], mc["globalHeadDim"])
    glob = {4, 9, 14, 19, 24, 29, 34}
    assert plan.windows == tuple(0 if i in glob else 512 for i in range(35))
    assert plan.head_dims == tuple(512 if i in glob else 256 for i in range(35))
    assert plan.kv_sources == tuple(range(15)) + tuple(14 if i in glob else 13 for i in range(15, 35))
    assert plan.ple.steps == ("ple_gather", "ple_project", "ple_norm", "ple_modulate")
    assert [d.kind for d in plan.layer] == ["qkv_rope_kv", "attention", "attn_out", "gate_up", "down"]
    # every decode step is carried out: the layer template, the PLE steps, the
    # variant steps (kv_write_shared, attention_global) and the sample
    covered = [n for d in plan.layer + plan.post + (plan.ple,) for n in d.steps]
    names = [s.name for s in g.phase("decode")]
    assert set(names) - set(covered) == {"kv_write_shared", "attention_global"}
    c = DecoderConfig.from_model_config(mc)
    assert (c.global_head_dim, c.ple_width, c.ple_vocab, c.ffn) == (512, 256, 262144, 6144)
    # a shared-KV count that leaves a type without an owner is an error
    e2b = graph_json("gemma-4-e2b-smoke.json")
    e2b["numKvSharedLayers"] = 31  # layers 4..34 shared: no earlier global layer owns a cache
    with pytest.raises(ex.StepGraphError, match="no earlier global layer"):
        ex.plan_decode(ex.load_step_graph(e2b), 35, 256, 512)


def test_golden_host_plans():
    # the reference's lowering goldens (runtime/zig/examples/doe-wgsl-host-plan.
    # *.json, checked at emit_csl_exec_v1_test.zig:352-447): launch lists with
    # attention type, window, decode-position source and KV alias, kernels in
    # order of first use with counts, EOS token.  The goldens name rmsnorm's
    # pattern "reduction"; the op table and its own test
    # (emit_csl_exec_v1_test.zig:8-17) map rmsnorm to "rms_norm", which is
    # followed here.  The PE grid is a Cerebras placement and not derived.
    for graph, golden in [("gemma-3-270m-smoke.json", "doe-wgsl-host-plan.gemma-3-270m-smoke.json"),
                          ("gemma-3-270m-manifest-smoke.json", "doe-wgsl-host-plan.gemma-3-270m-manifest-smoke.json"),
                          ("gemma-4-e2b-smoke.json", "doe-wgsl-host-plan.gemma-4-e2b-smoke.json")]:
        got = ex.lower_host_plan(ex.load_step_graph(GOLD / graph))
        want = graph_json("host_plan/" + golden)["hostPlan"]
        assert got["phases"] == want["phases"], graph
        assert got["eosTokenId"] == want["eosTokenId"]
        assert [(k["name"], k["count"]) for k in got["kernels"]] == [(k["name"], k["count"]) for k in want["kernels"]]
        for a, b in zip(got["kernels"], want["kernels"]):
            assert a["pattern"] == b["pattern"] or (a["name"], a["pattern"], b["pattern"]) == (
                "rmsnorm", "rms_norm", "reduction"), (graph, a, b)


def test_reference_shared_kv_and_validation_cases():
    # emit_csl_exec_v1_test.zig:268-299: shared KV launch metadata
    g = ex.load_step_graph({"grid": {"width": 8, "height": 1}, "slidingWindowSize": 512, "numKvSharedLayers": 4,
                            "steps": [
                                {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
                                {"phase": "decode", "op": "attention_sliding", "kernelKey": "attn_local",
                                 "attentionType": "sliding"},
                                {"phase": "decode", "op": "kv_write_shared", "kernelKey": "kv_shared",
                                 "kvCacheAlias": "layer.0.kv"},
                                {"phase": "decode", "op": "sample", "kernelKey": "sampler", "kind": "sample"}]})
    plan = ex.lower_host_plan(g)
    assert len(plan["kernels"]) == 4 and len(plan["phases"]["prefill"]) == 1
    d = plan["phases"]["decode"]
    assert len(d) == 3
    assert (d[0]["attentionType"], d[0]["slidingWindowSize"], d[0]["currentPosSource"]) == (
        "sliding", 512, "decode_position")
    assert d[1]["currentPosSource"] == "decode_position" and d[1]["kvCacheAlias"] == "layer.0.kv"
    # :301-320: kv_write_shared without numKvSharedLayers
    with pytest.raises(ex.StepGraphError, match="numKvSharedLayers"):
        ex.load_step_graph({"grid": {"width": 8, "height": 1}, "steps": [
            {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
            {"phase": "decode", "op": "kv_write_shared", "kernelKey": "kv_shared", "kvCacheAlias": "layer.0.kv"},
            {"phase": "decode", "op": "sample", "kernelKey": "sampler", "kind": "sample"}]})
    # :46-64, :82-110, :112-137: valid plans from steps, objects and tuples
    g = ex.load_step_graph({"grid": {"width": 16, "height": 2}, "eosTokenId": 7, "steps": [
        {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
        {"phase": "prefill", "op": "rmsnorm", "kernelKey": "norm_0"},
        {"phase": "decode", "op": "attention", "kernelKey": "attn_0"},
        {"phase": "decode", "op": "sample", "kernelKey": "sampler", "kind": "sample"}]})
    plan = ex.lower_host_plan(g)
    assert (len(plan["kernels"]), len(plan["phases"]["prefill"]), len(plan["phases"]["decode"]),
            plan["eosTokenId"]) == (4, 2, 2, 7)
    g = ex.load_step_graph({"grid": {"width": 8, "height": 1}, "steps": [
        ["prefill", "embed", "embed_gather"], ["decode", "attention", "attn_0"],
        ["decode", "sample", "sampler", None, "sample"]]})
    plan = ex.lower_host_plan(g)
    assert (len(plan["phases"]["prefill"]), len(plan["phases"]["decode"]), plan["eosTokenId"]) == (1, 2, None)
    # :197-229: layerPattern routing; both decode attention launches carry the
    # sliding/global type, the sliding one and kv_write read the decode position
    g = ex.load_step_graph({"grid": {"width": 8, "height": 1}, "slidingWindowSize": 512,
                            "layerPattern": {"type": "every_n", "period": 2, "offset": 1}, "steps": [
                                {"phase": "prefill", "op": "embed", "kernelKey": "embed_gather"},
                                {"phase": "decode", "op": "attention", "kernelKey": "attn_local"},
                                {"phase": "decode", "op": "kv_write", "kernelKey": "kv_write"},
                                {"phase": "decode", "op": "attention", "kernelKey": "attn_global"},
                                {"phase": "decode", "op": "sample", "kernelKey": "sampler", "kind": "sample"}]})
    d = ex.lower_host_plan(g)["phases"]["decode"]
    assert len(d) == 4
    assert (d[0]["attentionType"], d[0]["slidingWindowSize"], d[0]["currentPosSource"]) == (
        "sliding", 512, "decode_position")
    assert d[1]["currentPosSource"] == "decode_position"
    assert d[2]["attentionType"] == "global" and "slidingWindowSize" not in d[2]


def test_step_validation_rules():
    # emit_csl_exec_v1.zig:527-559 (validateStep), 335-389 (parseStepObject)
    base = [{"phase": "prefill", "op": "embed", "kernelKey": "e"}]
    tail = [{"phase": "decode", "op": "sample", "kernelKey": "s"}]

    def graph(*decode, **root):
        return {**root, "steps": base + list(decode) + tail}

    cases = [
        ({"phase": "decode", "op": "kv_write", "kernelKey": "k", "kvCacheAlias": "layer.0.kv"}, "kvCacheAlias"),
        ({"phase": "decode", "op": "kv_write_shared", "kernelKey": "k"}, "kvCacheAlias"),
        ({"phase": "decode", "op": "attention", "kernelKey": "a", "slidingWindowSize": 0}, "slidingWindowSize"),
        ({"phase": "decode", "op": "rmsnorm", "kernelKey": "n", "slidingWindowSize": 64}, "slidingWindowSize"),
        ({"phase": "decode", "op": "rmsnorm", "kernelKey": "n", "attentionType": "global"}, "attentionType"),
        ({"phase": "decode", "op": "attention_sliding", "kernelKey": "a", "attentionType": "global"},
         "attentionType"),
        ({"phase": "decode", "op": "rmsnorm", "kernelKey": "n", "repeat": 0}, "repeat"),
        ({"phase": "decode", "op": "gelu_gated", "kernelKey": "g"}, "inputsFrom"),
        ({"phase": "decode", "op": "gelu_gated", "kernelKey": "g", "inputsFrom": ["gate_proj"]}, "inputsFrom"),
    ]
    for step, msg in cases:
        with pytest.raises(ex.StepGraphError, match=msg):
            ex.load_step_graph(graph(step, numKvSharedLayers=4))
    with pytest.raises(ex.StepGraphError, match="weightsKey"):  # a sample step with weights
        ex.load_step_graph({"steps": base + [{"phase": "decode", "op": "sample", "kernelKey": "s",
                                               "weightsKey": "lm_head"}]})
    ok = ex.load_step_graph(graph({"phase": "decode", "op": "gelu_gated", "kernelKey": "g",
                                   "inputsFrom": ["gate_proj", "up_proj"], "repeat": 3}))
    assert ok.phase("decode")[0].repeat == 3 and ok.phase("decode")[0].inputs_from == ("gate_proj", "up_proj")
    # ordering (emit_csl_exec_v1.zig:683-706, 786-787)
    with pytest.raises(ex.StepGraphError, match="after a decode step"):
        ex.load_step_graph({"steps": base + tail + [{"phase": "prefill", "op": "rmsnorm", "kernelKey": "n"}]})
    with pytest.raises(ex.StepGraphError, match="sample step"):
        ex.load_step_graph({"steps": base + [{"phase": "decode", "op": "rmsnorm", "kernelKey": "n"}] + tail +
                            [{"phase": "decode", "op": "rmsnorm", "kernelKey": "n"}]})
    with pytest.raises(ex.StepGraphError, match="computes nothing"):
        ex.load_step_graph({"steps": base + tail})
    # the lm_head matmul lowers as dense_gemv, the 31B prefill GEMV as prefill_q4k_gemv
    g = ex.load_step_graph({"steps": [
        {"phase": "prefill", "op": "matmul", "kernelKey": "tiled_31b"},
        {"phase": "decode", "op": "matmul", "kernelKey": "lm_head_f16", "name": "lm_head"},
        {"phase": "decode", "op": "sample", "kernelKey": "s"}]})
    assert [k["pattern"] for k in ex.lower_host_plan(g)["kernels"]] == ["prefill_q4k_gemv", "dense_gemv", "sample"]


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
    # Gemma 4 fields: a global-layer head_dim and per-layer embeddings
    g4 = DecoderConfig.from_model_config({**mc, "globalHeadDim": 512, "pleWidth": 256, "pleVocabSize": 1000})
    assert (g4.global_head_dim, g4.ple_width, g4.ple_vocab) == (512, 256, 1000)


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


def test_gemma4_31b_graphs_plan_per_layer():
    # gemma-4-31b-smoke.json: 61 layers, layerPattern every 5 offset 4 (global
    # layers 4, 9, ..., 59), the others sliding over 512 keys, the last 4
    # layers (57..60) sharing KV: a sliding one reads layer 56's cache, the
    # global layer 59 that of layer 54; per-layer embeddings (pleWidth 256).
    g = ex.load_step_graph(GOLD / "gemma-4-31b-smoke.json")
    mc = g.model_config
    plan = ex.plan_decode(g, mc["numLayers"], mc["headDim"], mc.get("globalHeadDim"))
    assert len(plan.windows) == 61
    assert [i for i, w in enumerate(plan.windows) if w == 0] == list(range(4, 61, 5))
    assert all(w == 512 for i, w in enumerate(plan.windows) if i % 5 != 4)
    assert [(i, s) for i, s in enumerate(plan.kv_sources) if s != i] == [(57, 56), (58, 56), (59, 54), (60, 56)]
    assert plan.ple is not None
    # gemma-4-31b-af16-smoke.json lists only the sliding attention step: the
    # one-layer template repeats it in all 60 layers, none shares KV
    g16 = ex.load_step_graph(GOLD / "gemma-4-31b-af16-smoke.json")
    mc16 = g16.model_config
    plan16 = ex.plan_decode(g16, mc16["numLayers"], mc16["headDim"], mc16.get("globalHeadDim"))
    assert plan16.windows == (512,) * 60
    assert plan16.kv_sources in (None, (), tuple(range(60)))
    assert plan16.ple is None
