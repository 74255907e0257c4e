"""Execution-v1 step graphs (Doppler's ``doppler.execution/v1``) driving the
decode loop.

A step graph lists the per-token steps of a model: embed, per-layer norm /
projections / rope / attention / residual / FFN, final norm, lm_head, sample.
This module is the host-side counterpart of the reference's lowering
(runtime/zig/src/doe_wgsl/emit_csl_exec_v1.zig): it reads both graph forms,
checks every step against the op table, derives each decode layer's
attention type and window, and maps the decode phase onto the fused
dispatches ``doe_amd.model.Decoder.step`` issues.  A valid step this library
does not execute raises ``UnsupportedStep`` -- the reference's own policy
``unresolvedKernel: "error"`` -- rather than being skipped.

Graph forms (runtime/zig/examples/execution-v1/):
  * flat: ``{"steps": [{"name", "phase", "op", "kernelKey", "weightsKey"?,
    "attentionType"?, "slidingWindowSize"?}, ...]}`` plus optional
    ``slidingWindowSize``, ``layerPattern`` ``{"type": "every_n", "period",
    "offset"}``, ``numKvSharedLayers``, ``modelConfig`` (gemma-3-270m-smoke.json,
    gemma-4-e2b-smoke.json); a step may also be a tuple ``[phase, op,
    kernelKey, weightsKey?, kind?]``;
  * manifest: ``{"execution": {"kernels": {key: {"kernel": file}}, "preLayer",
    "prefill", "decode", "postLayer": [[name, kernelKey, weightsKey?], ...]}}``
    (gemma-3-270m-manifest-smoke.json): the op comes from the kernel file.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

# op -> (kernel pattern, allowed in prefill, allowed in decode, kind): the
# reference's op table (emit_csl_exec_v1.zig:114-177), used to reject unknown
# or misplaced ops and to lower a graph to its launch list.
_OPS = {
    "embed": ("gather", True, True, "compute"),
    "attention": ("attention_decode", False, True, "compute"),
    "attention_prefill": ("attention_tiled", True, False, "compute"),
    "attention_prefill_kv_axis_sharded": ("attention_prefill_kv_axis_sharded", True, False, "compute"),
    "conv1d_depthwise": ("conv1d_depthwise", True, True, "compute"),
    "l2_normalize": ("l2_normalize", True, True, "compute"),
    "linear_attention": ("linear_attention", True, True, "compute"),
    "attention_linear": ("attention_linear", True, True, "compute"),
    "rope": ("rope", True, True, "compute"),
    "rmsnorm": ("rms_norm", True, True, "compute"),
    "layernorm": ("reduction", True, True, "compute"),
    "softmax": ("reduction", True, True, "compute"),
    "gelu": ("gelu", True, True, "compute"),
    "silu": ("element_wise", True, True, "compute"),
    "gelu_gated": ("gelu_gated", True, True, "compute"),
    "silu_gated": ("silu_gated", True, True, "compute"),
    "sigmoid_gated": ("sigmoid_gated", True, True, "compute"),
    "o_gate": ("sigmoid_gated", True, True, "compute"),
    "relu": ("element_wise", True, True, "compute"),
    "scale": ("element_wise", True, True, "compute"),
    "bias_add": ("element_wise", True, True, "compute"),
    "residual": ("residual", True, True, "compute"),
    "cast": ("element_wise", True, True, "compute"),
    "dequant": ("dequant", True, True, "compute"),
    "matmul": ("tiled_matmul", True, True, "compute"),
    "matmul_q4k": ("fused_gemv_dequant", True, True, "compute"),
    "ffn": ("fused_ffn", True, True, "compute"),
    "kv_write": ("kv_write", True, True, "compute"),
    "kv_read": ("kv_read", True, True, "compute"),
    "sample": ("sample", True, True, "sample"),
    "ple_gather": ("gather", True, True, "compute"),
    "ple_project": ("tiled_matmul", True, True, "compute"),
    "ple_norm": ("reduction", True, True, "compute"),
    "ple_modulate": ("element_wise", True, True, "compute"),
    "attention_sliding": ("attention_decode", False, True, "compute"),
    "kv_write_shared": ("kv_write", True, True, "compute"),
}

# gate ops that take their two inputs from named earlier steps
# (emit_csl_exec_v1.zig:88-93; parseStepObject requires two inputsFrom)
_PAIRED_GATE_OPS = ("silu_gated", "sigmoid_gated", "gelu_gated", "o_gate")
# kernelKey of the 31B prefill Q4_K GEMV launches (emit_csl_exec_v1.zig:41, 605-607)
_PREFILL_Q4K_GEMV_KERNEL = "tiled_31b"
_PREFILL_Q4K_GEMV_PATTERN = "prefill_q4k_gemv"

# manifest form: kernel file -> op (emit_csl_exec_v1.zig:425-437)
_KERNEL_FILE_OPS = {
    "gather.wgsl": "embed",
    "rmsnorm.wgsl": "rmsnorm",
    "rope.wgsl": "rope",
    "residual.wgsl": "residual",
    "gelu.wgsl": "gelu",
    "sample.wgsl": "sample",
    "attention_decode_online_f16kv.wgsl": "attention",
    "attention_small_f16kv.wgsl": "attention_prefill",
    "matmul_f16w_f32a_tiled.wgsl": "matmul",
    "matmul_gemv_subgroup.wgsl": "matmul_q4k",
}


class StepGraphError(ValueError):
    """A malformed step graph (the reference's InvalidJson / UnknownOp /
    MalformedStep)."""


class UnsupportedStep(StepGraphError):
    """A valid step that this library does not execute."""


@dataclass(frozen=True)
class Step:
    phase: str
    op: str
    kernel_key: str
    name: str | None = None
    weights_key: str | None = None
    attention_type: str | None = None  # "global" | "sliding"
    sliding_window: int | None = None
    kv_cache_alias: str | None = None  # kv_write_shared: the cache it writes (another layer's)
    kind: str = "compute"
    repeat: int = 1
    inputs_from: tuple[str, ...] | None = None

    @property
    def pattern(self) -> str:
        """The kernel pattern of this launch (emit_csl_exec_v1.zig:589-607,
        stepPattern): the op's pattern, except tiled_matmul steps that are the
        31B prefill Q4_K GEMV or the lm_head (dense_gemv)."""
        pat = _OPS[self.op][0]
        if pat == "tiled_matmul":
            if self.phase == "prefill" and self.kernel_key == _PREFILL_Q4K_GEMV_KERNEL:
                return _PREFILL_Q4K_GEMV_PATTERN
            if _is_lm_head_name(self.name) or _is_lm_head_kernel(self.kernel_key) or self.weights_key == "lm_head":
                return "dense_gemv"
        return pat

    def label(self) -> str:
        return f"{self.phase} step {self.name or self.op!r} (op {self.op}, kernel {self.kernel_key})"


@dataclass(frozen=True)
class StepGraph:
    steps: tuple[Step, ...]
    model_family: str | None = None
    model_id: str | None = None
    eos_token_id: int | None = None
    sliding_window: int | None = None
    layer_pattern: tuple[int, int] | None = None  # (period, offset): layer i is global iff i % period == offset
    num_kv_shared_layers: int | None = None
    model_config: dict | None = None

    def phase(self, phase: str) -> list[Step]:
        return [s for s in self.steps if s.phase == phase]


def _u32(value, what: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or not 0 <= value < 2 ** 32:
        raise StepGraphError(f"{what} must be a u32 (got {value!r})")
    return value


def _opt_str(value, what: str) -> str | None:
    if value is None:
        return None
    if not isinstance(value, str) or not value:
        raise StepGraphError(f"{what} must be a non-empty string (got {value!r})")
    return value


def _is_lm_head_name(name) -> bool:
    return isinstance(name, str) and (name in ("lm_head", "lm_head_prefill") or name.startswith("lm_head_"))


def _is_lm_head_kernel(key) -> bool:
    return isinstance(key, str) and (key == "lm_head" or key.startswith("lm_head_"))


def _make_step(phase, op, kernel_key, *, name=None, weights_key=None, kind=None, attention_type=None,
               sliding_window=None, kv_cache_alias=None, repeat=None, inputs_from=None) -> Step:
    """One validated step (emit_csl_exec_v1.zig:335-389 parseStepObject and
    :527-559 validateStep)."""
    if phase not in ("prefill", "decode"):
        raise StepGraphError(f"unknown phase {phase!r}")
    if not isinstance(op, str) or op not in _OPS:
        raise StepGraphError(f"unknown op {op!r}")
    label = name or op
    if not isinstance(kernel_key, str) or not kernel_key:
        raise StepGraphError(f"step {label!r}: empty kernelKey")
    pattern, allow_prefill, allow_decode, op_kind = _OPS[op]
    if kind is not None and kind not in ("compute", "sample"):
        raise StepGraphError(f"step {label!r}: kind {kind!r}")
    if kind is not None and kind != op_kind:
        raise StepGraphError(f"step {label!r}: kind {kind!r} does not match op {op!r}")
    if (phase == "prefill" and not allow_prefill) or (phase == "decode" and not allow_decode):
        raise StepGraphError(f"step {label!r}: op {op!r} is not allowed in {phase}")
    weights_key = _opt_str(weights_key, "weightsKey")
    if op_kind == "sample" and weights_key is not None:
        raise StepGraphError(f"step {label!r}: a sample step takes no weightsKey")
    if attention_type is not None and attention_type not in ("global", "sliding"):
        raise StepGraphError(f"step {label!r}: attentionType {attention_type!r}")
    if attention_type is not None and pattern != "attention_decode":
        raise StepGraphError(f"step {label!r}: attentionType on op {op!r}, which is not decode attention")
    if sliding_window is not None:
        sliding_window = _u32(sliding_window, "slidingWindowSize")
        if sliding_window == 0 or pattern != "attention_decode":
            raise StepGraphError(f"step {label!r}: slidingWindowSize {sliding_window} on op {op!r}")
    if op == "attention_sliding" and attention_type not in (None, "sliding"):
        raise StepGraphError(f"step {label!r}: attention_sliding with attentionType {attention_type!r}")
    kv_cache_alias = _opt_str(kv_cache_alias, "kvCacheAlias")
    if (op == "kv_write_shared") != (kv_cache_alias is not None):
        raise StepGraphError(f"step {label!r}: kvCacheAlias belongs to kv_write_shared steps and they need one")
    repeat = 1 if repeat is None else _u32(repeat, "repeat")
    if repeat == 0:
        raise StepGraphError(f"step {label!r}: repeat 0")
    if inputs_from is not None:
        if not isinstance(inputs_from, list) or not inputs_from or not all(
                isinstance(v, str) for v in inputs_from):
            raise StepGraphError(f"step {label!r}: inputsFrom must be a non-empty list of step names")
        inputs_from = tuple(inputs_from)
    if op in _PAIRED_GATE_OPS and (inputs_from is None or len(inputs_from) != 2):
        raise StepGraphError(f"step {label!r}: op {op!r} needs inputsFrom with two step names")
    return Step(phase, op, kernel_key, _opt_str(name, "name"), weights_key, attention_type, sliding_window,
                kv_cache_alias, op_kind, repeat, inputs_from)


def _flat_step(value) -> Step:
    if isinstance(value, dict):
        for key in ("phase", "op", "kernelKey"):
            if key not in value:
                raise StepGraphError(f"step {value.get('name')!r} lacks {key!r}")
        return _make_step(value["phase"], value["op"], value["kernelKey"], name=value.get("name"),
                          weights_key=value.get("weightsKey"), kind=value.get("kind"),
                          attention_type=value.get("attentionType"), sliding_window=value.get("slidingWindowSize"),
                          kv_cache_alias=value.get("kvCacheAlias"), repeat=value.get("repeat"),
                          inputs_from=value.get("inputsFrom"))
    if isinstance(value, list):
        if not 3 <= len(value) <= 5:
            raise StepGraphError(f"step tuple of length {len(value)}")
        return _make_step(value[0], value[1], value[2], weights_key=value[3] if len(value) > 3 else None,
                          kind=value[4] if len(value) > 4 else None)
    raise StepGraphError(f"step must be an object or a tuple (got {type(value).__name__})")


def _manifest_steps(execution: dict) -> list[Step]:
    kernels = execution.get("kernels")
    if not isinstance(kernels, dict):
        raise StepGraphError("execution.kernels missing")
    kernel_ops = {}
    for key, meta in kernels.items():
        kfile = meta.get("kernel") if isinstance(meta, dict) else None
        if kfile not in _KERNEL_FILE_OPS:
            raise StepGraphError(f"kernel {key!r}: unknown kernel file {kfile!r}")
        kernel_ops[key] = _KERNEL_FILE_OPS[kfile]

    def tup(phase, value) -> Step:
        if not isinstance(value, list) or not 2 <= len(value) <= 3:
            raise StepGraphError(f"manifest step {value!r}")
        name, kernel_key = value[0], value[1]
        if kernel_key not in kernel_ops:
            raise StepGraphError(f"manifest step {name!r}: unknown kernel key {kernel_key!r}")
        return _make_step(phase, kernel_ops[kernel_key], kernel_key, name=name,
                          weights_key=value[2] if len(value) == 3 else None)

    for key in ("preLayer", "prefill", "decode", "postLayer"):
        if not isinstance(execution.get(key), list):
            raise StepGraphError(f"execution.{key} missing")
    prefill = [tup("prefill", v) for v in execution["preLayer"] + execution["prefill"]]
    decode = [tup("decode", v) for v in execution["decode"]]
    for v in execution["postLayer"]:
        name = v[0] if isinstance(v, list) and v else None
        # sample and lm_head belong to decode, *_prefill to prefill, the rest to both
        if name in ("sample", "lm_head"):
            decode.append(tup("decode", v))
        elif isinstance(name, str) and name.endswith("_prefill"):
            prefill.append(tup("prefill", v))
        else:
            prefill.append(tup("prefill", v))
            decode.append(tup("decode", v))
    return prefill + decode


def _check_phase_order(steps) -> None:
    """The lowering's ordering rules (emit_csl_exec_v1.zig:683-706, 786-787):
    every prefill step before every decode step, decode only after a prefill
    step, nothing after a phase's sample step, and a decode phase that
    computes something.  (That lowering also rejects a sample whose previous
    step is no logits producer, :689-698; the reference's own tests and golden
    host plans -- emit_csl_exec_v1_test.zig:268-300, 418-447 and
    doe-wgsl-host-plan.gemma-4-e2b-smoke.json, sample after attn_decode --
    expect those graphs to lower, so that rule is not applied here.)"""
    saw = {"prefill": False, "decode": False}
    closed = {"prefill": False, "decode": False}
    decode_compute = False
    for st in steps:
        if st.phase == "prefill" and saw["decode"]:
            raise StepGraphError(f"{st.label()} comes after a decode step")
        if st.phase == "decode" and not saw["prefill"]:
            raise StepGraphError(f"{st.label()} comes before any prefill step")
        if closed[st.phase]:
            raise StepGraphError(f"{st.label()} comes after the {st.phase} phase's sample step")
        saw[st.phase] = True
        if st.kind == "sample":
            closed[st.phase] = True
        elif st.phase == "decode":
            decode_compute = True
    if saw["decode"] and not decode_compute:
        raise StepGraphError("the decode phase computes nothing")


def load_step_graph(src) -> StepGraph:
    """A StepGraph from a path, a JSON string or an already-parsed dict."""
    if isinstance(src, dict):
        root = src
    else:
        text = Path(src).read_text() if isinstance(src, Path) or not str(src).lstrip().startswith("{") else src
        try:
            root = json.loads(text)
        except json.JSONDecodeError as e:
            raise StepGraphError(f"not JSON: {e}") from None
    if not isinstance(root, dict):
        raise StepGraphError("step graph must be a JSON object")
    if isinstance(root.get("execution"), dict):
        steps = _manifest_steps(root["execution"])
    elif isinstance(root.get("steps"), list):
        steps = [_flat_step(v) for v in root["steps"]]
    else:
        raise StepGraphError("step graph has neither 'execution' nor 'steps'")
    _check_phase_order(steps)
    pattern = None
    if root.get("layerPattern") is not None:
        lp = root["layerPattern"]
        if not isinstance(lp, dict) or lp.get("type") != "every_n":
            raise StepGraphError(f"layerPattern {lp!r}: only every_n is defined")
        period, offset = _u32(lp.get("period"), "layerPattern.period"), _u32(lp.get("offset"), "layerPattern.offset")
        if period == 0:
            raise StepGraphError("layerPattern.period is 0")
        pattern = (period, offset)
    sw = root.get("slidingWindowSize")
    shared = root.get("numKvSharedLayers")
    if any(st.op == "kv_write_shared" for st in steps) and not shared:
        # emit_csl_exec_v1.zig:720-723: an aliased cache write needs the
        # graph's shared-KV metadata
        raise StepGraphError("kv_write_shared step without numKvSharedLayers")
    eos = root.get("eosTokenId")
    return StepGraph(tuple(steps), root.get("modelFamily"), root.get("modelId"),
                     None if eos is None else _u32(eos, "eosTokenId"),
                     None if sw is None else _u32(sw, "slidingWindowSize"), pattern,
                     None if shared is None else _u32(shared, "numKvSharedLayers"), root.get("modelConfig"))


def _attention_type(graph: StepGraph, step: Step, layer_index: int | None) -> str | None:
    """emit_csl_exec_v1.zig:616-634 (deriveLaunchAttentionType): the op, then
    the step's attentionType, then layerPattern for the decode attention step
    of layer `layer_index`."""
    if step.op == "attention_sliding":
        return "sliding"
    if step.attention_type is not None:
        return step.attention_type
    if layer_index is not None and graph.layer_pattern is not None:
        period, offset = graph.layer_pattern
        return "global" if layer_index % period == offset else "sliding"
    return None


def _sliding_window(graph: StepGraph, step: Step, attention_type: str | None) -> int | None:
    """emit_csl_exec_v1.zig:637-642: the step's window, else the graph's."""
    if attention_type != "sliding":
        return None
    w = step.sliding_window if step.sliding_window is not None else graph.sliding_window
    if not w:
        raise StepGraphError(f"{step.label()}: sliding attention without slidingWindowSize")
    return w


def lower_host_plan(graph: StepGraph) -> dict:
    """The graph's launch list as the reference lowers it (lowerToHostPlan,
    emit_csl_exec_v1.zig:651-797), in its host-plan JSON form: the kernels in
    order of first use with the first step's pattern and the summed repeats,
    and per phase one launch per step with its attention type, sliding window,
    decode-position source and KV-cache alias.  (The PE grid is a Cerebras
    placement and is not derived.)"""
    kernels: dict[str, dict] = {}
    phases: dict[str, list] = {"prefill": [], "decode": []}
    attn_index = 0
    for st in graph.steps:
        pattern = st.pattern
        layer_index = None
        if st.phase == "decode" and pattern == "attention_decode":
            layer_index = attn_index
            attn_index += 1
        atype = _attention_type(graph, st, layer_index)
        window = _sliding_window(graph, st, atype)
        k = kernels.get(st.kernel_key)
        if k is None:
            kernels[st.kernel_key] = {"name": st.kernel_key, "pattern": pattern, "count": st.repeat}
        else:
            k["count"] += st.repeat
        launch = {"kernelName": st.kernel_key, "repeat": st.repeat}
        if atype is not None:
            launch["attentionType"] = atype
        if window is not None:
            launch["slidingWindowSize"] = window
        if atype == "sliding" or (st.phase == "decode" and pattern == "kv_write"):
            launch["currentPosSource"] = "decode_position"
        if st.kv_cache_alias is not None:
            launch["kvCacheAlias"] = st.kv_cache_alias
        phases[st.phase].append(launch)
    return {"kernels": list(kernels.values()), "phases": phases, "eosTokenId": graph.eos_token_id}


# ---------------------------------------------------------------------------
# Decode plan: the graph's decode phase on Decoder.step's fused dispatches.
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Dispatch:
    kind: str               # qkv_rope_kv | attention | attn_out | gate_up | down | lm_head_sample
    steps: tuple[str, ...]  # the graph steps it carries out


@dataclass(frozen=True)
class DecodePlan:
    layer: tuple[Dispatch, ...]  # one layer's dispatches (the same for every layer)
    post: tuple[Dispatch, ...]
    windows: tuple[int, ...]     # per layer: 0 = global attention, else the sliding window
    eos_token_id: int | None
    # per layer: head_dim (a global layer may use the model's globalHeadDim);
    # None = the model's head_dim in every layer
    head_dims: tuple[int, ...] | None = None
    # per layer: the layer whose KV cache its attention reads (itself, or for
    # a shared-KV layer the last earlier non-shared layer of the same
    # attention type); None = every layer its own
    kv_sources: tuple[int, ...] | None = None
    # the per-layer-embedding steps before the layers (ple_gather, ple_project,
    # ple_norm, ple_modulate), None when the graph has none
    ple: Dispatch | None = None
    # hybrid graphs (qwen-3-6-27b-smoke.json): per layer "attention" or
    # "linear_attention", and the linear-attention layers' steps (input_norm,
    # conv1d_depthwise, l2_normalize x 2, linear_attention); None = every
    # layer an attention layer
    layer_types: tuple[str, ...] | None = None
    linear: Dispatch | None = None


# One decoder layer: groups of ops, each group one fused dispatch.  Within a
# group, ops in a set may come in any order; "?" marks an optional op.
_LAYER = (
    ("qkv_rope_kv", ("rmsnorm", {"matmul_q4k": 3}, {"rope": 2}, "kv_write?")),
    ("attention", (("attention", "attention_sliding"),)),
    ("attn_out", ("matmul_q4k", "residual")),
    ("gate_up", ("rmsnorm", {"matmul_q4k": 2}, ("gelu", "gelu_gated"))),
    ("down", ("matmul_q4k", "residual")),
)


# The gated-attention layer of qwen-3-6-27b-smoke.json: q/k RMSNorms after the
# projections (queryKeyNorm), the attention output gate (o_gate: the
# attention output times sigmoid of q_proj's gate half, inputsFrom [q_proj,
# attention]) before o_proj, and a SwiGLU FFN (silu_gated).
_LAYER_GATED = (
    ("qkv_norm_rope_kv", ("rmsnorm", {"matmul_q4k": 3}, {"rmsnorm": 2}, {"rope": 2}, "kv_write?")),
    ("attention", (("attention", "attention_sliding"),)),
    ("gated_attn_out", ("o_gate", "matmul_q4k", "residual")),
    ("gate_up", ("rmsnorm", {"matmul_q4k": 2}, ("gelu", "gelu_gated", "silu_gated"))),
    ("down", ("matmul_q4k", "residual")),
)

# The linear-attention (gated DeltaNet) layer body of a hybrid graph, each
# op repeated once per such layer (repeat = their count).
_LINEAR_BODY = ("conv1d_depthwise", "l2_normalize", "l2_normalize", "linear_attention")


def _take_layer(steps: list[Step], i: int, layer=_LAYER) -> tuple[list[Dispatch], Step, int]:
    """Matches one layer starting at steps[i]; returns its dispatches, its
    attention step and the index after it."""
    out, attn = [], None
    for kind, pattern in layer:
        names = []
        for item in pattern:
            if isinstance(item, dict):  # ops in any order
                want = dict(item)
                while any(want.values()):
                    if i >= len(steps) or want.get(steps[i].op, 0) == 0:
                        got = steps[i].label() if i < len(steps) else "the end of the decode phase"
                        raise UnsupportedStep(f"{kind}: expected {sorted(k for k, v in want.items() if v)}, got {got}")
                    want[steps[i].op] -= 1
                    names.append(steps[i].name or steps[i].op)
                    i += 1
                continue
            opts = item if isinstance(item, tuple) else (item,)
            optional = isinstance(item, str) and item.endswith("?")
            opts = tuple(o.rstrip("?") for o in opts)
            if i < len(steps) and steps[i].op in opts:
                if kind == "attention":
                    attn = steps[i]
                names.append(steps[i].name or steps[i].op)
                i += 1
            elif not optional:
                got = steps[i].label() if i < len(steps) else "the end of the decode phase"
                raise UnsupportedStep(f"{kind}: expected {'/'.join(opts)}, got {got}")
        out.append(Dispatch(kind, tuple(names)))
    return out, attn, i


def _window(graph: StepGraph, attn: Step, layer: int) -> int:
    """0 for global attention, else the sliding window (emit_csl_exec_v1.zig:
    612-641: the op, then the step's attentionType, then layerPattern)."""
    if attn.op == "attention_sliding":
        kind = "sliding"
    elif attn.attention_type is not None:
        kind = attn.attention_type
    elif graph.layer_pattern is not None:
        period, offset = graph.layer_pattern
        kind = "global" if layer % period == offset else "sliding"
    else:
        kind = "global"
    if kind == "global":
        return 0
    w = attn.sliding_window if attn.sliding_window is not None else graph.sliding_window
    if not w:
        raise StepGraphError(f"layer {layer}: sliding attention without slidingWindowSize")
    return w


_PLE_STEPS = ("ple_gather", "ple_project", "ple_norm", "ple_modulate")


def plan_decode(graph: StepGraph, num_layers: int, head_dim: int | None = None,
                global_head_dim: int | None = None) -> DecodePlan:
    """The decode phase as Decoder.step's dispatches.  The graph lists either
    one layer (a template repeated num_layers times) or every layer.

    A one-layer template may be followed by variant steps for the layers the
    graph's metadata routes elsewhere (gemma-4-e2b-smoke.json): an attention
    step of the other type (the layerPattern's global layers; with a
    globalHeadDim they use that head_dim) and ``kv_write_shared`` (the last
    numKvSharedLayers layers write no cache of their own: their attention
    reads the cache of the last earlier non-shared layer of the same type).
    With both attention types listed the layerPattern decides each layer's
    type (emit_csl_exec_v1.zig:612-634)."""
    steps = graph.phase("decode")
    if not steps or steps[-1].op != "sample":
        raise StepGraphError("the decode phase must end with a sample step")
    # the post-layer tail: [final norm], [lm_head], sample
    j = len(steps) - 1
    post = ["sample"]
    if j > 0 and (steps[j - 1].weights_key == "lm_head" or steps[j - 1].name == "lm_head"):
        j -= 1
        post.insert(0, steps[j].name or steps[j].op)
    if j > 0 and steps[j - 1].op == "rmsnorm" and (steps[j - 1].name or "").startswith("final"):
        j -= 1
        post.insert(0, steps[j].name or steps[j].op)
    body = steps[:j]
    if body and body[0].op == "embed":  # the token embedding, done before the layers
        body = body[1:]
    ple = None
    if body and body[0].op == "ple_gather":
        ops_ = tuple(st.op for st in body[:4])
        if ops_ != _PLE_STEPS:
            raise UnsupportedStep(f"per-layer embedding steps {ops_}, expected {_PLE_STEPS}")
        ple = Dispatch("ple", tuple(st.name or st.op for st in body[:4]))
        body = body[4:]
    # a hybrid graph: input_norm, then the linear-attention body (each op
    # `repeat` times), then the attention layer, which starts from the same
    # input_norm
    body = list(body)
    linear, n_linear = None, 0
    if len(body) > 5 and body[0].op == "rmsnorm" and tuple(st.op for st in body[1:5]) == _LINEAR_BODY:
        reps = {st.repeat for st in body[1:5]}
        if len(reps) != 1:
            raise StepGraphError(f"linear-attention body steps repeat {sorted(reps)} times, not equally")
        n_linear = reps.pop()
        linear = Dispatch("linear_attention_layer", tuple(st.name or st.op for st in body[:5]))
        body = body[:1] + body[5:]
    # trailing variant steps of a one-layer template
    variants = []
    while body and body[-1].op in ("kv_write_shared", "attention", "attention_sliding"):
        variants.insert(0, body.pop())
    layer_pattern = _LAYER_GATED if any(st.op == "o_gate" for st in body) else _LAYER
    layers, attns, i = [], [], 0
    while i < len(body):
        disp, attn, i = _take_layer(body, i, layer_pattern)
        layers.append(disp)
        attns.append(attn)
    if not layers:
        raise StepGraphError("the decode phase has no layer")
    if variants and len(layers) != 1:
        raise UnsupportedStep("variant steps after a graph that lists more than one layer")
    shared_listed = any(v.op == "kv_write_shared" for v in variants)
    if shared_listed and not graph.num_kv_shared_layers:
        raise StepGraphError("kv_write_shared step without numKvSharedLayers")
    var_attn = [v for v in variants if v.op != "kv_write_shared"]
    layer_types = None
    if linear is not None:
        # n_linear linear-attention layers and one full-attention layer closing
        # each group of `period` (the Qwen3-Next layout, layer_types
        # [linear_attention] * (period - 1) + [full_attention] repeated: 16
        # attention and 48 linear layers of 64 at period 4; the reference's
        # frozen Qwen 3.6 activations of layer 3 are those of an attention
        # layer, bench/fixtures/r3-2-27b-doppler-frozen-af16/layer_3)
        n_attn = num_layers - n_linear
        if len(layers) != 1 or n_attn <= 0 or num_layers % n_attn:
            raise StepGraphError(f"{n_linear} linear-attention layers of {num_layers} do not tile into groups")
        period = num_layers // n_attn
        layer_types = tuple("attention" if li % period == period - 1 else "linear_attention"
                            for li in range(num_layers))
    if len(layers) == 1:
        attns = attns * num_layers
    elif len(layers) != num_layers:
        raise StepGraphError(f"the decode phase lists {len(layers)} layers, the model has {num_layers}")
    elif any(tuple(d.kind for d in L) != tuple(d.kind for d in layers[0]) for L in layers):
        raise UnsupportedStep("layers of different structure")
    kinds = {_attention_type(graph, a, None) or "global" for a in [attns[0], *var_attn]}
    if var_attn and kinds == {"global", "sliding"}:
        if graph.layer_pattern is None:
            raise StepGraphError("sliding and global attention steps without a layerPattern")
        period, offset = graph.layer_pattern
        sliding_step = next(a for a in [attns[0], *var_attn] if _attention_type(graph, a, None) == "sliding")
        types = ["global" if li % period == offset else "sliding" for li in range(num_layers)]
        windows = tuple(0 if t == "global" else _window(graph, sliding_step, li) for li, t in enumerate(types))
    else:
        windows = tuple(_window(graph, attns[li], li) for li in range(num_layers))
        types = ["global" if w == 0 else "sliding" for w in windows]
    head_dims = None
    if head_dim is not None and global_head_dim and global_head_dim != head_dim:
        head_dims = tuple(global_head_dim if t == "global" else head_dim for t in types)
    kv_sources = None
    n_shared = graph.num_kv_shared_layers or 0
    if n_shared:
        if n_shared >= num_layers:
            raise StepGraphError(f"numKvSharedLayers {n_shared} leaves no layer that owns a KV cache")
        first = num_layers - n_shared
        src = []
        for li in range(num_layers):
            if li < first:
                src.append(li)
                continue
            owners = [o for o in range(first) if types[o] == types[li]]
            if not owners:
                raise StepGraphError(f"shared-KV layer {li} ({types[li]}) has no earlier {types[li]} layer")
            src.append(owners[-1])
        kv_sources = tuple(src)
    return DecodePlan(tuple(layers[0]), (Dispatch("lm_head_sample", tuple(post)),), windows, graph.eos_token_id,
                      head_dims, kv_sources, ple, layer_types, linear)
