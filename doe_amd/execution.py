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

# op -> (allowed in prefill, allowed in decode, kind): the reference's op
# table (emit_csl_exec_v1.zig:114-160), used to reject unknown or misplaced ops.
_OPS = {
    "embed": (True, True, "compute"),
    "attention": (False, True, "compute"),
    "attention_prefill": (True, False, "compute"),
    "attention_prefill_kv_axis_sharded": (True, False, "compute"),
    "attention_sliding": (False, True, "compute"),
    "conv1d_depthwise": (True, True, "compute"),
    "l2_normalize": (True, True, "compute"),
    "linear_attention": (True, True, "compute"),
    "attention_linear": (True, True, "compute"),
    "rope": (True, True, "compute"),
    "rmsnorm": (True, True, "compute"),
    "layernorm": (True, True, "compute"),
    "softmax": (True, True, "compute"),
    "gelu": (True, True, "compute"),
    "silu": (True, True, "compute"),
    "gelu_gated": (True, True, "compute"),
    "silu_gated": (True, True, "compute"),
    "sigmoid_gated": (True, True, "compute"),
    "o_gate": (True, True, "compute"),
    "relu": (True, True, "compute"),
    "scale": (True, True, "compute"),
    "bias_add": (True, True, "compute"),
    "residual": (True, True, "compute"),
    "cast": (True, True, "compute"),
    "dequant": (True, True, "compute"),
    "matmul": (True, True, "compute"),
    "matmul_q4k": (True, True, "compute"),
    "ffn": (True, True, "compute"),
    "kv_write": (True, True, "compute"),
    "kv_write_shared": (True, True, "compute"),
    "kv_read": (True, True, "compute"),
    "sample": (True, True, "sample"),
    "ple_gather": (True, True, "compute"),
    "ple_project": (True, True, "compute"),
    "ple_norm": (True, True, "compute"),
    "ple_modulate": (True, True, "compute"),
}

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


def _make_step(phase, op, kernel_key, *, name=None, weights_key=None, kind=None, attention_type=None,
               sliding_window=None) -> Step:
    if phase not in ("prefill", "decode"):
        raise StepGraphError(f"unknown phase {phase!r}")
    if not isinstance(op, str) or op not in _OPS:
        raise StepGraphError(f"unknown op {op!r}")
    if not isinstance(kernel_key, str) or not kernel_key:
        raise StepGraphError(f"step {name or op!r}: empty kernelKey")
    allow_prefill, allow_decode, op_kind = _OPS[op]
    if kind is not None and kind != op_kind:
        raise StepGraphError(f"step {name or op!r}: kind {kind!r} does not match op {op!r}")
    if (phase == "prefill" and not allow_prefill) or (phase == "decode" and not allow_decode):
        raise StepGraphError(f"step {name or op!r}: op {op!r} is not allowed in {phase}")
    if attention_type is not None and attention_type not in ("global", "sliding"):
        raise StepGraphError(f"step {name or op!r}: attentionType {attention_type!r}")
    if sliding_window is not None:
        sliding_window = _u32(sliding_window, "slidingWindowSize")
    return Step(phase, op, kernel_key, _opt_str(name, "name"), _opt_str(weights_key, "weightsKey"), attention_type,
                sliding_window)


def _flat_step(value) -> Step:
    if isinstance(value, dict):
        for key in ("phase", "op", "kernelKey"):
            if key not in value:
                raise StepGraphError(f"step {value.get('name')!r} lacks {key!r}")
        return _make_step(value["phase"], value["op"], value["kernelKey"], name=value.get("name"),
                          weights_key=value.get("weightsKey"), kind=value.get("kind"),
                          attention_type=value.get("attentionType"), sliding_window=value.get("slidingWindowSize"))
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
    # a decode step needs a prefill step before it (the reference lowering's
    # MalformedStep for a decode-first list)
    first_prefill = next((i for i, st in enumerate(steps) if st.phase == "prefill"), None)
    first_decode = next((i for i, st in enumerate(steps) if st.phase == "decode"), None)
    if first_decode is not None and (first_prefill is None or first_decode < first_prefill):
        raise StepGraphError(f"{steps[first_decode].label()} comes before any prefill step")
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
    eos = root.get("eosTokenId")
    return StepGraph(tuple(steps), root.get("modelFamily"), root.get("modelId"),
                     None if eos is None else _u32(eos, "eosTokenId"),
                     None if sw is None else _u32(sw, "slidingWindowSize"), pattern,
                     None if shared is None else _u32(shared, "numKvSharedLayers"), root.get("modelConfig"))


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


# One decoder layer: groups of ops, each group one fused dispatch.  Within a
# group, ops in a set may come in any order; "?" marks an optional op.
_LAYER = (
    ("qkv_rope_kv", ("rmsnorm", {"matmul_q4k": 3}, {"rope": 2}, "kv_write?")),
    ("attention", (("attention", "attention_sliding"),)),
    ("attn_out", ("matmul_q4k", "residual")),
    ("gate_up", ("rmsnorm", {"matmul_q4k": 2}, ("gelu", "gelu_gated"))),
    ("down", ("matmul_q4k", "residual")),
)


def _take_layer(steps: list[Step], i: int) -> tuple[list[Dispatch], Step, int]:
    """Matches one layer starting at steps[i]; returns its dispatches, its
    attention step and the index after it."""
    out, attn = [], None
    for kind, pattern in _LAYER:
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


def plan_decode(graph: StepGraph, num_layers: int) -> DecodePlan:
    """The decode phase as Decoder.step's dispatches.  The graph lists either
    one layer (a template repeated num_layers times) or every layer."""
    if graph.num_kv_shared_layers:
        raise UnsupportedStep(f"numKvSharedLayers {graph.num_kv_shared_layers}: shared KV layers")
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
    layers, attns, i = [], [], 0
    while i < len(body):
        disp, attn, i = _take_layer(body, i)
        layers.append(disp)
        attns.append(attn)
    if not layers:
        raise StepGraphError("the decode phase has no layer")
    if len(layers) == 1:
        attns = attns * num_layers
    elif len(layers) != num_layers:
        raise StepGraphError(f"the decode phase lists {len(layers)} layers, the model has {num_layers}")
    elif any(tuple(d.kind for d in L) != tuple(d.kind for d in layers[0]) for L in layers):
        raise UnsupportedStep("layers of different structure")
    windows = tuple(_window(graph, attns[li], li) for li in range(num_layers))
    return DecodePlan(tuple(layers[0]), (Dispatch("lm_head_sample", tuple(post)),), windows, graph.eos_token_id)
