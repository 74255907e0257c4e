"""A Gemma-style decoder driven through the C ABI: the 2B-class decode loop.

Step order follows the reference's execution-v1 decode step list
(runtime/zig/examples/execution-v1/gemma-3-270m-smoke.json: embed;
per layer input_norm, q/k/v_proj, rope_q/rope_k, attention, o_proj,
attn_residual, post_attn_norm, gate/up_proj, activation (GeGLU), down_proj,
ffn_residual; final norm, lm_head, sample).  On the MI355X the neighbouring
steps are fused into the Q4_K GEMVs (a kernel boundary costs ~1.8 us here,
an in-kernel grid barrier more), five dispatches per layer:

  1. qkv   = Wqkv . rmsnorm(x), RoPE on q/k, k and v stored into the f16
             caches at pos              (q/k rows interleaved rotation pairs)
  2. attention(q, K cache, V cache, kv_len = pos + 1) as split partials
  3. x     = Wo . combine(partials) + x   (the split combine folded into the
                                           GEMV's activation load; residual
                                           epilogue)
  4. h     = gelu(Wg . n) * (Wu . n), n = rmsnorm(x)   (gate/up rows
             interleaved, GeGLU epilogue)
  5. x     = Wd . h + x                   (residual epilogue)

then the lm_head over rmsnorm(x) with per-workgroup argmax partials, and an
on-device advance that reduces them to the token and moves (pos, kv_len,
next token).  The whole step is captured once into a HIP graph and replayed;
nothing returns to the host until generation ends.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _lib, ops
from . import q4k as _q4k
from . import q8_0 as _q8_0
from .device import DeviceBuffer, Event, Graph, Stream, _stream_ptr


@dataclass(frozen=True)
class DecoderConfig:
    layers: int = 26
    hidden: int = 2304
    heads: int = 8
    kv_heads: int = 4
    head_dim: int = 256
    ffn: int = 9216
    vocab: int = 256000
    eps: float = 1e-6
    rope_base: float = 10000.0
    max_seq: int = 384
    embed_scale: float = 1.0
    attn_softcap: float = 0.0  # > 0: scores s -> softcap * tanh(s / softcap) (attention_head256_f16kv.wgsl:197-199)
    # projection weights: "q4k" (Q4_K_M, fused kernels) or "q8_0" (Q8_0 GEMVs
    # between the unfused norm / RoPE / KV-write / attention / GeGLU ops): the
    # modelConfig quantFormat of emit_csl_exec_v1.zig:279-284
    weight_format: str = "q4k"
    # RMSNorm weights used as 1 + w (Gemma 2/3) or as w (Gemma 4)
    norm_weight_offset: bool = True
    # Gemma 4 (modelConfig globalHeadDim, pleWidth, pleVocabSize;
    # emit_csl_exec_v1.zig:296-305): the head_dim of global-attention layers
    # (0: head_dim) with its rotary base (0: rope_base), and the width and
    # table rows of the per-layer embeddings (0: none; rows 0: vocab)
    global_head_dim: int = 0
    rope_base_global: float = 0.0
    # KV heads of global-attention layers (modelConfig numGlobalKeyValueHeads,
    # gemma-4-31b-af16-smoke.json:9); 0: kv_heads
    global_kv_heads: int = 0
    ple_width: int = 0
    ple_vocab: int = 0
    # the per-layer model projection's weights: "q4k" (Q4_K_M rows, as the
    # reference's E2B artifact stores per_layer_model_projection) or "f16"
    ple_proj_format: str = "q4k"

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def qkv_rows(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def row_bytes(self, k: int) -> int:
        """Bytes of one projection row of k weights in this model's format."""
        if self.weight_format == "q4k":
            return _q4k.row_bytes(k)
        if self.weight_format == "q8_0":
            return _q8_0.row_bytes(k)
        raise ValueError(f"weight_format {self.weight_format!r} is not q4k or q8_0")

    def weight_bytes_per_layer(self) -> int:
        rb = self.row_bytes
        return (self.qkv_rows * rb(self.hidden) + self.hidden * rb(self.q_dim)
                + 2 * self.ffn * rb(self.hidden) + self.hidden * rb(self.ffn))

    @property
    def ple_dim(self) -> int:
        """Per-layer embedding values per token: layers x ple_width."""
        return self.layers * self.ple_width

    @classmethod
    def from_model_config(cls, mc: dict, **overrides) -> "DecoderConfig":
        """From a step graph's modelConfig (hiddenDim, numHeads, headDim,
        numKeyValueHeads, numLayers, vocabSize, maxSeqLen, ffnExpansionFactor,
        globalHeadDim, numGlobalKeyValueHeads, pleWidth, pleVocabSize);
        quantFormat q4k or q8_0
        (f16 is not supported)."""
        from .execution import UnsupportedStep

        fmt = mc.get("quantFormat", "q4k")
        if fmt not in ("q4k", "q8_0"):
            raise UnsupportedStep(f"quantFormat {fmt!r}")
        # numKeyValueHeads absent: one kv head per query head (the reference's
        # kv_dim = (num_key_value_heads orelse num_heads) * head_dim,
        # csl_host_plan_tool.zig:412)
        kw = dict(layers=mc["numLayers"], hidden=mc["hiddenDim"], heads=mc["numHeads"],
                  kv_heads=mc.get("numKeyValueHeads") or mc["numHeads"], head_dim=mc["headDim"], vocab=mc["vocabSize"],
                  ffn=mc["hiddenDim"] * mc.get("ffnExpansionFactor", 4), weight_format=fmt,
                  global_head_dim=mc.get("globalHeadDim") or 0,
                  global_kv_heads=mc.get("numGlobalKeyValueHeads") or 0, ple_width=mc.get("pleWidth") or 0,
                  ple_vocab=mc.get("pleVocabSize") or 0)
        if "maxSeqLen" in mc:
            kw["max_seq"] = mc["maxSeqLen"]
        kw.update(overrides)
        return cls(**kw)

    def decode_bytes_per_token(self, kv_len: float) -> float:
        """Algorithmic HBM bytes of one decode step: every weight once, the
        KV cache up to kv_len, plus the embedding row."""
        w = self.layers * self.weight_bytes_per_layer() + self.vocab * self.hidden * 2
        kv = self.layers * 2 * self.kv_heads * kv_len * self.head_dim * 2
        return float(w + kv + self.hidden * 2)


def rope_table(max_pos: int, head_dim: int, base: float) -> np.ndarray:
    """freq_cis[pos][i] = (cos, sin)(pos * base^(-2i/D)), angle in float64,
    rounded once to f32 (the table layout rope.wgsl:27-29 reads)."""
    half = head_dim // 2
    inv = base ** (-2.0 * np.arange(half, dtype=np.float64) / head_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    t = np.empty((max_pos, half, 2), np.float32)
    t[:, :, 0] = np.cos(ang)
    t[:, :, 1] = np.sin(ang)
    return t.reshape(-1)


class LayerWeights:
    def __init__(self, cfg: DecoderConfig, head_dim: int | None = None, shared_kv: bool = False,
                 kv_heads: int | None = None):
        """head_dim, kv_heads: this layer's (a global layer's may differ);
        shared_kv: the layer projects q only and its attention reads an
        earlier layer's cache, so it has no k/v rows and no cache of its own."""
        rb = cfg.row_bytes
        self.head_dim = hd = head_dim or cfg.head_dim
        self.kv_heads = kv_heads or cfg.kv_heads
        self.shared_kv = shared_kv
        self.q_dim = cfg.heads * hd
        self.kv_dim = 0 if shared_kv else self.kv_heads * hd
        self.qkv_rows = self.q_dim + 2 * self.kv_dim
        # q/k rows as interleaved rotation pairs, gate/up rows interleaved
        # (gate_0, up_0, gate_1, ...) for the fused kernels (Q4_K and Q8_0)
        self.wqkv = DeviceBuffer(self.qkv_rows * rb(cfg.hidden))
        self.wo = DeviceBuffer(cfg.hidden * rb(self.q_dim))
        self.wgu = DeviceBuffer(2 * cfg.ffn * rb(cfg.hidden))
        self.wd = DeviceBuffer(cfg.hidden * rb(cfg.ffn))
        self.norm_attn = DeviceBuffer.empty((cfg.hidden,), np.float32)
        self.norm_ffn = DeviceBuffer.empty((cfg.hidden,), np.float32)
        self.k_cache = self.v_cache = None
        if not shared_kv:
            self.k_cache = DeviceBuffer.empty((self.kv_heads, cfg.max_seq, hd), np.float16)
            self.v_cache = DeviceBuffer.empty((self.kv_heads, cfg.max_seq, hd), np.float16)
        if cfg.ple_width:
            # the per-layer input block: gate [P][hidden], projection [hidden][P]
            # (Q4_K) and the norm of the projection
            self.w_ple_gate = DeviceBuffer(cfg.ple_width * rb(cfg.hidden))
            self.w_ple_out = DeviceBuffer(cfg.hidden * rb(cfg.ple_width))
            self.norm_ple = DeviceBuffer.empty((cfg.hidden,), np.float32)

    def weight_bytes(self) -> int:
        b = self.wqkv.nbytes + self.wo.nbytes + self.wgu.nbytes + self.wd.nbytes
        if hasattr(self, "w_ple_gate"):
            b += self.w_ple_gate.nbytes + self.w_ple_out.nbytes
        return b


class Decoder:
    """Device-resident weights, KV cache and activations of one decoder."""

    def __init__(self, cfg: DecoderConfig, keep_logits: bool = False, plan=None, ordered_residual: bool = True):
        """plan: an execution.DecodePlan (per-layer attention windows, head
        dims, KV-cache sources, per-layer embeddings); None = global attention
        in every layer at the model's head_dim, every layer its own cache.
        ordered_residual: Q4_K layers add the o_proj / down_proj K ranges into
        the residual stream in a fixed order (bit-identical steps); False adds
        them atomically in place (the f32 addition order varies run to run)."""
        from .execution import UnsupportedStep

        if plan is not None and plan.layer_types and "linear_attention" in plan.layer_types:
            # the step graph names the body's ops (doe_conv1d_depthwise,
            # doe_l2_normalize, doe_linear_attention run them) but not the
            # projections that feed them or the layer's output path
            raise UnsupportedStep("linear-attention (gated DeltaNet) layers: the graph lists conv1d_depthwise, "
                                  "l2_normalize and linear_attention but not the projections around them")
        if plan is not None and any(d.kind in ("qkv_norm_rope_kv", "gated_attn_out") for d in plan.layer):
            raise UnsupportedStep("q/k RMSNorm and attention-output-gate layers are planned, not decoded")
        self.ordered_residual = ordered_residual
        # K ranges of o_proj and down_proj (ordered residual).  Every workgroup
        # of the consuming GEMV reads every part, and those few lines are
        # shared by all of them: o_proj stays one range when its consumer,
        # gate/up, has at least four row groups per CU (2B shape: 1043 tok/s
        # against 1025 with two ranges; the atomic in-place form 1066), else
        # up to four (Gemma 3 270M: 2400 against 2381 with one; atomic 2465);
        # down_proj up to four (2B: 958 tok/s with two)
        from .device import device_info

        cus = device_info().get("cus", 256) or 256
        self.wo_parts = 1 if (2 * cfg.ffn + 15) // 16 >= 4 * cus else ops.MAX_GEMV_PARTS
        self.wd_parts = ops.MAX_GEMV_PARTS
        from .execution import UnsupportedStep

        self.cfg = cfg
        self.keep_logits = keep_logits  # also write the logits (tests); the sample does not need them
        c = cfg
        L = c.layers
        self.attn_windows = tuple(plan.windows) if plan is not None else (0,) * L
        self.head_dims = tuple(plan.head_dims) if plan is not None and plan.head_dims else (c.head_dim,) * L
        self.kv_sources = tuple(plan.kv_sources) if plan is not None and plan.kv_sources else tuple(range(L))
        for name, v in (("windows", self.attn_windows), ("head dims", self.head_dims),
                        ("KV sources", self.kv_sources)):
            if len(v) != L:
                raise ValueError(f"plan {name} cover {len(v)} layers, the model has {L}")
        if any(self.kv_sources[s] != s or s >= li for li, s in enumerate(self.kv_sources) if s != li):
            raise ValueError(f"KV sources {self.kv_sources}: a shared layer must read an earlier owning layer")
        if plan is not None and plan.ple is not None and not c.ple_width:
            raise UnsupportedStep("per-layer embedding steps in a model without pleWidth")
        self.ple = bool(c.ple_width)
        gemma4 = self.ple or any(s != li for li, s in enumerate(self.kv_sources)) or len(set(self.head_dims)) > 1
        if gemma4 and c.weight_format != "q4k":
            raise UnsupportedStep("per-layer embeddings, shared-KV layers and a global head_dim need q4k weights")
        # a global-attention layer's KV heads (numGlobalKeyValueHeads)
        self.kv_heads = tuple((c.global_kv_heads or c.kv_heads) if self.attn_windows[li] == 0 else c.kv_heads
                              for li in range(L))
        for li, s in enumerate(self.kv_sources):
            if self.kv_heads[s] != self.kv_heads[li]:
                raise ValueError(f"layer {li} reads the cache of layer {s}, which has other KV heads")
        self.layers = [LayerWeights(c, self.head_dims[li], self.kv_sources[li] != li, self.kv_heads[li])
                       for li in range(L)]
        self.embed = DeviceBuffer.empty((c.vocab, c.hidden), np.float16)
        self.lm_head = DeviceBuffer.empty((c.vocab, c.hidden), np.float16)
        self.norm_final = DeviceBuffer.empty((c.hidden,), np.float32)
        # rotary tables per (head_dim, base): a global layer may differ in both
        self._tables = {}
        self.freq_by_layer = []
        for li in range(L):
            key = (self.head_dims[li], c.rope_base_global or c.rope_base if self.attn_windows[li] == 0 else c.rope_base)
            if key not in self._tables:
                self._tables[key] = DeviceBuffer.from_array(rope_table(c.max_seq, key[0], key[1]))
            self.freq_by_layer.append(self._tables[key])
        self.freq_cis = self.freq_by_layer[0]
        self.x = DeviceBuffer.empty((c.hidden,), np.float32)
        self.xn = DeviceBuffer.empty((c.hidden,), np.float32)
        max_rows = max(Lw.qkv_rows for Lw in self.layers)
        self.qkv = DeviceBuffer.empty((max_rows,), np.float32)
        self.max_attn_splits = 8
        # split-attention partials: o [heads][S][D] then (m, l) [heads][S][2]
        self.attn_parts = DeviceBuffer.empty((c.heads * self.max_attn_splits * (max(self.head_dims) + 2),),
                                             np.float32)
        if self.ple:
            P, PD = c.ple_width, c.ple_dim
            self.ple_table = DeviceBuffer.empty((c.ple_vocab or c.vocab, PD), np.float16)
            if c.ple_proj_format == "q4k":
                self.ple_proj = DeviceBuffer(PD * _q4k.row_bytes(c.hidden))
            elif c.ple_proj_format == "f16":
                self.ple_proj = DeviceBuffer.empty((PD, c.hidden), np.float16)
            else:
                raise ValueError(f"ple_proj_format {c.ple_proj_format!r} is not q4k or f16")
            self.ple_norm = DeviceBuffer.empty((P,), np.float32)
            self.ple_e = DeviceBuffer.empty((PD,), np.float32)   # gathered rows
            self.ple_p = DeviceBuffer.empty((PD,), np.float32)   # projected
            self.ple_pn = DeviceBuffer.empty((PD,), np.float32)  # projected, normalised per layer
            self.ple_u = DeviceBuffer.empty((PD,), np.float32)   # per-layer inputs
            self.ple_g = DeviceBuffer.empty((P,), np.float32)
            self.ple_h = DeviceBuffer.empty((P,), np.float32)
            self.ple_y = DeviceBuffer.empty((c.hidden,), np.float32)
            self.ple_yn = DeviceBuffer.empty((c.hidden,), np.float32)
            self.ple_u_views = [self.ple_u.view(li * P * 4, P * 4, np.float32) for li in range(L)]
        self.h = DeviceBuffer.empty((c.ffn,), np.float32)
        # the residual stream without atomics (Q4_K layers): o_proj and
        # down_proj write their K ranges' row sums as parts; the next GEMV
        # adds the parts in order in its activation load, and the GEMV that
        # adds that stream as its residual forms the same sum in its epilogue
        self.parts_o = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, c.hidden), np.float32)
        self.parts_d = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, c.hidden), np.float32)
        hb = c.hidden * 4
        # (part 0, parts 1..) views: part 0 is the next GEMV's activation
        self._po = (self.parts_o.view(0, hb, np.float32), self.parts_o.view(hb, self.parts_o.nbytes - hb, np.float32))
        self._pd = (self.parts_d.view(0, hb, np.float32), self.parts_d.view(hb, self.parts_d.nbytes - hb, np.float32))
        self.logits = DeviceBuffer.empty((c.vocab,), np.float32)
        self.token = DeviceBuffer.empty((1,), np.int32)
        self.state = DeviceBuffer.empty((4,), np.int32)  # pos, kv_len, prompt_len, token
        self.ids = DeviceBuffer.empty((c.max_seq,), np.int32)
        self.argmax_parts = DeviceBuffer(1024 * 8)
        # views of the fused QKV output (the uniform model's shapes; per-layer
        # q views for layers of another head_dim)
        f4 = 4
        self.q_view = self.qkv.view(0, c.q_dim * f4, np.float32)
        self.qk_view = self.qkv.view(0, (c.q_dim + c.kv_dim) * f4, np.float32)
        self.k_view = self.qkv.view(c.q_dim * f4, c.kv_dim * f4, np.float32)
        self.v_view = self.qkv.view((c.q_dim + c.kv_dim) * f4, c.kv_dim * f4, np.float32)
        self.q_views = [self.qkv.view(0, Lw.q_dim * f4, np.float32) for Lw in self.layers]
        self.pos_view = self.state.view(0, 4, np.int32)
        self.kvlen_view = self.state.view(4, 4, np.int32)
        self.tok_view = self.state.view(12, 4, np.int32)

    def decode_bytes_per_token(self, kv_len: float) -> float:
        """Algorithmic HBM bytes of one decode step of this decoder: every
        layer's weights once (its own head width and KV heads), the K and V
        rows each layer's attention reads (a sliding layer at most its
        window), the lm_head, the embedding row and, with per-layer
        embeddings, the table row and the model projection."""
        c = self.cfg
        b = sum(L.weight_bytes() for L in self.layers) + c.vocab * c.hidden * 2 + c.hidden * 2
        for li, L in enumerate(self.layers):
            w = self.attn_windows[li]
            keys = min(kv_len, w) if w else kv_len
            b += 2 * L.kv_heads * keys * L.head_dim * 2
        if self.ple:
            b += c.ple_dim * 2 + self.ple_proj.nbytes
        return float(b)

    # ---- weights -------------------------------------------------------------
    def init_random(self, seed: int = 2, stream=None) -> None:
        """Seeded random-init weights of this architecture: Q4_K projections
        (d ~ |N(0,0.02)|, dmin ~ |N(0,0.01)|), f16 embedding and lm_head
        N(0,0.02), norm weights N(0,0.1) used as (1 + w)."""
        c = self.cfg
        sp = _stream_ptr(stream)
        s = seed * 1000

        def q4k(buf, tag):
            if c.weight_format == "q8_0":  # d ~ |N(0, 0.001)|: weights of ~0.06 like the Q4_K ones
                _lib.call("doe_fill_random_q8_0", C.c_void_p(buf.ptr), buf.nbytes // _q8_0.BLOCK_BYTES, s + tag,
                          0.001, sp)
                return
            _lib.call("doe_fill_random_q4k", C.c_void_p(buf.ptr), buf.nbytes // _q4k.BLOCK_BYTES, s + tag, 0.02,
                      0.01, sp)

        # norm weights: N(0, 0.1) used as 1 + w, or 1 + N(0, 0.1) used as w
        nmean = 0.0 if c.norm_weight_offset else 1.0

        def nrm(buf, tag, sigma, dtype_f16=False, mean=0.0):
            fn = "doe_fill_normal_f16" if dtype_f16 else "doe_fill_normal_f32"
            n = buf.nbytes // (2 if dtype_f16 else 4)
            _lib.call(fn, C.c_void_p(buf.ptr), n, s + tag, mean, sigma, sp)

        for i, L in enumerate(self.layers):
            base = 100 * (i + 1)
            q4k(L.wqkv, base + 1)
            q4k(L.wo, base + 2)
            q4k(L.wgu, base + 3)
            q4k(L.wd, base + 4)
            nrm(L.norm_attn, base + 5, 0.1, mean=nmean)
            nrm(L.norm_ffn, base + 6, 0.1, mean=nmean)
            if self.ple:
                q4k(L.w_ple_gate, base + 10)
                q4k(L.w_ple_out, base + 11)
                nrm(L.norm_ple, base + 12, 0.1, mean=nmean)
        nrm(self.embed, 7, 0.02, True)
        nrm(self.lm_head, 8, 0.02, True)
        nrm(self.norm_final, 9, 0.1, mean=nmean)
        if self.ple:
            nrm(self.ple_table, 13, 0.02, True)
            if c.ple_proj_format == "q4k":
                _lib.call("doe_fill_random_q4k", C.c_void_p(self.ple_proj.ptr),
                          self.ple_proj.nbytes // _q4k.BLOCK_BYTES, s + 14, 0.02, 0.01, sp)
            else:
                nrm(self.ple_proj, 14, 0.02, True)
            nrm(self.ple_norm, 15, 0.1, mean=nmean)

    # ---- one decode step -------------------------------------------------------
    def step(self, stream=None) -> None:
        """Enqueues one decode step at position state.pos on `stream`."""
        c = self.cfg
        ops.embed(self.embed, self.tok_view, self.x, 1, c.vocab, c.hidden, c.embed_scale, stream=stream)
        if self.ple:
            self._ple_inputs(stream)
        # Q4_K layers: the residual stream entering a layer is act + act_parts
        # (na parts); o_proj and down_proj write their K ranges as parts, range
        # 0 with the residual added; the next GEMV adds them in range order in
        # its activation load, and the one after it (o_proj after q/k/v_proj,
        # down_proj after gate/up_proj) adds the same parts in the same order
        # to its residual, so the sum is never stored.  Every add happens in a
        # fixed order: a step gives the same bits on every run.
        act, act_parts, na = self.x, None, 0
        last = len(self.layers) - 1
        for li, L in enumerate(self.layers):
            if c.weight_format == "q8_0":
                self._layer_q8_0(li, L, 1.0 / math.sqrt(c.head_dim), stream)
                continue
            if not self.ordered_residual:
                self._layer_q4k_atomic(li, L, stream)
                continue
            hd = L.head_dim
            src = self.layers[self.kv_sources[li]]  # the layer whose KV cache this one reads
            rope = dict(num_heads=c.heads, num_kv_heads=0 if L.shared_kv else L.kv_heads, head_dim=hd,
                        freq_cis=self.freq_by_layer[li], position_buffer=self.pos_view, key_cache=L.k_cache,
                        val_cache=L.v_cache, max_seq_len=c.max_seq)
            # input_norm + q/k/v_proj + rope + cache write
            ops.q4k_gemv_ex(L.wqkv, L.qkv_rows, c.hidden, activation=act, activation_parts=act_parts,
                            activation_nparts=na, output=self.qkv,
                            norm_weight=L.norm_attn, norm_eps=c.eps, norm_weight_offset=c.norm_weight_offset,
                            rope=rope, stream=stream)
            splits = ops.attention_partials(self.q_views[li], src.k_cache, src.v_cache, self.attn_parts, batch=1,
                                            num_heads=c.heads, num_kv_heads=L.kv_heads, head_dim=hd,
                                            kv_len=0, kv_stride=c.max_seq, scale=1.0 / math.sqrt(hd),
                                            max_splits=self.max_attn_splits, kv_len_buffer=self.kvlen_view,
                                            sliding_window=self.attn_windows[li], softcap=c.attn_softcap,
                                            stream=stream)
            # combine + o_proj + attn_residual as K-range parts
            # (the attention prologue takes one Q4_K block per wave: past 16
            # blocks o_proj needs more than one range, and then takes as many
            # as the parts allow)
            wo_parts = self.wo_parts if L.q_dim <= 4096 else ops.MAX_GEMV_PARTS
            no = ops.q4k_gemv_ex(L.wo, c.hidden, L.q_dim, attn_partials=self.attn_parts, attn_splits=splits,
                                 attn_num_heads=c.heads, attn_head_dim=hd, residual=act, residual_parts=act_parts,
                                 residual_nparts=na, output_parts=self.parts_o, max_output_parts=wo_parts,
                                 stream=stream)
            # post_attn_norm + gate/up_proj + GeGLU over the summed parts
            ops.q4k_gemv_ex(L.wgu, 2 * c.ffn, c.hidden, activation=self._po[0], activation_parts=self._po[1],
                            activation_nparts=no - 1, output=self.h, norm_weight=L.norm_ffn, norm_eps=c.eps,
                            norm_weight_offset=c.norm_weight_offset, gated=True, stream=stream)
            # down_proj + ffn_residual (the same sum of o_proj's parts) as K-range parts
            nd = ops.q4k_gemv_ex(L.wd, c.hidden, c.ffn, activation=self.h, residual=self._po[0],
                                 residual_parts=self._po[1], residual_nparts=no - 1, output_parts=self.parts_d,
                                 max_output_parts=self.wd_parts, stream=stream)
            if li == last or self.ple:
                # the lm_head and the per-layer input block read x whole
                self._sum_parts(self.parts_d, nd, self.x, stream)
                act, act_parts, na = self.x, None, 0
            else:
                act, act_parts, na = self._pd[0], self._pd[1], nd - 1
            if self.ple:
                self._ple_block(li, L, stream)
        nparts = ops.lm_head_sample(self.lm_head, self.x, c.vocab, c.hidden, self.argmax_parts,
                                    logits=self.logits if self.keep_logits else None, norm_weight=self.norm_final,
                                    norm_eps=c.eps, norm_weight_offset=c.norm_weight_offset, stream=stream)
        _lib.call("doe_decode_advance", C.c_void_p(self.state.ptr), C.c_void_p(self.token.ptr),
                  C.c_void_p(self.ids.ptr), c.max_seq, C.c_void_p(self.argmax_parts.ptr), nparts,
                  _stream_ptr(stream))

    def _sum_parts(self, parts: DeviceBuffer, n: int, out: DeviceBuffer, stream) -> None:
        """out = parts[0] + parts[1] + ... + parts[n - 1], added in that order."""
        hb = self.cfg.hidden * 4
        p = [parts.view(i * hb, hb, np.float32) for i in range(n)]
        if n == 1:
            out.copy_from(p[0], stream)
            return
        ops.residual(p[0], p[1], out, self.cfg.hidden, stream=stream)
        for i in range(2, n):
            ops.residual(out, p[i], out, self.cfg.hidden, stream=stream)

    def _layer_q4k_atomic(self, li: int, L: LayerWeights, stream) -> None:
        """A Q4_K layer whose o_proj / down_proj add their K ranges into x
        atomically (in place): the same five dispatches, but the f32 order of
        the residual adds varies from run to run."""
        c = self.cfg
        hd = L.head_dim
        src = self.layers[self.kv_sources[li]]
        ops.qkv_rope_kv(L.wqkv, self.x, self.qkv, hidden=c.hidden, num_heads=c.heads,
                        num_kv_heads=0 if L.shared_kv else L.kv_heads, head_dim=hd,
                        freq_cis=self.freq_by_layer[li], position_buffer=self.pos_view, key_cache=L.k_cache,
                        val_cache=L.v_cache, max_seq_len=c.max_seq, norm_weight=L.norm_attn, norm_eps=c.eps,
                        norm_weight_offset=c.norm_weight_offset, stream=stream)
        splits = ops.attention_partials(self.q_views[li], src.k_cache, src.v_cache, self.attn_parts, batch=1,
                                        num_heads=c.heads, num_kv_heads=L.kv_heads, head_dim=hd,
                                        kv_len=0, kv_stride=c.max_seq, scale=1.0 / math.sqrt(hd),
                                        max_splits=self.max_attn_splits, kv_len_buffer=self.kvlen_view,
                                        sliding_window=self.attn_windows[li], softcap=c.attn_softcap, stream=stream)
        ops.matmul_q4k_attn_out(L.wo, self.attn_parts, splits, c.heads, hd, self.x, c.hidden, residual=self.x,
                                stream=stream)
        ops.matmul_q4k_fused(L.wgu, self.x, self.h, 2 * c.ffn, c.hidden, norm_weight=L.norm_ffn, norm_eps=c.eps,
                             norm_weight_offset=c.norm_weight_offset, gated=True, stream=stream)
        ops.matmul_q4k_fused(L.wd, self.h, self.x, c.hidden, c.ffn, residual=self.x, stream=stream)
        if self.ple:
            self._ple_block(li, L, stream)

    def _ple_inputs(self, stream) -> None:
        """The step graph's ple_gather, ple_project, ple_norm and ple_modulate
        steps (emit_csl_exec_v1.zig:167-172: gather + matmul + reduction +
        element_wise), once per token, for every layer at once: the token's
        row of the per-layer embedding table scaled by sqrt(P), the embedding
        projected by the f16 model projection (scaled by hidden^-1/2) and
        RMS-normalised per layer, then (projected + gathered) / sqrt(2) -- the
        per-layer inputs of the Gemma 4 architecture (pleWidth P, every layer's
        P values side by side)."""
        c = self.cfg
        P, PD = c.ple_width, c.ple_dim
        ops.embed(self.ple_table, self.tok_view, self.ple_e, 1, c.ple_vocab or c.vocab, PD, math.sqrt(P),
                  stream=stream)
        self._ple_project(self.x, self.ple_p, 1, stream)
        ops.rmsnorm(self.ple_p, self.ple_norm, self.ple_pn, c.layers, P, self._ple_norm_eps(),
                    weight_offset=c.norm_weight_offset, stream=stream)
        ops.ple_modulate(self.ple_pn, self.ple_e, self.ple_u, PD, 2.0 ** -0.5, stream=stream)

    def _ple_project(self, x, out, rows: int, stream) -> None:
        """The ple_project step over `rows` embedding rows: W_proj x, scaled
        by hidden^-1/2 (the f16 form) or left unscaled for the per-layer
        RMSNorm to absorb (the Q4_K form: rmsnorm(a p, eps) = rmsnorm(p,
        eps / a^2), _ple_norm_eps)."""
        c = self.cfg
        if c.ple_proj_format == "q4k":
            if rows == 1:
                ops.matmul_q4k(self.ple_proj, x, out, c.ple_dim, c.hidden, stream)
            else:
                ops.matmul_gemm_f32_fused(x, self.ple_proj, out, rows, c.ple_dim, c.hidden, "q4k", stream=stream)
        elif rows == 1:
            ops.lm_head(self.ple_proj, x, out, c.ple_dim, c.hidden, alpha=c.hidden ** -0.5, stream=stream)
        else:
            ops.lm_head_gemv(x, self.ple_proj, out, rows, c.ple_dim, c.hidden, alpha=c.hidden ** -0.5, stream=stream)

    def _ple_norm_eps(self) -> float:
        c = self.cfg
        return c.eps * c.hidden if c.ple_proj_format == "q4k" else c.eps

    def _ple_block(self, li: int, L: LayerWeights, stream) -> None:
        """A layer's use of its per-layer input u (after ffn_residual): x +=
        rmsnorm(W_out . (gelu(W_gate . x) * u)) -- the Gemma 4 decoder layer's
        per-layer input block, which the step graph's PLE composite feeds."""
        c = self.cfg
        P = c.ple_width
        ops.matmul_q4k(L.w_ple_gate, self.x, self.ple_g, P, c.hidden, stream=stream)
        ops.gelu_gated(self.ple_g, self.ple_u_views[li], self.ple_h, P, stream=stream)
        ops.matmul_q4k(L.w_ple_out, self.ple_h, self.ple_y, c.hidden, P, stream=stream)
        ops.rmsnorm(self.ple_y, L.norm_ple, self.ple_yn, 1, c.hidden, c.eps, weight_offset=c.norm_weight_offset,
                    stream=stream)
        ops.residual(self.ple_yn, self.x, self.x, c.hidden, stream=stream)

    def _layer_q8_0(self, li: int, L: LayerWeights, scale: float, stream) -> None:
        """One layer with Q8_0 projections in the five dispatches of the Q4_K
        layer: input_norm + q/k/v_proj + rope_q / rope_k + the cache write,
        attention as split partials into the decoder's own buffer, combine +
        o_proj + attn_residual, post_attn_norm + gate/up_proj + activation,
        down_proj + ffn_residual.  No library workspace, so a captured graph
        stays valid whatever other attention calls the process makes."""
        c = self.cfg
        ops.qkv_rope_kv(L.wqkv, self.x, self.qkv, hidden=c.hidden, num_heads=c.heads, num_kv_heads=L.kv_heads,
                        head_dim=c.head_dim, freq_cis=self.freq_by_layer[li], position_buffer=self.pos_view,
                        key_cache=L.k_cache, val_cache=L.v_cache, max_seq_len=c.max_seq, norm_weight=L.norm_attn,
                        norm_eps=c.eps, norm_weight_offset=c.norm_weight_offset, stream=stream,
                        weight_format="q8_0")
        splits = ops.attention_partials(self.q_view, L.k_cache, L.v_cache, self.attn_parts, batch=1,
                                        num_heads=c.heads, num_kv_heads=L.kv_heads, head_dim=c.head_dim, kv_len=0,
                                        kv_stride=c.max_seq, scale=scale, max_splits=self.max_attn_splits,
                                        kv_len_buffer=self.kvlen_view, sliding_window=self.attn_windows[li],
                                        softcap=c.attn_softcap, stream=stream)
        ops.matmul_q8_0_attn_out(L.wo, self.attn_parts, splits, c.heads, c.head_dim, self.x, c.hidden,
                                 residual=self.x, stream=stream)
        ops.matmul_q4k_fused(L.wgu, self.x, self.h, 2 * c.ffn, c.hidden, norm_weight=L.norm_ffn, norm_eps=c.eps,
                             norm_weight_offset=c.norm_weight_offset, gated=True, stream=stream,
                             weight_format="q8_0")
        ops.matmul_q8_0(L.wd, self.h, self.x, c.hidden, c.ffn, residual=self.x, stream=stream)

    # ---- prompt ----------------------------------------------------------------
    def can_prefill(self) -> bool:
        """Batched prompts run for Q4_K and Q8_0 models, per-layer embeddings,
        shared-KV layers and a second (global) head_dim included."""
        return self.cfg.weight_format in ("q4k", "q8_0")

    def _prefill_buffers(self):
        if getattr(self, "_pf", None) is None:
            c, S = self.cfg, self.cfg.max_seq
            self._pf = {
                "x": DeviceBuffer.empty((S, c.hidden), np.float32),
                "qkv": DeviceBuffer.empty((S, max(L.qkv_rows for L in self.layers)), np.float32),
                "att": DeviceBuffer.empty((S, max(L.q_dim for L in self.layers)), np.float32),
                "h": DeviceBuffer.empty((S, c.ffn), np.float32),
            }
            if self.ple:
                P, PD = c.ple_width, c.ple_dim
                self._pf.update({
                    "pe": DeviceBuffer.empty((S, PD), np.float32),   # gathered rows
                    "pp": DeviceBuffer.empty((S, PD), np.float32),   # projected
                    "pn": DeviceBuffer.empty((S, PD), np.float32),   # normalised per layer
                    "pu": DeviceBuffer.empty((S, PD), np.float32),   # per-layer inputs [token][layer][P]
                    "pul": DeviceBuffer.empty((S, P), np.float32),   # one layer's inputs [token][P]
                    "pg": DeviceBuffer.empty((S, P), np.float32),
                    "ph": DeviceBuffer.empty((S, P), np.float32),
                    "py": DeviceBuffer.empty((S, c.hidden), np.float32),
                    "pyn": DeviceBuffer.empty((S, c.hidden), np.float32),
                })
        return self._pf

    def prefill(self, prompt: np.ndarray, stream=None) -> None:
        """The prompt in one batched pass -- the step graph's prefill phase
        (gemma-3-270m-smoke.json prefill steps: embed, then per layer
        input_norm + q/k/v_proj as one M-row GEMM, rope_q / rope_k with the
        cache write, causal attention of the whole prompt, o_proj +
        attn_residual, post_attn_norm + gate/up_proj + activation, down_proj +
        ffn_residual -- each "+" folded into the GEMM's pre-pass or the pass
        that sums its K splits), then the last token's final norm + lm_head +
        sample.
        Q4_K layers run the Q4_K GEMM, Q8_0 layers the Q8_0 GEMM; both the
        interleaved-pair RoPE of their decode step.
        Leaves the decoder where teacher-forced decode steps over the prompt
        would: cache rows 0..P-1 written, the first new token in ids[P],
        state = (P, P + 1, P, token)."""
        from .execution import UnsupportedStep

        if not self.can_prefill():
            raise UnsupportedStep("batched prompts need Q4_K or Q8_0 projections")
        c = self.cfg
        prompt = np.asarray(prompt, np.int32)
        P = int(prompt.size)
        if not 1 <= P < c.max_seq:
            raise ValueError(f"prompt of {P} tokens for max_seq {c.max_seq}")
        self.reset(prompt)
        self.state.upload(np.array([P - 1, P, P, prompt[-1]], np.int32))
        b = self._prefill_buffers()
        off = c.norm_weight_offset
        ids = self.ids.view(0, P * 4, np.int32)
        ops.embed(self.embed, ids, b["x"], P, c.vocab, c.hidden, c.embed_scale, stream=stream)
        # both formats hold q/k rows as interleaved rotation pairs and gate/up
        # rows interleaved
        fmt = c.weight_format
        gemm = ops.matmul_gemm_f32_fused  # the norms, residuals and GeGLU ride on the GEMMs
        if self.ple:
            self._prefill_ple_inputs(ids, P, b, stream)
        for li, L in enumerate(self.layers):
            hd = L.head_dim
            # a shared-KV layer writes no cache: its attention reads the cache
            # its source layer wrote earlier in this pass
            kvh = 0 if L.shared_kv else L.kv_heads
            src = self.layers[self.kv_sources[li]]
            gemm(b["x"], L.wqkv, b["qkv"], P, L.qkv_rows, c.hidden, fmt, norm_weight=L.norm_attn, norm_eps=c.eps,
                 norm_weight_offset=off, stream=stream)
            ops.qkv_rope_kv_rows(b["qkv"], P, L.qkv_rows, c.heads, kvh, hd, self.freq_by_layer[li], 0,
                                 L.k_cache if kvh else None, L.v_cache if kvh else None, c.max_seq, stream=stream)
            ops.attention_prefill_f16kv(b["qkv"], src.k_cache, src.v_cache, b["att"], num_heads=c.heads,
                                        num_kv_heads=L.kv_heads, head_dim=hd, query_len=P, kv_len=P,
                                        kv_stride=c.max_seq, start_pos=0, scale=1.0 / math.sqrt(hd),
                                        softcap=c.attn_softcap, sliding_window=self.attn_windows[li],
                                        q_row_stride=L.qkv_rows, out_row_stride=L.q_dim, stream=stream)
            gemm(b["att"], L.wo, b["x"], P, c.hidden, L.q_dim, fmt, residual=b["x"], stream=stream)
            gemm(b["x"], L.wgu, b["h"], P, 2 * c.ffn, c.hidden, fmt, norm_weight=L.norm_ffn, norm_eps=c.eps,
                 norm_weight_offset=off, activation=ops.GEGLU_PAIRS, stream=stream)
            gemm(b["h"], L.wd, b["x"], P, c.hidden, c.ffn, fmt, residual=b["x"], stream=stream)
            if self.ple:
                self._prefill_ple_block(li, L, P, b, stream)
        last = b["x"].view((P - 1) * c.hidden * 4, c.hidden * 4, np.float32)
        nparts = ops.lm_head_sample(self.lm_head, last, c.vocab, c.hidden, self.argmax_parts,
                                    logits=self.logits if self.keep_logits else None, norm_weight=self.norm_final,
                                    norm_eps=c.eps, norm_weight_offset=off, stream=stream)
        _lib.call("doe_decode_advance", C.c_void_p(self.state.ptr), C.c_void_p(self.token.ptr),
                  C.c_void_p(self.ids.ptr), c.max_seq, C.c_void_p(self.argmax_parts.ptr), nparts,
                  _stream_ptr(stream))

    def _prefill_ple_inputs(self, ids, P: int, b: dict, stream) -> None:
        """_ple_inputs for the P prompt tokens at once: the gathered rows, the
        f16 projection of the embeddings as one M = P GEMM, the per-layer
        RMSNorm over P * layers rows, then (projected + gathered) / sqrt(2)
        into pu [token][layer][ple_width]."""
        c = self.cfg
        W, PD = c.ple_width, c.ple_dim
        ops.embed(self.ple_table, ids, b["pe"], P, c.ple_vocab or c.vocab, PD, math.sqrt(W), stream=stream)
        self._ple_project(b["x"], b["pp"], P, stream)
        ops.rmsnorm(b["pp"], self.ple_norm, b["pn"], P * c.layers, W, self._ple_norm_eps(),
                    weight_offset=c.norm_weight_offset,
                    stream=stream)
        ops.ple_modulate(b["pn"], b["pe"], b["pu"], P * PD, 2.0 ** -0.5, stream=stream)

    def _prefill_ple_block(self, li: int, L: LayerWeights, P: int, b: dict, stream) -> None:
        """_ple_block for the P prompt rows: x += rmsnorm(W_out . (gelu(W_gate
        . x) * u)), u the layer's slice of every token's per-layer inputs."""
        c = self.cfg
        W, fmt = c.ple_width, c.weight_format
        ops.copy_rows(b["pul"], W * 4, b["pu"].view(li * W * 4, b["pu"].nbytes - li * W * 4), c.ple_dim * 4,
                      W * 4, P, stream=stream)
        ops.matmul_gemm_f32_fused(b["x"], L.w_ple_gate, b["pg"], P, W, c.hidden, fmt, stream=stream)
        ops.gelu_gated(b["pg"], b["pul"], b["ph"], P * W, stream=stream)
        ops.matmul_gemm_f32_fused(b["ph"], L.w_ple_out, b["py"], P, c.hidden, W, fmt, stream=stream)
        ops.rmsnorm(b["py"], L.norm_ple, b["pyn"], P, c.hidden, c.eps, weight_offset=c.norm_weight_offset,
                    stream=stream)
        ops.residual(b["pyn"], b["x"], b["x"], P * c.hidden, stream=stream)

    # ---- generation ----------------------------------------------------------
    def reset(self, prompt: np.ndarray) -> None:
        """Loads a prompt: ids[0:len] = prompt, state = (0, 1, len, prompt[0])."""
        c = self.cfg
        prompt = np.asarray(prompt, np.int32)
        if not 1 <= prompt.size <= c.max_seq:
            raise ValueError(f"prompt of {prompt.size} tokens for max_seq {c.max_seq}")
        ids = np.zeros(c.max_seq, np.int32)
        ids[: prompt.size] = prompt
        self.ids.upload(ids)
        self.state.upload(np.array([0, 1, prompt.size, prompt[0]], np.int32))

    def capture(self, stream: Stream, steps: int = 1) -> Graph:
        """Graph of `steps` consecutive decode steps.  The first step at a new
        shape allocates the attention workspace, so one eager step must run
        before capturing (reset() afterwards)."""
        def body():
            for _ in range(steps):
                self.step(stream)
        return Graph.capture(stream, body)

    def generate(self, prompt: np.ndarray, n_new: int, stream: Stream, graph: Graph | None = None,
                 steps_per_graph: int = 1, timing: dict | None = None, prefill: bool = False) -> np.ndarray:
        """Prompt, then `n_new` greedy tokens; returns ids[0 : len(prompt) +
        n_new].  The prompt runs as teacher-forced decode steps, or with
        `prefill` as one batched pass that also samples the first new token
        (then n_new - 1 decode steps follow).  With `timing`, records the
        seconds spent in the prompt and in the decode steps (HIP events)."""
        prompt = np.asarray(prompt, np.int32)
        total = prompt.size + n_new
        if total > self.cfg.max_seq:
            raise ValueError("prompt + n_new exceeds max_seq")
        e0, e1, e2 = Event(), Event(), Event()
        if prefill:
            if n_new < 1:
                raise ValueError("a batched prompt samples one token: n_new >= 1")
            e0.record(stream)
            self.prefill(prompt, stream)
            e1.record(stream)
            n_prompt_steps, n_new = 0, n_new - 1
        else:
            self.reset(prompt)
            n_prompt_steps = prompt.size - 1

        def run(n):
            if graph is None:
                for _ in range(n):
                    self.step(stream)
            else:
                full, rest = divmod(n, steps_per_graph)
                for _ in range(full):
                    graph.launch(stream)
                for _ in range(rest):
                    self.step(stream)

        if not prefill:
            e0.record(stream)
            run(n_prompt_steps)
            e1.record(stream)
        run(n_new)
        e2.record(stream)
        e2.synchronize()
        if timing is not None:
            timing["prompt_s"] = e0.elapsed_ms(e1) / 1e3
            timing["decode_s"] = e1.elapsed_ms(e2) / 1e3
        return self.ids.download()[:total]
