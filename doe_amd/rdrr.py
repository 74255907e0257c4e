"""Doppler RDRR artifacts: real Q4_K_M weights from local files into the
decode loop's device layout, byte for byte (no dequantisation on the host).

An RDRR artifact is a directory holding ``manifest.json`` and shard files
(bench/tools/doppler_rdrr_q4k.py:159-350):

  * ``shards``: ``[{"index", "filename"?, "size"?}]`` (a shard without a
    filename is ``shard_<index:05d>.bin``);
  * ``tensors``: ``{name: {"dtype", "shape", "layout"?, "size", "spans":
    [{"shardIndex" | "shard", "offset", "size"}]}}`` or, for a tensor in one
    shard, ``"shard"``, ``"offset"``, ``"size"`` on the tensor itself.  A
    tensor's bytes are its spans concatenated in order.

``Q4_K_M`` and ``Q8_0`` tensors are row-wise (Q8_0: ``ceil(cols / 32)``
blocks of 34 bytes per row).  ``Q4_K_M`` tensors are row-wise: ``shape [rows, cols...]``, each row
``ceil(cols / 256)`` blocks of 144 bytes (the tail block zero-padded), which
is the layout the GEMV and GEMM kernels read.  Step-graph weight keys
(``layer.3.self_attn.q_proj``, ``embed_tokens``, ``norm``, ...) resolve to the
tensor names the reference's weight mapping lists
(bench/tools/int4ple_runtime_weight_mappings.py:19-83).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

from . import q4k as _q4k
from . import q8_0 as _q8_0
from .ops import interleave_rope_rows


class RdrrError(ValueError):
    """A malformed artifact or a tensor that does not fit its use."""


def weight_key_candidates(key: str) -> list[str]:
    """Tensor names a step-graph weight key may be stored under, preferred first."""
    if key == "norm":
        return ["model.language_model.norm.weight", "model.norm.weight", "norm.weight"]
    if key == "embed_tokens":
        return ["model.language_model.embed_tokens.weight", "model.embed_tokens.weight", "embed_tokens.weight"]
    # the per-layer-embedding weights (gemma-4-e2b-smoke.json weightsKey
    # per_layer_inputs.*; tensor names of the reference's E2B artifact,
    # config/gemma-4-e2b-doppler-rdrr-int4ple-fixture.json:34,140)
    if key == "per_layer_inputs.embedTokensPerLayer":
        return ["model.language_model.embed_tokens_per_layer.weight", "model.embed_tokens_per_layer.weight"]
    if key == "per_layer_inputs.perLayerModelProjection":
        return ["model.language_model.per_layer_model_projection.weight", "model.per_layer_model_projection.weight"]
    if key == "per_layer_inputs.perLayerProjectionNorm":
        return ["model.language_model.per_layer_projection_norm.weight", "model.per_layer_projection_norm.weight"]
    if key == "lm_head":  # a tied head falls back to the embedding
        return ["model.language_model.lm_head.weight", "language_model.lm_head.weight", "model.lm_head.weight",
                "lm_head.weight"] + weight_key_candidates("embed_tokens")
    parts = key.split(".")
    if len(parts) >= 3 and parts[0] == "layer" and parts[1].isdigit():
        tail = ".".join(parts[2:])
        if parts[2] in ("self_attn", "mlp") and len(parts) < 4:
            raise RdrrError(f"weight key {key!r} names no tensor")
        return [f"model.language_model.layers.{parts[1]}.{tail}.weight", f"model.layers.{parts[1]}.{tail}.weight"]
    raise RdrrError(f"unsupported weight key {key!r}")


_DENSE = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16}


class RdrrArtifact:
    def __init__(self, root, manifest: dict | None = None):
        self.root = Path(root)
        if manifest is None:
            path = self.root / "manifest.json"
            try:
                manifest = json.loads(path.read_text())
            except (OSError, json.JSONDecodeError) as e:
                raise RdrrError(f"cannot read {path}: {e}") from None
        if not isinstance(manifest, dict) or not isinstance(manifest.get("tensors"), dict):
            raise RdrrError("manifest has no tensors table")
        self.manifest = manifest
        self.shards = {}
        for sh in manifest.get("shards", []):
            idx = int(sh["index"])
            self.shards[idx] = sh.get("filename") or f"shard_{idx:05d}.bin"
        self._maps: dict[str, np.memmap] = {}

    # ---- lookup ---------------------------------------------------------------
    def names(self) -> list[str]:
        return list(self.manifest["tensors"])

    def meta(self, name: str) -> dict:
        try:
            return self.manifest["tensors"][name]
        except KeyError:
            raise KeyError(f"tensor not in the RDRR manifest: {name}") from None

    def resolve(self, key: str) -> str:
        cands = weight_key_candidates(key)
        for c in cands:
            if c in self.manifest["tensors"]:
                return c
        raise KeyError(f"weight key {key!r}: none of {cands} is in the manifest")

    # ---- bytes ----------------------------------------------------------------
    def _spans(self, name: str) -> list[tuple[str, int, int]]:
        t = self.meta(name)
        raw = t.get("spans")
        if raw is None and t.get("shard") is not None:
            raw = [{"shardIndex": t["shard"], "offset": t["offset"], "size": t["size"]}]
        if not raw:
            raise RdrrError(f"{name}: no spans")
        out = []
        for sp in raw:
            idx = int(sp.get("shardIndex", sp.get("shard")))
            off, size = int(sp["offset"]), int(sp["size"])
            if off < 0 or size < 0:
                raise RdrrError(f"{name}: negative span {off}+{size}")
            out.append((self.shards.get(idx, f"shard_{idx:05d}.bin"), off, size))
        return out

    def _map(self, filename: str) -> np.memmap:
        m = self._maps.get(filename)
        if m is None:
            path = self.root / filename
            if not path.is_file():
                raise FileNotFoundError(f"shard file not found: {path}")
            m = np.memmap(path, dtype=np.uint8, mode="r")
            self._maps[filename] = m
        return m

    def read(self, name: str, start: int = 0, count: int | None = None) -> np.ndarray:
        """Bytes [start, start + count) of a tensor (all of it by default)."""
        size = int(self.meta(name).get("size", sum(s for _, _, s in self._spans(name))))
        count = size - start if count is None else count
        if start < 0 or count < 0 or start + count > size:
            raise RdrrError(f"{name}: byte range {start}:{start + count} outside its {size} bytes")
        out = np.empty(count, np.uint8)
        done, skip = 0, start
        for filename, off, span_size in self._spans(name):
            if done == count:
                break
            if skip >= span_size:
                skip -= span_size
                continue
            take = min(span_size - skip, count - done)
            m = self._map(filename)
            if off + skip + take > m.size:
                raise RdrrError(f"{name}: span {off}+{span_size} runs past {filename} ({m.size} bytes)")
            out[done:done + take] = m[off + skip:off + skip + take]
            done += take
            skip = 0
        if done != count:
            raise RdrrError(f"{name}: spans end after {done} of {count} bytes")
        return out

    # ---- typed views -----------------------------------------------------------
    def q4k_rows(self, name: str) -> np.ndarray:
        """A row-wise Q4_K_M tensor as its row bytes [rows][ceil(cols/256)*144]."""
        t = self.meta(name)
        if t.get("dtype") != "Q4_K_M":
            raise RdrrError(f"{name}: dtype {t.get('dtype')!r} is not Q4_K_M")
        if t.get("layout") != "row":
            raise RdrrError(f"{name}: Q4_K_M layout {t.get('layout')!r} is not row")
        shape = [int(v) for v in t.get("shape", [])]
        if len(shape) < 2:
            raise RdrrError(f"{name}: shape {shape} is not a matrix")
        rows, cols = shape[0], math.prod(shape[1:])
        rb = _q4k.row_bytes(cols)
        data = self.read(name)
        if data.size != rows * rb:
            raise RdrrError(f"{name}: {data.size} bytes, a {rows} x {cols} Q4_K_M matrix has {rows * rb}")
        return data.reshape(rows, rb)

    def q8_0_rows(self, name: str) -> np.ndarray:
        """A row-wise Q8_0 tensor as its row bytes [rows][ceil(cols/32)*34]
        (RDRR dtype "Q8_0": blockSizeElements 32, blockSizeBytes 34,
        bench/tools/run_doe_csl_int4ple_transcript.py:1559-1565).  The byte
        count must also pass the reference's Q8_0 size check (a nonzero whole
        number of blocks, runtime/zig/src/doe_wgsl/csl_spec.zig:135-140)."""
        t = self.meta(name)
        if t.get("dtype") != "Q8_0":
            raise RdrrError(f"{name}: dtype {t.get('dtype')!r} is not Q8_0")
        if t.get("layout", "row") != "row":
            raise RdrrError(f"{name}: Q8_0 layout {t.get('layout')!r} is not row")
        shape = [int(v) for v in t.get("shape", [])]
        if len(shape) < 2:
            raise RdrrError(f"{name}: shape {shape} is not a matrix")
        rows, cols = shape[0], math.prod(shape[1:])
        rb = _q8_0.row_bytes(cols)
        data = self.read(name)
        if data.size == 0 or data.size % _q8_0.BLOCK_BYTES:
            raise RdrrError(f"{name}: {data.size} bytes is not a whole number of Q8_0 blocks")
        if data.size != rows * rb:
            raise RdrrError(f"{name}: {data.size} bytes, a {rows} x {cols} Q8_0 matrix has {rows * rb}")
        return data.reshape(rows, rb)

    def dense(self, name: str, dtype) -> np.ndarray:
        """An F32 / F16 / BF16 tensor as `dtype` (float32 or float16)."""
        t = self.meta(name)
        src = t.get("dtype")
        if src not in _DENSE:
            raise RdrrError(f"{name}: dtype {src!r} is not dense")
        shape = tuple(int(v) for v in t.get("shape", []))
        raw = self.read(name).view(_DENSE[src])
        if raw.size != math.prod(shape):
            raise RdrrError(f"{name}: {raw.size} elements, shape {shape}")
        vals = (raw.astype(np.uint32) << 16).view(np.float32) if src == "BF16" else raw
        return np.asarray(vals, dtype).reshape(shape)


def _expect(arr: np.ndarray, shape: tuple, what: str) -> np.ndarray:
    if tuple(arr.shape) != tuple(shape):
        raise RdrrError(f"{what}: shape {tuple(arr.shape)}, the decoder needs {tuple(shape)}")
    return arr


def load_decoder_weights(art: RdrrArtifact, dec) -> None:
    """Fills a doe_amd.model.Decoder's device weights from the artifact: the
    Q4_K_M rows (or Q8_0 rows, for a decoder of that weight format) move
    unchanged, q/k rows reordered into rotation pairs and gate and up rows
    interleaved; norms and the f16 embedding / lm_head are
    uploaded as they are (BF16 or F32 sources converted to the decoder's
    dtype).  input_layernorm feeds attention, post_attention_layernorm the
    FFN (the step graph's post_attn_norm before gate_proj;
    int4ple_runtime_weight_mappings.py:136-153).

    Per layer the decoder's plan decides the shapes: a global layer's
    head_dim, and a shared-KV layer takes only its q_proj (its attention reads
    an earlier layer's cache; the artifact's k/v tensors of such a layer are
    not read).  With per-layer embeddings the table
    (embed_tokens_per_layer, F16), the model projection
    (per_layer_model_projection, Q4_K_M rows, or F16 for an f16-projection
    decoder), its norm, and every layer's per_layer_input_gate,
    per_layer_projection and post_per_layer_input_norm load too (the tensor
    names of config/gemma-4-e2b-doppler-rdrr-int4ple-fixture.json)."""
    c = dec.cfg
    q8 = c.weight_format == "q8_0"
    rb_h, rb_f = c.row_bytes(c.hidden), c.row_bytes(c.ffn)
    for i, L in enumerate(dec.layers):
        def rows(key, shape):
            name = art.resolve(f"layer.{i}.{key}")
            return _expect(art.q8_0_rows(name) if q8 else art.q4k_rows(name), shape, key)

        def vec(key):
            return _expect(art.dense(art.resolve(f"layer.{i}.{key}"), np.float32), (c.hidden,), key)

        hd = L.head_dim
        # the fused q/k/v kernels rotate interleaved pairs
        parts = [interleave_rope_rows(rows("self_attn.q_proj", (L.q_dim, rb_h)), hd)]
        if L.kv_dim:
            parts.append(interleave_rope_rows(rows("self_attn.k_proj", (L.kv_dim, rb_h)), hd))
            parts.append(rows("self_attn.v_proj", (L.kv_dim, rb_h)))
        L.wqkv.upload(np.concatenate(parts))
        L.wo.upload(rows("self_attn.o_proj", (c.hidden, c.row_bytes(L.q_dim))))
        gate = rows("mlp.gate_proj", (c.ffn, rb_h))
        up = rows("mlp.up_proj", (c.ffn, rb_h))
        gu = np.empty((2 * c.ffn, rb_h), np.uint8)
        gu[0::2], gu[1::2] = gate, up
        L.wgu.upload(gu)
        L.wd.upload(rows("mlp.down_proj", (c.hidden, rb_f)))
        L.norm_attn.upload(vec("input_layernorm"))
        L.norm_ffn.upload(vec("post_attention_layernorm"))
        if dec.ple:
            L.w_ple_gate.upload(rows("per_layer_input_gate", (c.ple_width, rb_h)))
            L.w_ple_out.upload(rows("per_layer_projection", (c.hidden, c.row_bytes(c.ple_width))))
            L.norm_ple.upload(vec("post_per_layer_input_norm"))
    if dec.ple:
        PD = c.ple_dim
        dec.ple_table.upload(_expect(art.dense(art.resolve("per_layer_inputs.embedTokensPerLayer"), np.float16),
                                     (c.ple_vocab or c.vocab, PD), "embed_tokens_per_layer"))
        proj = art.resolve("per_layer_inputs.perLayerModelProjection")
        if c.ple_proj_format == "q4k":
            dec.ple_proj.upload(_expect(art.q4k_rows(proj), (PD, _q4k.row_bytes(c.hidden)), "per_layer_model_projection"))
        else:
            dec.ple_proj.upload(_expect(art.dense(proj, np.float16), (PD, c.hidden), "per_layer_model_projection"))
        dec.ple_norm.upload(_expect(art.dense(art.resolve("per_layer_inputs.perLayerProjectionNorm"), np.float32),
                                    (c.ple_width,), "per_layer_projection_norm"))
    dec.embed.upload(_expect(art.dense(art.resolve("embed_tokens"), np.float16), (c.vocab, c.hidden), "embed_tokens"))
    dec.lm_head.upload(_expect(art.dense(art.resolve("lm_head"), np.float16), (c.vocab, c.hidden), "lm_head"))
    dec.norm_final.upload(_expect(art.dense(art.resolve("norm"), np.float32), (c.hidden,), "norm"))
