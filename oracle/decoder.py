"""CPU oracle of the decode step (TEST INFRASTRUCTURE ONLY: it checks the
decode loop in tests/ and bench.py, never on the product path): the same
step the Decoder runs, composed from the oracle's kernel restatements, on
weights downloaded from the device.  Per layer it follows the decoder's plan:
attention window, head_dim, the layer whose KV cache it reads (shared-KV
layers write none) and, with per-layer embeddings, the per-token PLE inputs
and each layer's per-layer input block."""
import math

import numpy as np

from . import oracle as ora


def ple_inputs(table: np.ndarray, proj: np.ndarray, norm_w: np.ndarray, token: int, x: np.ndarray, layers: int,
               width: int, hidden: int, eps: float, norm_offset: bool) -> np.ndarray:
    """Per-layer inputs [layers][width] of one token
    (bench/tools/run_gemma4_e2b_manifest_shape_execution.py:383-404,
    compute_per_layer_inputs): (rmsnorm_width(proj x / sqrt(hidden)) +
    sqrt(width) table[token]) / sqrt(2), each step an oracle function (the
    final combine one f32 add and one f32 multiply, as the kernel).  proj:
    f16 [layers * width][hidden], or Q4_K rows (uint8) whose product is
    scaled by hidden^-1/2 after the GEMV."""
    e = ora.embed_gather(table, np.array([token], np.int32), math.sqrt(width))[0]
    if proj.dtype == np.uint8:
        p = ora.q4k_gemv(proj, x, layers * width, hidden) * np.float32(hidden ** -0.5)
    else:
        p = ora.f16_gemv(proj, x, hidden ** -0.5)
    pn = ora.rmsnorm(p.reshape(layers, width), norm_w, eps, norm_offset).reshape(-1)
    u = np.add(pn, e, dtype=np.float32) * np.float32(2.0 ** -0.5)
    return u.astype(np.float32).reshape(layers, width)


def ple_block(w_gate: np.ndarray, w_out: np.ndarray, norm_w: np.ndarray, x: np.ndarray, u: np.ndarray, width: int,
              hidden: int, eps: float, norm_offset: bool) -> np.ndarray:
    """A layer's per-layer input block on the residual stream x
    (run_gemma4_e2b_manifest_shape_execution.py:358-367, the end of
    execute_layer, at layer_scalar 1): x + rmsnorm(W_out (gelu_tanh(W_gate
    x) * u)), W_gate and W_out Q4_K rows."""
    g = ora.q4k_gemv(w_gate, x, width, hidden)
    y = ora.q4k_gemv(w_out, ora.geglu(g, u), hidden, width)
    return ora.residual(ora.rmsnorm(y, norm_w, eps, norm_offset), x)


def plain_rows_from_rotation_pairs(rows: np.ndarray, head_dim: int) -> np.ndarray:
    """The device holds each head's q/k projection rows as rotation pairs:
    row 2i of a head is dimension i, row 2i + 1 is dimension i + head_dim/2.
    Returns the rows in plain dimension order (the order rope.wgsl rotates):
    plain row i of a head is device row 2i, plain row i + head_dim/2 is
    device row 2i + 1."""
    n = rows.shape[0]
    half = head_dim // 2
    head0 = np.arange(0, n, head_dim)[:, None]
    i = np.arange(half)[None, :]
    src = np.concatenate([head0 + 2 * i, head0 + 2 * i + 1], axis=1).reshape(-1)
    return np.ascontiguousarray(np.asarray(rows)[src])


class OracleDecoder:
    def __init__(self, dec):
        c = dec.cfg
        self.cfg = c
        self.layers = []
        tables = {}
        for li, L in enumerate(dec.layers):
            hd = L.head_dim
            # the device stores q/k rows as interleaved rotation pairs; the
            # oracle follows the rotate-half form of rope.wgsl on plain rows
            wqkv = L.wqkv.download().reshape(L.qkv_rows, -1)
            qk = L.q_dim + L.kv_dim
            wqkv[:qk] = plain_rows_from_rotation_pairs(wqkv[:qk], hd)
            key = id(dec.freq_by_layer[li])
            if key not in tables:
                tables[key] = dec.freq_by_layer[li].download()
            layer = {
                "hd": hd, "kvh": L.kv_heads, "shared": L.shared_kv, "src": dec.kv_sources[li], "q_dim": L.q_dim,
                "kv_dim": L.kv_dim,
                "rows": L.qkv_rows, "table": tables[key],
                "wqkv": wqkv, "wo": L.wo.download(), "wgu": L.wgu.download(), "wd": L.wd.download(),
                "n1": L.norm_attn.download(), "n2": L.norm_ffn.download(),
            }
            if not L.shared_kv:
                layer["kc"] = np.zeros((L.kv_heads, c.max_seq, hd), np.float16)
                layer["vc"] = np.zeros((L.kv_heads, c.max_seq, hd), np.float16)
            if dec.ple:
                layer.update(w_ple_gate=L.w_ple_gate.download(), w_ple_out=L.w_ple_out.download(),
                             n_ple=L.norm_ple.download())
            self.layers.append(layer)
        self.embed = dec.embed.download()
        self.lm_head = dec.lm_head.download()
        self.nf = dec.norm_final.download()
        self.windows = dec.attn_windows
        self.f16_operands = False
        self.f16_probs = False
        self._f16w = {}
        self.ple = dec.ple
        if self.ple:
            self.ple_table = dec.ple_table.download()
            self.ple_proj = dec.ple_proj.download()
            self.ple_norm = dec.ple_norm.download()

    def load_kv(self, dec, plain_k: bool = True) -> None:
        """Takes the device's KV caches ([kv_head][pos][dim] f16) as the
        oracle's own: a step at a later position then reads the context the
        device wrote (the prompt pass and the decode steps before it).  The
        device holds K in the rotation-pair order of its q/k rows (dims i and
        i + head_dim/2 at 2i and 2i + 1); the oracle in plain dim order.
        plain_k False keeps the device's order (a deliberate mismatch, for
        tests that show the check depends on the cache)."""
        for L, Ld in zip(self.layers, dec.layers):
            if not L["shared"]:
                kc = Ld.k_cache.download().reshape(L["kc"].shape).astype(np.float16)
                if plain_k:
                    kc = np.concatenate([kc[..., 0::2], kc[..., 1::2]], axis=-1)
                L["kc"] = np.ascontiguousarray(kc)
                L["vc"] = Ld.v_cache.download().reshape(L["vc"].shape).astype(np.float16)

    def gemv(self, w, x, n, k):
        if self.f16_operands:
            # the batched prompt's GEMM (q4k_gemm.hip): activation and
            # dequantized weight each rounded to f16 (round to nearest even),
            # their products exact in f32, accumulated in f32
            wh = self._f16_weights(w, n, k).astype(np.float32)
            return wh @ np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
        if self.cfg.weight_format == "q8_0":
            return ora.q8_0_gemv(w, x, n, k)
        return ora.q4k_gemv(w, x, n, k)

    def _attn_p_f16(self, q, kc, vc, hd, n, window, kvh):
        """The batched prompt's attention (attn_mq.hip) for a prompt within
        one 32-key block: exact scores (Q is split hi/lo there), the
        probabilities exp2(x - max) rounded to f16 and normalised by their
        own sum; the window and softcap of ora_attn_decode."""
        c = self.cfg
        G = c.heads // kvh
        lo = n - window if 0 < window <= n - 1 else 0
        out = np.zeros((c.heads, hd), np.float32)
        qh = np.asarray(q, np.float64).reshape(c.heads, hd)
        for h in range(c.heads):
            kk = kc[h // G, lo:n].astype(np.float64)
            vv = vc[h // G, lo:n].astype(np.float64)
            sc = (kk @ qh[h]) / math.sqrt(hd)
            if c.attn_softcap > 0:
                sc = np.tanh(sc / c.attn_softcap) * c.attn_softcap
            x = sc * math.log2(math.e)
            p = np.exp2(x - x.max()).astype(np.float16).astype(np.float64)
            out[h] = (p @ vv) / p.sum()
        return out.reshape(-1)

    def _f16_weights(self, w, n, k):
        key = id(w)
        if key not in self._f16w:
            deq = ora.q8_0_dequant(w, n, k) if self.cfg.weight_format == "q8_0" else ora.q4k_dequant_rowwise(w, n, k)
            self._f16w[key] = deq.astype(np.float16)
        return self._f16w[key]

    def ple_inputs(self, token: int, x: np.ndarray) -> np.ndarray:
        c = self.cfg
        return ple_inputs(self.ple_table, self.ple_proj, self.ple_norm, token, x, c.layers, c.ple_width, c.hidden,
                          c.eps, c.norm_weight_offset)

    def step(self, pos: int, token: int, f16_operands: bool = False, f16_probs: bool = False) -> np.ndarray:
        """One decode step.  Models of the batched prompt's precision (for a
        prompt of at most 32 tokens, one key block of its attention):
        `f16_probs` rounds the attention probabilities to f16 as the prompt's
        attention does (its f32-accurate GEMMs need no model);
        `f16_operands` also rounds the layer projections' operands to f16, as
        the prompt GEMMs' f16-operand form does.  The lm_head and
        per-layer-embedding GEMVs stay f32."""
        self.f16_operands = f16_operands
        self.f16_probs = f16_probs or f16_operands
        try:
            return self._step(pos, token)
        finally:
            self.f16_operands = False
            self.f16_probs = False

    def _step(self, pos: int, token: int) -> np.ndarray:
        c = self.cfg
        off = c.norm_weight_offset
        x = ora.embed_gather(self.embed, np.array([token], np.int32), c.embed_scale)[0]
        u = self.ple_inputs(token, x) if self.ple else None
        for li, L in enumerate(self.layers):
            hd = L["hd"]
            src = self.layers[L["src"]]
            xn = ora.rmsnorm(x, L["n1"], c.eps, off)
            qkv = self.gemv(L["wqkv"], xn, L["rows"], c.hidden)
            kvh = L["kvh"]
            nh = c.heads + (0 if L["shared"] else kvh)
            qk = ora.rope(qkv[: L["q_dim"] + L["kv_dim"]], L["table"], 1, nh, hd, pos)
            if not L["shared"]:
                k = qk[L["q_dim"]:]
                v = qkv[L["q_dim"] + L["kv_dim"]:]
                ora.kv_write(k, v, L["kc"], L["vc"], kvh, c.max_seq, hd, pos)
            if self.f16_probs:
                attn = self._attn_p_f16(qk[: L["q_dim"]], src["kc"], src["vc"], hd, pos + 1, self.windows[li], kvh)
            else:
                attn = ora.attn_decode(qk[: L["q_dim"]], src["kc"], src["vc"], c.heads, kvh, hd, pos + 1,
                                       c.max_seq, 1.0 / math.sqrt(hd), softcap=c.attn_softcap,
                                       sliding_window=self.windows[li]).reshape(-1)
            x = ora.residual(self.gemv(L["wo"], attn, c.hidden, L["q_dim"]), x)
            xn2 = ora.rmsnorm(x, L["n2"], c.eps, off)
            gu = self.gemv(L["wgu"], xn2, 2 * c.ffn, c.hidden)
            h = ora.geglu(gu[0::2], gu[1::2])  # interleaved gate/up rows
            x = ora.residual(self.gemv(L["wd"], h, c.hidden, c.ffn), x)
            if u is not None:
                x = ple_block(L["w_ple_gate"], L["w_ple_out"], L["n_ple"], x, u[li], c.ple_width, c.hidden, c.eps,
                              off)
        xn = ora.rmsnorm(x, self.nf, c.eps, off)
        return ora.f16_gemv(self.lm_head, xn)
