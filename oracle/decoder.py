"""CPU oracle of the decode step (TEST INFRASTRUCTURE ONLY: the checker of
the decode loop in tests/ and bench.py, never on the product path): the same
step the Decoder runs, composed from the oracle's kernel restatements, on
weights downloaded from the device.  Per layer it follows the decoder's plan:
attention window, head_dim, the layer whose KV cache it reads (shared-KV
layers write none) and, with per-layer embeddings, the per-token PLE inputs
and each layer's per-layer input block."""
import math

import numpy as np

from doe_amd.ops import deinterleave_rope_rows
from . import oracle as ora


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
            if c.weight_format == "q4k":  # Q8_0 rows are stored plain
                wqkv[:qk] = deinterleave_rope_rows(wqkv[:qk], hd)
            key = id(dec.freq_by_layer[li])
            if key not in tables:
                tables[key] = dec.freq_by_layer[li].download()
            layer = {
                "hd": hd, "shared": L.shared_kv, "src": dec.kv_sources[li], "q_dim": L.q_dim, "kv_dim": L.kv_dim,
                "rows": L.qkv_rows, "table": tables[key],
                "wqkv": wqkv, "wo": L.wo.download(), "wgu": L.wgu.download(), "wd": L.wd.download(),
                "n1": L.norm_attn.download(), "n2": L.norm_ffn.download(),
            }
            if not L.shared_kv:
                layer["kc"] = np.zeros((c.kv_heads, c.max_seq, hd), np.float16)
                layer["vc"] = np.zeros((c.kv_heads, c.max_seq, hd), np.float16)
            if dec.ple:
                layer.update(w_ple_gate=L.w_ple_gate.download(), w_ple_out=L.w_ple_out.download(),
                             n_ple=L.norm_ple.download())
            self.layers.append(layer)
        self.embed = dec.embed.download()
        self.lm_head = dec.lm_head.download()
        self.nf = dec.norm_final.download()
        self.windows = dec.attn_windows
        self.ple = dec.ple
        if self.ple:
            self.ple_table = dec.ple_table.download()
            self.ple_proj = dec.ple_proj.download()
            self.ple_norm = dec.ple_norm.download()

    def gemv(self, w, x, n, k):
        if self.cfg.weight_format == "q8_0":
            return ora.q8_0_gemv(w, x, n, k)
        return ora.q4k_gemv(w, x, n, k)

    def ple_inputs(self, token: int, x: np.ndarray) -> np.ndarray:
        """Per-layer inputs [layers][P]: (rmsnorm_P(W_proj x / sqrt(hidden)) +
        sqrt(P) table[token]) / sqrt(2), each step an oracle function (the
        final combine one f32 add and one f32 multiply, as the kernel)."""
        c = self.cfg
        P = c.ple_width
        e = ora.embed_gather(self.ple_table, np.array([token], np.int32), math.sqrt(P))[0]
        p = ora.f16_gemv(self.ple_proj, x, c.hidden ** -0.5)
        pn = ora.rmsnorm(p.reshape(c.layers, P), self.ple_norm, c.eps, c.norm_weight_offset).reshape(-1)
        u = np.add(pn, e, dtype=np.float32) * np.float32(2.0 ** -0.5)
        return u.astype(np.float32).reshape(c.layers, P)

    def step(self, pos: int, token: int) -> np.ndarray:
        c = self.cfg
        off = c.norm_weight_offset
        x = ora.embed_gather(self.embed, np.array([token], np.int32), c.embed_scale)[0]
        u = self.ple_inputs(token, x) if self.ple else None
        for li, L in enumerate(self.layers):
            hd = L["hd"]
            src = self.layers[L["src"]]
            xn = ora.rmsnorm(x, L["n1"], c.eps, off)
            qkv = self.gemv(L["wqkv"], xn, L["rows"], c.hidden)
            nh = c.heads + (0 if L["shared"] else c.kv_heads)
            qk = ora.rope(qkv[: L["q_dim"] + L["kv_dim"]], L["table"], 1, nh, hd, pos)
            if not L["shared"]:
                k = qk[L["q_dim"]:]
                v = qkv[L["q_dim"] + L["kv_dim"]:]
                ora.kv_write(k, v, L["kc"], L["vc"], c.kv_heads, c.max_seq, hd, pos)
            attn = ora.attn_decode(qk[: L["q_dim"]], src["kc"], src["vc"], c.heads, c.kv_heads, hd, pos + 1,
                                   c.max_seq, 1.0 / math.sqrt(hd), softcap=c.attn_softcap,
                                   sliding_window=self.windows[li]).reshape(-1)
            x = ora.residual(self.gemv(L["wo"], attn, c.hidden, L["q_dim"]), x)
            xn2 = ora.rmsnorm(x, L["n2"], c.eps, off)
            gu = self.gemv(L["wgu"], xn2, 2 * c.ffn, c.hidden)
            if c.weight_format == "q8_0":  # gate rows then up rows
                h = ora.geglu(gu[: c.ffn], gu[c.ffn:])
            else:  # interleaved gate/up rows
                h = ora.geglu(gu[0::2], gu[1::2])
            x = ora.residual(self.gemv(L["wd"], h, c.hidden, c.ffn), x)
            if u is not None:
                g = ora.q4k_gemv(L["w_ple_gate"], x, c.ple_width, c.hidden)
                y = ora.q4k_gemv(L["w_ple_out"], ora.geglu(g, u[li]), c.hidden, c.ple_width)
                x = ora.residual(ora.rmsnorm(y, L["n_ple"], c.eps, off), x)
        xn = ora.rmsnorm(x, self.nf, c.eps, off)
        return ora.f16_gemv(self.lm_head, xn)
