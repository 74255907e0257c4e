"""CPU oracle of the decode step (TEST INFRASTRUCTURE ONLY: the checker of
the decode loop in tests/ and bench.py, never on the product path): the same step the
Decoder runs, composed from the oracle's kernel restatements, on weights
downloaded from the device."""
import math

import numpy as np

from doe_amd import q4k
from doe_amd.ops import deinterleave_rope_rows
from . import oracle as ora


class OracleDecoder:
    def __init__(self, dec):
        c = dec.cfg
        self.cfg = c
        self.layers = []
        for L in dec.layers:
            # the device stores q/k rows as interleaved rotation pairs; the
            # oracle follows the rotate-half form of rope.wgsl on plain rows
            wqkv = L.wqkv.download().reshape(c.qkv_rows, -1)
            qk = c.q_dim + c.kv_dim
            if c.weight_format == "q4k":  # Q8_0 rows are stored plain
                wqkv[:qk] = deinterleave_rope_rows(wqkv[:qk], c.head_dim)
            self.layers.append({
                "wqkv": wqkv, "wo": L.wo.download(), "wgu": L.wgu.download(), "wd": L.wd.download(),
                "n1": L.norm_attn.download(), "n2": L.norm_ffn.download(),
                "kc": np.zeros((c.kv_heads, c.max_seq, c.head_dim), np.float16),
                "vc": np.zeros((c.kv_heads, c.max_seq, c.head_dim), np.float16),
            })
        self.embed = dec.embed.download()
        self.lm_head = dec.lm_head.download()
        self.nf = dec.norm_final.download()
        self.table = dec.freq_cis.download()
        self.windows = dec.attn_windows

    def gemv(self, w, x, n, k):
        if self.cfg.weight_format == "q8_0":
            return ora.q8_0_gemv(w, x, n, k)
        return ora.q4k_gemv(w, x, n, k)

    def step(self, pos: int, token: int) -> np.ndarray:
        c = self.cfg
        x = ora.embed_gather(self.embed, np.array([token], np.int32), c.embed_scale)[0]
        scale = 1.0 / math.sqrt(c.head_dim)
        for li, L in enumerate(self.layers):
            xn = ora.rmsnorm(x, L["n1"], c.eps, True)
            qkv = self.gemv(L["wqkv"], xn, c.qkv_rows, c.hidden)
            qk = ora.rope(qkv[: c.q_dim + c.kv_dim], self.table, 1, c.heads + c.kv_heads, c.head_dim, pos)
            k = qk[c.q_dim:]
            v = qkv[c.q_dim + c.kv_dim:]
            ora.kv_write(k, v, L["kc"], L["vc"], c.kv_heads, c.max_seq, c.head_dim, pos)
            attn = ora.attn_decode(qk[: c.q_dim], L["kc"], L["vc"], c.heads, c.kv_heads, c.head_dim, pos + 1,
                                   c.max_seq, scale, softcap=c.attn_softcap,
                                   sliding_window=self.windows[li]).reshape(-1)
            x = ora.residual(self.gemv(L["wo"], attn, c.hidden, c.q_dim), x)
            xn2 = ora.rmsnorm(x, L["n2"], c.eps, True)
            gu = self.gemv(L["wgu"], xn2, 2 * c.ffn, c.hidden)
            if c.weight_format == "q8_0":  # gate rows then up rows
                h = ora.geglu(gu[: c.ffn], gu[c.ffn:])
            else:  # interleaved gate/up rows
                h = ora.geglu(gu[0::2], gu[1::2])
            x = ora.residual(self.gemv(L["wd"], h, c.hidden, c.ffn), x)
        xn = ora.rmsnorm(x, self.nf, c.eps, True)
        return ora.f16_gemv(self.lm_head, xn)
