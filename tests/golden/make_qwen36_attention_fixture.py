"""Writes qwen36_layer3_attention.npz: real Qwen 3.6 27B activations of one
attention layer, cut from the reference's frozen Doppler reference
(bench/fixtures/r3-2-27b-doppler-frozen-af16/layer_3/, 18 prompt tokens of
"The color of the sky is", frozen-reference.manifest.json).

Kept: the query heads 0-5 after q_norm (post_qnorm), their KV head 0 after
k_norm (post_knorm) and v_proj (post_vproj), and the attention output of
those heads (attn_core_out), all before RoPE / after the attention core and
before the output gate.  The values are f16 numbers (Doppler computes in
f16), stored as f16, losslessly.

Run from the repository root: python tests/golden/make_qwen36_attention_fixture.py
"""
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/bench/fixtures/r3-2-27b-doppler-frozen-af16/layer_3")
OUT = Path(__file__).resolve().parent / "qwen36_layer3_attention.npz"
T, HQ, HKV, D, G = 18, 24, 4, 256, 6


def main() -> int:
    a = {n: np.load(SRC / f"{n}.npy", allow_pickle=False)
         for n in ("post_qnorm", "post_knorm", "post_vproj", "attn_core_out")}
    for n, v in a.items():
        assert np.array_equal(v.astype(np.float16).astype(np.float32), v), n  # f16 values
    q = a["post_qnorm"].reshape(T, HQ, D)[:, :G]
    k = a["post_knorm"].reshape(T, HKV, D)[:, :1]
    v = a["post_vproj"].reshape(T, HKV, D)[:, :1]
    out = a["attn_core_out"].reshape(T, HQ, D)[:, :G]
    np.savez_compressed(OUT, q=q.astype(np.float16), k=k.astype(np.float16), v=v.astype(np.float16),
                        out=out.astype(np.float16))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
