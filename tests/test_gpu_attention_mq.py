"""GPU parity of the multi-query attention (the reference dispatch at
query_len > 1, attention_head256_f16kv.wgsl:72-267, and the decoder-layout
prefill entry point) against the CPU oracle: ora_attn_prefill on the f16
inputs for the causal case, and per query the oracle decode attention over
exactly the keys the reference's rules make visible (kv_start, sliding
window, softcap, non-causal).  Ring and paged caches are checked as storage
invariants: the same keys stored another way give the same output.
Contract: rel-L2 <= 1e-3."""
import numpy as np
import pytest

from doe_amd import DeviceBuffer, ops

pytestmark = pytest.mark.gpu

up = DeviceBuffer.from_array


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def visible(abs_q, L, kv_start, causal, window):
    """Logical keys [lo, hi) of the query at abs_q (the reference's rule)."""
    hi = L
    if causal:
        hi = 0 if abs_q < kv_start else min(L, abs_q - kv_start + 1)
    lo = 0
    if window > 0 and abs_q >= window:
        mk = abs_q - window + 1
        if mk > kv_start:
            lo = min(L, mk - kv_start)
    return lo, hi


def oracle_rows(ora, q, k_rows, v_rows, hq, hkv, d, L, start_pos, kv_start, causal, window, scale, softcap):
    """Per query: the oracle decode attention over the visible cache rows
    (k_rows / v_rows: [capacity][hkv][d], logical key p at row kv_start + p)."""
    out = np.zeros((q.shape[0], hq, d), np.float32)
    for i in range(q.shape[0]):
        lo, hi = visible(start_pos + i, L, kv_start, causal, window)
        if hi <= lo:
            continue
        kr = np.ascontiguousarray(k_rows[kv_start + lo: kv_start + hi])
        vr = np.ascontiguousarray(v_rows[kv_start + lo: kv_start + hi])
        out[i] = ora.attn_decode(q[i], kr, vr, hq, hkv, d, hi - lo, hi - lo, scale, softcap=softcap, kv_layout=1)
    return out


@pytest.mark.parametrize("hq,hkv,d,ql,start", [(8, 4, 256, 37, 0), (8, 1, 512, 20, 5), (4, 4, 128, 100, 0),
                                               (16, 2, 64, 17, 30), (8, 8, 256, 16, 0), (2, 1, 512, 3, 0)])
def test_dispatch_causal_prompt_matches_oracle_prefill(dev, ora, hq, hkv, d, ql, start):
    # a prompt of ql queries at positions start .. start + ql - 1 over a cache
    # holding start + ql rows ([pos][kv_head][dim], the reference's order)
    print(f"[mq] hq={hq} hkv={hkv} d={d} ql={ql} start={start}", flush=True)
    rng = np.random.default_rng(hq * 100 + d + ql)
    L = start + ql
    cap = L + 3
    q = rng.standard_normal((ql, hq, d)).astype(np.float32)
    k = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    out = DeviceBuffer.empty((ql, hq, d), np.float32)
    ops.attention_dispatch(up(q), up(k), up(v), out, kv_capacity=cap, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                           seq_len=L, query_len=ql, scale=scale, is_causal=1, start_pos=start)
    # ora_attn_prefill takes f32 K/V [kv_head][pos][dim]
    kf = np.ascontiguousarray(k[:L].astype(np.float32).transpose(1, 0, 2))
    vf = np.ascontiguousarray(v[:L].astype(np.float32).transpose(1, 0, 2))
    want = ora.attn_prefill(q, kf, vf, hq, hkv, d, ql, L, start, scale, True)
    err = rel_l2(out.download(), want)
    print(f"  rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-3, err


@pytest.mark.parametrize("case", ["window", "softcap", "kv_start", "noncausal", "all_masked"])
def test_dispatch_key_rules_match_oracle(dev, ora, case):
    rng = np.random.default_rng(hash(case) % 1000)
    hq, hkv, d, ql = 8, 2, 256, 40
    cap = 96
    start, kv_start, causal, window, softcap, L = 30, 0, 1, 0, 0.0, 70
    if case == "window":
        window = 9
    elif case == "softcap":
        softcap = 0.5  # small cap: tanh saturates, the scores change visibly
    elif case == "kv_start":
        kv_start, start, L = 7, 40, 60  # logical key p at row 7 + p
    elif case == "noncausal":
        causal = 0
    else:  # queries before kv_start see nothing: zeros
        kv_start, start, L = 50, 0, 20
    q = (rng.standard_normal((ql, hq, d)) * 3).astype(np.float32)
    k = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    out = DeviceBuffer.empty((ql, hq, d), np.float32)
    ops.attention_dispatch(up(q), up(k), up(v), out, kv_capacity=cap, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                           seq_len=L, query_len=ql, scale=scale, is_causal=causal, start_pos=start, kv_start=kv_start,
                           sliding_window=window, attn_softcap=softcap)
    want = oracle_rows(ora, q, k, v, hq, hkv, d, L, start, kv_start, causal, window, scale, softcap)
    got = out.download()
    if case == "all_masked":
        assert not want.any() and not got.any()
        return
    err = rel_l2(got, want)
    print(f"[mq {case}] rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-3, err


def test_dispatch_ring_and_pages_are_storage_invariant(dev):
    # the same logical keys in a contiguous cache, a ring of `window` rows
    # (kv_layout 1) and pages (kv_layout 2) give the same prompt output
    rng = np.random.default_rng(77)
    hq, hkv, d, ql, start, window = 4, 2, 128, 24, 40, 16
    L = start + ql
    q = rng.standard_normal((ql, hq, d)).astype(np.float32)
    keys = rng.standard_normal((L, hkv, d)).astype(np.float16)
    vals = rng.standard_normal((L, hkv, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    common = dict(num_heads=hq, num_kv_heads=hkv, head_dim=d, seq_len=L, query_len=ql, scale=scale, is_causal=1,
                  start_pos=start, sliding_window=window)
    o_flat = DeviceBuffer.empty((ql, hq, d), np.float32)
    ops.attention_dispatch(up(q), up(keys), up(vals), o_flat, kv_capacity=L, **common)
    # paged: page size 8, pages stored in reverse order
    ps = 8
    npg = (L + ps - 1) // ps
    table = np.arange(npg, dtype=np.uint32)[::-1].copy()
    kp = np.zeros((npg * ps, hkv, d), np.float16)
    vp = np.zeros_like(kp)
    for lp in range(npg):
        kp[table[lp] * ps: table[lp] * ps + ps][: min(ps, L - lp * ps)] = keys[lp * ps: lp * ps + ps]
        vp[table[lp] * ps: table[lp] * ps + ps][: min(ps, L - lp * ps)] = vals[lp * ps: lp * ps + ps]
    o_pg = DeviceBuffer.empty((ql, hq, d), np.float32)
    ops.attention_dispatch(up(q), up(kp), up(vp), o_pg, kv_capacity=npg * ps, page_table=up(table), kv_layout=2,
                           page_size=ps, **common)
    assert rel_l2(o_pg.download(), o_flat.download()) < 1e-6
    # ring: only the window's worth of rows exists; query i needs keys back to
    # start + i - window + 1, so a ring of `window` rows holds them only for
    # the last query -- check that query alone
    ring = np.zeros((window, hkv, d), np.float16)
    vring = np.zeros_like(ring)
    for p in range(L - window, L):
        ring[p % window] = keys[p]
        vring[p % window] = vals[p]
    # (query_len 1 runs the split-K decode kernel: the same query against the
    # flat cache through that kernel is the storage-invariant comparison; the
    # two kernels agree within the 1e-3 contract)
    o_ring = DeviceBuffer.empty((1, hq, d), np.float32)
    o_last = DeviceBuffer.empty((1, hq, d), np.float32)
    last = dict(common, query_len=1, start_pos=L - 1)
    ops.attention_dispatch(up(q[-1:]), up(ring), up(vring), o_ring, kv_capacity=window, kv_layout=1, **last)
    ops.attention_dispatch(up(q[-1:]), up(keys), up(vals), o_last, kv_capacity=L, **last)
    assert rel_l2(o_ring.download(), o_last.download()) < 1e-6
    assert rel_l2(o_last.download()[0], o_flat.download()[-1]) < 1e-3


@pytest.fixture
def mq_splits(request, dev):
    """Forces the multi-query attention's key split (attn_mq.splits; 0 the
    automatic choice, 1 none) and restores the automatic choice."""
    ops.tune("attn_mq.splits", request.param)
    yield request.param
    ops.tune("attn_mq.splits", 0)


@pytest.mark.parametrize("mq_splits", [0, 1, 2, 3, 5], indirect=True)
@pytest.mark.parametrize("hq,hkv,d", [(8, 4, 256), (4, 1, 512), (2, 1, 64)])
def test_prefill_f16kv_decoder_layout(dev, ora, hq, hkv, d, mq_splits):
    # the decoder's cache ([kv_head][max_seq][dim]) and the q part of fused
    # q/k/v rows (row stride q + 2 kv dims): a prompt continuing at position
    # 10, window 12, softcap 30; the key blocks split 1..5 ways over the grid
    # (5: more splits than key blocks, some empty) and merged
    rng = np.random.default_rng(d + hq)
    ql, start, maxs, window, softcap = 33, 10, 64, 12, 30.0
    L = start + ql
    row = (hq + 2 * hkv) * d
    qkv = rng.standard_normal((ql, row)).astype(np.float32)
    kc = rng.standard_normal((hkv, maxs, d)).astype(np.float16)
    vc = rng.standard_normal((hkv, maxs, d)).astype(np.float16)
    scale = 1.0 / np.sqrt(d)
    out = DeviceBuffer.empty((ql, hq * d + 8), np.float32)  # padded output rows
    ops.attention_prefill_f16kv(up(qkv), up(kc), up(vc), out, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                                query_len=ql, kv_len=L, kv_stride=maxs, start_pos=start, scale=scale, softcap=softcap,
                                sliding_window=window, q_row_stride=row, out_row_stride=hq * d + 8)
    q = qkv[:, : hq * d].reshape(ql, hq, d)
    krows = np.ascontiguousarray(kc.transpose(1, 0, 2))
    vrows = np.ascontiguousarray(vc.transpose(1, 0, 2))
    want = oracle_rows(ora, q, krows, vrows, hq, hkv, d, L, start, 0, 1, window, scale, softcap)
    got = out.download()[:, : hq * d].reshape(ql, hq, d)
    err = rel_l2(got, want)
    print(f"[mq decoder layout {hq}/{hkv}x{d} splits {mq_splits}] rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-3, err
