#!/usr/bin/env python3
"""Benchmark of the Q4_K decode hot path on one MI355X.

Headline (`value`): Q4_K_M decode GEMV throughput in GB/s of algorithmic
bytes on the 2B-class FFN-up shape M=1, N=9216, K=2304 (weights 11,943,936 B
+ x 9,216 B + y 36,864 B = 11,990,016 B per GEMV).  One step is one GEMV
on one of at least 48 distinct weight copies (rotated, so every copy is read
again only after 47 others, 561 MB: the weights stream from HBM, not from the
256 MB Infinity Cache).  A timed window is exactly `--steps` back-to-back
launches; `--windows` windows continue the rotation inside one HIP graph
(host launch cost is not timed), with a device timestamp on the kernel's
stream between windows, and the headline is the median window divided by
`--steps`.  HIP events around the timed graph replay give the mean over the
whole timed region beside it.  Inputs are synthetic and seeded.

`roofline` reports that per-launch time against the 8 TB/s HBM peak, with
the HBM traffic per launch measured by rocprofv3 counters (read from the
committed profile summary).  `cpu_baseline` times the single-threaded CPU
oracle on a bounded sample of the same workload on this host: the median of
its per-GEMV times.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Q4_K GEMV HBM GB/s (% of peak) + decode tok/s, 2B-class bs=1"
HBM_PEAK_GBS = 8000.0
N, K = 9216, 2304
GEMV_BYTES = N * (K // 256) * 144 + 4 * K + 4 * N  # 11,990,016
CPU_DECODE_RUNS = 5  # oracle decode steps per CPU baseline (the median is reported)
MIN_COPIES = 48  # 48 x 11.94 MB = 573 MB: more than twice the 256 MB Infinity Cache


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def timed_gemv_windows(doe, n, k, steps, warmup, copies, windows, seed):
    """Q4_K GEMVs over distinct weight copies, timed in windows of exactly
    `steps` back-to-back launches.  The windows continue one rotation over
    the copies, so every copy is read again only after the `copies - 1`
    others: with at least 48 copies of the 12 MB config that is more than
    the 256 MB Infinity Cache holds.  All windows sit in one HIP graph with a
    device timestamp (doe_device_timestamp, the GPU's constant 100 MHz clock,
    on the kernel's stream) before the first window and after each one, and
    the graph replays once untimed (a full rotation, and at least `warmup`
    launches) before the timed replay, which HIP events on the same stream
    also bracket.  A graph launch of its own per window would put ~10 us of
    graph-launch time into every window (0.5 us per launch at 20 launches);
    event records inside a graph cannot be timed.  Returns the per-window
    times: the headline is the median window divided by `steps`, the events
    give the mean over the timed region (timestamp kernels included)."""
    import ctypes as C

    from doe_amd import DeviceBuffer, Event, Graph, Stream, _lib, ops, q4k

    rng = np.random.default_rng(seed)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    if steps <= copies:
        copies = steps * -(-copies // steps)  # whole windows per rotation
    per_rot = copies // math.gcd(copies, steps)  # windows that end a rotation
    windows = per_rot * -(-max(windows, per_rot) // per_rot)  # whole rotations per replay
    bufs = [DeviceBuffer.from_array(w)]
    for _ in range(copies - 1):
        b = DeviceBuffer(w.nbytes)
        b.copy_from(bufs[0])
        bufs.append(b)
    dx = DeviceBuffer.from_array(x)
    dy = DeviceBuffer.empty((n,), np.float32)
    ts = DeviceBuffer.empty((windows + 1,), np.uint64)
    hz = C.c_int64()
    _lib.call("doe_device_timestamp_hz", C.byref(hz))
    doe.synchronize()
    s = Stream()
    sp = C.c_void_p(s.handle)

    def body():
        _lib.call("doe_device_timestamp", C.c_void_p(ts.ptr), sp)
        for i in range(windows):
            for j in range(steps):
                ops.matmul_q4k(bufs[(i * steps + j) % copies], dx, dy, n, k, s)
            _lib.call("doe_device_timestamp", C.c_void_p(ts.ptr + 8 * (i + 1)), sp)

    graph = Graph.capture(s, body)
    for _ in range(max(1, -(-warmup // (windows * steps)))):
        graph.launch(s)  # untimed: a full rotation (and the warmup launches)
    s.synchronize()
    doe.synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(s)
    graph.launch(s)
    e1.record(s)
    e1.synchronize()
    doe.synchronize()
    wall = time.perf_counter() - t0
    stamps = ts.download().astype(np.int64)
    win_ms = [float(d) / hz.value * 1e3 for d in np.diff(stamps)]
    ev_ms = e0.elapsed_ms(e1)
    from oracle import oracle as ora  # the reference answer, outside the timed region

    got = dy.download()
    want = ora.q4k_gemv(w, x, n, k)
    rel = float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want))
    graph.destroy()
    s.destroy()
    for c in bufs + [dx, dy, ts]:
        c.free()
    med = float(np.median(win_ms))
    return {
        "steps": steps,
        "copies": copies,
        "windows": windows,
        "reuse_distance_bytes": (copies - 1) * w.nbytes,
        "ms_per_step": med / steps,
        "mean_ms_per_step": float(np.mean(win_ms)) / steps,
        "event_ms_per_step": ev_ms / (windows * steps),
        "window_ms": win_ms,
        "wall_s": wall,
        "rel_l2": rel,
        "w": w,
        "x": x,
    }


def bench_gemv(args, doe):
    copies = max(args.copies, MIN_COPIES)
    log(f"gemv: N={N} K={K}, windows of {args.steps} launches over >= {copies} rotating weight copies")
    r = timed_gemv_windows(doe, N, K, args.steps, args.warmup, copies, args.windows, seed=0)
    log(f"gemv: rel_l2 vs oracle {r['rel_l2']:.3e}; {r['ms_per_step'] * 1e3:.3f} us/launch (median of "
        f"{r['windows']} windows of {r['steps']} launches over {r['copies']} copies; window mean "
        f"{r['mean_ms_per_step'] * 1e3:.3f}, HIP events over the timed region {r['event_ms_per_step'] * 1e3:.3f}), "
        f"wall {r['wall_s']:.3f}s")
    r["value_gbs"] = GEMV_BYTES / (r["ms_per_step"] * 1e-3) / 1e9
    r["kernel"] = "q4k_gemv_mfma_kernel<0, 1, 1, 0> (doe_amd/csrc/q4k_gemv.hip)"
    return r


GL_N = 65536


def bench_gemv_large(args, doe):
    """The same Q4_K GEMV at N=65536, K=2304 (85 MB of weights per launch,
    the streaming kernel), where the per-dispatch latency is amortised over
    more bytes: windows of 50 launches over 10 rotating copies (850 MB)."""
    byt = GL_N * (K // 256) * 144 + 4 * K + 4 * GL_N
    copies = max(2, -(-768 * 2 ** 20 // (GL_N * (K // 256) * 144)))
    r = timed_gemv_windows(doe, GL_N, K, 5 * copies, 0, copies, args.windows, seed=5)
    gbs = byt / (r["ms_per_step"] * 1e-3) / 1e9
    log(f"gemv N={GL_N} K={K}: {r['ms_per_step'] * 1e3:.2f} us/launch, {gbs:.0f} GB/s "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of peak), rel_l2 {r['rel_l2']:.2e}")
    return {"workload": f"q4k_gemv M=1 N={GL_N} K={K}, {r['copies']} rotating weight copies, median of "
                        f"{r['windows']} windows of {r['steps']} launches in one HIP graph",
            "kernel": "q4k_gemv_stream_kernel<0, 1, 2, 1> (doe_amd/csrc/q4k_gemv.hip)",
            "launches_per_window": r["steps"], "windows": r["windows"],
            "us_per_launch": round(r["ms_per_step"] * 1e3, 3),
            "mean_us_per_launch": round(r["mean_ms_per_step"] * 1e3, 3),
            "event_us_per_launch": round(r["event_ms_per_step"] * 1e3, 3), "bytes_per_launch": byt,
            "achieved_gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "rel_l2_vs_oracle": r["rel_l2"]}


ATT_HQ, ATT_HKV, ATT_D, ATT_T = 8, 4, 256, 4096
ATT_BYTES = 2 * ATT_HKV * ATT_T * ATT_D * 2 + 2 * ATT_HQ * ATT_D * 2  # K + V + q + o = 16,785,408


def bench_attention(args, doe):
    """GQA decode attention (8 q / 4 kv heads, head_dim 256, context 4096, f16
    q/K/V, f16 out) over rotating KV-cache copies; HIP events around graph
    replays of back-to-back calls."""
    from doe_amd import DeviceBuffer, Event, Graph, Stream, ops

    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, ATT_HQ, ATT_D)).astype(np.float16)
    k = rng.standard_normal((1, ATT_HKV, ATT_T, ATT_D)).astype(np.float16)
    v = rng.standard_normal((1, ATT_HKV, ATT_T, ATT_D)).astype(np.float16)
    ncopy = args.attn_copies
    dq = DeviceBuffer.from_array(q)
    ks, vs = [DeviceBuffer.from_array(k)], [DeviceBuffer.from_array(v)]
    for _ in range(ncopy - 1):
        kb, vb = DeviceBuffer(k.nbytes), DeviceBuffer(v.nbytes)
        kb.copy_from(ks[0])
        vb.copy_from(vs[0])
        ks.append(kb)
        vs.append(vb)
    out = DeviceBuffer.empty((1, ATT_HQ, ATT_D), np.float16)
    doe.synchronize()
    s = Stream()

    def body():
        for kb, vb in zip(ks, vs):
            ops.attention(dq, kb, vb, out, batch=1, num_heads=ATT_HQ, num_kv_heads=ATT_HKV, head_dim=ATT_D,
                          kv_len=ATT_T, kv_stride=ATT_T, scale=1.0 / 16, q_f16=True, out_f16=True, stream=s)

    body()  # first call outside capture allocates the split workspace
    s.synchronize()
    graph = Graph.capture(s, body)
    graph.launch(s)
    s.synchronize()
    reps = max(1, -(-args.attn_steps // ncopy))
    e0, e1 = Event(), Event()
    e0.record(s)
    for _ in range(reps):
        graph.launch(s)
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / (reps * ncopy)
    from oracle import oracle as ora

    want = ora.attn_decode(q[0].astype(np.float32), k[0], v[0], ATT_HQ, ATT_HKV, ATT_D, ATT_T, ATT_T, 1.0 / 16)
    got = out.download()[0].astype(np.float64)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    graph.destroy()
    s.destroy()
    for b in ks + vs:
        b.free()
    gbs = ATT_BYTES / (ms * 1e-3) / 1e9
    log(f"attention: {ms * 1e3:.2f} us/call, {gbs:.0f} GB/s, rel_l2 {rel:.2e}")
    return {
        "workload": f"GQA decode attention Hq={ATT_HQ} Hkv={ATT_HKV} D={ATT_D} T={ATT_T}, f16 q/K/V/out, "
                    f"{ncopy} rotating KV copies",
        "us_per_call": round(ms * 1e3, 3),
        "bytes_per_call": ATT_BYTES,
        "achieved_gbs": round(gbs, 1),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "rel_l2_vs_oracle": rel,
    }


def bench_decode(args, doe, cfg=None, plan=None, label="2B-class decoder", cpu_runs=CPU_DECODE_RUNS):
    """2B-class decode loop at batch 1 (26 layers, hidden 2304, 8/4 heads of
    256, FFN 9216 GeGLU, Q4_K projections, f16 lm_head over 256000): a
    128-token prompt then `--decode-steps` greedy steps, each step a replay of
    a captured HIP graph; tokens/s over the decode steps (HIP events).  cfg /
    plan: another model shape and its execution-v1 decode plan."""
    from doe_amd import Stream
    from doe_amd.model import Decoder, DecoderConfig

    cfg = cfg or DecoderConfig()
    # a batched prompt samples one token before the first decode step: room
    # for prompt + 1 + decode_steps ids (the KV cache uses one row fewer),
    # and a row for the parity step after the trajectory
    need = args.prompt_len + args.decode_steps + 2
    if cfg.max_seq < need:
        cfg = dataclasses.replace(cfg, max_seq=need)
    dec = Decoder(cfg, plan=plan)
    dec.init_random(seed=2)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, cfg.vocab, args.prompt_len, dtype=np.int64).astype(np.int32)
    s = Stream()
    dec.reset(prompt)
    dec.step(s)  # allocates the attention workspace outside capture
    s.synchronize()
    spg = args.steps_per_graph  # 0: eager launches (no graph), e.g. under a profiler
    graph = dec.capture(s, spg) if spg > 0 else None
    # the prompt as one batched pass (uniform Q4_K models), then exactly
    # --decode-steps decode steps; else the prompt as teacher-forced steps
    pf = dec.can_prefill() and not args.no_prefill
    n_new = args.decode_steps + (1 if pf else 0)
    dec.generate(prompt, min(16, n_new), s, graph=graph, steps_per_graph=max(spg, 1), prefill=pf)  # warm
    timing = {}
    ids = dec.generate(prompt, n_new, s, graph=graph, steps_per_graph=max(spg, 1), timing=timing, prefill=pf)
    if graph is not None:
        graph.destroy()
    end = trajectory_end_parity(dec, s) if cpu_runs > 1 else None
    parity, cpu = decode_parity_and_cpu(dec, prompt, s, cpu_runs)
    if end is not None:
        parity.update(end)
    tok_s = args.decode_steps / timing["decode_s"]
    mean_len = args.prompt_len + (args.decode_steps + 1) / 2.0
    bpt = dec.decode_bytes_per_token(mean_len)
    gbs = bpt * tok_s / 1e9
    prompt_mode = "one batched prefill pass" if pf else f"{args.prompt_len - 1} teacher-forced decode steps"
    log(f"decode ({label}): {tok_s:.1f} tok/s ({timing['decode_s'] * 1e3 / args.decode_steps:.3f} ms/token), "
        f"prompt {timing['prompt_s'] * 1e3:.2f} ms ({prompt_mode}, {args.prompt_len / timing['prompt_s']:.0f} "
        f"prompt tok/s), {gbs:.0f} GB/s of algorithmic bytes")
    return {
        "workload": f"{label} bs=1: {cfg.layers} layers, hidden {cfg.hidden}, {cfg.heads}/{cfg.kv_heads} "
                    f"heads x {cfg.head_dim}, FFN {cfg.ffn} GeGLU, vocab {cfg.vocab}; "
                    f"{'Q8_0' if cfg.weight_format == 'q8_0' else 'Q4_K'} projections, f16 "
                    f"lm_head, f16 KV; prompt {args.prompt_len} then {args.decode_steps} greedy steps; "
                    f"random-init weights; " + (f"{spg} steps per HIP graph" if spg > 0 else "eager launches"),
        "tok_s": round(tok_s, 2),
        "ms_per_token": round(timing["decode_s"] * 1e3 / args.decode_steps, 4),
        "bytes_per_token": int(bpt),
        "achieved_gbs": round(gbs, 1),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "ceiling_tok_s_at_peak": round(HBM_PEAK_GBS * 1e9 / bpt, 1),
        "prompt_s": round(timing["prompt_s"], 5),
        "prompt_tok_s": round(args.prompt_len / timing["prompt_s"], 1),
        "prompt_mode": prompt_mode,
        "last_tokens": [int(t) for t in ids[-4:]],
        "parity": parity,
        "cpu_baseline": cpu,
    }


def trajectory_end_parity(dec, s):
    """Outside the timed region, where the timed trajectory ended: one more
    eager decode step (attention over every key the prompt pass and the
    decode steps wrote) against the oracle decoder's step at that position,
    which reads the KV cache the device wrote."""
    from oracle.decoder import OracleDecoder

    pos, _, _, tok = (int(v) for v in dec.state.download())
    if pos + 1 > dec.cfg.max_seq:
        return None
    oracle = OracleDecoder(dec)
    oracle.load_kv(dec)
    dec.keep_logits = True
    dec.step(s)
    s.synchronize()
    got = dec.logits.download().astype(np.float64)
    gtok = int(dec.token.download()[0])
    dec.keep_logits = False
    want = oracle.step(pos, tok)
    del oracle
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    log(f"  decode parity at the trajectory's end: position {pos} ({pos + 1} keys), logits rel_l2 {rel:.2e}, "
        f"token {gtok} vs oracle {int(np.argmax(want))}")
    return {"end_position": pos, "end_logits_rel_l2_vs_oracle": rel, "end_token_equal": gtok == int(np.argmax(want))}


def decode_parity_and_cpu(dec, prompt, s, runs=CPU_DECODE_RUNS):
    """Outside the timed region: one eager decode step at position 0 with the
    logits kept, against the oracle decoder (the CPU restatement composed from
    the oracle's kernels, on the device's weights); the oracle step's own
    single-threaded time is the decode CPU baseline."""
    from oracle.decoder import OracleDecoder

    dec.keep_logits = True
    dec.reset(prompt)
    dec.step(s)
    s.synchronize()
    got = dec.logits.download().astype(np.float64)
    tok = int(dec.token.download()[0])
    dec.keep_logits = False
    oracle = OracleDecoder(dec)
    times = []
    for _ in range(runs):  # step 0 again each time: the same work, the same logits
        t0 = time.perf_counter()
        want = oracle.step(0, int(prompt[0]))
        times.append(time.perf_counter() - t0)
    el = float(np.median(times))
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    del oracle
    log(f"  decode parity: step-0 logits rel_l2 {rel:.2e}, token {tok} vs oracle {int(np.argmax(want))}; "
        f"oracle step {el:.2f} s (median of {len(times)})")
    parity = {"step0_logits_rel_l2_vs_oracle": rel, "step0_token_equal": tok == int(np.argmax(want)),
              "tolerance": 1e-3}
    cpu = {"value": round(1.0 / el, 4), "unit": "tok/s", "cores": 1, "kind": "port", "runs": len(times),
           "sample": f"{'median of ' if len(times) > 1 else ''}{len(times)} full-size decode step"
                     f"{'s' if len(times) > 1 else ''} (position 0, every weight of every layer and "
                     f"the lm_head) of the single-threaded C oracle decoder (f32 left-fold, -O2 "
                     f"-ffp-contract=off), {el:.2f} s each, on {cpu_model()} ({os.cpu_count()} logical cores on "
                     f"host); attention at position 0 reads 1 key (< 1% of a token's bytes at the benchmarked "
                     f"lengths)"}
    return parity, cpu


def bench_decode_graph(args, doe):
    """The decode loop planned from the reference's gemma-3-270m execution-v1
    manifest graph (runtime/zig/examples/execution-v1/gemma-3-270m-manifest-
    smoke.json, kept as a test fixture) at that model's shapes: 18 layers,
    hidden 640, 4/1 heads of 256, FFN 2048, vocab 262144; random weights."""
    from doe_amd import execution as ex
    from doe_amd.model import DecoderConfig

    graph = ex.load_step_graph(ROOT / "tests" / "golden" / "execution_v1" / "gemma-3-270m-manifest-smoke.json")
    cfg = DecoderConfig(layers=18, hidden=640, heads=4, kv_heads=1, head_dim=256, ffn=2048, vocab=262144,
                        max_seq=384)
    res = bench_decode(args, doe, cfg, ex.plan_decode(graph, cfg.layers),
                       label=f"{graph.model_id} (execution-v1 manifest graph)")
    return res


def bench_decode_31b(args, doe):
    """The decode loop planned from the reference's Gemma 4 31B af16 graph
    (runtime/zig/examples/execution-v1/gemma-4-31b-af16-smoke.json, kept as
    a test fixture) at that model's full shapes: 60 layers, hidden 5376, 32 /
    16 heads of 256, FFN 21504 GeGLU, vocab 262144, every layer sliding over
    512 keys (the graph's attention_sliding step); Q4_K projections, f16
    lm_head and KV; random-init weights.  Step-0 parity against the oracle
    decoder; its CPU baseline is one oracle step (~16 GB of Q4_K weights)."""
    from doe_amd import execution as ex
    from doe_amd.model import DecoderConfig

    graph = ex.load_step_graph(ROOT / "tests" / "golden" / "execution_v1" / "gemma-4-31b-af16-smoke.json")
    mc = graph.model_config
    cfg = DecoderConfig.from_model_config(mc, max_seq=384, norm_weight_offset=False, rope_base_global=1e6)
    plan = ex.plan_decode(graph, cfg.layers, cfg.head_dim, cfg.global_head_dim)
    return bench_decode(args, doe, cfg, plan, label=f"{graph.model_id} (execution-v1 graph, 31B-class)", cpu_runs=1)


GEMM_M, GEMM_N, GEMM_K = 2048, 21504, 5376
GEMM_FLOP = 2 * GEMM_M * GEMM_N * GEMM_K  # 473,520,144,384
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16


def to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bench_gemm(args, doe):
    """Q4_K dequant-fused prefill GEMM at the 31B-class shape (M=2048 tokens,
    K=5376, N=21504; bf16 activations N(0,1), Q4_K weights, f32 output); HIP
    events around back-to-back calls (each call = the bf16->f16 row pre-pass
    plus the GEMM kernel); sampled parity against the oracle."""
    import ctypes as C

    from doe_amd import DeviceBuffer, Event, Stream, _lib, ops
    from doe_amd import q4k as q4kmod

    rng = np.random.default_rng(3)
    a = to_bf16(rng.standard_normal((GEMM_M, GEMM_K), dtype=np.float32))
    da = DeviceBuffer.from_array(a)
    db = DeviceBuffer(GEMM_N * q4kmod.row_bytes(GEMM_K))
    _lib.call("doe_fill_random_q4k", C.c_void_p(db.ptr), db.nbytes // q4kmod.BLOCK_BYTES, 33, 0.02, 0.01,
              C.c_void_p(None))
    dc = DeviceBuffer.empty((GEMM_M, GEMM_N), np.float32)
    s = Stream()
    for _ in range(2):
        ops.matmul_q4k_gemm(da, db, dc, GEMM_M, GEMM_N, GEMM_K, stream=s)
    s.synchronize()
    reps = args.gemm_steps
    e0, e1 = Event(), Event()
    e0.record(s)
    for _ in range(reps):
        ops.matmul_q4k_gemm(da, db, dc, GEMM_M, GEMM_N, GEMM_K, stream=s)
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    from oracle import oracle as ora

    b = db.download().reshape(GEMM_N, -1)
    mi = np.arange(0, GEMM_M, 8, dtype=np.int64)
    ni = np.sort(rng.integers(0, GEMM_N, mi.size)).astype(np.int64)
    want = ora.q4k_gemm_sampled(a, b, GEMM_M, GEMM_N, GEMM_K, mi, ni)
    got = dc.download()[mi, ni].astype(np.float64)
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    s.destroy()
    for buf in (da, db, dc):
        buf.free()
    tflops = GEMM_FLOP / (ms * 1e-3) / 1e12
    log(f"gemm: {ms * 1e3:.1f} us/call, {tflops:.0f} TFLOP/s ({100 * tflops / MFMA_F16_PEAK_TFLOPS:.1f}% of "
        f"the f16 MFMA peak), sampled rel_l2 {rel:.2e}")
    return {
        "workload": f"q4k_gemm M={GEMM_M} N={GEMM_N} K={GEMM_K}: bf16 activations, Q4_K_M weights, f32 out "
                    f"(f16 matrix cores, f32 accumulate)",
        "us_per_call": round(ms * 1e3, 2),
        "flop_per_call": GEMM_FLOP,
        "achieved_tflops": round(tflops, 1),
        "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
        "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "rel_l2_vs_oracle_sampled": rel,
    }


PF_HQ, PF_HKV, PF_D, PF_S = 32, 16, 128, 2048
PF_FLOP = PF_HQ * PF_D * 4 * PF_S * (PF_S + 1) // 2  # causal: q.k and p.v over keys 0..i


def bench_prefill_attention(args, doe):
    """Causal GQA prefill attention at the 31B-class shape (32 q / 16 kv heads,
    head_dim 128, 2048 tokens, bf16 q/K/V N(0,1), f32 out); HIP events around
    back-to-back calls; oracle parity on sampled rows."""
    from doe_amd import DeviceBuffer, Event, Stream, ops

    rng = np.random.default_rng(4)
    q = to_bf16(rng.standard_normal((PF_S, PF_HQ, PF_D), dtype=np.float32))
    k = to_bf16(rng.standard_normal((PF_HKV, PF_S, PF_D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((PF_HKV, PF_S, PF_D), dtype=np.float32))
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    out = DeviceBuffer.empty((PF_S, PF_HQ, PF_D), np.float32)
    s = Stream()
    scale = 1.0 / math.sqrt(PF_D)

    def call():
        ops.attention_prefill(dq, dk, dv, out, num_heads=PF_HQ, num_kv_heads=PF_HKV, head_dim=PF_D, q_len=PF_S,
                              kv_len=PF_S, scale=scale, causal=True, stream=s)

    for _ in range(2):
        call()
    s.synchronize()
    reps = args.gemm_steps
    e0, e1 = Event(), Event()
    e0.record(s)
    for _ in range(reps):
        call()
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    from oracle import oracle as ora

    f = lambda b: (b.astype(np.uint32) << 16).view(np.float32)
    got = out.download()
    errs = []
    for r0, r1 in ((0, 8), (1024, 1032), (2040, 2048)):
        want = ora.attn_prefill(f(q), f(k), f(v), PF_HQ, PF_HKV, PF_D, PF_S, PF_S, 0, scale, True, (r0, r1))
        errs.append(float(np.linalg.norm(got[r0:r1] - want[r0:r1]) / np.linalg.norm(want[r0:r1])))
    s.destroy()
    for b in (dq, dk, dv, out):
        b.free()
    tflops = PF_FLOP / (ms * 1e-3) / 1e12
    log(f"prefill attention: {ms * 1e3:.1f} us/call, {tflops:.0f} TFLOP/s "
        f"({100 * tflops / MFMA_F16_PEAK_TFLOPS:.1f}% of the bf16/f16 MFMA peak), sampled rel_l2 {max(errs):.2e}")
    return {
        "workload": f"causal GQA prefill attention Hq={PF_HQ} Hkv={PF_HKV} D={PF_D} S={PF_S}, bf16 q/K/V, f32 out",
        "us_per_call": round(ms * 1e3, 2),
        "flop_per_call": PF_FLOP,
        "achieved_tflops": round(tflops, 1),
        "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "rel_l2_vs_oracle_sampled": max(errs),
    }


C4_B, C4_HQ, C4_HKV, C4_D, C4_T = 8, 64, 8, 128, 32768
C4_GEMVS = (("qkv", 9216, 5120), ("ffn_up", 25600, 5120), ("ffn_down", 5120, 25600))


def bench_config4(args, doe):
    """27B-class long-context decode at batch 8, per layer: GQA attention over
    32768 cached positions per sequence (64 q / 8 kv heads, head_dim 128, f16
    K/V = 1 GiB) and the int4 group-32 GEMVs (QKV 5120->9216, FFN 5120->25600
    ->5120, f16 scales) at M = 8.  HIP events around back-to-back calls; the
    GEMVs rotate weight copies so the 256 MB Infinity Cache cannot hold them."""
    import ctypes as C

    from doe_amd import DeviceBuffer, Event, Stream, _lib, ops

    s = Stream()
    sp = C.c_void_p(s.handle)

    def timed(fn, reps):
        fn(0)
        s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for i in range(reps):
            fn(i)
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    res = {}
    # attention
    k = DeviceBuffer.empty((C4_B, C4_HKV, C4_T, C4_D), np.float16)
    v = DeviceBuffer.empty((C4_B, C4_HKV, C4_T, C4_D), np.float16)
    _lib.call("doe_fill_normal_f16", C.c_void_p(k.ptr), k.nbytes // 2, 41, 0.0, 1.0, sp)
    _lib.call("doe_fill_normal_f16", C.c_void_p(v.ptr), v.nbytes // 2, 42, 0.0, 1.0, sp)
    q = DeviceBuffer.empty((C4_B, C4_HQ, C4_D), np.float16)
    _lib.call("doe_fill_normal_f16", C.c_void_p(q.ptr), q.nbytes // 2, 43, 0.0, 1.0, sp)
    o = DeviceBuffer.empty((C4_B, C4_HQ, C4_D), np.float16)
    ms = timed(lambda i: ops.attention(q, k, v, o, batch=C4_B, num_heads=C4_HQ, num_kv_heads=C4_HKV, head_dim=C4_D,
                                       kv_len=C4_T, kv_stride=C4_T, scale=1.0 / math.sqrt(C4_D), q_f16=True,
                                       out_f16=True, stream=s), 10)
    att_bytes = k.nbytes + v.nbytes + q.nbytes + o.nbytes
    res["attention"] = {"us_per_call": round(ms * 1e3, 2), "bytes_per_call": att_bytes,
                        "achieved_gbs": round(att_bytes / (ms * 1e-3) / 1e9, 1)}
    for b in (k, v, q, o):
        b.free()
    # int4 GEMVs
    rng = np.random.default_rng(44)
    x = DeviceBuffer.from_array(rng.standard_normal((C4_B, 25600), dtype=np.float32))
    total_us, total_bytes = res["attention"]["us_per_call"], att_bytes
    for name, n, kdim in C4_GEMVS:
        wbytes, sbytes = n * kdim // 2, n * (kdim // 32) * 2
        copies = max(2, -(-768 * 2 ** 20 // (wbytes + sbytes)))
        ws = [DeviceBuffer(wbytes) for _ in range(copies)]
        ss = [DeviceBuffer(sbytes) for _ in range(copies)]
        for i in range(copies):
            _lib.call("doe_fill_uniform_i32", C.c_void_p(ws[i].ptr), wbytes // 4, 50 + i, -2 ** 31, 2 ** 31 - 1, sp)
            _lib.call("doe_fill_normal_f16", C.c_void_p(ss[i].ptr), sbytes // 2, 60 + i, 0.0, 0.02, sp)
        y = DeviceBuffer.empty((C4_B, n), np.float32)
        ms = timed(lambda i: ops.matmul_int4g32(ws[i % copies], ss[i % copies], x, y, C4_B, n, kdim, stream=s),
                   4 * copies)
        byt = wbytes + sbytes + C4_B * kdim * 4 + C4_B * n * 4
        res[name] = {"m_n_k": [C4_B, n, kdim], "us_per_call": round(ms * 1e3, 2), "bytes_per_call": byt,
                     "achieved_gbs": round(byt / (ms * 1e-3) / 1e9, 1), "weight_copies": copies}
        total_us += ms * 1e3
        total_bytes += byt
        for b in ws + ss + [y]:
            b.free()
    x.free()
    s.destroy()
    res["layer_us"] = round(total_us, 2)
    res["layer_bytes"] = total_bytes
    res["layer_gbs"] = round(total_bytes / (total_us * 1e-6) / 1e9, 1)
    log(f"config4 (batch 8, 32k context): attention {res['attention']['us_per_call']} us "
        f"({res['attention']['achieved_gbs']} GB/s); int4 GEMVs " +
        ", ".join(f"{nm} {res[nm]['us_per_call']} us ({res[nm]['achieved_gbs']} GB/s)" for nm, _, _ in C4_GEMVS))
    return {"workload": "27B-class batch-8 long-context decode layer: GQA attention 64q/8kv x 128 over 32768 "
                        "positions (f16 KV, 1 GiB), int4 group-32 GEMVs with f16 scales at M=8", **res}


Q8_N, Q8_K = 9216, 2304


def bench_q8_0(args, doe):
    """The Q8_0 GEMV at the headline GEMV's shape (9216 x 2304, 34-byte
    blocks): rotating weight copies (more bytes than the 256 MB Infinity
    Cache) replayed in a HIP graph, HIP events around the replays."""
    from doe_amd import DeviceBuffer, Event, Graph, Stream, ops, q8_0
    from oracle import oracle as ora

    rng = np.random.default_rng(7)
    w = q8_0.random_q8_0(rng, Q8_N, Q8_K)
    x = rng.standard_normal(Q8_K, dtype=np.float32)
    copies = max(2, -(-384 * 2 ** 20 // w.nbytes))
    bufs = [DeviceBuffer.from_array(w)]
    for _ in range(copies - 1):
        b = DeviceBuffer(w.nbytes)
        b.copy_from(bufs[0])
        bufs.append(b)
    dx = DeviceBuffer.from_array(x)
    dy = DeviceBuffer.empty((Q8_N,), np.float32)
    s = Stream()
    graph = Graph.capture(s, lambda: [ops.matmul_q8_0(c, dx, dy, Q8_N, Q8_K, stream=s) for c in bufs])
    graph.launch(s)
    s.synchronize()
    reps = max(1, -(-args.steps // copies))
    e0, e1 = Event(), Event()
    e0.record(s)
    for _ in range(reps):
        graph.launch(s)
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / (reps * copies)
    rel = float(np.linalg.norm(dy.download().astype(np.float64) - ora.q8_0_gemv(w, x, Q8_N, Q8_K)) /
                np.linalg.norm(ora.q8_0_gemv(w, x, Q8_N, Q8_K)))
    graph.destroy()
    s.destroy()
    for b in bufs:
        b.free()
    byt = w.nbytes + Q8_K * 4 + Q8_N * 4
    gbs = byt / (ms * 1e-3) / 1e9
    log(f"q8_0 gemv {Q8_N}x{Q8_K}: {ms * 1e3:.2f} us, {gbs:.1f} GB/s, rel_l2 {rel:.2e}")
    return {"workload": f"q8_0_gemv M=1 N={Q8_N} K={Q8_K} (Q8_0 weights, f32 activation/output), "
                        f"{copies} rotating weight copies, HIP-graph replay",
            "kernel": "q8_0_gemv_kernel<2, 1> (doe_amd/csrc/q8_0_gemv.hip)",
            "us_per_call": round(ms * 1e3, 3), "bytes_per_call": byt, "achieved_gbs": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "rel_l2_vs_oracle": rel}


def bench_hbm_copy(args, doe):
    """STREAM-style checks of the HBM figure the rooflines use, on 2 GiB
    buffers: a device-to-device copy by the runtime's copy kernel (read and
    written bytes both counted), and this library's own read stream
    (doe_read_xor_u32: every 16-byte word loaded once, XOR-folded to one
    checksum), ten of each between HIP events."""
    import ctypes as C

    from doe_amd import DeviceBuffer, Event, Stream, _lib

    nbytes = 1 << 31
    src, dst = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    s = Stream()
    sp = C.c_void_p(s.handle)
    _lib.call("doe_fill_uniform_i32", C.c_void_p(src.ptr), nbytes // 4, 77, -2 ** 31, 2 ** 31 - 1, sp)
    dst.copy_from(src, s)
    s.synchronize()
    reps = 10

    def timed(fn):
        e0, e1 = Event(), Event()
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    ms = timed(lambda: dst.copy_from(src, s))
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    ck = DeviceBuffer.empty((2,), np.uint32)
    read = lambda: _lib.call("doe_read_xor_u32", C.c_void_p(src.ptr), nbytes, C.c_void_p(ck.ptr), 0, sp)
    read()
    s.synchronize()
    first = int(ck.download()[0])
    ms_r = timed(read)
    same = int(ck.download()[0]) == first
    gbs_r = nbytes / (ms_r * 1e-3) / 1e9
    s.destroy()
    for b in (src, dst, ck):
        b.free()
    log(f"hbm copy: 2 GiB device-to-device in {ms * 1e3:.1f} us = {gbs:.0f} GB/s read + write "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of the {HBM_PEAK_GBS:.0f} GB/s figure); read stream {ms_r * 1e3:.1f} us "
        f"= {gbs_r:.0f} GB/s ({100 * gbs_r / HBM_PEAK_GBS:.1f}%), checksum stable: {same}")
    return {"kind": "STREAM copy: hipMemcpyAsync device to device, read + write bytes counted",
            "bytes_per_copy": nbytes, "us_per_copy": round(ms * 1e3, 1), "achieved_gbs": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "read_stream": {"kind": "doe_read_xor_u32: 2 GiB read once with 16-byte non-temporal loads "
                                    "(512 x 256 threads), XOR-folded",
                            "bytes": nbytes, "us": round(ms_r * 1e3, 1), "achieved_gbs": round(gbs_r, 1),
                            "frac_of_hbm_peak": round(gbs_r / HBM_PEAK_GBS, 4), "checksum_stable": same}}


def traffic_bytes(summary: str):
    """HBM bytes per launch recorded in a committed rocprofv3 summary
    (line `traffic_bytes_per_launch: <int>`), or None."""
    path = ROOT / "profiles" / summary
    try:
        for line in path.read_text().splitlines():
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def cpu_baseline(w, x, seconds: float):
    """The single-threaded C oracle on the full config-0 GEMV, called back to
    back for about `seconds` (at least 5 calls); the value is the algorithmic
    bytes over the median call time."""
    from oracle import oracle as ora

    ora.lib()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        ora.q4k_gemv(w, x, N, K)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {
        "value": GEMV_BYTES / med / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "runs": len(times),
        "median_s": med,
        "sample": f"median of {len(times)} full N={N} K={K} Q4_K GEMVs ({med * 1e3:.2f} ms each; single-threaded "
                  f"C oracle, f32 left-fold, -O2 -ffp-contract=off) on {cpu_model()} "
                  f"({os.cpu_count()} logical cores on host)",
    }


def cpu_baseline_all_cores(w, x, seconds: float):
    """The same oracle GEMV with its rows split over the host's cores (at
    most 16 threads, the CPU share of one GPU on the box); reported beside
    the single-threaded baseline, never as it."""
    from oracle import oracle as ora

    threads = max(1, min(os.cpu_count() or 1, 16))
    ora.q4k_gemv_threads(w, x, N, K, threads)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        ora.q4k_gemv_threads(w, x, N, K, threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {
        "value": GEMV_BYTES / med / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "runs": len(times),
        "median_s": med,
        "sample": f"median of {len(times)} full N={N} K={K} Q4_K GEMVs ({med * 1e3:.2f} ms each; the C oracle's "
                  f"rows split over {threads} threads, each row as single-threaded) on {cpu_model()} "
                  f"({os.cpu_count()} logical cores on host)",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="GEMV launches per timed window")
    ap.add_argument("--warmup", type=int, default=5, help="untimed GEMV launches after the first full rotation")
    ap.add_argument("--copies", type=int, default=64, help="rotating weight copies (at least 48 are used)")
    ap.add_argument("--windows", type=int, default=12, help="timed windows; the headline is their median")
    ap.add_argument("--attn-copies", type=int, default=48)
    ap.add_argument("--attn-steps", type=int, default=480)
    ap.add_argument("--prompt-len", type=int, default=128)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--steps-per-graph", type=int, default=8)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-31b", action="store_true", help="skip the 31B-class decode line")
    ap.add_argument("--no-prefill", action="store_true", help="run prompts as teacher-forced decode steps")
    ap.add_argument("--gemm-steps", type=int, default=20)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the library has no "
              f"multi-GPU path", file=sys.stderr)
        return 2
    if int(os.environ.get("RANK", "0")) != 0:
        return 0

    import doe_amd

    if not doe_amd.LIB_PATH.exists():
        print(f"{doe_amd.LIB_PATH} is not built", file=sys.stderr)
        return 1
    doe_amd.init(0)
    info = doe_amd.device_info()
    log(f"device {info}")

    g = bench_gemv(args, doe_amd)
    gl = None if args.no_gemm else bench_gemv_large(args, doe_amd)
    att = bench_attention(args, doe_amd)
    dec = None if args.no_decode else bench_decode(args, doe_amd)
    dec_graph = None if args.no_decode else bench_decode_graph(args, doe_amd)
    dec_q8 = None
    if not args.no_decode:
        from doe_amd.model import DecoderConfig

        dec_q8 = bench_decode(args, doe_amd, cfg=DecoderConfig(weight_format="q8_0"),
                              label="2B-class decoder, Q8_0 weights")
    dec_31b = None if args.no_decode or args.no_31b else bench_decode_31b(args, doe_amd)
    gemm = None if args.no_gemm else bench_gemm(args, doe_amd)
    pfa = None if args.no_gemm else bench_prefill_attention(args, doe_amd)
    c4 = None if args.no_gemm else bench_config4(args, doe_amd)
    q8 = bench_q8_0(args, doe_amd)
    hbm = bench_hbm_copy(args, doe_amd)
    cpu = cpu_all = None
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_seconds:.0f} s of the single-threaded oracle")
        cpu = cpu_baseline(g["w"], g["x"], args.cpu_seconds)
        log("cpu baseline, all cores: ~3 s of the oracle with its rows over the host threads")
        cpu_all = cpu_baseline_all_cores(g["w"], g["x"], 3.0)

    out = {
        "metric": METRIC,
        "value": round(g["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["steps"],
        "warmup": args.warmup,
        "ms_per_step": g["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"q4k_gemv M=1 N={N} K={K} (Q4_K_M weights, f32 activation/output), "
                        f"{g['copies']} rotating weight copies ({g['reuse_distance_bytes'] / 2 ** 20:.0f} MiB read "
                        f"between two reads of a copy), median of {g['windows']} windows of {g['steps']} "
                        f"back-to-back launches in one HIP graph, device timestamps between windows",
            "weight_copies": g["copies"],
            "windows": g["windows"],
            "bytes_per_step": GEMV_BYTES,
            "pct_of_hbm_peak": round(100.0 * g["value_gbs"] / HBM_PEAK_GBS, 2),
            "rel_l2_vs_oracle": g["rel_l2"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(g["value_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["value_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes("q4k_gemv_n9216_k2304.md"),
            "kernel": g["kernel"],
            "kernel_us": round(g["ms_per_step"] * 1e3, 3),
            "mean_kernel_us": round(g["mean_ms_per_step"] * 1e3, 3),
            "event_kernel_us": round(g["event_ms_per_step"] * 1e3, 3),
            "launches_per_window": g["steps"],
            "windows": g["windows"],
        },
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "gemv_n65536": gl,
        "attention_decode": att,
        "decode": dec,
        "decode_graph_gemma3_270m": dec_graph,
        "decode_q8_0": dec_q8,
        "decode_graph_gemma4_31b_af16": dec_31b,
        "prefill_gemm": gemm,
        "prefill_attention": pfa,
        "config4_decode_layer": c4,
        "q8_0_gemv": q8,
        "hbm_stream_copy": hbm,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
