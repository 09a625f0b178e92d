"""Benchmark of the Q4_K / Q6_K matmul hot path on one MI355X.

Workload (Llama-3.1-8B FFN decode at batch 1): one step =
fused Q4_K gate+up+SwiGLU GEMV (2 x 14336x4096) followed by the Q6_K
ffn_down GEMV (4096x14336) on its output.  `value` is the algorithmic HBM
bytes of one step divided by the measured step time (GB/s).  Weights are
seeded synthetic GGUF blocks generated in device memory; several distinct
weight copies are cycled so each step streams from HBM, not from the 256 MB
Infinity Cache.

Extra objects on the same JSON line: config 0 ("gemv_4096", the single
Q4_K GEMV), config 3 ("prefill_gemm": TFLOP/s at M = 64..512), config 2
("decode_stream"), config 4 ("e2e_qwen3_8b") and the CPU baseline.  Every
timed region is preceded by an untimed clock ramp of about 0.3 s of the
same launches, enqueued back to back and still running when the timed
region is enqueued behind them (the timed launches start on a busy GPU).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
K_FFN, N_FFN = 4096, 14336
Q4K_BYTES, Q6K_BYTES = 144, 210
# algorithmic bytes: N*(K/256)*B + 4K (x) + 4N (y)
GATE_UP_BYTES = 2 * N_FFN * (K_FFN // 256) * Q4K_BYTES + 4 * K_FFN + 4 * N_FFN      # 66,134,016
DOWN_BYTES = K_FFN * (N_FFN // 256) * Q6K_BYTES + 4 * N_FFN + 4 * K_FFN            # 48,242,688
STEP_BYTES = GATE_UP_BYTES + DOWN_BYTES
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the Qwen3-8B end-to-end leg (config 4)")
    ap.add_argument("--gemm-pmc", action="store_true", help="only launch the M=512 GEMMs (for rocprofv3 --pmc)")
    ap.add_argument("--no-stream", action="store_true", help="skip the full decode weight stream leg (config 2)")
    ap.add_argument("--stream-tokens", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run plain copies of known size (PMC traffic calibration)")
    return ap.parse_args()


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def bench_decode(lib, torch, steps, warmup):
    from rocmforge_amd import synth

    dev = torch.device("cuda:0")
    set_bytes = 2 * N_FFN * (K_FFN // 256) * Q4K_BYTES + K_FFN * (N_FFN // 256) * Q6K_BYTES
    copies = max(2, -(-4 * MALL_BYTES // set_bytes))          # >= 4x the Infinity Cache
    sets = []
    for c in range(copies):
        wg = synth.torch_weights("q4_k", N_FFN, K_FFN, seed=3 * c + 1, device=dev)
        wu = synth.torch_weights("q4_k", N_FFN, K_FFN, seed=3 * c + 2, device=dev)
        wd = synth.torch_weights("q6_k", K_FFN, N_FFN, seed=3 * c + 3, device=dev)
        sets.append((wg, wu, wd))
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(K_FFN, device=dev, generator=g)
    h = torch.empty(N_FFN, device=dev)
    y = torch.empty(K_FFN, device=dev)
    stream = torch.cuda.current_stream()
    st = ctypes.c_void_p(stream.cuda_stream)
    gu = lib.gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch
    dn = lib.gemv_q6_k_f32_launch

    def step(i, ev=None):
        wg, wu, wd = sets[i % copies]
        if ev is not None:
            ev[0].record(stream)
        rc = gu(vp(wg), vp(wu), vp(x), vp(h), K_FFN, N_FFN, st)
        if ev is not None:
            ev[1].record(stream)
        rc |= dn(vp(wd), vp(h), vp(y), N_FFN, K_FFN, st)
        if ev is not None:
            ev[2].record(stream)
        if rc:
            raise RuntimeError(f"launch failed: hipError {rc}")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    # The decode step is launched the way a decode loop launches it: captured
    # into a HIP graph and replayed.
    # The launchers allocate nothing and never synchronise, so they capture.
    def capture(fn_list):
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            with torch.cuda.graph(g, stream=cs):
                cst = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for f in fn_list:
                    f(cst)
        torch.cuda.current_stream().wait_stream(cs)
        torch.cuda.synchronize()
        return g

    def gu_call(c):
        return lambda cst: gu(vp(sets[c][0]), vp(sets[c][1]), vp(x), vp(h), K_FFN, N_FFN, cst)

    def dn_call(c):
        return lambda cst: dn(vp(sets[c][2]), vp(h), vp(y), N_FFN, K_FFN, cst)

    # one graph holds exactly K steps (weight copy i % copies at step i);
    # two more hold K launches of each kernel alone, for per-kernel times
    g_step = capture([f for i in range(steps) for f in (gu_call(i % copies), dn_call(i % copies))])
    g_gu = capture([gu_call(i % copies) for i in range(steps)])
    g_dn = capture([dn_call(i % copies) for i in range(steps)])

    def timed(g):
        ramp(torch, g.replay)      # leaves its last batch in flight
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps   # ms per step / per launch

    g_step.replay()   # first replays upload the graphs; not timed
    g_gu.replay()
    g_dn.replay()
    t0 = time.perf_counter()
    step_ms = timed(g_step)   # the timed region: exactly K steps
    wall = time.perf_counter() - t0
    gu_ms = timed(g_gu)
    dn_ms = timed(g_dn)
    return {
        "wall": wall, "steps_run": steps, "step_ms": step_ms, "copies": copies,
        "gate_up_ms": gu_ms, "down_ms": dn_ms, "x": x, "h": h, "y": y,
    }


def ramp(torch, fn, seconds=0.3):
    """Untimed clock ramp: about `seconds` of back-to-back fn calls (a graph
    replay or a launch loop) before a timed region, so the timed launches run
    at the clocks a busy GPU settles at.  All calls are enqueued without a
    wait (a wait between calls leaves the GPU idling, and after an idle spell
    it runs a K = 20 graph ~5 % slower), and they are still running when the
    timed region is enqueued behind them."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-5)
    for _ in range(min(4000, max(1, int(seconds / one)))):
        fn()


# one Q4_K GEMV 4096x4096 with the Q8_0 quantisation of x
# inline (gemv_q4_k_f32_q8_inline_launch), seed 0, as the reference's
# examples/bench_q4_k_gemv_isolated.rs times it.  Distinct weight copies
# (>= 4x the Infinity Cache) are cycled so every launch streams from HBM.
GEMV0_K = GEMV0_N = 4096
GEMV0_BYTES = GEMV0_N * (GEMV0_K // 256) * Q4K_BYTES + 4 * GEMV0_K + 4 * GEMV0_N   # 9,469,952


def bench_gemv_cfg0(lib, torch, launches):
    from rocmforge_amd import synth

    dev = torch.device("cuda:0")
    wbytes = GEMV0_N * (GEMV0_K // 256) * Q4K_BYTES
    copies = -(-4 * MALL_BYTES // wbytes)
    ws = [synth.torch_weights("q4_k", GEMV0_N, GEMV0_K, seed=c, device=dev) for c in range(copies)]
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn(GEMV0_K, device=dev, generator=g)
    y = torch.empty(GEMV0_N, device=dev)
    fn = lib.gemv_q4_k_f32_q8_inline_launch
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for i in range(launches):
                if fn(vp(ws[i % copies]), vp(x), vp(y), GEMV0_K, GEMV0_N, st):
                    raise RuntimeError("config 0 launch failed")
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    graph.replay()
    ramp(torch, graph.replay)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    gbs = GEMV0_BYTES / (us * 1e-6) / 1e9
    return {"workload": "BASELINE config 0: Q4_K GEMV 4096x4096 + Q8_0-inline x, batch 1, seed 0",
            "launcher": "gemv_q4_k_f32_q8_inline_launch", "bytes_per_launch": GEMV0_BYTES,
            "weight_copies_cycled": copies, "launches": launches, "us": round(us, 3), "gbs": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


# the full decode weight stream of a Llama-3.1-8B-shaped
# stack at batch 1 -- per layer the QKV projection (Q4_K, 4096 + 1024 + 1024
# rows x 4096, one fused Q8-inline launch over the three tensors), the O
# projection with the residual add fused (Q4_K 4096x4096), the fused
# gate+up+SwiGLU (2 x Q4_K 14336x4096) and ffn_down with the residual add
# fused (Q6_K 4096x14336); then the Q6_K lm_head (128256x4096).  Attention,
# norms and RoPE are not part of the path: the O projection reads the Q
# output in place of the attention output.
L_LAYERS, Q_N, KV_N, VOCAB = 32, 4096, 1024, 128256
QKV_N = Q_N + 2 * KV_N
STREAM_WEIGHT_BYTES = (L_LAYERS * (QKV_N * (K_FFN // 256) * Q4K_BYTES + K_FFN * (K_FFN // 256) * Q4K_BYTES
                                   + 2 * N_FFN * (K_FFN // 256) * Q4K_BYTES + K_FFN * (N_FFN // 256) * Q6K_BYTES)
                       + VOCAB * (K_FFN // 256) * Q6K_BYTES)   # 4,841,250,816


def bench_decode_stream(lib, torch, tokens):
    from rocmforge_amd import synth

    dev = torch.device("cuda:0")
    layers = []
    for l in range(L_LAYERS):
        # Q, K, V as the three separate GGUF tensors (4096 + 1024 + 1024 rows)
        layers.append(([synth.torch_weights("q4_k", n, K_FFN, seed=1000 + 5 * l + 7919 * i, device=dev)
                        for i, n in enumerate((Q_N, KV_N, KV_N))],
                       synth.torch_weights("q4_k", K_FFN, K_FFN, seed=1001 + 5 * l, device=dev),
                       synth.torch_weights("q4_k", N_FFN, K_FFN, seed=1002 + 5 * l, device=dev),
                       synth.torch_weights("q4_k", N_FFN, K_FFN, seed=1003 + 5 * l, device=dev),
                       synth.torch_weights("q6_k", K_FFN, N_FFN, seed=1004 + 5 * l, device=dev)))
    lm_head = synth.torch_weights("q6_k", VOCAB, K_FFN, seed=999, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    x = torch.randn(K_FFN, device=dev, generator=g)
    hidden = torch.randn(K_FFN, device=dev, generator=g)
    q, k, v = torch.empty(Q_N, device=dev), torch.empty(KV_N, device=dev), torch.empty(KV_N, device=dev)
    ffn = torch.empty(N_FFN, device=dev)
    logits = torch.empty(VOCAB, device=dev)

    def token(st):
        rc = 0
        for wqkv, wo, wg, wu, wd in layers:
            wq, wk, wv = wqkv
            rc |= lib.gemv_qkv_q4_k_f32_q8_inline_launch(vp(wq), vp(wk), vp(wv), None, None, None, vp(x), vp(q),
                                                         vp(k), vp(v), K_FFN, Q_N, KV_N, st)
            rc |= lib.gemv_q4_k_f32_q8_inline_residual_launch(vp(wo), vp(q), vp(hidden), vp(hidden), K_FFN, K_FFN,
                                                              st)
            rc |= lib.gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch(vp(wg), vp(wu), vp(hidden), vp(ffn), K_FFN, N_FFN,
                                                                    st)
            rc |= lib.gemv_q6_k_f32_residual_launch(vp(wd), vp(ffn), vp(hidden), vp(x), N_FFN, K_FFN, st)
        rc |= lib.gemv_q6_k_f32_launch(vp(lm_head), vp(x), vp(logits), K_FFN, VOCAB, st)
        if rc:
            raise RuntimeError(f"decode stream launch failed: hipError {rc}")

    st0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    token(st0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            token(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    graph.replay()
    ramp(torch, graph.replay)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(tokens):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / tokens
    gbs = STREAM_WEIGHT_BYTES / (ms * 1e-3) / 1e9
    return {"workload": "BASELINE config 2: 32 x (QKV 6144x4096 Q4_K as one fused launch over the 4096/1024/1024-row "
                        "Q, K, V tensors, O 4096x4096 Q4_K + residual, gate+up 2x14336x4096 Q4_K, "
                        "down 4096x14336 Q6_K + residual) + lm_head 128256x4096 Q6_K, batch 1",
            "launches_per_token": 4 * L_LAYERS + 1, "weight_bytes_per_token": STREAM_WEIGHT_BYTES,
            "tokens": tokens, "ms_per_token": round(ms, 4), "gbs": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def calibrate_copy(torch, mbytes=256, reps=10):
    """Plain device-to-device copies of a known size, run under rocprofv3
    --pmc to scale FETCH_SIZE / WRITE_SIZE (each copy reads and writes
    `mbytes` MiB)."""
    n = (mbytes << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_per_copy": n * 4, "reps": reps}))


def read_traffic():
    """HBM bytes per gate+up launch from the committed rocprofv3 --pmc summary
    (profiles/gemv_gate_up_llama8b_traffic.md, line 'traffic_bytes_per_launch:')."""
    f = ROOT / "profiles" / "gemv_gate_up_llama8b_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip().replace(",", ""))
    return None


def bench_gemm(lib, torch):
    """Prefill GEMM TFLOP/s at Llama-3.1-8B FFN shapes, M = 64..512: Q4_K
    14336x4096 (gate/up) and Q6_K 4096x14336 (down).  Distinct weight copies
    (>= 4x the Infinity Cache) are cycled so the weights stream from HBM; A
    (the activations, 0.25-8 MB) is the same for every launch, as the output
    of the previous layer would be."""
    from rocmforge_amd import synth

    dev = torch.device("cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    shapes = [("q4_k", N_FFN, K_FFN, Q4K_BYTES, lib.wmma_gemm_q4_k_launch),
              ("q6_k", K_FFN, N_FFN, Q6K_BYTES, lib.wmma_gemm_q6_k_launch)]
    for fmt, n, k, bb, fn in shapes:
        copies = -(-4 * MALL_BYTES // (n * (k // 256) * bb))
        wsets = [synth.torch_weights(fmt, n, k, seed=50 + c, device=dev) for c in range(copies)]
        for m in (64, 128, 256, 512):
            a = torch.randn(m, k, device=dev).to(torch.bfloat16).float()
            d = torch.empty(m, n, device=dev)

            def run(iters):
                for i in range(iters):
                    rc = fn(vp(a), vp(wsets[i % copies]), vp(d), m, n, k, st)
                    if rc:
                        raise RuntimeError(f"gemm launch failed {rc}")

            ramp(torch, lambda: run(copies))
            iters = 4 * copies
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            run(iters)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000 / iters
            tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
            res[f"{fmt}_{n}x{k}_M{m}"] = {"us": round(us, 2), "tflops": round(tflops, 1),
                                          "frac_fp16_peak": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                                          "weight_copies_cycled": copies}
            if True:
                # the same GEMM on activations the caller already rounded to fp16
                # (rf_gemm_q*_k_f16_launch): identical operands, no staging pass
                a16 = a.half()
                fn16 = lib.rf_gemm_q4_k_f16_launch if fmt == "q4_k" else lib.rf_gemm_q6_k_f16_launch

                def run16(iters):
                    for i in range(iters):
                        rc = fn16(vp(a16), vp(wsets[i % copies]), vp(d), m, n, k, st)
                        if rc:
                            raise RuntimeError(f"gemm launch failed {rc}")

                ramp(torch, lambda: run16(copies))
                e0.record()
                run16(iters)
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1000 / iters
                tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
                res[f"{fmt}_{n}x{k}_M{m}_fp16_activations"] = {
                    "us": round(us, 2), "tflops": round(tflops, 1),
                    "frac_fp16_peak": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                    "launcher": fn16.__name__, "weight_copies_cycled": copies}
    return res


def bench_mfma_peak(lib, torch):
    """Sustained v_mfma_f32_32x32x16_f16 rate on this MI355X: one 256-thread
    workgroup per CU, every wave issuing 8 independent MFMA chains, on fp16
    operands drawn N(0,1) (the prefill GEMMs' activation distribution) and
    on zeros (least switching activity), each timed over ~3 ms with HIP events
    after an untimed ramp.  Reported beside the 2.5 PFLOP/s dense fp16 figure
    the GEMM fractions are priced against."""
    dev = torch.device("cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    out = torch.empty(cus * 256, device=dev)
    res = {"instruction": "v_mfma_f32_32x32x16_f16", "workgroups": cus, "waves_per_simd": 1,
           "published_dense_fp16_tflops": FP16_MFMA_PEAK_TFLOPS}
    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    for name, a in (("normal", torch.randn(4096, generator=g).half()), ("zeros", torch.zeros(4096).half())):
        a = a.to(dev)
        iters = 20000

        def run():
            rc = lib.rf_mfma_peak_launch(vp(a), vp(out), cus, iters, st)
            if rc:
                raise RuntimeError(f"mfma peak launch failed {rc}")

        ramp(torch, run)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            run()
        e1.record()
        torch.cuda.synchronize()
        s = e0.elapsed_time(e1) / 1000 / 3
        flops = cus * 4 * iters * 8 * 32768
        res[f"{name}_operands_tflops"] = round(flops / s / 1e12, 1)
        res[f"{name}_frac_published"] = round(flops / s / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4)
    return res


def gemm_pmc(lib, torch):
    """Ten untimed launches of each M = 512 prefill GEMM (Q4_K 14336x4096 and
    Q6_K 4096x14336, each on fp32 and on fp16 activations), for counter collection
    under rocprofv3 --pmc."""
    from rocmforge_amd import synth
    dev = torch.device("cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for fmt, n, k, fn in (("q4_k", N_FFN, K_FFN, lib.wmma_gemm_q4_k_launch),
                          ("q6_k", K_FFN, N_FFN, lib.wmma_gemm_q6_k_launch)):
        wsets = [synth.torch_weights(fmt, n, k, seed=50 + c, device=dev) for c in range(6)]
        a = torch.randn(512, k, device=dev).to(torch.bfloat16).float()
        d = torch.empty(512, n, device=dev)
        for i in range(10):
            fn(vp(a), vp(wsets[i % 6]), vp(d), 512, n, k, st)
        a16 = a.half()
        fn16 = lib.rf_gemm_q4_k_f16_launch if fmt == "q4_k" else lib.rf_gemm_q6_k_f16_launch
        for i in range(10):
            fn16(vp(a16), vp(wsets[i % 6]), vp(d), 512, n, k, st)
        torch.cuda.synchronize()
    print(json.dumps({"gemm_pmc": "done"}), flush=True)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, min_runs, seconds):
    """Median wall time of fn over at least min_runs calls and about
    `seconds` (after one untimed call)."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(seconds):
    """The reference CPU algorithm (C port in oracle/) on the bench workloads,
    on this host's cores (all the CPUs this process may run on):
      * config 1 step: Q4_K x Q8_K AVX2 gate/up on all threads + silu_fuse,
        then the scalar Q6_K ffn_down on ONE thread (the reference's rayon
        split is over batch rows, so a single-token Q6_K GEMV runs on one
        thread) -- the headline figure;
      * the same step with the Q6_K GEMV on all threads (labelled variant);
      * config 0: the Q4_K GEMV 4096x4096;
      * config 3: the prefill GEMMs (gemm_q4_k_q8_k_avx2, gemm_q6_k_fallback,
        both parallel over the M rows) at M = 64..512, one call each.
    The GEMV figures are medians of repeated runs."""
    from oracle import oracle as O
    from rocmforge_amd import synth

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    wg = synth.q4_k_weights(N_FFN, K_FFN, seed=1)
    wu = synth.q4_k_weights(N_FFN, K_FFN, seed=2)
    wd = synth.q6_k_weights(K_FFN, N_FFN, seed=3)
    x = synth.activations(K_FFN, seed=0)
    h = np.ascontiguousarray(O.cpu_gate_up(wg, wu, x, N_FFN, K_FFN, threads))
    per = seconds / 4
    t_step, n_step = _median_time(lambda: (O.cpu_gate_up(wg, wu, x, N_FFN, K_FFN, threads),
                                           O.cpu_gemv_q6k(wd, h, K_FFN, N_FFN, 1)), 5, per)
    t_step_all, n_all = _median_time(lambda: (O.cpu_gate_up(wg, wu, x, N_FFN, K_FFN, threads),
                                              O.cpu_gemv_q6k(wd, h, K_FFN, N_FFN, threads)), 5, per / 2)
    w0 = synth.q4_k_weights(GEMV0_N, GEMV0_K, seed=0)
    t0_, n0_ = _median_time(lambda: O.cpu_gemv_q4k(w0, x, GEMV0_N, GEMV0_K, threads), 5, per / 4)
    gemm = {}
    for fmt, n, k, w in (("q4_k", N_FFN, K_FFN, wg), ("q6_k", K_FFN, N_FFN, wd)):
        for m in (64, 128, 256, 512):
            a = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
            t0 = time.perf_counter()
            O.cpu_gemm(fmt, w, a, m, n, k, threads)
            dt = time.perf_counter() - t0
            gemm[f"{fmt}_{n}x{k}_M{m}"] = {"ms": round(dt * 1e3, 1),
                                           "gflops": round(2.0 * m * n * k / dt / 1e9, 2)}
    return {
        "value": round(STEP_BYTES / t_step / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"config 1 step (gate+up {N_FFN}x{K_FFN} Q4_K x Q8_K AVX2 on {threads} threads + Q6_K down "
                  f"{K_FFN}x{N_FFN} scalar on 1 thread, as the reference runs one token): median of {n_step} "
                  f"steps = {t_step * 1e3:.1f} ms/step",
        "cpu_model": _cpu_model(), "nproc": os.cpu_count(), "threads_used": threads,
        "variant_q6k_all_threads": {"gbs": round(STEP_BYTES / t_step_all / 1e9, 3),
                                    "ms_per_step": round(t_step_all * 1e3, 2), "runs": n_all},
        "config0_gemv_4096": {"gbs": round(GEMV0_BYTES / t0_ / 1e9, 3), "us": round(t0_ * 1e6, 1), "runs": n0_},
        "prefill_gemm": gemm,
        "note": "C port of the reference CPU path (oracle/cpu_baseline.c); Q4_K via AVX2 maddubs/madd "
                "(the reference's dispatch uses AVX2 for Q4_K even on AVX-512 hosts); prefill GEMMs timed once "
                "per M (a single call takes 0.1-10 s)",
    }


def bench_e2e(torch, prompt_len=512, steps=128):
    """Qwen3-8B-shaped greedy generation (36 layers, hidden
    4096, FFN 12288, 32 q / 8 kv heads of 128, per-head Q/K RMSNorm, vocab
    151936, Q4_K_M type mix, seeded random weights): a 512-token prompt,
    then 128 decode steps replayed from one captured HIP graph."""
    from rocmforge_amd import engine as E
    cfg = E.ModelConfig.qwen3_8b()
    w = E.synthetic_weights(cfg, seed=0, signed=True)
    eng = E.Engine(cfg, w, max_seq=prompt_len + steps + 64)
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, cfg.vocab, prompt_len)]
    eng.prefill(prompt)                                   # warm
    eng.capture_decode()
    times = []
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill(prompt)
        times.append(time.perf_counter() - t0)
    t_pf = min(times)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    eng._graph.replay()                                   # one warm replay, then back to the prompt's end
    eng.prefill(prompt)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        eng._graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms_tok = start.elapsed_time(end) / steps
    stream_bytes = sum(t[0].numel() for lw in w.layers for t in lw.mats.values()) + w.lm_head[0].numel()
    return {
        "workload": "BASELINE config 4: Qwen3-8B-shaped greedy decode, Q4_K_M mix, seeded random weights",
        "prefill_tokens": prompt_len, "prefill_ms": round(t_pf * 1e3, 3),
        "prefill_tok_s": round(prompt_len / t_pf, 1),
        "decode_steps": steps, "decode_ms_per_token": round(ms_tok, 4),
        "decode_tok_s": round(1e3 / ms_tok, 1),
        "decode_weight_bytes_per_token": int(stream_bytes),
        "decode_weight_GBps": round(stream_bytes / (ms_tok * 1e-3) / 1e9, 1),
        "note": "prefill wall time includes host launch of every kernel (no graph); decode timed with HIP "
                "events over graph replays",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(sharding over several GPUs is not implemented)"}))
        sys.exit(2)
    import torch

    import rocmforge_amd
    lib = rocmforge_amd.load()
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (cuda:0)")
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    if args.gemm_pmc:
        gemm_pmc(lib, torch)
        return

    r = bench_decode(lib, torch, args.steps, args.warmup)
    ms = r["step_ms"]
    value = STEP_BYTES / (ms * 1e-3) / 1e9
    gu_gbs = GATE_UP_BYTES / (r["gate_up_ms"] * 1e-3) / 1e9
    dn_gbs = DOWN_BYTES / (r["down_ms"] * 1e-3) / 1e9
    out = {
        "metric": "decode GEMV HBM GB/s (% of peak) + prefill GEMM TFLOP/s at Llama-3.1-8B shapes",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps_run"],
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights; int8 dot + fp32",
        "data": "synthetic (seeded GGUF Q4_K/Q6_K blocks, x ~ N(0,1))",
        "config": {"workload": "BASELINE config 1: Llama-3.1-8B FFN decode, batch 1: fused Q4_K gate+up+SwiGLU "
                               "2x14336x4096 then Q6_K ffn_down 4096x14336",
                   "bytes_per_step": STEP_BYTES, "weight_copies_cycled": r["copies"],
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "kernel": "rf_q4k_q8_gemv_kernel<gate_up>",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "avg_launch_us": round(r["gate_up_ms"] * 1e3, 3), "bytes_per_launch": GATE_UP_BYTES},
        "kernels": {"gate_up_us": round(r["gate_up_ms"] * 1e3, 3), "gate_up_gbs": round(gu_gbs, 1),
                    "q6k_down_us": round(r["down_ms"] * 1e3, 3), "q6k_down_gbs": round(dn_gbs, 1)},
    }
    out["gemv_4096"] = bench_gemv_cfg0(lib, torch, max(args.steps, 100))
    if not args.no_gemm:
        out["prefill_gemm"] = bench_gemm(lib, torch)
        out["mfma_peak"] = bench_mfma_peak(lib, torch)
    if not args.no_stream:
        out["decode_stream"] = bench_decode_stream(lib, torch, args.stream_tokens)
    if not args.no_e2e:
        out["e2e_qwen3_8b"] = bench_e2e(torch)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
