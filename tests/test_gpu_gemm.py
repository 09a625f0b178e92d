"""GPU parity of the prefill GEMMs (wmma_gemm_q4_k_launch / wmma_gemm_q6_k_launch)
through the C ABI, against the oracle's float64 product of the fp16-rounded
operands (the reference stages both operands through __float2half).

Tolerance (BASELINE: 2e-3 relative): per element
  |D - D_ref| <= 2e-3 * |D_ref| + 2e-5 * S,   S = (|fp16 A| @ |fp16 W|^T)[r, c],
S being the sum of the magnitudes of the products an output adds up: the
second term is the fp32 accumulation allowance (a K-term fp32 sum can be off
by up to K * 2^-24 * S; the MFMA sums measure below 1e-5 * S), so outputs that
cancel to near zero are judged against the size of what cancelled.  The
operands themselves are pinned bit for bit by the identity tests below.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from rocmforge_amd import synth
from tests import gpu_util as G
from tests.test_oracle import _byte_level_q4k_block, _byte_level_q6k_block

pytestmark = pytest.mark.gpu


def _run(rf, fmt, a, w, m, n, k):
    da, dw = G.to_dev(a), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    fn = rf.wmma_gemm_q4_k_launch if fmt == "q4_k" else rf.wmma_gemm_q6_k_launch
    G.call(fn, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    return G.host(d).reshape(m, n)


def _check(got, fmt, a, w, m, n, k, what):
    ref = O.gemm(fmt, a, w, m, n, k)
    S = O.gemm_abs(fmt, a, w, m, n, k)
    err = np.abs(got.astype(np.float64) - ref)
    tol = 2e-3 * np.abs(ref) + 2e-5 * S
    assert (err[tol == 0] == 0).all(), what          # outputs of all-zero rows are exactly zero
    pos = tol > 0
    worst = (err[pos] / tol[pos]).max()
    print(f"{what}: max_abs={err.max():.3e} max|ref|={np.abs(ref).max():.3e} max err/S={(err[pos] / S[pos]).max():.2e} "
          f"worst={worst:.3f}", flush=True)
    assert worst <= 1.0, what


@pytest.mark.parametrize("fmt,n,k", [("q4_k", 64, 256), ("q6_k", 64, 256),      # general kernel
                                     ("q4_k", 256, 512), ("q6_k", 256, 2048)])  # weight-ring kernel
def test_gemm_byte_level_identity(rf, dev, fmt, n, k):
    # the reference's byte-level test (wmma_q4_k_correctness.rs:89-185,
    # wmma_q6_k_correctness.rs:75-160): A = I (64 x k), every W row the same
    # hand-built block, so D[r, c] = dequant[r] bit for bit.
    m = 64
    blk = _byte_level_q4k_block() if fmt == "q4_k" else _byte_level_q6k_block()
    w = np.tile(blk, (n, k // 256))
    a = np.zeros((m, k), np.float32)
    a[np.arange(m), np.arange(m)] = 1.0
    got = _run(rf, fmt, a, w, m, n, k)
    deq = O.dequant_f16(fmt, w, n, k)[0]
    for c in range(n):
        np.testing.assert_array_equal(got[:, c], deq[:m])


@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 64, 64, 256), ("q4_k", 128, 192, 512), ("q4_k", 192, 128, 768), ("q4_k", 256, 256, 1024),
    ("q6_k", 64, 64, 256), ("q6_k", 128, 320, 768), ("q6_k", 256, 128, 1024),
])
def test_gemm_small_shapes(rf, dev, fmt, m, n, k):
    a = synth.activations(k, seed=m + n, m=m)
    w = synth.weights(fmt, n, k, seed=k)
    _check(_run(rf, fmt, a, w, m, n, k), fmt, a, w, m, n, k, f"{fmt} {m}x{n}x{k}")


# One case per launcher branch for N % 256 == 0, K % 512 == 0 (the tiled
# kernels): 256 x 256 or 128 x 128 shared-dequantisation tiles (where they
# come to about one workgroup per CU); otherwise ring tiles of 128 rows (Q6_K, or
# Q4_K when they fill the CUs unsplit -- the M = 512 Llama case -- or fit one
# round of CUs where 64-row tiles would need two) or
# 64 rows, with split-K when the tiles leave CUs idle; and (Q6_K with
# K % 2048 != 0) the register-weight kernel.
@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 64, 256, 512),      # ring, 64-row tiles, 1 split
    ("q4_k", 192, 256, 1024),    # ring, 64-row tiles, 2 splits
    ("q4_k", 128, 512, 2048),    # ring, 64-row tiles, 4 splits
    ("q4_k", 384, 512, 512),     # ring, 64-row tiles, 1 split
    ("q4_k", 2048, 8192, 512),   # 256 x 256 shared-dequantisation tiles (256 tiles)
    ("q4_k", 256, 14336, 512),   # 128 x 128 shared-dequantisation tiles (224 tiles)
    ("q4_k", 512, 12288, 512),   # ring, 128-row tiles: one round of CUs where 64-row tiles take two
    ("q6_k", 64, 256, 2048),     # ring, 64-row tiles, 4 splits
    ("q6_k", 256, 512, 4096),    # ring, 128-row tiles, 8 splits
    ("q6_k", 128, 256, 1536),    # register weights, 128-row tiles, 3 splits
    ("q6_k", 64, 256, 512),      # register weights, 64-row tiles, 1 split
    ("q6_k", 2048, 7168, 512),   # 256 x 256 tiles, rows 2-byte aligned (420 bytes)
    ("q6_k", 256, 14336, 1536),  # 128 x 128 tiles (two threads per weight row), 1260-byte rows
])
def test_gemm_tiled_kernel_branches(rf, dev, fmt, m, n, k):
    a = synth.activations(k, seed=m + 3 * n, m=m)
    w = synth.weights(fmt, n, k, seed=k + 1)
    _check(_run(rf, fmt, a, w, m, n, k), fmt, a, w, m, n, k, f"{fmt} {m}x{n}x{k}")


@pytest.mark.parametrize("fmt,n,k", [("q4_k", 14336, 4096), ("q6_k", 4096, 14336), ("q4_k", 4096, 12288)])
@pytest.mark.parametrize("m", [64, 128, 256, 512])
def test_gemm_llama_ffn_shapes(rf, dev, fmt, n, k, m):
    # BASELINE config 3 at full size, and the Qwen3-8B Q4_K down projection
    # (4096 x 12288: at M = 512 the 256 x 128 tiles split over K in four);
    # A is bf16-valued N(0,1)
    a = torch.from_numpy(synth.activations(k, seed=7, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.weights(fmt, n, k, seed=8)
    _check(_run(rf, fmt, a, w, m, n, k), fmt, a, w, m, n, k, f"{fmt} M={m} {n}x{k}")


@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 512, 14336, 512),   # ring tiles, 128 rows
    ("q4_k", 256, 28672, 768),   # ring tiles, 128 rows, three super-blocks
    ("q4_k", 128, 512, 2048),    # ring tiles with split-K
    ("q6_k", 512, 4096, 2048),   # ring tiles, 128 rows
])
def test_gemm_identity_random_weights(rf, dev, fmt, m, n, k):
    # A = [I | 0] (m x k): every output is one product 1 * w, so D[r, c] is the
    # fp16 dequantised weight W[c, r] bit for bit -- the B operand of every
    # kernel lane, its k order and its rounding checked exhaustively
    a = np.zeros((m, k), np.float32)
    a[np.arange(m), np.arange(m)] = 1.0
    w = synth.weights(fmt, n, k, seed=m + k)
    got = _run(rf, fmt, a, w, m, n, k)
    deq = O.dequant_f16(fmt, w, n, k)
    np.testing.assert_array_equal(got, deq[:, :m].T.astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(512, 14336, 4096), (256, 14336, 4096), (64, 14336, 4096), (128, 4096, 4096),
                                   (576, 6144, 4096), (320, 256, 1024), (128, 14336, 4096), (512, 4096, 4096),
                                   (512, 4096, 12288), (256, 4096, 12288), (192, 192, 512), (64, 64, 256)])
def test_gemm_q4k_fp16_activations(rf, dev, m, n, k):
    # 256 x 128 tiles at 512 x 14336 (and split over K at 512 x 4096 x 12288);
    # elsewhere the K-sliced 64 / 128 / 256-row tiles, including partial row
    # tiles and N = 64, 192
    # rf_gemm_q4_k_f16_launch on A rounded to fp16 by the caller: the operands
    # of wmma_gemm_q4_k_launch on fp32 A, so the same oracle and bar
    a = torch.from_numpy(synth.activations(k, seed=m + 11, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.q4_k_weights(n, k, seed=k + 5)
    a16 = a.astype(np.float16)
    da, dw = G.to_dev(a16.view(np.int16)), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    _check(G.host(d).reshape(m, n), "q4_k", a, w, m, n, k, f"fp16-A q4_k M={m} {n}x{k}")


@pytest.mark.parametrize("m,n,k", [(512, 4096, 14336), (256, 4096, 14336), (64, 4096, 14336), (192, 1024, 2048),
                                   (576, 128, 4096), (128, 64, 2048)])
def test_gemm_q6k_fp16_activations(rf, dev, m, n, k):
    # rf_gemm_q6_k_f16_launch: the operands of wmma_gemm_q6_k_launch on fp32 A
    # rounded to fp16 by the caller; M = 192 and 576 leave a partial 128-row tile
    a = torch.from_numpy(synth.activations(k, seed=m + 13, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.weights("q6_k", n, k, seed=k + 9)
    da, dw = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q6_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    _check(G.host(d).reshape(m, n), "q6_k", a, w, m, n, k, f"fp16-A q6_k M={m} {n}x{k}")


@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (256, 4096, 12288), (64, 128, 512), (192, 64, 1024)])
def test_gemm_q4k_fp16_accumulate(rf, dev, m, n, k):
    # inout += product: bit for bit the plain launch's sums plus the old
    # contents (the K-sliced tiles serve both; rows past M stay put)
    a = torch.from_numpy(synth.activations(k, seed=m + 23, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.q4_k_weights(n, k, seed=k + 7)
    da, dw = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(w)
    r = synth.activations(n, seed=9, m=m + 64)
    dr = G.to_dev(r)
    G.call(rf.rf_gemm_q4_k_f16_accumulate_launch, G.ptr(da), G.ptr(dw), G.ptr(dr), m, n, k)
    got = G.host(dr).reshape(m + 64, n)
    np.testing.assert_array_equal(got[m:], r[m:])
    ref = O.gemm("q4_k", a, w, m, n, k)
    err = np.abs(got[:m].astype(np.float64) - r[:m] - ref)
    tol = 2e-3 * np.abs(ref) + 1e-5 * np.abs(ref).max() + 1e-6 * np.abs(r[:m])
    assert (err <= tol).all(), f"q4_k f16 accumulate {m}x{n}x{k}: worst {(err / tol).max():.3f}"
    if m * n <= 64 * 4096:
        # where the plain launch takes the same K-sliced tiles, bit for bit
        d = G.empty(m * n, torch.float32)
        G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
        np.testing.assert_array_equal(got[:m], r[:m] + G.host(d).reshape(m, n))


def test_gemm_q6k_fp16_rejections(rf, dev):
    d = G.empty(64 * 64, torch.float32)
    a = G.to_dev(np.zeros((64, 4096), np.int16))
    w = G.to_dev(synth.weights("q6_k", 64, 4096, seed=1))
    f = rf.rf_gemm_q6_k_f16_launch
    s = G.stream()
    assert f(G.ptr(a), G.ptr(w), G.ptr(d), 64, 64, 1024, s) != 0       # K % 2048
    assert f(G.ptr(a), G.ptr(w), G.ptr(d), 64, 32, 4096, s) != 0       # N % 64
    assert f(G.ptr(a), G.ptr(w), G.ptr(d), 96, 64, 4096, s) != 0       # M % 64
    assert f(ctypes.c_void_p(a.data_ptr() + 2), G.ptr(w), G.ptr(d), 64, 64, 4096, s) != 0   # A alignment
    assert f(G.ptr(a), ctypes.c_void_p(w.data_ptr() + 4), G.ptr(d), 64, 64, 4096, s) != 0   # weight alignment
    assert f(None, G.ptr(w), G.ptr(d), 64, 64, 4096, s) != 0


def test_gemm_q4k_fp16_activations_identity(rf, dev):
    # A = [I | 0] in fp16: D[r, c] = dequantised W[c, r] bit for bit (the
    # natural-order B operands of the fp16 path)
    m, n, k = 512, 14336, 512
    a = np.zeros((m, k), np.float16)
    a[np.arange(m), np.arange(m)] = 1.0
    w = synth.q4_k_weights(n, k, seed=77)
    da, dw = G.to_dev(a.view(np.int16)), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    np.testing.assert_array_equal(G.host(d).reshape(m, n), O.dequant_f16("q4_k", w, n, k)[:, :m].T)


@pytest.mark.parametrize("fmt,n,k,m,a16", [
    ("q4_k", 14336, 4096, 512, False),   # ring tiles, 128 rows
    ("q4_k", 14336, 4096, 512, True),    # fp16 activations: 256 x 128 tiles, K halves on wave pairs
    ("q4_k", 14336, 4096, 128, False),   # ring tiles of 64 rows, split-K
    ("q6_k", 4096, 14336, 512, False),   # ring tiles of 128 rows
    ("q6_k", 4096, 14336, 512, True),    # fp16 activations: 128 x 64 tiles, K slices on waves
])
def test_gemm_every_weight_at_full_size(rf, dev, fmt, n, k, m, a16):
    # A = I over successive m-column windows of K: D = W^T window by window,
    # so every one of the n*k dequantised weights the kernel uses is compared
    # bit for bit with the oracle's fp16(fp32 value) -- the reference's double
    # rounding, which differs from one rounding of the exact value for a few
    # Q4_K weights per matrix (7 of 58.7M with these seeds)
    w = synth.weights(fmt, n, k, seed=4101)
    want = O.dequant_f16(fmt, w, n, k)
    dw = G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    for b in range(k // m):
        a = np.zeros((m, k), np.float16 if a16 else np.float32)
        a[np.arange(m), b * m + np.arange(m)] = 1.0
        if a16:
            fn = rf.rf_gemm_q4_k_f16_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_f16_launch
            G.call(fn, G.ptr(G.to_dev(a.view(np.int16))), G.ptr(dw), G.ptr(d), m, n, k)
        else:
            fn = rf.wmma_gemm_q4_k_launch if fmt == "q4_k" else rf.wmma_gemm_q6_k_launch
            G.call(fn, G.ptr(G.to_dev(a)), G.ptr(dw), G.ptr(d), m, n, k)
        got = G.host(d).reshape(m, n).T
        bad = np.argwhere(got != want[:, b * m:(b + 1) * m])
        assert bad.size == 0, f"window {b}: {len(bad)} weights differ, first {bad[:4].tolist()}"


def test_gemm_zero_padded_rows(rf, dev):
    # prefill buffers are padded to 64 rows with zeros (cache.rs:781-834)
    m, n, k = 128, 128, 512
    a = synth.activations(k, seed=3, m=m)
    a[77:] = 0.0
    w = synth.q4_k_weights(n, k, seed=4)
    got = _run(rf, "q4_k", a, w, m, n, k)
    assert np.all(got[77:] == 0.0)
    _check(got, "q4_k", a, w, m, n, k, "padded")


def test_gemm_staging_slots_across_streams(rf, dev):
    # The fp32-activation entry points stage A in a per-stream slot of the
    # library (4 per GPU).  Six streams launching at once: every result
    # within the GEMM bar of the oracle (streams without a slot take the fp32
    # kernels); once they have finished, their slots pass to new streams, and
    # every stream then gives the bits of the staged path.
    m, n, k = 64, 512, 1024
    cases = []
    for i in range(6):
        a = synth.activations(k, seed=100 + i, m=m)
        w = synth.weights("q4_k", n, k, seed=200 + i)
        cases.append((a, w, G.to_dev(a), G.to_dev(w)))
    ref_bits = []
    for a, w, da, dw in cases:                      # the current stream: staged path
        d = G.empty(m * n, torch.float32)
        G.call(rf.wmma_gemm_q4_k_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
        ref_bits.append(G.host(d))
    for rnd in range(2):
        streams = [torch.cuda.Stream() for _ in range(6)]
        outs = [G.empty(m * n, torch.float32) for _ in range(6)]
        torch.cuda.synchronize()
        for (a, w, da, dw), s, d in zip(cases, streams, outs):
            rc = rf.wmma_gemm_q4_k_launch(G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k, ctypes.c_void_p(s.cuda_stream))
            assert rc == 0
        torch.cuda.synchronize()
        for i, ((a, w, da, dw), d) in enumerate(zip(cases, outs)):
            _check(G.host(d).reshape(m, n), "q4_k", a, w, m, n, k, f"stream {i} round {rnd}")
        # one stream at a time, each after the last finished: every one gets a slot
        for (a, w, da, dw), s, d, rb in zip(cases, streams, outs, ref_bits):
            rc = rf.wmma_gemm_q4_k_launch(G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k, ctypes.c_void_p(s.cuda_stream))
            assert rc == 0
            torch.cuda.synchronize()
            np.testing.assert_array_equal(G.host(d), rb)
        del streams


@pytest.mark.parametrize("warm", [True, False])
def test_gemm_reference_entry_points_capture(rf, dev, warm):
    # wmma_gemm_q4_k_launch / wmma_gemm_q6_k_launch captured into a HIP graph
    # (staging pass, K-split GEMM and reduction).  A stream that has launched
    # a GEMM before holds a staging slot, so its capture runs the staged path:
    # every replay, with eager GEMM work in between, gives the eager result bit
    # for bit.  A stream whose first GEMM is captured can only take a free
    # slot (slots are not handed over during capture), else the fp32 kernels:
    # every replay the same bits, within the GEMM bar of the oracle
    shapes = [("q4_k", 64, 512, 1024), ("q6_k", 64, 256, 2048), ("q6_k", 256, 512, 4096)]
    bufs = []
    for fmt, m, n, k in shapes:
        a = synth.activations(k, seed=m + n, m=m)
        w = synth.weights(fmt, n, k, seed=k + 5)
        da, dw = G.to_dev(a), G.to_dev(w)
        eager, out = G.empty(m * n, torch.float32), G.empty(m * n, torch.float32)
        fn = rf.wmma_gemm_q4_k_launch if fmt == "q4_k" else rf.wmma_gemm_q6_k_launch
        G.call(fn, G.ptr(da), G.ptr(dw), G.ptr(eager), m, n, k)
        bufs.append((fmt, m, n, k, a, w, da, dw, eager, out, fn))
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    if warm:
        for fmt, m, n, k, a, w, da, dw, eager, out, fn in bufs:
            assert fn(G.ptr(da), G.ptr(dw), G.ptr(out), m, n, k, ctypes.c_void_p(cs.cuda_stream)) == 0
        torch.cuda.synchronize()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(g, stream=cs):
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for fmt, m, n, k, a, w, da, dw, eager, out, fn in bufs:
                assert fn(G.ptr(da), G.ptr(dw), G.ptr(out), m, n, k, st) == 0
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    first = None
    for rep in range(3):
        for *_, out, fn in bufs:
            out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [G.host(b[9]) for b in bufs]
        first = first or got
        for (fmt, m, n, k, a, w, da, dw, eager, out, fn), o, f in zip(bufs, got, first):
            np.testing.assert_array_equal(o, f)                 # every replay the same bits
            if warm:
                np.testing.assert_array_equal(o, G.host(eager))
            # eager work on the current stream between replays
            G.call(fn, G.ptr(da), G.ptr(dw), G.ptr(eager), m, n, k)
    for (fmt, m, n, k, a, w, *_), o in zip(bufs, first):
        _check(o.reshape(m, n), fmt, a, w, m, n, k, f"captured {fmt} {m}x{n}x{k}")
