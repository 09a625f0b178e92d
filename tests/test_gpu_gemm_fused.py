"""GPU parity of the prefill GEMM launchers that have no reference
counterpart: several weight matrices as column segments of one launch
(rf_gemm_q*_k_segments_launch, rf_gemm_qk_f16_segments_launch), D += product
(rf_gemm_q*_k_accumulate_launch) and gate/up with SwiGLU in the epilogue
(rf_gemm_q*_k_swiglu_launch).

Each segment / accumulated product is checked against the oracle's float64
product of the fp16-rounded operands at the GEMM bar
  |D - D_ref| <= 2e-3 * |D_ref| + 1e-5 * max|D_ref|   (plus 1e-6 * |R| for D = R + product),
and bit for bit against the launch that runs the same tiles: a segment
against its matrix alone on fp16 activations rounded on the host (the fp32
launchers stage A as fp16 first), an accumulated product against R plus the
single-GEMM launcher (the same tiles and K split; one fp32 add of R).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from rocmforge_amd import synth
from tests import gpu_util as G

pytestmark = pytest.mark.gpu


def _check(got, ref, what, base=None):
    scale = np.abs(ref).max()
    err = np.abs(got.astype(np.float64) - ref - (0.0 if base is None else base.astype(np.float64)))
    tol = 2e-3 * np.abs(ref) + 1e-5 * scale + (0.0 if base is None else 1e-6 * np.abs(base))
    worst = (err / tol).max()
    print(f"{what}: max_abs={err.max():.3e} max|ref|={scale:.3e} worst={worst:.3f}", flush=True)
    assert worst <= 1.0, what


def _single(rf, fmt, a_dev, w, m, n, k):
    dw = G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    fn = rf.wmma_gemm_q4_k_launch if fmt == "q4_k" else rf.wmma_gemm_q6_k_launch
    G.call(fn, G.ptr(a_dev), G.ptr(dw), G.ptr(d), m, n, k)
    return G.host(d).reshape(m, n)


def _segments(rf, fmt, a_dev, ws, m, ns, k):
    dws = [G.to_dev(w) for w in ws]
    ds = [G.empty(m * n, torch.float32).fill_(float("nan")) for n in ns]
    wp = [G.ptr(t) for t in dws] + [ctypes.c_void_p(0)] * (3 - len(ws))
    dp = [G.ptr(t) for t in ds] + [ctypes.c_void_p(0)] * (3 - len(ns))
    nn = list(ns) + [0] * (3 - len(ns))
    fn = rf.rf_gemm_q4_k_segments_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_segments_launch
    G.call(fn, G.ptr(a_dev), *wp, *dp, m, *nn, k)
    return [G.host(d).reshape(m, n) for d, n in zip(ds, ns)]


def _f16_alone(rf, fmt, a16_dev, w, m, n, k):
    # one matrix through the fp16-activation segments launcher
    dw = G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    z = ctypes.c_void_p(0)
    t = 12 if fmt == "q4_k" else 14
    G.call(rf.rf_gemm_qk_f16_segments_launch, G.ptr(a16_dev), G.ptr(dw), z, z, t, 12, 12, G.ptr(d), z, z, m, n, 0, 0,
           k)
    return G.host(d).reshape(m, n)


@pytest.mark.parametrize("fmt,m,ns,k", [
    ("q4_k", 512, (1024, 256, 256), 512),     # Q/K/V shape, narrowed
    ("q4_k", 64, (512, 256, 256), 1024),      # one 64-row M tile
    ("q4_k", 128, (768, 256), 512),           # two segments (V in another type)
    ("q6_k", 128, (512, 256), 2048),
    ("q6_k", 256, (256, 256, 512), 2048),
])
def test_segments_match_oracle_and_single(rf, dev, fmt, m, ns, k):
    a = synth.activations(k, seed=m + k, m=m)
    ws = [synth.weights(fmt, n, k, seed=10 + i) for i, n in enumerate(ns)]
    da = G.to_dev(a)
    a16 = G.to_dev(a.astype(np.float16).view(np.int16))
    got = _segments(rf, fmt, da, ws, m, ns, k)
    again = _segments(rf, fmt, da, ws, m, ns, k)
    for i, (g, g2, w, n) in enumerate(zip(got, again, ws, ns)):
        _check(g, O.gemm(fmt, a, w, m, n, k), f"{fmt} segment {i} {m}x{n}x{k}")
        np.testing.assert_array_equal(g, g2)                               # the same bits on every run
        np.testing.assert_array_equal(g, _f16_alone(rf, fmt, a16, w, m, n, k))


@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 64, 256, 512),       # 64-row K-sliced tiles, K split over 2 workgroups
    ("q4_k", 256, 14336, 512),    # 128-row tiles, no K split
    ("q4_k", 128, 512, 2048),     # K split over 8 workgroups, added onto the caller's values
    ("q6_k", 256, 512, 4096),
    ("q6_k", 512, 1024, 2048),
    ("q4_k", 512, 4096, 12288),   # 256-row tiles, K split in two, the sum added in the reduction
])
def test_accumulate_adds_to_contents(rf, dev, fmt, m, n, k):
    a = synth.activations(k, seed=3 * m + n, m=m)
    w = synth.weights(fmt, n, k, seed=k + 2)
    r = np.random.default_rng(m + n).standard_normal((m, n)).astype(np.float32) * 4.0
    da, dw, dr = G.to_dev(a), G.to_dev(w), G.to_dev(r.ravel())
    fn = rf.rf_gemm_q4_k_accumulate_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_accumulate_launch
    G.call(fn, G.ptr(da), G.ptr(dw), G.ptr(dr), m, n, k)
    got = G.host(dr).reshape(m, n)
    _check(got, O.gemm(fmt, a, w, m, n, k), f"{fmt} accumulate {m}x{n}x{k}", base=r)
    np.testing.assert_array_equal(got, r + _single(rf, fmt, da, w, m, n, k))


@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 128, 384, 512),       # 3 tile pairs, 128-row tiles
    ("q4_k", 64, 256, 1024),       # 64-row tiles (no K split even where one would pay)
    ("q4_k", 512, 1536, 2048),
    ("q6_k", 128, 256, 2048),
    ("q6_k", 64, 256, 2048),       # Q6_K, 64-row tiles
    ("q4_k", 512, 12288, 4096),    # Qwen3-8B gate/up at full size
    ("q6_k", 256, 12288, 4096),    # the same shape in Q6_K
])
def test_swiglu_pairs(rf, dev, fmt, m, n, k):
    # out = silu(A Wg^T) * (A Wu^T): the products within the GEMM bar of the
    # oracle, and within fp32 rounding of silu(g) * u over the two single
    # GEMMs (which may sum in another order where they take a K split)
    a = synth.activations(k, seed=m + n + 1, m=m)
    wg = synth.weights(fmt, n, k, seed=21)
    wu = synth.weights(fmt, n, k, seed=22)
    da, dg, du = G.to_dev(a), G.to_dev(wg), G.to_dev(wu)
    d = G.empty(m * n, torch.float32).fill_(float("nan"))
    fn = rf.rf_gemm_q4_k_swiglu_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_swiglu_launch
    G.call(fn, G.ptr(da), G.ptr(dg), G.ptr(du), G.ptr(d), m, n, k)
    got = G.host(d).reshape(m, n).astype(np.float64)
    g = O.gemm(fmt, a, wg, m, n, k)
    u = O.gemm(fmt, a, wu, m, n, k)
    ref = g / (1.0 + np.exp(-g)) * u
    # the bar on each product carries through silu(g) * u: d(silu)/dg <= 1.1
    eg = 2e-3 * np.abs(g) + 1e-5 * np.abs(g).max()
    eu = 2e-3 * np.abs(u) + 1e-5 * np.abs(u).max()
    tol = 1.1 * eg * np.abs(u) + np.abs(g / (1.0 + np.exp(-g))) * eu + 1e-6 * np.abs(ref).max()
    worst = (np.abs(got - ref) / tol).max()
    print(f"{fmt} swiglu {m}x{n}x{k}: worst={worst:.3f}", flush=True)
    assert worst <= 1.0
    gs = _single(rf, fmt, da, wg, m, n, k)
    us = _single(rf, fmt, da, wu, m, n, k)
    with np.errstate(over="ignore"):          # exp(-g) = inf for g << 0 gives silu = -0
        sil = (gs / (np.float32(1.0) + np.exp(-gs)) * us).astype(np.float32)
    assert np.allclose(got, sil, rtol=1e-5, atol=1e-6 * np.abs(sil).max())


@pytest.mark.parametrize("fmt,m,n,k", [("q4_k", 512, 12288, 4096), ("q4_k", 64, 256, 1024), ("q6_k", 128, 256, 2048)])
def test_swiglu_pairs_f16_out(rf, dev, fmt, m, n, k):
    # rf_gemm_q*_k_swiglu_f16_launch: the fp32 launcher's values rounded to
    # fp16 (nearest even), bit for bit
    a = synth.activations(k, seed=m + n + 3, m=m)
    wg = synth.weights(fmt, n, k, seed=31)
    wu = synth.weights(fmt, n, k, seed=32)
    da, dg, du = G.to_dev(a), G.to_dev(wg), G.to_dev(wu)
    d32 = G.empty(m * n, torch.float32)
    d16 = G.empty(m * n, torch.int16)
    f32 = rf.rf_gemm_q4_k_swiglu_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_swiglu_launch
    f16 = rf.rf_gemm_q4_k_swiglu_f16_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_swiglu_f16_launch
    G.call(f32, G.ptr(da), G.ptr(dg), G.ptr(du), G.ptr(d32), m, n, k)
    G.call(f16, G.ptr(da), G.ptr(dg), G.ptr(du), G.ptr(d16), m, n, k)
    want = G.host(d32).astype(np.float16)
    got = G.host(d16).view(np.float16)
    np.testing.assert_array_equal(got.view(np.int16), want.view(np.int16))


@pytest.mark.parametrize("m,n,k", [(512, 4096, 12288), (192, 128, 2048), (64, 256, 4096)])
def test_q6k_f16_accumulate(rf, dev, m, n, k):
    # inout += product: bit for bit the plain fp16-activation launch plus the
    # old contents (one fp32 add per output), and within the GEMM bar of the
    # oracle; M = 192 leaves a partial 128-row tile whose rows past M stay put;
    # M = 512 (256-row tiles) and M = 64 (64-row tiles, two per CU) split K,
    # the product then added in the reduction
    a = torch.from_numpy(synth.activations(k, seed=m + 17, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.weights("q6_k", n, k, seed=k + 3)
    da, dw = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(w)
    r = synth.activations(n, seed=5, m=m + 64)
    dr = G.to_dev(r)
    G.call(rf.rf_gemm_q6_k_f16_accumulate_launch, G.ptr(da), G.ptr(dw), G.ptr(dr), m, n, k)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q6_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    got = G.host(dr).reshape(m + 64, n)
    np.testing.assert_array_equal(got[:m], r[:m] + G.host(d).reshape(m, n))
    np.testing.assert_array_equal(got[m:], r[m:])
    _check(got[:m], O.gemm("q6_k", a, w, m, n, k), f"q6_k f16 accumulate {m}x{n}x{k}", base=r[:m])


def test_rejections(rf, dev):
    m, k = 64, 512
    da = G.to_dev(synth.activations(k, seed=1, m=m))
    w = G.to_dev(synth.weights("q4_k", 512, k, seed=1))
    d = G.empty(m * 512, torch.float32)
    s = G.stream()
    z = ctypes.c_void_p(0)
    P = G.ptr
    seg = rf.rf_gemm_q4_k_segments_launch
    assert seg(P(da), P(w), z, z, P(d), z, z, m, 512, 0, 0, k, s) == 0
    torch.cuda.synchronize()
    assert seg(P(da), P(w), z, z, P(d), z, z, m, 320, 0, 0, k, s) != 0          # not whole 256-column tiles
    assert seg(P(da), P(w), z, P(w), P(d), z, P(d), m, 256, 0, 256, k, s) != 0   # third segment without second
    assert seg(P(da), P(w), z, z, P(d), z, z, m, 256, 256, 0, k, s) != 0         # segment without pointers
    assert seg(P(da), P(w), z, z, P(d), z, z, 96, 256, 0, 0, k, s) != 0          # M % 64
    assert seg(P(da), P(w), z, z, P(d), z, z, m, 256, 0, 0, 256, s) != 0         # K % 512
    assert rf.rf_gemm_q6_k_segments_launch(P(da), P(w), z, z, P(d), z, z, m, 256, 0, 0, 1024, s) != 0  # Q6_K K % 2048
    acc = rf.rf_gemm_q4_k_accumulate_launch
    assert acc(P(da), P(w), z, m, 256, k, s) != 0                                # no output
    assert acc(ctypes.c_void_p(da.data_ptr() + 4), P(w), P(d), m, 256, k, s) != 0   # A misaligned
    assert acc(P(da), P(w), P(d), m, 64, k, s) != 0                              # N % 256
    sw = rf.rf_gemm_q4_k_swiglu_launch
    assert sw(P(da), P(w), P(w), P(d), m, 64, k, s) != 0                         # N % 128
    assert sw(P(da), P(w), z, P(d), m, 128, k, s) != 0                           # no up weights


# (M, [(type, width)], K): Q4_K / Q6_K mixes of the prefill Q/K/V
@pytest.mark.parametrize("m,segs,k", [
    (512, [("q4_k", 4096), ("q4_k", 1024), ("q6_k", 1024)], 4096),    # Qwen3-8B layer with a Q6_K V
    (320, [("q4_k", 512), ("q4_k", 128), ("q4_k", 128)], 2048),       # all Q4_K, partial 128-row tile
    (320, [("q4_k", 512), ("q6_k", 128), ("q4_k", 192)], 2048),       # Q6_K on 128-row tiles beside 256-row Q4_K
    (64, [("q6_k", 192), ("q4_k", 64)], 2048),                        # two segments, one 64-row M tile
])
def test_f16_segments_mixed_types(rf, dev, m, segs, k):
    # each segment bit for bit its matrix alone through the same launcher
    # (the same 128 x 64 tiles: segment routing moves no bits), and within
    # the GEMM bar of the oracle
    a = torch.from_numpy(synth.activations(k, seed=m + 3, m=m)).to(torch.bfloat16).float().numpy()
    da = G.to_dev(a.astype(np.float16).view(np.int16))
    ws = [synth.weights(f, n, k, seed=30 + i) for i, (f, n) in enumerate(segs)]
    dws = [G.to_dev(w) for w in ws]
    ds = [G.empty(m * n, torch.float32).fill_(float("nan")) for _, n in segs]
    z = ctypes.c_void_p(0)
    types = [12 if f == "q4_k" else 14 for f, _ in segs] + [12] * (3 - len(segs))
    G.call(rf.rf_gemm_qk_f16_segments_launch, G.ptr(da), *([G.ptr(t) for t in dws] + [z] * (3 - len(segs))), *types,
           *([G.ptr(t) for t in ds] + [z] * (3 - len(segs))), m, *([n for _, n in segs] + [0] * (3 - len(segs))), k)
    for i, ((f, n), w, dw, d) in enumerate(zip(segs, ws, dws, ds)):
        got = G.host(d).reshape(m, n)
        np.testing.assert_array_equal(got, _f16_alone(rf, f, da, w, m, n, k))
        _check(got, O.gemm(f, a, w, m, n, k), f"f16 segment {i} {f} {m}x{n}x{k}")


def test_f16_segments_rejections(rf, dev):
    m, k = 64, 2048
    da = G.to_dev(np.zeros(m * k, np.int16))
    w = G.to_dev(synth.weights("q4_k", 64, k, seed=1))
    d = G.empty(m * 64, torch.float32)
    s = G.stream()
    z = ctypes.c_void_p(0)
    P = G.ptr
    f = rf.rf_gemm_qk_f16_segments_launch
    assert f(P(da), P(w), z, z, 12, 12, 12, P(d), z, z, m, 64, 0, 0, k, s) == 0
    torch.cuda.synchronize()
    assert f(P(da), P(w), z, z, 13, 12, 12, P(d), z, z, m, 64, 0, 0, k, s) != 0       # not Q4_K / Q6_K
    assert f(P(da), P(w), z, z, 14, 12, 12, P(d), z, z, m, 64, 0, 0, 1024, s) != 0    # Q6_K needs K % 2048
    assert f(P(da), P(w), z, z, 12, 12, 12, P(d), z, z, m, 96, 0, 0, k, s) != 0       # width % 64
    assert f(P(da), P(w), z, P(w), 12, 12, 12, P(d), z, P(d), m, 64, 0, 64, k, s) != 0  # third without second
    assert f(P(da), P(w), P(w), z, 12, 12, 12, P(d), z, z, m, 64, 64, 0, k, s) != 0     # segment without output
    assert f(P(da), P(w), z, z, 12, 12, 12, P(d), z, z, 96, 64, 0, 0, k, s) != 0      # M % 64
    assert f(ctypes.c_void_p(da.data_ptr() + 2), P(w), z, z, 12, 12, 12, P(d), z, z, m, 64, 0, 0, k, s) != 0


@pytest.mark.parametrize("m,n,k,f16", [(512, 12288, 4096, True), (512, 12288, 4096, False), (320, 192, 1024, True),
                                       (64, 64, 256, False)])
def test_q4k_f16_swiglu(rf, dev, m, n, k, f16):
    # gate and up in one launch with SwiGLU in the epilogue: at 512 x 12288
    # (the 256 x 128 tiles the plain launcher takes there too) bit for bit two
    # fp16-activation GEMMs and the SwiGLU kernel; every shape within the bar
    # of the oracle's silu(gate) * up (plus the fp16 rounding of the output)
    a = torch.from_numpy(synth.activations(k, seed=m + 9, m=m)).to(torch.bfloat16).float().numpy()
    da = G.to_dev(a.astype(np.float16).view(np.int16))
    wg, wu = synth.weights("q4_k", n, k, seed=41), synth.weights("q4_k", n, k, seed=42)
    dwg, dwu = G.to_dev(wg), G.to_dev(wu)
    out = G.empty(m * n, torch.int16 if f16 else torch.float32)
    G.call(rf.rf_gemm_q4_k_f16_swiglu_launch, G.ptr(da), G.ptr(dwg), G.ptr(dwu), G.ptr(out), int(f16), m, n, k)
    got = G.host(out).view(np.float16).astype(np.float32) if f16 else G.host(out)
    got = got.reshape(m, n)
    if m == 512:
        g, u = G.empty(m * n, torch.float32), G.empty(m * n, torch.float32)
        G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dwg), G.ptr(g), m, n, k)
        G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dwu), G.ptr(u), m, n, k)
        ref = G.empty(m * n, torch.int16 if f16 else torch.float32)
        if f16:
            G.call(rf.rf_silu_mul_f16_on_stream, G.ptr(g), G.ptr(u), G.ptr(ref), m * n)
            np.testing.assert_array_equal(G.host(out), G.host(ref))
        else:
            G.call(rf.rf_silu_mul_on_stream, G.ptr(g), G.ptr(u), G.ptr(ref), m * n)
            np.testing.assert_array_equal(G.host(out), G.host(ref))
    gr, ur = O.gemm("q4_k", a, wg, m, n, k), O.gemm("q4_k", a, wu, m, n, k)
    ref = gr / (1.0 + np.exp(-gr)) * ur
    scale = np.abs(ref).max()
    err = np.abs(got.astype(np.float64) - ref)
    tol = (4e-3 if f16 else 2e-3) * np.abs(ref) + 1e-4 * scale
    print(f"q4_k f16 swiglu {m}x{n}x{k}: worst={(err / tol).max():.3f}", flush=True)
    assert (err / tol).max() <= 1.0


@pytest.mark.parametrize("m,n,k", [(512, 12288, 1024), (256, 12288, 1024), (64, 256, 512), (320, 128, 256),
                                   (512, 4096, 12288)])
def test_q4k_f16_swiglu_up(rf, dev, m, n, k):
    # the up GEMM with the SwiGLU in its store (the gate product read back):
    # bit for bit the plain fp16-activation GEMM and the SwiGLU kernel, on
    # each tile kind (256 x 128 tiles at 512 x 12288, K-sliced 256-row tiles
    # unsplit at 256 x 12288 and split over K at 512 x 4096 x 12288 -- the
    # SwiGLU then in the split reduction --, 128- and 64-row tiles, a partial
    # last tile at M = 320)
    a = torch.from_numpy(synth.activations(k, seed=m + 3, m=m)).to(torch.bfloat16).float().numpy()
    da = G.to_dev(a.astype(np.float16).view(np.int16))
    wu = G.to_dev(synth.weights("q4_k", n, k, seed=43))
    gate = G.to_dev((np.random.default_rng(m).standard_normal(m * n) * 3).astype(np.float32))
    out = G.empty(m * n, torch.int16)
    G.call(rf.rf_gemm_q4_k_f16_swiglu_up_launch, G.ptr(da), G.ptr(wu), G.ptr(gate), G.ptr(out), m, n, k)
    u = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(wu), G.ptr(u), m, n, k)
    ref = G.empty(m * n, torch.int16)
    G.call(rf.rf_silu_mul_f16_on_stream, G.ptr(gate), G.ptr(u), G.ptr(ref), m * n)
    np.testing.assert_array_equal(G.host(out), G.host(ref))


def test_q4k_f16_swiglu_up_full_k_oracle(rf, dev):
    # the up GEMM the Qwen3-8B prefill runs at 512 tokens (M = 512, N = 12288,
    # K = 4096: 256 x 128 tiles, 64 chunks of K) against the oracle:
    # out = fp16(silu(g) * u), u the float64 product of the fp16 operands.
    # Bar per element: the GEMM bar on u (2e-3 |u| + 2e-5 S, S the sum of the
    # product magnitudes u adds up) carried through the factor |silu(g)|, plus
    # one fp16 rounding of the output (half an ulp: 2^-11 |out| relative,
    # 2^-25 absolute below the normal range)
    m, n, k = 512, 12288, 4096
    a = torch.from_numpy(synth.activations(k, seed=51, m=m)).to(torch.bfloat16).float().numpy()
    wu = synth.weights("q4_k", n, k, seed=52)
    g = (np.random.default_rng(53).standard_normal(m * n) * 3).astype(np.float32)
    da, dwu, dg = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(wu), G.to_dev(g)
    out = G.empty(m * n, torch.int16)
    G.call(rf.rf_gemm_q4_k_f16_swiglu_up_launch, G.ptr(da), G.ptr(dwu), G.ptr(dg), G.ptr(out), m, n, k)
    got = G.host(out).view(np.float16).astype(np.float64).reshape(m, n)
    u = O.gemm("q4_k", a, wu, m, n, k)
    S = O.gemm_abs("q4_k", a, wu, m, n, k)
    g64 = g.astype(np.float64).reshape(m, n)
    silu = g64 / (1.0 + np.exp(-g64))
    ref = silu * u
    tol = np.abs(silu) * (2e-3 * np.abs(u) + 2e-5 * S) + 2.0 ** -11 * np.abs(ref) + 2.0 ** -25
    worst = (np.abs(got - ref) / tol).max()
    print(f"q4_k f16 swiglu_up {m}x{n}x{k}: worst={worst:.3f}", flush=True)
    assert worst <= 1.0


def test_q4k_f16_swiglu_up_rejections(rf, dev):
    m, n, k = 64, 128, 256
    da = G.to_dev(np.zeros(m * k, np.int16))
    w = G.to_dev(synth.weights("q4_k", n, k, seed=1))
    g = G.empty(m * n, torch.float32)
    o = G.empty(m * n, torch.int16)
    s = G.stream()
    z = ctypes.c_void_p(0)
    P = G.ptr
    f = rf.rf_gemm_q4_k_f16_swiglu_up_launch
    assert f(P(da), P(w), P(g), P(o), m, n, k, s) == 0
    torch.cuda.synchronize()
    assert f(P(da), P(w), z, P(o), m, n, k, s) != 0                              # no gate
    assert f(P(da), P(w), P(g), ctypes.c_void_p(g.data_ptr() + 64), m, n, k, s) != 0   # output inside the gate
    assert f(P(da), P(w), P(g), P(o), m, 96, k, s) != 0                          # N % 128
    assert f(P(da), P(w), P(g), P(o), 32, n, k, s) != 0                          # M % 64
    assert f(P(da), P(w), P(g), P(o), m, n, 320, s) != 0                         # K % 256


def test_q4k_f16_swiglu_rejections(rf, dev):
    m, k = 64, 256
    da = G.to_dev(np.zeros(m * k, np.int16))
    w = G.to_dev(synth.weights("q4_k", 64, k, seed=1))
    d = G.empty(m * 64, torch.float32)
    s = G.stream()
    z = ctypes.c_void_p(0)
    P = G.ptr
    f = rf.rf_gemm_q4_k_f16_swiglu_launch
    assert f(P(da), P(w), P(w), P(d), 0, m, 64, k, s) == 0
    torch.cuda.synchronize()
    assert f(P(da), P(w), z, P(d), 0, m, 64, k, s) != 0          # no up weights
    assert f(P(da), P(w), P(w), P(d), 0, m, 96, k, s) != 0       # N % 64
    assert f(P(da), P(w), P(w), P(d), 0, 32, 64, k, s) != 0      # M % 64
    assert f(P(da), P(w), P(w), P(d), 0, m, 64, 320, s) != 0     # K % 256


# (format, M, N, K): the down projection of a prefill layer into the residual
# stream with the next layer's attention norm -- split over K (the norm taken
# in the reduction: N = 2048, 4096, 6144) and unsplit (the separate norm)
@pytest.mark.parametrize("fmt,m,n,k", [
    ("q4_k", 512, 4096, 12288),    # 256 x 128 tiles split over K in four
    ("q6_k", 512, 4096, 12288),    # 256 x 64 tiles split over K
    ("q4_k", 64, 2048, 4096),      # 64-row tiles split over K, one 2048 group per row
    ("q6_k", 128, 6144, 2048),     # three 2048 groups per row
    ("q4_k", 512, 4096, 4096),     # 128-row tiles, no split: the separate norm
])
def test_accumulate_rmsnorm_bits(rf, dev, fmt, m, n, k):
    # inout and the fp16 norm bit for bit the accumulate launcher followed by
    # rf_rms_norm_batched_f16_on_stream; the norm within its own bar of the
    # float64 RMSNorm of the accumulated rows
    a = torch.from_numpy(synth.activations(k, seed=m + n, m=m)).to(torch.bfloat16).float().numpy()
    da = G.to_dev(a.astype(np.float16).view(np.int16))
    dw = G.to_dev(synth.weights(fmt, n, k, seed=k + 5))
    r0 = np.random.default_rng(n).standard_normal((m, n)).astype(np.float32)
    gw = (np.random.default_rng(k).random(n) + 0.5).astype(np.float32)
    dg = G.to_dev(gw)
    eps = ctypes.c_float(1e-6)
    ref_io, got_io = G.to_dev(r0), G.to_dev(r0)
    ref_o = G.empty(m * n, torch.int16).fill_(-1)
    got_o = G.empty(m * n, torch.int16).fill_(-1)
    acc = rf.rf_gemm_q4_k_f16_accumulate_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_f16_accumulate_launch
    G.call(acc, G.ptr(da), G.ptr(dw), G.ptr(ref_io), m, n, k)
    G.call(rf.rf_rms_norm_batched_f16_on_stream, G.ptr(ref_io), G.ptr(dg), G.ptr(ref_o), n, eps, m)
    fused = (rf.rf_gemm_q4_k_f16_accumulate_rmsnorm_launch if fmt == "q4_k"
             else rf.rf_gemm_q6_k_f16_accumulate_rmsnorm_launch)
    G.call(fused, G.ptr(da), G.ptr(dw), G.ptr(got_io), G.ptr(dg), eps, G.ptr(got_o), m, n, k)
    np.testing.assert_array_equal(G.host(got_io), G.host(ref_io))
    np.testing.assert_array_equal(G.host(got_o), G.host(ref_o))
    h = G.host(got_io).reshape(m, n).astype(np.float64)
    want = h / np.sqrt((h * h).mean(axis=1, keepdims=True) + 1e-6) * gw
    got = G.host(got_o).view(np.float16).reshape(m, n).astype(np.float64)
    assert (np.abs(got - want) <= 1e-3 * np.abs(want) + 1e-4).all(), f"{fmt} {m}x{n}x{k} norm"
