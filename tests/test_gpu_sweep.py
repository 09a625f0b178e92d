"""Seeded random-shape sweep of the launchers, through the C ABI, against the
oracle at the bars of test_gpu_gemv.py / test_gpu_gemm.py.

The fixed-shape tests pin the kernels at the shapes they were tuned for and at
the edges each kernel's routing names; this sweep draws shapes at random (a
fixed seed, so every run draws the same ones) to reach the combinations of
tile counts, K splits, ragged row counts and ring positions that no one
picked by hand: GEMV row counts from 1 to a few thousand with K up to the
Q8 LDS limit (30720, the K-split kernel for long rows included), and GEMM
shapes M, N multiples of 64, K of 256 (of 2048 where a Q6_K fp16 tile needs
it).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rocmforge_amd import synth
from tests import gpu_util as G
from tests.test_gpu_gemm import _check as gemm_check
from tests.test_gpu_gemv import _check as gemv_check

pytestmark = pytest.mark.gpu

_R = np.random.default_rng(20261202)


def _gemv_shapes(count, k_max_blocks, long_rows=0):
    out = []
    for _ in range(count):
        k = 256 * int(_R.integers(1, k_max_blocks + 1))
        n = int(_R.integers(1, 5001))
        out.append((k, n))
    for _ in range(long_rows):       # K a multiple of 4096 from 8192: the K-split Q8 kernel
        out.append((4096 * int(_R.integers(2, 8)), int(_R.integers(1, 5001))))
    return out


def _gemm_shapes(count, k_unit=256, k_max_units=24, n_max=48):
    return [(64 * int(_R.integers(1, 9)), 64 * int(_R.integers(1, n_max + 1)),
             k_unit * int(_R.integers(1, k_max_units + 1))) for _ in range(count)]


Q8_SHAPES = _gemv_shapes(8, 120, long_rows=3)
F32_SHAPES = _gemv_shapes(6, 160)
Q6_SHAPES = _gemv_shapes(8, 160)
GEMM_SHAPES = _gemm_shapes(8)
Q6_F16_SHAPES = _gemm_shapes(5, k_unit=2048, k_max_units=4)


@pytest.mark.parametrize("k,n", Q8_SHAPES)
def test_sweep_q4k_q8(rf, dev, k, n):
    w = synth.q4_k_weights(n, k, seed=k + 3 * n)
    w2 = synth.q4_k_weights(n, k, seed=k + 3 * n + 1)
    x = synth.activations(k, seed=k - n)
    r = synth.activations(n, seed=n + 7) * 10
    dw, dw2, dx, dr = G.to_dev(w), G.to_dev(w2), G.to_dev(x), G.to_dev(r)
    ref = O.gemv_q4k_q8(w, x, k, n)
    y = G.empty(n, torch.float32)
    G.call(rf.gemv_q4_k_f32_q8_inline_launch, G.ptr(dw), G.ptr(dx), G.ptr(y), k, n)
    gemv_check(G.host(y), ref, f"sweep q8 {n}x{k}")
    G.call(rf.gemv_q4_k_f32_q8_inline_residual_launch, G.ptr(dw), G.ptr(dx), G.ptr(dr), G.ptr(dr), k, n)
    gemv_check(G.host(dr), ref + r.astype(np.float64), f"sweep q8 residual {n}x{k}")
    G.call(rf.gemv_gate_up_swiglu_q4_k_f32_q8_inline_launch, G.ptr(dw), G.ptr(dw2), G.ptr(dx), G.ptr(y), k, n)
    gemv_check(G.host(y), O.swiglu(ref, O.gemv_q4k_q8(w2, x, k, n)), f"sweep q8 gate_up {n}x{k}")


@pytest.mark.parametrize("k,n", F32_SHAPES)
def test_sweep_q4k_f32(rf, dev, k, n):
    w = synth.q4_k_weights(n, k, seed=k + 5 * n)
    x = synth.activations(k, seed=k + n)
    dw, dx = G.to_dev(w), G.to_dev(x)
    y = G.empty(n, torch.float32)
    G.call(rf.gemv_q4_k_f32_launch, G.ptr(dw), G.ptr(dx), G.ptr(y), k, n)
    gemv_check(G.host(y), O.gemv_q4k_f32(w, x, k, n), f"sweep f32 {n}x{k}")


@pytest.mark.parametrize("k,n", Q6_SHAPES)
def test_sweep_q6k(rf, dev, k, n):
    w = synth.q6_k_weights(n, k, seed=k + 7 * n)
    x = synth.activations(k, seed=k + 2 * n)
    r = synth.activations(n, seed=n + 11) * 10
    dw, dx, dr = G.to_dev(w), G.to_dev(x), G.to_dev(r)
    ref = O.gemv_q6k(w, x, k, n)
    y = G.empty(n, torch.float32)
    G.call(rf.gemv_q6_k_f32_launch, G.ptr(dw), G.ptr(dx), G.ptr(y), k, n)
    gemv_check(G.host(y), ref, f"sweep q6 {n}x{k}")
    G.call(rf.gemv_q6_k_f32_residual_launch, G.ptr(dw), G.ptr(dx), G.ptr(dr), G.ptr(dr), k, n)
    gemv_check(G.host(dr), ref + r.astype(np.float64), f"sweep q6 residual {n}x{k}")


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_sweep_gemm_reference_entry(rf, dev, fmt, m, n, k):
    a = torch.from_numpy(synth.activations(k, seed=m + n, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.weights(fmt, n, k, seed=k + n + m)
    da, dw = G.to_dev(a), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    fn = rf.wmma_gemm_q4_k_launch if fmt == "q4_k" else rf.wmma_gemm_q6_k_launch
    G.call(fn, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    gemm_check(G.host(d).reshape(m, n), fmt, a, w, m, n, k, f"sweep {fmt} M={m} {n}x{k}")
    # D += product on the same operands: the caller's contents plus the sums
    # (N % 256 and K % 512, Q6_K K % 2048; other shapes are rejected)
    r = synth.activations(n, seed=m + 3, m=m)
    dr = G.to_dev(r)
    acc = rf.rf_gemm_q4_k_accumulate_launch if fmt == "q4_k" else rf.rf_gemm_q6_k_accumulate_launch
    if n % 256 or k % (512 if fmt == "q4_k" else 2048):
        assert acc(G.ptr(da), G.ptr(dw), G.ptr(dr), m, n, k, G.stream()) == 1       # hipErrorInvalidValue
        torch.cuda.synchronize()
        np.testing.assert_array_equal(G.host(dr).reshape(m, n), r)                   # nothing written
        return
    G.call(acc, G.ptr(da), G.ptr(dw), G.ptr(dr), m, n, k)
    got = G.host(dr).reshape(m, n)
    ref = O.gemm(fmt, a, w, m, n, k)
    err = np.abs(got.astype(np.float64) - r - ref)
    tol = 2e-3 * np.abs(ref) + 2e-5 * O.gemm_abs(fmt, a, w, m, n, k) + 1e-6 * np.abs(r)
    assert (err <= tol).all(), f"sweep {fmt} accumulate M={m} {n}x{k}: worst {(err / tol).max():.3f}"


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_sweep_gemm_q4k_fp16_activations(rf, dev, m, n, k):
    a = torch.from_numpy(synth.activations(k, seed=m + 2 * n, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.q4_k_weights(n, k, seed=k + 2 * n)
    da, dw = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q4_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    gemm_check(G.host(d).reshape(m, n), "q4_k", a, w, m, n, k, f"sweep fp16-A q4_k M={m} {n}x{k}")


@pytest.mark.parametrize("m,n,k", Q6_F16_SHAPES)
def test_sweep_gemm_q6k_fp16_activations(rf, dev, m, n, k):
    a = torch.from_numpy(synth.activations(k, seed=m + 3 * n, m=m)).to(torch.bfloat16).float().numpy()
    w = synth.weights("q6_k", n, k, seed=k + 3 * n)
    da, dw = G.to_dev(a.astype(np.float16).view(np.int16)), G.to_dev(w)
    d = G.empty(m * n, torch.float32)
    G.call(rf.rf_gemm_q6_k_f16_launch, G.ptr(da), G.ptr(dw), G.ptr(d), m, n, k)
    gemm_check(G.host(d).reshape(m, n), "q6_k", a, w, m, n, k, f"sweep fp16-A q6_k M={m} {n}x{k}")
