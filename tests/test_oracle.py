"""Pins the C oracle (oracle/qk_oracle.c) on the CPU.

Each oracle function is checked against something it does not share code
with: numpy's IEEE float16, the reference's golden JSON of real Qwen3-8B
Q4_K blocks, hand-worked byte-level blocks from the reference's own tests,
an independent numpy decoder (tests/qk_numpy.py), brute-force integer dots
and closed-form invariants of the Q8_0 quantiser.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from rocmforge_amd import synth
from tests import qk_numpy as NP

GOLDEN = Path(__file__).resolve().parent / "golden" / "q4_k_m_qwen3_8b_ffn_gate_layer0_first3_blocks.json"


# ---- fp16 conversions -------------------------------------------------------

def test_f16_to_f32_all_halves_match_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_bits_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    # random bit patterns over the whole float range + the half range
    a = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = (rng.standard_normal(1 << 18) * np.exp2(rng.integers(-30, 20, 1 << 18))).astype(np.float32)
    # exact ties between adjacent halves (round-half-even cases), incl. subnormals
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 1e-30, 2**-24, 2**-25, 2**-25 * 1.0000001, 3 * 2**-26,
                      -0.0, 0.0, np.inf, -np.inf], np.float32)
    for x in (a[np.isfinite(a)], b, ties, -ties, edges):
        got = O.round_f16(x)
        with np.errstate(over="ignore"):
            ref = x.astype(np.float16).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert O.f32_to_f16_bits(np.float32(1e-30)) == 0
    assert O.f32_to_f16_bits(np.float32(70000.0)) == 0x7C00
    assert O.f32_to_f16_bits(np.float32(0.5)) == 0x3800


# ---- Q4_K: golden vectors from real Qwen3-8B blocks -------------------------

def _golden_blocks():
    data = json.loads(GOLDEN.read_text())
    assert data["block_size_bytes"] == 144
    return data["blocks"]


def test_q4k_scale_min_golden():
    for b in _golden_blocks():
        raw = bytes.fromhex(b["raw_hex"])
        assert list(raw[4:16]) == b["scales_bytes"]
        for e in b["unpacked_scale_min_per_subblock"]:
            assert O.q4k_scale_min(e["j"], raw[4:16]) == (e["scale_6bit"], e["min_6bit"])


def test_q4k_dequant_golden():
    for b in _golden_blocks():
        raw = np.frombuffer(bytes.fromhex(b["raw_hex"]), np.uint8)
        assert O.f16_bits_to_f32(int(raw[0]) | int(raw[1]) << 8) == b["d_fp32"]
        assert O.f16_bits_to_f32(int(raw[2]) | int(raw[3]) << 8) == b["dmin_fp32"]
        v64 = O.q4k_dequant(raw, 1, f64=True)
        # the golden values were produced in float64 by the reference's generator
        np.testing.assert_allclose(v64[:64], b["dequantized_first_64"], rtol=0, atol=1e-15)
        np.testing.assert_allclose(v64[-8:], b["dequantized_last_8"], rtol=0, atol=1e-15)
        v32 = O.q4k_dequant(raw, 1, f64=False)
        np.testing.assert_allclose(v32[:64], b["dequantized_first_64"], rtol=1e-6, atol=1e-9)


def test_q4k_docs_worked_example():
    # docs/q4_k_m_block_format.md:186-219: value[0] = d*58*nib - dmin*39 = -0.01575.
    # The doc prints nib = 6, but qs[0] = 0x63 holds 3 in its low nibble, and
    # only 3 reproduces -0.01575 (6 would give -0.00136): the doc's 6 is a typo.
    raw = np.frombuffer(bytes.fromhex(_golden_blocks()[0]["raw_hex"]), np.uint8)
    assert (raw[16] & 0x0F) == 3
    assert O.q4k_dequant(raw, 1)[0] == pytest.approx(-0.01574993133544922, abs=1e-12)


def _byte_level_q4k_block():
    # tests/wmma_q4_k_correctness.rs:111-125 of the reference
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.25], np.float16).view(np.uint8)
    blk[4:8] = [3, 5, 7, 9]
    blk[8:12] = [1, 2, 3, 4]
    blk[12:16] = [0x00, 0x11, 0x22, 0x33]
    i = np.arange(128)
    blk[16:] = (((i + 1) & 15) << 4) | (i & 15)
    return blk


def test_q4k_byte_level_block():
    blk = _byte_level_q4k_block()
    v = O.q4k_dequant(blk, 1)
    # hand-worked: sub-block 0 scale 3 min 1: elem i = 0.5*3*(i&15) - 0.25*1
    assert v[0] == -0.25 and v[5] == 0.5 * 3 * 5 - 0.25
    # sub-block 1 (high nibbles of qs[0..31]) scale 5 min 2: elem 32+i = 2.5*((i+1)&15) - 0.5
    assert v[32] == 2.5 * 1 - 0.5 and v[32 + 15] == 2.5 * 0 - 0.5
    # sub-block 4 scale 0 min 0 -> all zero; sub-block 7 scale 3 min 3
    assert np.all(v[128:160] == 0.0)
    assert v[224] == 0.5 * 3 * ((96 + 1) & 15) - 0.25 * 3
    np.testing.assert_array_equal(v, NP.q4k_dequant(blk))


def test_q4k_dequant_matches_numpy_decoder():
    w = synth.q4_k_weights(64, 1024, seed=3)
    for row in range(0, 64, 7):
        a = O.q4k_dequant(w[row], 4)
        np.testing.assert_array_equal(a, NP.q4k_dequant(w[row]))


# ---- Q6_K -------------------------------------------------------------------

def _byte_level_q6k_block():
    # tests/wmma_q6_k_correctness.rs:84-103 of the reference
    blk = np.zeros(210, np.uint8)
    i = np.arange(128)
    blk[0:128] = (((i + 1) & 15) << 4) | (i & 15)
    blk[128:192] = (np.arange(64) * 7) & 0xFF
    blk[192:208] = np.array([4, -3, 7, -5, 2, -1, 6, -4, 1, 3, -2, 5, -6, 8, -7, 2], np.int8).view(np.uint8)
    blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
    return blk


def test_q6k_byte_level_block():
    blk = _byte_level_q6k_block()
    v = O.q6k_dequant(blk, 1)
    # elem 0: ql[0]&15 = 0, qh[0] = 0 -> q6 = 0 -> 0.5*4*(0-32) = -64
    assert v[0] == -64.0
    # elem 1: ql[1]&15 = 1, (qh[1]=7)&3 = 3 -> q6 = 1|48 = 49 -> 0.5*4*17 = 34
    assert v[1] == 34.0
    # elem 32+1 (q=1): ql[33]&15 = 1, (7>>2)&3 = 1 -> 17 -> 0.5*sc[2]=7 * (17-32) = -52.5
    assert v[33] == -52.5
    # elem 64+16 (q=2, l=16): ql[16]>>4 = 1, qh[16]=112 -> (112>>4)&3 = 3 -> 49; sc[4+1]=-1 -> -8.5
    assert v[80] == -8.5
    # second half, elem 128+96+31 (q=3, l=31): ql[64+32+31]=ql[127] >> 4 = 0, qh[32+31]=441&255=185 ->
    # (185>>6)&3 = 2 -> q6 = 32 -> 0
    assert v[255] == 0.0
    np.testing.assert_array_equal(v.astype(np.float64), NP.q6k_dequant(blk))


def test_q6k_dequant_matches_numpy_decoder():
    w = synth.q6_k_weights(32, 1024, seed=4)
    for row in range(0, 32, 5):
        np.testing.assert_array_equal(O.q6k_dequant(w[row], 4).astype(np.float64), NP.q6k_dequant(w[row]))


# ---- Q8_0 quantiser -----------------------------------------------------------

def _q8_inputs():
    rng = np.random.default_rng(7)
    parts = [rng.standard_normal(32 * 512).astype(np.float32)]
    mags = np.exp2(rng.integers(-40, 40, size=512)).astype(np.float32)
    parts.append((rng.standard_normal((512, 32)) * mags[:, None]).astype(np.float32).ravel())
    z = np.zeros(32 * 4, np.float32)
    z[32 + 5] = 1e-35   # d underflows to 0 -> inf scale -> clamp
    z[64:96] = -0.0
    parts.append(z)
    parts.append(np.full(32, 3e38, np.float32))           # d overflows to inf -> q = 0
    parts.append(np.linspace(-127, 127, 32).astype(np.float32))
    return np.concatenate(parts)


def test_q8_0_matches_numpy_semantics():
    x = _q8_inputs()
    d, q = O.q8_0_quantize(x)
    dn, qn = NP.q8_0_quantize(x)
    assert np.array_equal(d, dn)
    assert np.array_equal(q, qn)


def test_q8_0_edge_blocks_and_invariants():
    x = _q8_inputs()
    d, q = O.q8_0_quantize(x)
    qb = q.reshape(-1, 32).astype(np.int32)
    assert np.abs(qb).max() <= 127
    df = d.view(np.float16).astype(np.float32)
    xb = x.reshape(-1, 32)
    # all-zero block: d = 0 and q = -127 everywhere (0 * inf = NaN -> fmaxf -> -127)
    zero_rows = np.where(np.all(xb == 0, axis=1))[0]
    assert len(zero_rows) >= 2
    for r in zero_rows:
        assert d[r] in (0, 0x8000) and np.all(qb[r] == -127)
    # tiny block: d underflows, the non-zero element saturates, zeros -> -127
    tiny = np.where((np.abs(xb).max(axis=1) > 0) & (df == 0))[0]
    assert len(tiny) >= 1
    # overflow block: d = inf, inv = 0, q = 0
    big = np.where(np.isinf(df))[0]
    assert len(big) >= 1 and np.all(qb[big] == 0)
    # normal blocks: |x/d - q| < 1 (truncation) and the amax element maps to 126 or 127
    ok = np.isfinite(df) & (df > 0) & (np.abs(xb).max(axis=1) / 127 >= 6.1e-5)
    r = xb[ok] / df[ok][:, None]
    assert np.all(np.abs(r - qb[ok]) < 1.0 + 1e-6)
    amax_q = np.abs(qb[ok])[np.arange(ok.sum()), np.argmax(np.abs(xb[ok]), axis=1)]
    assert np.all((amax_q == 127) | (amax_q == 126))


def test_q8_0_brute_force_all_fp16_scales():
    # for every normal fp16 d, a block whose amax is 127*d must round-trip to
    # d exactly and map its amax element to +-127
    h = np.arange(0x0400, 0x7BFF, 37, dtype=np.uint16)
    dv = h.view(np.float16).astype(np.float32)
    x = np.zeros((len(h), 32), np.float32)
    x[:, 3] = dv * np.float32(127.0)
    x[:, 7] = -dv * np.float32(50.0)
    x = x.ravel()
    d, q = O.q8_0_quantize(x)
    dn, qn = NP.q8_0_quantize(x)
    assert np.array_equal(d, dn) and np.array_equal(q, qn)
    # the fp16 scale recovers d exactly; the amax element truncates to 126 or
    # 127 (127*d is rounded to fp32 before the division)
    assert np.array_equal(d, h)
    qa = q.reshape(-1, 32)[:, 3]
    assert np.all((qa == 127) | (qa == 126)) and (qa == 127).mean() > 0.5
    assert np.all(q.reshape(-1, 32)[:, 7] == -50) or np.all(np.abs(q.reshape(-1, 32)[:, 7] + 50) <= 1)


# ---- integer partials and GEMVs ---------------------------------------------

def test_q4k_q8_partials_brute_force():
    k, n = 512, 5
    w = synth.q4_k_weights(n, k, seed=11)
    x = synth.activations(k, seed=12)
    _, xq = O.q8_0_quantize(x)
    dots, sums = O.q4k_q8_partials(w, xq, k, n)
    for row in range(n):
        _, _, _, _, nib = NP.q4k_fields(w[row])
        nib = nib.reshape(-1)
        want = (nib * xq.astype(np.int64)).reshape(-1, 32).sum(axis=1)
        assert np.array_equal(dots[row], want)
    assert np.array_equal(sums, xq.reshape(-1, 32).astype(np.int64).sum(axis=1))


def test_gemv_q4k_q8_oracle_against_numpy():
    k, n = 1024, 33
    w = synth.q4_k_weights(n, k, seed=21)
    x = synth.activations(k, seed=22)
    y = O.gemv_q4k_q8(w, x, k, n)
    dh, xq = NP.q8_0_quantize(x)
    xd = dh.view(np.float16).astype(np.float64)
    qsum = xq.reshape(-1, 32).astype(np.int64).sum(axis=1)
    want = np.empty(n)
    for row in range(n):
        d, dmin, sc, m, nib = NP.q4k_fields(w[row])
        dots = (nib.reshape(-1) * xq.astype(np.int64)).reshape(-1, 32).sum(axis=1).reshape(-1, 8)
        terms = xd.reshape(-1, 8) * (d[:, None] * sc * dots - dmin[:, None] * m * qsum.reshape(-1, 8))
        want[row] = terms.sum()
    np.testing.assert_allclose(y, want, rtol=1e-12, atol=1e-12)


def test_gemv_q4k_q8_close_to_fp32_activation_gemv():
    # the reference's own criterion (tests/q4_k_q8_inline_correctness.rs:145-207):
    # Q8 activations stay within 1.5e-2 of max|y| of the fp32-activation GEMV.
    # A dropped dmin term or a sign slip moves this by orders of magnitude.
    k, n = 4096, 64
    w = synth.q4_k_weights(n, k, seed=31)
    x = synth.activations(k, seed=32)
    yq = O.gemv_q4k_q8(w, x, k, n)
    yf = O.gemv_q4k_f32(w, x, k, n)
    assert np.abs(yq - yf).max() / np.abs(yf).max() < 1.5e-2
    dq = np.stack([NP.q4k_dequant(w[r]) for r in range(n)])
    np.testing.assert_allclose(yf, dq @ x.astype(np.float64), rtol=1e-10, atol=1e-10)


def test_gemv_q6k_oracle_against_numpy():
    k, n = 1024, 17
    w = synth.q6_k_weights(n, k, seed=41)
    x = synth.activations(k, seed=42)
    dq = np.stack([NP.q6k_dequant(w[r]) for r in range(n)])
    np.testing.assert_allclose(O.gemv_q6k(w, x, k, n), dq @ x.astype(np.float64), rtol=1e-10, atol=1e-10)


def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0])
    u = np.array([2.0, 3.0, 4.0, 1.0, 1.0])
    out = O.swiglu(g, u)
    np.testing.assert_allclose(out, g / (1 + np.exp(-g)) * u, rtol=1e-15)
    assert out[0] == 0.0 and out[3] == pytest.approx(20.0, rel=1e-8)


def test_gemm_operands_are_fp16_rounded():
    m, n, k = 4, 8, 256
    a = synth.activations(k, seed=51, m=m)
    w = synth.q4_k_weights(n, k, seed=52)
    wf = O.dequant_f16("q4_k", w, n, k)
    assert np.array_equal(wf, wf.astype(np.float16).astype(np.float32))
    ref = np.stack([NP.q4k_dequant(w[r]) for r in range(n)]).astype(np.float32).astype(np.float16)
    assert np.array_equal(wf, ref.astype(np.float32))
    d = O.gemm("q4_k", a, w, m, n, k)
    want = a.astype(np.float16).astype(np.float64) @ ref.astype(np.float64).T
    np.testing.assert_allclose(d, want, rtol=1e-12, atol=1e-12)
    # the accumulation scale of the GEMM tolerance: sum of |products|
    s_abs = O.gemm_abs("q4_k", a, w, m, n, k)
    want_abs = np.abs(a.astype(np.float16).astype(np.float64)) @ np.abs(ref.astype(np.float64)).T
    np.testing.assert_allclose(s_abs, want_abs, rtol=1e-12, atol=1e-12)
    assert (s_abs >= np.abs(d) - 1e-9).all()


# ---- CPU timing port ----------------------------------------------------------
# Its arithmetic is the reference's AVX2 path (src/cpu/kernels/gemm_q4k_q8.rs:
# 90-195), including two quirks of that port of llama.cpp: the min term keeps
# only SIMD lane 0 of acc_m (sub-blocks 0 and 1), and acc_m starts at dmin
# instead of 0.  The model below restates exactly that arithmetic in numpy.

def _ref_cpu_q4k_model(w, x, n, k):
    xb = x.reshape(-1, 256).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    dq = np.where(amax > 1e-7, amax / np.float32(127), np.float32(1)).astype(np.float32)
    v = xb / dq[:, None]
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127).astype(np.int64)   # f32::round
    y = np.zeros(n)
    for row in range(n):
        d, dmin, sc, m, nib = NP.q4k_fields(w[row])
        nb = nib.reshape(-1, 8, 32)
        qq = q.reshape(-1, 8, 32)
        dots = (nb * qq).sum(axis=2)
        bs = qq.sum(axis=2)
        main = dq * d * (sc * dots).sum(axis=1)
        dm = -dq * dmin
        minterm = dm * (m[:, 0] * bs[:, 0] + m[:, 1] * bs[:, 1]) + dm
        y[row] = (main + minterm).sum()
    return y


def test_cpu_port_restates_reference_arithmetic():
    k, n = 1024, 32
    w4 = synth.q4_k_weights(n, k, seed=61)
    w6 = synth.q6_k_weights(n, k, seed=62)
    x = synth.activations(k, seed=63)
    y4 = O.cpu_gemv_q4k(w4, x, n, k, 2)
    ref4 = _ref_cpu_q4k_model(w4, x, n, k)
    np.testing.assert_allclose(y4, ref4, rtol=1e-4, atol=1e-4 * np.abs(ref4).max())
    y6 = O.cpu_gemv_q6k(w6, x, n, k, 1)
    ref6 = O.gemv_q6k(w6, x, k, n)
    np.testing.assert_allclose(y6, ref6, rtol=1e-4, atol=1e-4 * np.abs(ref6).max())
