"""Pins of the oracle's layer operations (oracle/qk_oracle.c, or_rms_norm ..
or_argmax): the reference's own tests of these ops (src/cpu/ops_tests.rs),
closed forms, and brute force on small inputs -- each chosen so that a
plausible slip (a dropped eps, a wrong pair index, a missing scale, an
off-by-one causal mask, the wrong tie rule) fails one of them."""
import math

import numpy as np
import pytest

from oracle import oracle as O


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


# ---- RMSNorm -------------------------------------------------------------------

def test_rms_norm_reference_cases():
    # ops_tests.rs:12-23 and :25-41
    out = O.rms_norm([3.0, 4.0], [1.0, 1.0], 1e-6)
    r = math.sqrt(12.5 + 1e-6)
    assert abs(out[0] - 3 / r) < 1e-6 and abs(out[1] - 4 / r) < 1e-6
    out = O.rms_norm([3.0, 4.0, 6.0, 8.0], [1.0, 1.0], 1e-6, rows=2)
    assert abs(out[2] - 6 / math.sqrt(50 + 1e-6)) < 1e-6


def test_rms_norm_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096).astype(np.float32)
    one = np.ones(4096, np.float32)
    y = O.rms_norm(x, one, 0.0)
    assert abs(np.mean(y * y) - 1.0) < 1e-12                   # unit RMS without eps
    assert np.allclose(O.rms_norm(x * 8.0, one, 0.0), y, rtol=1e-12)   # scale invariance
    w = rng.standard_normal(4096).astype(np.float32)
    assert np.allclose(O.rms_norm(x, w, 0.0), y * w, rtol=1e-12)
    # eps enters inside the root: constant rows c give c / sqrt(c^2 + eps)
    c = np.full(128, 0.01, np.float32)
    assert np.allclose(O.rms_norm(c, np.ones(128, np.float32), 1e-4), 0.01 / math.sqrt(1e-4 + 1e-4), rtol=1e-6)


# ---- RoPE ---------------------------------------------------------------------------

def test_rope_position_zero_identity():
    # ops_tests.rs:55-77
    x = np.array([1.0, 2.0, 3.0, 4.0])
    for neox in (True, False):
        assert np.array_equal(O.rope(x, 1, 1, 4, 0, 10000.0, neox), x)


def test_rope_theta_values():
    # theta_0 = 1; theta_i = base^(-2i/d) within an ulp of float
    assert O.rope_theta(0, 128, 1e6) == 1.0
    for i in (1, 17, 63):
        t = 1e6 ** (-(2 * i) / 128)
        assert abs(O.rope_theta(i, 128, 1e6) - t) <= np.spacing(np.float32(t))
    assert O.rope_theta(5, 128, 1e4, np.full(64, 4.0, np.float32)) == np.float32(O.rope_theta(5, 128, 1e4)) / 4


def test_rope_exact_angles_and_norms():
    rng = np.random.default_rng(1)
    d, nh = 128, 3
    x = rng.standard_normal(nh * d)
    for neox in (True, False):
        for pos in (1, 7, 511):
            y = O.rope(x, 1, nh, d, pos, 1e6, neox)
            for h in range(nh):
                b = h * d
                for i in (0, 1, 40):
                    i0, i1 = (i, i + d // 2) if neox else (2 * i, 2 * i + 1)
                    a = float(np.float32(pos) * np.float32(O.rope_theta(i, d, 1e6)))
                    assert y[b + i0] == pytest.approx(x[b + i0] * math.cos(a) - x[b + i1] * math.sin(a), abs=1e-12)
                    assert y[b + i1] == pytest.approx(x[b + i0] * math.sin(a) + x[b + i1] * math.cos(a), abs=1e-12)
                    # pair norm preserved
                    assert math.hypot(y[b + i0], y[b + i1]) == pytest.approx(math.hypot(x[b + i0], x[b + i1]))


def test_rope_classic_is_interleaved_neox():
    # classic pairs (2i, 2i+1) = NeoX pairs (i, i + d/2) after interleaving the halves
    rng = np.random.default_rng(2)
    d = 64
    x = rng.standard_normal(d)
    perm = np.empty(d, int)
    perm[0::2], perm[1::2] = np.arange(d // 2), np.arange(d // 2) + d // 2
    assert np.allclose(O.rope(x[perm], 1, 1, d, 9, 1e4, False), O.rope(x, 1, 1, d, 9, 1e4, True)[perm], atol=1e-14)


def test_rope_rows_take_consecutive_positions():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 2 * 16))
    y = O.rope(x, 3, 2, 16, 5, 1e4, True).reshape(3, -1)
    for s in range(3):
        assert np.array_equal(y[s], O.rope(x[s], 1, 2, 16, 5 + s, 1e4, True))


# ---- decode attention --------------------------------------------------------------------

def test_attn_decode_reference_case():
    # ops_tests.rs:99-125: scores (1, 0), values 1 and 2 -> (e + 2) / (e + 1)
    out = O.attn_decode([1, 0, 0, 0], f16([1, 0, 0, 0, 0, 1, 0, 0]), f16([1] * 4 + [2] * 4), 2, 1, 1, 4, 1.0)
    assert np.allclose(out, (math.e + 2) / (math.e + 1), rtol=1e-12)


def test_attn_decode_closed_forms():
    rng = np.random.default_rng(4)
    seq, nh, nkv, d = 37, 4, 2, 16
    k = rng.standard_normal((seq, nkv * d))
    v = rng.standard_normal((seq, nkv * d))
    kc, vc = f16(k), f16(v)
    vf = vc.view(np.float16).astype(np.float64).reshape(seq, nkv, d)
    # q = 0: uniform weights -> mean of V for the head's KV group
    out = O.attn_decode(np.zeros(nh * d), kc, vc, seq, nh, nkv, d, 0.125).reshape(nh, d)
    for h in range(nh):
        assert np.allclose(out[h], vf[:, h // 2].mean(axis=0), rtol=1e-12)
    # one dominant score -> that position's V
    kd = np.zeros((seq, nkv * d), np.float32)
    kd[11, :] = 1.0
    q = np.full(nh * d, 40.0, np.float32)
    out = O.attn_decode(q, f16(kd), vc, seq, nh, nkv, d, 1.0).reshape(nh, d)
    assert np.allclose(out[3], vf[11, 1], rtol=1e-9)


def test_attn_decode_brute_force_softmax():
    rng = np.random.default_rng(5)
    seq, nh, nkv, d = 50, 8, 2, 32
    q = rng.standard_normal(nh * d).astype(np.float32)
    kc, vc = f16(rng.standard_normal((seq, nkv * d))), f16(rng.standard_normal((seq, nkv * d)))
    scale = float(np.float32(1 / math.sqrt(d)))          # the launchers take the scale as fp32
    out = O.attn_decode(q, kc, vc, seq, nh, nkv, d, scale).reshape(nh, d)
    kf = kc.view(np.float16).astype(np.float64).reshape(seq, nkv, d)
    vf = vc.view(np.float16).astype(np.float64).reshape(seq, nkv, d)
    for h in range(nh):
        s = kf[:, h // 4] @ q[h * d:(h + 1) * d].astype(np.float64) * scale
        p = np.exp(s - s.max())
        assert np.allclose(out[h], p @ vf[:, h // 4] / p.sum(), rtol=1e-10)


# ---- prefill attention (fp16 tile semantics) ----------------------------------------------------

def test_attn_prefill_brute_force_causal():
    # with fp16-exact inputs the tile-wise rounding of P is the only
    # difference from a direct causal softmax: relative 2^-11 at most
    rng = np.random.default_rng(6)
    seq, nh, nkv, d = 130, 4, 2, 16
    def h(a):
        return a.astype(np.float16).astype(np.float32)
    q, k, v = (h(rng.standard_normal((seq, n * d))) for n in (nh, nkv, nkv))
    out = O.attn_prefill_f16(q, k, v, seq, nh, nkv, d, 0.25).reshape(seq, nh, d)
    for hh in range(nh):
        kh = hh // 2
        for r in (0, 1, 63, 64, 65, 129):
            s = k[:r + 1, kh * d:(kh + 1) * d].astype(np.float64) @ q[r, hh * d:(hh + 1) * d] * 0.25
            p = np.exp(s - s.max())
            ref = p @ v[:r + 1, kh * d:(kh + 1) * d] / p.sum()
            assert np.allclose(out[r, hh], ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max()), (hh, r)
    # row 0 attends only to key 0
    assert np.allclose(out[0, 0], v[0, :d], rtol=1e-12)


def test_attn_prefill_rounds_like_fp16():
    # P is rounded to fp16: a score gap whose exp is not a half moves the output by its rounding
    q = np.zeros((2, 4), np.float32)
    k = np.zeros((2, 4), np.float32)
    v = np.array([[0, 0, 0, 0], [1, 1, 1, 1]], np.float32)
    k[0, 0], q[1, 0] = 1.0, 0.3     # row 1: scores 0.3 (key 0) and 0 (key 1)
    out = O.attn_prefill_f16(q, k, v, 2, 1, 1, 4, 1.0).reshape(2, 4)
    q16 = float(np.float16(0.3))
    e1 = float(np.float16(np.float32(math.exp(0 - q16))))       # P of key 1, rounded
    l = 1.0 + math.exp(-q16)                                     # l from the unrounded exps
    assert out[1, 0] == pytest.approx(e1 / l, rel=1e-12)


# ---- SwiGLU, argmax -------------------------------------------------------------------------

def test_silu_reference_values():
    # ops_tests.rs:43-53
    out = O.silu_mul([0.0, 1.0, -1.0], [1.0, 1.0, 1.0])
    assert abs(out[0]) < 1e-12 and abs(out[1] - 0.7310585786300049) < 1e-12
    assert abs(out[2] + 0.2689414213699951) < 1e-12


def test_argmax_reference_and_ties():
    # ops_tests.rs:90-97, then the device tie rule (larger index) and NaN
    assert O.argmax([1.0, 5.0, 3.0, 2.0]) == 1
    assert O.argmax([-1.0, -5.0, -3.0]) == 0
    assert O.argmax([2.0, 7.0, 7.0, 1.0, 7.0, 0.0]) == 4
    assert O.argmax([np.nan, 1.0, np.nan]) == 1
    rng = np.random.default_rng(7)
    x = rng.standard_normal(151936).astype(np.float32)
    assert O.argmax(x) == int(np.argmax(x))
