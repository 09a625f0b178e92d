"""GPU parity of the layer operations around the matmuls (model_ops.hip),
through the C ABI, against the oracle (oracle/qk_oracle.c or_rms_norm ..
or_argmax, pinned in tests/test_oracle_ops.py).

Bars: bit-exact for integer and conversion work (argmax index, fp16 V
copies, f32->f16, the decode-state counter); fp32 arithmetic against the
float64 oracle at REL = 1e-5 of the output's max magnitude (per element,
plus 1e-5 relative), the fp16 K cache within one fp16 ulp of the oracle's
rounded value (the fp32 rotation may sit either side of a rounding
boundary), and the Q4_K embedding at 2 fp32 ulps of the f64 dequant.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import gpu_util as G

pytestmark = pytest.mark.gpu

REL = 1e-5


def _close(y, ref, what, rel=REL):
    y = np.asarray(y, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    scale = np.abs(ref).max()
    err = np.abs(y - ref)
    bad = err > rel * scale + rel * np.abs(ref)
    print(f"{what}: max err {err.max() / scale:.3e} of max|ref|", flush=True)
    assert not bad.any(), f"{what}: {bad.sum()} elements off, worst {err.max() / scale:.3e}"


def _call0(fn, *args):
    """Launchers whose reference signature has no stream (null stream)."""
    print(f"[gpu] {fn.__name__}", flush=True)
    assert fn(*args) == 0
    torch.cuda.synchronize()


def _f16_ulps(got_bits, ref):
    got = got_bits.view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return np.abs(got - ref) / np.maximum(ulp, 2.0 ** -24)


@pytest.mark.parametrize("n,rows", [(4096, 1), (128, 40), (4096, 70), (12288, 3), (100, 9), (1000, 2)])
def test_rms_norm(rf, dev, n, rows):
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal(n * rows) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    dx, dw = G.to_dev(x), G.to_dev(w)
    out = G.empty(n * rows, torch.float32)
    if rows == 1:
        G.call(rf.gpu_rms_norm, G.ptr(dx), G.ptr(dw), G.ptr(out), n, 1e-6)
    else:
        G.call(rf.gpu_rms_norm_batched_on_stream, G.ptr(dx), G.ptr(dw), G.ptr(out), n, 1e-6, rows)
    _close(G.host(out), O.rms_norm(x, w, 1e-6, rows), f"rms_norm {n}x{rows}")
    # in place (the per-head Q/K norms write back into q / k)
    _call0(rf.gpu_rms_norm_batched, G.ptr(dx), G.ptr(dw), G.ptr(dx), n, 1e-6, rows)
    np.testing.assert_array_equal(G.host(dx), G.host(out))


@pytest.mark.parametrize("neox", [1, 0])
@pytest.mark.parametrize("pos", [0, 7, 639, 40000])
def test_rope_heads(rf, dev, neox, pos):
    nh, d = 32, 128
    rng = np.random.default_rng(pos + neox)
    x = rng.standard_normal(nh * d).astype(np.float32)
    ref = O.rope(x, 1, nh, d, pos, 1e6, bool(neox))
    dx = G.to_dev(x)
    G.call(rf.gpu_rope_heads, G.ptr(dx), pos, nh, d, 1e6, neox)
    _close(G.host(dx), ref, f"rope pos {pos} neox {neox}")
    # state variant reads the position from device memory; freq_scale divides theta
    fs = (1.0 + rng.random(d // 2)).astype(np.float32)
    dx, dpos, dfs = G.to_dev(x), G.to_dev(np.array([pos, pos + 1], np.int32)), G.to_dev(fs)
    G.call(rf.gpu_rope_heads_state_scaled, G.ptr(dx), G.ptr(dpos), nh, d, 1e6, neox, G.ptr(dfs))
    _close(G.host(dx), O.rope(x, 1, nh, d, pos, 1e6, bool(neox), fs), f"rope state scaled pos {pos}")


def test_rope_heads_batched(rf, dev):
    seq, nh, d = 33, 8, 128
    x = np.random.default_rng(9).standard_normal(seq * nh * d).astype(np.float32)
    dx = G.to_dev(x)
    _call0(rf.gpu_rope_heads_batched, G.ptr(dx), 5, nh, d, 1e4, seq, 1)
    _close(G.host(dx), O.rope(x, seq, nh, d, 5, 1e4, True), "rope batched")
    dx = G.to_dev(x)
    G.call(rf.rf_rope_heads_batched_on_stream, G.ptr(dx), 5, nh, d, 1e4, seq, 0, None)
    _close(G.host(dx), O.rope(x, seq, nh, d, 5, 1e4, False), "rope batched on stream, classic")


@pytest.mark.parametrize("state", [False, True])
def test_kv_write_rope(rf, dev, state):
    nkv, d, max_seq, pos = 8, 128, 64, 37
    rng = np.random.default_rng(11)
    k = rng.standard_normal(nkv * d).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    kc = G.to_dev(np.full(max_seq * nkv * d, 0x7E00, np.uint16))    # NaN fill: untouched rows stay NaN
    vc = G.to_dev(np.full(max_seq * nkv * d, 0x7E00, np.uint16))
    dk, dv = G.to_dev(k), G.to_dev(v)
    if state:
        dpos = G.to_dev(np.array([pos, pos + 1], np.int32))
        G.call(rf.gpu_kv_write_rope_state, G.ptr(kc), G.ptr(vc), G.ptr(dk), G.ptr(dv), G.ptr(dpos), nkv, d, 1e6, 1)
    else:
        G.call(rf.gpu_kv_write_rope, G.ptr(kc), G.ptr(vc), G.ptr(dk), G.ptr(dv), pos, nkv, d, 1e6, 1)
    kc, vc = G.host(kc).reshape(max_seq, -1), G.host(vc).reshape(max_seq, -1)
    np.testing.assert_array_equal(vc[pos], v.astype(np.float16).view(np.uint16))
    assert (_f16_ulps(kc[pos], O.rope(k, 1, nkv, d, pos, 1e6, True)) <= 1.0).all()
    others = np.delete(np.arange(max_seq), pos)
    assert (kc[others] == 0x7E00).all() and (vc[others] == 0x7E00).all()


def test_kv_write_batched(rf, dev):
    kv, max_seq, start, seq = 1024, 80, 9, 40
    rng = np.random.default_rng(12)
    k = rng.standard_normal(seq * kv).astype(np.float32)
    v = rng.standard_normal(seq * kv).astype(np.float32)
    kc, vc = G.empty(max_seq * kv, torch.int16), G.empty(max_seq * kv, torch.int16)
    dk, dv = G.to_dev(k), G.to_dev(v)           # held: a temporary's block would be reused by the next copy
    _call0(rf.gpu_kv_write_batched, G.ptr(kc), G.ptr(vc), G.ptr(dk), G.ptr(dv), start, kv, max_seq, seq)
    kc, vc = G.host(kc).view(np.uint16).reshape(max_seq, kv), G.host(vc).view(np.uint16).reshape(max_seq, kv)
    np.testing.assert_array_equal(kc[start:start + seq], k.astype(np.float16).view(np.uint16).reshape(seq, kv))
    np.testing.assert_array_equal(vc[start:start + seq], v.astype(np.float16).view(np.uint16).reshape(seq, kv))
    # beyond the cache: rejected before any launch
    import ctypes
    p = ctypes.c_void_p(0x100000)               # never dereferenced: the range check rejects first
    assert rf.gpu_kv_write_batched(p, p, p, p, 50, kv, max_seq, seq) != 0


@pytest.mark.parametrize("with_norm", [True, False])
@pytest.mark.parametrize("neox", [1, 0])
@pytest.mark.parametrize("table", [False, True])
def test_fused_qk_norm_rope_kv(rf, dev, with_norm, neox, table):
    # the one-launch Qwen3 step against the oracle, and against the separate launchers
    nh, nkv, d, max_seq, pos = 32, 8, 128, 700, 641
    rng = np.random.default_rng(13 + neox)
    q = (rng.standard_normal(nh * d) * 4).astype(np.float32)
    k = (rng.standard_normal(nkv * d) * 4).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    dq, dk, dv, dqn, dkn = (G.to_dev(a) for a in (q, k, v, qn, kn))
    kc, vc = G.empty(max_seq * nkv * d, torch.int16), G.empty(max_seq * nkv * d, torch.int16)
    dpos = G.to_dev(np.array([pos, pos + 1], np.int32))
    theta = None
    if table:
        theta = G.empty(d // 2, torch.float32)
        G.call(rf.rf_rope_theta_table, G.ptr(theta), d, 1e6)
        want = np.array([O.rope_theta(i, d, 1e6) for i in range(d // 2)], np.float32)
        np.testing.assert_array_equal(G.host(theta), want)
    G.call(rf.rf_qk_norm_rope_kv_write_state, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn) if with_norm else None,
           G.ptr(dkn) if with_norm else None, G.ptr(kc), G.ptr(vc), G.ptr(dpos), nh, nkv, d, 1e-6, 1e6, neox, None,
           G.ptr(theta) if table else None, None)
    qr = O.rms_norm(q, qn, 1e-6, nh) if with_norm else q.astype(np.float64)
    kr = O.rms_norm(k, kn, 1e-6, nkv) if with_norm else k.astype(np.float64)
    _close(G.host(dq), O.rope(qr, 1, nh, d, pos, 1e6, bool(neox)), "fused q")
    kc_h = G.host(kc).view(np.uint16).reshape(max_seq, -1)
    vc_h = G.host(vc).view(np.uint16).reshape(max_seq, -1)
    assert (_f16_ulps(kc_h[pos], O.rope(kr, 1, nkv, d, pos, 1e6, bool(neox))) <= 1.0).all()
    np.testing.assert_array_equal(vc_h[pos], v.astype(np.float16).view(np.uint16))
    # same results as norm + rope + kv_write launched separately
    dq2, dk2 = G.to_dev(q), G.to_dev(k)
    kc2, vc2 = G.empty(max_seq * nkv * d, torch.int16), G.empty(max_seq * nkv * d, torch.int16)
    if with_norm:
        G.call(rf.gpu_rms_norm_batched_on_stream, G.ptr(dq2), G.ptr(dqn), G.ptr(dq2), d, 1e-6, nh)
        G.call(rf.gpu_rms_norm_batched_on_stream, G.ptr(dk2), G.ptr(dkn), G.ptr(dk2), d, 1e-6, nkv)
    G.call(rf.gpu_rope_heads_state, G.ptr(dq2), G.ptr(dpos), nh, d, 1e6, neox)
    G.call(rf.gpu_kv_write_rope_state, G.ptr(kc2), G.ptr(vc2), G.ptr(dk2), G.ptr(dv), G.ptr(dpos), nkv, d, 1e6, neox)
    a, b = G.host(dq), G.host(dq2)
    if not with_norm:       # the same rotation, so the same bits
        np.testing.assert_array_equal(a, b)
    assert np.abs(a - b).max() <= 4 * np.spacing(np.abs(b).max())
    kc2_h = G.host(kc2).view(np.uint16).reshape(max_seq, -1)
    assert (np.abs(kc_h[pos].view(np.float16).astype(np.float64) - kc2_h[pos].view(np.float16).astype(np.float64))
            <= np.spacing(np.abs(kc2_h[pos].view(np.float16))).astype(np.float64)).all()


@pytest.mark.parametrize("seq,nh,nkv,d", [(1, 32, 8, 128), (2, 32, 8, 128), (100, 32, 8, 128), (640, 32, 8, 128),
                                          (5000, 32, 8, 128), (300, 16, 16, 64), (257, 8, 2, 256)])
def test_attn_decode(rf, dev, seq, nh, nkv, d):
    rng = np.random.default_rng(seq + d)
    max_seq = seq + 3
    q = rng.standard_normal(nh * d).astype(np.float32)
    kc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.uint16)
    scale = 1.0 / math.sqrt(d)
    ref = O.attn_decode(q, kc, vc, seq, nh, nkv, d, scale)
    dq, dkc, dvc = G.to_dev(q), G.to_dev(kc.view(np.int16)), G.to_dev(vc.view(np.int16))
    out = G.empty(nh * d, torch.float32)
    G.call(rf.gpu_flash_attn_decode_strided_multi_head, G.ptr(out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), seq, nh, nkv,
           d, scale)
    _close(G.host(out), ref, f"attn decode seq {seq} d {d}")
    out2 = G.empty(nh * d, torch.float32)
    dlen = G.to_dev(np.array([seq], np.int32))
    G.call(rf.gpu_flash_attn_decode_strided_multi_head_state, G.ptr(out2), G.ptr(dq), G.ptr(dkc), G.ptr(dvc),
           G.ptr(dlen), nh, nkv, d, scale)
    np.testing.assert_array_equal(G.host(out2), G.host(out))
    # the split path in a caller workspace (positions over many workgroups)
    wsb = int(rf.rf_flash_attn_decode_workspace_bytes(nh, d))
    assert wsb == nh * 64 * (d + 4) * 4
    # NaN-filled: splits without positions must not read their stale slots
    ws = torch.full((wsb // 4,), float("nan"), dtype=torch.float32, device="cuda:0")
    out3, out4 = G.empty(nh * d, torch.float32), G.empty(nh * d, torch.float32)
    G.call(rf.rf_flash_attn_decode_ws, G.ptr(out3), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), seq, nh, nkv, d, scale,
           G.ptr(ws), wsb)
    _close(G.host(out3), ref, f"split attn decode seq {seq} d {d}")
    G.call(rf.rf_flash_attn_decode_state_ws, G.ptr(out4), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh, nkv, d,
           scale, G.ptr(ws), wsb)
    np.testing.assert_array_equal(G.host(out4), G.host(out3))
    # a workspace below the size the query gives is rejected, and so is none
    assert rf.rf_flash_attn_decode_ws(G.ptr(out3), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), seq, nh, nkv, d, scale,
                                      G.ptr(ws), wsb - 4, G.stream()) != 0
    assert rf.rf_flash_attn_decode_ws(G.ptr(out3), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), seq, nh, nkv, d, scale,
                                      None, wsb, G.stream()) != 0


@pytest.mark.parametrize("seq,nh,nkv,d", [(1, 32, 8, 128), (3, 32, 8, 128), (64, 32, 8, 128), (65, 32, 8, 128),
                                          (640, 32, 8, 128), (2048, 32, 8, 128), (300, 16, 16, 64),
                                          (257, 8, 2, 256), (100, 32, 2, 128)])
def test_attn_decode_bounded(rf, dev, seq, nh, nkv, d):
    # one workgroup per query head (max_seq <= 2048; GQA groups of any size,
    # here up to 16): the oracle's attention within 1e-5, no workspace needed;
    # past 2048 the split path with its workspace, the same bits as
    # rf_flash_attn_decode_state_ws
    rng = np.random.default_rng(seq + 3 * d + nkv)
    max_seq = seq + 3
    q = rng.standard_normal(nh * d).astype(np.float32)
    kc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.uint16)
    scale = 1.0 / math.sqrt(d)
    ref = O.attn_decode(q, kc, vc, seq, nh, nkv, d, scale)
    dq, dkc, dvc = G.to_dev(q), G.to_dev(kc.view(np.int16)), G.to_dev(vc.view(np.int16))
    dlen = G.to_dev(np.array([seq], np.int32))
    bound = min(max_seq, 2048)
    out = G.empty(nh * d, torch.float32).fill_(float("nan"))
    G.call(rf.rf_flash_attn_decode_state_bounded, G.ptr(out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh, nkv,
           d, scale, bound, None, 0)
    _close(G.host(out), ref, f"head-path attn decode seq {seq} d {d} group {nh // nkv}")
    again = G.empty(nh * d, torch.float32)
    G.call(rf.rf_flash_attn_decode_state_bounded, G.ptr(again), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh,
           nkv, d, scale, bound, None, 0)
    np.testing.assert_array_equal(G.host(again), G.host(out))
    if nh // nkv <= 8:
        wsb = int(rf.rf_flash_attn_decode_workspace_bytes(nh, d))
        ws = G.empty(wsb // 4, torch.float32)
        o_split, o_big = G.empty(nh * d, torch.float32), G.empty(nh * d, torch.float32)
        G.call(rf.rf_flash_attn_decode_state_ws, G.ptr(o_split), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh,
               nkv, d, scale, G.ptr(ws), wsb)
        G.call(rf.rf_flash_attn_decode_state_bounded, G.ptr(o_big), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen),
               nh, nkv, d, scale, 4096, G.ptr(ws), wsb)
        np.testing.assert_array_equal(G.host(o_big), G.host(o_split))
    s = G.stream()
    assert rf.rf_flash_attn_decode_state_bounded(G.ptr(out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh, nkv,
                                                 d, scale, 0, None, 0, s) != 0           # no bound
    assert rf.rf_flash_attn_decode_state_bounded(G.ptr(out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh, nkv,
                                                 d, scale, 4096, None, 0, s) != 0        # split path needs a workspace


@pytest.mark.parametrize("n", [1, 1000, 1024, 1025, 151936])
def test_argmax(rf, dev, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    cases = [x]
    if n > 10:
        t = x.copy()
        t[[3, n // 2, n - 2]] = 50.0           # ties: the larger index
        c = x.copy()
        c[5] = np.nan
        c[7] = np.inf
        cases += [t, c, np.full(n, -np.inf, np.float32)]
    np_ = (n + 1023) // 1024
    for c in cases:
        dx = G.to_dev(c)
        pv, pi, out = G.empty(np_, torch.float32), G.empty(np_, torch.int32), G.empty(1, torch.int32)
        G.call(rf.gpu_argmax_f32_on_stream, G.ptr(dx), G.ptr(pv), G.ptr(pi), G.ptr(out), n)
        assert int(G.host(out)[0]) == O.argmax(c)


def test_embed_q4_k(rf, dev):
    from rocmforge_amd import synth
    hidden, vocab = 4096, 300
    emb = synth.q4_k_weights(vocab, hidden, seed=21)
    de = G.to_dev(emb)
    out = G.empty(hidden, torch.float32)
    G.call(rf.gpu_embed_q4_k_token, G.ptr(de), G.ptr(out), hidden, vocab, 123)
    ref = O.q4k_dequant(emb[123], hidden // 256)
    np.testing.assert_allclose(G.host(out), ref, rtol=2.5e-7, atol=1e-12)
    ids = np.array([0, 299, 5, -1, 300, 123], np.int32)
    outb = G.to_dev(np.full(len(ids) * hidden, 7.0, np.float32))
    dids = G.to_dev(ids)
    G.call(rf.gpu_embed_q4_k_batch, G.ptr(de), G.ptr(dids), G.ptr(outb), hidden, vocab, len(ids))
    ob = G.host(outb).reshape(len(ids), hidden)
    for s, t in enumerate(ids):
        if 0 <= t < vocab:
            np.testing.assert_allclose(ob[s], O.q4k_dequant(emb[t], hidden // 256), rtol=2.5e-7, atol=1e-12)
        else:
            assert (ob[s] == 7.0).all()       # out-of-range ids leave the row untouched
    assert rf.gpu_embed_q4_k_token(G.ptr(de), G.ptr(out), hidden, vocab, vocab, None) != 0


def test_elementwise(rf, dev):
    n = 12288 + 5
    rng = np.random.default_rng(31)
    a = (rng.standard_normal(n) * 4).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    da, db, out = G.to_dev(a), G.to_dev(b), G.empty(n, torch.float32)
    G.call(rf.gpu_add, G.ptr(da), G.ptr(db), G.ptr(out), n)
    np.testing.assert_array_equal(G.host(out), a + b)
    G.call(rf.gpu_mul_on_stream, G.ptr(da), G.ptr(db), G.ptr(out), n)
    np.testing.assert_array_equal(G.host(out), a * b)
    G.call(rf.gpu_silu_on_stream, G.ptr(da), G.ptr(out), n)
    _close(G.host(out), O.silu_mul(a, np.ones(n, np.float32)), "silu")
    G.call(rf.rf_silu_mul_on_stream, G.ptr(da), G.ptr(db), G.ptr(out), n)
    _close(G.host(out), O.silu_mul(a, b), "silu_mul")
    h = G.empty(n, torch.int16)
    G.call(rf.convert_f32_to_f16, G.ptr(da), G.ptr(h), n)
    np.testing.assert_array_equal(G.host(h).view(np.uint16), a.astype(np.float16).view(np.uint16))
    st = G.to_dev(np.array([4, 5], np.int32))
    G.call(rf.gpu_increment_decode_state_on_stream, G.ptr(st))
    assert list(G.host(st)) == [5, 6]


# fp16 operands: P rounded per tile may land on the other side of an fp16
# rounding boundary than the oracle's; the GEMM bar applies
PREFILL_REL = 2e-3


@pytest.mark.parametrize("seq,nq,nkv,causal", [(64, 2, 1, 1), (128, 4, 2, 1), (512, 32, 8, 1), (192, 4, 4, 0),
                                               (320, 8, 2, 1)])
def test_attn_prefill(rf, dev, seq, nq, nkv, causal):
    rng = np.random.default_rng(seq + nq)
    d = 128
    q = rng.standard_normal(seq * nq * d).astype(np.float32)
    k = rng.standard_normal(seq * nkv * d).astype(np.float32)
    v = rng.standard_normal(seq * nkv * d).astype(np.float32)
    scale = 1.0 / math.sqrt(d)
    dq, dk, dv = (G.to_dev(a.astype(np.float16).view(np.int16)) for a in (q, k, v))
    out = G.empty(seq * nq * d, torch.float32)
    G.call(rf.wmma_attention_prefill_gqa_causal_launch, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(out), seq, nq, nkv,
           causal, scale)
    got = G.host(out).reshape(seq, nq, d)
    if causal:
        ref = O.attn_prefill_f16(q, k, v, seq, nq, nkv, d, scale).reshape(seq, nq, d)
    else:
        # full attention of query r = the causal oracle's last row with q[r] there
        rows = [0, 63, 64, seq - 1]
        got = got[rows]
        ref = np.empty((len(rows), nq, d))
        for i, r in enumerate(rows):
            qq = np.tile(q.reshape(seq, -1)[r], (seq, 1))
            ref[i] = O.attn_prefill_f16(qq, k, v, seq, nq, nkv, d, scale).reshape(seq, nq, d)[-1]
    err = np.abs(got - ref)
    print(f"prefill attention seq {seq}: max err {err.max() / np.abs(ref).max():.3e}", flush=True)
    assert (err <= PREFILL_REL * np.abs(ref).max() + PREFILL_REL * np.abs(ref)).all()


@pytest.mark.parametrize("seq,nh,nkv,d", [(1, 32, 8, 128), (641, 32, 8, 128), (100, 8, 8, 64), (70, 8, 2, 256)])
def test_attention_with_folded_qk_step(rf, dev, seq, nh, nkv, d):
    # one launch = the standalone Q/K step + attention, bit for bit (caches too)
    rng = np.random.default_rng(seq + nh)
    max_seq = seq + 5
    q = (rng.standard_normal(nh * d) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * d) * 3).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    qn, kn = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    cache = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.int16)
    dq, dk, dv, dqn, dkn = (G.to_dev(a) for a in (q, k, v, qn, kn))
    st = G.to_dev(np.array([seq - 1, seq], np.int32))
    kc1, vc1, kc2, vc2 = (G.to_dev(cache) for _ in range(4))
    out1, out2 = G.empty(nh * d, torch.float32), G.empty(nh * d, torch.float32)
    scale = 1.0 / math.sqrt(d)
    wsb = int(rf.rf_flash_attn_decode_workspace_bytes(nh, d))
    ws = G.empty(wsb // 4, torch.float32)
    G.call(rf.rf_attn_decode_qk_norm_rope_state, G.ptr(out1), G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn), G.ptr(dkn),
           G.ptr(kc1), G.ptr(vc1), G.ptr(st), nh, nkv, d, 1e-6, 1e6, 1, None, None, None, scale, G.ptr(ws), wsb)
    np.testing.assert_array_equal(G.host(dq), q)        # the raw q is left as it was
    G.call(rf.rf_qk_norm_rope_kv_write_state, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn), G.ptr(dkn), G.ptr(kc2),
           G.ptr(vc2), G.ptr(st), nh, nkv, d, 1e-6, 1e6, 1, None, None, None)
    dlen = G.to_dev(np.array([seq], np.int32))
    G.call(rf.rf_flash_attn_decode_state_ws, G.ptr(out2), G.ptr(dq), G.ptr(kc2), G.ptr(vc2), G.ptr(dlen), nh, nkv, d,
           scale, G.ptr(ws), wsb)
    np.testing.assert_array_equal(G.host(out1), G.host(out2))
    np.testing.assert_array_equal(G.host(kc1), G.host(kc2))
    np.testing.assert_array_equal(G.host(vc1), G.host(vc2))
    # and against the oracle: normalised, rotated q over the updated caches
    qr = O.rope(O.rms_norm(q, qn, 1e-6, nh), 1, nh, d, seq - 1, 1e6, True)
    ref = O.attn_decode(qr.astype(np.float32), G.host(kc1).view(np.uint16), G.host(vc1).view(np.uint16), seq, nh,
                        nkv, d, scale)
    _close(G.host(out1), ref, f"attention with qk step seq {seq}")


@pytest.mark.parametrize("seq,nh,nkv,d", [(1, 32, 8, 128), (2, 32, 8, 128), (641, 32, 8, 128), (100, 8, 8, 64),
                                          (70, 8, 2, 256), (200, 32, 2, 128)])
def test_attention_with_folded_qk_step_bounded(rf, dev, seq, nh, nkv, d):
    # the bounded launch (one workgroup per query head) = the standalone Q/K
    # step + the bounded attention, bit for bit (caches too: the new K/V row
    # written once, by the workgroup of the group's first query head, and read
    # by every head from registers), and the oracle within 1e-5
    rng = np.random.default_rng(seq + nh + 1)
    max_seq = seq + 5
    q = (rng.standard_normal(nh * d) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * d) * 3).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    qn, kn = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    cache = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.int16)
    dq, dk, dv, dqn, dkn = (G.to_dev(a) for a in (q, k, v, qn, kn))
    st = G.to_dev(np.array([seq - 1, seq], np.int32))
    kc1, vc1, kc2, vc2 = (G.to_dev(cache) for _ in range(4))
    out1, out2 = G.empty(nh * d, torch.float32), G.empty(nh * d, torch.float32)
    scale = 1.0 / math.sqrt(d)
    G.call(rf.rf_attn_decode_qk_norm_rope_state_bounded, G.ptr(out1), G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn),
           G.ptr(dkn), G.ptr(kc1), G.ptr(vc1), G.ptr(st), nh, nkv, d, 1e-6, 1e6, 1, None, None, None, scale, max_seq,
           None, 0)
    np.testing.assert_array_equal(G.host(dq), q)        # the raw q is left as it was
    G.call(rf.rf_qk_norm_rope_kv_write_state, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn), G.ptr(dkn), G.ptr(kc2),
           G.ptr(vc2), G.ptr(st), nh, nkv, d, 1e-6, 1e6, 1, None, None, None)
    dlen = G.to_dev(np.array([seq], np.int32))
    G.call(rf.rf_flash_attn_decode_state_bounded, G.ptr(out2), G.ptr(dq), G.ptr(kc2), G.ptr(vc2), G.ptr(dlen), nh,
           nkv, d, scale, max_seq, None, 0)
    np.testing.assert_array_equal(G.host(out1), G.host(out2))
    np.testing.assert_array_equal(G.host(kc1), G.host(kc2))
    np.testing.assert_array_equal(G.host(vc1), G.host(vc2))
    qr = O.rope(O.rms_norm(q, qn, 1e-6, nh), 1, nh, d, seq - 1, 1e6, True)
    ref = O.attn_decode(qr.astype(np.float32), G.host(kc1).view(np.uint16), G.host(vc1).view(np.uint16), seq, nh,
                        nkv, d, scale)
    _close(G.host(out1), ref, f"bounded attention with qk step seq {seq}")


@pytest.mark.parametrize("scaled", [False, True])
def test_rope_cos_sin_table_follows_theta_table(rf, dev, scaled):
    # a caller's theta table that is not the standard one (a scaled RoPE
    # expressed through d_theta): the cos / sin table built from it rotates
    # like the trig path given the same d_theta, bit for bit
    nh, nkv, d, max_seq, base, pos = 8, 2, 128, 64, 1e6, 61
    rng = np.random.default_rng(7)
    std = G.empty(d // 2, torch.float32)
    G.call(rf.rf_rope_theta_table, G.ptr(std), d, base)
    theta = G.to_dev((G.host(std) * (1 + 0.05 * rng.random(d // 2))).astype(np.float32))
    fs = G.to_dev((1 + rng.random(d // 2)).astype(np.float32)) if scaled else None
    fsp = G.ptr(fs) if scaled else None
    cs = G.empty(max_seq * d, torch.float32)
    G.call(rf.rf_rope_cos_sin_table, G.ptr(cs), max_seq, d, base, G.ptr(theta), fsp)
    th = G.host(theta) / (G.host(fs) if scaled else 1.0)
    ang = (np.float32(pos) * th.astype(np.float32)).astype(np.float64)
    row = G.host(cs).reshape(max_seq, d // 2, 2)[pos]
    assert np.abs(row[:, 0] - np.cos(ang)).max() <= 4e-7
    qn, kn = G.to_dev(np.ones(d, np.float32)), G.to_dev(np.ones(d, np.float32))
    q = (rng.standard_normal(nh * d) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * d) * 3).astype(np.float32)
    dk, dv = G.to_dev(k), G.to_dev(k)
    st = G.to_dev(np.array([pos, pos + 1], np.int32))
    outs = []
    for table in (None, G.ptr(cs)):
        dq = G.to_dev(q)
        kc, vc = G.empty(max_seq * nkv * d, torch.int16).zero_(), G.empty(max_seq * nkv * d, torch.int16).zero_()
        G.call(rf.rf_qk_norm_rope_kv_write_state, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(qn), G.ptr(kn), G.ptr(kc),
               G.ptr(vc), G.ptr(st), nh, nkv, d, 1e-6, base, 1, fsp, G.ptr(theta), table)
        outs.append((G.host(dq), G.host(kc)))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("d,neox,scaled", [(128, 1, False), (128, 0, False), (64, 1, True), (256, 0, True),
                                           (256, 1, False)])
def test_rope_cos_sin_table_same_bits(rf, dev, d, neox, scaled):
    # the cos / sin table replaces cosf / sinf in the three fused Q/K launchers:
    # same values, so the outputs and caches must match the trig path bit for bit
    nh, nkv, max_seq, base = 16, 4, 300, 1e6
    rng = np.random.default_rng(d + neox)
    fs = G.to_dev((1 + rng.random(d // 2)).astype(np.float32)) if scaled else None
    theta = G.empty(d // 2, torch.float32)
    G.call(rf.rf_rope_theta_table, G.ptr(theta), d, base)
    cs = G.empty(max_seq * d, torch.float32)
    G.call(rf.rf_rope_cos_sin_table, G.ptr(cs), max_seq, d, base, G.ptr(theta), G.ptr(fs) if scaled else None)
    # the table against double-precision cos / sin of the same float angle
    th = G.host(theta).astype(np.float32)
    if scaled:
        th = (th / G.host(fs)).astype(np.float32)
    ang = (np.arange(max_seq, dtype=np.float32)[:, None] * th[None, :]).astype(np.float64)
    tab = G.host(cs).reshape(max_seq, d // 2, 2)
    assert np.abs(tab[..., 0] - np.cos(ang)).max() <= 4e-7
    assert np.abs(tab[..., 1] - np.sin(ang)).max() <= 4e-7
    fsp = G.ptr(fs) if scaled else None
    qn, kn = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    dqn, dkn = G.to_dev(qn), G.to_dev(kn)
    # decode step at a late position
    pos = max_seq - 3
    q = (rng.standard_normal(nh * d) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * d) * 3).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    dk, dv = G.to_dev(k), G.to_dev(v)
    st = G.to_dev(np.array([pos, pos + 1], np.int32))
    outs = []
    for table in (None, G.ptr(cs)):
        dq = G.to_dev(q)
        kc, vc = G.empty(max_seq * nkv * d, torch.int16).zero_(), G.empty(max_seq * nkv * d, torch.int16).zero_()
        G.call(rf.rf_qk_norm_rope_kv_write_state, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn), G.ptr(dkn), G.ptr(kc),
               G.ptr(vc), G.ptr(st), nh, nkv, d, 1e-6, base, neox, fsp, G.ptr(theta), table)
        outs.append((G.host(dq), G.host(kc)))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    # the step folded into the attention
    wsb = int(rf.rf_flash_attn_decode_workspace_bytes(nh, d))
    ws = G.empty(wsb // 4, torch.float32)
    cache = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.int16)
    outs = []
    for table in (None, G.ptr(cs)):
        dq = G.to_dev(q)
        kc, vc = G.to_dev(cache), G.to_dev(cache)
        out = G.empty(nh * d, torch.float32)
        G.call(rf.rf_attn_decode_qk_norm_rope_state, G.ptr(out), G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn),
               G.ptr(dkn), G.ptr(kc), G.ptr(vc), G.ptr(st), nh, nkv, d, 1e-6, base, neox, fsp, G.ptr(theta), table,
               1.0 / math.sqrt(d), G.ptr(ws), wsb)
        outs.append((G.host(out), G.host(kc)))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    # the prompt rows: 37 query rows from position 200, 30 of them with K/V rows
    start, rq, rkv = 200, 37, 30
    qr = (rng.standard_normal(rq * nh * d) * 3).astype(np.float32)
    kr = (rng.standard_normal(rq * nkv * d) * 3).astype(np.float32)
    vr = rng.standard_normal(rq * nkv * d).astype(np.float32)
    dq, dk, dv = G.to_dev(qr), G.to_dev(kr), G.to_dev(vr)
    outs = []
    for table in (None, G.ptr(cs)):
        q16 = G.empty(rq * nh * d, torch.int16)
        kc, vc = G.empty(max_seq * nkv * d, torch.int16).zero_(), G.empty(max_seq * nkv * d, torch.int16).zero_()
        G.call(rf.rf_qk_norm_rope_kv_write_rows, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(dqn), G.ptr(dkn), G.ptr(q16),
               G.ptr(kc), G.ptr(vc), start, rq, rkv, nh, nkv, d, max_seq, 1e-6, base, neox, fsp, G.ptr(theta), table)
        outs.append((G.host(q16), G.host(kc), G.host(vc)))
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    # the table covers max_seq positions: query rows past it are rejected
    s0 = G.stream()
    assert rf.rf_qk_norm_rope_kv_write_rows(G.ptr(dq), G.ptr(dk), G.ptr(dv), None, None, G.ptr(q16), G.ptr(kc),
                                            G.ptr(vc), max_seq - 10, 20, 5, nh, nkv, d, max_seq, 1e-6, base, neox,
                                            fsp, None, G.ptr(cs), s0) != 0
    assert rf.rf_qk_norm_rope_kv_write_rows(G.ptr(dq), G.ptr(dk), G.ptr(dv), None, None, G.ptr(q16), G.ptr(kc),
                                            G.ptr(vc), max_seq - 10, 20, 5, nh, nkv, d, max_seq, 1e-6, base, neox,
                                            fsp, None, None, s0) == 0
    torch.cuda.synchronize()


def test_argmax_advances_state(rf, dev):
    x = np.random.default_rng(3).standard_normal(151936).astype(np.float32)
    n = x.size
    dx = G.to_dev(x)
    pv, pi, out = G.empty(149, torch.float32), G.empty(149, torch.int32), G.empty(1, torch.int32)
    st = G.to_dev(np.array([9, 10], np.int32))
    G.call(rf.rf_argmax_f32_advance_state_on_stream, G.ptr(dx), G.ptr(pv), G.ptr(pi), G.ptr(out), n, G.ptr(st))
    assert int(G.host(out)[0]) == O.argmax(x) and list(G.host(st)) == [10, 11]


def test_attn_prefill_first_token_is_its_value(rf, dev):
    # tests/wmma_attention_gqa_causal_correctness.rs:270-305 of the reference: row 0 attends to
    # key 0 only, so its output is V[0] exactly (P = 1, l = 1) for every head
    seq, nq, nkv, d = 128, 8, 2, 128
    rng = np.random.default_rng(77)
    q, k, v = (rng.standard_normal(seq * n * d).astype(np.float16) for n in (nq, nkv, nkv))
    dq, dk, dv = (G.to_dev(a.view(np.int16)) for a in (q, k, v))
    out = G.empty(seq * nq * d, torch.float32)
    G.call(rf.wmma_attention_prefill_gqa_causal_launch, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(out), seq, nq, nkv, 1,
           1.0 / math.sqrt(d))
    row0 = G.host(out).reshape(seq, nq, d)[0]
    v0 = v.reshape(seq, nkv, d)[0].astype(np.float32)
    for h in range(nq):
        np.testing.assert_array_equal(row0[h], v0[h // (nq // nkv)])


def test_attn_prefill_gqa_full_seq256(rf, dev):
    # the reference's gqa_only cases (non-causal), at its largest length
    seq, nq, nkv, d = 256, 8, 2, 128
    rng = np.random.default_rng(78)
    q, k, v = (rng.standard_normal(seq * n * d).astype(np.float32) for n in (nq, nkv, nkv))
    dq, dk, dv = (G.to_dev(a.astype(np.float16).view(np.int16)) for a in (q, k, v))
    out = G.empty(seq * nq * d, torch.float32)
    scale = 1.0 / math.sqrt(d)
    G.call(rf.wmma_attention_prefill_gqa_causal_launch, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(out), seq, nq, nkv, 0,
           scale)
    got = G.host(out).reshape(seq, nq, d)
    for r in (0, 100, 255):
        qq = np.tile(q.reshape(seq, -1)[r], (seq, 1))
        ref = O.attn_prefill_f16(qq, k, v, seq, nq, nkv, d, scale).reshape(seq, nq, d)[-1]
        err = np.abs(got[r] - ref)
        assert (err <= PREFILL_REL * np.abs(ref).max() + PREFILL_REL * np.abs(ref)).all(), r


# ---- against the reference's own layer kernels (oracle/_ref/libref_ops.so) -------------

def _ref_ops():
    if not O.REF_OPS_LIB.exists():
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    return ctypes.CDLL(str(O.REF_OPS_LIB), mode=ctypes.RTLD_LOCAL)


def _both(ref, rf, name, argtypes, args_ours, args_ref):
    for lib, args in ((rf, args_ours), (ref, args_ref)):
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
        print(f"[gpu] {name} ({'ours' if lib is rf else 'reference'})", flush=True)
        assert fn(*args) == 0
        torch.cuda.synchronize()


def test_against_reference_layer_kernels(rf, dev):
    """The same inputs through the reference's norm / rope / kv-write / decode
    attention / argmax / embedding kernels and ours."""
    ref = _ref_ops()
    vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    rng = np.random.default_rng(123)
    n = 4096
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dx, dw = G.to_dev(x), G.to_dev(w)
    a, b = G.empty(n, torch.float32), G.empty(n, torch.float32)
    _both(ref, rf, "gpu_rms_norm", [vp, vp, vp, i, f, vp], (G.ptr(dx), G.ptr(dw), G.ptr(a), n, 1e-6, None),
          (G.ptr(dx), G.ptr(dw), G.ptr(b), n, 1e-6, None))
    assert _rel_err(G.host(a), G.host(b)) <= 1e-6
    # rope (their theta uses powf in fp32; ours is within an ulp of it)
    nh, d = 32, 128
    q = rng.standard_normal(nh * d).astype(np.float32)
    for pos in (3, 100):
        qa, qb = G.to_dev(q), G.to_dev(q)
        _both(ref, rf, "gpu_rope_heads", [vp, i, i, i, f, i, vp], (G.ptr(qa), pos, nh, d, 1e6, 1, None),
              (G.ptr(qb), pos, nh, d, 1e6, 1, None))
        assert _rel_err(G.host(qa), G.host(qb)) <= 1e-5
    # kv write with rope into fp16 caches
    nkv, max_seq, pos = 8, 16, 11
    k = rng.standard_normal(nkv * d).astype(np.float32)
    v = rng.standard_normal(nkv * d).astype(np.float32)
    dk, dv = G.to_dev(k), G.to_dev(v)
    caches = [G.to_dev(np.zeros(max_seq * nkv * d, np.int16)) for _ in range(4)]
    _both(ref, rf, "gpu_kv_write_rope", [vp, vp, vp, vp, i, i, i, f, i, vp],
          (G.ptr(caches[0]), G.ptr(caches[1]), G.ptr(dk), G.ptr(dv), pos, nkv, d, 1e6, 1, None),
          (G.ptr(caches[2]), G.ptr(caches[3]), G.ptr(dk), G.ptr(dv), pos, nkv, d, 1e6, 1, None))
    np.testing.assert_array_equal(G.host(caches[1]), G.host(caches[3]))          # V: the same conversion
    ko = G.host(caches[0]).view(np.float16).astype(np.float64)
    kr = G.host(caches[2]).view(np.float16).astype(np.float64)
    assert (np.abs(ko - kr) <= np.spacing(np.abs(kr).astype(np.float16)).astype(np.float64)).all()
    # decode attention over 640 cached positions, GQA 4
    seq, nkv = 640, 8
    qd = rng.standard_normal(nh * d).astype(np.float32)
    kc = G.to_dev(rng.standard_normal(seq * nkv * d).astype(np.float16).view(np.int16))
    vc = G.to_dev(rng.standard_normal(seq * nkv * d).astype(np.float16).view(np.int16))
    dq = G.to_dev(qd)
    oa, ob = G.empty(nh * d, torch.float32), G.empty(nh * d, torch.float32)
    sc = 1.0 / math.sqrt(d)
    _both(ref, rf, "gpu_flash_attn_decode_strided_multi_head", [vp, vp, vp, vp, i, i, i, i, f, vp],
          (G.ptr(oa), G.ptr(dq), G.ptr(kc), G.ptr(vc), seq, nh, nkv, d, sc, None),
          (G.ptr(ob), G.ptr(dq), G.ptr(kc), G.ptr(vc), seq, nh, nkv, d, sc, None))
    assert _rel_err(G.host(oa), G.host(ob)) <= 1e-5
    # argmax with ties
    lg = rng.standard_normal(151936).astype(np.float32)
    lg[[10, 5000, 151000]] = 9.0
    dl = G.to_dev(lg)
    parts = [G.empty(149, torch.float32), G.empty(149, torch.int32), G.empty(1, torch.int32)]
    parts2 = [G.empty(149, torch.float32), G.empty(149, torch.int32), G.empty(1, torch.int32)]
    _both(ref, rf, "gpu_argmax_f32", [vp, vp, vp, vp, i], (G.ptr(dl), *[G.ptr(t) for t in parts], 151936),
          (G.ptr(dl), *[G.ptr(t) for t in parts2], 151936))
    assert int(G.host(parts[2])[0]) == int(G.host(parts2[2])[0]) == 151000
    # Q4_K embedding row
    from rocmforge_amd import synth
    emb = G.to_dev(synth.q4_k_weights(64, 4096, seed=5))
    ea, eb = G.empty(4096, torch.float32), G.empty(4096, torch.float32)
    _both(ref, rf, "gpu_embed_q4_k_token", [vp, vp, i, i, i, vp], (G.ptr(emb), G.ptr(ea), 4096, 64, 17, None),
          (G.ptr(emb), G.ptr(eb), 4096, 64, 17, None))
    assert _rel_err(G.host(ea), G.host(eb)) <= 1e-6


def _rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b).max() / np.abs(b).max()


def test_rms_norm_and_swiglu_f16_outputs(rf, dev):
    # the fp16-output forms are __float2half of the fp32 launchers' values, bit for bit
    rows, n = 70, 4096
    x = np.random.default_rng(3).standard_normal((rows, n)).astype(np.float32)
    wt = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    dx, dw = G.to_dev(x), G.to_dev(wt)
    d32 = G.empty(rows * n, torch.float32)
    d16 = G.empty(rows * n, torch.int16)
    G.call(rf.gpu_rms_norm_batched_on_stream, G.ptr(dx), G.ptr(dw), G.ptr(d32), n, 1e-6, rows)
    G.call(rf.rf_rms_norm_batched_f16_on_stream, G.ptr(dx), G.ptr(dw), G.ptr(d16), n, 1e-6, rows)
    np.testing.assert_array_equal(G.host(d16), G.host(d32).astype(np.float16).view(np.int16))
    g = np.random.default_rng(5).standard_normal(rows * n).astype(np.float32) * 4
    u = np.random.default_rng(6).standard_normal(rows * n).astype(np.float32)
    dg, du = G.to_dev(g), G.to_dev(u)
    G.call(rf.rf_silu_mul_on_stream, G.ptr(dg), G.ptr(du), G.ptr(d32), rows * n)
    G.call(rf.rf_silu_mul_f16_on_stream, G.ptr(dg), G.ptr(du), G.ptr(d16), rows * n)
    np.testing.assert_array_equal(G.host(d16), G.host(d32).astype(np.float16).view(np.int16))
    assert rf.rf_rms_norm_batched_f16_on_stream(None, G.ptr(dw), G.ptr(d16), n, 1e-6, rows, G.stream()) != 0
    assert rf.rf_silu_mul_f16_on_stream(G.ptr(dg), G.ptr(du), None, 8, G.stream()) != 0


def test_attention_prefill_f16_output(rf, dev):
    # rf_attention_prefill_gqa_causal_f16_launch: __float2half of the fp32
    # launcher's output, bit for bit
    seq, nq, nkv, d = 192, 8, 2, 128
    rng = np.random.default_rng(11)
    q = rng.standard_normal((seq, nq * d)).astype(np.float16)
    k = rng.standard_normal((seq, nkv * d)).astype(np.float16)
    v = rng.standard_normal((seq, nkv * d)).astype(np.float16)
    dq, dk, dv = (G.to_dev(t.view(np.int16)) for t in (q, k, v))
    o32 = G.empty(seq * nq * d, torch.float32)
    o16 = G.empty(seq * nq * d, torch.int16)
    for causal in (1, 0):
        G.call(rf.wmma_attention_prefill_gqa_causal_launch, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(o32), seq, nq, nkv,
               causal, 0.088)
        G.call(rf.rf_attention_prefill_gqa_causal_f16_launch, G.ptr(dq), G.ptr(dk), G.ptr(dv), G.ptr(o16), seq, nq,
               nkv, causal, 0.088)
        np.testing.assert_array_equal(G.host(o16), G.host(o32).astype(np.float16).view(np.int16))
