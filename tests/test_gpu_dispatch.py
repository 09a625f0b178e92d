"""The host routing (rf_gpu_dispatch_*) on the GPU: each arm produces the
same result as its launcher called directly, and the prefill arm's M
padding (ops.rs:1674, padded_m = round_up(seq_len, 64)) gives the oracle's
product on the real rows."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rocmforge_amd import ops, synth
from rocmforge_amd.ops import GgmlType, WeightMeta
from tests import gpu_util as G

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _default_launchers(rf):
    ops._lib()
    rf.rf_dispatch_set_launchers(None)
    ops.refresh_runtime_env_flags()


def test_gemv_arms_match_direct_launch(rf, dev):
    k, n = 4096, 1024
    w4 = G.to_dev(synth.q4_k_weights(n, k, seed=11))
    w6 = G.to_dev(synth.q6_k_weights(n, k, seed=12))
    x = G.to_dev(synth.activations(k, seed=13))
    for w, t, direct in ((w4, GgmlType.Q4_K, rf.gemv_q4_k_f32_q8_inline_launch), (w6, GgmlType.Q6_K,
                                                                                 rf.gemv_q6_k_f32_launch)):
        y0, y1 = G.empty(n, torch.float32), G.empty(n, torch.float32)
        G.call(direct, G.ptr(w), G.ptr(x), G.ptr(y0), k, n)
        print(f"[gpu] dispatch gemv {t.name} {n}x{k}", flush=True)
        ops.gpu_dispatch_gemv_on_stream(w, WeightMeta(t, [k, n]), x, y1, n, k, G.stream())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(G.host(y0), G.host(y1))


def test_fused_qkv_arm(rf, dev):
    # all-Q4_K (one fused launch, bias folded in) and a Q6_K V (three GEMVs)
    k, nq, nkv = 4096, 1024, 256
    ws = [synth.q4_k_weights(n, k, seed=31 + i) for i, n in enumerate((nq, nkv, nkv))]
    w6 = synth.q6_k_weights(nkv, k, seed=34)
    bq = synth.activations(nq, seed=35)
    x = synth.activations(k, seed=36)
    dws, dw6, dbq, dx = [G.to_dev(w) for w in ws], G.to_dev(w6), G.to_dev(bq), G.to_dev(x)
    outs = [G.empty(n, torch.float32) for n in (nq, nkv, nkv)]
    metas = [WeightMeta(GgmlType.Q4_K, [k, n]) for n in (nq, nkv, nkv)]
    print("[gpu] dispatch fused qkv, all Q4_K", flush=True)
    ops.gpu_dispatch_fused_qkv_on_stream(dws[0], metas[0], dbq, dws[1], metas[1], None, dws[2], metas[2], None, dx,
                                         outs[0], outs[1], outs[2], nq, nkv, k, G.stream())
    torch.cuda.synchronize()
    for i, n in enumerate((nq, nkv, nkv)):
        ref = O.gemv_q4k_q8(ws[i], x, k, n) + (bq.astype(np.float64) if i == 0 else 0.0)
        assert np.abs(G.host(outs[i]) - ref).max() / np.abs(ref).max() < 1e-5, i
    print("[gpu] dispatch fused qkv, Q6_K V", flush=True)
    ops.gpu_dispatch_fused_qkv_on_stream(dws[0], metas[0], None, dws[1], metas[1], None, dw6,
                                         WeightMeta(GgmlType.Q6_K, [k, nkv]), None, dx, outs[0], outs[1], outs[2],
                                         nq, nkv, k, G.stream())
    torch.cuda.synchronize()
    ref = O.gemv_q6k(w6, x, k, nkv)
    assert np.abs(G.host(outs[2]) - ref).max() / np.abs(ref).max() < 1e-5


def test_residual_and_fused_arms(rf, dev):
    k, n = 4096, 512
    wq = synth.q4_k_weights(n, k, seed=21)
    wu = synth.q4_k_weights(n, k, seed=22)
    x = synth.activations(k, seed=23)
    r = synth.activations(n, seed=24)
    dw, du, dx = G.to_dev(wq), G.to_dev(wu), G.to_dev(x)
    out = G.to_dev(r.copy())
    print("[gpu] dispatch residual in place", flush=True)
    assert ops.gpu_dispatch_gemv_residual_on_stream(dw, WeightMeta(GgmlType.Q4_K, [k, n]), dx, out, out, k, n,
                                                    G.stream())
    torch.cuda.synchronize()
    ref = O.gemv_q4k_q8(wq, x, k, n) + r
    assert np.abs(G.host(out) - ref).max() / np.abs(ref).max() < 1e-5
    sw = G.empty(n, torch.float32)
    print("[gpu] dispatch fused gate+up", flush=True)
    ops.gpu_dispatch_fused_gate_up_on_stream(dw, WeightMeta(GgmlType.Q4_K, [k, n]), du,
                                             WeightMeta(GgmlType.Q4_K, [k, n]), dx, sw, n, k, G.stream())
    torch.cuda.synchronize()
    ref = O.swiglu(O.gemv_q4k_q8(wq, x, k, n), O.gemv_q4k_q8(wu, x, k, n))
    assert np.abs(G.host(sw) - ref).max() / np.abs(ref).max() < 1e-5


@pytest.mark.parametrize("fmt,seq", [("q4_k", 100), ("q6_k", 70), ("q6_k", 5)])
def test_gemm_arm_pads_rows(rf, dev, fmt, seq):
    n, k = 256, 1024
    padded = -(-seq // 64) * 64
    a = np.zeros((padded, k), np.float32)
    a[:seq] = synth.activations(k, seed=seq, m=seq)
    w = synth.weights(fmt, n, k, seed=31)
    da, dw = G.to_dev(a), G.to_dev(w)
    d = torch.zeros(padded * n, dtype=torch.float32, device="cuda:0")
    t = GgmlType.Q4_K if fmt == "q4_k" else GgmlType.Q6_K
    print(f"[gpu] dispatch gemm {fmt} seq={seq} padded={padded}", flush=True)
    ops.gpu_dispatch_gemm(dw, WeightMeta(t, [k, n]), da, d, n, k, seq)
    torch.cuda.synchronize()
    got = G.host(d).reshape(padded, n)
    ref = O.gemm(fmt, a[:seq], w, seq, n, k)
    err = np.abs(got[:seq].astype(np.float64) - ref)
    assert (err / (2e-3 * np.abs(ref) + 1e-5 * np.abs(ref).max())).max() <= 1.0
    assert np.all(got[seq:] == 0.0)
