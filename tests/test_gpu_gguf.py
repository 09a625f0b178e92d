"""GGUF file -> device -> dispatch, on the GPU.

A seeded synthetic Q4_K_M model (Q6_K attn_v / ffn_down on the layers the
Q4_K_M rule picks, Q6_K output.weight) is written, opened, and each matrix
uploaded verbatim (weights.rs:835-851) and run through the host routing the
reference's decode step uses per layer: fused QKV (one launch for an all-Q4_K
layer, three GEMVs where V is Q6_K), fused gate/up + SwiGLU, the residual
down projection (fused for Q4_K; GEMV + add where the arm reports nothing
dispatched, as the reference's caller does for Q6_K), and the LM head, both
an explicit output.weight and one tied to the token embeddings
(weights.rs:868-887).  Every output is checked against the oracle on the
bytes read from the file, at the GEMV tolerance of tests/test_gpu_gemv.py.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from rocmforge_amd import gguf as g
from rocmforge_amd import ops, synth
from rocmforge_amd.ops import GgmlType, TensorRole
from tests import gpu_util as G

pytestmark = pytest.mark.gpu

REL_TOL, ELEM_TOL = 1e-5, 1.0
LAYERS, HIDDEN, FF, HEADS, KV_HEADS, VOCAB = 4, 1024, 3072, 8, 2, 4096


@pytest.fixture(autouse=True)
def _default_launchers(rf):
    ops._lib()
    rf.rf_dispatch_set_launchers(None)
    ops.refresh_runtime_env_flags()


def _ref_gemv(view, x):
    k, n = view.dims
    w = np.ascontiguousarray(view.data).reshape(n, -1)
    return (O.gemv_q4k_q8 if view.ggml_type == GgmlType.Q4_K else O.gemv_q6k)(w, x, k, n)


def _check(y, ref, what):
    rel, elem = G.gemv_error(y, ref)
    print(f"{what}: rel={rel:.3e} elem={elem:.3f}", flush=True)
    assert rel <= REL_TOL and elem <= ELEM_TOL, f"{what}: rel {rel:.3e} elem {elem:.3f}"


def test_q4_k_m_file_through_dispatch(rf, dev, tmp_path):
    path = tmp_path / "q4km.gguf"
    synth.write_q4_k_m_gguf(path, "qwen3", LAYERS, HIDDEN, FF, HEADS, KV_HEADS, VOCAB, seed=5)
    f = g.GgufFile.open(path)
    m = f.metadata
    h, ff, hd = m.embedding_length(), m.feed_forward_length(), m.head_dim()
    q_size, kv_size = m.attention_head_count() * hd, m.attention_head_count_kv() * hd
    assert (h, ff, q_size, kv_size) == (HIDDEN, FF, 1024, 256)
    model = g.load_model(f)
    assert len(model.layers) == LAYERS and not model.lm_head_tied
    seen_fused_qkv = seen_q6_v = False
    for i, lw in enumerate(model.layers):
        p = f"blk.{i}."
        for name in g.LAYER_MATRICES:
            assert np.array_equal(G.host(lw[name][0]), f.tensor(f"{p}{name}.weight").data), name
        assert lw.bias == {"attn_q": None, "attn_k": None, "attn_v": None}
        assert np.array_equal(G.host(lw.attn_q_norm), f.tensor(f"{p}attn_q_norm.weight").data)
        x = synth.activations(h, seed=100 + i)
        dx = G.to_dev(x)
        (wq, mq), (wk, mk), (wv, mv) = lw["attn_q"], lw["attn_k"], lw["attn_v"]
        types = [mq.wtype, mk.wtype, mv.wtype]
        seen_fused_qkv |= types == [GgmlType.Q4_K] * 3
        seen_q6_v |= types[2] == GgmlType.Q6_K
        outs = [G.empty(n, torch.float32) for n in (q_size, kv_size, kv_size)]
        print(f"[gpu] gguf layer {i} qkv {[t.name for t in types]}", flush=True)
        ops.gpu_dispatch_fused_qkv_on_stream(wq, mq, None, wk, mk, None, wv, mv, None, dx, outs[0], outs[1], outs[2],
                                             q_size, kv_size, h, G.stream())
        torch.cuda.synchronize()
        for o, t in zip(outs, ("q", "k", "v")):
            _check(G.host(o), _ref_gemv(f.tensor(f"{p}attn_{t}.weight"), x), f"layer {i} attn_{t}")

        (wg, mg), (wu, mu) = lw["ffn_gate"], lw["ffn_up"]
        act = G.empty(ff, torch.float32)
        print(f"[gpu] gguf layer {i} gate_up", flush=True)
        ops.gpu_dispatch_fused_gate_up_on_stream(wg, mg, wu, mu, dx, act, ff, h, G.stream())
        torch.cuda.synchronize()
        ref_act = O.swiglu(_ref_gemv(f.tensor(f"{p}ffn_gate.weight"), x), _ref_gemv(f.tensor(f"{p}ffn_up.weight"), x))
        _check(G.host(act), ref_act, f"layer {i} gate_up")

        a = G.host(act)                      # the down projection's input: the GPU's activations
        wd, md = lw["ffn_down"]
        res = synth.activations(h, seed=200 + i)
        dres, out = G.to_dev(res), G.empty(h, torch.float32)
        print(f"[gpu] gguf layer {i} down {md.wtype.name}", flush=True)
        done = ops.gpu_dispatch_gemv_residual_on_stream(wd, md, act, dres, out, ff, h, G.stream())
        assert done == (md.wtype == GgmlType.Q4_K)
        if not done:
            ops.gpu_dispatch_gemv_on_stream(wd, md, act, out, h, ff, G.stream())
            out += dres
        torch.cuda.synchronize()
        _check(G.host(out), _ref_gemv(f.tensor(f"{p}ffn_down.weight"), a) + res, f"layer {i} down")
    assert seen_fused_qkv and seen_q6_v

    x = synth.activations(h, seed=300)
    buf, meta = model.lm_head
    assert meta.role == TensorRole.LM_HEAD and meta.wtype == GgmlType.Q6_K
    logits = G.empty(VOCAB, torch.float32)
    print("[gpu] gguf lm_head", flush=True)
    ops.gpu_dispatch_gemv_on_stream(buf, meta, G.to_dev(x), logits, VOCAB, h, G.stream())
    torch.cuda.synchronize()
    _check(G.host(logits), _ref_gemv(f.tensor("output.weight"), x), "lm_head")


def test_qkv_bias_from_file(rf, dev, tmp_path):
    # qwen2-style biases: folded into the fused launch for an all-Q4_K layer;
    # a layer whose V is Q6_K has no fused kernel with a bias here, and the
    # arm says so (NotInLibrary) rather than dropping the bias
    path = tmp_path / "qwen2.gguf"
    synth.write_q4_k_m_gguf(path, "qwen2", 3, 512, 512, 4, 2, 256, seed=8)
    f = g.GgufFile.open(path)
    h, hd = 512, f.metadata.head_dim()
    q_size, kv_size = 4 * hd, 2 * hd
    x = synth.activations(h, seed=9)
    dx = G.to_dev(x)
    for i in range(3):
        lw = g.load_layer(f, i)
        (wq, mq), (wk, mk), (wv, mv) = lw["attn_q"], lw["attn_k"], lw["attn_v"]
        b = lw.bias
        outs = [G.empty(n, torch.float32) for n in (q_size, kv_size, kv_size)]
        args = (wq, mq, b["attn_q"], wk, mk, b["attn_k"], wv, mv, b["attn_v"], dx, outs[0], outs[1], outs[2], q_size,
                kv_size, h, G.stream())
        print(f"[gpu] gguf qwen2 layer {i} qkv+bias V={mv.wtype.name}", flush=True)
        if mv.wtype == GgmlType.Q6_K:
            with pytest.raises(ops.NotInLibrary):
                ops.gpu_dispatch_fused_qkv_on_stream(*args)
            continue
        ops.gpu_dispatch_fused_qkv_on_stream(*args)
        torch.cuda.synchronize()
        for o, t in zip(outs, ("q", "k", "v")):
            bias = f.tensor(f"blk.{i}.attn_{t}.bias").data.view(np.float32).astype(np.float64)
            _check(G.host(o), _ref_gemv(f.tensor(f"blk.{i}.attn_{t}.weight"), x) + bias, f"qwen2 layer {i} attn_{t}")


def test_tied_lm_head(rf, dev, tmp_path):
    path = tmp_path / "tied.gguf"
    synth.write_q4_k_m_gguf(path, "llama", 1, 512, 512, 4, 4, 2048, seed=6, tied=True)
    f = g.GgufFile.open(path)
    buf, meta, tied = g.load_lm_head(f)
    assert tied and meta.role == TensorRole.TIED_LM_HEAD and meta.wtype == GgmlType.Q4_K
    x = synth.activations(512, seed=7)
    logits = G.empty(2048, torch.float32)
    print("[gpu] gguf tied lm_head", flush=True)
    ops.gpu_dispatch_gemv_on_stream(buf, meta, G.to_dev(x), logits, 2048, 512, G.stream())
    torch.cuda.synchronize()
    _check(G.host(logits), _ref_gemv(f.tensor("token_embd.weight"), x), "tied lm_head")
