"""A llama/qwen-style model on the library's kernels: prefill and greedy
decode, the decode step capturable as one HIP graph.

The layer order is the reference's GPU decode step
(src/gpu/forward.rs:2327-2535): RMSNorm -> QKV (fused when all Q4_K) ->
per-head Q/K RMSNorm + RoPE + fp16 KV write -> attention -> O projection
with the residual -> RMSNorm -> fused gate/up + SwiGLU -> down projection
with the residual; then the output norm, the LM head and a greedy argmax
(forward.rs:290-376).  Decode reads the position from device memory
(state = {pos, seq_len}, advanced by a kernel at the end of the step), so a
captured step replays for every token.  Prefill follows
gpu_prefill_layer_forward_hybrid (forward.rs:886-1198): GEMMs over rows
padded to 64, batched norms / RoPE / KV write, the MFMA prefill attention,
residual adds, and the LM head on the last row.

Weights come from a GGUF file (gguf.load_model) or are generated on the
device from a seed in the Q4_K_M type mix (synthetic_weights).  Everything
runs through the C ABI of librocmforge_cdna4.so; there is no other
implementation to fall back to.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

from . import _lib, ops
from .ops import GgmlType, TensorRole, WeightMeta


@dataclass
class ModelConfig:
    n_layers: int
    hidden: int
    ff: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    rope_base: float = 1e6
    neox: bool = True
    qk_norm: bool = True

    @property
    def q_size(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.n_kv_heads * self.head_dim

    @classmethod
    def qwen3_8b(cls) -> "ModelConfig":
        return cls(36, 4096, 12288, 32, 8, 128, 151936)

    @classmethod
    def from_gguf(cls, f) -> "ModelConfig":
        m = f.metadata
        arch = m.architecture
        return cls(m.block_count(), m.embedding_length(), m.feed_forward_length(), m.attention_head_count(),
                   m.attention_head_count_kv() or m.attention_head_count(), m.head_dim(),
                   m.vocab_size() or f.desc("token_embd.weight").dims[1], m.rms_norm_eps(1e-6),
                   m.rope_freq_base(1e6 if arch == "qwen3" else 1e4), arch in ("qwen2", "qwen3"),
                   f.has_tensor("blk.0.attn_q_norm.weight"))


@dataclass
class Layer:
    attn_norm: object
    ffn_norm: object
    mats: dict            # name -> (uint8 device tensor, WeightMeta)
    q_norm: object = None
    k_norm: object = None


@dataclass
class Weights:
    token_emb: tuple
    output_norm: object
    lm_head: tuple
    layers: list


def weights_from_gguf(f, device="cuda:0") -> Weights:
    from . import gguf
    mw = gguf.load_model(f, device)
    layers = [Layer(lw.attn_norm, lw.ffn_norm, dict(lw.matrices), lw.attn_q_norm, lw.attn_k_norm)
              for lw in mw.layers]
    return Weights(mw.token_emb, mw.output_norm, mw.lm_head, layers)


def synthetic_weights(cfg: ModelConfig, seed: int = 0, device="cuda:0", signed: bool = False) -> Weights:
    """Seeded random weights of the configuration in the Q4_K_M type mix
    (Q6_K attn_v / ffn_down on the layers gguf.q4_k_m_uses_q6_k picks and
    Q6_K output.weight), generated in device memory.  signed: Q4_K blocks of
    random sign (synth.torch_weights), which keeps the activations of a deep
    stack in range."""
    import torch

    from . import synth
    from .gguf import q4_k_m_uses_q6_k
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    s = [seed * 7919]

    def mat(n, k, q6=False):
        s[0] += 1
        fmt = "q6_k" if q6 else "q4_k"
        w = synth.torch_weights(fmt, n, k, seed=s[0], device=device, signed=signed).reshape(-1)
        return w, WeightMeta(GgmlType.Q6_K if q6 else GgmlType.Q4_K, [k, n])

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, device=device, generator=gen)).float()

    h, kv, q = cfg.hidden, cfg.kv_size, cfg.q_size
    layers = []
    for i in range(cfg.n_layers):
        q6 = q4_k_m_uses_q6_k(i, cfg.n_layers)
        mats = {"attn_q": mat(q, h), "attn_k": mat(kv, h), "attn_v": mat(kv, h, q6), "attn_output": mat(h, q),
                "ffn_gate": mat(cfg.ff, h), "ffn_up": mat(cfg.ff, h), "ffn_down": mat(h, cfg.ff, q6)}
        layers.append(Layer(norm(h), norm(h), mats, norm(cfg.head_dim) if cfg.qk_norm else None,
                            norm(cfg.head_dim) if cfg.qk_norm else None))
    emb = mat(cfg.vocab, h)
    lm_w, lm_meta = mat(cfg.vocab, h, True)
    lm_meta.role = TensorRole.LM_HEAD
    return Weights(emb, norm(h), (lm_w, lm_meta), layers)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _chk(rc, what):
    if rc != 0:
        raise ops.HipApiError(rc, what)


# The prefill attention kernel (wmma_attention_prefill_gqa_causal_launch) is
# built for head_dim 128 and its launcher takes no head_dim to check.
PREFILL_HEAD_DIM = 128


def check_prefill_config(cfg) -> None:
    """Raises ValueError for a model the prefill path cannot run: the
    prefill attention reads Q/K/V rows of n_heads * 128 / n_kv_heads * 128
    values, so any other head_dim would be read with the wrong strides."""
    if cfg.head_dim != PREFILL_HEAD_DIM:
        raise ValueError(f"prefill needs head_dim {PREFILL_HEAD_DIM} (the prefill attention kernel's); "
                         f"this model has head_dim {cfg.head_dim}")


class Engine:
    """Prefill + greedy decode of one sequence of up to max_seq tokens."""

    def __init__(self, cfg: ModelConfig, weights: Weights, max_seq: int = 1024, device="cuda:0",
                 fuse_norm: bool = True, fold_qk: bool = True, fuse_gemm: bool = True, ffn_f16: bool = True,
                 rope_table: bool = True, attn_bounded: bool = False, norm_in_down: bool = True):
        """fuse_norm: decode with the RMSNorms folded into the GEMVs that
        consume them, the per-head Q/K step into the attention and the state
        advance into the argmax (same bits as the separate launches);
        fold_qk: the per-head Q/K step folded into the attention (with
        fuse_norm; same bits; measured on MI355X at the Qwen3-8B shape
        1.83 ms/token against 1.89 with the separate step);
        fuse_gemm: prefill projections that share an input in one segmented
        GEMM launch, and the O / FFN-down products added straight into the
        residual stream (same per-element products; the sums of a K split
        land in another order);
        ffn_f16: (with fuse_gemm) a Q4_K gate/up prefill on fp16 activations:
        the FFN norm rounded to fp16 feeds two 256 x 128-tile GEMMs and the
        SwiGLU (the same operand values as the fp32 launchers);
        rope_table: the fused Q/K launchers read cos / sin of every
        position's RoPE angles from a table made here once (the values their
        cosf / sinf would give, so the same bits);
        attn_bounded: the decode attention is told that the sequence never
        exceeds max_seq (the cache length), so for caches of up to 2048
        positions it runs one workgroup per query head with the partials
        merged inside it, instead of the split kernel and its merge launch
        (the same attention within fp32 rounding; measured on MI355X at the
        Qwen3-8B shape 1.843 ms/token against 1.816 for the split path, so
        off by default);
        norm_in_down: (with the fp16 prefill path) the next layer's attention
        norm taken by the FFN-down launch that adds into the residual stream
        (rf_gemm_q*_k_f16_accumulate_rmsnorm_launch: in the split-K
        reduction's pass over the rows; the same bits as the separate norm)."""
        import torch
        self.cfg, self.w, self.max_seq, self.dev = cfg, weights, max_seq, device
        self.fuse_norm = fuse_norm
        self.fold_qk = fold_qk and fuse_norm
        self.fuse_gemm = fuse_gemm
        self.rope_table = rope_table
        self.attn_bounded = attn_bounded
        self.norm_in_down = norm_in_down
        self.lib = _lib.load()
        ops._lib()
        f32, i16 = torch.float32, torch.int16
        z = lambda n, dt=f32: torch.zeros(n, dtype=dt, device=device)
        c = cfg
        self.kc = [z(max_seq * c.kv_size, i16) for _ in range(c.n_layers)]
        self.vc = [z(max_seq * c.kv_size, i16) for _ in range(c.n_layers)]
        self.hidden, self.normed = z(c.hidden), z(c.hidden)
        self.q, self.k, self.v, self.attn = z(c.q_size), z(c.kv_size), z(c.kv_size), z(c.q_size)
        self.act, self.tmp, self.logits = z(c.ff), z(c.hidden), z(c.vocab)
        n_part = (c.vocab + 1023) // 1024
        self.part_v, self.part_i = z(n_part), z(n_part, torch.int32)
        self.token = z(1, torch.int32)
        self.state = z(2, torch.int32)      # {pos, seq_len}
        self.scale = 1.0 / math.sqrt(c.head_dim)
        # RoPE thetas and the split decode attention's workspace: caller-owned
        # buffers, made here once (the launchers allocate nothing)
        self.theta = z(max(c.head_dim // 2, 1))
        ws_bytes = int(self.lib.rf_flash_attn_decode_workspace_bytes(c.n_heads, c.head_dim))
        self.attn_ws = z((ws_bytes + 3) // 4)
        self.attn_ws_bytes = ws_bytes
        _chk(self.lib.rf_rope_theta_table(_p(self.theta), c.head_dim, c.rope_base, self._stream()), "theta table")
        self.cos_sin = None
        if rope_table and c.head_dim % 2 == 0:
            self.cos_sin = z(max_seq * c.head_dim)      # [pos][head_dim / 2] (cos, sin) pairs
            _chk(self.lib.rf_rope_cos_sin_table(_p(self.cos_sin), max_seq, c.head_dim, c.rope_base, _p(self.theta),
                                                None, self._stream()), "cos / sin table")
        self._graph = None
        self._pf = None
        self._act16 = False      # the last prefill layer's SwiGLU output went to the fp16 buffer
        self.ffn_f16 = ffn_f16
        self._ffn16 = False      # the last prefill layer ran gate/up on the fp16 norm
        self._att16 = False      # the last prefill layer's attention output went to the fp16 buffer
        self._qkv16 = False      # the last prefill layer ran Q/K/V on the fp16 attention norm

    # ---- decode ---------------------------------------------------------------------------
    def _stream(self):
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def decode_launches(self, trace=None):
        """One token: reads self.token and self.state, writes the next token
        into self.token and advances the state.  trace(name, layer) is called
        after each operation when given (eager runs only)."""
        import torch
        L, c, st = self.lib, self.cfg, self._stream()
        t = trace or (lambda name, layer: None)
        _chk(L.gpu_embed_q4_k_batch(_p(self.w.token_emb[0]), _p(self.token), _p(self.hidden), c.hidden, c.vocab, 1,
                                    st), "embed")
        t("embed", -1)
        pos_p = _p(self.state)
        len_p = ctypes.c_void_p(self.state.data_ptr() + 4)
        for i, lw in enumerate(self.w.layers):
            m = lw.mats
            if self.fuse_norm:
                self._qkv_normed(m, lw.attn_norm, st)
            else:
                _chk(L.gpu_rms_norm(_p(self.hidden), _p(lw.attn_norm), _p(self.normed), c.hidden, c.eps, st), "norm")
                t("attn_norm", i)
                ops.gpu_dispatch_fused_qkv_on_stream(m["attn_q"][0], m["attn_q"][1], None, m["attn_k"][0],
                                                     m["attn_k"][1], None, m["attn_v"][0], m["attn_v"][1], None,
                                                     self.normed, self.q, self.k, self.v, c.q_size, c.kv_size,
                                                     c.hidden, st)
            t("qkv", i)
            if self.fold_qk and self.attn_bounded and (self.max_seq <= 2048 or c.n_heads // c.n_kv_heads <= 8):
                _chk(L.rf_attn_decode_qk_norm_rope_state_bounded(_p(self.attn), _p(self.q), _p(self.k), _p(self.v),
                                                                 _p(lw.q_norm), _p(lw.k_norm), _p(self.kc[i]),
                                                                 _p(self.vc[i]), pos_p, c.n_heads, c.n_kv_heads,
                                                                 c.head_dim, c.eps, c.rope_base, int(c.neox), None,
                                                                 _p(self.theta), _p(self.cos_sin), self.scale,
                                                                 self.max_seq, _p(self.attn_ws), self.attn_ws_bytes,
                                                                 st),
                     "qk step + attention")
            elif self.fold_qk and c.n_heads // c.n_kv_heads <= 8:
                _chk(L.rf_attn_decode_qk_norm_rope_state(_p(self.attn), _p(self.q), _p(self.k), _p(self.v),
                                                         _p(lw.q_norm), _p(lw.k_norm), _p(self.kc[i]), _p(self.vc[i]),
                                                         pos_p, c.n_heads, c.n_kv_heads, c.head_dim, c.eps,
                                                         c.rope_base, int(c.neox), None, _p(self.theta),
                                                         _p(self.cos_sin), self.scale,
                                                         _p(self.attn_ws), self.attn_ws_bytes, st),
                     "qk step + attention")
            else:
                _chk(L.rf_qk_norm_rope_kv_write_state(_p(self.q), _p(self.k), _p(self.v), _p(lw.q_norm),
                                                      _p(lw.k_norm), _p(self.kc[i]), _p(self.vc[i]), pos_p,
                                                      c.n_heads, c.n_kv_heads, c.head_dim, c.eps, c.rope_base,
                                                      int(c.neox), None, _p(self.theta), _p(self.cos_sin), st),
                     "qk_rope_kv")
                t("qk_rope_kv", i)
                if self.attn_bounded:
                    _chk(L.rf_flash_attn_decode_state_bounded(_p(self.attn), _p(self.q), _p(self.kc[i]),
                                                              _p(self.vc[i]), len_p, c.n_heads, c.n_kv_heads,
                                                              c.head_dim, self.scale, self.max_seq,
                                                              _p(self.attn_ws), self.attn_ws_bytes, st), "attention")
                else:
                    _chk(L.rf_flash_attn_decode_state_ws(_p(self.attn), _p(self.q), _p(self.kc[i]), _p(self.vc[i]),
                                                         len_p, c.n_heads, c.n_kv_heads, c.head_dim, self.scale,
                                                         _p(self.attn_ws), self.attn_ws_bytes, st), "attention")
            t("attention", i)
            self._residual_gemv(m["attn_output"], self.attn, c.q_size, st)
            t("attn_output", i)
            if self.fuse_norm and m["ffn_gate"][1].wtype == GgmlType.Q4_K and m["ffn_up"][1].wtype == GgmlType.Q4_K:
                _chk(L.rf_gemv_gate_up_q4_k_q8_rmsnorm_launch(_p(m["ffn_gate"][0]), _p(m["ffn_up"][0]),
                                                              _p(self.hidden), _p(lw.ffn_norm), c.eps, _p(self.act),
                                                              c.hidden, c.ff, st), "gate_up+norm")
            else:
                _chk(L.gpu_rms_norm(_p(self.hidden), _p(lw.ffn_norm), _p(self.normed), c.hidden, c.eps, st), "norm")
                t("ffn_norm", i)
                ops.gpu_dispatch_fused_gate_up_on_stream(m["ffn_gate"][0], m["ffn_gate"][1], m["ffn_up"][0],
                                                         m["ffn_up"][1], self.normed, self.act, c.ff, c.hidden, st)
            t("gate_up", i)
            self._residual_gemv(m["ffn_down"], self.act, c.ff, st)
            t("ffn_down", i)
        lm_w, lm_meta = self.w.lm_head
        if self.fuse_norm and lm_meta.wtype == GgmlType.Q6_K and self._q6_norm_ok(c.hidden):
            _chk(L.rf_gemv_q6_k_rmsnorm_launch(_p(lm_w), _p(self.hidden), _p(self.w.output_norm), c.eps,
                                               _p(self.logits), c.hidden, c.vocab, st), "lm_head+norm")
        else:
            _chk(L.gpu_rms_norm(_p(self.hidden), _p(self.w.output_norm), _p(self.normed), c.hidden, c.eps, st),
                 "norm")
            t("output_norm", -1)
            ops.gpu_dispatch_gemv_on_stream(lm_w, lm_meta, self.normed, self.logits, c.vocab, c.hidden, st)
        t("lm_head", -1)
        if self.fuse_norm:
            _chk(L.rf_argmax_f32_advance_state_on_stream(_p(self.logits), _p(self.part_v), _p(self.part_i),
                                                         _p(self.token), c.vocab, _p(self.state), st), "argmax")
        else:
            _chk(L.gpu_argmax_f32_on_stream(_p(self.logits), _p(self.part_v), _p(self.part_i), _p(self.token),
                                            c.vocab, st), "argmax")
            _chk(L.gpu_increment_decode_state_on_stream(_p(self.state), st), "state")
        t("argmax", -1)

    @staticmethod
    def _q6_norm_ok(k):
        return (k // 256) % 8 == 0 and k <= 16384

    def _qkv_normed(self, m, norm_w, st):
        """q, k, v = W rmsnorm(hidden): one launch when all three are Q4_K
        or Q/K are Q4_K and V is Q6_K, else one normalising GEMV per
        matrix."""
        L, c = self.lib, self.cfg
        mats = [m["attn_q"], m["attn_k"], m["attn_v"]]
        outs = [(self.q, c.q_size), (self.k, c.kv_size), (self.v, c.kv_size)]
        if all(mt[1].wtype == GgmlType.Q4_K for mt in mats):
            _chk(L.rf_gemv_qkv_q4_k_q8_rmsnorm_launch(_p(mats[0][0]), _p(mats[1][0]), _p(mats[2][0]), None, None,
                                                      None, _p(self.hidden), _p(norm_w), c.eps, _p(self.q),
                                                      _p(self.k), _p(self.v), c.hidden, c.q_size, c.kv_size, st),
                 "qkv+norm")
            return
        if ([mt[1].wtype for mt in mats] == [GgmlType.Q4_K, GgmlType.Q4_K, GgmlType.Q6_K]
                and c.hidden in (2048, 4096, 8192)):
            _chk(L.rf_gemv_qkv_q4_k_q6_k_v_rmsnorm_launch(_p(mats[0][0]), _p(mats[1][0]), _p(mats[2][0]), None, None,
                                                          None, _p(self.hidden), _p(norm_w), c.eps, _p(self.q),
                                                          _p(self.k), _p(self.v), c.hidden, c.q_size, c.kv_size, st),
                 "qkv+norm (q6_k v)")
            return
        for (w, meta), (out, n) in zip(mats, outs):
            if meta.wtype == GgmlType.Q4_K:
                _chk(L.rf_gemv_q4_k_q8_rmsnorm_launch(_p(w), _p(self.hidden), _p(norm_w), c.eps, _p(out), c.hidden,
                                                      n, st), "gemv+norm")
            elif meta.wtype == GgmlType.Q6_K and self._q6_norm_ok(c.hidden):
                _chk(L.rf_gemv_q6_k_rmsnorm_launch(_p(w), _p(self.hidden), _p(norm_w), c.eps, _p(out), c.hidden, n,
                                                   st), "gemv+norm")
            else:
                _chk(L.gpu_rms_norm(_p(self.hidden), _p(norm_w), _p(self.normed), c.hidden, c.eps, st), "norm")
                ops.gpu_dispatch_gemv_on_stream(w, meta, self.normed, out, n, c.hidden, st)

    def _residual_gemv(self, wm, x, k, st):
        """hidden += W x: the fused residual kernels (Q4_K through the
        dispatch arm, Q6_K through its residual launcher), else GEMV + add."""
        w, meta = wm
        c = self.cfg
        if meta.wtype == GgmlType.Q6_K:
            _chk(self.lib.gemv_q6_k_f32_residual_launch(_p(w), _p(x), _p(self.hidden), _p(self.hidden), k, c.hidden,
                                                        st), "q6_k residual")
            return
        if not ops.gpu_dispatch_gemv_residual_on_stream(w, meta, x, self.hidden, self.hidden, k, c.hidden, st):
            ops.gpu_dispatch_gemv_on_stream(w, meta, x, self.tmp, c.hidden, k, st)
            _chk(self.lib.gpu_add(_p(self.hidden), _p(self.tmp), _p(self.hidden), c.hidden, st), "add")

    def capture_decode(self):
        """Capture one decode step as a graph (after one eager warm-up step
        on the capture stream, whose effect on the state is undone)."""
        import torch
        s = torch.cuda.Stream()
        saved = (self.token.clone(), self.state.clone(), [k.clone() for k in self.kc], [v.clone() for v in self.vc])
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.decode_launches()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.token.copy_(saved[0])
        self.state.copy_(saved[1])
        for a, b in zip(self.kc + self.vc, saved[2] + saved[3]):
            a.copy_(b)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self.decode_launches()
        torch.cuda.synchronize()
        self._graph = g
        return g

    def decode(self, n: int, graph: bool = True) -> list:
        """n greedy steps from the current token/state; returns the tokens
        produced (each step's argmax), reading them back once at the end."""
        import torch
        if self.state.cpu()[0].item() + n > self.max_seq:
            raise ValueError("sequence would exceed max_seq")
        out = torch.empty(n, dtype=torch.int32, device=self.dev)
        if graph and self._graph is None:
            self.capture_decode()
        for i in range(n):
            if graph:
                self._graph.replay()
            else:
                self.decode_launches()
            out[i:i + 1].copy_(self.token)
        torch.cuda.synchronize()
        return out.cpu().tolist()

    # ---- prefill ------------------------------------------------------------------------------
    def _prefill_buffers(self, mp):
        import torch
        if self._pf is not None and self._pf["mp"] >= mp:
            return self._pf
        c = self.cfg
        z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device=self.dev)
        self._pf = {"mp": mp, "x": z(mp * c.hidden), "xn": z(mp * c.hidden), "q": z(mp * c.q_size),
                    "k": z(mp * c.kv_size), "v": z(mp * c.kv_size), "q16": z(mp * c.q_size, torch.int16),
                    "k16": z(mp * c.kv_size, torch.int16), "v16": z(mp * c.kv_size, torch.int16),
                    "att": z(mp * c.q_size), "tmp": z(mp * c.hidden), "g": z(mp * c.ff), "u": z(mp * c.ff),
                    "g16": z(mp * c.ff, torch.int16), "xn16": z(mp * c.hidden, torch.int16),
                    "att16": z(mp * c.q_size, torch.int16),
                    "ids": z(mp, torch.int32)}
        return self._pf

    def _qkv16_ok(self, lw) -> bool:
        """Whether a prefill layer runs Q/K/V as fp16 segments on its attention
        norm rounded to fp16."""
        c = self.cfg
        types = [lw.mats[n][1].wtype for n in ("attn_q", "attn_k", "attn_v")]
        return (self.fuse_gemm and self.ffn_f16 and all(ty in (GgmlType.Q4_K, GgmlType.Q6_K) for ty in types)
                and c.q_size % 64 == 0 and c.kv_size % 64 == 0
                and c.hidden % (2048 if GgmlType.Q6_K in types else 256) == 0)

    def prefill(self, tokens, trace=None) -> int:
        """Runs the prompt (positions 0..M-1), fills the KV caches, sets the
        state to {M, M + 1} and self.token to the greedy next token, which
        it returns."""
        import torch
        L, c = self.lib, self.cfg
        check_prefill_config(c)
        M = len(tokens)
        if M < 1 or M > self.max_seq:
            raise ValueError("prompt length out of range")
        mp = -(-M // 64) * 64
        b = self._prefill_buffers(mp)
        t = trace or (lambda name, layer: None)
        st = self._stream()
        for key in ("x", "q", "k", "v"):
            b[key].zero_()
        b["ids"][:M].copy_(torch.as_tensor(tokens, dtype=torch.int32))
        _chk(L.gpu_embed_q4_k_batch(_p(self.w.token_emb[0]), _p(b["ids"]), _p(b["x"]), c.hidden, c.vocab, M, st),
             "embed")
        t("embed", -1)
        normed_ahead = False     # this layer's fp16 attention norm was written by the last FFN-down launch
        for i, lw in enumerate(self.w.layers):
            m = lw.mats
            qkv = [(m["attn_q"], b["q"], c.q_size), (m["attn_k"], b["k"], c.kv_size),
                   (m["attn_v"], b["v"], c.kv_size)]
            types = [wm[1].wtype for wm, _, _ in qkv]
            # Q/K/V on the attention norm rounded to fp16 (the operand values the fp32
            # launchers round it to): one launch of K-sliced tiles whatever the type mix
            self._qkv16 = self._qkv16_ok(lw)
            if self._qkv16:
                if not normed_ahead:
                    _chk(L.rf_rms_norm_batched_f16_on_stream(_p(b["x"]), _p(lw.attn_norm), _p(b["xn16"]), c.hidden,
                                                             c.eps, mp, st), "norm f16")
                _chk(L.rf_gemm_qk_f16_segments_launch(_p(b["xn16"]), *[_p(wm[0]) for wm, _, _ in qkv],
                                                      *[int(ty) for ty in types], *[_p(o) for _, o, _ in qkv], mp,
                                                      c.q_size, c.kv_size, c.kv_size, c.hidden, st), "qkv f16")
            else:
                _chk(L.gpu_rms_norm_batched_on_stream(_p(b["x"]), _p(lw.attn_norm), _p(b["xn"]), c.hidden, c.eps, mp,
                                                      st), "norm")
                self._gemm_group(qkv, b["xn"], c.hidden, M, st)
            t("qkv", i)
            if self.fuse_norm and c.head_dim in (64, 128, 256) and mp <= self.max_seq:
                # per-head norms, RoPE, the KV-cache rows and fp16 Q in one launch (the
                # launches below, with each head's sum of squares taken in another
                # order); K and V for the attention are the fp16 cache rows
                _chk(L.rf_qk_norm_rope_kv_write_rows(_p(b["q"]), _p(b["k"]), _p(b["v"]), _p(lw.q_norm),
                                                     _p(lw.k_norm), _p(b["q16"]), _p(self.kc[i]), _p(self.vc[i]), 0,
                                                     mp, M, c.n_heads, c.n_kv_heads, c.head_dim, self.max_seq, c.eps,
                                                     c.rope_base, int(c.neox), None, _p(self.theta),
                                                     _p(self.cos_sin), st), "qk rows")
                t("qk_rope_kv", i)
                k16, v16 = self.kc[i], self.vc[i]
            else:
                if lw.q_norm is not None:
                    _chk(L.gpu_rms_norm_batched_on_stream(_p(b["q"]), _p(lw.q_norm), _p(b["q"]), c.head_dim, c.eps,
                                                          M * c.n_heads, st), "q norm")
                    _chk(L.gpu_rms_norm_batched_on_stream(_p(b["k"]), _p(lw.k_norm), _p(b["k"]), c.head_dim, c.eps,
                                                          M * c.n_kv_heads, st), "k norm")
                _chk(L.rf_rope_heads_batched_on_stream(_p(b["q"]), 0, c.n_heads, c.head_dim, c.rope_base, M,
                                                       int(c.neox), None, st), "rope q")
                _chk(L.rf_rope_heads_batched_on_stream(_p(b["k"]), 0, c.n_kv_heads, c.head_dim, c.rope_base, M,
                                                       int(c.neox), None, st), "rope k")
                _chk(L.rf_kv_write_batched_on_stream(_p(self.kc[i]), _p(self.vc[i]), _p(b["k"]), _p(b["v"]), 0,
                                                     c.kv_size, self.max_seq, M, st), "kv write")
                t("qk_rope_kv", i)
                # K and V: the fp16 cache rows just written are the attention's operands
                # (same [position][kv heads * d] layout; keys past the prompt are seen
                # only by the padding queries, whose outputs are never used; real queries
                # weigh them by an exact zero, and every cache row holds finite fp16)
                _chk(L.convert_f32_to_f16(_p(b["q"]), _p(b["q16"]), mp * c.q_size, st), "to f16")
                if mp <= self.max_seq:
                    k16, v16 = self.kc[i], self.vc[i]
                else:
                    for src, dst in (("k", "k16"), ("v", "v16")):
                        _chk(L.convert_f32_to_f16(_p(b[src]), _p(b[dst]), mp * c.kv_size, st), "to f16")
                    k16, v16 = b["k16"], b["v16"]
            # a Q4_K O projection reads the attention output as fp16 (the operand its
            # fp32 launcher would round it to) through the K-sliced 128 x 64 tiles
            self._att16 = (self.fuse_gemm and self.ffn_f16 and m["attn_output"][1].wtype == GgmlType.Q4_K
                           and c.hidden % 64 == 0 and c.q_size % 256 == 0)
            if self._att16:
                _chk(L.rf_attention_prefill_gqa_causal_f16_launch(_p(b["q16"]), _p(k16), _p(v16), _p(b["att16"]),
                                                                  mp, c.n_heads, c.n_kv_heads, 1, self.scale, st),
                     "attention f16")
            else:
                _chk(L.wmma_attention_prefill_gqa_causal_launch(_p(b["q16"]), _p(k16), _p(v16), _p(b["att"]),
                                                               mp, c.n_heads, c.n_kv_heads, 1, self.scale, st),
                     "attention")
            t("attention", i)
            if self._att16:
                _chk(L.rf_gemm_q4_k_f16_accumulate_launch(_p(b["att16"]), _p(m["attn_output"][0]), _p(b["x"]), mp,
                                                          c.hidden, c.q_size, st), "gemm f16 accumulate")
            else:
                self._gemm_residual(m["attn_output"], b["att"], b["x"], b["tmp"], c.hidden, c.q_size, M, st)
            t("attn_output", i)
            gt, ut = m["ffn_gate"][1].wtype, m["ffn_up"][1].wtype
            gu16 = (self.fuse_gemm and self.ffn_f16 and gt == ut == GgmlType.Q4_K and c.ff % 128 == 0
                    and c.hidden % 256 == 0)
            if gu16:
                _chk(L.rf_rms_norm_batched_f16_on_stream(_p(b["x"]), _p(lw.ffn_norm), _p(b["xn16"]), c.hidden, c.eps,
                                                         mp, st), "norm f16")
            else:
                _chk(L.gpu_rms_norm_batched_on_stream(_p(b["x"]), _p(lw.ffn_norm), _p(b["xn"]), c.hidden, c.eps, mp,
                                                      st), "norm")
            self._ffn16 = gu16
            pair = gt == ut and c.ff % 128 == 0 and self._fusable(gt, 256, c.hidden)
            # a Q6_K down projection reads the SwiGLU output as fp16 (the operand its
            # fp32 launcher would round it to) through the 128 x 64-tile kernel
            self._act16 = (pair or gu16) and self._down_f16(m["ffn_down"][1].wtype)
            if gu16 and self._pair16(mp):
                # gate and up in one launch on the fp16 norm (256 x 128 tiles of 64 gate
                # and the same 64 up rows), SwiGLU in the epilogue
                _chk(L.rf_gemm_q4_k_f16_swiglu_launch(_p(b["xn16"]), _p(m["ffn_gate"][0]), _p(m["ffn_up"][0]),
                                                      _p(b["g16"] if self._act16 else b["g"]), int(self._act16), mp,
                                                      c.ff, c.hidden, st), "gemm f16 swiglu")
            elif gu16:
                # gate and up as two GEMMs on the fp16 norm; the SwiGLU in the up GEMM's
                # store when the down projection takes fp16, else its own kernel
                _chk(L.rf_gemm_q4_k_f16_launch(_p(b["xn16"]), _p(m["ffn_gate"][0]), _p(b["g"]), mp, c.ff, c.hidden,
                                               st), "gemm f16")
                if self._act16:
                    _chk(L.rf_gemm_q4_k_f16_swiglu_up_launch(_p(b["xn16"]), _p(m["ffn_up"][0]), _p(b["g"]),
                                                             _p(b["g16"]), mp, c.ff, c.hidden, st), "gemm f16 swiglu up")
                else:
                    _chk(L.rf_gemm_q4_k_f16_launch(_p(b["xn16"]), _p(m["ffn_up"][0]), _p(b["u"]), mp, c.ff, c.hidden,
                                                   st), "gemm f16")
                    _chk(L.rf_silu_mul_on_stream(_p(b["g"]), _p(b["u"]), _p(b["g"]), mp * c.ff, st), "swiglu")
            elif self._act16:
                fn = L.rf_gemm_q4_k_swiglu_f16_launch if gt == GgmlType.Q4_K else L.rf_gemm_q6_k_swiglu_f16_launch
                _chk(fn(_p(b["xn"]), _p(m["ffn_gate"][0]), _p(m["ffn_up"][0]), _p(b["g16"]), mp, c.ff, c.hidden,
                        st), "gemm swiglu f16")
            elif pair:
                # gate and up in one launch, SwiGLU in its epilogue
                fn = L.rf_gemm_q4_k_swiglu_launch if gt == GgmlType.Q4_K else L.rf_gemm_q6_k_swiglu_launch
                _chk(fn(_p(b["xn"]), _p(m["ffn_gate"][0]), _p(m["ffn_up"][0]), _p(b["g"]), mp, c.ff, c.hidden, st),
                     "gemm swiglu")
            else:
                self._gemm(m["ffn_gate"], b["xn"], b["g"], c.ff, c.hidden, M, st)
                self._gemm(m["ffn_up"], b["xn"], b["u"], c.ff, c.hidden, M, st)
                _chk(L.rf_silu_mul_on_stream(_p(b["g"]), _p(b["u"]), _p(b["g"]), mp * c.ff, st), "swiglu")
            t("gate_up", i)
            nxt = self.w.layers[i + 1] if i + 1 < len(self.w.layers) else None
            normed_ahead = False
            if self._act16 and self.norm_in_down and nxt is not None and self._qkv16_ok(nxt):
                # the next layer's fp16 attention norm taken with the residual add
                q6 = m["ffn_down"][1].wtype == GgmlType.Q6_K
                fn = (L.rf_gemm_q6_k_f16_accumulate_rmsnorm_launch if q6
                      else L.rf_gemm_q4_k_f16_accumulate_rmsnorm_launch)
                _chk(fn(_p(b["g16"]), _p(m["ffn_down"][0]), _p(b["x"]), _p(nxt.attn_norm), c.eps, _p(b["xn16"]), mp,
                        c.hidden, c.ff, st), "gemm f16 accumulate + norm")
                normed_ahead = True
            elif self._act16:
                fn = (L.rf_gemm_q6_k_f16_accumulate_launch if m["ffn_down"][1].wtype == GgmlType.Q6_K
                      else L.rf_gemm_q4_k_f16_accumulate_launch)
                _chk(fn(_p(b["g16"]), _p(m["ffn_down"][0]), _p(b["x"]), mp, c.hidden, c.ff, st),
                     "gemm f16 accumulate")
            else:
                self._gemm_residual(m["ffn_down"], b["g"], b["x"], b["tmp"], c.hidden, c.ff, M, st)
            t("ffn_down", i)
        last = ctypes.c_void_p(b["x"].data_ptr() + 4 * (M - 1) * c.hidden)
        _chk(L.gpu_rms_norm(last, _p(self.w.output_norm), _p(self.normed), c.hidden, c.eps, st), "norm")
        ops.gpu_dispatch_gemv_on_stream(self.w.lm_head[0], self.w.lm_head[1], self.normed, self.logits, c.vocab,
                                        c.hidden, st)
        _chk(L.gpu_argmax_f32_on_stream(_p(self.logits), _p(self.part_v), _p(self.part_i), _p(self.token), c.vocab,
                                        st), "argmax")
        self.state.copy_(torch.tensor([M, M + 1], dtype=torch.int32))
        t("lm_head", -1)
        torch.cuda.synchronize()
        return int(self.token.item())

    def _down_f16(self, wtype):
        """The FFN down projection on fp16 activations: Q6_K with K = ff a
        multiple of 2048 (rf_gemm_q6_k_f16_accumulate_launch), or Q4_K with
        the fp16 FFN path (rf_gemm_q4_k_f16_accumulate_launch); N = hidden a
        multiple of 64."""
        c = self.cfg
        if not self.fuse_gemm or c.hidden % 64:
            return False
        if wtype == GgmlType.Q6_K:
            return c.ff % 2048 == 0
        return self.ffn_f16 and wtype == GgmlType.Q4_K and c.ff % 256 == 0

    def _pair16(self, mp):
        """Gate and up on fp16 activations as one paired launch when its 256-row
        tiles come to one round of CUs and the last one is at least half full
        (measured on MI355X at 12288 x 4096: M = 256 75 us against 111 us for two
        GEMMs and the SwiGLU kernel; M = 512 150 against 133, M = 128 73 against
        58); otherwise two GEMMs and the SwiGLU kernel."""
        import torch
        cus = torch.cuda.get_device_properties(self.dev).multi_processor_count
        tail = mp % 256
        return -(-mp // 256) * (self.cfg.ff // 64) <= cus and (tail == 0 or tail > 128)

    def _fusable(self, wtype, n, k):
        return (self.fuse_gemm and wtype in (GgmlType.Q4_K, GgmlType.Q6_K) and n % 256 == 0
                and k % (2048 if wtype == GgmlType.Q6_K else 512) == 0)

    def _gemm_group(self, items, a, k, m, st):
        """items = [((w, meta), out, n), ...] over one input: runs of up to
        three matrices of one type go through one segmented launch (the Q/K/V
        projections); the rest one GEMM each."""
        mp = -(-m // 64) * 64
        i = 0
        while i < len(items):
            t = items[i][0][1].wtype
            j = i
            while j < len(items) and j - i < 3 and items[j][0][1].wtype == t and self._fusable(t, items[j][2], k):
                j += 1
            if j - i < 2:
                (wm, out, n) = items[i]
                self._gemm(wm, a, out, n, k, m, st)
                i += 1
                continue
            run = items[i:j] + [((None, None), None, 0)] * (3 - (j - i))
            fn = (self.lib.rf_gemm_q4_k_segments_launch if t == GgmlType.Q4_K
                  else self.lib.rf_gemm_q6_k_segments_launch)
            _chk(fn(_p(a), *[_p(r[0][0]) for r in run], *[_p(r[1]) for r in run], mp, *[r[2] for r in run], k, st),
                 "gemm segments")
            i = j

    def _gemm_residual(self, wm, a, x, tmp, n, k, m, st):
        """x[:m] += a W^T: one accumulating launch where the shape allows
        (its padding rows then take the padding rows' product too), else a
        GEMM into tmp and an add of the m real rows."""
        w, meta = wm
        if self._fusable(meta.wtype, n, k):
            mp = -(-m // 64) * 64
            fn = (self.lib.rf_gemm_q4_k_accumulate_launch if meta.wtype == GgmlType.Q4_K
                  else self.lib.rf_gemm_q6_k_accumulate_launch)
            _chk(fn(_p(a), _p(w), _p(x), mp, n, k, st), "gemm accumulate")
            return
        self._gemm(wm, a, tmp, n, k, m, st)
        _chk(self.lib.gpu_add(_p(x), _p(tmp), _p(x), m * n, st), "add")

    def _gemm(self, wm, a, out, n, k, m, st):
        """out[m_pad x n] = a[m_pad x k] W^T through the prefill GEMM launchers
        (rows padded to 64; the padding rows of a are zero)."""
        w, meta = wm
        mp = -(-m // 64) * 64
        fn = self.lib.wmma_gemm_q4_k_launch if meta.wtype == GgmlType.Q4_K else self.lib.wmma_gemm_q6_k_launch
        _chk(fn(_p(a), _p(w), _p(out), mp, n, k, st), "gemm")
