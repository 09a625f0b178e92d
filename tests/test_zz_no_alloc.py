"""The allocation-free decode attention (rf_flash_attn_decode_state_noalloc)
against the workspace entry point it mirrors (rf_flash_attn_decode_state_ws),
through the C ABI: two calls in a row, the second on a smaller input, then
the size limit of the library's fixed array."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import gpu_util as G

pytestmark = pytest.mark.gpu


def _case(rng, seq, nh, nkv, d):
    max_seq = seq + 3
    q = rng.standard_normal(nh * d).astype(np.float32)
    kc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.int16)
    vc = rng.standard_normal(max_seq * nkv * d).astype(np.float16).view(np.int16)
    return q, kc, vc


def test_noalloc_attention_matches_workspace_entry_point(rf, dev):
    rng = np.random.default_rng(2024)
    # the larger call first, then a smaller one: the second must not see the
    # first call's partials (the array keeps the last call's contents)
    for seq, nh, nkv, d in [(1500, 64, 8, 256), (37, 8, 2, 64)]:
        q, kc, vc = _case(rng, seq, nh, nkv, d)
        dq, dkc, dvc = G.to_dev(q), G.to_dev(kc), G.to_dev(vc)
        dlen = G.to_dev(np.array([seq], np.int32))
        scale = 1.0 / math.sqrt(d)
        wsb = int(rf.rf_flash_attn_decode_workspace_bytes(nh, d))
        ws = torch.full((wsb // 4,), float("nan"), dtype=torch.float32, device="cuda:0")
        ref_out = G.empty(nh * d, torch.float32)
        out = G.empty(nh * d, torch.float32)
        print(f"[case] seq {seq} nh {nh} nkv {nkv} d {d}", flush=True)
        G.call(rf.rf_flash_attn_decode_state_ws, G.ptr(ref_out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh,
               nkv, d, scale, G.ptr(ws), wsb)
        G.call(rf.rf_flash_attn_decode_state_noalloc, G.ptr(out), G.ptr(dq), G.ptr(dkc), G.ptr(dvc), G.ptr(dlen), nh,
               nkv, d, scale)
        np.testing.assert_array_equal(G.host(out), G.host(ref_out))
        ref = O.attn_decode(q, kc.view(np.uint16), vc.view(np.uint16), seq, nh, nkv, d, scale)
        err = np.abs(G.host(out).astype(np.float64) - ref).max() / np.abs(ref).max()
        assert err <= 1e-5, err


def test_noalloc_attention_rejects_sizes_beyond_the_array(rf, dev):
    dq = G.to_dev(np.zeros(128 * 256, np.float32))      # finite q (fresh memory may hold anything)
    dkc = G.empty(16 * 256, torch.int16)
    dlen = G.to_dev(np.array([4], np.int32))
    # 128 heads x (256 + 4) = 33280 > 16640
    rc = rf.rf_flash_attn_decode_state_noalloc(G.ptr(dq), G.ptr(dq), G.ptr(dkc), G.ptr(dkc), G.ptr(dlen), 128, 8,
                                               256, 0.0625, G.stream())
    assert rc != 0
    # the limit itself is accepted: 64 heads x 260
    out = G.empty(64 * 256, torch.float32)
    kc = G.to_dev(np.zeros(4 * 8 * 256, np.int16))
    G.call(rf.rf_flash_attn_decode_state_noalloc, G.ptr(out), G.ptr(dq), G.ptr(kc), G.ptr(kc), G.ptr(dlen), 64, 8,
           256, 0.0625)
    assert np.isfinite(G.host(out)).all()
