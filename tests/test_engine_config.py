"""Host-side checks of the model engine that need no GPU."""
import pytest

from rocmforge_amd import engine as E


def test_prefill_rejects_head_dims_the_attention_kernel_cannot_take():
    # the prefill attention launcher takes no head_dim: rows of n_heads * 128
    # values are what it reads, so other head dims must be refused up front
    cfg = E.ModelConfig.qwen3_8b()
    E.check_prefill_config(cfg)                 # head_dim 128: accepted
    for hd in (64, 96, 256):
        bad = E.ModelConfig(**{**cfg.__dict__, "head_dim": hd})
        with pytest.raises(ValueError, match="head_dim"):
            E.check_prefill_config(bad)
