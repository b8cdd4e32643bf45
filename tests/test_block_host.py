"""Host side of the block-slice harness (CPU only, no kernel launch): the
synthetic parameters have the LTX-2.3 video block's shapes and dtypes, and an
FP8 linear's codes decode back to its float weights within e4m3's step."""

from __future__ import annotations

import torch

from opengenie_amd.block import FP8Linear, random_video_block


def test_random_block_shapes():
    blk = random_video_block(4096, 32, device="cpu", seed=3)
    assert blk.table.shape == (9, 4096) and blk.table.dtype == torch.bfloat16
    assert blk.prompt_table.shape == (2, 4096)
    for a in (blk.attn1, blk.attn2):
        for lin in (a.to_q, a.to_k, a.to_v, a.to_out):
            assert lin.weight.shape == (4096, 4096) and lin.weight.dtype == torch.float8_e4m3fn
            assert lin.weight_scale.dim() == 0 and lin.input_scale.dim() == 0
            assert lin.bias.shape == (4096,) and lin.bias.dtype == torch.bfloat16
        assert a.heads == 32 and a.q_norm_weight.shape == (4096,)
    assert blk.ff_up.weight.shape == (16384, 4096) and blk.ff_down.weight.shape == (4096, 16384)
    assert blk.attn1.to_gate_logits is None
    assert random_video_block(4096, 32, device="cpu", gated=True).attn1.to_gate_logits.out_features == 32


def test_fp8_linear_quantized_round_trip():
    w = torch.randn(256, 512) * 0.02
    lin = FP8Linear.quantized(w, 0.01, None)
    back = lin.weight.float() * lin.weight_scale
    assert float(lin.weight.float().abs().max()) == 448.0
    # e4m3 keeps 3 mantissa bits: relative step 2^-3 at most, absolute
    # 2^-9 * scale below the normal range.
    err = (back - w).abs()
    assert bool((err <= torch.maximum(w.abs() * 2 ** -4, torch.full_like(w, 2 ** -10) * lin.weight_scale)).all())
