"""The allocation-free per-head FP8 quantizer (oga_fp8_quantize_per_head_noalloc)
against the workspace entry point it mirrors (oga_fp8_quantize_per_head),
bit for bit, through the C ABI: two calls in a row on one device, the first
using the whole static scratch, the second a smaller input that reuses it."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu


def _run(lib, name, x, heads, head_dim, workspace=None):
    from opengenie_amd import _lib

    b, n = x.shape[0], x.shape[1]
    xdt = _lib.DT_F16 if x.dtype == torch.float16 else _lib.DT_BF16
    q = torch.empty(x.shape, device="cuda", dtype=torch.uint8)
    s = torch.empty((b, heads), device="cuda", dtype=torch.float32)
    st = torch.cuda.current_stream().cuda_stream
    if workspace is None:
        _lib.call(name, x.data_ptr(), xdt, q.data_ptr(), s.data_ptr(), b, n, heads, head_dim, st)
    else:
        _lib.call(name, x.data_ptr(), xdt, q.data_ptr(), s.data_ptr(), workspace.data_ptr(), b, n, heads, head_dim,
                  st)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def test_per_head_noalloc_matches_workspace_entry_point():
    from opengenie_amd import _lib

    lib = _lib.load()
    cap = int(lib.oga_fp8_per_head_noalloc_max_bytes())
    assert cap == 1 << 20
    g = torch.Generator(device="cuda")
    g.manual_seed(20260601)
    # (1, 131072, 32, 128): 8192 token blocks x 32 heads x 4 bytes = the whole
    # scratch; then (2, 1000, 16, 64), a smaller call reusing it, in bf16 and
    # in fp16.
    for shape, dtype in [((1, 131072, 32, 128), torch.bfloat16), ((2, 1000, 16, 64), torch.bfloat16),
                         ((2, 1000, 16, 64), torch.float16)]:
        b, n, h, d = shape
        need = int(lib.oga_fp8_per_head_workspace_bytes(b, n, h, d))
        assert 0 < need <= cap
        x = (torch.randn(shape, generator=g, device="cuda") * 3.0).to(dtype)
        x.view(-1)[:: 9973] = 0.0
        ws = torch.empty((need // 4,), device="cuda", dtype=torch.float32)
        q_ref, s_ref = _run(lib, "oga_fp8_quantize_per_head", x, h, d, workspace=ws)
        q, s = _run(lib, "oga_fp8_quantize_per_head_noalloc", x, h, d)
        assert_same_bits(s, s_ref, f"per-head scale {shape} {dtype}")
        assert np.array_equal(q, q_ref), (shape, dtype)
        del x, ws


def test_per_head_noalloc_rejects_shapes_beyond_the_scratch():
    from opengenie_amd import _lib

    lib = _lib.load()
    # 131073 tokens x 32 heads need 8193 blocks of partials: one block more than
    # the scratch holds. Rejected before any pointer is used or kernel launched.
    rc = lib.oga_fp8_quantize_per_head_noalloc(None, _lib.DT_BF16, None, None, 1, 131073, 32, 128, None)
    assert rc == -2
    assert b"static scratch" in lib.oga_last_error()
