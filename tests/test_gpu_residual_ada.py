"""GPU parity of the residual gate fused with the AdaZero pass that reads
its output (`fused_residual_gate_adazero_from_ada`, one pass over the rows):
x_new bit for bit the residual gate of the reference (:204-262 with a bias,
:640-692 without), out bit for bit AdaZero of x_new (:40-91), as bf16 rows
or as the e4m3 codes of the FP8 linear's input quantizer (:144-161). The
oracle composes its own residual gate, AdaZero and quantizer; at the
configured size the pass is compared with the separate HIP calls.

Every test runs with OPENGENIE_AMD_STRICT=1 and checks the HIP path ran,
except the fallback test, which checks the separate calls' path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ltx_ops as O
from oracle.numerics import bf16_round
from tests.helpers import assert_same_bits, nan_canon, np32, randn, to_T

pytestmark = pytest.mark.gpu
DEV = "cuda"
C = 4096


@pytest.fixture(autouse=True)
def _strict(monkeypatch):
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    from opengenie_amd import ltx_ops

    ltx_ops.reset_hip_calls()
    yield


def _ran(name):
    from opengenie_amd import ltx_ops

    assert ltx_ops.collect_hip_calls().get(name, 0) > 0, f"{name} did not take the HIP path"


def g(t):
    return t.to(DEV)


def _case(seed, rows, batch, params, tdt, sdt):
    """CPU x, y, table and the timestep row shared by every token (ts[:, :1]
    expanded over the tokens)."""
    x = randn((batch, rows, C), seed)
    y = randn((batch, rows, C), seed + 1, std=0.7)
    table = randn((params, C), seed + 2, dtype=tdt, std=0.02 if tdt == torch.bfloat16 else 1.0)
    ts = randn((batch, 1, params * C), seed + 3, dtype=sdt, std=0.5).expand(batch, rows, params * C)
    return x, y, table, ts


def gts(ts):
    """A shared-row timestep on the GPU, still stride 0 over the tokens
    (moving the expanded view itself would materialise every row)."""
    return g(ts[:, :1]).expand(ts.shape)


def _codes_ref(t, scale, zero_dim):
    with np.errstate(over="ignore", invalid="ignore"):
        return O.fp8_quantize_e4m3(O.bf(bf16_round(t.v)), scale, zero_dim, device="cuda")


@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("out_kind", ["bf16", "e4m3_0dim", "e4m3_1"])
@pytest.mark.parametrize("rows,batch,params,tdt,sdt", [
    (37, 1, 9, torch.float32, torch.bfloat16),   # fewer rows than waves
    (300, 2, 9, torch.bfloat16, torch.bfloat16),  # two batches, each its own timestep row
    (1100, 1, 6, torch.float32, torch.float32),   # float32 Ada values, several rows per wave
])
def test_residual_gate_adazero_matches_oracle(rows, batch, params, tdt, sdt, out_kind, bias_dtype):
    from opengenie_amd.ltx_ops import fused_residual_gate_adazero_from_ada

    x, y, table, ts = _case(900 + rows, rows, batch, params, tdt, sdt)
    bias = randn((C,), 950 + rows, dtype=bias_dtype, std=0.01) if bias_dtype is not None else None
    s = None
    if out_kind != "bf16":
        s = torch.tensor(0.02) if out_kind == "e4m3_0dim" else torch.tensor([0.5 / 448])
    gi, si, ci = params - 1, 3, 4
    x_new, out = fused_residual_gate_adazero_from_ada(
        g(x), g(y), g(table), gts(ts), gate_index=gi, shift_index=si, scale_index=ci, eps=1e-6,
        bias=g(bias) if bias is not None else None, input_scale=g(s) if s is not None else None)
    _ran("fused_residual_gate_adazero_from_ada")
    if bias is not None:
        xr = O.residual_gate_bias_from_ada(to_T(x), to_T(y), to_T(bias), to_T(table), to_T(ts), gi)
    else:
        xr = O.residual_gate_from_ada(to_T(x), to_T(y), to_T(table), to_T(ts), gi)
    assert_same_bits(np32(x_new.cpu()), bf16_round(xr.v), "x_new")
    nr = O.adazero_from_ada(O.bf(bf16_round(xr.v)), 1e-6, to_T(table), to_T(ts), si, ci)
    if s is None:
        assert out.dtype == torch.bfloat16
        assert_same_bits(np32(out.cpu()), bf16_round(nr.v), "AdaZero of x_new")
    else:
        assert out.dtype == torch.float8_e4m3fn
        got = out.view(torch.uint8).cpu().numpy()
        ref = _codes_ref(nr, float(s.reshape(())), out_kind == "e4m3_0dim").reshape(got.shape)
        assert np.array_equal(got, ref), int((got != ref).sum())


def _separate(x, y, table, ts, bias, s, gi, si, ci):
    from opengenie_amd import ltx_ops as L

    if bias is not None:
        xn = L.fused_residual_gate_bias_from_ada(x, y, bias, table, ts, gate_index=gi)
    else:
        xn = L.fused_residual_gate_from_ada(x, y, table, ts, gate_index=gi)
    if s is None:
        return xn, L.fused_adazero_from_ada(xn, 1e-6, table, ts, shift_index=si, scale_index=ci)
    return xn, L.fused_adazero_from_ada_fp8(xn, 1e-6, table, ts, s, shift_index=si, scale_index=ci)


@pytest.mark.parametrize("with_bias,e4m3", [(True, True), (False, True), (False, False)])
def test_residual_gate_adazero_full_size_equals_separate_calls(with_bias, e4m3):
    """At 9216 x 4096 (the configured video tokens): both outputs bit for
    bit those of the separate HIP passes, on the block's shapes (gate 2 and
    the cross-attention's AdaZero rows 6/7; gate 8 and the feed-forward's
    rows 3/4)."""
    from opengenie_amd.ltx_ops import fused_residual_gate_adazero_from_ada

    rows = 9216
    gi, si, ci = (2, 6, 7) if with_bias else (8, 3, 4)
    x, y, table, ts = _case(990, rows, 1, 9, torch.float32, torch.bfloat16)
    x, y, table, ts = g(x), g(y), g(table), gts(ts)
    bias = g(randn((C,), 995, std=0.01)) if with_bias else None
    s = g(torch.tensor(0.0123)) if e4m3 else None
    x_new, out = fused_residual_gate_adazero_from_ada(x, y, table, ts, gate_index=gi, shift_index=si,
                                                      scale_index=ci, eps=1e-6, bias=bias, input_scale=s)
    xs, os_ = _separate(x, y, table, ts, bias, s, gi, si, ci)
    torch.cuda.synchronize()
    _ran("fused_residual_gate_adazero_from_ada")
    assert torch.equal(x_new.view(torch.int16), xs.view(torch.int16))
    if e4m3:
        assert torch.equal(out.view(torch.uint8), os_.view(torch.uint8))
    else:
        assert torch.equal(out.view(torch.int16), os_.view(torch.int16))


def test_residual_gate_adazero_special_values():
    """Rows whose x_new holds a NaN, an infinity (an overflowing gate product)
    or a mean square beyond float32, beside ordinary rows, in one workgroup:
    the rows that cannot produce a NaN take the clamp without the NaN select,
    the others keep it. x_new bit for bit (NaN == NaN), codes NaN-sign-free,
    against the separate HIP passes."""
    from opengenie_amd.ltx_ops import fused_residual_gate_adazero_from_ada

    rows = 300
    x, y, table, ts = _case(1000, rows, 1, 9, torch.bfloat16, torch.bfloat16)
    y[0, 7, 11] = float("nan")
    y[0, 100, 5] = 3.0e38
    x[0, 150] = x[0, 150] * 1e30
    x[0, 151] = 0.0
    y[0, 151] = 0.0
    bias = randn((C,), 1005, std=0.01)
    args = (g(x), g(y), g(table), gts(ts))
    s = g(torch.tensor(0.02))
    x_new, out = fused_residual_gate_adazero_from_ada(*args, gate_index=2, shift_index=6, scale_index=7, eps=1e-6,
                                                      bias=g(bias), input_scale=s)
    xs, os_ = _separate(*args, g(bias), s, 2, 6, 7)
    torch.cuda.synchronize()
    _ran("fused_residual_gate_adazero_from_ada")
    assert_same_bits(np32(x_new.cpu()), np32(xs.cpu()), "x_new")
    assert np.isnan(np32(x_new.cpu())[0, 7, 11])
    got, ref = out.view(torch.uint8).cpu().numpy(), os_.view(torch.uint8).cpu().numpy()
    assert np.array_equal(nan_canon(got), nan_canon(ref))
    assert ((got[0, 7] & 0x7F) == 0x7F).all()


def test_residual_gate_adazero_in_place_through_c_abi():
    """x_out may be x: each row is read before it is written, by one wave."""
    from opengenie_amd import _lib
    from opengenie_amd.ltx_ops import fused_residual_gate_adazero_from_ada

    rows = 777
    x, y, table, ts = _case(1010, rows, 1, 9, torch.float32, torch.bfloat16)
    x, y, table, ts = g(x), g(y), g(table), gts(ts)
    s = g(torch.tensor(0.02))
    x_new, out = fused_residual_gate_adazero_from_ada(x, y, table, ts, gate_index=8, shift_index=3, scale_index=4,
                                                      eps=1e-6, input_scale=s)
    xi = x.clone()
    q = torch.empty(x.shape, device=DEV, dtype=torch.float8_e4m3fn)
    tsv = ts.reshape(1, rows, 9, C)
    _lib.call("oga_residual_gate_adazero_from_ada", xi.data_ptr(), y.data_ptr(), None, 0, xi.data_ptr(),
              q.data_ptr(), 1, rows, C, table.data_ptr(), _lib.DT_F32, table.stride(0), table.stride(1),
              tsv.data_ptr(), _lib.DT_BF16, _lib.strides(tsv.stride()), 8, 3, 4, 1e-6, s.data_ptr(), 1,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(xi.view(torch.int16), x_new.view(torch.int16))
    assert torch.equal(q.view(torch.uint8), out.view(torch.uint8))


def test_residual_gate_adazero_falls_back_to_the_separate_calls(monkeypatch):
    """Per-token timesteps, 2048 columns and a misaligned y view are not the
    pass's inputs: the separate calls run (their own HIP paths), with the
    same results; in strict mode such an input raises instead."""
    from opengenie_amd import ltx_ops as L

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    x, y, table, ts_row = _case(1020, 64, 1, 9, torch.float32, torch.bfloat16)
    ts_tok = randn((1, 64, 9 * C), 1024, std=0.5)
    s = g(torch.tensor(0.02))
    for xx, yy, tt, tb in ((x, y, ts_tok, table),
                           (x[..., :2048].contiguous(), y[..., :2048].contiguous(),
                            ts_tok.reshape(1, 64, 9, C)[..., :2048].reshape(1, 64, -1).contiguous(),
                            table[:, :2048].contiguous())):
        args = tuple(g(t) for t in (xx, yy, tb, tt))
        L.reset_hip_calls()
        x_new, out = L.fused_residual_gate_adazero_from_ada(*args, gate_index=8, shift_index=3, scale_index=4,
                                                            eps=1e-6, input_scale=s)
        calls = L.collect_hip_calls()
        assert calls.get("fused_residual_gate_adazero_from_ada", 0) == 0, calls
        assert calls.get("fused_residual_gate_from_ada", 0) == 1 and calls.get("fused_adazero_from_ada_fp8") == 1
        xs, os_ = _separate(*args, None, s, 8, 3, 4)
        torch.cuda.synchronize()
        assert torch.equal(x_new.view(torch.int16), xs.view(torch.int16))
        assert torch.equal(out.view(torch.uint8), os_.view(torch.uint8))
    # a y view one element off its 16-byte alignment
    yb = g(torch.empty(64 * C + 8, dtype=torch.bfloat16))
    ym = yb[1:1 + 64 * C].view(1, 64, C)
    ym.copy_(g(y))
    L.reset_hip_calls()
    x_new, out = L.fused_residual_gate_adazero_from_ada(g(x), ym, g(table), gts(ts_row), gate_index=8,
                                                        shift_index=3, scale_index=4, eps=1e-6, input_scale=s)
    assert L.collect_hip_calls().get("fused_residual_gate_adazero_from_ada", 0) == 0
    xs, os_ = _separate(g(x), ym, g(table), gts(ts_row), None, s, 8, 3, 4)
    torch.cuda.synchronize()
    assert torch.equal(x_new.view(torch.int16), xs.view(torch.int16))
    assert torch.equal(out.view(torch.uint8), os_.view(torch.uint8))
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    with pytest.raises(RuntimeError):
        L.fused_residual_gate_adazero_from_ada(*(g(t) for t in (x, y, table, ts_tok)), gate_index=8, shift_index=3,
                                               scale_index=4, eps=1e-6, input_scale=s)
