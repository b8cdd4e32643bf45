"""GPU parity of the dense attention kernel (the reference's FA3 video
self-attention call) and of its FP8 input path.

Bar: against float64 softmax attention on the same bf16 inputs, the kernel
(bf16 output, P rounded to bf16 before P.V, float32 accumulation) is within
|err| <= 2e-3 + 2e-2 * |ref| element-wise, and its RMS error is below 0.4%
of the output RMS. The e4m3 dequantization (the fallback for inputs the FP8
kernel does not take) is bit-exact. The FP8 kernel (both products on e4m3
MFMA, P rounded to e4m3 as FA3 does) is checked against float64 attention on
the exactly dequantized inputs, and against bf16 attention on the
unquantized inputs with the reference benchmark's statistics (max_abs, rms,
mean_rel; benchmarks/video_self_attention_bench.py:288-305): RMS error below
12% of the bf16 output's RMS.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ltx_ops as O
from oracle.numerics import bf16_round
from tests.helpers import assert_same_bits, np32, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _strict(monkeypatch):
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    from opengenie_amd import ltx_ops

    ltx_ops.reset_hip_calls()
    yield


def _ran(name):
    from opengenie_amd import ltx_ops

    assert ltx_ops.collect_hip_calls().get(name, 0) > 0, f"{name} did not take the HIP path"


def _ref(q, k, v, scale=None):
    """float64 attention on [B, N, H, D] numpy arrays -> [B, Nq, H, D]."""
    qt, kt, vt = (np.ascontiguousarray(np32(t).transpose(0, 2, 1, 3)) for t in (q, k, v))
    o = O.attention(qt, kt, vt, scale)
    return o.transpose(0, 2, 1, 3)


def _check(out, ref, what):
    got = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    bound = 2e-3 + 2e-2 * np.abs(ref)
    worst = float((err / bound).max())
    rms_rel = float(np.sqrt((err ** 2).mean()) / np.sqrt((ref ** 2).mean()))
    print(f"{what}: max_abs {err.max():.3e} rms_rel {rms_rel:.3e} worst/bound {worst:.3f}")
    assert worst <= 1.0, (what, worst)
    assert rms_rel < 4e-3, (what, rms_rel)


@pytest.mark.parametrize("b,nq,nk,h", [(1, 128, 128, 1), (1, 256, 256, 2), (2, 300, 300, 3), (1, 100, 77, 2),
                                       (1, 64, 1000, 1), (1, 1024, 1024, 4),
                                       # more than 16 key steps: the 8-wave, three-pair kernel
                                       (1, 300, 1100, 2), (2, 200, 1536, 3)])
def test_attention_matches_oracle(b, nq, nk, h):
    """Up to 16 key steps (1024 keys) the 4-wave, two-pair form of the kernel
    runs, beyond that the 8-wave, three-pair form; both against the oracle."""
    from opengenie_amd.attention import flash_attn_func

    q = randn((b, nq, h, 128), 500 + nq)
    k = randn((b, nk, h, 128), 501 + nk)
    v = randn((b, nk, h, 128), 502 + nk)
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    _ran("flash_attn_func")
    _check(out, _ref(q, k, v), f"attn b{b} nq{nq} nk{nk} h{h}")


@pytest.mark.parametrize("b,nq,nk,h", [(1, 128, 1100, 1), (1, 2048, 1500, 20)])
def test_attention_key_split_and_whole_agree(b, nq, nk, h):
    """flash_attn_func cuts a last partial round of query blocks into key
    parts merged by a second kernel (oga_attention_ws; only beyond 16 key
    steps); oga_attention runs every block over all keys. Both meet the
    oracle bar, and they differ only in float32 summation order."""
    from opengenie_amd import _lib
    from opengenie_amd.attention import _strides3, flash_attn_func

    q = randn((b, nq, h, 128), 800 + nq).to(DEV)
    k = randn((b, nk, h, 128), 801 + nk).to(DEV)
    v = randn((b, nk, h, 128), 802 + nk).to(DEV)
    assert _lib.load().oga_attention_workspace_bytes(b, nq, nk, h, 128) > 0  # the split path runs
    split = flash_attn_func(q, k, v)
    whole = torch.empty_like(q)
    _lib.call("oga_attention", q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(), _strides3(v),
              whole.data_ptr(), _strides3(whole), b, nq, nk, h, 128, 128 ** -0.5,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = _ref(q.cpu(), k.cpu(), v.cpu())
    _check(split, ref, f"attn split b{b} nq{nq} nk{nk} h{h}")
    _check(whole, ref, f"attn whole b{b} nq{nq} nk{nk} h{h}")
    diff = (split.float() - whole.float()).abs()
    assert float(diff.max()) <= 2 ** -7 * float(whole.float().abs().max()), float(diff.max())


def test_attention_workspace_contract():
    """A workspace smaller than the query's size is an argument error (the
    output untouched); no workspace (null, 0 bytes) runs every block whole,
    bit-identical to oga_attention."""
    from opengenie_amd import _lib
    from opengenie_amd.attention import _strides3

    b, nq, nk, h = 1, 256, 1200, 3
    q = randn((b, nq, h, 128), 900).to(DEV)
    k = randn((b, nk, h, 128), 901).to(DEV)
    v = randn((b, nk, h, 128), 902).to(DEV)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    need = int(lib.oga_attention_workspace_bytes(b, nq, nk, h, 128))
    assert need > 0 and need % 16 == 0
    assert lib.oga_attention_workspace_bytes(b, nq, nk, h, 64) == 0
    args = lambda o: (q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(), _strides3(v),
                      o.data_ptr(), _strides3(o), b, nq, nk, h, 128, 128 ** -0.5)
    small = torch.empty((need // 4,), device=DEV, dtype=torch.float32)
    out = torch.zeros_like(q)
    rc = lib.oga_attention_ws(*args(out), small.data_ptr(), need - 16, st)
    assert rc < 0 and b"workspace" in lib.oga_last_error()
    torch.cuda.synchronize()
    assert not out.any()
    none = torch.empty_like(q)
    assert lib.oga_attention_ws(*args(none), None, 0, st) == 0
    whole = torch.empty_like(q)
    assert lib.oga_attention(*args(whole), st) == 0
    torch.cuda.synchronize()
    assert torch.equal(none.view(torch.int16), whole.view(torch.int16))


def test_attention_few_keys_take_no_split():
    """Up to 16 key steps the workspace query is 0 (no key split: each part
    would repeat the block's Q loads and O stores), so oga_attention_ws and
    oga_attention give the same bits; beyond them a partial last round is split."""
    from opengenie_amd import _lib
    from opengenie_amd.attention import _strides3, flash_attn_func

    lib = _lib.load()
    assert lib.oga_attention_workspace_bytes(1, 9216, 256, 32, 128) == 0
    assert lib.oga_attention_workspace_bytes(1, 9216, 1024, 32, 128) == 0
    assert lib.oga_attention_workspace_bytes(1, 9216, 9216, 32, 128) > 0
    b, nq, nk, h = 1, 2000, 256, 8
    q = randn((b, nq, h, 128), 950).to(DEV)
    k = randn((b, nk, h, 128), 951).to(DEV)
    v = randn((b, nk, h, 128), 952).to(DEV)
    out = flash_attn_func(q, k, v)
    whole = torch.empty_like(q)
    _lib.call("oga_attention", q.data_ptr(), _strides3(q), k.data_ptr(), _strides3(k), v.data_ptr(), _strides3(v),
              whole.data_ptr(), _strides3(whole), b, nq, nk, h, 128, 128 ** -0.5,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), whole.view(torch.int16))
    _check(out, _ref(q.cpu(), k.cpu(), v.cpu()), "attn few keys")


def test_attention_scale_and_large_scores():
    """A larger softmax scale sharpens the distribution (online max matters)."""
    from opengenie_amd.attention import flash_attn_func

    q = randn((1, 200, 2, 128), 600, std=3.0)
    k = randn((1, 333, 2, 128), 601, std=3.0)
    v = randn((1, 333, 2, 128), 602)
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), softmax_scale=0.2)
    torch.cuda.synchronize()
    _check(out, _ref(q, k, v, 0.2), "attn sharp")


def test_attention_video_interface_packed_qkv():
    """FlashAttention3.__call__ form: (B, N, H*D) views of one packed QKV tensor."""
    from opengenie_amd.attention import attention_video

    qkv = randn((1, 160, 3, 4 * 128), 700)
    g = qkv.to(DEV)
    q, k, v = g[:, :, 0], g[:, :, 1], g[:, :, 2]
    assert not q.is_contiguous()
    out = attention_video(q, k, v, heads=4)
    torch.cuda.synchronize()
    assert out.shape == (1, 160, 512)
    qn, kn, vn = (qkv[:, :, i].reshape(1, 160, 4, 128) for i in range(3))
    _check(out.view(1, 160, 4, 128), _ref(qn, kn, vn), "attn packed")


def test_fp8_dequant_bit_exact():
    from opengenie_amd.attention import _dequant

    x = randn((2, 33, 4, 128), 800, std=2.0)
    codes = torch.randint(0, 256, x.shape, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    ds = torch.rand((2, 4)) * 0.05 + 1e-3
    out = _dequant(codes.to(DEV).view(torch.float8_e4m3fn), ds.to(DEV))
    torch.cuda.synchronize()
    assert_same_bits(out.float().cpu().numpy(), O.fp8_dequant_per_head(codes.numpy(), ds.numpy()), "dequant")


def _fp8_exact(t8: torch.Tensor, ds: torch.Tensor) -> np.ndarray:
    """e4m3 codes [B, N, H, D] times their [B, H] descale, in float64 (no rounding)."""
    from oracle.numerics import e4m3_decode

    return e4m3_decode(t8.view(torch.uint8).cpu().numpy()).astype(np.float64) * \
        ds.cpu().numpy().astype(np.float64)[:, None, :, None]


def _fp8_rounding_bound(qe: np.ndarray, ke: np.ndarray, ve: np.ndarray) -> np.ndarray:
    """Per-element bound, from the rounding model, of what rounding P to e4m3
    (nearest even) does to the output, for [B, N, H, D] float64 inputs. The
    kernel's running max m lags a row's true max by at most 0.8 (base 2),
    with FlashAttention-3's FP8 offset, so every P = 2^(s - m + 8) is below
    2^8.8 < 448 (finite in e4m3) and a row's largest P is at least 256.
    Rounding moves a P in e4m3's normal range by at most 2^-4 P and one below
    2^-6 (spacing 2^-9) by at most 2^-10, i.e. 2^-18 in units of 256 or of
    the largest P; so, with p_j = exp(s_j - max) and l = sum_j p_j (float32,
    unrounded):
        |out - ref| <= (2^-4 sum_j p_j |v_j| + 2^-18 sum_j |v_j|) / l.
    A key split keeps the bound: each part's P are relative to its own max,
    which is at most the global one."""
    q, k, v = (np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qe, ke, ve))  # [B, H, N, D]
    s = (q @ np.swapaxes(k, -1, -2)) * q.shape[-1] ** -0.5
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    lsum = p.sum(axis=-1, keepdims=True)
    av = np.abs(v)
    bound = (2.0 ** -4 * (p @ av) + 2.0 ** -18 * av.sum(axis=-2, keepdims=True)) / lsum
    return bound.transpose(0, 2, 1, 3)


def _check_fp8(out: np.ndarray, ref: np.ndarray, bound: np.ndarray, what: str) -> float:
    """The FP8 kernel rounds P to e4m3 for the P.V product, as FA3's FP8 path
    does. Against float64 attention on the exactly dequantized inputs: every
    element within the rounding bound above (times 1 + 2^-6 for the float32
    scores and sums, plus the bf16 rounding of the output, 2^-8 |ref|); RMS
    error below 3.5% of the reference RMS (e4m3 keeps 3 mantissa bits: a
    rounding's relative error is uniform within +-2^-4 of the leading power
    of two, about 2.6% RMS over the mantissa range); and no systematic scale
    (least-squares slope of out on ref within 1% of 1), which a biased
    rounding of P or a wrong descale would move."""
    out = out.astype(np.float64)
    err = np.abs(out - ref)
    ref_rms = float(np.sqrt((ref ** 2).mean()))
    worst = float((err / ((1 + 2.0 ** -6) * bound + 2.0 ** -8 * np.abs(ref) + 1e-6)).max())
    rms_rel = float(np.sqrt((err ** 2).mean()) / ref_rms)
    slope = float((out * ref).sum() / (ref * ref).sum())
    print(f"{what}: max_abs {err.max():.3e} rms_rel {rms_rel:.3e} worst/bound {worst:.3f} slope {slope:.5f}")
    assert worst <= 1.0, (what, worst)
    assert rms_rel < 3.5e-2, (what, rms_rel)
    assert abs(slope - 1.0) < 1e-2, (what, slope)
    return rms_rel


@pytest.mark.parametrize("b,nq,nk,h", [(1, 512, 512, 8), (2, 200, 200, 8), (1, 300, 777, 16), (1, 2304, 2304, 32)])
def test_fp8_attention_kernel(b, nq, nk, h):
    """e4m3 Q/K/V from the per-head quantizer through the FP8 kernel, against
    float64 attention on the dequantized inputs (ragged key counts, batch 2,
    nq != nk, a partial query block)."""
    from opengenie_amd.attention import flash_attn_func
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    q = randn((b, nq, h, 128), 910).to(DEV)
    k = randn((b, nk, h, 128), 911).to(DEV)
    v = randn((b, nk, h, 128), 912).to(DEV)
    q8, qs = fused_fp8_quantize_e4m3_per_head_4d(q)
    k8, ks = fused_fp8_quantize_e4m3_per_head_4d(k)
    v8, vs = fused_fp8_quantize_e4m3_per_head_4d(v)
    out = flash_attn_func(q8, k8, v8, q_descale=qs, k_descale=ks, v_descale=vs)
    torch.cuda.synchronize()
    _ran("flash_attn_func_fp8")
    qe, ke, ve = (_fp8_exact(t, s) for t, s in ((q8, qs), (k8, ks), (v8, vs)))
    ref = O.attention(*[np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qe, ke, ve)]).transpose(0, 2, 1, 3)
    _check_fp8(out.float().cpu().numpy(), ref, _fp8_rounding_bound(qe, ke, ve), f"fp8 kernel {b}x{nq}x{nk}x{h}")


def test_fp8_attention_key_split():
    """17 query blocks x 16 heads = 272 workgroups of the FP8 kernel: on a
    256-CU device the 16 past the whole round run as key parts merged by the
    combine kernel (asserted from the workspace query, which then exceeds the
    V rewrite; 1100 keys, more than the 16 steps below which no split is
    made). Against float64 attention with the e4m3 bars."""
    from opengenie_amd import _lib
    from opengenie_amd.attention import flash_attn_func
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    b, nq, nk, h = 1, 17 * 384, 1100, 16
    lib = _lib.load()
    vt_bytes = b * h * 128 * ((nk + 63) // 64 * 64)
    if int(lib.oga_attention_fp8_workspace_bytes(b, nq, nk, h, 128)) <= vt_bytes:
        pytest.skip("this device runs the 272 workgroups without a key split")
    q = randn((b, nq, h, 128), 940).to(DEV)
    k = randn((b, nk, h, 128), 941).to(DEV)
    v = randn((b, nk, h, 128), 942).to(DEV)
    q8, qs = fused_fp8_quantize_e4m3_per_head_4d(q)
    k8, ks = fused_fp8_quantize_e4m3_per_head_4d(k)
    v8, vs = fused_fp8_quantize_e4m3_per_head_4d(v)
    out = flash_attn_func(q8, k8, v8, q_descale=qs, k_descale=ks, v_descale=vs)
    torch.cuda.synchronize()
    _ran("flash_attn_func_fp8")
    qe, ke, ve = (_fp8_exact(t, s) for t, s in ((q8, qs), (k8, ks), (v8, vs)))
    ref = O.attention(*[np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qe, ke, ve)]).transpose(0, 2, 1, 3)
    _check_fp8(out.float().cpu().numpy(), ref, _fp8_rounding_bound(qe, ke, ve), "fp8 key split")


def test_fp8_attention_strided_views():
    """q, k, v as strided [B, N, H, D] views of one packed e4m3 buffer."""
    from opengenie_amd.attention import flash_attn_func

    gg = torch.Generator().manual_seed(930)
    codes = torch.randint(0, 256, (1, 333, 3, 8, 128), generator=gg, dtype=torch.uint8)
    codes[(codes & 0x7F) >= 0x70] = 0x38  # no NaN, moderate magnitudes
    ds = torch.rand((3, 1, 8), generator=gg) * 0.05 + 0.01
    g = codes.to(DEV).view(torch.float8_e4m3fn)
    q8, k8, v8 = g[:, :, 0], g[:, :, 1], g[:, :, 2]
    assert not q8.is_contiguous()
    dsg = ds.to(DEV)
    out = flash_attn_func(q8, k8, v8, q_descale=dsg[0], k_descale=dsg[1], v_descale=dsg[2])
    torch.cuda.synchronize()
    _ran("flash_attn_func_fp8")
    ex = [_fp8_exact(codes[:, :, i].contiguous().view(torch.float8_e4m3fn), ds[i]) for i in range(3)]
    ref = O.attention(*[np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in ex]).transpose(0, 2, 1, 3)
    _check_fp8(out.float().cpu().numpy(), ref, _fp8_rounding_bound(*ex), "fp8 strided")


def test_fp8_attention_config_shape_against_bf16():
    """Config 5: q, k, v (1, 9216, 32, 128) bf16 ~N(0,1), per-head e4m3 through
    the FP8 kernel. Against bf16 attention on the unquantized inputs with the
    reference benchmark's statistics (max_abs, mean_abs, rms, mean_rel;
    video_self_attention_bench.py:288-305): RMS error below 12% of the bf16
    output's RMS. Sampled query rows of 4 heads against float64 attention on
    the dequantized inputs, to the FP8 bar above."""
    from opengenie_amd.attention import flash_attn_func
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3_per_head_4d

    n = 9216
    q, k, v = (randn((1, n, 32, 128), 920 + i).to(DEV) for i in range(3))
    ref16 = flash_attn_func(q, k, v).float()
    q8, qs = fused_fp8_quantize_e4m3_per_head_4d(q)
    k8, ks = fused_fp8_quantize_e4m3_per_head_4d(k)
    v8, vs = fused_fp8_quantize_e4m3_per_head_4d(v)
    out = flash_attn_func(q8, k8, v8, q_descale=qs, k_descale=ks, v_descale=vs)
    torch.cuda.synchronize()
    _ran("flash_attn_func_fp8")
    diff = (out.float() - ref16).abs()
    stats = {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()),
             "rms": float(diff.square().mean().sqrt()),
             "mean_rel": float((diff / ref16.abs().clamp_min(1e-6)).mean())}
    print("fp8 vs bf16 at 1x9216x32x128:", stats)
    assert stats["rms"] < 0.12 * float(ref16.square().mean().sqrt()), stats
    heads = [0, 7, 19, 31]
    rows = np.arange(0, n, 97)  # 96 query rows, both split and whole query blocks
    qe = _fp8_exact(q8, qs)[:, rows][:, :, heads]
    ke = _fp8_exact(k8, ks)[:, :, heads]
    ve = _fp8_exact(v8, vs)[:, :, heads]
    ref = O.attention(*[np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qe, ke, ve)]).transpose(0, 2, 1, 3)
    got = out.float().cpu().numpy()[:, rows][:, :, heads]
    _check_fp8(got, ref, _fp8_rounding_bound(qe, ke, ve), "fp8 config 5 sampled rows")


def test_attention_config_shape():
    """Config 5 on the bf16 kernel: q, k, v (1, 9216, 32, 128) ~N(0,1), the
    schedule the benchmark times (1152 blocks of 256 queries: 4.5 rounds of
    the CUs, the last round's blocks cut in key parts and merged). All 9216
    query rows of heads 0 (first round) and 31 (every block in the key-split
    round), and every 31st row of heads 13 and 30, against float64 attention
    at the bf16 bar above."""
    from opengenie_amd import _lib
    from opengenie_amd.attention import flash_attn_func

    n, h = 9216, 32
    lib = _lib.load()
    assert int(lib.oga_attention_workspace_bytes(1, n, n, h, 128)) > 0  # the key split is planned
    q, k, v = (randn((1, n, h, 128), 960 + i) for i in range(3))
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    _ran("flash_attn_func")
    rows = np.unique(np.concatenate([np.arange(0, n, 31), [n - 1]]))
    qn, kn, vn = (np32(t).astype(np.float64) for t in (q, k, v))
    got = out.float().cpu().numpy().astype(np.float64)
    for head in (13, 30):
        s = qn[0, rows, head] @ kn[0, :, head].T * 128 ** -0.5
        p = np.exp(s - s.max(axis=1, keepdims=True))
        ref = (p @ vn[0, :, head]) / p.sum(axis=1, keepdims=True)
        err = np.abs(got[0, rows, head] - ref)
        worst = float((err / (2e-3 + 2e-2 * np.abs(ref))).max())
        rms_rel = float(np.sqrt((err ** 2).mean()) / np.sqrt((ref ** 2).mean()))
        print(f"attention 1x9216x32x128 head {head}: worst/bound {worst:.3f} rms_rel {rms_rel:.3e}")
        assert worst <= 1.0 and rms_rel < 4e-3, (head, worst, rms_rel)
    # whole heads: float64 softmax attention on the device
    # block = head * 36 + query block; the whole rounds of the 256 CUs run
    # blocks 0 .. 1023, so head 0 is in the first round and head 31 (blocks
    # 1116 .. 1151) wholly in the key-split round
    assert 0 * 36 + 35 < 4 * 256 <= 31 * 36
    for head in (0, 31):
        qd, kd, vd = (t[0, :, head].to(DEV, torch.float64) for t in (q, k, v))
        sd = (qd @ kd.T) * 128 ** -0.5
        pd = torch.exp(sd - sd.amax(dim=1, keepdim=True))
        ref = ((pd @ vd) / pd.sum(dim=1, keepdim=True)).cpu().numpy()
        del sd, pd
        err = np.abs(got[0, :, head] - ref)
        worst = float((err / (2e-3 + 2e-2 * np.abs(ref))).max())
        rms_rel = float(np.sqrt((err ** 2).mean()) / np.sqrt((ref ** 2).mean()))
        print(f"attention 1x9216x32x128 whole head {head}: worst/bound {worst:.3f} rms_rel {rms_rel:.3e}")
        assert worst <= 1.0 and rms_rel < 4e-3, (head, worst, rms_rel)


@pytest.mark.parametrize("b,nq,nk,h", [(1, 300, 256, 4),     # few keys: the 4-wave form
                                       (2, 200, 1536, 3),    # the 8-wave form
                                       (1, 9216, 9216, 32),  # the configured shape: key-split last round
                                       (1, 9216, 256, 32)])  # the text cross-attention's shape
@pytest.mark.parametrize("zero_dim", [True, False])
def test_attention_e4m3_out_is_the_quantized_attention(b, nq, nk, h, zero_dim):
    """attention_video_e4m3_out: the codes the output projection's input
    quantizer writes for the bf16 attention output, bit for bit, from one
    pass: against `fused_fp8_quantize_e4m3(attention_video(...))` (the same
    deterministic kernel, so the same bf16 output) and against the oracle's
    quantizer applied to that bf16 output; the key-split merge included
    (9216 queries x 32 heads leave a partial last round)."""
    from opengenie_amd.attention import attention_video, attention_video_e4m3_out
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3

    q = randn((b, nq, h * 128), 700 + nq, std=2.0).to(DEV)
    k = randn((b, nk, h * 128), 701 + nk, std=2.0).to(DEV)
    v = randn((b, nk, h * 128), 702 + nk).to(DEV)
    scale = 0.004
    s = torch.tensor(scale, device=DEV) if zero_dim else torch.tensor([scale], device=DEV)
    codes = attention_video_e4m3_out(q, k, v, h, s)
    _ran("attention_video_e4m3_out")
    o = attention_video(q, k, v, h)
    ref = fused_fp8_quantize_e4m3(o, s)
    torch.cuda.synchronize()
    assert codes.dtype == torch.float8_e4m3fn and codes.shape == (b, nq, h * 128)
    got = codes.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, ref.view(torch.uint8).cpu().numpy())
    rows = slice(0, min(nq, 600))  # the oracle's quantizer on part of the rows
    want = O.fp8_quantize_e4m3(O.bf(np32(o[:, rows].cpu())), scale, zero_dim, device="cuda")
    assert np.array_equal(got[:, rows], want.reshape(got[:, rows].shape))
    if zero_dim:
        assert (np.abs(np32(codes.float().cpu())) == 448).any()  # saturated tails


def test_attention_e4m3_out_falls_back_to_the_two_calls(monkeypatch):
    """A head size the kernel does not take runs attention then the
    quantizer (torch's attention here); strict mode raises instead."""
    from opengenie_amd import ltx_ops as L
    from opengenie_amd.attention import attention_video, attention_video_e4m3_out

    monkeypatch.delenv("OPENGENIE_AMD_STRICT", raising=False)
    q, k, v = (randn((1, 64, 4 * 64), 720 + i).to(DEV) for i in range(3))
    s = torch.tensor(0.01, device=DEV)
    L.reset_hip_calls()
    codes = attention_video_e4m3_out(q, k, v, 4, s)
    assert L.collect_hip_calls().get("attention_video_e4m3_out", 0) == 0
    ref = L.fused_fp8_quantize_e4m3(attention_video(q, k, v, 4), s)
    assert torch.equal(codes.view(torch.uint8), ref.view(torch.uint8))
    monkeypatch.setenv("OPENGENIE_AMD_STRICT", "1")
    with pytest.raises(RuntimeError):
        attention_video_e4m3_out(q, k, v, 4, s)


@pytest.mark.parametrize("b,nq,nk,h", [(1, 1, 1, 1), (2, 31, 33, 3), (1, 33, 64, 2), (2, 1000, 65, 3),
                                       (1, 700, 200, 4), (1, 4096, 256, 32), (3, 97, 256, 1),
                                       # more (batch, head) pairs than CUs: one workgroup each
                                       (3, 70, 100, 100)])
def test_attention_few_keys_resident_kernel(b, nq, nk, h):
    """Up to 256 keys the K and V of a head stay in LDS for the workgroup's
    life and each wave runs its 32-query groups on its own: partial key
    tiles (1, 33, 65, 200 keys), partial query groups, one query, several
    batches and heads, grids of fewer than 8 and of no multiple of 8
    workgroups (the XCD-contiguous numbering); against the oracle, and the
    e4m3 output against the quantizer on the bf16 output."""
    from opengenie_amd.attention import attention_video, attention_video_e4m3_out, flash_attn_func
    from opengenie_amd.ltx_ops import fused_fp8_quantize_e4m3

    q = randn((b, nq, h, 128), 960 + nq)
    k = randn((b, nk, h, 128), 961 + nk)
    v = randn((b, nk, h, 128), 962 + nk)
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV))
    _ran("flash_attn_func")
    _check(out, _ref(q, k, v), f"few keys b{b} nq{nq} nk{nk} h{h}")
    qf, kf, vf = (t.reshape(b, t.shape[1], h * 128).to(DEV) for t in (q, k, v))
    s = torch.tensor(0.01, device=DEV)
    codes = attention_video_e4m3_out(qf, kf, vf, h, s)
    ref = fused_fp8_quantize_e4m3(attention_video(qf, kf, vf, h), s)
    torch.cuda.synchronize()
    assert torch.equal(codes.view(torch.uint8), ref.view(torch.uint8))
    assert torch.equal(out.reshape(b, nq, h * 128).view(torch.int16), attention_video(qf, kf, vf, h).view(torch.int16))
