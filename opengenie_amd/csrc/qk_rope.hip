// Video self-attention preattention: per-token RMSNorm over the full hidden
// size (learned weight) followed by split RoPE per head, for q and k in one
// pass sharing the cos/sin tile.
//
// Reference: ltx_serve/triton_ltx_ops.py :320-378 (dual q/k), :381-429 (QKV
// pack), :432-505 (separate), :508-587 (bias) with the torch path :958-973
// and the split-RoPE restatement of tests/test_triton_ltx_ops.py:232-249:
//   n = R(x * inv_rms * w)
//   first  half d <  64: o = R( R?(n[d]*cos[d])    - R?(n[d+64]*sin[d]) )
//   second half d >= 64: o = R( R?(n[d]*cos[d-64]) + R?(n[d-64]*sin[d-64]) )
// R? rounds iff cos/sin are bf16.
//
// Layout: one wavefront per token row, head_dim 128. Lane l of vector step j
// holds columns j*512 + 8l .. +7, i.e. head 4j + l/16, head dims 8(l%16)..+7.
// The RoPE partner of lane l (same head, other half) is lane l^8 of the same
// 16-lane DPP row, fetched with one row_ror:8 DPP move per packed dword. The
// 8 cos/sin values a lane needs are one 128-bit load, shared by q and k.
#include "common.h"
#include "host.h"

namespace oga {

struct RopeArgs {
  const uint16_t* x0;
  const uint16_t* x1;
  const uint16_t* v;
  const void* w0;
  const void* w1;
  const void* b0;
  const void* b1;
  const void* cos;
  const void* sin;
  uint16_t* o0;
  uint16_t* o1;
  uint16_t* ov;
  int64_t c_sb, c_sh, c_st;
  int64_t s_sb, s_sh, s_st;
  int64_t out_stride;  // elements between consecutive output rows
  int64_t tokens;
  int cols;
  int w_dt, b_dt, cs_dt;
  int cs_vec;
  float eps;
};

OGA_DEVICE void lds_put8(float* s, int c0, const float* v) {
  *(float4*)(s + c0) = make_float4(v[0], v[1], v[2], v[3]);
  *(float4*)(s + c0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
OGA_DEVICE void lds_get8(const float* s, int c0, float* v) {
  const float4 a = *(const float4*)(s + c0);
  const float4 b = *(const float4*)(s + c0 + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// RMS normaliser of one packed row (after the optional bias, which the
// row already carries): inv = 1/sqrt(mean(x^2) + eps), exact sum of squares.
template <int CH>
OGA_DEVICE float row_inv(const uint4* xv, float eps) {
  double ss[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    float xf[8];
    unpack8(xv[j], xf);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double d = (double)xf[i];
      ss[i & 3] = fma(d, d, ss[i & 3]);
    }
  }
  return rms_inv((ss[0] + ss[1]) + (ss[2] + ss[3]), CH * 512, eps);
}

// x <- R(x + R(bias)) for one vector step (bias already rounded in LDS).
OGA_DEVICE uint4 add_bias8(const uint4& xv, const float* B, int c0) {
  float xf[8], bv[8];
  unpack8(xv, xf);
  lds_get8(B, c0, bv);
#pragma unroll
  for (int i = 0; i < 8; ++i) xf[i] = xf[i] + bv[i];
  return pack8(xf);
}

// n = R(x * inv * w) for one vector step, packed.
OGA_DEVICE uint4 norm8(const uint4& xv, const float* W, int c0, float inv) {
  float xf[8], wv[8], n[8];
  unpack8(xv, xf);
  lds_get8(W, c0, wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) n[i] = (xf[i] * inv) * wv[i];
  return pack8(n);
}

// Split RoPE of one vector step: partner values come from lane l^8.
OGA_DEVICE uint4 rope8(const uint4& nv, const float* cs, const float* sn, bool second, bool cs_bf) {
  uint4 pv;
  pv.x = row_swap8(nv.x);
  pv.y = row_swap8(nv.y);
  pv.z = row_swap8(nv.z);
  pv.w = row_swap8(nv.w);
  float n[8], p[8], o[8];
  unpack8(nv, n);
  unpack8(pv, p);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float a = n[i] * cs[i];
    float b = p[i] * sn[i];
    if (cs_bf) {
      a = rbf(a);
      b = rbf(b);
    }
    o[i] = second ? a + b : a - b;
  }
  return pack8(o);
}

// Grid (blocks_per_batch, batch); a 4-wave workgroup stages the norm weights
// (and biases) in LDS as float, then each wave strides over token rows.
// ROPE false: the plain RMSNorm n = R(x * inv * w) (w = 1 without a weight),
// with no cos/sin and no partner exchange.
template <int CH, int NT, bool BIAS, bool PACK, int CDT, bool VEC, bool ROPE = true>
__global__ __launch_bounds__(256) void k_rmsnorm_rope(RopeArgs a) {
  constexpr int C = CH * 512;
  __shared__ float W0[C];
  __shared__ float W1[NT == 2 ? C : 1];
  __shared__ float B0[BIAS ? C : 1];
  __shared__ float B1[BIAS && NT == 2 ? C : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.y;
#pragma unroll 1
  for (int c0 = tid * 8; c0 < C; c0 += 256 * 8) {
    float v[8];
    if (ROPE || a.w0) {
      load8(a.w0, a.w_dt, c0, 1, true, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 1.0f;
    }
    lds_put8(W0, c0, v);
    if (NT == 2) {
      load8(a.w1, a.w_dt, c0, 1, true, v);
      lds_put8(W1, c0, v);
    }
    if (BIAS) {
      load8(a.b0, a.b_dt, c0, 1, true, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = rbf(v[i]);
      lds_put8(B0, c0, v);
      if (NT == 2) {
        load8(a.b1, a.b_dt, c0, 1, true, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = rbf(v[i]);
        lds_put8(B1, c0, v);
      }
    }
  }
  __syncthreads();

  const bool second = (lane & 8) != 0;
  const int hd0 = (lane & 7) * 8;
  constexpr bool cs_bf = CDT == OGA_DT_BF16;
  const int64_t step = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + w; t < a.tokens; t += step) {
    const int64_t r = b * a.tokens + t;
    uint4 x0[CH], x1[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) x0[j] = *(const uint4*)(a.x0 + r * C + j * 512 + lane * 8);
    if (NT == 2) {
#pragma unroll
      for (int j = 0; j < CH; ++j) x1[j] = *(const uint4*)(a.x1 + r * C + j * 512 + lane * 8);
    }
    if (BIAS) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        x0[j] = add_bias8(x0[j], B0, j * 512 + lane * 8);
        if (NT == 2) x1[j] = add_bias8(x1[j], B1, j * 512 + lane * 8);
      }
    }
    // cos/sin of every head this lane touches go out with q/k, as loaded.
    const int64_t cbase = b * a.c_sb + t * a.c_st + hd0;
    const int64_t sbase = b * a.s_sb + t * a.s_st + hd0;
    Raw8<CDT> cr[VEC ? CH : 1], sr[VEC ? CH : 1];
    if (ROPE && VEC) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int64_t head = j * 4 + (lane >> 4);
        cr[j] = raw8_load<CDT>(a.cos, cbase + head * a.c_sh);
        sr[j] = raw8_load<CDT>(a.sin, sbase + head * a.s_sh);
      }
    }
    const float inv0 = row_inv<CH>(x0, a.eps);
    const float inv1 = NT == 2 ? row_inv<CH>(x1, a.eps) : 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c0 = j * 512 + lane * 8;
      if constexpr (!ROPE) {
        st_nt16(a.o0 + r * a.out_stride + c0, norm8(x0[j], W0, c0, inv0));
        if (NT == 2) st_nt16(a.o1 + r * a.out_stride + c0, norm8(x1[j], W1, c0, inv1));
        __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      const int64_t head = j * 4 + (lane >> 4);
      float cs[8], sn[8];
      if (VEC) {
        raw8_get<CDT>(cr[VEC ? j : 0], cs);
        raw8_get<CDT>(sr[VEC ? j : 0], sn);
      } else {
        load8_t<CDT, false>(a.cos, cbase + head * a.c_sh, 1, cs);
        load8_t<CDT, false>(a.sin, sbase + head * a.s_sh, 1, sn);
      }
      st_nt16(a.o0 + r * a.out_stride + c0, rope8(norm8(x0[j], W0, c0, inv0), cs, sn, second, cs_bf));
      if (NT == 2)
        st_nt16(a.o1 + r * a.out_stride + c0, rope8(norm8(x1[j], W1, c0, inv1), cs, sn, second, cs_bf));
      if (PACK) st_nt16(a.ov + r * a.out_stride + c0, *(const uint4*)(a.v + r * C + c0));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int NT, bool BIAS, bool PACK>
static int launch_rope(RopeArgs& a, int64_t batch, hipStream_t st) {
  if (batch == 0 || a.tokens == 0) return OGA_OK;
  if (batch > 65535) return unsupported("batch > 65535");
  const dim3 grid = balanced_row_grid(batch, a.tokens);
  if (a.cols == 4096) {
    if (a.cs_dt == OGA_DT_BF16) {
      if (a.cs_vec)
        hipLaunchKernelGGL((k_rmsnorm_rope<8, NT, BIAS, PACK, OGA_DT_BF16, true>), grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((k_rmsnorm_rope<8, NT, BIAS, PACK, OGA_DT_BF16, false>), grid, dim3(256), 0, st, a);
    } else {
      if (a.cs_vec)
        hipLaunchKernelGGL((k_rmsnorm_rope<8, NT, BIAS, PACK, OGA_DT_F32, true>), grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((k_rmsnorm_rope<8, NT, BIAS, PACK, OGA_DT_F32, false>), grid, dim3(256), 0, st, a);
    }
  } else {
    if (a.cs_dt == OGA_DT_BF16) {
      if (a.cs_vec)
        hipLaunchKernelGGL((k_rmsnorm_rope<4, NT, BIAS, PACK, OGA_DT_BF16, true>), grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((k_rmsnorm_rope<4, NT, BIAS, PACK, OGA_DT_BF16, false>), grid, dim3(256), 0, st, a);
    } else {
      if (a.cs_vec)
        hipLaunchKernelGGL((k_rmsnorm_rope<4, NT, BIAS, PACK, OGA_DT_F32, true>), grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((k_rmsnorm_rope<4, NT, BIAS, PACK, OGA_DT_F32, false>), grid, dim3(256), 0, st, a);
    }
  }
  return launch_status();
}

static int rope_common(RopeArgs& a, const void* x0, const void* x1, const void* w0, const void* w1, int w_dt,
                       const void* cos, const void* sin, int cs_dt, const int64_t* cst, const int64_t* sst,
                       int64_t batch, int64_t tokens, int64_t cols, int64_t heads, float eps) {
  if (cols != 2048 && cols != 4096) return unsupported("cols must be 2048 or 4096");
  if (heads * 128 != cols) return unsupported("head_dim must be 128 (heads=%lld, cols=%lld)", (long long)heads,
                                              (long long)cols);
  if (batch < 0 || tokens < 0) return fail("bad shape");
  if (!x0 || !w0 || !cos || !sin || !cst || !sst) return fail("null pointer");
  if (!dt_ok(w_dt) || !dt_ok(cs_dt)) return fail("weight/cos dtype must be bf16 or f32");
  if (cst[3] != 1 || sst[3] != 1) return fail("cos/sin last stride must be 1");
  if (!aligned(x0, 16) || (x1 && !aligned(x1, 16))) return fail("q/k must be 16-byte aligned");
  if (!aligned(w0, 8 * dt_size(w_dt)) || (w1 && !aligned(w1, 8 * dt_size(w_dt))))
    return fail("weights must be aligned to 8 elements");
  a.x0 = (const uint16_t*)x0;
  a.x1 = (const uint16_t*)x1;
  a.w0 = w0;
  a.w1 = w1;
  a.w_dt = w_dt;
  a.cos = cos;
  a.sin = sin;
  a.cs_dt = cs_dt;
  a.c_sb = cst[0];
  a.c_sh = cst[1];
  a.c_st = cst[2];
  a.s_sb = sst[0];
  a.s_sh = sst[1];
  a.s_st = sst[2];
  a.cs_vec = vec8_ok(cos, cs_dt, a.c_sb, a.c_sh, a.c_st, 1) && vec8_ok(sin, cs_dt, a.s_sb, a.s_sh, a.s_st, 1);
  a.tokens = tokens;
  a.cols = (int)cols;
  a.out_stride = cols;
  a.eps = eps;
  return OGA_OK;
}

}  // namespace oga

using namespace oga;

extern "C" int oga_video_qk_rmsnorm_rope(const void* q, const void* k, const void* q_weight, const void* k_weight,
                                         int weight_dtype, const void* cos, const void* sin, int cs_dtype,
                                         const int64_t cos_strides[4], const int64_t sin_strides[4], void* q_out,
                                         void* k_out, int64_t batch, int64_t tokens, int64_t cols, int64_t heads,
                                         float eps, void* stream) {
  RopeArgs a{};
  if (!k || !k_weight || !q_out || !k_out) return fail("null pointer");
  int rc = rope_common(a, q, k, q_weight, k_weight, weight_dtype, cos, sin, cs_dtype, cos_strides, sin_strides,
                       batch, tokens, cols, heads, eps);
  if (rc) return rc;
  if (!aligned(q_out, 16) || !aligned(k_out, 16)) return fail("outputs must be 16-byte aligned");
  a.o0 = (uint16_t*)q_out;
  a.o1 = (uint16_t*)k_out;
  return launch_rope<2, false, false>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_video_rmsnorm_rope(const void* x, const void* weight, int weight_dtype, const void* cos,
                                      const void* sin, int cs_dtype, const int64_t cos_strides[4],
                                      const int64_t sin_strides[4], void* out, int64_t batch, int64_t tokens,
                                      int64_t cols, int64_t heads, float eps, void* stream) {
  RopeArgs a{};
  if (!out) return fail("null pointer");
  int rc = rope_common(a, x, nullptr, weight, nullptr, weight_dtype, cos, sin, cs_dtype, cos_strides, sin_strides,
                       batch, tokens, cols, heads, eps);
  if (rc) return rc;
  if (!aligned(out, 16)) return fail("output must be 16-byte aligned");
  a.o0 = (uint16_t*)out;
  return launch_rope<1, false, false>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_rmsnorm(const void* x, const void* weight, int weight_dtype, void* out, int64_t rows,
                           int64_t cols, float eps, void* stream) {
  RopeArgs a{};
  if (cols != 2048 && cols != 4096) return unsupported("cols must be 2048 or 4096");
  if (rows < 0) return fail("bad shape");
  if (!x || !out) return fail("null pointer");
  if (weight && !dt_ok(weight_dtype)) return fail("weight dtype must be bf16 or f32");
  if (!aligned(x, 16) || !aligned(out, 16)) return fail("x and out must be 16-byte aligned");
  if (weight && !aligned(weight, 8 * dt_size(weight_dtype))) return fail("weight must be aligned to 8 elements");
  if (rows == 0) return OGA_OK;
  a.x0 = (const uint16_t*)x;
  a.w0 = weight;
  a.w_dt = weight_dtype;
  a.o0 = (uint16_t*)out;
  a.tokens = rows;
  a.cols = (int)cols;
  a.out_stride = cols;
  a.eps = eps;
  const dim3 grid = balanced_row_grid(1, rows);
  if (cols == 4096)
    hipLaunchKernelGGL((k_rmsnorm_rope<8, 1, false, false, OGA_DT_BF16, false, false>), grid, dim3(256), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((k_rmsnorm_rope<4, 1, false, false, OGA_DT_BF16, false, false>), grid, dim3(256), 0,
                       (hipStream_t)stream, a);
  return launch_status();
}

extern "C" int oga_video_qk_bias_rmsnorm_rope(const void* q, const void* k, const void* q_bias, const void* k_bias,
                                              int bias_dtype, const void* q_weight, const void* k_weight,
                                              int weight_dtype, const void* cos, const void* sin, int cs_dtype,
                                              const int64_t cos_strides[4], const int64_t sin_strides[4],
                                              void* q_out, void* k_out, int64_t batch, int64_t tokens,
                                              int64_t cols, int64_t heads, float eps, void* stream) {
  RopeArgs a{};
  if (!k || !k_weight || !q_out || !k_out || !q_bias || !k_bias) return fail("null pointer");
  if (!dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  if (!aligned(q_bias, 8 * dt_size(bias_dtype)) || !aligned(k_bias, 8 * dt_size(bias_dtype)))
    return fail("biases must be aligned to 8 elements");
  int rc = rope_common(a, q, k, q_weight, k_weight, weight_dtype, cos, sin, cs_dtype, cos_strides, sin_strides,
                       batch, tokens, cols, heads, eps);
  if (rc) return rc;
  if (!aligned(q_out, 16) || !aligned(k_out, 16)) return fail("outputs must be 16-byte aligned");
  a.b0 = q_bias;
  a.b1 = k_bias;
  a.b_dt = bias_dtype;
  a.o0 = (uint16_t*)q_out;
  a.o1 = (uint16_t*)k_out;
  return launch_rope<2, true, false>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_video_qkv_rmsnorm_rope_pack(const void* q, const void* k, const void* v, const void* q_weight,
                                               const void* k_weight, int weight_dtype, const void* cos,
                                               const void* sin, int cs_dtype, const int64_t cos_strides[4],
                                               const int64_t sin_strides[4], void* qkv_out, int64_t batch,
                                               int64_t tokens, int64_t cols, int64_t heads, float eps,
                                               void* stream) {
  RopeArgs a{};
  if (!k || !v || !k_weight || !qkv_out) return fail("null pointer");
  if (!aligned(v, 16) || !aligned(qkv_out, 16)) return fail("v/qkv must be 16-byte aligned");
  int rc = rope_common(a, q, k, q_weight, k_weight, weight_dtype, cos, sin, cs_dtype, cos_strides, sin_strides,
                       batch, tokens, cols, heads, eps);
  if (rc) return rc;
  a.v = (const uint16_t*)v;
  a.o0 = (uint16_t*)qkv_out;
  a.o1 = (uint16_t*)qkv_out + cols;
  a.ov = (uint16_t*)qkv_out + 2 * cols;
  a.out_stride = 3 * cols;
  return launch_rope<2, false, true>(a, batch, (hipStream_t)stream);
}
