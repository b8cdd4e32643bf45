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
  int64_t rows, tokens;
  int cols;
  int w_dt, b_dt, cs_dt;
  int cs_vec;
  int rows_per_wave;
  float eps;
};

OGA_DEVICE int64_t rope_wave_id() { return (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); }

// Normalised (and weight-scaled) row of one tensor as packed bf16 pairs.
template <int CH, bool BIAS>
OGA_DEVICE void norm_row(const uint16_t* x, const void* w, int w_dt, const void* bias, int b_dt, int64_t r,
                         int cols, float eps, int lane, uint4* nv) {
  float xf[CH][8];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const uint4 u = *(const uint4*)(x + r * cols + j * 512 + lane * 8);
    unpack8(u, xf[j]);
    if (BIAS) {
      float bv[8];
      load8(bias, b_dt, j * 512 + lane * 8, 1, true, bv);
#pragma unroll
      for (int i = 0; i < 8; ++i) xf[j][i] = rbf(xf[j][i] + rbf(bv[i]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double d = (double)xf[j][i];
      ss = fma(d, d, ss);
    }
  }
  const float inv = rms_inv(ss, cols, eps);
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    float wv[8], n[8];
    load8(w, w_dt, j * 512 + lane * 8, 1, true, wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = (xf[j][i] * inv) * wv[i];
    nv[j] = pack8(n);
  }
}

template <int CH>
OGA_DEVICE void rope_row(const uint4* nv, const float (*cs)[8], const float (*sn)[8], bool second, bool cs_bf,
                         uint16_t* out, int lane) {
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    uint4 pv;
    pv.x = row_swap8(nv[j].x);
    pv.y = row_swap8(nv[j].y);
    pv.z = row_swap8(nv[j].z);
    pv.w = row_swap8(nv[j].w);
    float n[8], p[8], o[8];
    unpack8(nv[j], n);
    unpack8(pv, p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float a = n[i] * cs[j][i];
      float b = p[i] * sn[j][i];
      if (cs_bf) {
        a = rbf(a);
        b = rbf(b);
      }
      o[i] = second ? a + b : a - b;
    }
    *(uint4*)(out + j * 512 + lane * 8) = pack8(o);
  }
}

template <int CH, int NT, bool BIAS, bool PACK>
__global__ __launch_bounds__(256) void k_rmsnorm_rope(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = rope_wave_id() * a.rows_per_wave;
  if (r0 >= a.rows) return;
  const int64_t r1 = min(r0 + (int64_t)a.rows_per_wave, a.rows);
  const bool second = (lane & 8) != 0;
  const int hd0 = (lane & 7) * 8;
  const bool cs_bf = a.cs_dt == OGA_DT_BF16;

  for (int64_t r = r0; r < r1; ++r) {
    const int64_t b = r / a.tokens;
    const int64_t t = r - b * a.tokens;

    float cs[CH][8], sn[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int64_t head = j * 4 + (lane >> 4);
      load8(a.cos, a.cs_dt, b * a.c_sb + head * a.c_sh + t * a.c_st + hd0, 1, a.cs_vec, cs[j]);
      load8(a.sin, a.cs_dt, b * a.s_sb + head * a.s_sh + t * a.s_st + hd0, 1, a.cs_vec, sn[j]);
    }

    uint4 nv[CH];
    norm_row<CH, BIAS>(a.x0, a.w0, a.w_dt, a.b0, a.b_dt, r, a.cols, a.eps, lane, nv);
    rope_row<CH>(nv, cs, sn, second, cs_bf, a.o0 + r * a.out_stride, lane);
    if (NT == 2) {
      norm_row<CH, BIAS>(a.x1, a.w1, a.w_dt, a.b1, a.b_dt, r, a.cols, a.eps, lane, nv);
      rope_row<CH>(nv, cs, sn, second, cs_bf, a.o1 + r * a.out_stride, lane);
    }
    if (PACK) {
#pragma unroll
      for (int j = 0; j < CH; ++j)
        *(uint4*)(a.ov + r * a.out_stride + j * 512 + lane * 8) =
            *(const uint4*)(a.v + r * a.cols + j * 512 + lane * 8);
    }
  }
}

template <int NT, bool BIAS, bool PACK>
static int launch_rope(RopeArgs& a, hipStream_t st) {
  if (a.rows == 0) return OGA_OK;
  const int64_t target_waves = (int64_t)cu_count() * 16;
  int64_t rpw = (a.rows + target_waves - 1) / target_waves;
  a.rows_per_wave = (int)(rpw < 1 ? 1 : (rpw > 64 ? 64 : rpw));
  const int64_t waves = (a.rows + a.rows_per_wave - 1) / a.rows_per_wave;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (a.cols == 4096)
    hipLaunchKernelGGL((k_rmsnorm_rope<8, NT, BIAS, PACK>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_rmsnorm_rope<4, NT, BIAS, PACK>), grid, dim3(256), 0, st, a);
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
  a.rows = batch * tokens;
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
  return launch_rope<2, false, false>(a, (hipStream_t)stream);
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
  return launch_rope<1, false, false>(a, (hipStream_t)stream);
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
  return launch_rope<2, true, false>(a, (hipStream_t)stream);
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
  return launch_rope<2, false, true>(a, (hipStream_t)stream);
}
