// Token-row kernels: AdaZero (RMSNorm + Ada scale/shift) and the Ada-gated
// elementwise fusions, for hidden sizes 2048 and 4096.
//
// Layout: one wavefront owns one token row at a time. Lane l of the wave owns
// columns {j*512 + 8l .. j*512 + 8l + 7 : j < C/512}, so every HBM access is
// a 128-bit load or store and the 64 lanes of one instruction cover 1 KiB of
// contiguous memory. Per-column constants (table rows, bias, and, when the
// timestep row is shared by all tokens, the finished Ada values) live in
// registers for all rows the wave processes. The RMS reduction is a per-lane
// float64 accumulation followed by a DPP/ds_swizzle butterfly.
//
// Reference semantics: ltx_serve/triton_ltx_ops.py :8-141 (AdaZero, AdaLN
// affine), :204-262 (residual gate + bias), :590-611 (residual gate),
// :640-739 (residual gate / mul from Ada), with the torch rounding chain of
// the fallbacks (:9-10, :50-60, :102-112, :214-228, :591-592, :650-659,
// :702-711, :983-998).
#include "common.h"
#include "host.h"

namespace oga {

// value(b, t, c) of one Ada index: R?ts(R?tab(table[c]) + ts[b, t, c]), or,
// with no table, the tensor ts itself (materialised scale/shift/gate).
struct AdaSrc {
  const void* tab;
  const void* ts;
  int64_t tab_off, tab_sc;
  int64_t ts_off, ts_sb, ts_st, ts_sc;
  int tab_dt, ts_dt;
  int tab_vec, ts_vec;
};

OGA_DEVICE bool round_tab(const AdaSrc& s) { return s.tab && s.tab_dt == OGA_DT_F32 && s.ts_dt == OGA_DT_BF16; }
OGA_DEVICE bool round_val(const AdaSrc& s) { return s.tab && s.ts_dt == OGA_DT_BF16; }

// Table part of 8 columns starting at col0 (already rounded if torch rounds).
OGA_DEVICE void ada_table8(const AdaSrc& s, int col0, float* t) {
  if (!s.tab) {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = 0.0f;
    return;
  }
  load8(s.tab, s.tab_dt, s.tab_off + (int64_t)col0 * s.tab_sc, s.tab_sc, s.tab_vec, t);
  if (round_tab(s)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = rbf(t[i]);
  }
}

// Finished Ada values for 8 columns of row (b, t), given the table part.
OGA_DEVICE void ada_value8(const AdaSrc& s, const float* tabv, int64_t b, int64_t t, int col0, float* v) {
  load8(s.ts, s.ts_dt, s.ts_off + b * s.ts_sb + t * s.ts_st + (int64_t)col0 * s.ts_sc, s.ts_sc, s.ts_vec, v);
  if (s.tab) {
    const bool r = round_val(s);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float a = tabv[i] + v[i];
      v[i] = r ? rbf(a) : a;
    }
  }
}

OGA_DEVICE int64_t wave_id() { return (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); }

// ------------------------------------------------------------------ AdaZero
struct AdaZeroArgs {
  const uint16_t* x;
  uint16_t* y;
  int64_t rows, tokens;
  int cols;
  float eps;
  int rows_per_wave;
  AdaSrc shift, scale;
};

// y = R( R?( n * R?(1 + scale) ) + shift ),  n = R(x * inv_rms)
// R? rounds iff the scale values are bf16 (torch: bf16 * bf16 -> bf16).
template <int CH, bool UNIFORM>
__global__ __launch_bounds__(256) void k_adazero(AdaZeroArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = wave_id() * a.rows_per_wave;
  if (r0 >= a.rows) return;
  const int64_t r1 = min(r0 + (int64_t)a.rows_per_wave, a.rows);
  const bool scale_bf = a.scale.ts_dt == OGA_DT_BF16;

  // UNIFORM: c0 = shift, c1 = R?(1 + scale), finished per column for batch cb.
  // Otherwise: c0/c1 hold the table parts of shift/scale.
  float c0[CH][8], c1[CH][8];
  int64_t cb = -1;
  if (!UNIFORM) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      ada_table8(a.shift, j * 512 + lane * 8, c0[j]);
      ada_table8(a.scale, j * 512 + lane * 8, c1[j]);
    }
  }

  for (int64_t r = r0; r < r1; ++r) {
    const int64_t b = r / a.tokens;
    const int64_t t = r - b * a.tokens;
    uint4 xv[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) xv[j] = *(const uint4*)(a.x + r * a.cols + j * 512 + lane * 8);

    if (UNIFORM && b != cb) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        float tab[8];
        const int col0 = j * 512 + lane * 8;
        ada_table8(a.shift, col0, tab);
        ada_value8(a.shift, tab, b, 0, col0, c0[j]);
        ada_table8(a.scale, col0, tab);
        ada_value8(a.scale, tab, b, 0, col0, c1[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float f = 1.0f + c1[j][i];
          c1[j][i] = scale_bf ? rbf(f) : f;
        }
      }
      cb = b;
    }

    double ss = 0.0;
    float xf[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      unpack8(xv[j], xf[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const double d = (double)xf[j][i];
        ss = fma(d, d, ss);
      }
    }
    const float inv = rms_inv(ss, a.cols, a.eps);

#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int col0 = j * 512 + lane * 8;
      float sh[8], f[8];
      if (UNIFORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) { sh[i] = c0[j][i]; f[i] = c1[j][i]; }
      } else {
        ada_value8(a.shift, c0[j], b, t, col0, sh);
        ada_value8(a.scale, c1[j], b, t, col0, f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = 1.0f + f[i];
          f[i] = scale_bf ? rbf(v) : v;
        }
      }
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float n = rbf(xf[j][i] * inv);
        float p = n * f[i];
        if (scale_bf) p = rbf(p);
        o[i] = p + sh[i];
      }
      *(uint4*)(a.y + r * a.cols + col0) = pack8(o);
    }
  }
}

// ---------------------------------------------------- Ada-gated elementwise
enum EwOp { EW_ADALN = 0, EW_MUL = 1, EW_RESID = 2, EW_RESID_BIAS = 3 };

struct EwArgs {
  const uint16_t* x;
  const uint16_t* y;
  uint16_t* out;
  const void* bias;
  int bias_dt;
  int64_t rows, tokens;
  int cols;
  int rows_per_wave;
  AdaSrc s0;  // shift (ADALN) or gate
  AdaSrc s1;  // scale (ADALN only)
};

// ADALN:      out = R( R?(x * R?(1 + scale)) + shift )
// MUL:        out = R( x * gate )
// RESID:      out = R( x + R?(y * gate) )
// RESID_BIAS: out = R( x + R?(R(y + R(bias)) * gate) )
// R? rounds iff the Ada values are bf16.
template <int CH, int OP, bool UNIFORM>
__global__ __launch_bounds__(256) void k_ada_ew(EwArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = wave_id() * a.rows_per_wave;
  if (r0 >= a.rows) return;
  const int64_t r1 = min(r0 + (int64_t)a.rows_per_wave, a.rows);
  const bool v_bf = a.s0.ts_dt == OGA_DT_BF16;
  const bool f_bf = a.s1.ts_dt == OGA_DT_BF16;

  // UNIFORM: c0/c1 are finished values (gate, or shift and R?(1+scale)).
  // Otherwise: table parts.
  float c0[CH][8], c1[CH][8], bi[CH][8];
  int64_t cb = -1;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int col0 = j * 512 + lane * 8;
    if (!UNIFORM) {
      ada_table8(a.s0, col0, c0[j]);
      if (OP == EW_ADALN) ada_table8(a.s1, col0, c1[j]);
    }
    if (OP == EW_RESID_BIAS) {
      load8(a.bias, a.bias_dt, col0, 1, true, bi[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) bi[j][i] = rbf(bi[j][i]);
    }
  }

  for (int64_t r = r0; r < r1; ++r) {
    const int64_t b = r / a.tokens;
    const int64_t t = r - b * a.tokens;
    uint4 xv[CH], yv[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      xv[j] = *(const uint4*)(a.x + r * a.cols + j * 512 + lane * 8);
      if (OP == EW_RESID || OP == EW_RESID_BIAS) yv[j] = *(const uint4*)(a.y + r * a.cols + j * 512 + lane * 8);
    }
    if (UNIFORM && b != cb) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        float tab[8];
        const int col0 = j * 512 + lane * 8;
        ada_table8(a.s0, col0, tab);
        ada_value8(a.s0, tab, b, 0, col0, c0[j]);
        if (OP == EW_ADALN) {
          ada_table8(a.s1, col0, tab);
          ada_value8(a.s1, tab, b, 0, col0, c1[j]);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float f = 1.0f + c1[j][i];
            c1[j][i] = f_bf ? rbf(f) : f;
          }
        }
      }
      cb = b;
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int col0 = j * 512 + lane * 8;
      float g[8], f[8];
      if (UNIFORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) { g[i] = c0[j][i]; f[i] = c1[j][i]; }
      } else {
        ada_value8(a.s0, c0[j], b, t, col0, g);
        if (OP == EW_ADALN) {
          ada_value8(a.s1, c1[j], b, t, col0, f);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float v = 1.0f + f[i];
            f[i] = f_bf ? rbf(v) : v;
          }
        }
      }
      float xf[8], yf[8], o[8];
      unpack8(xv[j], xf);
      if (OP == EW_RESID || OP == EW_RESID_BIAS) unpack8(yv[j], yf);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (OP == EW_ADALN) {
          float p = xf[i] * f[i];
          if (f_bf) p = rbf(p);
          o[i] = p + g[i];
        } else if (OP == EW_MUL) {
          o[i] = xf[i] * g[i];
        } else {
          float yy = yf[i];
          if (OP == EW_RESID_BIAS) yy = rbf(yy + bi[j][i]);
          float p = yy * g[i];
          if (v_bf) p = rbf(p);
          o[i] = xf[i] + p;
        }
      }
      *(uint4*)(a.out + r * a.cols + col0) = pack8(o);
    }
  }
}

// ------------------------------------------------- generic-width elementwise
// out = R(x + R(bias[col])) for any (rows, cols); 8 elements per thread when
// cols % 8 == 0 (128-bit path), element-wise otherwise.
__global__ __launch_bounds__(256) void k_bias_add(const uint16_t* x, const void* bias, int bias_dt, uint16_t* out,
                                                  int64_t n, int64_t cols, int vec) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 >= n) return;
  if (vec) {
    const int64_t col = i0 % cols;
    float xf[8], bf[8], o[8];
    unpack8(*(const uint4*)(x + i0), xf);
    load8(bias, bias_dt, col, 1, true, bf);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = xf[i] + rbf(bf[i]);
    *(uint4*)(out + i0) = pack8(o);
  } else {
    for (int64_t i = i0; i < min(i0 + 8, n); ++i) {
      const int64_t col = i % cols;
      float bv = bias_dt == OGA_DT_BF16 ? __uint_as_float(((uint32_t)((const uint16_t*)bias)[col]) << 16)
                                        : ((const float*)bias)[col];
      float o = __uint_as_float(((uint32_t)x[i]) << 16) + rbf(bv);
      out[i] = (uint16_t)(pack_bf16(o, 0.0f) & 0xFFFF);
    }
  }
}

// out[r, h*D + d] = R(x[r, h*D + d] * gate[r*g0 + h*g1])
__global__ __launch_bounds__(256) void k_head_gate_mul(const uint16_t* x, const uint16_t* gates, int64_t g0,
                                                       int64_t g1, uint16_t* out, int64_t n, int64_t cols,
                                                       int64_t dim_head, int vec) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 >= n) return;
  const int64_t hi = min(i0 + 8, n);
  if (vec) {  // 8 elements in one row and one head (dim_head % 8 == 0)
    const int64_t r = i0 / cols, c = i0 - (i0 / cols) * cols;
    const float g = __uint_as_float(((uint32_t)gates[r * g0 + (c / dim_head) * g1]) << 16);
    float xf[8], o[8];
    unpack8(*(const uint4*)(x + i0), xf);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = xf[i] * g;
    *(uint4*)(out + i0) = pack8(o);
  } else {
    for (int64_t i = i0; i < hi; ++i) {
      const int64_t r = i / cols, c = i - (i / cols) * cols;
      const float g = __uint_as_float(((uint32_t)gates[r * g0 + (c / dim_head) * g1]) << 16);
      const float o = __uint_as_float(((uint32_t)x[i]) << 16) * g;
      out[i] = (uint16_t)(pack_bf16(o, 0.0f) & 0xFFFF);
    }
  }
}

// ------------------------------------------------------------------- host
static bool valid_ada_inputs(int64_t batch, int64_t tokens, int64_t cols) {
  return batch >= 0 && tokens >= 0 && (cols == 2048 || cols == 4096);
}

static int make_ada_src(AdaSrc& s, const void* table, int tab_dt, int64_t tab_s0, int64_t tab_s1, const void* ts,
                        int ts_dt, const int64_t* st4, int index, int64_t params) {
  if (!dt_ok(tab_dt) || !dt_ok(ts_dt)) return fail("table/timestep dtype must be bf16 or f32");
  if (index < 0 || index >= params) return fail("Ada index %d out of range for a table with %lld rows", index,
                                               (long long)params);
  if (!table || !ts || !st4) return fail("null table/timestep");
  s.tab = table;
  s.tab_dt = tab_dt;
  s.tab_off = (int64_t)index * tab_s0;
  s.tab_sc = tab_s1;
  s.tab_vec = vec8_ok(table, tab_dt, s.tab_off, 0, 0, tab_s1);
  s.ts = ts;
  s.ts_dt = ts_dt;
  s.ts_off = (int64_t)index * st4[2];
  s.ts_sb = st4[0];
  s.ts_st = st4[1];
  s.ts_sc = st4[3];
  s.ts_vec = vec8_ok(ts, ts_dt, s.ts_off, s.ts_sb, s.ts_st, s.ts_sc);
  return OGA_OK;
}

static void make_direct_src(AdaSrc& s, const void* p, int dt, const int64_t* st3) {
  s.tab = nullptr;
  s.tab_dt = OGA_DT_F32;
  s.tab_off = 0;
  s.tab_sc = 0;
  s.tab_vec = 0;
  s.ts = p;
  s.ts_dt = dt;
  s.ts_off = 0;
  s.ts_sb = st3[0];
  s.ts_st = st3[1];
  s.ts_sc = st3[2];
  s.ts_vec = vec8_ok(p, dt, 0, s.ts_sb, s.ts_st, s.ts_sc);
}

// Rows per wave: one row per wave until every SIMD holds four waves; beyond
// that a wave takes several rows, which amortises the per-column constants.
static int rows_per_wave_for(int64_t rows) {
  const int64_t target_waves = (int64_t)cu_count() * 4 * 4;
  int64_t rpw = (rows + target_waves - 1) / target_waves;
  if (rpw < 1) rpw = 1;
  if (rpw > 64) rpw = 64;
  return (int)rpw;
}

static dim3 row_grid(int64_t rows, int rpw) {
  const int64_t waves = (rows + rpw - 1) / rpw;
  return dim3((unsigned)((waves + 3) / 4));
}

template <int CH>
static int launch_adazero(AdaZeroArgs& a, bool uniform, hipStream_t st) {
  const dim3 grid = row_grid(a.rows, a.rows_per_wave);
  if (uniform)
    hipLaunchKernelGGL((k_adazero<CH, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_adazero<CH, false>), grid, dim3(256), 0, st, a);
  return launch_status();
}

static int run_adazero(AdaZeroArgs& a, hipStream_t st) {
  if (a.rows == 0) return OGA_OK;
  a.rows_per_wave = rows_per_wave_for(a.rows);
  const bool uniform = a.shift.ts_st == 0 && a.scale.ts_st == 0;
  return a.cols == 4096 ? launch_adazero<8>(a, uniform, st) : launch_adazero<4>(a, uniform, st);
}

template <int CH, int OP>
static int launch_ew_ch(EwArgs& a, bool uniform, hipStream_t st) {
  const dim3 grid = row_grid(a.rows, a.rows_per_wave);
  if (uniform)
    hipLaunchKernelGGL((k_ada_ew<CH, OP, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_ada_ew<CH, OP, false>), grid, dim3(256), 0, st, a);
  return launch_status();
}

template <int OP>
static int run_ew(EwArgs& a, hipStream_t st) {
  if (a.rows == 0) return OGA_OK;
  a.rows_per_wave = rows_per_wave_for(a.rows);
  const bool uniform = a.s0.ts_st == 0 && (OP != EW_ADALN || a.s1.ts_st == 0);
  return a.cols == 4096 ? launch_ew_ch<8, OP>(a, uniform, st) : launch_ew_ch<4, OP>(a, uniform, st);
}

static int check_rows(const void* x, const void* y, int64_t batch, int64_t tokens, int64_t cols) {
  if (!valid_ada_inputs(batch, tokens, cols)) return unsupported("cols must be 2048 or 4096 (got %lld)", (long long)cols);
  if (!x || !y) return fail("null x/out");
  if (!aligned(x, 16) || !aligned(y, 16)) return fail("x/out must be 16-byte aligned");
  return OGA_OK;
}

}  // namespace oga

using namespace oga;

extern "C" int oga_adazero_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                    const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                    const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                    int shift_index, int scale_index, float eps, void* stream) {
  int rc = check_rows(x, y, batch, tokens, cols);
  if (rc) return rc;
  AdaZeroArgs a{};
  a.x = (const uint16_t*)x;
  a.y = (uint16_t*)y;
  a.rows = batch * tokens;
  a.tokens = tokens;
  a.cols = (int)cols;
  a.eps = eps;
  const int64_t params = INT64_MAX;
  if ((rc = make_ada_src(a.shift, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, params))) return rc;
  if ((rc = make_ada_src(a.scale, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, params))) return rc;
  return run_adazero(a, (hipStream_t)stream);
}

extern "C" int oga_adazero(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols, const void* scale,
                           int scale_dtype, const int64_t scale_strides[3], const void* shift, int shift_dtype,
                           const int64_t shift_strides[3], float eps, void* stream) {
  int rc = check_rows(x, y, batch, tokens, cols);
  if (rc) return rc;
  if (!scale || !shift || !scale_strides || !shift_strides) return fail("null scale/shift");
  if (!dt_ok(scale_dtype) || !dt_ok(shift_dtype)) return fail("scale/shift dtype must be bf16 or f32");
  AdaZeroArgs a{};
  a.x = (const uint16_t*)x;
  a.y = (uint16_t*)y;
  a.rows = batch * tokens;
  a.tokens = tokens;
  a.cols = (int)cols;
  a.eps = eps;
  make_direct_src(a.shift, shift, shift_dtype, shift_strides);
  make_direct_src(a.scale, scale, scale_dtype, scale_strides);
  return run_adazero(a, (hipStream_t)stream);
}

static int ew_common(EwArgs& a, const void* x, const void* y, void* out, int64_t batch, int64_t tokens, int64_t cols) {
  int rc = check_rows(x, out, batch, tokens, cols);
  if (rc) return rc;
  if (y && !aligned(y, 16)) return fail("y must be 16-byte aligned");
  a.x = (const uint16_t*)x;
  a.y = (const uint16_t*)y;
  a.out = (uint16_t*)out;
  a.rows = batch * tokens;
  a.tokens = tokens;
  a.cols = (int)cols;
  return OGA_OK;
}

extern "C" int oga_adaln_affine_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                         const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                         const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                         int shift_index, int scale_index, void* stream) {
  EwArgs a{};
  int rc = ew_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s1, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, INT64_MAX))) return rc;
  return run_ew<EW_ADALN>(a, (hipStream_t)stream);
}

extern "C" int oga_mul_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                const void* timestep, int ts_dtype, const int64_t ts_strides[4], int gate_index,
                                void* stream) {
  EwArgs a{};
  int rc = ew_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_ew<EW_MUL>(a, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_from_ada(const void* x, const void* y, void* out, int64_t batch, int64_t tokens,
                                          int64_t cols, const void* table, int table_dtype, int64_t tab_s0,
                                          int64_t tab_s1, const void* timestep, int ts_dtype,
                                          const int64_t ts_strides[4], int gate_index, void* stream) {
  EwArgs a{};
  if (!y) return fail("null y");
  int rc = ew_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_ew<EW_RESID>(a, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_bias_from_ada(const void* x, const void* y, const void* bias, int bias_dtype,
                                               void* out, int64_t batch, int64_t tokens, int64_t cols,
                                               const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                               const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                               int gate_index, void* stream) {
  EwArgs a{};
  if (!y || !bias) return fail("null y/bias");
  if (!dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  if (!aligned(bias, 32)) return fail("bias must be 32-byte aligned");
  int rc = ew_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  a.bias = bias;
  a.bias_dt = bias_dtype;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_ew<EW_RESID_BIAS>(a, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_bf16(const void* x, const void* y, const void* gate, const int64_t gate_strides[3],
                                      void* out, int64_t batch, int64_t tokens, int64_t cols, void* stream) {
  EwArgs a{};
  if (!y || !gate || !gate_strides) return fail("null y/gate");
  int rc = ew_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  make_direct_src(a.s0, gate, OGA_DT_BF16, gate_strides);
  a.s1 = a.s0;
  return run_ew<EW_RESID>(a, (hipStream_t)stream);
}

extern "C" int oga_bias_add_bf16(const void* x, const void* bias, int bias_dtype, void* out, int64_t rows,
                                 int64_t cols, void* stream) {
  if (!x || !bias || !out) return fail("null pointer");
  if (!dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  if (rows < 0 || cols <= 0) return fail("bad shape");
  const int64_t n = rows * cols;
  if (n == 0) return OGA_OK;
  const int vec = (cols % 8 == 0) && aligned(x, 16) && aligned(out, 16) && aligned(bias, 8 * dt_size(bias_dtype));
  const int64_t threads = (n + 7) / 8;
  hipLaunchKernelGGL(k_bias_add, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, bias, bias_dtype, (uint16_t*)out, n, cols, vec);
  return launch_status();
}

extern "C" int oga_head_gate_mul_bf16(const void* x, const void* gates, int64_t g_s0, int64_t g_s1, void* out,
                                      int64_t rows, int64_t heads, int64_t dim_head, void* stream) {
  if (!x || !gates || !out) return fail("null pointer");
  if (rows < 0 || heads <= 0 || dim_head <= 0) return fail("bad shape");
  const int64_t cols = heads * dim_head;
  const int64_t n = rows * cols;
  if (n == 0) return OGA_OK;
  const int vec = (dim_head % 8 == 0) && aligned(x, 16) && aligned(out, 16);
  const int64_t threads = (n + 7) / 8;
  hipLaunchKernelGGL(k_head_gate_mul, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)gates, g_s0, g_s1, (uint16_t*)out, n, cols, dim_head, vec);
  return launch_status();
}
