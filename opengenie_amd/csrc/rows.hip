// Token-row kernels: AdaZero (RMSNorm + Ada scale/shift) and the Ada-gated
// elementwise fusions, for hidden sizes 2048 and 4096.
//
// Layout: every HBM access is a 128-bit load or store of 8 consecutive
// columns, and the 64 lanes of one instruction cover 1 KiB of contiguous
// memory. Per-column constants (table rows, bias, and, when the timestep row
// is shared by all tokens, the finished Ada values) are computed once per
// wave or workgroup into registers. k_elem (no row reduction) streams whole
// rows per workgroup with several rows' loads in flight and no LDS;
// k_adazero_rows gives each token row to one wave (its reduction stays in
// the wave), with the Ada constants computed once per workgroup in LDS;
// k_adazero_gather serves operands that cannot be read 16 bytes at a time.
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

// ------------------------------------------------------------- row ops
// One family for AdaZero and the Ada-gated elementwise ops:
//   ADAZERO:    y = R( R?(n * R?(1 + scale)) + shift ),  n = R(x * inv_rms)
//   ADALN:      y = R( R?(x * R?(1 + scale)) + shift )
//   MUL:        y = R( x * gate )
//   RESID:      y = R( x + R?(y_in * gate) )
//   RESID_BIAS: y = R( x + R?(R(y_in + R(bias)) * gate) )
// R? rounds iff the Ada values are bf16 (torch: bf16 op bf16 -> bf16).
// s0 is the shift (ADAZERO/ADALN) or the gate; s1 the scale.
enum RowOp { OP_ADAZERO = 0, OP_ADALN = 1, OP_MUL = 2, OP_RESID = 3, OP_RESID_BIAS = 4 };

struct RowArgs {
  const uint16_t* x;
  const uint16_t* y;
  uint16_t* out;
  const void* bias;
  int bias_dt;
  int64_t tokens;
  int cols;
  float eps;
  AdaSrc s0, s1;
  // AdaZero with e4m3 output (out then holds one byte per element): the
  // input quantizer of the FP8 linear that follows, with its scale.
  int q8;
  const float* qscale;
  int q_zero_dim;
  // AdaZero after a residual gate (k_adazero_rows with RES): the gate's Ada
  // source and the residual output x' = R(x + R?(y_in * gate)); the AdaZero
  // then normalises x'.
  AdaSrc s2;
  uint16_t* xout;
};

template <int OP>
struct RowTraits {
  static constexpr bool kTwo = OP == OP_ADAZERO || OP == OP_ADALN;  // uses s1
  static constexpr bool kY = OP == OP_RESID || OP == OP_RESID_BIAS;
  static constexpr bool kBias = OP == OP_RESID_BIAS;
};

// ------------------------------------------------------ elementwise ops
// The Ada ops with no row reduction (AdaLN affine, mul, residual gates).
// A workgroup (256 lanes) streams whole token rows of one batch: lane i
// covers the CH/4 vectors i, i + 256, ... of a row (columns 8i .. 8i+7,
// 2048 + 8i .. for 4096 columns), so the workgroup reads and writes each row
// as one contiguous piece, and at any moment the grid's accesses fall in a
// narrow window of rows (few DRAM pages open). Workgroup x takes rows
// kElemRows*x .. +kElemRows-1, then the same rows gridDim.x*kElemRows
// further on, with every load of those rows in flight together. The
// per-column constants (the table rows, the bias, and the finished Ada
// values when the timestep row is shared by all tokens) are computed once
// per workgroup into registers. No LDS, no barrier. Measured at 14080 x
// 4096 with per-token timesteps: 1 row at a time and 32 workgroups per CU
// (75-76 us) against 2 or 4 rows and 8 or 16 workgroups (75-79 us), and
// 80 us for waves that each stream one 1 KiB chunk of 14 consecutive rows.
#ifndef OGA_ELEM_ROWS_IN_FLIGHT
#define OGA_ELEM_ROWS_IN_FLIGHT 1
#endif
#ifndef OGA_ELEM_WG_PER_CU
#define OGA_ELEM_WG_PER_CU 32
#endif
constexpr int kElemRows = OGA_ELEM_ROWS_IN_FLIGHT;
template <int CH, int OP, bool UNIFORM, int D0, int D1, bool VEC>
__global__ __launch_bounds__(256) void k_elem(RowArgs a) {
  using Tr = RowTraits<OP>;
  constexpr int C = CH * 512;
  constexpr int H = CH / 4;  // vectors per lane and row
  constexpr bool B0 = D0 == OGA_DT_BF16;
  constexpr bool B1 = D1 == OGA_DT_BF16;
  constexpr int U = kElemRows;
  const int64_t b = blockIdx.y;
  int col[H];
#pragma unroll
  for (int h = 0; h < H; ++h) col[h] = (h * 256 + (int)threadIdx.x) * 8;

  const bool tab0 = a.s0.tab != nullptr;
  const bool tab1 = a.s1.tab != nullptr;
  float c0[H][8], c1[H][8], bb[H][8];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    ada_table8(a.s0, col[h], c0[h]);
    if (Tr::kTwo) ada_table8(a.s1, col[h], c1[h]);
    if (UNIFORM) {
      float v[8];
      ada_value8(a.s0, c0[h], b, 0, col[h], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) c0[h][i] = v[i];
      if (Tr::kTwo) {
        ada_value8(a.s1, c1[h], b, 0, col[h], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float f = 1.0f + v[i];
          c1[h][i] = B1 ? rbf(f) : f;
        }
      }
    }
    if (Tr::kBias) {
      load8(a.bias, a.bias_dt, col[h], 1, true, bb[h]);
#pragma unroll
      for (int i = 0; i < 8; ++i) bb[h][i] = rbf(bb[h][i]);
    }
  }

  const int64_t ts0 = a.s0.ts_off + b * a.s0.ts_sb;
  const int64_t ts1 = a.s1.ts_off + b * a.s1.ts_sb;
  constexpr bool kPre = !UNIFORM && VEC;
  for (int64_t t0 = (int64_t)blockIdx.x * U; t0 < a.tokens; t0 += (int64_t)gridDim.x * U) {
    uint4 xv[U][H], yv[U][H];
    Raw8<D0> p0[U][H];
    Raw8<D1> p1[U][H];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u;
      if (t < a.tokens) {
        const int64_t r = b * a.tokens + t;
#pragma unroll
        for (int h = 0; h < H; ++h) {
          xv[u][h] = *(const uint4*)(a.x + r * C + col[h]);
          if (Tr::kY) yv[u][h] = *(const uint4*)(a.y + r * C + col[h]);
          if (kPre) {
            p0[u][h] = raw8_load<D0>(a.s0.ts, ts0 + t * a.s0.ts_st + col[h]);
            if (Tr::kTwo) p1[u][h] = raw8_load<D1>(a.s1.ts, ts1 + t * a.s1.ts_st + col[h]);
          }
        }
      }
    }
    // Every load of the group issued before any use (the scheduler may
    // otherwise sink one into the arithmetic, which then waits for it alone).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = t0 + u;
      if (t >= a.tokens) break;
      const int64_t r = b * a.tokens + t;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float v0[8], v1[8], xf[8], o[8];
        if (UNIFORM) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            v0[i] = c0[h][i];
            v1[i] = Tr::kTwo ? c1[h][i] : 0.0f;
          }
        } else {
          float tsv[8];
          if (kPre) raw8_get<D0>(p0[u][h], tsv);
          else load8_t<D0, false>(a.s0.ts, ts0 + t * a.s0.ts_st + (int64_t)col[h] * a.s0.ts_sc, a.s0.ts_sc, tsv);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float sum = tab0 ? c0[h][i] + tsv[i] : tsv[i];
            v0[i] = (tab0 && B0) ? rbf(sum) : sum;
          }
          if (Tr::kTwo) {
            if (kPre) raw8_get<D1>(p1[u][h], tsv);
            else load8_t<D1, false>(a.s1.ts, ts1 + t * a.s1.ts_st + (int64_t)col[h] * a.s1.ts_sc, a.s1.ts_sc, tsv);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              float sum = tab1 ? c1[h][i] + tsv[i] : tsv[i];
              if (tab1 && B1) sum = rbf(sum);
              const float f = 1.0f + sum;
              v1[i] = B1 ? rbf(f) : f;
            }
          }
        }
        unpack8(xv[u][h], xf);
        if (OP == OP_ADALN) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float p = xf[i] * v1[i];
            if (B1) p = rbf(p);
            o[i] = p + v0[i];
          }
        } else if (OP == OP_MUL) {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = xf[i] * v0[i];
        } else {
          float yf[8];
          unpack8(yv[u][h], yf);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float yy = yf[i];
            if (Tr::kBias) yy = rbf(yy + bb[h][i]);
            float p = yy * v0[i];
            if (B0) p = rbf(p);
            o[i] = xf[i] + p;
          }
        }
        st_nt16(a.out + r * C + col[h], pack8(o));
      }
    }
  }
}

// ------------------------------------------------------- AdaZero (gather)
// The form of AdaZero for operands that cannot be read 16 bytes at a time
// (a column stride other than 1, or misaligned rows); see k_adazero_rows
// for the vectorised form.
// y = R(R?(R(x * inv_rms) * R?(1 + scale)) + shift). A workgroup of CH waves
// streams a run of consecutive token rows; wave w owns columns w*512 + 8l ..
// +7 of every row. Each wave keeps the loads of the next kAdaAhead rows in
// flight while it finishes the current one (the first ones go out before
// the Ada constants are computed), so a workgroup's reads of later rows
// overlap its writes of earlier ones. Per row a wave adds up the squares
// of its chunk (float64: squares of bf16 values are exact), and after one
// barrier every wave combines the CH partial sums of the row (double-
// buffered in LDS: a wave writes the partials of row u + 2 only after the
// barrier of row u + 1, which every wave reaches after reading those of row
// u) into the row's normaliser and writes its chunk.
#ifndef OGA_ADA_AHEAD
#define OGA_ADA_AHEAD 2
#endif
constexpr int kAdaAhead = OGA_ADA_AHEAD;
static_assert(kAdaAhead >= 1 && kAdaAhead <= 4, "prefetch depth");
template <int CH, bool UNIFORM, int D0, int D1, bool VEC>
__global__ __launch_bounds__(512) void k_adazero_gather(RowArgs a, int rows_per_wg) {
  constexpr int C = CH * 512;
  constexpr bool B1 = D1 == OGA_DT_BF16;
  constexpr bool B0 = D0 == OGA_DT_BF16;
  __shared__ double part[2][CH];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t b = blockIdx.y;
  const int col0 = wv * 512 + lane * 8;
  const int64_t t0 = (int64_t)blockIdx.x * rows_per_wg;
  const int nr = (int)min((int64_t)rows_per_wg, a.tokens - t0);  // >= 1 by the grid
  const int64_t tsc0 = a.s0.ts_off + b * a.s0.ts_sb + (int64_t)col0 * a.s0.ts_sc;
  const int64_t tsc1 = a.s1.ts_off + b * a.s1.ts_sb + (int64_t)col0 * a.s1.ts_sc;
  constexpr bool kPre = !UNIFORM && VEC;
  const uint16_t* const xrow = a.x + (b * a.tokens + t0) * C + col0;
  uint16_t* const orow = a.out + (b * a.tokens + t0) * C + col0;

  // Row u of the run lives in slot u % kAdaAhead. (nr and every branch on
  // it are uniform over the workgroup, so every wave reaches each barrier.)
  uint4 xv[kAdaAhead];
  Raw8<D0> p0[kPre ? kAdaAhead : 1];
  Raw8<D1> p1[kPre ? kAdaAhead : 1];
  auto issue = [&](int u, auto k_c) {
    constexpr int K = decltype(k_c)::value;
    xv[K] = *(const uint4*)(xrow + (int64_t)u * C);
    if constexpr (kPre) {
      const int64_t t = t0 + u;
      p0[K] = raw8_load<D0>(a.s0.ts, tsc0 + t * a.s0.ts_st);
      p1[K] = raw8_load<D1>(a.s1.ts, tsc1 + t * a.s1.ts_st);
    }
  };
  auto prologue = [&](auto k_c) {
    if (decltype(k_c)::value < nr) issue(decltype(k_c)::value, k_c);
  };
  prologue(IC<0>{});
  if constexpr (kAdaAhead > 1) prologue(IC<1>{});
  if constexpr (kAdaAhead > 2) prologue(IC<2>{});
  if constexpr (kAdaAhead > 3) prologue(IC<3>{});

  const bool tab0 = a.s0.tab != nullptr;
  const bool tab1 = a.s1.tab != nullptr;
  float c0[8], c1[8];
  ada_table8(a.s0, col0, c0);
  ada_table8(a.s1, col0, c1);
  if (UNIFORM) {
    float v[8];
    ada_value8(a.s0, c0, b, 0, col0, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) c0[i] = v[i];
    ada_value8(a.s1, c1, b, 0, col0, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float f = 1.0f + v[i];
      c1[i] = B1 ? rbf(f) : f;
    }
  }

  auto row = [&](int u, auto k_c) {
    constexpr int K = decltype(k_c)::value;
    const int64_t t = t0 + u;
    float xf[8];
    unpack8(xv[K], xf);
    double ss[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double d = (double)xf[i];
      ss[i & 3] = fma(d, d, ss[i & 3]);
    }
    const double w = wave_sum_d((ss[0] + ss[1]) + (ss[2] + ss[3]));
    if (lane == 0) part[u & 1][wv] = w;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int c = 0; c < CH; ++c) tot += part[u & 1][c];
    const float mean = (float)(tot / (double)C);
    const float inv = 1.0f / sqrtf(mean + a.eps);
    float v0[8], v1[8], o[8];
    if (UNIFORM) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v0[i] = c0[i];
        v1[i] = c1[i];
      }
    } else {
      float tsv[8];
      if constexpr (kPre) raw8_get<D0>(p0[K], tsv);
      else load8_t<D0, false>(a.s0.ts, tsc0 + t * a.s0.ts_st, a.s0.ts_sc, tsv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float sum = tab0 ? c0[i] + tsv[i] : tsv[i];
        v0[i] = (tab0 && B0) ? rbf(sum) : sum;
      }
      if constexpr (kPre) raw8_get<D1>(p1[K], tsv);
      else load8_t<D1, false>(a.s1.ts, tsc1 + t * a.s1.ts_st, a.s1.ts_sc, tsv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float sum = tab1 ? c1[i] + tsv[i] : tsv[i];
        if (tab1 && B1) sum = rbf(sum);
        const float f = 1.0f + sum;
        v1[i] = B1 ? rbf(f) : f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float p = rbf(xf[i] * inv) * v1[i];
      if (B1) p = rbf(p);
      o[i] = p + v0[i];
    }
    st_nt16(orow + (int64_t)u * C, pack8(o));
  };
  auto step = [&](int base, auto k_c) {
    const int u = base + decltype(k_c)::value;
    if (u < nr) {
      row(u, k_c);
      if (u + kAdaAhead < nr) issue(u + kAdaAhead, k_c);
    }
  };
  for (int base = 0; base < nr; base += kAdaAhead) {
    step(base, IC<0>{});
    if constexpr (kAdaAhead > 1) step(base, IC<1>{});
    if constexpr (kAdaAhead > 2) step(base, IC<2>{});
    if constexpr (kAdaAhead > 3) step(base, IC<3>{});
  }
}

// ------------------------------------------------ AdaZero, wave per row
// y = R(R?(R(x * inv_rms) * R?(1 + scale)) + shift) with one wave per token
// row: lane l holds columns j*512 + 8l .. +7 of every 512-column chunk j, so
// a row's sum of squares is a wave reduction (DPP, no LDS, no barrier) and a
// row is written as soon as its own loads have landed. The kAdaWaves waves
// of a workgroup first fill LDS with the per-column constants in float32:
// with one timestep row shared by all tokens, the finished Ada values (shift
// and R?(1 + scale)); otherwise the table parts R?(table[i]), to which each
// row adds its own timestep values. One barrier publishes the constants. A
// wave then streams rows t = v, v + V, ... of its batch (V waves per batch),
// with the next row's loads in flight while it finishes the current one when
// the timestep row is shared. Two values are rounded per v_cvt_pk_bf16_f32.
#ifndef OGA_ADA_WAVES
#define OGA_ADA_WAVES 12
#endif
constexpr int kAdaWaves = OGA_ADA_WAVES;
// The residual-gate form holds a second row buffer (y_in) and takes more
// registers: two waves per SIMD.
constexpr int kResAdaWaves = 8;
enum { RES_NONE = 0, RES_GATE = 1, RES_GATE_BIAS = 2 };
template <int RES>
constexpr int ada_waves() { return RES == RES_NONE ? kAdaWaves : kResAdaWaves; }
#ifndef OGA_ADA_SCHED_GROUP
#define OGA_ADA_SCHED_GROUP 2
#endif
constexpr int kAdaSchedGroup = OGA_ADA_SCHED_GROUP;
enum { TAB_NONE = 0, TAB_BF16 = 1, TAB_F32 = 2 };

// Q8 (Q8_F32, Q8_BF16): each finished bf16 row goes straight into the FP8
// linear's input quantizer, e4m3(clamp(R(y) * r, +-448)) with r as
// k_fp8_quant takes it (the float32 reciprocal of the scale; for a 0-dim
// scale, Q8_BF16, r and the product are rounded to bf16), so only the codes
// reach memory. The scale's kind is a template flag, not a per-value select.
// The clamp must keep NaN (torch.clamp propagates it), which costs a compare
// and a select beside v_med3_f32 per value. A row whose sum of squares is
// finite, with finite Ada values (checked once per workgroup when they are
// shared by all tokens) and a finite r >= 2^-126, cannot produce a NaN (x*inv
// is then finite, (1 + scale) and shift finite, so y is finite or an
// overflowed infinity, and y*r is never inf*0), so such rows take
// v_med3_f32 alone; the others keep the NaN-preserving clamp.
//
// RES (RES_GATE, RES_GATE_BIAS; shared timestep row only): the row is first
// the residual gate x' = R(x + R?(y_in * gate)) (RES_GATE_BIAS:
// R(x + R?(R(y_in + R(bias)) * gate))), as k_elem computes it, stored to
// xout; AdaZero then normalises x'. The gate comes from the same table and
// timestep tensor as shift and scale (so the same dtypes), and lands in LDS
// with R(bias) beside them.
enum { Q8_NONE = 0, Q8_F32 = 1, Q8_BF16 = 2 };
template <int CH, bool UNIFORM, int D0, int D1, int TAB, int Q8 = Q8_NONE, int RES = RES_NONE>
__global__ __launch_bounds__(64 * ada_waves<RES>()) void k_adazero_rows(RowArgs a, int64_t waves_per_batch) {
  static_assert(RES == RES_NONE || (UNIFORM && D0 == D1), "the residual form takes a shared timestep row");
  constexpr int NW = ada_waves<RES>();
  constexpr int C = CH * 512;
  constexpr int G = C / 8;  // groups of 8 columns
  constexpr int NT = 64 * NW;
  constexpr int GPT = (G + NT - 1) / NT;
  constexpr bool B0 = D0 == OGA_DT_BF16;
  constexpr bool B1 = D1 == OGA_DT_BF16;
  constexpr bool HT = TAB != TAB_NONE;
  constexpr int TD = TAB == TAB_F32 ? OGA_DT_F32 : OGA_DT_BF16;
  constexpr int NC = RES == RES_NONE ? 2 : 4;
  __shared__ float4 cst[NC][2 * G];  // [shift | scale part | gate | R(bias)][column / 4]
  __shared__ uint32_t ada_bad[NW];   // per wave: a shared Ada value is not finite
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t V = waves_per_batch;
  const int64_t v = (int64_t)blockIdx.x * NW + w;
  // A wave past the batch's V waves takes no rows but joins the fill.
  const int64_t t_first = v < V ? v : a.tokens;

  // The constant loads (table rows and, when shared, the timestep row),
  // then the first row's loads. Every one is unconditional (a wave without
  // rows loads row tokens - 1 and stores nothing; a thread past the column
  // groups repeats group gi % G and writes the same values): a branch around
  // a load would make the compiler wait for every outstanding load at its
  // merge. Loads complete in order, so with the constants first the fill and
  // its barrier wait for them alone and run while the row is still in
  // flight (rows first made the fill wait for the row too: 6.47 against
  // 6.41 us at 1x2304x4096, 13.71 against 13.44 us with per-token
  // timesteps).
  Raw8<TD> tr0[GPT], tr1[GPT], tr2[GPT];
  Raw8<D0> u0[GPT], u2[GPT];
  Raw8<D1> u1[GPT];
  uint4 bias_raw[GPT][2];  // bf16: [0]; float32: [0], [1]
#pragma unroll
  for (int q = 0; q < GPT; ++q) {
    const int gi = (tid + q * NT) % G;
    if constexpr (HT) {
      tr0[q] = raw8_load<TD>(a.s0.tab, a.s0.tab_off + gi * 8);
      tr1[q] = raw8_load<TD>(a.s1.tab, a.s1.tab_off + gi * 8);
      if constexpr (RES != RES_NONE) tr2[q] = raw8_load<TD>(a.s2.tab, a.s2.tab_off + gi * 8);
    }
    if constexpr (UNIFORM) {
      u0[q] = raw8_load<D0>(a.s0.ts, a.s0.ts_off + b * a.s0.ts_sb + gi * 8);
      u1[q] = raw8_load<D1>(a.s1.ts, a.s1.ts_off + b * a.s1.ts_sb + gi * 8);
      if constexpr (RES != RES_NONE) u2[q] = raw8_load<D0>(a.s2.ts, a.s2.ts_off + b * a.s2.ts_sb + gi * 8);
    }
    if constexpr (RES == RES_GATE_BIAS) {  // a uniform branch; only constant loads are in flight here
      if (a.bias_dt == OGA_DT_BF16) {
        bias_raw[q][0] = *(const uint4*)((const uint16_t*)a.bias + gi * 8);
        bias_raw[q][1] = make_uint4(0, 0, 0, 0);
      } else {
        bias_raw[q][0] = *(const uint4*)((const float*)a.bias + gi * 8);
        bias_raw[q][1] = *(const uint4*)((const float*)a.bias + gi * 8 + 4);
      }
    }
  }
  const uint16_t* const xb = a.x + b * a.tokens * C + lane * 8;
  uint16_t* const yb = a.out + b * a.tokens * C + lane * 8;
  uint8_t* const qb = (uint8_t*)a.out + b * a.tokens * C + lane * 8;
  float qr = 0.0f;
  if constexpr (Q8 != Q8_NONE) {
    qr = 1.0f / a.qscale[0];
    if constexpr (Q8 == Q8_BF16) qr = rbf(qr);
  }
  const uint16_t* const ib = a.y + b * a.tokens * C + lane * 8;  // RES: y_in rows
  uint16_t* const xo = a.xout + b * a.tokens * C + lane * 8;      // RES: x' rows
  uint4 xv[CH], yv[CH];
  {
    const int64_t tl = t_first < a.tokens ? t_first : a.tokens - 1;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      xv[j] = *(const uint4*)(xb + tl * C + j * 512);
      if constexpr (RES != RES_NONE) yv[j] = *(const uint4*)(ib + tl * C + j * 512);
    }
  }
  // Constants to LDS.
  bool bad_const = false;
#pragma unroll
  for (int q = 0; q < GPT; ++q) {
    const int gi = (tid + q * NT) % G;
    {
      float c0[8], c1[8];
      if constexpr (HT) {
        raw8_get<TD>(tr0[q], c0);
        raw8_get<TD>(tr1[q], c1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // table.to(ts dtype)
          if (TAB == TAB_F32 && B0) c0[i] = rbf(c0[i]);
          if (TAB == TAB_F32 && B1) c1[i] = rbf(c1[i]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) c0[i] = c1[i] = 0.0f;
      }
      if constexpr (UNIFORM) {
        float s[8];
        raw8_get<D0>(u0[q], s);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float sum = HT ? c0[i] + s[i] : s[i];
          c0[i] = (HT && B0) ? rbf(sum) : sum;
        }
        raw8_get<D1>(u1[q], s);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float sum = HT ? c1[i] + s[i] : s[i];
          if (HT && B1) sum = rbf(sum);
          const float f = 1.0f + sum;
          c1[i] = B1 ? rbf(f) : f;
        }
      }
      if constexpr (Q8 != Q8_NONE && UNIFORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) bad_const |= !__builtin_isfinite(c0[i]) || !__builtin_isfinite(c1[i]);
      }
      if constexpr (RES != RES_NONE) {
        // the gate: R?(R?tab(table) + ts) as k_elem's ada_value8 computes it
        float c2[8], s[8];
        if constexpr (HT) {
          raw8_get<TD>(tr2[q], c2);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (TAB == TAB_F32 && B0) c2[i] = rbf(c2[i]);
        }
        raw8_get<D0>(u2[q], s);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float sum = HT ? c2[i] + s[i] : s[i];
          c2[i] = (HT && B0) ? rbf(sum) : sum;
        }
        cst[2][2 * gi] = make_float4(c2[0], c2[1], c2[2], c2[3]);
        cst[2][2 * gi + 1] = make_float4(c2[4], c2[5], c2[6], c2[7]);
        if constexpr (RES == RES_GATE_BIAS) {
          float bb[8];
          if (a.bias_dt == OGA_DT_BF16) {
            unpack8(bias_raw[q][0], bb);
          } else {
            const uint4 l = bias_raw[q][0], h = bias_raw[q][1];
            const uint32_t w8[8] = {l.x, l.y, l.z, l.w, h.x, h.y, h.z, h.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) bb[i] = rbf(__uint_as_float(w8[i]));
          }
          cst[3][2 * gi] = make_float4(bb[0], bb[1], bb[2], bb[3]);
          cst[3][2 * gi + 1] = make_float4(bb[4], bb[5], bb[6], bb[7]);
        }
      }
      cst[0][2 * gi] = make_float4(c0[0], c0[1], c0[2], c0[3]);
      cst[0][2 * gi + 1] = make_float4(c0[4], c0[5], c0[6], c0[7]);
      cst[1][2 * gi] = make_float4(c1[0], c1[1], c1[2], c1[3]);
      cst[1][2 * gi + 1] = make_float4(c1[4], c1[5], c1[6], c1[7]);
    }
  }
  if constexpr (Q8 != Q8_NONE && UNIFORM) {
    const uint64_t bm = __ballot(bad_const);
    if (lane == 0) ada_bad[w] = bm != 0;
  }
  // LDS writes done, then the barrier; no vmcnt drain (the row loads stay
  // in flight across it).
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // Rows may take the NaN-free clamp (Q8): the workgroup's shared Ada values
  // and r are finite (r normal); each row adds its own finite sum of squares.
  bool clean_consts = false;
  if constexpr (Q8 != Q8_NONE && UNIFORM) {
    uint32_t any_bad = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) any_bad |= ada_bad[i];
    clean_consts = !any_bad && __builtin_isfinite(qr) && qr >= 0x1p-126f;
  }

  const int64_t ts0 = a.s0.ts_off + b * a.s0.ts_sb + lane * 8;
  const int64_t ts1 = a.s1.ts_off + b * a.s1.ts_sb + lane * 8;
  // Per-token timesteps in bf16 are loaded for the whole row up front; in
  // float32 (twice the registers) chunk by chunk.
  constexpr bool kTsRow = !UNIFORM && B0 && B1;
  // One row t from the loaded buffer `cur`; with a shared timestep row the
  // loads of the wave's next row go into `nxt` right after `cur` is
  // unpacked. The first row is peeled off the loop: with one row per wave
  // (2304 tokens) no loop-carried register copies are made at all.
  auto row = [&](auto first_c, int64_t t, uint4(&cur)[CH], uint4(&nxt)[CH], uint4(&cury)[CH],
                 uint4(&nxty)[CH]) {
    if (!decltype(first_c)::value && !UNIFORM) {
#pragma unroll
      for (int j = 0; j < CH; ++j) cur[j] = *(const uint4*)(xb + t * C + j * 512);
    }
    Raw8<D0> p0[kTsRow ? CH : 1];
    Raw8<D1> p1[kTsRow ? CH : 1];
    if constexpr (kTsRow) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        p0[j] = raw8_load<D0>(a.s0.ts, ts0 + t * a.s0.ts_st + j * 512);
        p1[j] = raw8_load<D1>(a.s1.ts, ts1 + t * a.s1.ts_st + j * 512);
      }
    }
    float f[CH][8];
    double ss[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if constexpr (RES != RES_NONE) {  // x' = R(x + R?(y_in' * gate)), stored, then normalised
        const int gi = j * 64 + lane;
        const float4 g0 = cst[2][2 * gi], g1 = cst[2][2 * gi + 1];
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        float bv[8];
        if constexpr (RES == RES_GATE_BIAS) {
          const float4 b0 = cst[3][2 * gi], b1 = cst[3][2 * gi + 1];
          bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
          bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
        }
        float xf[8], yf[8], o[8];
        unpack8(cur[j], xf);
        unpack8(cury[j], yf);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float yy = yf[i];
          if constexpr (RES == RES_GATE_BIAS) yy = rbf(yy + bv[i]);
          float p = yy * gv[i];
          if constexpr (B0) p = rbf(p);
          o[i] = xf[i] + p;
        }
        const uint4 xp = pack8(o);
        st_nt16(xo + t * C + j * 512, xp);
        unpack8(xp, f[j]);
      } else {
        unpack8(cur[j], f[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss[i & 3] = fma((double)f[j][i], (double)f[j][i], ss[i & 3]);
    }
    if constexpr (UNIFORM) {  // the next row's loads
      const int64_t tn = t + V;
      if (tn < a.tokens) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          nxt[j] = *(const uint4*)(xb + tn * C + j * 512);
          if constexpr (RES != RES_NONE) nxty[j] = *(const uint4*)(ib + tn * C + j * 512);
        }
      }
    }
    const double tot = wave_sum_d((ss[0] + ss[1]) + (ss[2] + ss[3]));
    const float inv = 1.0f / sqrtf((float)(tot / (double)C) + a.eps);
    // The chunks of the row; CLEAN: the row cannot produce a NaN (see above).
    auto tail = [&](auto clean_c) {
    constexpr bool CLEAN = decltype(clean_c)::value;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      // Groups of kAdaSchedGroup chunks: keeps the constants' LDS reads (and
      // float32 timestep loads) from being hoisted for all chunks at once.
      if (kAdaSchedGroup > 0 && j % kAdaSchedGroup == 0) __builtin_amdgcn_sched_barrier(0);
      const int gi = j * 64 + lane;
      const float4 a0 = cst[0][2 * gi], a1 = cst[0][2 * gi + 1];
      const float4 m0 = cst[1][2 * gi], m1 = cst[1][2 * gi + 1];
      float v0[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      float v1[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
      if constexpr (!UNIFORM) {
        float s0v[8], s1v[8];
        if constexpr (kTsRow) {
          raw8_get<D0>(p0[j], s0v);
          raw8_get<D1>(p1[j], s1v);
        } else {
          raw8_get<D0>(raw8_load<D0>(a.s0.ts, ts0 + t * a.s0.ts_st + j * 512), s0v);
          raw8_get<D1>(raw8_load<D1>(a.s1.ts, ts1 + t * a.s1.ts_st + j * 512), s1v);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float sum = HT ? v0[i] + s0v[i] : s0v[i];
          v0[i] = (HT && B0) ? rbf(sum) : sum;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float sum = HT ? v1[i] + s1v[i] : s1v[i];
          if (HT && B1) sum = rbf(sum);
          const float fv = 1.0f + sum;
          v1[i] = B1 ? rbf(fv) : fv;
        }
      }
      // y = R(R(R(x * inv) * (1 + scale)) + shift) per value (the middle
      // rounding with a bf16 table); each intermediate R as one conversion
      // that leaves the float (rbf), the output packed in pairs.
      float pv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = rbf(f[j][i] * inv) * v1[i];
        pv[i] = (B1 ? rbf(p) : p) + v0[i];
      }
      if constexpr (Q8 != Q8_NONE) {
        float qv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float q = rbf(pv[i]) * qr;
          if constexpr (Q8 == Q8_BF16) q = rbf(q);
          qv[i] = CLEAN ? __builtin_amdgcn_fmed3f(q, -448.0f, 448.0f) : clamp448(q);
        }
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 o = {e4m3x4_valu(qv[0], qv[1], qv[2], qv[3]), e4m3x4_valu(qv[4], qv[5], qv[6], qv[7])};
        __builtin_nontemporal_store(o, (u32x2*)(qb + t * C + j * 512));
      } else {
        st_nt16(yb + t * C + j * 512, make_uint4(pack_bf16(pv[0], pv[1]), pack_bf16(pv[2], pv[3]),
                                                 pack_bf16(pv[4], pv[5]), pack_bf16(pv[6], pv[7])));
      }
    }
    };
    if constexpr (Q8 != Q8_NONE && UNIFORM) {
      if (clean_consts && __builtin_isfinite(tot))
        tail(IC<1>{});
      else
        tail(IC<0>{});
    } else {
      tail(IC<0>{});
    }
  };
  // Rows alternate between two load buffers, so a row's next-row loads never
  // need a register copy at the loop's end.
  if (t_first < a.tokens) {
    uint4 xw[CH], yw[CH];
    row(IC<1>{}, t_first, xv, xw, yv, yw);  // its loads went out before the fill
    for (int64_t t = t_first + V; t < a.tokens; t += 2 * V) {
      row(IC<0>{}, t, xw, xv, yw, yv);
      if (t + V < a.tokens) row(IC<0>{}, t + V, xv, xw, yv, yw);
    }
  }
}

// Grid of k_adazero_rows: one workgroup of kAdaWaves waves per CU at most;
// rows = ceil(batch*tokens / (CUs * kAdaWaves)) rows per wave, and V =
// ceil(tokens / rows) waves per batch, so every wave gets rows or rows - 1.
static void adazero_rows_grid(int64_t batch, int64_t tokens, dim3& grid, int64_t& waves_per_batch,
                              int64_t& rows_per_wave, int waves = kAdaWaves) {
  const int64_t slots = (int64_t)cu_count() * waves;
  int64_t rows = (batch * tokens + slots - 1) / slots;
  if (rows < 1) rows = 1;
  const int64_t v = (tokens + rows - 1) / rows;
  rows_per_wave = (tokens + v - 1) / v;
  waves_per_batch = v;
  grid = dim3((unsigned)((v + waves - 1) / waves), (unsigned)batch);
}

// Grid of k_adazero: about OGA_ADA_WGS_PER_CU workgroups per CU, each
// streaming an equal run of rows.
#ifndef OGA_ADA_WGS_PER_CU
#define OGA_ADA_WGS_PER_CU 4
#endif
static void adazero_grid(int64_t batch, int64_t tokens, dim3& grid, int& rows_per_wg) {
  const int64_t target_wgs = (int64_t)cu_count() * OGA_ADA_WGS_PER_CU;
  int64_t per_batch = target_wgs / batch;
  if (per_batch < 1) per_batch = 1;
  int64_t rows = (tokens + per_batch - 1) / per_batch;
  if (rows > INT32_MAX) rows = INT32_MAX;
  rows_per_wg = (int)rows;
  grid = dim3((unsigned)((tokens + rows - 1) / rows), (unsigned)batch);
}

// Grid of k_elem: up to OGA_ELEM_WG_PER_CU workgroups per CU over all
// batches, each taking kElemRows rows at a time; `rows_per_wg` is the most
// rows one workgroup (and each of its waves) streams.
static void elem_grid(int64_t batch, int64_t tokens, dim3& grid, int64_t& rows_per_wg) {
  const int64_t steps = (tokens + kElemRows - 1) / kElemRows;
  int64_t x = (int64_t)cu_count() * OGA_ELEM_WG_PER_CU / batch;
  if (x < 1) x = 1;
  if (x > steps) x = steps;
  rows_per_wg = (steps + x - 1) / x * kElemRows;
  grid = dim3((unsigned)x, (unsigned)batch);
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
    st_nt16(out + i0, pack8(o));
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
    st_nt16(out + i0, pack8(o));
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

template <int CH, bool UNIFORM, int D0, int D1, int Q8>
static void launch_adazero_q8(RowArgs& a, dim3 grid, dim3 block, int64_t vpb, hipStream_t st) {
  if (!a.s0.tab)
    hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_NONE, Q8>), grid, block, 0, st, a, vpb);
  else if (a.s0.tab_dt == OGA_DT_BF16)
    hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_BF16, Q8>), grid, block, 0, st, a, vpb);
  else
    hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_F32, Q8>), grid, block, 0, st, a, vpb);
}

// The residual form: 4096 columns, a shared timestep row, one Ada dtype.
template <int D, int TAB, int Q8>
static void launch_res_ada_q(RowArgs& a, int res, dim3 grid, int64_t vpb, hipStream_t st) {
  const dim3 block(64 * kResAdaWaves);
  if (res == RES_GATE_BIAS)
    hipLaunchKernelGGL((k_adazero_rows<8, true, D, D, TAB, Q8, RES_GATE_BIAS>), grid, block, 0, st, a, vpb);
  else
    hipLaunchKernelGGL((k_adazero_rows<8, true, D, D, TAB, Q8, RES_GATE>), grid, block, 0, st, a, vpb);
}
template <int D, int TAB>
static void launch_res_ada_t(RowArgs& a, int res, dim3 grid, int64_t vpb, hipStream_t st) {
  if (!a.q8)
    launch_res_ada_q<D, TAB, Q8_NONE>(a, res, grid, vpb, st);
  else if (a.q_zero_dim)
    launch_res_ada_q<D, TAB, Q8_BF16>(a, res, grid, vpb, st);
  else
    launch_res_ada_q<D, TAB, Q8_F32>(a, res, grid, vpb, st);
}
static int launch_res_ada(RowArgs& a, int res, int64_t batch, hipStream_t st) {
  dim3 grid;
  int64_t vpb = 0, rpw = 0;
  adazero_rows_grid(batch, a.tokens, grid, vpb, rpw, kResAdaWaves);
  const bool d_bf = a.s0.ts_dt == OGA_DT_BF16, t_bf = a.s0.tab_dt == OGA_DT_BF16;
  if (d_bf && t_bf)
    launch_res_ada_t<OGA_DT_BF16, TAB_BF16>(a, res, grid, vpb, st);
  else if (d_bf)
    launch_res_ada_t<OGA_DT_BF16, TAB_F32>(a, res, grid, vpb, st);
  else if (t_bf)
    launch_res_ada_t<OGA_DT_F32, TAB_BF16>(a, res, grid, vpb, st);
  else
    launch_res_ada_t<OGA_DT_F32, TAB_F32>(a, res, grid, vpb, st);
  return launch_status();
}

template <int CH, int OP, bool UNIFORM, int D0, int D1>
static void launch_row_v(RowArgs& a, int64_t batch, bool vec, hipStream_t st) {
  if constexpr (OP != OP_ADAZERO) {
    dim3 grid;
    int64_t rpw = 0;
    elem_grid(batch, a.tokens, grid, rpw);
    if (vec)
      hipLaunchKernelGGL((k_elem<CH, OP, UNIFORM, D0, D1, true>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((k_elem<CH, OP, UNIFORM, D0, D1, false>), grid, dim3(256), 0, st, a);
  } else if (vec) {
    dim3 grid;
    int64_t vpb = 0, rpw = 0;
    adazero_rows_grid(batch, a.tokens, grid, vpb, rpw);
    const dim3 block(64 * kAdaWaves);
    if (a.q8) {
      if (a.q_zero_dim)
        launch_adazero_q8<CH, UNIFORM, D0, D1, Q8_BF16>(a, grid, block, vpb, st);
      else
        launch_adazero_q8<CH, UNIFORM, D0, D1, Q8_F32>(a, grid, block, vpb, st);
    } else if (!a.s0.tab)
      hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_NONE>), grid, block, 0, st, a, vpb);
    else if (a.s0.tab_dt == OGA_DT_BF16)
      hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_BF16>), grid, block, 0, st, a, vpb);
    else
      hipLaunchKernelGGL((k_adazero_rows<CH, UNIFORM, D0, D1, TAB_F32>), grid, block, 0, st, a, vpb);
  } else {
    dim3 grid;
    int rpw = 0;
    adazero_grid(batch, a.tokens, grid, rpw);
    hipLaunchKernelGGL((k_adazero_gather<CH, UNIFORM, D0, D1, false>), grid, dim3(64 * CH), 0, st, a, rpw);
  }
}

template <int CH, int OP, bool UNIFORM>
static int launch_row_u(RowArgs& a, int64_t batch, bool vec, hipStream_t st) {
  const int d0 = a.s0.ts_dt, d1 = a.s1.ts_dt;
  if (d0 == OGA_DT_BF16 && d1 == OGA_DT_BF16)
    launch_row_v<CH, OP, UNIFORM, OGA_DT_BF16, OGA_DT_BF16>(a, batch, vec, st);
  else if (d0 == OGA_DT_F32 && d1 == OGA_DT_F32)
    launch_row_v<CH, OP, UNIFORM, OGA_DT_F32, OGA_DT_F32>(a, batch, vec, st);
  else if (OP == OP_ADAZERO && d0 == OGA_DT_BF16)
    launch_row_v<CH, OP_ADAZERO, UNIFORM, OGA_DT_BF16, OGA_DT_F32>(a, batch, vec, st);
  else if (OP == OP_ADAZERO)
    launch_row_v<CH, OP_ADAZERO, UNIFORM, OGA_DT_F32, OGA_DT_BF16>(a, batch, vec, st);
  else
    return unsupported("Ada values of different dtypes");
  return launch_status();
}

template <int CH, int OP>
static int launch_row_ch(RowArgs& a, int64_t batch, bool uniform, bool vec, hipStream_t st) {
  return uniform ? launch_row_u<CH, OP, true>(a, batch, vec, st) : launch_row_u<CH, OP, false>(a, batch, vec, st);
}

template <int OP>
static int run_row(RowArgs& a, int64_t batch, hipStream_t st) {
  if (batch == 0 || a.tokens == 0) return OGA_OK;
  if (batch > 65535) return unsupported("batch > 65535");
  constexpr bool two = RowTraits<OP>::kTwo;
  const bool uniform = a.s0.ts_st == 0 && (!two || a.s1.ts_st == 0);
  bool vec = a.s0.ts_vec && (!two || a.s1.ts_vec);
  if (OP == OP_ADAZERO && a.s0.tab)  // k_adazero_rows reads table rows 16 bytes at a time
    vec = vec && a.s0.tab_vec && a.s1.tab_vec && a.s0.tab_dt == a.s1.tab_dt;
  if (a.q8 && !vec) return unsupported("e4m3 output needs 16-byte table and timestep rows");
  return a.cols == 4096 ? launch_row_ch<8, OP>(a, batch, uniform, vec, st)
                        : launch_row_ch<4, OP>(a, batch, uniform, vec, st);
}

static int check_rows(const void* x, const void* y, int64_t batch, int64_t tokens, int64_t cols) {
  if (!valid_ada_inputs(batch, tokens, cols)) return unsupported("cols must be 2048 or 4096 (got %lld)", (long long)cols);
  if (!x || !y) return fail("null x/out");
  if (!aligned(x, 16) || !aligned(y, 16)) return fail("x/out must be 16-byte aligned");
  return OGA_OK;
}

}  // namespace oga

using namespace oga;

static int row_common(RowArgs& a, const void* x, const void* y, void* out, int64_t batch, int64_t tokens,
                      int64_t cols) {
  int rc = check_rows(x, out, batch, tokens, cols);
  if (rc) return rc;
  if (y && !aligned(y, 16)) return fail("y must be 16-byte aligned");
  a.x = (const uint16_t*)x;
  a.y = (const uint16_t*)y;
  a.out = (uint16_t*)out;
  a.tokens = tokens;
  a.cols = (int)cols;
  return OGA_OK;
}

extern "C" int oga_adazero_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                    const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                    const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                    int shift_index, int scale_index, float eps, void* stream) {
  RowArgs a{};
  int rc = row_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  a.eps = eps;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s1, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, INT64_MAX))) return rc;
  return run_row<OP_ADAZERO>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_adazero_from_ada_fp8(const void* x, void* q, int64_t batch, int64_t tokens, int64_t cols,
                                        const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                        const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                        int shift_index, int scale_index, float eps, const float* input_scale,
                                        int scale_zero_dim, void* stream) {
  RowArgs a{};
  int rc = row_common(a, x, nullptr, q, batch, tokens, cols);
  if (rc) return rc;
  if (!input_scale) return fail("null input scale");
  a.eps = eps;
  a.q8 = 1;
  a.qscale = input_scale;
  a.q_zero_dim = scale_zero_dim ? 1 : 0;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s1, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, INT64_MAX))) return rc;
  return run_row<OP_ADAZERO>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_adazero(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols, const void* scale,
                           int scale_dtype, const int64_t scale_strides[3], const void* shift, int shift_dtype,
                           const int64_t shift_strides[3], float eps, void* stream) {
  RowArgs a{};
  int rc = row_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  if (!scale || !shift || !scale_strides || !shift_strides) return fail("null scale/shift");
  if (!dt_ok(scale_dtype) || !dt_ok(shift_dtype)) return fail("scale/shift dtype must be bf16 or f32");
  a.eps = eps;
  make_direct_src(a.s0, shift, shift_dtype, shift_strides);
  make_direct_src(a.s1, scale, scale_dtype, scale_strides);
  return run_row<OP_ADAZERO>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_adaln_affine_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                         const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                         const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                         int shift_index, int scale_index, void* stream) {
  RowArgs a{};
  int rc = row_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s1, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, INT64_MAX))) return rc;
  return run_row<OP_ADALN>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_mul_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                                const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                const void* timestep, int ts_dtype, const int64_t ts_strides[4], int gate_index,
                                void* stream) {
  RowArgs a{};
  int rc = row_common(a, x, nullptr, y, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_row<OP_MUL>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_from_ada(const void* x, const void* y, void* out, int64_t batch, int64_t tokens,
                                          int64_t cols, const void* table, int table_dtype, int64_t tab_s0,
                                          int64_t tab_s1, const void* timestep, int ts_dtype,
                                          const int64_t ts_strides[4], int gate_index, void* stream) {
  RowArgs a{};
  if (!y) return fail("null y");
  int rc = row_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_row<OP_RESID>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_bias_from_ada(const void* x, const void* y, const void* bias, int bias_dtype,
                                               void* out, int64_t batch, int64_t tokens, int64_t cols,
                                               const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                               const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                               int gate_index, void* stream) {
  RowArgs a{};
  if (!y || !bias) return fail("null y/bias");
  if (!dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
  if (!aligned(bias, 32)) return fail("bias must be 32-byte aligned");
  int rc = row_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  a.bias = bias;
  a.bias_dt = bias_dtype;
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  a.s1 = a.s0;
  return run_row<OP_RESID_BIAS>(a, batch, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_adazero_from_ada(const void* x, const void* y, const void* bias, int bias_dtype,
                                                 void* x_out, void* out, int64_t batch, int64_t tokens, int64_t cols,
                                                 const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                                 const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                                 int gate_index, int shift_index, int scale_index, float eps,
                                                 const float* input_scale, int scale_zero_dim, void* stream) {
  RowArgs a{};
  if (!y || !x_out) return fail("null y/x_out");
  int rc = row_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  if (!aligned(x_out, 16)) return fail("x_out must be 16-byte aligned");
  if (cols != 4096) return unsupported("the residual-gate AdaZero takes 4096 columns");
  if (bias) {
    if (!dt_ok(bias_dtype)) return fail("bias dtype must be bf16 or f32");
    if (!aligned(bias, 32)) return fail("bias must be 32-byte aligned");
  }
  a.bias = bias;
  a.bias_dt = bias_dtype;
  a.xout = (uint16_t*)x_out;
  a.eps = eps;
  if (input_scale) {
    a.q8 = 1;
    a.qscale = input_scale;
    a.q_zero_dim = scale_zero_dim ? 1 : 0;
  }
  if ((rc = make_ada_src(a.s0, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, shift_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s1, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, scale_index, INT64_MAX))) return rc;
  if ((rc = make_ada_src(a.s2, table, table_dtype, tab_s0, tab_s1, timestep, ts_dtype, ts_strides, gate_index, INT64_MAX))) return rc;
  if (batch == 0 || tokens == 0) return OGA_OK;
  if (batch > 65535) return unsupported("batch > 65535");
  if (ts_strides[1] != 0) return unsupported("the residual-gate AdaZero takes a timestep row shared by all tokens");
  if (!(a.s0.ts_vec && a.s1.ts_vec && a.s2.ts_vec && a.s0.tab_vec && a.s1.tab_vec && a.s2.tab_vec))
    return unsupported("the residual-gate AdaZero needs 16-byte table and timestep rows");
  return launch_res_ada(a, bias ? RES_GATE_BIAS : RES_GATE, batch, (hipStream_t)stream);
}

extern "C" int oga_residual_gate_bf16(const void* x, const void* y, const void* gate, const int64_t gate_strides[3],
                                      void* out, int64_t batch, int64_t tokens, int64_t cols, void* stream) {
  RowArgs a{};
  if (!y || !gate || !gate_strides) return fail("null y/gate");
  int rc = row_common(a, x, y, out, batch, tokens, cols);
  if (rc) return rc;
  make_direct_src(a.s0, gate, OGA_DT_BF16, gate_strides);
  a.s1 = a.s0;
  return run_row<OP_RESID>(a, batch, (hipStream_t)stream);
}

extern "C" int64_t oga_rows_per_wave(int kind, int64_t batch, int64_t tokens, int64_t cols) {
  if (batch < 1 || tokens < 1 || (cols != 2048 && cols != 4096)) return 0;
  if (kind == OGA_ROWS_ADAZERO) {  // the vectorised kernel, k_adazero_rows
    dim3 grid;
    int64_t vpb = 0, rpw = 0;
    adazero_rows_grid(batch, tokens, grid, vpb, rpw);
    return rpw;
  }
  if (kind == OGA_ROWS_ELEMENTWISE) {
    dim3 grid;
    int64_t rpw = 0;
    elem_grid(batch, tokens, grid, rpw);
    return rpw;
  }
  return 0;
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
