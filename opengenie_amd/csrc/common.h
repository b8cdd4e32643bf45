// Shared device helpers for the CDNA4 (gfx950) kernels of opengenie_amd.
//
// Conventions used by every kernel in this library:
//  * bf16 tensors are moved as 16-byte vectors (8 elements per lane); one
//    wavefront (64 lanes) covers 512 contiguous columns per vector step.
//  * Arithmetic is float32. A value is rounded to bf16 (round to nearest
//    even, v_cvt_pk_bf16_f32) exactly where torch's result dtype for the same
//    expression is bf16; the host decides which by the operand dtypes.
//  * The library is built with -ffp-contract=off so that a*b+c is never fused
//    into one rounding unless written as fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/opengenie_amd.h"

#define OGA_DEVICE __device__ __forceinline__

namespace oga {

constexpr int kWave = 64;

// A compile-time integer as a value (unrolled steps pass their index this
// way so that register arrays are indexed by constants).
template <int N>
struct IC {
  static constexpr int value = N;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- bf16 bits
OGA_DEVICE float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
OGA_DEVICE float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Pack two floats (already bf16 values or not) into two bf16 with RNE.
OGA_DEVICE uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

// Round a float to the nearest bf16 (ties to even) and return it as float:
// one v_cvt_pk_bf16_f32 with +0 in the low half, whose 32 bits are then the
// float of the bf16 value (NaN and infinities included), no shift.
OGA_DEVICE float rbf(float v) { return __uint_as_float(pack_bf16(0.0f, v)); }

// 8 bf16 <-> 8 floats
OGA_DEVICE void unpack8(const uint4& u, float* f) {
  f[0] = bf16_lo(u.x); f[1] = bf16_hi(u.x);
  f[2] = bf16_lo(u.y); f[3] = bf16_hi(u.y);
  f[4] = bf16_lo(u.z); f[5] = bf16_hi(u.z);
  f[6] = bf16_lo(u.w); f[7] = bf16_hi(u.w);
}
OGA_DEVICE uint4 pack8(const float* f) {
  uint4 u;
  u.x = pack_bf16(f[0], f[1]);
  u.y = pack_bf16(f[2], f[3]);
  u.z = pack_bf16(f[4], f[5]);
  u.w = pack_bf16(f[6], f[7]);
  return u;
}

// ---------------------------------------------------------------- fp16 bits
OGA_DEVICE float f16_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
OGA_DEVICE float f16_lo(uint32_t w) { return f16_bits(w & 0xFFFFu); }
OGA_DEVICE float f16_hi(uint32_t w) { return f16_bits(w >> 16); }
// Round a float to the nearest fp16 (ties to even, overflow to infinity,
// v_cvt_f16_f32) and return it as float. The empty asm keeps v a float32
// value in a register: without it the compiler folds a product rounded to
// fp16 into v_fma_mix_f16(a, b, +0), whose +0 addend turns a -0 product
// into +0.
OGA_DEVICE float rhf(float v) {
  asm("" : "+v"(v));
  return (float)(_Float16)v;
}

// Pack two floats into two fp16 (nearest even, v_cvt_f16_f32 each); the
// empty asm keeps the operands float32 registers (see rhf).
OGA_DEVICE uint32_t pack_f16(float lo, float hi) {
  asm("" : "+v"(lo), "+v"(hi));
  const _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// The 16-bit activation dtypes (XDT = OGA_DT_BF16 or OGA_DT_F16): a value of
// x's dtype from its bits, rounding to x's dtype, and 8 elements of a
// 16-byte vector as floats.
template <int XDT>
OGA_DEVICE float x16_bits(uint32_t b) {
  return XDT == OGA_DT_F16 ? f16_bits(b) : __uint_as_float(b << 16);
}
template <int XDT>
OGA_DEVICE float rx16(float v) {
  return XDT == OGA_DT_F16 ? rhf(v) : rbf(v);
}
template <int XDT>
OGA_DEVICE void unpack8x(const uint4& u, float* f) {
  if (XDT == OGA_DT_F16) {
    f[0] = f16_lo(u.x); f[1] = f16_hi(u.x);
    f[2] = f16_lo(u.y); f[3] = f16_hi(u.y);
    f[4] = f16_lo(u.z); f[5] = f16_hi(u.z);
    f[6] = f16_lo(u.w); f[7] = f16_hi(u.w);
  } else {
    unpack8(u, f);
  }
}

// 16-byte store of a streamed output: non-temporal, so it does not evict
// the inputs still being read from the caches.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
OGA_DEVICE void st_nt16(void* p, const uint4& v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, (u32x4*)p);
}

// ------------------------------------------------------ typed 8-wide loads
// Loads 8 consecutive logical elements starting at element offset `off` with
// element stride `sc`, converting to float. `vec` (uniform) says the 8
// elements are contiguous and 16/32-byte aligned, so one or two 128-bit loads
// suffice; otherwise the elements are gathered one by one.
OGA_DEVICE void load8(const void* base, int dt, int64_t off, int64_t sc, bool vec, float* f) {
  if (dt == OGA_DT_BF16) {
    const uint16_t* p = (const uint16_t*)base;
    if (vec) {
      uint4 u = *(const uint4*)(p + off);
      unpack8(u, f);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(((uint32_t)p[off + i * sc]) << 16);
    }
  } else {
    const float* p = (const float*)base;
    if (vec) {
      float4 a = *(const float4*)(p + off);
      float4 b = *(const float4*)(p + off + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = p[off + i * sc];
    }
  }
}

// Compile-time-typed 8-wide load (DT = OGA_DT_BF16 or OGA_DT_F32); VEC
// selects 128-bit loads (contiguous, aligned) or an element gather.
template <int DT, bool VEC>
OGA_DEVICE void load8_t(const void* base, int64_t off, int64_t sc, float* f) {
  if (DT == OGA_DT_BF16) {
    const uint16_t* p = (const uint16_t*)base + off;
    if (VEC) {
      unpack8(*(const uint4*)p, f);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(((uint32_t)p[i * sc]) << 16);
    }
  } else {
    const float* p = (const float*)base + off;
    if (VEC) {
      const float4 a = *(const float4*)p;
      const float4 b = *(const float4*)(p + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = p[i * sc];
    }
  }
}

// 8 consecutive elements of a bf16 (one 16-byte vector) or float32 (two)
// tensor, held as loaded; `raw8_get` converts them to float.
template <int DT>
struct Raw8 {
  uint4 u[DT == OGA_DT_BF16 ? 1 : 2];
};
template <int DT>
OGA_DEVICE Raw8<DT> raw8_load(const void* base, int64_t off) {
  Raw8<DT> r;
  if (DT == OGA_DT_BF16) {
    r.u[0] = *(const uint4*)((const uint16_t*)base + off);
  } else {
    r.u[0] = *(const uint4*)((const float*)base + off);
    r.u[DT == OGA_DT_BF16 ? 0 : 1] = *(const uint4*)((const float*)base + off + 4);
  }
  return r;
}
template <int DT>
OGA_DEVICE void raw8_get(const Raw8<DT>& r, float* f) {
  if (DT == OGA_DT_BF16) {
    unpack8(r.u[0], f);
  } else {
    const uint4 a = r.u[0], b = r.u[DT == OGA_DT_BF16 ? 0 : 1];
    f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y); f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
    f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y); f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
  }
}

// ------------------------------------------------------------- reductions
// Wave-wide sum of a double with DPP butterflies inside each 16-lane row,
// a ds_swizzle across the two rows of each half, and readlane across halves.
// Every lane returns the same (uniform) value.
OGA_DEVICE double dpp_xor_d(double v, int ctrl_sel) {
  int lo = __builtin_bit_cast(int2, v).x;
  int hi = __builtin_bit_cast(int2, v).y;
  int2 r;
  switch (ctrl_sel) {
    case 0:  // quad_perm [1,0,3,2]: lane ^ 1
      r.x = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, true);
      r.y = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, true);
      break;
    case 1:  // quad_perm [2,3,0,1]: lane ^ 2
      r.x = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, true);
      r.y = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, true);
      break;
    case 2:  // row_half_mirror: lane i <-> 7-i inside each group of 8
      r.x = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xF, 0xF, true);
      r.y = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xF, 0xF, true);
      break;
    case 3:  // row_mirror: lane i <-> 15-i inside each row of 16
      r.x = __builtin_amdgcn_mov_dpp(lo, 0x140, 0xF, 0xF, true);
      r.y = __builtin_amdgcn_mov_dpp(hi, 0x140, 0xF, 0xF, true);
      break;
    default:  // ds_swizzle bitmask mode, xor 0x10: swap 16-lane rows in each 32
      r.x = __builtin_amdgcn_ds_swizzle(lo, 0x401F);
      r.y = __builtin_amdgcn_ds_swizzle(hi, 0x401F);
      break;
  }
  return __builtin_bit_cast(double, r);
}

OGA_DEVICE double wave_sum_d(double v) {
  v += dpp_xor_d(v, 0);
  v += dpp_xor_d(v, 1);
  v += dpp_xor_d(v, 2);
  v += dpp_xor_d(v, 3);
  v += dpp_xor_d(v, 4);
  int2 w = __builtin_bit_cast(int2, v);
  int2 a, b;
  a.x = __builtin_amdgcn_readlane(w.x, 0);
  a.y = __builtin_amdgcn_readlane(w.y, 0);
  b.x = __builtin_amdgcn_readlane(w.x, 32);
  b.y = __builtin_amdgcn_readlane(w.y, 32);
  return __builtin_bit_cast(double, a) + __builtin_bit_cast(double, b);
}

// Value held by lane (l ^ 8) inside the same 16-lane row: row_ror:8.
OGA_DEVICE uint32_t row_swap8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true);
}

// The RMS normaliser of one row, shared by every lane of the wave:
// inv = 1 / sqrt(float(sum_sq / cols) + eps), with sum_sq the exact-in-double
// sum of the squares (each square of a bf16 value is exact in float32).
// sqrtf and the division are IEEE correctly rounded in this build.
OGA_DEVICE float rms_inv(double lane_sum_sq, int cols, float eps) {
  double s = wave_sum_d(lane_sum_sq);
  float mean = (float)(s / (double)cols);
  return 1.0f / sqrtf(mean + eps);
}

// ------------------------------------------------------------- e4m3 (OCP)
// float -> float8_e4m3fn, round to nearest even, via v_cvt_pk_fp8_f32. The
// callers clamp to +-448 first (NaN passes through), so the saturation mode
// of the instruction never matters. Packs 4 values into one dword.
OGA_DEVICE uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// e4m3x4 without the zero the builtin's first conversion starts from: that
// conversion writes the low half and its high half is overwritten by the
// second, so the first goes through inline assembly with an output-only
// destination (no v_mov of a zero per word). Its leading s_nop 0 is the one
// wait state a VALU read of a transcendental's result needs on gfx950, which
// the compiler inserts for its own instructions but not before inline
// assembly. For VALU-computed inputs only (an MFMA result needs more wait
// states).
OGA_DEVICE uint32_t e4m3x4_valu(float a, float b, float c, float d) {
  int w;
  asm("s_nop 0\n\tv_cvt_pk_fp8_f32 %0, %1, %2" : "=v"(w) : "v"(a), "v"(b));
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// clamp(v, -448, 448) that keeps NaN (torch.clamp propagates NaN).
OGA_DEVICE float clamp448(float v) {
  float c = fminf(fmaxf(v, -448.0f), 448.0f);
  return (v != v) ? v : c;
}

}  // namespace oga
