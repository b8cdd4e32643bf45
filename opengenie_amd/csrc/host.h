// Host-side helpers shared by the entry points: argument errors, launch
// status, alignment checks and grid sizing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/opengenie_amd.h"

namespace oga {

// Records a printf-style message for oga_last_error() and returns OGA_EINVAL.
int fail(const char* fmt, ...);
int unsupported(const char* fmt, ...);

// Status of the launch just issued: 0 or the pending hipError_t.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OGA_OK : (int)e;
}

inline bool aligned(const void* p, int64_t bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

inline int dt_size(int dt) { return dt == OGA_DT_BF16 ? 2 : 4; }

inline bool dt_ok(int dt) { return dt == OGA_DT_BF16 || dt == OGA_DT_F32; }

// True when an operand read 8 elements at a time along its last axis can use
// 128-bit loads: unit column stride and every other stride/offset keeps the
// 8-element group aligned to the group's byte size.
inline bool vec8_ok(const void* p, int dt, int64_t offset, int64_t s0, int64_t s1, int64_t sc) {
  if (sc != 1) return false;
  const int64_t g = 8 * (int64_t)dt_size(dt);
  const int64_t es = dt_size(dt);
  if ((uintptr_t)p % (uintptr_t)g) return false;
  if ((offset * es) % g || (s0 * es) % g || (s1 * es) % g) return false;
  return true;
}

// Number of compute units of the current device (cached per device id).
int cu_count();

// Grid (workgroups per batch, batch) of 4-wave workgroups for kernels in
// which each wave walks token rows t, t + 4*gridDim.x, ... of its batch:
// up to 64 waves per CU over the launch (about one row per wave at 9216
// tokens; measured 59.9 us against 61.9 us for 16 for the Q/K RMSNorm+RoPE
// at 9216 x 4096), sized so that every wave gets the same number of rows
// (the last pass over the rows is not left part-empty).
#ifndef OGA_ROW_WAVES_PER_CU
#define OGA_ROW_WAVES_PER_CU 64
#endif
inline dim3 balanced_row_grid(int64_t batch, int64_t tokens) {
  const int64_t target_waves = (int64_t)cu_count() * OGA_ROW_WAVES_PER_CU;
  const int64_t rows = batch * tokens;
  int64_t per_wave = (rows + target_waves - 1) / target_waves;
  if (per_wave < 1) per_wave = 1;
  int64_t waves = (tokens + per_wave - 1) / per_wave;  // per batch
  int64_t wgs = (waves + 3) / 4;
  if (wgs < 1) wgs = 1;
  return dim3((unsigned)wgs, (unsigned)batch);
}

}  // namespace oga
