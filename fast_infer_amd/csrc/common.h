// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/fast_infer_amd.h"

namespace fi {

typedef _Float16 half_t;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;  // the only head_dim the kernels implement
constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima: exp2(x - kNegBig) stays finite and
// exp2(-inf - kNegBig) == 0, so rows that have seen no valid key produce no NaN.
constexpr float kNegBig = -1.0e30f;

// ---------------------------------------------------------------------------
// Error reporting (host side): one message per calling thread.
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// Device helpers

// C[16x16] += A[16x32] * B[32x16] on one wave (v_mfma_f32_16x16x32_f16).
// Lane l supplies row l%16 of A and column l%16 of B, reduction slots 8*(l/16)..+7,
// and receives C rows 4*(l/16)..+3 of column l%16.
__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane max/sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float row4_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
__device__ __forceinline__ float row4_sum(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Order this wave's LDS writes before its later LDS reads (and reads before later
// writes) when lanes exchange data through LDS within one wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Pack two fp16 values (given as the low/high 16 bits of two dwords) into one dword.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u32x4(half8 v) { return __builtin_bit_cast(u32x4, v); }

// Round-to-nearest-even fp32 -> fp16 of four values.
__device__ __forceinline__ half4 to_half4(floatx4 v) {
  half4 r;
  r[0] = (half_t)v[0];
  r[1] = (half_t)v[1];
  r[2] = (half_t)v[2];
  r[3] = (half_t)v[3];
  return r;
}

}  // namespace fi
