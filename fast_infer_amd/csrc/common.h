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

// The attention kernels lay out K/V rows, Q and O fragments for 128 columns.  A smaller
// head_dim (a multiple of 8) runs the same code: the 16-byte chunks past it are loaded as
// zeros, which add nothing to the dot products, and are never stored.
constexpr int kHeadDim = 128;
inline bool head_dim_ok(int64_t d) { return d >= 8 && d <= kHeadDim && d % 8 == 0; }
constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima: exp2(x - kNegBig) stays finite and
// exp2(-inf - kNegBig) == 0, so rows that have seen no valid key produce no NaN.
constexpr float kNegBig = -1.0e30f;

// ---------------------------------------------------------------------------
// Error reporting (host side): one message per calling thread.
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);
// Compute units of the device that runs `stream` (cached per device).
int device_cu_count(hipStream_t stream);
// Whether workgroups whose block ids are congruent modulo 8 run on one XCD on the device of
// `st` (one probe launch and a synchronous copy on `st` at the device's first call; false,
// and not yet probed, while `st` is being captured).
bool xcd_groups_ok(hipStream_t st);
// Slot (0 .. slots - 1) of `st` among the streams that asked for `purpose` on its device, in
// order of first request, or -1 once `slots` streams hold one.  Kernels keep one set of
// cross-workgroup counters per slot, so calls on different streams never share counters.
constexpr int kXcdPurposes = 1;  // the split-K INT4 GEMM
constexpr int kXcdMaxSlots = 16;
int xcd_stream_slot(hipStream_t st, int purpose, int slots);

// ---------------------------------------------------------------------------
// Device helpers

// C[16x16] += A[16x32] * B[32x16] on one wave (v_mfma_f32_16x16x32_f16).
// Lane l supplies row l%16 of A and column l%16 of B, reduction slots 8*(l/16)..+7,
// and receives C rows 4*(l/16)..+3 of column l%16.
__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Raw buffer descriptor (stride 0, 32-bit format, no swizzle) over `num_records` bytes at
// `base`, as four scalar words for the inline-asm copies below.
typedef int rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ rsrc_t raw_rsrc(const void* base, int num_records) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return rsrc_t{(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xffff, num_records, 0x00020000};
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// One direct-to-LDS copy: each lane's 16 bytes at buffer offset voffset + soffset go to LDS
// byte lds + 16 * lane (buffer_load_dwordx4 ... lds; out-of-range lanes write zeros).  Issued
// through inline asm so the compiler does not track it: it cannot prove later LDS reads
// disjoint from an outstanding copy and would wait for every copy in flight before each of
// them, which undoes any copy-ahead pipeline.  Callers order these copies themselves, with
// wait_vmcnt and barriers; the "memory" clobber keeps other memory accesses from moving
// across them.  M0 is set here without being declared: LLVM treats M0 as a reserved
// register and ignores it in a clobber list, so declaring it would not make the compiler
// save a live value.  The copies are sound only while no other instruction of the calling
// kernels uses M0; tests/test_device_code.py checks that in the compiled code (every M0
// write is this helper's, directly followed by its copy).
__device__ __forceinline__ void lds_copy16(rsrc_t rsrc, uint32_t lds, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
               : "memory");
}

// lds_copy16 with the non-temporal (streaming) cache policy, for data read once.
__device__ __forceinline__ void lds_copy16_nt(rsrc_t rsrc, uint32_t lds, int voffset,
                                              int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :
               : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
               : "memory");
}

// Wait until at most N of this wave's vector-memory operations are outstanding (vmcnt
// only; LDS and export counters untouched).  The kernels that stage through direct-to-LDS
// loads count their own copies: loads complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until this wave's LDS (and scalar-memory) operations are done (lgkmcnt only).
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

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
