// INT4 group-quantized linear layers for gfx950: quantize, dequantize, and C = X * W^T
// with the dequantization fused into the MFMA loop.
//
// Wire format (loader.py:9-41): W [N, K] is stored as int8 bytes [N, K/2]; byte j of a
// row holds k = 2j in its low nibble and k = 2j+1 in its high nibble, each a 4-bit two's
// complement value in [-8, 7]; scales are fp16 [N, K/128], one per 128-wide group.
// The weight the reference multiplies with is fp16(q * scale) (matmul.py:83-84 and
// :309-326): one rounding of an exact product, which is what v_pk_mul_f16 computes.
//
// C[m, n] = fp16( sum_k X[m, k] * W[n, k] ), fp32 accumulation (matmul.py:14-132,
// :135-186), by the rows M of X:
//   M <= 16          gemv_kernel: one workgroup per 16 output columns, K split over its waves;
//   17..64, packed   gemm_sk_kernel: loader and multiplier waves, K split over workgroups
//                    whose partial sums are added inside the launch (sk_reduce_kernel when
//                    the stream has no counters);
//   17..128          gemm_kernel (packed weights from 65 rows), below;
//   >= 129           the weight dequantized once into the workspace, then
//                    wide_gemm_kernel, an fp16 GEMM.
//
// gemm_kernel: one workgroup = 4 waves = 64 output columns (16 per wave) x MT rows, over a
// slice of the K groups.  Per 128-wide group, X[MT, 128] is staged in LDS (double
// buffered, rows padded to 272 bytes so the 16 rows a wave reads are on distinct banks);
// each lane loads 16 bytes of its weight row (32 int4 values), dequantizes them in
// registers and feeds v_mfma_f32_16x16x32_f16 with W as the A operand and X^T as the B
// operand.  In k-step s (0..3) of a group, lane group g = lane/16 supplies k = 32g + 8s
// .. +7: the 16 bytes one lane loads are exactly its four k-steps.  Small grids split the
// K groups over blockIdx.z; a second kernel adds the fp32 partials in a fixed order.
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace fi {
namespace gemm {

constexpr int kThreads = 256;
constexpr int kNTile = 64;
constexpr int kGroup = 128;     // K per scale group and per pipeline step
constexpr int kLdsRow = 136;    // halves per staged X row (128 + 8 pad)

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

struct Params {
  const half_t* x;
  int64_t x_stride;  // elements between rows of X
  int M, K, N;
  const uint8_t* w;  // int4 bytes [N, K/2] or fp16 [N, K]
  int64_t w_stride;  // bytes (int4) or elements (fp16) between rows of W
  const half_t* scales;
  int64_t s_stride;  // elements between rows of scales
  half_t* out;
  int64_t out_stride;
  float* partial;    // [splits, M, N] fp32 when splits > 1
  int groups_per_split;
  const half_t* norm_w;  // RMSNorm weight [K] when the norm is fused into the X operand
  float eps;
  // gemm_sk_kernel: column tiles, K splits and the per-tile arrival counters
  int tiles;
  int ksplit;
  unsigned* counters;
};

__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// Eight int4 values (natural k order, nibble i = k0 + i) -> fp16(q * s).
//
// With e = d >> 4, byte j of e holds nibble 2j + 1 in its low half.  Two byte
// permutations put byte j of d beside byte j of e, so that the low nibbles at bits 0 and
// 16 are the k pairs (0, 1) and (4, 5), and 8 bits higher (2, 3) and (6, 7): every pair
// comes out in MFMA order, with no permutation after the arithmetic (22 VALU instructions as
// compiled: each mask-and-insert is a v_and_b32 + v_or_b32 pair).
__device__ __forceinline__ half8 dequant8(uint32_t d, half2_t s2) {
#pragma clang fp contract(off)
  d ^= 0x88888888u;  // two's complement nibble n -> n + 8 in [0, 15]
  const uint32_t e = d >> 4;
  const uint32_t lo = __builtin_amdgcn_perm(e, d, 0x05040100u);  // d.b0 d.b1 e.b0 e.b1
  const uint32_t hi = __builtin_amdgcn_perm(e, d, 0x07060302u);  // d.b2 d.b3 e.b2 e.b3
  // 0x6400 | v is the fp16 value 1024 + v; minus 1032 gives the signed nibble exactly
  const half2_t bias = {(half_t)1032.0f, (half_t)1032.0f};
  u32x4 r;
  r[0] = as_u32((as_h2((lo & 0x000F000Fu) | 0x64006400u) - bias) * s2);         // k0, k1
  r[1] = as_u32((as_h2(((lo >> 8) & 0x000F000Fu) | 0x64006400u) - bias) * s2);  // k2, k3
  r[2] = as_u32((as_h2((hi & 0x000F000Fu) | 0x64006400u) - bias) * s2);         // k4, k5
  r[3] = as_u32((as_h2(((hi >> 8) & 0x000F000Fu) | 0x64006400u) - bias) * s2);  // k6, k7
  return as_half8(r);
}

// Store C[m][nb .. nb + 3] (columns past N dropped): to the fp32 partials of split
// blockIdx.z, or as fp16 to the output.
__device__ __forceinline__ void store_row_piece(const Params& p, floatx4 v, int m, int nb) {
  if (p.partial) {
    float* dst = p.partial + ((int64_t)blockIdx.z * p.M + m) * p.N + nb;
    if (nb + 3 < p.N && (p.N & 3) == 0) {
      *(floatx4*)dst = v;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < p.N) dst[i] = v[i];
    }
  } else {
    half_t* dst = p.out + (int64_t)m * p.out_stride + nb;
    const half4 h = to_half4(v);
    if (nb + 3 < p.N && ((uintptr_t)dst & 7) == 0) {
      *(half4*)dst = h;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < p.N) dst[i] = h[i];
    }
  }
}

// Store a workgroup's 64-column x (16 * kMSub)-row tile.  Lane (row, grp) of wave w holds
// C[m0 + 16j + row][n0 + 16w + 4grp + i] in acc[j][i].  With K split over blockIdx.z the
// tile goes to the fp32 partials (reduce_kernel adds them), otherwise to the fp16 output.
template <int kMSub>
__device__ __forceinline__ void store_tile(const Params& p, const floatx4 (&acc)[kMSub], int m0,
                                           int n0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int nb = n0 + wave * 16 + 4 * (lane >> 4);
#pragma unroll
  for (int j = 0; j < kMSub; ++j) {
    const int m = m0 + 16 * j + row;
    if (m < p.M) store_row_piece(p, acc[j], m, nb);
  }
}

// ---------------------------------------------------------------------------------------
// RMSNorm (kernels/rms_norm.py:8-43): y = fp16((x * r) * w) with r = rsqrt(sum(x^2)/K + eps),
// all in fp32.  One wave reduces one row.

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Rows up to kRowChunks * 512 elements are held in registers (16 bytes per lane per 512
// elements), every load issued before the first use; longer rows loop.
constexpr int kRowChunks = 16;

__device__ __forceinline__ float sum_sq8(u32x4 v) {
  const half8 h = as_half8(v);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += (float)h[e] * (float)h[e];
  return s;
}

// r of one row of K (a multiple of 8) elements, computed by the calling wave
__device__ __forceinline__ float row_rsqrt(const half_t* xrow, int K, float eps, int lane) {
  float s = 0.f;
  if (K <= kRowChunks * 512) {
    u32x4 v[kRowChunks];
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int k = lane * 8 + i * 512;
      v[i] = k < K ? *(const u32x4*)(xrow + k) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) s += sum_sq8(v[i]);
  } else {
    for (int k = lane * 8; k < K; k += 512) s += sum_sq8(*(const u32x4*)(xrow + k));
  }
  s = wave_sum(s);
  return rsqrtf(s / (float)K + eps);
}

// eight normalized elements: fp16((x * r) * w), products rounded separately (no fma)
__device__ __forceinline__ u32x4 norm8(u32x4 xv, float r, u32x4 wv) {
#pragma clang fp contract(off)
  const half8 x = as_half8(xv);
  const half8 w = as_half8(wv);
  half8 y;
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (half_t)(((float)x[e] * r) * (float)w[e]);
  return as_u32x4(y);
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const half_t* x, int64_t x_stride, int M,
                                                      int K, const half_t* w, float eps,
                                                      half_t* out, int64_t out_stride) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const half_t* xr = x + (int64_t)m * x_stride;
  half_t* o = out + (int64_t)m * out_stride;
  if (K <= kRowChunks * 512) {  // the row is read once, into registers
    u32x4 v[kRowChunks], wv[kRowChunks];
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int k = lane * 8 + i * 512;
      v[i] = k < K ? *(const u32x4*)(xr + k) : u32x4{0, 0, 0, 0};
      wv[i] = k < K ? *(const u32x4*)(w + k) : u32x4{0, 0, 0, 0};
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) s += sum_sq8(v[i]);
    const float r = rsqrtf(wave_sum(s) / (float)K + eps);
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int k = lane * 8 + i * 512;
      if (k < K) *(u32x4*)(o + k) = norm8(v[i], r, wv[i]);
    }
    return;
  }
  const float r = row_rsqrt(xr, K, eps, lane);
  for (int k = lane * 8; k < K; k += 512)
    *(u32x4*)(o + k) = norm8(*(const u32x4*)(xr + k), r, *(const u32x4*)(w + k));
}

// One row normalized by the calling wave into dst (LDS or global), K a multiple of 8.
__device__ __forceinline__ void norm_row_to(const half_t* xr, const half_t* w, int K, float eps,
                                            half_t* dst, int lane) {
  if (K <= kRowChunks * 512) {
    u32x4 v[kRowChunks];
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int k = lane * 8 + i * 512;
      v[i] = k < K ? *(const u32x4*)(xr + k) : u32x4{0, 0, 0, 0};
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) s += sum_sq8(v[i]);
    const float r = rsqrtf(wave_sum(s) / (float)K + eps);
#pragma unroll
    for (int i = 0; i < kRowChunks; ++i) {
      const int k = lane * 8 + i * 512;
      if (k < K) *(u32x4*)(dst + k) = norm8(v[i], r, *(const u32x4*)(w + k));
    }
    return;
  }
  const float r = row_rsqrt(xr, K, eps, lane);
  for (int k = lane * 8; k < K; k += 512)
    *(u32x4*)(dst + k) = norm8(*(const u32x4*)(xr + k), r, *(const u32x4*)(w + k));
}

template <int MT, bool kInt4>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(Params p) {
  constexpr int kMSub = MT / 16;          // 16-row MFMA tiles per wave
  constexpr int kXLoads = MT / 16;        // 16-byte X loads per thread per group
  __shared__ __attribute__((aligned(16))) half_t xs[2][MT * kLdsRow];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int n = blockIdx.x * kNTile + wave * 16 + row;  // this lane's weight row
  const int nc = n < p.N ? n : p.N - 1;                 // rows past N compute, never store
  const int m0 = blockIdx.y * MT;
  const int groups = p.K / kGroup;
  const int g_begin = blockIdx.z * p.groups_per_split;
  const int g_end = min(g_begin + p.groups_per_split, groups);

  // X staging: thread t moves 16 bytes of rows t/16 + 16i, chunk t%16
  const int xr = threadIdx.x >> 4;
  const int xc = threadIdx.x & 15;
  u32x4 xreg[kXLoads];
  auto load_x = [&](int g) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
      const int m = m0 + xr + 16 * i;
      if (m < p.M)
        xreg[i] = *(const u32x4*)(p.x + (int64_t)m * p.x_stride + g * kGroup + xc * 8);
      else
        xreg[i] = u32x4{0, 0, 0, 0};
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      *(u32x4*)(&xs[buf][(xr + 16 * i) * kLdsRow + xc * 8]) = xreg[i];
  };

  // weights of this lane for one group: 16 bytes (int4) or 4 x 16 bytes (fp16)
  u32x4 wreg[kInt4 ? 1 : 4];
  half_t sreg = (half_t)0.0f;
  auto load_w = [&](int g) {
    if constexpr (kInt4) {
      wreg[0] = *(const u32x4*)(p.w + (int64_t)nc * p.w_stride + g * (kGroup / 2) + grp * 16);
      sreg = p.scales[(int64_t)nc * p.s_stride + g];
    } else {
      const half_t* wr = (const half_t*)p.w + (int64_t)nc * p.w_stride + g * kGroup + grp * 32;
#pragma unroll
      for (int s = 0; s < 4; ++s) wreg[s] = *(const u32x4*)(wr + 8 * s);
    }
  };

  floatx4 acc[kMSub];
#pragma unroll
  for (int j = 0; j < kMSub; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (g_begin < g_end) {
    load_x(g_begin);
    load_w(g_begin);
  }
  int buf = 0;
  for (int g = g_begin; g < g_end; ++g) {
    store_x(buf);
    __syncthreads();
    half8 wf[4];
    if constexpr (kInt4) {
      const half2_t s2 = {sreg, sreg};
#pragma unroll
      for (int s = 0; s < 4; ++s) wf[s] = dequant8(wreg[0][s], s2);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) wf[s] = as_half8(wreg[s]);
    }
    if (g + 1 < g_end) {  // next group's loads overlap this group's MFMAs
      load_x(g + 1);
      load_w(g + 1);
    }
    const half_t* xb = &xs[buf][row * kLdsRow + grp * 32];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int j = 0; j < kMSub; ++j) {
        const half8 xf = as_half8(*(const u32x4*)(xb + j * 16 * kLdsRow + 8 * s));
        acc[j] = mfma16x16x32(wf[s], xf, acc[j]);
      }
    }
    buf ^= 1;
  }

  store_tile<kMSub>(p, acc, m0, blockIdx.x * kNTile);
}

// ---------------------------------------------------------------------------------------
// Packed-weight GEMM for 17..64 rows with the K split added up in the same launch.
//
// A workgroup of eight multiplying waves and four loading waves computes a 64-column x MT-row
// tile over a slice of G <= 8 K groups.  Multiplying wave w = 4h + q takes output columns
// 32h .. 32h + 31 (column half h) and the q-th quarter of each phase's k-steps (32 k each),
// so the two waves of a SIMD (w and w + 4) read the same X fragments for different weights,
// and each weight is unpacked once.  Within a wave the next k-step's unpack is interleaved
// with the current k-step's MFMAs.  X fragments are read from LDS once per 32 output columns.
//
// The loading waves copy the slice's X tiles (MT rows x 256 bytes per group, 16-byte chunks
// XOR-permuted by row % 16) and W tiles (64 columns x 64 bytes per group, 16-byte chunks
// XOR-permuted by (column / 2) % 4) global -> LDS with `buffer_load ... lds`, in two phases
// (the first ceil(G / 2) groups, then the rest while the first phase is multiplied), so that
// a full memory queue stalls only those waves.  The multiplying waves load only the scales
// of their columns.  The four quarters' sums of each column half are then added through LDS
// in quarter order.
//
// K split: the workgroups of one column tile have block ids congruent modulo 8, which the
// dispatcher places on one XCD (checked once per device before this kernel is used), so a
// tile's partial sums and its arrival counter are shared through that XCD's L2.  Each
// workgroup stores its partial tile, waits until the stores are done, and increments the
// tile's counter; the workgroup that arrives last loads the other partials (bypassing L1),
// adds all of them in split order (the same sum whichever workgroup is last), writes the
// fp16 tile and sets the counter back to zero for the next call.  No workgroup waits for
// another.  Block id b: XCD group b % 8, split (b / 8) / T8, tile 8 * ((b / 8) % T8) + b % 8,
// with T8 = ceil(tiles / 8).
constexpr int kSkWaves = 8;                         // multiplying waves
constexpr int kSkLoaders = 4;                       // loading waves
constexpr int kSkMaxGroups = 8;                     // K groups per workgroup
constexpr int kSkTilesPerXcd = 256;                 // counters per XCD group and stream
constexpr int kSkMaxTiles = 8 * kSkTilesPerXcd;     // column tiles per call
constexpr int kSkStreamSlots = kXcdMaxSlots;        // streams per device with their own counters

template <int MT>
struct SkTile {
  static constexpr int kX = MT * 256;              // X tile of one group
  static constexpr int kW = kNTile * 64;           // W tile of one group
  static constexpr int kSlot = kX + kW;
  static constexpr int kXCopies = MT / 4;          // 1 KiB copies (16 rows of one X panel)
  static constexpr int kCopies = kXCopies + 4;     // + 4 of 16 W columns
  static constexpr int kMSub = MT / 16;            // 16-row blocks
  static constexpr int kBlocks = 4 * kMSub;        // 16 x 16 output blocks
  static constexpr int kOwn = kBlocks / kSkWaves;  // blocks each wave finishes
  static constexpr int kLds = kSkMaxGroups * kSlot;
  static_assert(kLds <= 160 * 1024, "the slots fit one CU's LDS");
  static_assert(kBlocks * 4 * 1024 + 16 <= kLds, "the reduction area fits the slots");
  static_assert(kOwn >= 1 && kBlocks % kSkWaves == 0, "whole blocks per wave");
};

// fp16 store of C[m][nb .. nb + 3] (columns past N dropped)
__device__ __forceinline__ void store_half4(const Params& p, floatx4 v, int m, int nb) {
  half_t* dst = p.out + (int64_t)m * p.out_stride + nb;
  const half4 h = to_half4(v);
  if (nb + 3 < p.N && ((uintptr_t)dst & 7) == 0) {
    *(half4*)dst = h;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nb + i < p.N) dst[i] = h[i];
  }
}

// dequant8 with each mask-and-insert as one v_and_or_b32 (the mask from a scalar register,
// the fp16 exponent bits from a vector register): 18 VALU instructions per eight weights,
// the same values bit for bit.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
  return r;
}

__device__ __forceinline__ half8 dequant8_ao(uint32_t d, half2_t s2, uint32_t mask, uint32_t bits) {
#pragma clang fp contract(off)
  d ^= 0x88888888u;
  const uint32_t e = d >> 4;
  const uint32_t lo = __builtin_amdgcn_perm(e, d, 0x05040100u);
  const uint32_t hi = __builtin_amdgcn_perm(e, d, 0x07060302u);
  const half2_t bias = {(half_t)1032.0f, (half_t)1032.0f};
  u32x4 r;
  r[0] = as_u32((as_h2(and_or(lo, mask, bits)) - bias) * s2);
  r[1] = as_u32((as_h2(and_or(lo >> 8, mask, bits)) - bias) * s2);
  r[2] = as_u32((as_h2(and_or(hi, mask, bits)) - bias) * s2);
  r[3] = as_u32((as_h2(and_or(hi >> 8, mask, bits)) - bias) * s2);
  return as_half8(r);
}

template <int MT>
__global__ __launch_bounds__((kSkWaves + kSkLoaders) * 64, 1) void gemm_sk_kernel(Params p) {
  using T = SkTile<MT>;
  constexpr int kMSub = T::kMSub;
  __shared__ __attribute__((aligned(16))) char lds[T::kLds];

  const int t8 = (p.tiles + 7) >> 3;
  const int xg = blockIdx.x & 7, kk = blockIdx.x >> 3;
  const int s = kk / t8;
  const int t = 8 * (kk - s * t8) + xg;
  if (t >= p.tiles) return;  // padding of the last XCD group (uniform, before any barrier)

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool producer = w >= kSkWaves;
  const int l = w - kSkWaves;  // loading wave index
  const int h = (w >> 2) & 1;  // column half
  const int q = w & 3;         // k-step of every group
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int n0 = t * kNTile;
  const int groups = p.K / kGroup;
  const int g_begin = s * p.groups_per_split;
  const int G = min(p.groups_per_split, groups - g_begin);  // 1 .. 8 (host plan)
  const int GA = (G + 1) >> 1;                               // groups of phase A
  const int GB = G - GA;                                     // of phase B

  floatx4 acc[2][kMSub];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int i = 0; i < kMSub; ++i) acc[jj][i] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (producer) {
    // X rows past M and weight rows past N read zeros through the buffer bounds
    const rsrc_t xr = raw_rsrc(p.x, (int)((min(MT, p.M) - 1) * p.x_stride * 2 + p.K * 2));
    const rsrc_t wr = raw_rsrc(p.w + (int64_t)n0 * p.w_stride,
                              (int)((min(kNTile, p.N - n0) - 1) * p.w_stride + p.K / 2));
    // X of a group is stored as four panels, panel c holding 16-byte chunks 4c .. 4c + 3 of
    // every row (64 bytes per row); sub-chunk kk of row r of panel c sits at slot
    // kk ^ ((r / 2) % 4) ^ c.  Loading wave l fills panel l: its copy i covers rows 16i ..
    // 16i + 15 (row 16i + lane / 4, slot lane % 4).  Then W columns 16cw .. 16cw + 15 (column
    // 16cw + lane / 4, slot lane % 4 <- 16-byte chunk slot ^ ((column / 2) % 4)); loading wave
    // l issues W copy cw = l of every group.  Both layouts make the fragment reads of 16
    // consecutive rows (columns) at one chunk conflict-free; per-lane offsets at group 0.
    constexpr int kXPer = T::kXCopies / kSkLoaders;
    static_assert(T::kXCopies % kSkLoaders == 0 && kSkLoaders == 4,
                  "one X panel per loading wave, whole 16-row copies");
    int xoff[kXPer];
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int r = 16 * i + (lane >> 2);
      const int kk = (lane & 3) ^ ((lane >> 3) & 3) ^ l;
      xoff[i] = r * (int)p.x_stride * 2 + ((4 * l + kk) << 4);
    }
    const int woff = (16 * l + (lane >> 2)) * (int)p.w_stride + (((lane & 3) ^ ((lane >> 3) & 3)) << 4);
    auto issue = [&](int u0, int gp) {
#pragma unroll 1
      for (int u = u0; u < u0 + gp; ++u) {
        const uint32_t base = lds_addr(lds + u * T::kSlot);
        const int g = g_begin + u;
#pragma unroll
        for (int i = 0; i < kXPer; ++i)
          lds_copy16(xr, base + l * (MT * 64) + i * 1024, xoff[i], g * 256);
        lds_copy16(wr, base + T::kX + l * 1024, woff, g * (kGroup / 2));
      }
    };
    // phase A, then phase B while the other waves multiply phase A
    issue(0, GA);
    wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (GB > 0) {
      issue(GA, GB);
      wait_vmcnt<0>();
      asm volatile("s_barrier" ::: "memory");
    }
  } else {
    // Wave (h, q) multiplies the q-th quarter of each phase's k-steps (a k-step is 32 k of one
    // group: lane group grp supplies k = 32 grp + 8k .. +7, weight dword k of the lane's 16
    // bytes and X chunk 4 grp + k) for its two column blocks j = 2h, 2h + 1.  In a phase of gp
    // groups from u0 these are k-steps q gp .. q gp + gp - 1, in group u0 + (q gp) / 4 and
    // possibly the next one (the same group for all four when gp = 4).  The scales of the
    // lane's columns (16j + row; past N the last column, times zero weights) for those two
    // groups: sv[jj][second].  These are the only memory loads of these waves, so the
    // compiler's own wait before their first use waits for nothing else.
    struct Scales {  // bits of sv[jj][0] in the low half, sv[jj][1] in the high half
      uint32_t v0, v1;
    };
    auto load_scales = [&](int u0, int gp) {
      const int uf = u0 + (q * gp) / 4;
      const int us = min(uf + 1, G - 1);
      uint32_t v[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint16_t* sp = (const uint16_t*)p.scales +
                             (int64_t)min(n0 + 16 * (2 * h + jj) + row, p.N - 1) * p.s_stride + g_begin;
        v[jj] = (uint32_t)sp[uf] | ((uint32_t)sp[us] << 16);
      }
      return Scales{v[0], v[1]};
    };
    const Scales sca = load_scales(0, GA);
    const Scales scb = GB > 0 ? load_scales(GA, GB) : sca;
    const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t bits = 0x64006400u;

    // One phase, software pipelined: k-step i + 2's fragments are read and k-step i + 1's
    // weights unpacked while k-step i's MFMAs run.
    auto run_phase = [&](int u0, int gp, const Scales sv) {
      const int ks0 = q * gp;
      const int uf = u0 + ks0 / 4;
      u32x4 xv[3][kMSub];
      uint32_t wd[3][2];
      bool sec[3];
      half8 wf[2][2];
      auto read = [&](int b, int i) {  // k-step ks0 + i
        const int ks = ks0 + i;
        const int u = u0 + ks / 4, k = ks & 3;
        const char* slot = lds + u * T::kSlot;
#pragma unroll
        for (int ii = 0; ii < kMSub; ++ii)
          xv[b][ii] = *(const u32x4*)(slot + grp * (MT * 64) + (16 * ii + row) * 64 +
                                      ((k ^ ((row >> 1) & 3) ^ grp) << 4));
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          wd[b][jj] = *(const uint32_t*)(slot + T::kX + (16 * (2 * h + jj) + row) * 64 +
                                         ((grp ^ ((row >> 1) & 3)) << 4) + 4 * k);
        sec[b] = u != uf;
      };
      auto unpack = [&](int b, int i) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint32_t both = jj ? sv.v1 : sv.v0;
          const half_t sc = __builtin_bit_cast(half_t, (uint16_t)(both >> (sec[b] ? 16 : 0)));
          wf[i & 1][jj] = dequant8_ao(wd[b][jj], half2_t{sc, sc}, mask, bits);
        }
      };
      read(0, 0);
      read(1, min(1, gp - 1));
      unpack(0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < gp) {  // uniform
          if (i + 2 < gp) read((i + 2) % 3, i + 2);
          // k-step i + 1's unpack (unused past the phase) between k-step i's MFMAs
          if (i < 3) unpack((i + 1) % 3, i + 1);
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int ii = 0; ii < kMSub; ++ii) {
              acc[jj][ii] = mfma16x16x32(wf[i & 1][jj], as_half8(xv[i % 3][ii]), acc[jj][ii]);
              if (i < 3) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 36 / (2 * kMSub), 0);  // then VALU
              }
            }
        }
      }
    };

    asm volatile("s_barrier" ::: "memory");  // phase A has landed
    run_phase(0, GA, sca);
    if (GB > 0) {
      asm volatile("s_barrier" ::: "memory");  // phase B has landed
      run_phase(GA, GB, scb);
    }
  }

  // The quarters' sums, added in quarter order through the (now idle) slots: block b = 4 i + j
  // of quarter q at red[(b * 4 + q) * 64 + lane]; wave (h, q) finishes blocks 2 i + jj = q * kOwn
  // .. + kOwn - 1 of its half.  The loading waves only take part in the barriers.
  floatx4* red = (floatx4*)lds;
  __syncthreads();  // every wave is done with the slots
  if (!producer) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int i = 0; i < kMSub; ++i)
        red[((4 * i + 2 * h + jj) * 4 + q) * 64 + lane] = acc[jj][i];
  }
  __syncthreads();
  floatx4 v[T::kOwn];
  int ob[T::kOwn];  // block index (4 i + j) of each finished block
#pragma unroll
  for (int o = 0; o < T::kOwn; ++o) {
    const int hb = q * T::kOwn + o;  // block within the half: 2 i + jj
    const int b = 4 * (hb >> 1) + 2 * h + (hb & 1);
    ob[o] = b;
    v[o] = red[(b * 4) * 64 + lane];
#pragma unroll
    for (int qq = 1; qq < 4; ++qq) v[o] += red[(b * 4 + qq) * 64 + lane];
  }

  if (p.ksplit > 1) {
    // partial tile of (t, s): block b at [b][lane], 1 KiB per block
    floatx4* part = (floatx4*)p.partial + (int64_t)t * p.ksplit * T::kBlocks * 64;
    if (!producer) {
#pragma unroll
      for (int o = 0; o < T::kOwn; ++o) part[((int64_t)s * T::kBlocks + ob[o]) * 64 + lane] = v[o];
    }
    if (!p.counters) return;  // no counters: sk_reduce_kernel adds the splits
    wait_vmcnt<0>();  // the stores are in L2 before the counter moves
    __syncthreads();
    unsigned* flag = (unsigned*)(lds + T::kLds - 16);
    if (threadIdx.x == 0) {
      unsigned* ctr = p.counters + (t & 7) * kSkTilesPerXcd + (t >> 3);
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (old == (unsigned)p.ksplit - 1)  // every other split has arrived: clear for the next call
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      *flag = old;
    }
    __syncthreads();
    if (*flag != (unsigned)p.ksplit - 1 || producer) return;
    // the partials of every split, added in split order (own sums in place of split s),
    // loaded with sc0 (L1 bypassed, served by the XCD's L2)
    const __amdgpu_buffer_rsrc_t pr =
        __builtin_amdgcn_make_buffer_rsrc(part, (short)0, p.ksplit * T::kBlocks * 1024, 0x00020000);
    // every load of a batch of eight splits goes out before the first add
    floatx4 sum[T::kOwn] = {};
    for (int s0 = 0; s0 < p.ksplit; s0 += 8) {
      floatx4 pv[T::kOwn][8] = {};
#pragma unroll
      for (int o = 0; o < T::kOwn; ++o)
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (s0 + k < p.ksplit && s0 + k != s)
            pv[o][k] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                             pr, (((s0 + k) * T::kBlocks + ob[o]) * 64 + lane) * 16, 0, 1));
#pragma unroll
      for (int o = 0; o < T::kOwn; ++o)
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (s0 + k < p.ksplit) sum[o] += s0 + k == s ? v[o] : pv[o][k];
    }
#pragma unroll
    for (int o = 0; o < T::kOwn; ++o) v[o] = sum[o];
  }
  if (producer) return;
#pragma unroll
  for (int o = 0; o < T::kOwn; ++o) {
    const int m = 16 * (ob[o] >> 2) + row;
    if (m < p.M) store_half4(p, v[o], m, n0 + 16 * (ob[o] & 3) + 4 * grp);
  }
}

// gemm_sk_kernel's split sums in a second launch, for streams without arrival counters: the
// same additions in the same order as the last workgroup of a tile (from 0.f, split 0 first),
// so both paths give the same bits.  One thread per (tile, 16 x 16 block, lane).
template <int MT>
__global__ __launch_bounds__(256) void sk_reduce_kernel(Params p) {
  using T = SkTile<MT>;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.tiles * T::kBlocks * 64) return;
  const int lane = (int)(idx & 63);
  const int b = (int)((idx >> 6) % T::kBlocks);
  const int t = (int)(idx / (64 * T::kBlocks));
  const floatx4* part = (const floatx4*)p.partial + (int64_t)t * p.ksplit * T::kBlocks * 64;
  floatx4 sum = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.ksplit; ++s) sum += part[((int64_t)s * T::kBlocks + b) * 64 + lane];
  const int m = 16 * (b >> 2) + (lane & 15);
  if (m < p.M) store_half4(p, sum, m, t * kNTile + 16 * (b & 3) + 4 * (lane >> 4));
}

// Arrival counters of gemm_sk_kernel: one per column tile and stream slot, laid out
// [XCD group][tile / 8] so that each XCD group's counters share no cache line with another's.
__device__ __attribute__((aligned(256))) unsigned sk_counters[kSkStreamSlots * kSkMaxTiles];


// Prefill-sized calls: the MFMA kernels above spend most of their time dequantizing (each
// weight is dequantized once per row tile) at these sizes, so the weight is dequantized once
// into the workspace and a plain fp16 GEMM runs on it: wide_gemm_kernel.
//
// C[M, N] = X[M, K] * W[N, K]^T, fp16 in and out, fp32 accumulation, K a multiple of 64.
// One workgroup per 256 x 256 tile of C, four waves, one per SIMD.  Wave w owns 128 rows
// (m, 128 * (w / 2)..) x 128 columns (n, 128 * (w % 2)..) of the tile: 8 x 8 MFMA tiles of
// v_mfma_f32_16x16x32_f16, W as the A operand and X^T as the B operand, 256 fp32 sums held
// in the accumulation registers (AGPRs), so each 16-byte fragment read from LDS feeds eight
// MFMAs (a 64 x 128 wave tile feeds four to eight).  Per 64-wide K step the tile's X and W
// rows (128 bytes each, 16-byte chunk c of row r at slot c ^ ((r / 2) % 8), so the 16 rows a
// quarter-wave reads fall on distinct banks) are copied global->LDS with buffer_load ... lds
// into one of two 64 KiB stages.  A step is two k-substeps of 64 MFMAs: the second
// substep's 16 fragments are read between the first substep's MFMAs; after 48 of the second
// substep's MFMAs the wave waits for its copies of the next step and passes a barrier (every
// wave has then read this step's stage and landed the next), and the next step's first
// fragments are read between the last 16 MFMAs.  The copies of step t + 1 go out between
// the first substep's MFMAs of step t, into the stage every wave finished reading before
// the previous step's barrier.
constexpr int kGemmTile = 256;                     // rows and columns of C per workgroup
constexpr int kGemmK = 64;                         // K per step
constexpr int kGemmThreads = 256;
constexpr int kGemmRowB = kGemmK * 2;              // bytes per LDS row
constexpr int kGemmOperand = kGemmTile * kGemmRowB;  // 32 KiB: X or W rows of one step
constexpr int kGemmStage = 2 * kGemmOperand;         // 64 KiB: X rows, then W rows

struct GemmParams {
  const half_t* x;
  int64_t ldx;
  const half_t* w;
  int64_t ldw;
  half_t* o;
  int64_t ldo;
  int M, N, K;
  int tiles_m;
  int band;     // tiles_m / 8 when tiles_m % 8 == 0 (row tiles banded by XCD), else 0
  int vec_out;  // output rows 16-byte aligned and N % 8 == 0: 16-byte stores
};

__global__ __launch_bounds__(kGemmThreads, 1) void wide_gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kGemmStage];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave & 1, wm = wave >> 1;  // wave tile: columns 128 * wn.., rows 128 * wm..
  // Tile order: with p.band, block id L runs on XCD L % 8 and XCD e takes row tiles
  // e * band .. e * band + band - 1 against every column tile, so the X rows of its tiles
  // stay in its own L2; otherwise row tiles vary fastest.
  int tm, tn;
  {
    const int L = blockIdx.x;
    if (p.band) {
      const int t = L >> 3;
      tm = (L & 7) * p.band + t % p.band;
      tn = t / p.band;
    } else {
      tm = L % p.tiles_m;
      tn = L / p.tiles_m;
    }
  }
  const int m0 = tm * kGemmTile, n0 = tn * kGemmTile;
  const int rows_x = min(kGemmTile, p.M - m0), rows_w = min(kGemmTile, p.N - n0);
  // descriptors over exactly the tile's rows: lanes of rows past M or N read zeros
  const rsrc_t xr = raw_rsrc(p.x + (int64_t)m0 * p.ldx,
                             (int)(((int64_t)(rows_x - 1) * p.ldx + p.K) * 2));
  const rsrc_t wr = raw_rsrc(p.w + (int64_t)n0 * p.ldw,
                             (int)(((int64_t)(rows_w - 1) * p.ldw + p.K) * 2));
  // this wave copies rows 64w .. 64w + 63 of X and of W: eight instructions of 8 rows each
  // per operand; lane l fills slot l % 8 of row r0 + l / 8 with chunk (l % 8) ^ ((r / 2) % 8)
  int xoff[8], woff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xoff[i] = r < rows_x ? (int)((int64_t)r * p.ldx * 2) + (c << 4) : 0x7ffffff0;
    woff[i] = r < rows_w ? (int)((int64_t)r * p.ldw * 2) + (c << 4) : 0x7ffffff0;
  }
  const uint32_t lds0 = lds_addr(lds);
  const int steps = p.K / kGemmK;
  // copy q (0..15) of step kt: X rows for q < 8, W rows for q >= 8
  auto copy = [&](int kt, int q) {
    const uint32_t base = lds0 + (kt & 1) * kGemmStage;
    if (q < 8)
      lds_copy16(xr, base + (64 * wave + 8 * q) * kGemmRowB, xoff[q], kt * kGemmRowB);
    else
      lds_copy16(wr, base + kGemmOperand + (64 * wave + 8 * (q - 8)) * kGemmRowB, woff[q - 8],
                 kt * kGemmRowB);
  };

  floatx4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // fragment q of k-substep s: W tile q (q < 8) or X tile q - 8, row 16 * tile + fr, chunk
  // 4s + fg; rows 16i + fr share (row / 2) % 8 with row fr
  const int fr = lane & 15, fg = lane >> 4;
  const int sw = (fr >> 1) & 7;
  const int xrow0 = (128 * wm + fr) * kGemmRowB;
  const int wrow0 = kGemmOperand + (128 * wn + fr) * kGemmRowB;
  auto frag = [&](const char* st, int s, int q) {
    const int row0 = q < 8 ? wrow0 + q * 16 * kGemmRowB : xrow0 + (q - 8) * 16 * kGemmRowB;
    return as_half8(*(const u32x4*)(st + row0 + (((4 * s + fg) ^ sw) << 4)));
  };
  half8 f0[16], f1[16];
  // the scheduler keeps each group of MFMAs with its reads and copies (sched_barrier)
  auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

#pragma unroll
  for (int q = 0; q < 16; ++q) copy(0, q);
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  fence();
#pragma unroll
  for (int q = 0; q < 16; ++q) f0[q] = frag(lds, 0, q);
  fence();
  auto step = [&](int kt, auto more_c) {
    constexpr bool more = decltype(more_c)::value;  // a step follows
    const char* st = lds + (kt & 1) * kGemmStage;
    // substep 0 on f0; substep 1's fragments read and the next step's copies issued
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      f1[g] = frag(st, 1, g);
      if constexpr (more) copy(kt + 1, g);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int e = 4 * g + t, i = e >> 3, j = e & 7;
        acc[i][j] = mfma16x16x32(f0[i], f0[8 + j], acc[i][j]);
      }
      fence();
    }
    // substep 1 on f1: 48 MFMAs, the wait and barrier, then 16 MFMAs with the next step's
    // substep-0 fragments read between them
#pragma unroll
    for (int g = 0; g < 12; ++g) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int e = 4 * g + t, i = e >> 3, j = e & 7;
        acc[i][j] = mfma16x16x32(f1[i], f1[8 + j], acc[i][j]);
      }
      fence();
    }
    if constexpr (more) {
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      fence();
    }
    const char* nst = lds + ((kt + 1) & 1) * kGemmStage;
#pragma unroll
    for (int g = 12; g < 16; ++g) {
      if constexpr (more) {
#pragma unroll
        for (int u = 0; u < 4; ++u) f0[4 * (g - 12) + u] = frag(nst, 0, 4 * (g - 12) + u);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int e = 4 * g + t, i = e >> 3, j = e & 7;
        acc[i][j] = mfma16x16x32(f1[i], f1[8 + j], acc[i][j]);
      }
      fence();
    }
  };
  for (int kt = 0; kt + 1 < steps; ++kt) step(kt, std::true_type{});
  step(steps - 1, std::false_type{});
  __builtin_amdgcn_s_barrier();  // every wave is done with the stages
  fence();

  // Lane (m = 16j + fr, fg) holds C[m][16i + 4fg .. +3] of the wave's block.  Rows go
  // through the wave's own 32 KiB of LDS (fp16, 256 bytes a row, chunk c of row m at
  // c ^ (m % 16)) so that 16 lanes store one row's 256 bytes.
  char* cs = lds + wave * (128 * 256);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int m = 16 * j + fr;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = 2 * i + (fg >> 1);
      *(half4*)(cs + m * 256 + ((c ^ (m & 15)) << 4) + ((fg & 1) << 3)) = to_half4(acc[i][j]);
    }
  }
  wave_lds_sync();
  const int sr = lane >> 4, sc = lane & 15;
  const int gn = n0 + 128 * wn + 8 * sc;
#pragma unroll 4
  for (int q = 0; q < 32; ++q) {
    const int m = 4 * q + sr;
    const u32x4 v = *(const u32x4*)(cs + m * 256 + ((sc ^ (m & 15)) << 4));
    const int gm = m0 + 128 * wm + m;
    if (gm >= p.M || gn >= p.N) continue;
    half_t* dst = p.o + (int64_t)gm * p.ldo + gn;
    if (p.vec_out) {
      *(u32x4*)dst = v;
    } else {
      const half8 h = as_half8(v);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (gn + e < p.N) dst[e] = h[e];
    }
  }
}

// C[M, N] (ldc) = X[M, K] (ldx) * W[N, K]^T (ldw), all fp16 row-major, fp32 accumulation;
// K a multiple of 64, rows of X and W 16-byte aligned.
inline int f16_gemm(const half_t* x, int64_t ldx, const half_t* w, int64_t ldw, half_t* out,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  if (K % kGemmK || ((int64_t)(kGemmTile - 1) * std::max(ldx, ldw) + K) * 2 >= 0x7ffffff0) {
    set_error("fi_int4_matmul: 256 rows of X or W span 2^31 bytes or more");
    return FI_ERR_UNSUPPORTED;
  }
  GemmParams p;
  p.x = x;
  p.ldx = ldx;
  p.w = w;
  p.ldw = ldw;
  p.o = out;
  p.ldo = ldc;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.tiles_m = (int)((M + kGemmTile - 1) / kGemmTile);
  const int64_t tiles_n = (N + kGemmTile - 1) / kGemmTile;
  const int64_t tiles = p.tiles_m * tiles_n;
  if (tiles > 0x7fffffff) {
    set_error("fi_int4_matmul: too many output tiles");
    return FI_ERR_UNSUPPORTED;
  }
  p.band = p.tiles_m % 8 == 0 ? p.tiles_m / 8 : 0;
  p.vec_out = ((uintptr_t)out & 15) == 0 && ldc % 8 == 0 && N % 8 == 0;
  hipLaunchKernelGGL(wide_gemm_kernel, dim3((unsigned)tiles), dim3(kGemmThreads), 0, st, p);
  return check_launch("fi_int4_matmul");
}

// Decode-sized calls (16 rows of X per blockIdx.y): one workgroup per 16 output columns.
// The kW waves take interleaved groups (g = wave, wave + kW, ...), so K is split inside
// the workgroup and no partials leave it.  Each lane issues the loads of kChunk groups at
// once (16 weight bytes, the scale, and 64 bytes of its X row per group) before any math,
// so one memory latency covers the chunk; the kW waves' sums are added through LDS in
// a fixed order.
template <bool kInt4, int kChunk, bool kNorm, int kW>
__global__ __launch_bounds__(64 * kW, kNorm ? 1 : 2) void gemv_kernel(Params p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + row;
  const int nc = n < p.N ? n : p.N - 1;
  const int m = blockIdx.y * 16 + row;  // the X row this lane supplies
  const bool m_ok = m < p.M;
  // MFMA output column j depends on X row j only, and the columns of rows past M are never
  // stored: those lanes read zeros (or, from the normalized rows in LDS, a valid row)
  const int groups = p.K / kGroup;
  // fused norm: the workgroup's (at most 16, in practice a few) rows are normalized once
  // into LDS, [rows, K] fp16, and the X operand is read from there
  extern __shared__ __attribute__((aligned(16))) half_t xn[];
  const int rows_n = min(16, p.M - (int)blockIdx.y * 16);
  const half_t* xrow_n = xn + min(row, rows_n - 1) * p.K;

  // Issue the loads of one chunk (kChunk groups of this wave, g0, g0 + kW, ...): every load
  // goes out before any math and without branches (groups past the end reload the last
  // group and are skipped), so one latency covers the chunk.
  u32x4 wv[kInt4 ? kChunk : 4 * kChunk];
  half_t sv[kChunk];
  u32x4 xv[kNorm ? 1 : 4 * kChunk];
  // X through a buffer descriptor over this workgroup's rows: lanes of rows past M use an
  // offset past the end and read zeros with no memory request and no branch (the host
  // rejects calls whose 16 rows span more than 0x7ffffff0 bytes)
  const __amdgpu_buffer_rsrc_t xr_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (int64_t)blockIdx.y * 16 * p.x_stride), (short)0,
      (int)(((int64_t)(rows_n - 1) * p.x_stride + p.K) * 2), 0x00020000);
  const int x_off0 = m_ok ? (int)(((int64_t)row * p.x_stride + grp * 32) * 2) : 0x7ffffff0;
  auto load_chunk = [&](int g0) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int g = min(g0 + kW * c, groups - 1);
      if constexpr (kInt4) {
        wv[c] = *(const u32x4*)(p.w + (int64_t)nc * p.w_stride + g * (kGroup / 2) + grp * 16);
        sv[c] = p.scales[(int64_t)nc * p.s_stride + g];
      } else {
        const half_t* wr = (const half_t*)p.w + (int64_t)nc * p.w_stride + g * kGroup + grp * 32;
#pragma unroll
        for (int s = 0; s < 4; ++s) wv[4 * c + s] = *(const u32x4*)(wr + 8 * s);
      }
      if constexpr (!kNorm) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xv[4 * c + s] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         xr_rsrc, m_ok ? x_off0 + (g * kGroup + 8 * s) * 2 : x_off0, 0, 0));
      }
    }
  };

  // the first chunk's weights are in flight while the rows are normalized; the scheduling
  // barriers keep every load of a chunk ahead of its math (the scheduler would otherwise
  // start the math after the first few loads and issue the rest one latency later)
  if constexpr (kNorm) {
    // Wave r normalizes row r.  Its x row and the norm weight are loaded before the first
    // chunk's weights: loads complete in issue order, so the norm waits for its own data
    // only and runs while the weights stream in.  Rows longer than kRowChunks * 512, and rows
    // past the kW-th, are normalized after the weights' loads by norm_row_to.
    const bool in_regs = p.K <= kRowChunks * 512 && wave < rows_n;  // uniform
    u32x4 xr_v[kRowChunks], nw_v[kRowChunks];
    if (in_regs) {
      const half_t* xrow = p.x + (int64_t)(blockIdx.y * 16 + wave) * p.x_stride;
#pragma unroll
      for (int i = 0; i < kRowChunks; ++i) {
        const int k = lane * 8 + i * 512;
        xr_v[i] = k < p.K ? *(const u32x4*)(xrow + k) : u32x4{0, 0, 0, 0};
        nw_v[i] = k < p.K ? *(const u32x4*)(p.norm_w + k) : u32x4{0, 0, 0, 0};
      }
    }
    load_chunk(wave);
    __builtin_amdgcn_sched_barrier(0);
    if (in_regs) {
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < kRowChunks; ++i) sq += sum_sq8(xr_v[i]);
      const float r = rsqrtf(wave_sum(sq) / (float)p.K + p.eps);
#pragma unroll
      for (int i = 0; i < kRowChunks; ++i) {
        const int k = lane * 8 + i * 512;
        if (k < p.K) *(u32x4*)(xn + wave * p.K + k) = norm8(xr_v[i], r, nw_v[i]);
      }
    }
    for (int r = in_regs ? wave + kW : wave; r < rows_n; r += kW)
      norm_row_to(p.x + (int64_t)(blockIdx.y * 16 + r) * p.x_stride, p.norm_w, p.K, p.eps,
                  xn + r * p.K, lane);
    __syncthreads();
  } else {
    load_chunk(wave);
    __builtin_amdgcn_sched_barrier(0);
  }

  // two accumulators, alternating by k-step, halve the chain of dependent MFMAs
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 acc2 = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int g0 = wave; g0 < groups; g0 += kW * kChunk) {
    if (g0 != wave) {
      load_chunk(g0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (g0 + kW * c < groups) {  // uniform across the wave
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          half8 wf;
          if constexpr (kInt4)
            wf = dequant8(wv[c][s], half2_t{sv[c], sv[c]});
          else
            wf = as_half8(wv[4 * c + s]);
          u32x4 xf;
          if constexpr (kNorm)
            xf = *(const u32x4*)(xrow_n + (g0 + kW * c) * kGroup + grp * 32 + 8 * s);
          else
            xf = xv[4 * c + s];
          if (s & 1)
            acc2 = mfma16x16x32(wf, as_half8(xf), acc2);
          else
            acc = mfma16x16x32(wf, as_half8(xf), acc);
        }
      }
      // one group's operands at a time: unbounded hoisting of the X reads and the
      // dequantization ahead of the MFMAs would spill
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  acc += acc2;

  __shared__ floatx4 red[kW][64];
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    floatx4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < kW; ++w) t += red[w][lane];
    if (m_ok) {
      const int nb = n0 + 4 * grp;
      half_t* dst = p.out + (int64_t)m * p.out_stride + nb;
      const half4 h = to_half4(t);
      if (nb + 3 < p.N && ((uintptr_t)dst & 7) == 0) {
        *(half4*)dst = h;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nb + i < p.N) dst[i] = h[i];
      }
    }
  }
}

// out[m, n] = fp16(sum over splits of partial[s, m, n]), splits added in order.
template <int V>
__global__ __launch_bounds__(256) void reduce_kernel(const float* partial, int splits, int M,
                                                     int N, half_t* out, int64_t out_stride) {
  // V consecutive outputs of one row per thread (V = 4: N % 4 == 0 and 8-byte aligned output
  // rows).  The partials of up to 8 splits are loaded before any is added, so one memory
  // latency covers them; the sum runs in split order from 0.f either way.
  typedef float fv __attribute__((ext_vector_type(V)));
  const int64_t total = (int64_t)M * N;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V; i < total;
       i += (int64_t)gridDim.x * blockDim.x * V) {
    fv s = {};
    for (int k0 = 0; k0 < splits; k0 += 8) {
      fv v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < splits)
          v[k] = __builtin_nontemporal_load((const fv*)(partial + (k0 + k) * total + i));
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < splits) s += v[k];
    }
    const int m = (int)(i / N);
    const int nn = (int)(i - (int64_t)m * N);
    half_t* dst = out + (int64_t)m * out_stride + nn;
    if constexpr (V == 4) {
      *(half4*)dst = to_half4(s);
    } else {
      dst[0] = (half_t)s[0];
    }
  }
}

// ---------------------------------------------------------------------------------------
// loader.py:9-41: symmetric groupwise INT4 quantization, with the reference's fp16 tensor
// arithmetic: amax = max|w| over the group (fp16), clamped below at fp16(1e-6); scale =
// fp16(fp32(amax) * fp32(1/7)) (torch multiplies by the reciprocal when a CUDA tensor is
// divided by a Python scalar); q = round_half_even(fp16(fp32(w) / fp32(scale))), clamped to
// [-8, 7].  gs / 8 lanes per group (gs a power of two from 8 to 512), 8 values per lane;
// a group's lanes are consecutive lanes of one wave, so they enter and leave the loop together.
__global__ __launch_bounds__(256) void quantize_kernel(const half_t* w, int64_t w_stride, int N,
                                                       int K, int gs, uint8_t* packed,
                                                       int64_t p_stride, half_t* scales,
                                                       int64_t s_stride) {
  const int groups = K / gs;
  const int lanes = gs / 8;          // per group
  const int shift = __builtin_ctz(lanes);
  const int64_t total = (int64_t)N * groups;
  const int lane16 = threadIdx.x & (lanes - 1);
  for (int64_t gi = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> shift; gi < total;
       gi += ((int64_t)gridDim.x * blockDim.x) >> shift) {
    const int nrow = (int)(gi / groups);
    const int g = (int)(gi - (int64_t)nrow * groups);
    const half8 v = as_half8(
        *(const u32x4*)(w + (int64_t)nrow * w_stride + (int64_t)g * gs + lane16 * 8));
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)v[e]));
    for (int d = 1; d < lanes; d <<= 1) amax = fmaxf(amax, __shfl_xor(amax, d, lanes));
    const float lo = (float)(half_t)1e-6f;
    amax = fmaxf(amax, lo);
    const half_t scale = (half_t)(amax * (1.0f / 7.0f));
    const float sf = (float)scale;
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float qf = (float)(half_t)((float)v[e] / sf);
      const float qr = fminf(fmaxf(__builtin_rintf(qf), -8.f), 7.f);
      word |= ((uint32_t)(int)qr & 0xFu) << (4 * e);
    }
    *(uint32_t*)(packed + (int64_t)nrow * p_stride + (int64_t)g * (gs / 2) + lane16 * 4) = word;
    if (lane16 == 0) scales[(int64_t)nrow * s_stride + g] = scale;
  }
}

// matmul.py:309-326 (_dequant_storage): W = fp16(q * scale), 8 values per thread (gs, the
// group size, a multiple of 8).
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* packed, int64_t p_stride,
                                                         const half_t* scales, int64_t s_stride,
                                                         int N, int K, int gs, half_t* w,
                                                         int64_t w_stride) {
  const int per_row = K / 8;
  const int64_t total = (int64_t)N * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int nrow = (int)(i / per_row);
    const int c = (int)(i - (int64_t)nrow * per_row);
    const uint32_t d = *(const uint32_t*)(packed + (int64_t)nrow * p_stride + c * 4);
    const half_t s = scales[(int64_t)nrow * s_stride + (c * 8) / gs];
    *(u32x4*)(w + (int64_t)nrow * w_stride + c * 8) = as_u32x4(dequant8(d, half2_t{s, s}));
  }
}

// Kernel, tile rows and split count for an (M, N, K) call; shared by the size query and
// the launch.  gemv_rows: X rows per gemv launch row (0 = use the tiled kernel).
struct Plan {
  int mt;
  int splits;
  int gemv_rows;
  bool dense;  // prefill-sized: dequantize once, then a plain fp16 GEMM (f16_gemm)
  bool sk;       // packed weights, 17..64 rows: gemm_sk_kernel (K split added in-launch)
};

// Dispatch thresholds (rows of X), chosen by measurement on MI355X: the one-pass kernel
// up to 16 rows, the tiled split-K kernels up to 128, the plain fp16 GEMM above.
constexpr int kGemvMaxM = 16;
constexpr int kDenseMinM = 129;

// int4: packed weights.  cus: compute units of the device.
inline Plan plan(int64_t M, int64_t N, int64_t K, bool int4, int cus) {
  Plan pl;
  pl.gemv_rows = 0;
  pl.dense = false;
  pl.sk = false;
  if (M >= kDenseMinM) {
    pl.dense = true;
    pl.mt = 0;
    pl.splits = 1;
    return pl;
  }
  if (M <= kGemvMaxM && (M + 15) / 16 <= 65535) {
    pl.gemv_rows = 16;
    pl.mt = 16;
    pl.splits = 1;
    return pl;
  }
  const int64_t groups = K / kGroup;
  const int64_t tiles = (N + kNTile - 1) / kNTile;
  if (int4 && M <= 64) {
    // one workgroup per (column tile, K split), at most eight groups each, about one per CU
    pl.sk = true;
    pl.mt = M <= 32 ? 32 : 64;
    const int64_t lo = (groups + kSkMaxGroups - 1) / kSkMaxGroups;
    const int64_t s = std::max<int64_t>(lo, std::min<int64_t>(groups, cus / tiles));
    const int64_t per = (groups + s - 1) / s;
    pl.splits = (int)((groups + per - 1) / per);
    return pl;
  }
  pl.mt = M <= 16 ? 16 : M <= 32 ? 32 : M <= 64 ? 64 : 128;
  const int64_t wgs = ((N + kNTile - 1) / kNTile) * ((M + pl.mt - 1) / pl.mt);
  int64_t s = 1;
  if (wgs < 256) {
    s = (512 + wgs - 1) / wgs;
    // keep the fp32 partials (written and read once) below the weight bytes
    const int64_t cap = std::max<int64_t>(1, K / (16 * std::max<int64_t>(M, 1)));
    s = std::min<int64_t>(std::min<int64_t>(s, cap), groups);
  }
  // every split gets the same whole number of groups
  const int64_t per = (groups + s - 1) / std::max<int64_t>(s, 1);
  pl.splits = (int)((groups + per - 1) / std::max<int64_t>(per, 1));
  if (pl.splits < 1) pl.splits = 1;
  return pl;
}

}  // namespace gemm
}  // namespace fi

namespace {

using fi::half_t;
using fi::gemm::f16_gemm;
using fi::gemm::dequantize_kernel;
using fi::gemm::rmsnorm_kernel;

// Shared validation for the linear-layer entry points; FI_OK when the operands are usable.
int check_linear(const char* fn, const void* x, int64_t x_stride, int64_t M, int64_t K,
                 const void* w, int64_t w_stride, const void* scales, int64_t s_stride,
                 int64_t N, int64_t groupsize, const void* out, int64_t out_stride) {
  using namespace fi;
  using namespace fi::gemm;
  if (M < 0 || N < 0 || K < 0) {
    set_error("%s: negative size", fn);
    return FI_ERR_INVALID;
  }
  if (M == 0 || N == 0) return FI_OK;
  const bool int4 = scales != nullptr;
  if (int4 && groupsize != kGroup) {
    set_error("%s: groupsize %lld not supported (only %d)", fn, (long long)groupsize, kGroup);
    return FI_ERR_UNSUPPORTED;
  }
  if (K == 0 || K % kGroup) {
    set_error("%s: K %lld must be a positive multiple of %d", fn, (long long)K, kGroup);
    return FI_ERR_UNSUPPORTED;
  }
  if (M >= (1ll << 30) || N >= (1ll << 30) || K >= (1ll << 30)) {
    set_error("%s: sizes too large", fn);
    return FI_ERR_UNSUPPORTED;
  }
  if (!x || !w || !out) {
    set_error("%s: null pointer", fn);
    return FI_ERR_INVALID;
  }
  const bool x_ok = ((uintptr_t)x & 15) == 0 && x_stride % 8 == 0 && x_stride >= K;
  const bool w_ok = int4 ? (((uintptr_t)w & 15) == 0 && w_stride % 16 == 0 && w_stride >= K / 2 &&
                            ((uintptr_t)scales & 1) == 0 && s_stride >= K / kGroup)
                         : (((uintptr_t)w & 15) == 0 && w_stride % 8 == 0 && w_stride >= K);
  if (!x_ok || !w_ok || ((uintptr_t)out & 1) || out_stride < N) {
    set_error("%s: rows must be 16-byte aligned and strides cover the rows "
              "(x_stride %lld, w_stride %lld, out_stride %lld)", fn, (long long)x_stride,
              (long long)w_stride, (long long)out_stride);
    return FI_ERR_INVALID;
  }
  return FI_OK;
}

// Arrival counters of gemm_sk_kernel for the stream `st`: one set per stream slot (other
// streams add their splits in a second launch), each zero at load and left zero by every
// call; only on a device where block ids congruent modulo 8 share an XCD.
unsigned* sk_counters_for(hipStream_t st) {
  using fi::gemm::kSkMaxTiles;
  constexpr int kMaxDevices = 64;
  static std::atomic<unsigned*> base[kMaxDevices];
  if (!fi::xcd_groups_ok(st)) return nullptr;
  const int slot = fi::xcd_stream_slot(st, 0, fi::gemm::kSkStreamSlots);
  if (slot < 0) return nullptr;
  hipDevice_t d;
  if (hipStreamGetDevice(st, &d) != hipSuccess || (int)d < 0 || (int)d >= kMaxDevices) return nullptr;
  unsigned* b = base[(int)d].load();
  if (!b) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != (int)d && hipSetDevice((int)d) != hipSuccess) return nullptr;
    void* addr = nullptr;
    const bool ok = hipGetSymbolAddress(&addr, HIP_SYMBOL(fi::gemm::sk_counters)) == hipSuccess;
    if (cur != (int)d) (void)hipSetDevice(cur);
    if (!ok || !addr) return nullptr;
    b = (unsigned*)addr;
    base[(int)d].store(b);
  }
  return b + (size_t)slot * kSkMaxTiles;
}

// gemm_sk_kernel addresses X and the weight tile rows with 32-bit buffer offsets.
bool dma_ok_sk(const fi::gemm::Params& p, const fi::gemm::Plan& pl) {
  using namespace fi::gemm;
  const int64_t x_span = (int64_t)pl.mt * p.x_stride * 2 + (int64_t)p.K * 2;
  const int64_t w_span = (int64_t)kNTile * p.w_stride + p.K / 2;
  return x_span < (1ll << 31) - 4096 && w_span < (1ll << 31) - 4096;
}

// kNorm: the RMSNorm is fused into the decode kernel (only on the gemv path).
template <bool kNorm>
void launch_linear(const fi::gemm::Params& base, bool int4, const fi::gemm::Plan& pl,
                   void* workspace, hipStream_t st) {
  using namespace fi::gemm;
  Params p = base;
  if (pl.sk && dma_ok_sk(p, pl)) {
    // the split's arrival counters; without them (more than kSkMaxTiles column tiles, a
    // stream past the per-device sets, a device whose dispatch does not group block ids by
    // XCD, or a first call under graph capture) the workgroups only store their partials and
    // sk_reduce_kernel adds them
    const int groups = p.K / kGroup;
    p.groups_per_split = (groups + pl.splits - 1) / pl.splits;
    p.partial = (float*)workspace;
    p.tiles = (p.N + kNTile - 1) / kNTile;
    p.ksplit = pl.splits;
    p.counters = pl.splits > 1 && p.tiles <= kSkMaxTiles ? sk_counters_for(st) : nullptr;
    const dim3 grid((unsigned)(8 * pl.splits * ((p.tiles + 7) / 8)));
    const dim3 block((kSkWaves + kSkLoaders) * 64);
    if (pl.mt == 32)
      hipLaunchKernelGGL(gemm_sk_kernel<32>, grid, block, 0, st, p);
    else
      hipLaunchKernelGGL(gemm_sk_kernel<64>, grid, block, 0, st, p);
    if (pl.splits > 1 && !p.counters) {
      const int64_t threads = (int64_t)p.tiles * 4 * (pl.mt / 16) * 64;
      const dim3 rgrid((unsigned)((threads + 255) / 256));
      if (pl.mt == 32)
        hipLaunchKernelGGL(sk_reduce_kernel<32>, rgrid, dim3(256), 0, st, p);
      else
        hipLaunchKernelGGL(sk_reduce_kernel<64>, rgrid, dim3(256), 0, st, p);
    }
    return;
  }
  if (kNorm || pl.gemv_rows) {
    p.partial = nullptr;
    p.groups_per_split = p.K / kGroup;
    const dim3 grid((unsigned)((p.N + 15) / 16), (unsigned)((p.M + 15) / 16), 1);
    const size_t lds = kNorm ? (size_t)std::min(p.M, 16) * p.K * sizeof(half_t) : 0;
    // packed weights: eight waves (two per SIMD hide the dequantization's VALU latency),
    // except with the fused norm, whose registers allow only one such workgroup per CU
    if (int4 && !kNorm)
      hipLaunchKernelGGL((gemv_kernel<true, 3, false, 8>), grid, dim3(512), lds, st, p);
    else if (int4)
      hipLaunchKernelGGL((gemv_kernel<true, 6, kNorm, 4>), grid, dim3(kThreads), lds, st, p);
    else
      hipLaunchKernelGGL((gemv_kernel<false, 3, kNorm, 4>), grid, dim3(kThreads), lds, st, p);
    return;
  }
  p.partial = pl.splits > 1 ? (float*)workspace : nullptr;
  const int groups = p.K / kGroup;
  p.groups_per_split = (groups + pl.splits - 1) / pl.splits;
  const dim3 grid((unsigned)((p.N + kNTile - 1) / kNTile), (unsigned)((p.M + pl.mt - 1) / pl.mt),
                  (unsigned)pl.splits);
#define FI_GEMM_LAUNCH(MT)                                                                    \
  do {                                                                                      \
    if (int4)                                                                               \
      hipLaunchKernelGGL((gemm_kernel<MT, true>), grid, dim3(kThreads), 0, st, p);           \
    else                                                                                    \
      hipLaunchKernelGGL((gemm_kernel<MT, false>), grid, dim3(kThreads), 0, st, p);          \
  } while (0)
  switch (pl.mt) {
    case 16: FI_GEMM_LAUNCH(16); break;
    case 32: FI_GEMM_LAUNCH(32); break;
    case 64: FI_GEMM_LAUNCH(64); break;
    default: FI_GEMM_LAUNCH(128); break;
  }
#undef FI_GEMM_LAUNCH
  if (pl.splits > 1) {
    const int64_t total = (int64_t)p.M * p.N;
    const bool v4 = p.N % 4 == 0 && p.out_stride % 4 == 0 && ((uintptr_t)p.out & 7) == 0;
    const int64_t blocks = std::min<int64_t>((total / (v4 ? 4 : 1) + 255) / 256, 4096);
    if (v4)
      hipLaunchKernelGGL(reduce_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st,
                         (const float*)workspace, pl.splits, p.M, p.N, p.out, p.out_stride);
    else
      hipLaunchKernelGGL(reduce_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, st,
                         (const float*)workspace, pl.splits, p.M, p.N, p.out, p.out_stride);
  }
}

fi::gemm::Params make_params(const void* x, int64_t x_stride, int64_t M, int64_t K,
                             const void* w, int64_t w_stride, const void* scales,
                             int64_t s_stride, int64_t N, void* out, int64_t out_stride) {
  fi::gemm::Params p;
  p.x = (const half_t*)x;
  p.x_stride = x_stride;
  p.M = (int)M;
  p.K = (int)K;
  p.N = (int)N;
  p.w = (const uint8_t*)w;
  p.w_stride = w_stride;
  p.scales = (const half_t*)scales;
  p.s_stride = s_stride;
  p.out = (half_t*)out;
  p.out_stride = out_stride;
  p.partial = nullptr;
  p.groups_per_split = 0;
  p.norm_w = nullptr;
  p.eps = 0.f;
  p.tiles = 0;
  p.ksplit = 1;
  p.counters = nullptr;
  return p;
}

// fp32 partials of a split call: gemm_sk_kernel's [tile][split][MT x 64] blocks, which also
// hold the two-launch path's [split][M][N] for the same split
size_t split_bytes(int64_t M, int64_t N, const fi::gemm::Plan& pl) {
  using fi::gemm::kNTile;
  if (pl.splits <= 1) return 0;
  if (pl.sk) return (size_t)pl.splits * ((N + kNTile - 1) / kNTile) * pl.mt * kNTile * sizeof(float);
  return (size_t)pl.splits * M * N * sizeof(float);
}

// The norm is fused into the decode kernel for a few rows (each workgroup normalizes them
// into LDS once); otherwise a separate RMSNorm pass writes the normalized rows into the
// workspace first (every column tile would re-read and re-normalize its rows).
bool fuse_norm(int64_t M, int64_t K, const fi::gemm::Plan& pl) {
  // up to 4 rows (measured: the fused call is faster than norm pass + GEMM there); the
  // decode kernel keeps its normalized rows in LDS: at most 64 KB of them
  constexpr int64_t kFuseMaxM = 4;
  return pl.gemv_rows && M <= kFuseMaxM && std::min<int64_t>(M, 16) * K * 2 <= 65536;
}

size_t round256(int64_t n) { return (size_t)((n + 255) / 256 * 256); }

size_t norm_rows_bytes(int64_t M, int64_t K) { return round256(M * K * 2); }

// Workspace layout of a call: [normalized rows (separate norm pass)] [dequantized weight
// (dense path, packed weights)] [fp32 partials (split K)], each 256-byte aligned.
struct Layout {
  size_t rows, weight, split, total;
};

Layout layout(int64_t M, int64_t N, int64_t K, const fi::gemm::Plan& pl, bool int4, bool norm) {
  Layout l;
  l.rows = norm && !fuse_norm(M, K, pl) ? norm_rows_bytes(M, K) : 0;
  l.weight = pl.dense && int4 ? round256(N * K * 2) : 0;
  l.split = round256((int64_t)split_bytes(M, N, pl));
  l.total = l.rows + l.weight + l.split;
  return l;
}

// What the size queries report: the larger of the packed and the fp16 weight forms.
size_t workspace_bytes_for(int64_t M, int64_t N, int64_t K, bool norm) {
  using fi::gemm::plan;
  const int cus = fi::device_cu_count(nullptr);
  return std::max(layout(M, N, K, plan(M, N, K, true, cus), true, norm).total,
                  layout(M, N, K, plan(M, N, K, false, cus), false, norm).total);
}

// One linear-layer call on any path; norm_w non-null applies RMSNorm to X first.
int run_linear(const char* fn, const void* x, int64_t x_stride, int64_t M, int64_t K,
               const void* norm_w, float eps, const void* w, int64_t w_stride,
               const void* scales, int64_t s_stride, int64_t N, void* out, int64_t out_stride,
               void* workspace, size_t workspace_bytes, hipStream_t st) {
  using namespace fi;
  using namespace fi::gemm;
  const bool int4 = scales != nullptr;
  const bool norm = norm_w != nullptr;
  const Plan pl = plan(M, N, K, int4, device_cu_count(st));
  const Layout l = layout(M, N, K, pl, int4, norm);
  if (l.total && (!workspace || workspace_bytes < l.total || ((uintptr_t)workspace & 255))) {
    set_error("%s: workspace of %zu bytes (256-byte aligned) needed, %zu given", fn, l.total,
              workspace ? workspace_bytes : (size_t)0);
    return FI_ERR_WORKSPACE;
  }
  if (!pl.dense && (M + (pl.mt ? pl.mt : 16) - 1) / (pl.mt ? pl.mt : 16) > 65535) {
    set_error("%s: M %lld too large", fn, (long long)M);
    return FI_ERR_UNSUPPORTED;
  }
  // the decode kernel addresses a workgroup's 16 X rows through one buffer descriptor whose
  // size must stay below the offset its idle lanes use (0x7ffffff0)
  const bool fused = norm && fuse_norm(M, K, pl);
  const int64_t gemv_x_stride = norm && !fused ? K : x_stride;
  if (pl.gemv_rows && (std::min<int64_t>(M, 16) - 1) * gemv_x_stride * 2 + K * 2 > 0x7ffffff0) {
    set_error("%s: 16 rows of X span 2^31 bytes or more (x_stride %lld)", fn,
              (long long)x_stride);
    return FI_ERR_UNSUPPORTED;
  }
  char* ws = (char*)workspace;
  Params p = make_params(x, x_stride, M, K, w, w_stride, scales, s_stride, N, out, out_stride);
  if (fused) {
    p.norm_w = (const half_t*)norm_w;
    p.eps = eps;
    launch_linear<true>(p, int4, pl, nullptr, st);
    return check_launch(fn);
  }
  if (norm) {  // separate norm pass into the workspace
    half_t* normed = (half_t*)ws;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st,
                       (const half_t*)x, x_stride, (int)M, (int)K, (const half_t*)norm_w, eps,
                       normed, K);
    p.x = normed;
    p.x_stride = K;
  }
  if (pl.dense) {
    const half_t* w16 = (const half_t*)w;
    int64_t ldw = w_stride;
    if (int4) {  // dequantize once into the workspace
      half_t* deq = (half_t*)(ws + l.rows);
      const int64_t items = N * (K / 8);
      const int64_t blocks = std::min<int64_t>((items + 255) / 256, 65536);
      hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                         (const uint8_t*)w, w_stride, (const half_t*)scales, s_stride, (int)N,
                         (int)K, kGroup, deq, K);
      w16 = deq;
      ldw = K;
    }
    const int rc = check_launch(fn);
    if (rc != FI_OK) return rc;
    return f16_gemm(p.x, p.x_stride, w16, ldw, (half_t*)out, out_stride, M, N, K, st);
  }
  launch_linear<false>(p, int4, pl, ws + l.rows + l.weight, st);
  return check_launch(fn);
}

}  // namespace

extern "C" size_t fi_int4_matmul_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % fi::gemm::kGroup) return 0;
  return workspace_bytes_for(M, N, K, false);
}

extern "C" int fi_int4_matmul(const void* x, int64_t x_stride, int64_t M, int64_t K,
                              const void* w, int64_t w_stride, const void* scales,
                              int64_t s_stride, int64_t N, int64_t groupsize, void* out,
                              int64_t out_stride, void* workspace, size_t workspace_bytes,
                              void* stream) {
  using namespace fi;
  clear_error();
  int rc = check_linear("fi_int4_matmul", x, x_stride, M, K, w, w_stride, scales, s_stride, N,
                        groupsize, out, out_stride);
  if (rc != FI_OK || M == 0 || N == 0) return rc;
  return run_linear("fi_int4_matmul", x, x_stride, M, K, nullptr, 0.f, w, w_stride, scales,
                    s_stride, N, out, out_stride, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t fi_rmsnorm_int4_matmul_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % fi::gemm::kGroup) return 0;
  return workspace_bytes_for(M, N, K, true);
}

extern "C" int fi_rmsnorm_int4_matmul(const void* x, int64_t x_stride, int64_t M, int64_t K,
                                      const void* norm_weight, float eps, const void* w,
                                      int64_t w_stride, const void* scales, int64_t s_stride,
                                      int64_t N, int64_t groupsize, void* out,
                                      int64_t out_stride, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  using namespace fi;
  clear_error();
  int rc = check_linear("fi_rmsnorm_int4_matmul", x, x_stride, M, K, w, w_stride, scales,
                        s_stride, N, groupsize, out, out_stride);
  if (rc != FI_OK || M == 0 || N == 0) return rc;
  if (!norm_weight || ((uintptr_t)norm_weight & 15)) {
    set_error("fi_rmsnorm_int4_matmul: norm weight missing or not 16-byte aligned");
    return FI_ERR_INVALID;
  }
  return run_linear("fi_rmsnorm_int4_matmul", x, x_stride, M, K, norm_weight, eps, w, w_stride,
                    scales, s_stride, N, out, out_stride, workspace, workspace_bytes,
                    (hipStream_t)stream);
}

extern "C" int fi_rmsnorm(const void* x, int64_t x_stride, int64_t M, int64_t hidden,
                          const void* weight, float eps, void* out, int64_t out_stride,
                          void* stream) {
  using namespace fi;
  using namespace fi::gemm;
  clear_error();
  if (M < 0 || hidden < 0 || hidden >= (1ll << 30) || M >= (1ll << 30)) {
    set_error("fi_rmsnorm: invalid sizes M %lld hidden %lld", (long long)M, (long long)hidden);
    return FI_ERR_INVALID;
  }
  if (M == 0 || hidden == 0) return FI_OK;
  if (hidden % 8) {
    set_error("fi_rmsnorm: hidden %lld must be a multiple of 8", (long long)hidden);
    return FI_ERR_UNSUPPORTED;
  }
  if (!x || !weight || !out) {
    set_error("fi_rmsnorm: null pointer");
    return FI_ERR_INVALID;
  }
  if (((uintptr_t)x & 15) || ((uintptr_t)weight & 15) || ((uintptr_t)out & 15) ||
      x_stride % 8 || out_stride % 8 || x_stride < hidden || out_stride < hidden) {
    set_error("fi_rmsnorm: rows must be 16-byte aligned and strides cover the rows");
    return FI_ERR_INVALID;
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, (const half_t*)x, x_stride, (int)M, (int)hidden,
                     (const half_t*)weight, eps, (half_t*)out, out_stride);
  return check_launch("fi_rmsnorm");
}

extern "C" int fi_int4_quantize(const void* w, int64_t w_stride, int64_t N, int64_t K,
                                int64_t groupsize, void* packed, int64_t p_stride,
                                void* scales, int64_t s_stride, void* stream) {
  using namespace fi;
  using namespace fi::gemm;
  clear_error();
  if (groupsize < 8 || groupsize > 512 || (groupsize & (groupsize - 1))) {
    set_error("fi_int4_quantize: groupsize %lld not supported (a power of two from 8 to 512)",
              (long long)groupsize);
    return FI_ERR_UNSUPPORTED;
  }
  if (N < 0 || K < 0 || K % groupsize || N >= (1ll << 30) || K >= (1ll << 30)) {
    set_error("fi_int4_quantize: invalid sizes N %lld K %lld", (long long)N, (long long)K);
    return FI_ERR_INVALID;
  }
  if (N == 0 || K == 0) return FI_OK;
  if (!w || !packed || !scales) {
    set_error("fi_int4_quantize: null pointer");
    return FI_ERR_INVALID;
  }
  if (((uintptr_t)w & 15) || w_stride % 8 || w_stride < K || ((uintptr_t)packed & 3) ||
      p_stride % 4 || p_stride < K / 2 || ((uintptr_t)scales & 1) || s_stride < K / groupsize) {
    set_error("fi_int4_quantize: misaligned rows or short strides");
    return FI_ERR_INVALID;
  }
  const int64_t lanes = N * K / 8;  // gs / 8 per group
  const int64_t blocks = std::min<int64_t>((lanes + 255) / 256, 65536);
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)w, w_stride, (int)N, (int)K, (int)groupsize,
                     (uint8_t*)packed, p_stride,
                     (half_t*)scales, s_stride);
  return check_launch("fi_int4_quantize");
}

extern "C" int fi_int4_dequantize(const void* packed, int64_t p_stride, const void* scales,
                                  int64_t s_stride, int64_t N, int64_t K, int64_t groupsize,
                                  void* w, int64_t w_stride, void* stream) {
  using namespace fi;
  using namespace fi::gemm;
  clear_error();
  if (groupsize < 8 || groupsize > 512 || (groupsize & (groupsize - 1))) {
    set_error("fi_int4_dequantize: groupsize %lld not supported (a power of two from 8 to 512)",
              (long long)groupsize);
    return FI_ERR_UNSUPPORTED;
  }
  if (N < 0 || K < 0 || K % groupsize || N >= (1ll << 30) || K >= (1ll << 30)) {
    set_error("fi_int4_dequantize: invalid sizes N %lld K %lld", (long long)N, (long long)K);
    return FI_ERR_INVALID;
  }
  if (N == 0 || K == 0) return FI_OK;
  if (!w || !packed || !scales) {
    set_error("fi_int4_dequantize: null pointer");
    return FI_ERR_INVALID;
  }
  if (((uintptr_t)w & 15) || w_stride % 8 || w_stride < K || ((uintptr_t)packed & 3) ||
      p_stride % 4 || p_stride < K / 2 || ((uintptr_t)scales & 1) || s_stride < K / groupsize) {
    set_error("fi_int4_dequantize: misaligned rows or short strides");
    return FI_ERR_INVALID;
  }
  const int64_t items = N * (K / 8);
  const int64_t blocks = std::min<int64_t>((items + 255) / 256, 65536);
  hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)packed, p_stride,
                     (const half_t*)scales, s_stride, (int)N, (int)K, (int)groupsize,
                     (half_t*)w, w_stride);
  return check_launch("fi_int4_dequantize");
}
