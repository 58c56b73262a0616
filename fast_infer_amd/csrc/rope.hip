// Rotary position embedding fused with the paged KV write, for gfx950.
//
// Replaces apply_rope (kernels/rope.py:26-44) at the call site model.py:101 and, when a
// pool is given, the K/V stores that follow it (model.py:117 -> :162-183 for prefill,
// model.py:120 -> :185-201 for decode): one pass reads q, k and v (strided views of the
// QKV projection output are fine), writes rotated q, optionally rotated k, and copies
// rotated k and v straight into their pool slots.
//
// Arithmetic is the reference's fp16 tensor arithmetic, op by op (rope.py:37-42):
//   out = fp16( fp16(x * cos) + fp16(rotate_half(x) * sin) ),
// each product and the sum formed in fp32 and rounded to fp16 (round-to-nearest-even),
// rotate_half(x)[i] = -x[i + D/2] for i < D/2 and x[i - D/2] for i >= D/2 (D = head_dim,
// a multiple of 16), with cos/sin the reference's fp16 table rows at the token's position.
// Results are therefore bit-exact.
//
// Work item: one head row of one token is D/16 lanes; lane c handles elements 8c..8c+7 and
// their rotation partners 8c+D/2..8c+D/2+7 (16-byte loads and stores).
#include "common.h"

namespace fi {
namespace rope {

struct Params {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  const half_t* cos_t;  // [table_rows, head_dim]
  const half_t* sin_t;
  int table_rows;
  half_t* q_out;
  int64_t qo_sb, qo_st, qo_sh;
  half_t* k_out;  // optional
  int64_t ko_sb, ko_st, ko_sh;
  half_t* k_cache;  // optional pool [N, bs, Hkv, 128]
  half_t* v_cache;
  int64_t num_pool_blocks;
  int block_size;
  const int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
  int num_tokens;
  int num_q_heads;
  int num_kv_heads;
  int start_pos;
  const int32_t* start_pos_per_seq;
  int heads;      // head rows per token in the grid: q heads, then k heads, then v heads
  int head_dim;   // D, a multiple of 16: a row's two halves are D / 16 chunks of 8 each
  int half;       // D / 2, the rotate-half partner distance
  int cpr;        // D / 16 work items per row
  int64_t items;  // batch * num_tokens * heads * cpr
};

__device__ __forceinline__ half_t rot1(half_t x, half_t c, half_t y, half_t s) {
  // fp16(fp16(x*c) + fp16(y*s)); the fp32 products of fp16 values are exact.  No
  // contraction: a fused multiply-add would round once where the reference rounds twice.
#pragma clang fp contract(off)
  const half_t a = (half_t)((float)x * (float)c);
  const half_t b = (half_t)((float)y * (float)s);
  return (half_t)((float)a + (float)b);
}

// Index is uint32_t whenever the work items fit (32-bit division by the runtime head and
// token counts is a short sequence; 64-bit division is a long software routine).
template <typename Index>
__global__ __launch_bounds__(256) void rope_store_kernel(Params p) {
  const Index heads = (Index)p.heads;
  const Index items = (Index)p.items;
  for (Index it = (Index)blockIdx.x * blockDim.x + threadIdx.x; it < items;
       it += (Index)gridDim.x * blockDim.x) {
    const Index cpr = (Index)p.cpr;
    const Index row = it / cpr;  // (b, t, head)
    const int c = (int)(it - row * cpr);
    const int hh = (int)(row % heads);
    const Index bt = row / heads;
    const int t = (int)(bt % (Index)p.num_tokens);
    const int b = (int)(bt / (Index)p.num_tokens);
    const int pos = (p.start_pos_per_seq ? p.start_pos_per_seq[b] : p.start_pos) + t;
    if (pos < 0 || pos >= p.table_rows) continue;  // no table row: the token is skipped

    // pool slot of this token (k and v rows); -1 when there is no pool or no valid block
    int64_t dst = -1;
    if (p.k_cache && hh >= p.num_q_heads) {
      const int lb = pos / p.block_size;
      if (lb < p.max_blocks_per_seq) {
        const int64_t phys = p.block_table[(int64_t)b * p.bt_stride + lb];
        if (phys >= 0 && phys < p.num_pool_blocks) {
          const int hk = hh - p.num_q_heads - (hh >= p.num_q_heads + p.num_kv_heads ? p.num_kv_heads : 0);
          dst = ((phys * p.block_size + pos % p.block_size) * p.num_kv_heads + hk) * p.head_dim;
        }
      }
    }

    if (hh >= p.num_q_heads + p.num_kv_heads) {  // v: plain copy into the pool
      if (dst < 0) continue;
      const int hk = hh - p.num_q_heads - p.num_kv_heads;
      const half_t* src = p.v + (int64_t)b * p.v_sb + (int64_t)t * p.v_st + (int64_t)hk * p.v_sh;
      *(u32x4*)(p.v_cache + dst + 8 * c) = *(const u32x4*)(src + 8 * c);
      *(u32x4*)(p.v_cache + dst + p.half + 8 * c) = *(const u32x4*)(src + p.half + 8 * c);
      continue;
    }

    const bool is_q = hh < p.num_q_heads;
    const half_t* src = is_q ? p.q + (int64_t)b * p.q_sb + (int64_t)t * p.q_st + (int64_t)hh * p.q_sh
                             : p.k + (int64_t)b * p.k_sb + (int64_t)t * p.k_st +
                                   (int64_t)(hh - p.num_q_heads) * p.k_sh;
    const half8 lo = as_half8(*(const u32x4*)(src + 8 * c));        // x[8c .. 8c+7]
    const half8 hi = as_half8(*(const u32x4*)(src + p.half + 8 * c));  // x[D/2+8c .. +7]
    const half_t* cr = p.cos_t + (int64_t)pos * p.head_dim;
    const half_t* sr = p.sin_t + (int64_t)pos * p.head_dim;
    const half8 clo = as_half8(*(const u32x4*)(cr + 8 * c));
    const half8 chi = as_half8(*(const u32x4*)(cr + p.half + 8 * c));
    const half8 slo = as_half8(*(const u32x4*)(sr + 8 * c));
    const half8 shi = as_half8(*(const u32x4*)(sr + p.half + 8 * c));
    half8 olo, ohi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      olo[e] = rot1(lo[e], clo[e], -hi[e], slo[e]);  // i < D/2: partner -x[i+D/2]
      ohi[e] = rot1(hi[e], chi[e], lo[e], shi[e]);   // i >= D/2: partner x[i-D/2]
    }
    if (is_q) {
      half_t* o = p.q_out + (int64_t)b * p.qo_sb + (int64_t)t * p.qo_st + (int64_t)hh * p.qo_sh;
      *(u32x4*)(o + 8 * c) = as_u32x4(olo);
      *(u32x4*)(o + p.half + 8 * c) = as_u32x4(ohi);
    } else {
      if (p.k_out) {
        half_t* o = p.k_out + (int64_t)b * p.ko_sb + (int64_t)t * p.ko_st +
                    (int64_t)(hh - p.num_q_heads) * p.ko_sh;
        *(u32x4*)(o + 8 * c) = as_u32x4(olo);
        *(u32x4*)(o + p.half + 8 * c) = as_u32x4(ohi);
      }
      if (dst >= 0) {
        *(u32x4*)(p.k_cache + dst + 8 * c) = as_u32x4(olo);
        *(u32x4*)(p.k_cache + dst + p.half + 8 * c) = as_u32x4(ohi);
      }
    }
  }
}

}  // namespace rope
}  // namespace fi

extern "C" int fi_rope_store_kv(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                                const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                                const void* cos_table, const void* sin_table,
                                int64_t table_rows, void* q_out, int64_t qo_sb, int64_t qo_st,
                                int64_t qo_sh, void* k_out, int64_t ko_sb, int64_t ko_st,
                                int64_t ko_sh, void* k_cache, void* v_cache,
                                int64_t num_pool_blocks, int64_t block_size,
                                const int32_t* block_table, int64_t bt_stride,
                                int64_t max_blocks_per_seq, int64_t batch, int64_t num_tokens,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t start_pos, const int32_t* start_pos_per_seq,
                                void* stream) {
  using namespace fi;
  using namespace fi::rope;
  clear_error();
  if (head_dim < 16 || head_dim % 16 != 0 || head_dim > (1 << 16)) {
    set_error("fi_rope_store_kv: head_dim %lld not supported (a positive multiple of 16)",
              (long long)head_dim);
    return FI_ERR_UNSUPPORTED;
  }
  if (batch < 0 || num_tokens < 0 || num_q_heads < 0 || num_kv_heads < 0 || table_rows < 0) {
    set_error("fi_rope_store_kv: negative size");
    return FI_ERR_INVALID;
  }
  if (batch == 0 || num_tokens == 0 || num_q_heads + num_kv_heads == 0) return FI_OK;
  if (batch * num_tokens > (1ll << 31) || table_rows > (1ll << 30) ||
      start_pos > (1ll << 30) || start_pos < -(1ll << 30) || num_tokens > (1ll << 30)) {
    set_error("fi_rope_store_kv: sizes too large");
    return FI_ERR_UNSUPPORTED;
  }
  const bool pool = k_cache != nullptr;
  if (!cos_table || !sin_table || (num_q_heads > 0 && (!q || !q_out)) ||
      (num_kv_heads > 0 && !k) || (pool && (!v || !v_cache || !block_table))) {
    set_error("fi_rope_store_kv: null pointer");
    return FI_ERR_INVALID;
  }
  if (pool && (block_size <= 0 || num_pool_blocks < 0 || max_blocks_per_seq < 0)) {
    set_error("fi_rope_store_kv: invalid pool sizes");
    return FI_ERR_INVALID;
  }
  const uintptr_t ptrs = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)cos_table |
                         (uintptr_t)sin_table | (uintptr_t)q_out | (uintptr_t)k_out |
                         (uintptr_t)k_cache | (uintptr_t)v_cache;
  const int64_t strides = q_sb | q_st | q_sh | k_sb | k_st | k_sh | v_sb | v_st | v_sh | qo_sb |
                          qo_st | qo_sh | ko_sb | ko_st | ko_sh;
  if ((ptrs & 15u) || strides % 8 != 0) {
    set_error("fi_rope_store_kv: rows must be 16-byte aligned (strides multiple of 8)");
    return FI_ERR_INVALID;
  }

  Params p;
  p.q = (const half_t*)q;
  p.k = (const half_t*)k;
  p.v = (const half_t*)v;
  p.q_sb = q_sb; p.q_st = q_st; p.q_sh = q_sh;
  p.k_sb = k_sb; p.k_st = k_st; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_st = v_st; p.v_sh = v_sh;
  p.cos_t = (const half_t*)cos_table;
  p.sin_t = (const half_t*)sin_table;
  p.table_rows = (int)table_rows;
  p.q_out = (half_t*)q_out;
  p.qo_sb = qo_sb; p.qo_st = qo_st; p.qo_sh = qo_sh;
  p.k_out = (half_t*)k_out;
  p.ko_sb = ko_sb; p.ko_st = ko_st; p.ko_sh = ko_sh;
  p.k_cache = (half_t*)k_cache;
  p.v_cache = (half_t*)v_cache;
  p.num_pool_blocks = num_pool_blocks;
  p.block_size = (int)block_size;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;
  p.num_tokens = (int)num_tokens;
  p.num_q_heads = (int)num_q_heads;
  p.num_kv_heads = (int)num_kv_heads;
  p.start_pos = (int)start_pos;
  p.start_pos_per_seq = start_pos_per_seq;
  // k rows only when rotated k goes somewhere, v rows only with a pool
  const int64_t nk = (k_out || pool) ? num_kv_heads : 0;
  const int64_t nv = pool ? num_kv_heads : 0;
  p.heads = (int)(num_q_heads + nk + nv);
  p.head_dim = (int)head_dim;
  p.half = (int)(head_dim / 2);
  p.cpr = (int)(head_dim / 16);
  p.items = batch * num_tokens * p.heads * p.cpr;
  if (p.items == 0) return FI_OK;
  const int64_t blocks = (p.items + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
  if (p.items < (1ll << 31))
    hipLaunchKernelGGL(rope_store_kernel<uint32_t>, dim3(grid), dim3(256), 0,
                       (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(rope_store_kernel<int64_t>, dim3(grid), dim3(256), 0,
                       (hipStream_t)stream, p);
  return check_launch("fi_rope_store_kv");
}
