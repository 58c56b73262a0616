// Paged KV-pool scatter: the byte copies of model.py:162-201 and kv_cache.py:69-103
// as one launch.  Each work item moves one 16-byte chunk (8 fp16) of a K row and the
// same chunk of the matching V row.
#include "common.h"

namespace fi {

struct KvStoreParams {
  const half_t* k;
  const half_t* v;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  half_t* k_cache;
  half_t* v_cache;
  int64_t num_pool_blocks;
  int64_t block_size;
  int64_t num_kv_heads;
  const int32_t* block_table;
  int64_t bt_stride;
  int64_t max_blocks_per_seq;
  int64_t batch;
  int64_t num_tokens;
  int64_t start_pos;
  const int32_t* start_pos_per_seq;
  int64_t head_dim;      // a multiple of 8
  int64_t total_chunks;  // batch * num_tokens * num_kv_heads * (head_dim / 8)
};

__global__ __launch_bounds__(256) void kv_store_kernel(KvStoreParams p) {
  const int64_t chunks = p.head_dim / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < p.total_chunks;
       idx += stride) {
    const int64_t chunk = idx % chunks;
    int64_t rest = idx / chunks;
    const int64_t h = rest % p.num_kv_heads;
    rest /= p.num_kv_heads;
    const int64_t t = rest % p.num_tokens;
    const int64_t b = rest / p.num_tokens;

    const int64_t start = p.start_pos_per_seq ? (int64_t)p.start_pos_per_seq[b] : p.start_pos;
    const int64_t pos = start + t;
    if (pos < 0) continue;
    const int64_t lb = pos / p.block_size;
    if (lb >= p.max_blocks_per_seq) continue;
    const int64_t phys = p.block_table[b * p.bt_stride + lb];
    if (phys < 0 || phys >= p.num_pool_blocks) continue;

    const int64_t dst =
        ((phys * p.block_size + pos % p.block_size) * p.num_kv_heads + h) * p.head_dim + chunk * 8;
    const u32x4 kv = *(const u32x4*)(p.k + b * p.k_sb + t * p.k_st + h * p.k_sh + chunk * 8);
    const u32x4 vv = *(const u32x4*)(p.v + b * p.v_sb + t * p.v_st + h * p.v_sh + chunk * 8);
    *(u32x4*)(p.k_cache + dst) = kv;
    *(u32x4*)(p.v_cache + dst) = vv;
  }
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace fi

extern "C" int fi_kv_store(const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                           const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                           void* k_cache, void* v_cache, int64_t num_pool_blocks,
                           int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                           const int32_t* block_table, int64_t bt_stride,
                           int64_t max_blocks_per_seq, int64_t batch, int64_t num_tokens,
                           int64_t start_pos, const int32_t* start_pos_per_seq,
                           void* stream) {
  using namespace fi;
  clear_error();
  if (head_dim < 8 || head_dim % 8 != 0) {
    set_error("fi_kv_store: head_dim %lld not supported (a positive multiple of 8)",
              (long long)head_dim);
    return FI_ERR_UNSUPPORTED;
  }
  if (batch < 0 || num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 ||
      num_pool_blocks < 0 || max_blocks_per_seq < 0) {
    set_error("fi_kv_store: negative or zero size");
    return FI_ERR_INVALID;
  }
  if (batch == 0 || num_tokens == 0) return FI_OK;
  if (!k || !v || !k_cache || !v_cache || !block_table) {
    set_error("fi_kv_store: null pointer");
    return FI_ERR_INVALID;
  }
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) ||
      (k_sb | k_st | k_sh | v_sb | v_st | v_sh) % 8 != 0) {
    set_error("fi_kv_store: k/v rows must be 16-byte aligned (strides multiple of 8)");
    return FI_ERR_INVALID;
  }
  KvStoreParams p;
  p.k = (const half_t*)k;
  p.v = (const half_t*)v;
  p.k_sb = k_sb; p.k_st = k_st; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_st = v_st; p.v_sh = v_sh;
  p.k_cache = (half_t*)k_cache;
  p.v_cache = (half_t*)v_cache;
  p.num_pool_blocks = num_pool_blocks;
  p.block_size = block_size;
  p.num_kv_heads = num_kv_heads;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = max_blocks_per_seq;
  p.batch = batch;
  p.num_tokens = num_tokens;
  p.start_pos = start_pos;
  p.start_pos_per_seq = start_pos_per_seq;
  p.head_dim = head_dim;
  p.total_chunks = batch * num_tokens * num_kv_heads * (head_dim / 8);
  int64_t blocks = (p.total_chunks + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(kv_store_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, p);
  return check_launch("fi_kv_store");
}
