// Device-resident block manager for the paged KV pool: per-sequence lengths, block
// allocation from a FIFO queue of free blocks, release of finished sequences.
//
// The reference allocates on the host, one block at a time (kv_cache.py:50-63, called by
// the loops of model.py:172-174 and :196-198) and keeps one shared token count
// (model.py:169-170, :193-194).  Here the whole batch is served by one launch on the
// caller's stream, so a decode step needs no host round trip and rows may have different
// lengths.  Allocation order is the reference's: rows in order, each row's new blocks taken
// from the front of the free queue in logical order (free_blocks.pop(0)).
//
// Device state (int32, owned by the caller):
//   block_table [max_batch, bt_stride]  physical block of each logical block, -1 = none
//   num_alloc   [max_batch]             blocks allocated to the row (entries 0..n-1 valid)
//   seq_lens    [max_batch]             tokens stored for the row
//   free_queue  [num_blocks]            ring buffer of free block ids
//   state       [4]                     head (queue index of the next free block), count
//                                       (free blocks), status (first error, sticky until
//                                       reset: FI_KV_OUT_OF_BLOCKS / FI_KV_TABLE_FULL /
//                                       FI_KV_NEGATIVE_COUNT), the row of that error
//
// Every kernel here is one workgroup of 1024 threads; thread t owns a contiguous range of
// rows so that a workgroup-wide exclusive scan gives each row its place in row order.
#include <algorithm>

#include "common.h"

namespace fi {
namespace kvm {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

// Exclusive scan of v over the workgroup in thread order; *total gets the sum.
__device__ int block_exclusive_scan(int v, int* s_wave, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kWaves ? s_wave[lane] : 0;
#pragma unroll
    for (int d = 1; d < kWaves; d <<= 1) {
      const int y = __shfl_up(w, d, 64);
      if (lane >= d) w += y;
    }
    if (lane < kWaves) s_wave[lane] = w;  // inclusive wave prefix
  }
  __syncthreads();
  const int before = (wave > 0 ? s_wave[wave - 1] : 0) + x - v;
  *total = s_wave[kWaves - 1];
  __syncthreads();  // s_wave may be reused by the caller's next scan
  return before;
}

struct AppendParams {
  int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
  int32_t* num_alloc;
  int32_t* seq_lens;
  const int32_t* free_queue;
  int32_t* state;
  int num_blocks;
  int block_size;
  int batch;
  const int32_t* num_new;  // per row, or null: num_new_all for every row
  int num_new_all;
  int32_t* start_out;  // optional: the row's length before the call
  int32_t* lens_out;   // optional: the row's length after the call
};

__global__ __launch_bounds__(kThreads) void append_kernel(AppendParams p) {
  __shared__ int s_wave[kWaves];
  __shared__ int s_fail;       // first row that cannot be served (batch = none)
  __shared__ int s_fail_kind;  // its error code
  __shared__ int s_alloc;      // blocks handed out by this call
  __shared__ int s_head, s_count;
  const int per = (p.batch + kThreads - 1) / kThreads;
  const int r0 = min(p.batch, (int)threadIdx.x * per);
  const int r1 = min(p.batch, r0 + per);
  const int N = p.num_blocks;
  if (threadIdx.x == 0) {  // only thread 0 touches state: it reads here, writes at the end
    s_head = ((p.state[0] % N) + N) % N;
    s_count = min(max(p.state[1], 0), N);
    s_fail = p.batch;
    s_fail_kind = 0;
    s_alloc = 0;
  }

  // blocks row b holds (clamped, so a damaged count cannot index outside its table row)
  auto held = [&](int b) -> int { return min(max(p.num_alloc[b], 0), p.max_blocks_per_seq); };
  // blocks row b still needs; -1 marks a row that can never be served
  auto deficit = [&](int b, int* kind) -> int {
    const int n = p.num_new ? p.num_new[b] : p.num_new_all;
    if (n < 0) {
      *kind = FI_KV_NEGATIVE_COUNT;
      return -1;
    }
    const int64_t len = (int64_t)p.seq_lens[b] + n;
    const int64_t need = (len + p.block_size - 1) / p.block_size;
    if (need > p.max_blocks_per_seq) {
      *kind = FI_KV_TABLE_FULL;
      return -1;
    }
    return (int)max<int64_t>(0, need - held(b));
  };

  int mine = 0;
  for (int b = r0; b < r1; ++b) {
    int kind = 0;
    const int d = deficit(b, &kind);
    mine += d > 0 ? d : 0;
  }
  int total;
  const int base = block_exclusive_scan(mine, s_wave, &total);  // (its barriers publish s_*)
  const int head0 = s_head;
  const int count0 = s_count;

  // first row whose blocks run past the free queue, or that can never be served
  int cum = base;
  for (int b = r0; b < r1; ++b) {
    int kind = 0;
    const int d = deficit(b, &kind);
    if (d < 0) {
      atomicMin(&s_fail, b);
      break;
    }
    cum += d;
    if (cum > count0) {
      atomicMin(&s_fail, b);
      break;
    }
  }
  __syncthreads();
  const int fail = s_fail;
  if (fail < p.batch && (int)threadIdx.x == min(fail / per, kThreads - 1)) {
    int kind = 0;
    s_fail_kind = deficit(fail, &kind) < 0 ? kind : FI_KV_OUT_OF_BLOCKS;
  }

  // hand out blocks to rows before the failing one, in row order
  cum = base;
  int handed = 0;
  for (int b = r0; b < r1; ++b) {
    int kind = 0;
    const int d = deficit(b, &kind);
    const int old_len = p.seq_lens[b];
    int new_len = old_len;
    if (b < fail) {
      const int n = p.num_new ? p.num_new[b] : p.num_new_all;
      const int have = held(b);
      int32_t* row = p.block_table + (int64_t)b * p.bt_stride;
      for (int j = 0; j < d; ++j) row[have + j] = p.free_queue[((int64_t)head0 + cum + j) % N];
      p.num_alloc[b] = have + d;
      new_len = old_len + n;
      p.seq_lens[b] = new_len;
      handed += d;
    }
    cum += d > 0 ? d : 0;
    if (p.start_out) p.start_out[b] = old_len;
    if (p.lens_out) p.lens_out[b] = new_len;
  }
  if (handed) atomicAdd(&s_alloc, handed);
  __syncthreads();
  if (threadIdx.x == 0) {
    p.state[0] = (head0 + s_alloc) % N;
    p.state[1] = count0 - s_alloc;
    if (fail < p.batch && p.state[2] == 0) {
      p.state[2] = s_fail_kind;
      p.state[3] = fail;
    }
  }
}

struct ReleaseParams {
  int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
  int32_t* num_alloc;
  int32_t* seq_lens;
  int32_t* free_queue;
  int32_t* state;
  int num_blocks;
  int batch;
  const int32_t* release;  // per row: nonzero = release the row
};

// A released row's blocks go to the back of the free queue in (row, logical) order; its
// table entries become -1 and its length 0.
__global__ __launch_bounds__(kThreads) void release_kernel(ReleaseParams p) {
  __shared__ int s_wave[kWaves];
  __shared__ int s_head, s_count;
  const int per = (p.batch + kThreads - 1) / kThreads;
  const int r0 = min(p.batch, (int)threadIdx.x * per);
  const int r1 = min(p.batch, r0 + per);
  const int N = p.num_blocks;
  if (threadIdx.x == 0) {
    s_head = ((p.state[0] % N) + N) % N;
    s_count = min(max(p.state[1], 0), N);
  }
  auto owned = [&](int b) -> int {
    return p.release[b] ? min(max(p.num_alloc[b], 0), p.max_blocks_per_seq) : 0;
  };
  int mine = 0;
  for (int b = r0; b < r1; ++b) mine += owned(b);
  int total;
  const int base = block_exclusive_scan(mine, s_wave, &total);
  const int count0 = s_count;
  const int64_t tail = (int64_t)s_head + count0;
  int64_t cum = base;
  for (int b = r0; b < r1; ++b) {
    if (!p.release[b]) continue;
    const int n = owned(b);
    int32_t* row = p.block_table + (int64_t)b * p.bt_stride;
    for (int j = 0; j < n; ++j) {
      p.free_queue[(tail + cum + j) % N] = row[j];
      row[j] = -1;
    }
    cum += n;
    p.num_alloc[b] = 0;
    p.seq_lens[b] = 0;
  }
  if (threadIdx.x == 0) p.state[1] = min(count0 + total, N);
}

struct ResetParams {
  int32_t* block_table;
  int64_t bt_stride;
  int max_batch;
  int32_t* num_alloc;
  int32_t* seq_lens;
  int32_t* free_queue;
  int32_t* state;
  int num_blocks;
};

__global__ __launch_bounds__(256) void reset_kernel(ResetParams p) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t cells = (int64_t)p.max_batch * p.bt_stride;
  for (int64_t i = first; i < cells; i += stride) p.block_table[i] = -1;
  for (int64_t i = first; i < p.num_blocks; i += stride) p.free_queue[i] = (int32_t)i;
  for (int64_t i = first; i < p.max_batch; i += stride) {
    p.num_alloc[i] = 0;
    p.seq_lens[i] = 0;
  }
  if (first == 0) {
    p.state[0] = 0;
    p.state[1] = p.num_blocks;
    p.state[2] = 0;
    p.state[3] = -1;
  }
}

}  // namespace kvm
}  // namespace fi

namespace {

int check_state(const char* fn, const void* table, int64_t bt_stride, int64_t max_blocks,
                const void* num_alloc, const void* seq_lens, const void* free_queue,
                const void* state, int64_t num_blocks, int64_t rows) {
  using namespace fi;
  if (!table || !num_alloc || !seq_lens || !free_queue || !state) {
    set_error("%s: null pointer", fn);
    return FI_ERR_INVALID;
  }
  if (num_blocks <= 0 || num_blocks >= (1ll << 30) || max_blocks <= 0 ||
      max_blocks > bt_stride || rows < 0 || rows > (1 << 24) || bt_stride >= (1ll << 30)) {
    set_error("%s: invalid sizes (num_blocks %lld, max_blocks_per_seq %lld, stride %lld, "
              "rows %lld)", fn, (long long)num_blocks, (long long)max_blocks,
              (long long)bt_stride, (long long)rows);
    return FI_ERR_INVALID;
  }
  return FI_OK;
}

}  // namespace

extern "C" int fi_kv_append(int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                            int32_t* num_alloc, int32_t* seq_lens, const int32_t* free_queue,
                            int32_t* state, int64_t num_blocks, int64_t block_size,
                            int64_t batch, const int32_t* num_new, int64_t num_new_all,
                            int32_t* start_pos_out, int32_t* context_lens_out, void* stream) {
  using namespace fi;
  clear_error();
  int rc = check_state("fi_kv_append", block_table, bt_stride, max_blocks_per_seq, num_alloc,
                       seq_lens, free_queue, state, num_blocks, batch);
  if (rc != FI_OK) return rc;
  if (block_size <= 0 || block_size >= (1 << 20)) {
    set_error("fi_kv_append: invalid block_size %lld", (long long)block_size);
    return FI_ERR_INVALID;
  }
  if (!num_new && (num_new_all < 0 || num_new_all >= (1ll << 30))) {
    set_error("fi_kv_append: invalid token count %lld", (long long)num_new_all);
    return FI_ERR_INVALID;
  }
  if (batch == 0) return FI_OK;
  kvm::AppendParams p;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;
  p.num_alloc = num_alloc;
  p.seq_lens = seq_lens;
  p.free_queue = free_queue;
  p.state = state;
  p.num_blocks = (int)num_blocks;
  p.block_size = (int)block_size;
  p.batch = (int)batch;
  p.num_new = num_new;
  p.num_new_all = (int)num_new_all;
  p.start_out = start_pos_out;
  p.lens_out = context_lens_out;
  hipLaunchKernelGGL(kvm::append_kernel, dim3(1), dim3(kvm::kThreads), 0, (hipStream_t)stream,
                     p);
  return check_launch("fi_kv_append");
}

extern "C" int fi_kv_release(int32_t* block_table, int64_t bt_stride,
                             int64_t max_blocks_per_seq, int32_t* num_alloc, int32_t* seq_lens,
                             int32_t* free_queue, int32_t* state, int64_t num_blocks,
                             int64_t batch, const int32_t* release_rows, void* stream) {
  using namespace fi;
  clear_error();
  int rc = check_state("fi_kv_release", block_table, bt_stride, max_blocks_per_seq, num_alloc,
                       seq_lens, free_queue, state, num_blocks, batch);
  if (rc != FI_OK) return rc;
  if (batch == 0) return FI_OK;
  if (!release_rows) {
    set_error("fi_kv_release: null release mask");
    return FI_ERR_INVALID;
  }
  kvm::ReleaseParams p;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;
  p.num_alloc = num_alloc;
  p.seq_lens = seq_lens;
  p.free_queue = free_queue;
  p.state = state;
  p.num_blocks = (int)num_blocks;
  p.batch = (int)batch;
  p.release = release_rows;
  hipLaunchKernelGGL(kvm::release_kernel, dim3(1), dim3(kvm::kThreads), 0, (hipStream_t)stream,
                     p);
  return check_launch("fi_kv_release");
}

extern "C" int fi_kv_reset(int32_t* block_table, int64_t bt_stride, int64_t max_blocks_per_seq,
                           int64_t max_batch, int32_t* num_alloc, int32_t* seq_lens,
                           int32_t* free_queue, int32_t* state, int64_t num_blocks,
                           void* stream) {
  using namespace fi;
  clear_error();
  int rc = check_state("fi_kv_reset", block_table, bt_stride, max_blocks_per_seq, num_alloc,
                       seq_lens, free_queue, state, num_blocks, max_batch);
  if (rc != FI_OK) return rc;
  kvm::ResetParams p;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_batch = (int)max_batch;
  p.num_alloc = num_alloc;
  p.seq_lens = seq_lens;
  p.free_queue = free_queue;
  p.state = state;
  p.num_blocks = (int)num_blocks;
  const int64_t cells = std::max<int64_t>(max_batch * bt_stride, num_blocks);
  const int64_t blocks = std::min<int64_t>((cells + 255) / 256, 1024);
  hipLaunchKernelGGL(kvm::reset_kernel, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256),
                     0, (hipStream_t)stream, p);
  return check_launch("fi_kv_reset");
}
