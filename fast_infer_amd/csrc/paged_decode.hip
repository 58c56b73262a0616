// Paged-attention decode for gfx950: one query token per sequence attends to its
// context stored in a paged KV pool [num_blocks, block_size, num_kv_heads, 128].
//
// Replaces _paged_attention_kernel (kernels/attention.py:116-188).  Same math —
// scores q.k * sm_scale over the first ctx tokens, softmax, weighted sum of V — but
// organised for an HBM-bound MI355X kernel:
//   * one workgroup serves all query heads of a GQA group, so each K/V row is read
//     from HBM once (the reference reads it once per query head, :137-139);
//   * the context is split into partitions (flash-decoding); each workgroup turns one
//     partition into an unnormalised partial (m, l, o) and a second small kernel
//     merges the partials; a single-partition call writes the output directly;
//   * each wave streams 16-token K and V tiles global->LDS with the buffer unit (no
//     register staging, whole 256-byte rows per request), double-buffered in a
//     wave-private LDS region, so many loads stay in flight at low register cost;
//   * QK^T and PV run on MFMA with the GQA heads as the 16-wide N dimension:
//     S^T = K * Q^T (v_mfma_f32_16x16x32_f16, K fragments read from LDS) and
//     O^T = V^T * P^T (v_mfma_f32_16x16x16_f16, V^T fragments from the LDS transpose
//     read ds_read_b64_tr_b16, P^T straight from the S^T accumulator lanes).
//   * Online softmax is fp32 in log2 units (exp2 with sm_scale * log2(e) folded in).
//   * Tiles are laid over token positions, never over blocks, so the block size only
//     decides where a tile row's bytes come from: with a multiple of 16 a tile sits in one
//     block (one descriptor per tile); any other size gives each row its own block, through
//     per-lane offsets into a descriptor over the whole pool (pools under 4 GiB) or through
//     one descriptor per row.
#include <mutex>

#include "common.h"

namespace fi {

namespace decode {

constexpr int kWaves = 4;                          // waves per workgroup
constexpr int kTileTokens = 16;                    // tokens per wave tile (one MFMA tile)
constexpr int kWgTokens = kWaves * kTileTokens;    // tokens per workgroup round
constexpr int kTileBytes = kTileTokens * kHeadDim * 2;  // one K (or V) tile in LDS: 4 KiB
constexpr int kBufBytes = 2 * kTileBytes;          // K + V tile of one wave
constexpr int kMaxHeadsPerWg = 16;                 // MFMA N dimension
constexpr int kMaxSplitTokens = 4096;                       // cap on the partition size
constexpr int kMaxSplitEntries = kMaxSplitTokens / 16 + 1;  // table entries of a partition
// Table entries a partition may stage when block_size is not a multiple of 16 (up to
// tokens_per_split / block_size + 2 of them): 14 KiB, which keeps two workgroups per CU.
constexpr int kAnyBlockEntries = 3584;
// How a tile's K/V rows are addressed (the partition kernel's template argument):
constexpr int kTileBlock = 0;  // block_size % 16 == 0: a 16-token tile lies in one block
constexpr int kLanePool = 1;   // any block_size, pool under kFarOffset bytes: per-lane offsets
constexpr int kRowBlock = 2;   // any block_size, any pool: one descriptor per tile row
// Buffer offset past the end of any pool the kLanePool path serves: loads return 0.
constexpr uint32_t kFarOffset = 0xFFFFFF00u;
constexpr int kMaxSplits = 1024;                            // partitions per row
constexpr int kOutOfRange = 0x40000000;  // buffer offset beyond any block: loads return 0
// The K/V loads use the non-temporal cache policy (lds_copy16_nt): each byte is read once per
// call, and not allocating it in L2 streams measurably faster than default-policy loads.

// the wave merge reuses one tile buffer array: [wave][head][128] fp32
static_assert(kWaves * kMaxHeadsPerWg * kHeadDim * 4 <= kWaves * kBufBytes,
              "merge area must fit in one buffer array");

struct Params {
  const half_t* q;
  int64_t q_sb, q_sh;
  const half_t* k_cache;
  const half_t* v_cache;
  int64_t num_pool_blocks;
  int block_size;
  int num_kv_heads;
  const int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
  const int32_t* context_lens;
  int num_tokens;
  half_t* o;
  int64_t o_sb, o_sh;
  int num_q_heads;
  int group;         // query heads per kv head
  int heads_per_wg;  // query heads served by one workgroup (divides group, <= 16)
  float scale_log2;  // sm_scale * log2(e)
  int tokens_per_split;
  int max_splits;
  float* part_o;   // [batch][num_q_heads][max_splits][128]
  float* part_ml;  // [batch][num_q_heads][max_splits][2]
  int direct;      // 1 -> a single partition, write o
  int head_dim;    // D <= kHeadDim, a multiple of 8: LDS rows and fragments stay kHeadDim
  int d_chunks;    // wide, and the 16-byte chunks past D are loaded as zeros
};

__device__ __forceinline__ int row_context(const Params& p, int b) {
  int ctx = p.context_lens ? p.context_lens[b] : p.num_tokens;
  ctx = ctx < p.num_tokens ? ctx : p.num_tokens;
  const int cap = p.max_blocks_per_seq * p.block_size;
  ctx = ctx < cap ? ctx : cap;
  return ctx < 0 ? 0 : ctx;
}

// Buffer descriptor covering one kv head's rows of one pool block; a block outside the
// pool gets zero records, so every load through it returns 0 without touching memory.
__device__ __forceinline__ rsrc_t block_rsrc(const half_t* pool, int64_t phys,
                                            int64_t block_bytes, int kv_off) {
  const bool ok = phys >= 0;
  const char* base = (const char*)pool + (ok ? phys * block_bytes : 0) + kv_off;
  return raw_rsrc(base, ok ? (int)(block_bytes - kv_off) : 0);
}

// LDS tile layout: 16 rows (tokens) of 256 bytes.  K row r keeps 16-byte chunk c at slot
// c ^ r, so the 16 lanes of a K fragment read (16 rows, one chunk) hit 16 distinct bank
// slots.  V row r keeps chunk c at slot c ^ 2(r % 8), so the 32-byte column pairs a
// transpose read takes from 8 consecutive rows land in 8 distinct pair slots.
__device__ __forceinline__ int kslot(int r, int c) { return r * 256 + ((c ^ r) << 4); }
__device__ __forceinline__ int vslot(int r, int c) { return r * 256 + ((c ^ ((r & 7) << 1)) << 4); }

// Issue the direct-to-LDS loads of one 16-token tile (tokens tile..tile+15 of the row)
// into buf (K at +0, V at +kTileBytes).  One instruction moves 4 rows; lane l fills slot
// l % 16 of row 4q + l / 16 and so fetches the chunk stored there.  Tokens at or past
// split_end, and tiles whose table entry is outside the pool, read zeros.
__device__ __forceinline__ bool issue_tile(const Params& p, const int* s_tab, int tab0,
                                           int tile, int split_end, int kv_off,
                                           int64_t block_bytes, int row_bytes, char* buf,
                                           int lane) {
  int64_t phys = -1;
  if (tile < split_end) phys = __builtin_amdgcn_readfirstlane(s_tab[tile / p.block_size - tab0]);
  const rsrc_t kr = block_rsrc(p.k_cache, phys, block_bytes, kv_off);
  const rsrc_t vr = block_rsrc(p.v_cache, phys, block_bytes, kv_off);
  const uint32_t lds = lds_addr(buf);
  const int slot0 = tile % p.block_size;  // 16-token tiles never straddle a block
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * q + (lane >> 4);
    const bool in = tile + row < split_end;
    const int kc = (lane & 15) ^ row;
    const int vc = (lane & 15) ^ ((row & 7) << 1);
    const int koff = in && kc < p.d_chunks ? (slot0 + row) * row_bytes + (kc << 4) : kOutOfRange;
    const int voff = in && vc < p.d_chunks ? (slot0 + row) * row_bytes + (vc << 4) : kOutOfRange;
    lds_copy16_nt(kr, lds + q * 1024, koff, 0);
    lds_copy16_nt(vr, lds + kTileBytes + q * 1024, voff, 0);
  }
  return phys >= 0;
}

// issue_tile for a block_size that is not a multiple of 16 and a pool of fewer than
// kFarOffset bytes: the 16 rows of a tile may lie in up to 16 pool blocks, so the
// descriptors kr / vr span the whole pool (from this kv head's first column) and each lane
// adds its row's block and slot to its own offset; the copies stay four 4-row copies per
// tile.  Returns the tile's row mask: bit r is set when token tile + r is before split_end
// and its table entry is inside the pool.
__device__ __forceinline__ uint32_t issue_tile_lanes(const Params& p, const int* s_tab, int tab0,
                                                     int tile, int split_end, rsrc_t kr,
                                                     rsrc_t vr, uint32_t block_bytes,
                                                     int row_bytes, char* buf, int lane) {
  const uint32_t lds = lds_addr(buf);
  const int grp = lane >> 4;
  uint32_t rows = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * q + grp;
    const int tok = tile + row;
    const bool in = tok < split_end;
    const int blk = tok / p.block_size;
    const int slot = tok - blk * p.block_size;
    // entries tab0 .. (split_end - 1) / block_size are staged; rows past split_end read none
    const int phys = in ? s_tab[blk - tab0] : -1;
    const bool valid = phys >= 0;
    // lanes 0, 16, 32, 48 hold rows 4q .. 4q + 3
    const uint64_t m = __builtin_amdgcn_ballot_w64(valid);
    rows |= (uint32_t)((m & 1u) | ((m >> 15) & 2u) | ((m >> 30) & 4u) | ((m >> 45) & 8u)) << (4 * q);
    // phys < num_pool_blocks, so the row's offset is below the pool size (< 2^32)
    const uint32_t at = (uint32_t)phys * block_bytes + (uint32_t)(slot * row_bytes);
    const int kc = (lane & 15) ^ row;
    const int vc = (lane & 15) ^ ((row & 7) << 1);
    const uint32_t koff = valid && kc < p.d_chunks ? at + (uint32_t)(kc << 4) : kFarOffset;
    const uint32_t voff = valid && vc < p.d_chunks ? at + (uint32_t)(vc << 4) : kFarOffset;
    lds_copy16_nt(kr, lds + q * 1024, (int)koff, 0);
    lds_copy16_nt(vr, lds + kTileBytes + q * 1024, (int)voff, 0);
  }
  return rows;
}

// issue_tile for a block_size that is not a multiple of 16 and a pool of any size: every
// row gets its own descriptor (as in issue_tile), and each of the four 4-row copies becomes
// four copies with one 16-lane row group active (lane l still fills slot l % 16 of row
// 4q + l / 16).  Returns the row mask as issue_tile_lanes does.
__device__ __forceinline__ uint32_t issue_tile_rows(const Params& p, const int* s_tab, int tab0,
                                                    int tile, int split_end, int kv_off,
                                                    int64_t block_bytes, int row_bytes,
                                                    char* buf, int lane) {
  const uint32_t lds = lds_addr(buf);
  const int grp = lane >> 4;
  uint32_t rows = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * q + grp;
    const int tok = tile + row;
    const bool in = tok < split_end;
    const int blk = tok / p.block_size;
    const int slot = tok - blk * p.block_size;
    // entries tab0 .. (split_end - 1) / block_size are staged; rows past split_end read none
    const int phys_lane = in ? s_tab[blk - tab0] : -1;
    const int kc = (lane & 15) ^ row;
    const int vc = (lane & 15) ^ ((row & 7) << 1);
    const int koff = kc < p.d_chunks ? slot * row_bytes + (kc << 4) : kOutOfRange;
    const int voff = vc < p.d_chunks ? slot * row_bytes + (vc << 4) : kOutOfRange;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int phys = __builtin_amdgcn_readlane(phys_lane, 16 * j);  // row 4q + j
      rows |= (phys >= 0 ? 1u : 0u) << (4 * q + j);
      const rsrc_t kr = block_rsrc(p.k_cache, phys, block_bytes, kv_off);
      const rsrc_t vr = block_rsrc(p.v_cache, phys, block_bytes, kv_off);
      if (grp == j) {
        lds_copy16_nt(kr, lds + q * 1024, koff, 0);
        lds_copy16_nt(vr, lds + kTileBytes + q * 1024, voff, 0);
      }
    }
  }
  return rows;
}

// Load instructions one tile issue leaves outstanding per wave.
template <int kAddr>
constexpr int kIssuePerTile = kAddr == kRowBlock ? 32 : 8;

// Online-softmax update with one resident 16-token tile at `tile`.
// `rows`: the tile's row mask for kLanePool / kRowBlock; for kTileBlock, nonzero when the
// tile's block is inside the pool.
template <int kAddr>
__device__ __forceinline__ void consume_tile(const Params& p, const char* buf, uint32_t rows, int tile,
                                             int split_end, const half8 (&qf)[4], int col,
                                             int g, float& m_run, float& l_run,
                                             floatx4 (&acc)[8]) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  // S^T = K * Q^T: lane holds tokens tile + 4g + r of head column col.
  floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s = mfma16x16x32(as_half8(*(const u32x4*)(buf + kslot(col, 4 * i + g))), qf[i], s);

  float x[4];
  float tmax = kNegBig;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int tok = tile + 4 * g + r;
    const bool valid = kAddr == kTileBlock ? rows != 0 && tok < split_end
                                           : ((rows >> (4 * g + r)) & 1u) != 0;
    x[r] = valid ? s[r] * p.scale_log2 : -__builtin_inff();
    tmax = fmaxf(tmax, x[r]);
  }
  tmax = row4_max(tmax);
  const float m_new = fmaxf(m_run, tmax);
  const float alpha = fast_exp2(m_run - m_new);
  m_run = m_new;
  // P is rounded to fp16 for the PV MFMA; l sums those same rounded values, so the
  // numerator and the denominator use identical weights.
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  half4 pf;
#pragma unroll
  for (int r = 0; r < 4; ++r) pf[r] = (half_t)fast_exp2(x[r] - m_new);
  const h2 one2 = {(half_t)1.f, (half_t)1.f};
  float psum = __builtin_amdgcn_fdot2(h2{pf[0], pf[1]}, one2, 0.f, false);
  psum = __builtin_amdgcn_fdot2(h2{pf[2], pf[3]}, one2, psum, false);
  l_run = l_run * alpha + psum;

  // O^T += V^T * P^T (16 keys): lane (col, g) of the transpose read gets keys 4g..4g+3
  // of head_dim column 16dt + col (row 4g + col/4, columns 16dt + 4(col%4)..+3).
  const int vrow = 4 * g + (col >> 2);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const int c = 2 * dt + ((col & 3) >> 1);
    const char* ptr = buf + kTileBytes + vslot(vrow, c) + ((col & 1) << 3);
    const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s4 __attribute__((address_space(3)))*)ptr);
    acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4, v), pf,
                                                    acc[dt] * alpha, 0, 0, 0);
  }
}

template <int kAddr>
__global__ __launch_bounds__(256, 2) void partition_kernel(Params p) {
  // two tile buffers per wave (distinct objects, so the compiler tracks the copies into
  // one separately from reads of the other)
  __shared__ __attribute__((aligned(16))) char buf0[kWaves * kBufBytes];
  __shared__ __attribute__((aligned(16))) char buf1[kWaves * kBufBytes];
  __shared__ float s_ml[kWaves * kMaxHeadsPerWg * 2];
  __shared__ int s_tab[kAddr == kTileBlock ? kMaxSplitEntries : kAnyBlockEntries];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index (uniform)
  const int col = lane & 15;  // MFMA column: query head within the workgroup
  const int g = lane >> 4;    // 16-lane row of the wave
  const int hgroups_per_kv = p.group / p.heads_per_wg;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  // Head group of this workgroup, rotated by partition and row.  The hardware deals
  // consecutive workgroups to the XCDs in turn, so with gridDim.x = 8 XCD k would read head
  // group k of every (row, partition).  The head slices of a pool row do not all stream
  // equally fast, and the XCDs serving the slow ones would finish last; rotated, every XCD
  // serves every head group equally often.
  const int hg = (int)((blockIdx.x + blockIdx.y + blockIdx.z) % gridDim.x);
  const int kvh = hg / hgroups_per_kv;
  const int head0 = kvh * p.group + (hg % hgroups_per_kv) * p.heads_per_wg;

  const int ctx = row_context(p, b);
  const int split_start = split * p.tokens_per_split;
  // no tokens here: the merge reads only the row's first ceil(ctx / tokens_per_split)
  // partials, so this partition writes nothing
  if (!p.direct && split_start >= ctx) return;
  const int split_end = min(split_start + p.tokens_per_split, ctx);

  // Block-table entries of this partition, validated once, staged in LDS.
  const int tab0 = split_start / p.block_size;
  if (split_end > split_start) {
    const int n_ent = (split_end - 1) / p.block_size - tab0 + 1;
    for (int i = threadIdx.x; i < n_ent; i += blockDim.x) {
      const int64_t e = p.block_table[(int64_t)b * p.bt_stride + tab0 + i];
      s_tab[i] = (e >= 0 && e < p.num_pool_blocks) ? (int)e : -1;
    }
  }

  __syncthreads();

  const int row_bytes = p.num_kv_heads * p.head_dim * 2;  // one pool slot, all kv heads
  const int64_t block_bytes = (int64_t)p.block_size * row_bytes;
  const int kv_off = kvh * p.head_dim * 2;
  char* wb0 = buf0 + w * kBufBytes;
  char* wb1 = buf1 + w * kBufBytes;

  // Wave w takes tiles w, w + kWaves, ... of the partition, double-buffered: the copy of
  // tile k+1 is in flight while tile k is consumed, and a buffer is refilled (tile k+2)
  // as soon as its tile is consumed.  The first two copies go out before the Q loads.
  const int first = split_start + w * kTileTokens;
  const int n_t = first < split_end ? (split_end - first + kWgTokens - 1) / kWgTokens : 0;
  // kLanePool: descriptors over the whole pools from this kv head's first column (the host
  // checked that the pool is smaller than kFarOffset bytes)
  const uint32_t pool_records =
      p.num_pool_blocks > 0 ? (uint32_t)(p.num_pool_blocks * block_bytes - kv_off) : 0u;
  const rsrc_t pool_k = raw_rsrc((const char*)p.k_cache + kv_off, (int)pool_records);
  const rsrc_t pool_v = raw_rsrc((const char*)p.v_cache + kv_off, (int)pool_records);
  auto issue = [&](int tile, char* wb) -> uint32_t {
    if (kAddr == kLanePool)
      return issue_tile_lanes(p, s_tab, tab0, tile, split_end, pool_k, pool_v,
                              (uint32_t)block_bytes, row_bytes, wb, lane);
    if (kAddr == kRowBlock)
      return issue_tile_rows(p, s_tab, tab0, tile, split_end, kv_off, block_bytes, row_bytes, wb,
                             lane);
    return issue_tile(p, s_tab, tab0, tile, split_end, kv_off, block_bytes, row_bytes, wb, lane)
               ? 1u : 0u;
  };
  uint32_t ok0 = 0, ok1 = 0;
  if (n_t > 0) ok0 = issue(first, wb0);
  if (n_t > 1) ok1 = issue(first + kWgTokens, wb1);

  // Q^T fragments (B operand of S^T = K * Q^T): column `col` is query head head0+col;
  // MFMA i takes head_dim d = 32*i + 8*g + s in reduction slot 8*g + s (the K
  // fragment uses the same map).
  half8 qf[4];
  {
    const bool valid = col < p.heads_per_wg;
    const half_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(head0 + (valid ? col : 0)) * p.q_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (valid && 32 * i + 8 * g < p.head_dim) v = *(const u32x4*)(qrow + 32 * i + 8 * g);
      qf[i] = as_half8(v);
    }
  }
  // The compiler does not see the tile copies (inline asm), so it would guard the first use
  // of qf inside the loop with a wait for every outstanding load, on every iteration.  One
  // explicit wait here (the first two tiles were issued just before) leaves it nothing to
  // guard.
  wait_vmcnt<0>();

  float m_run = kNegBig;
  float l_run = 0.f;
  floatx4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int k = 0; k < n_t; k += 2) {
    const int t0 = first + k * kWgTokens;
    consume_tile<kAddr>(p, wb0, ok0, t0, split_end, qf, col, g, m_run, l_run, acc);
    if (k + 1 >= n_t) break;
    if (k + 2 < n_t) {
      ok0 = issue(t0 + 2 * kWgTokens, wb0);
      wait_vmcnt<kIssuePerTile<kAddr>>();
    } else {
      wait_vmcnt<0>();
    }
    consume_tile<kAddr>(p, wb1, ok1, t0 + kWgTokens, split_end, qf, col, g, m_run, l_run, acc);
    if (k + 2 >= n_t) break;
    if (k + 3 < n_t) {
      ok1 = issue(t0 + 3 * kWgTokens, wb1);
      wait_vmcnt<kIssuePerTile<kAddr>>();
    } else {
      wait_vmcnt<0>();
    }
  }

  l_run = row4_sum(l_run);

  // ---- merge the four waves through LDS (reuses the first buffer array).
  __syncthreads();
  float* cmb_o = (float*)buf0;  // [w][col][128]
  if (col < p.heads_per_wg) {
    float* dst = cmb_o + (w * kMaxHeadsPerWg + col) * kHeadDim + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *(floatx4*)(dst + 16 * dt) = acc[dt];
    if (g == 0) {
      s_ml[(w * kMaxHeadsPerWg + col) * 2 + 0] = m_run;
      s_ml[(w * kMaxHeadsPerWg + col) * 2 + 1] = l_run;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < p.heads_per_wg * kHeadDim; idx += blockDim.x) {
    const int c = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float mw[kWaves];
    float mx = kNegBig;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      mw[ww] = s_ml[(ww * kMaxHeadsPerWg + c) * 2];
      mx = fmaxf(mx, mw[ww]);
    }
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const float sc = fast_exp2(mw[ww] - mx);
      L += sc * s_ml[(ww * kMaxHeadsPerWg + c) * 2 + 1];
      O += sc * cmb_o[(ww * kMaxHeadsPerWg + c) * kHeadDim + d];
    }
    const int h = head0 + c;
    if (p.direct) {
      if (d < p.head_dim)
        p.o[(int64_t)b * p.o_sb + (int64_t)h * p.o_sh + d] = (half_t)(L > 0.f ? O / L : 0.f);
    } else {
      const int64_t slot = ((int64_t)b * p.num_q_heads + h) * p.max_splits + split;
      p.part_o[slot * kHeadDim + d] = O;
      if (d == 0) {
        p.part_ml[slot * 2 + 0] = mx;
        p.part_ml[slot * 2 + 1] = L;
      }
    }
  }
}

// Merge the partition partials of one (row, query head): o = sum_s e^(m_s-M) o_s /
// sum_s e^(m_s-M) l_s, zeros for an empty row.  The row's length gives its partition
// count (the partitions past it wrote nothing); those partials' loads are issued at
// once, and partials with l = 0 (no valid key) are selected away, never multiplied.
__global__ __launch_bounds__(kHeadDim) void merge_kernel(Params p) {
  constexpr int kBatch = 16;  // partials loaded per round (one round for up to 16 partitions)
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t slot0 = ((int64_t)b * p.num_q_heads + h) * p.max_splits;
  const int ctx = row_context(p, b);
  const int nparts = min((ctx + p.tokens_per_split - 1) / p.tokens_per_split, p.max_splits);
  float mx = kNegBig, L = 0.f, O = 0.f;
  for (int s0 = 0; s0 < nparts; s0 += kBatch) {
    float m[kBatch], l[kBatch], o[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int s = s0 + k < nparts ? s0 + k : nparts - 1;
      // read once: non-temporal
      m[k] = __builtin_nontemporal_load(p.part_ml + (slot0 + s) * 2);
      l[k] = __builtin_nontemporal_load(p.part_ml + (slot0 + s) * 2 + 1);
      o[k] = __builtin_nontemporal_load(p.part_o + (slot0 + s) * kHeadDim + d);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const bool use = s0 + k < nparts && l[k] > 0.f;
      const float mk = use ? m[k] : kNegBig;
      const float mn = fmaxf(mx, mk);
      const float a = fast_exp2(mx - mn);
      const float w = use ? fast_exp2(mk - mn) : 0.f;
      L = L * a + w * l[k];
      O = O * a + (use ? w * o[k] : 0.f);
      mx = mn;
    }
  }
  if (d < p.head_dim)
    p.o[(int64_t)b * p.o_sb + (int64_t)h * p.o_sh + d] = (half_t)(L > 0.f ? O / L : 0.f);
}

// Partition size (tokens, a multiple of kWgTokens) for a call: about kTargetWgs
// workgroups in total if every row had the maximum length, 128..384 tokens each (short
// partitions keep every CU streaming at small batch; longer ones amortise the
// workgroup's table and merge work; the merge reads ~0.5 KiB per partition and head).
// A context of at most 512 tokens is one partition with no merge.
static int tokens_per_split(int64_t batch, int64_t wg_per_row, int64_t num_tokens) {
  constexpr int64_t target = 2048;
  int64_t tps;
  if (num_tokens <= 512) {
    tps = num_tokens;
  } else {
    const int64_t per_row = batch * wg_per_row;
    int64_t want = (target + per_row - 1) / per_row;
    if (want < 1) want = 1;
    tps = (num_tokens + want - 1) / want;
    if (tps > 384) tps = 384;
  }
  const int64_t min_tps = (num_tokens + kMaxSplits - 1) / kMaxSplits;
  if (tps < min_tps) tps = min_tps;
  tps = (tps + kWgTokens - 1) / kWgTokens * kWgTokens;
  if (tps < 128) tps = 128;
  if (tps > kMaxSplitTokens) tps = kMaxSplitTokens;
  return (int)tps;
}

static int heads_per_wg(int64_t group) {
  for (int h = kMaxHeadsPerWg; h >= 1; --h)
    if (group % h == 0) return h;
  return 1;
}

}  // namespace decode
}  // namespace fi

extern "C" size_t fi_paged_attention_workspace_size(int64_t batch, int64_t num_q_heads,
                                                    int64_t num_kv_heads,
                                                    int64_t max_num_tokens, int64_t head_dim) {
  using namespace fi::decode;
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_num_tokens <= 0 ||
      !fi::head_dim_ok(head_dim) || num_q_heads % num_kv_heads != 0)
    return 0;
  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t wg_per_row = num_kv_heads * (group / heads_per_wg(group));
  const int64_t tps = tokens_per_split(batch, wg_per_row, max_num_tokens);
  const int64_t splits = (max_num_tokens + tps - 1) / tps;
  if (splits <= 1) return 0;
  return (size_t)(batch * num_q_heads * splits * (fi::kHeadDim + 2) * sizeof(float));
}

namespace {

// Validation and launch shared by both entry points.  `fn` names the entry point in
// error messages; `workspace` is the caller's buffer or the library's static scratch.
int paged_fwd(const char* fn, const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache,
              const void* v_cache, int64_t num_pool_blocks, int64_t block_size,
              int64_t num_kv_heads, const int32_t* block_table, int64_t bt_stride,
              int64_t max_blocks_per_seq, const int32_t* context_lens, int64_t num_tokens,
              void* o, int64_t o_sb, int64_t o_sh, int64_t batch, int64_t num_q_heads,
              int64_t head_dim, float sm_scale, void* workspace, size_t workspace_bytes,
              void* stream) {
  using namespace fi;
  using namespace fi::decode;
  if (!head_dim_ok(head_dim)) {
    set_error("%s: head_dim %lld not supported (a multiple of 8 up to %d)", fn,
              (long long)head_dim, kHeadDim);
    return FI_ERR_UNSUPPORTED;
  }
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_tokens < 0 ||
      num_pool_blocks < 0 || max_blocks_per_seq < 0 || num_q_heads % num_kv_heads != 0) {
    set_error("%s: invalid sizes (batch %lld, heads %lld/%lld, tokens %lld)", fn,
              (long long)batch, (long long)num_q_heads, (long long)num_kv_heads,
              (long long)num_tokens);
    return FI_ERR_INVALID;
  }
  if (block_size <= 0) {
    set_error("%s: block_size %lld must be positive", fn, (long long)block_size);
    return FI_ERR_INVALID;
  }
  if (batch == 0) return FI_OK;
  if (num_tokens > (int64_t)kMaxSplitTokens * kMaxSplits ||
      block_size * num_kv_heads * head_dim * 2 > ((int64_t)1 << 30)) {
    set_error("%s: num_tokens %lld or block bytes too large", fn,
              (long long)num_tokens);
    return FI_ERR_UNSUPPORTED;
  }
  if (!q || !k_cache || !v_cache || !o || (!block_table && num_tokens > 0)) {
    set_error("%s: null pointer", fn);
    return FI_ERR_INVALID;
  }
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u ||
      (q_sb | q_sh) % 8 != 0) {
    set_error("%s: q and the pools must be 16-byte aligned", fn);
    return FI_ERR_INVALID;
  }

  const int64_t group = num_q_heads / num_kv_heads;
  Params p;
  p.q = (const half_t*)q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.k_cache = (const half_t*)k_cache;
  p.v_cache = (const half_t*)v_cache;
  p.num_pool_blocks = num_pool_blocks;
  p.block_size = (int)block_size;
  p.num_kv_heads = (int)num_kv_heads;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;
  p.context_lens = context_lens;
  p.num_tokens = (int)num_tokens;
  p.o = (half_t*)o;
  p.o_sb = o_sb;
  p.o_sh = o_sh;
  p.num_q_heads = (int)num_q_heads;
  p.group = (int)group;
  p.heads_per_wg = heads_per_wg(group);
  p.scale_log2 = sm_scale * kLog2e;
  const int64_t wg_per_row = num_kv_heads * (group / p.heads_per_wg);
  p.tokens_per_split = tokens_per_split(batch, wg_per_row, num_tokens > 0 ? num_tokens : 1);
  int64_t splits = (num_tokens + p.tokens_per_split - 1) / p.tokens_per_split;
  if (splits < 1) splits = 1;
  p.max_splits = (int)splits;
  p.direct = splits == 1;
  p.head_dim = (int)head_dim;
  p.d_chunks = (int)(head_dim / 8);
  // A partition stages the table entries of its tokens in LDS: at most
  // (tokens_per_split - 1) / block_size + 2 of them (always within kMaxSplitEntries for a
  // multiple of 16).
  const int64_t block_bytes = block_size * num_kv_heads * head_dim * 2;  // <= 1 GiB here
  const int addr = block_size % 16 == 0 ? kTileBlock
                   : num_pool_blocks <= ((int64_t)kFarOffset - 1) / block_bytes ? kLanePool
                                                                                : kRowBlock;
  if (addr != kTileBlock && (p.tokens_per_split - 1) / block_size + 2 > kAnyBlockEntries) {
    set_error("%s: num_tokens %lld too large for block_size %lld", fn, (long long)num_tokens,
              (long long)block_size);
    return FI_ERR_UNSUPPORTED;
  }
  p.part_o = nullptr;
  p.part_ml = nullptr;
  if (!p.direct) {
    const size_t need =
        fi_paged_attention_workspace_size(batch, num_q_heads, num_kv_heads, num_tokens, head_dim);
    if (!workspace || workspace_bytes < need) {
      set_error("%s: workspace of %zu bytes needed, %zu given", fn, need,
                workspace ? workspace_bytes : (size_t)0);
      return FI_ERR_WORKSPACE;
    }
    p.part_o = (float*)workspace;
    p.part_ml = p.part_o + batch * num_q_heads * splits * kHeadDim;
  }
  if (batch > 65535 || splits > 65535) {
    set_error("%s: grid too large", fn);
    return FI_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)wg_per_row, (unsigned)splits, (unsigned)batch);
  const dim3 block(kWaves * 64);
  if (addr == kTileBlock)
    hipLaunchKernelGGL(partition_kernel<kTileBlock>, grid, block, 0, (hipStream_t)stream, p);
  else if (addr == kLanePool)
    hipLaunchKernelGGL(partition_kernel<kLanePool>, grid, block, 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(partition_kernel<kRowBlock>, grid, block, 0, (hipStream_t)stream, p);
  int rc = check_launch(fn);
  if (rc != FI_OK || p.direct) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)num_q_heads, (unsigned)batch), dim3(kHeadDim), 0,
                     (hipStream_t)stream, p);
  return check_launch(fn);
}

// Scratch of fi_paged_attention_fwd_noalloc: the split-K partials, in a file-scope device
// array.  Each device holds its own copy from module load until the process ends.  Host
// code never uses the array's name as an address (on the host it is only a stand-in for
// the symbol): the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = FI_PAGED_NOALLOC_SCRATCH_BYTES;
__device__ __attribute__((aligned(256))) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the current device (looked up on the first call there).
int scratch_address(const char* fn, void** out) {
  using namespace fi;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no usable current HIP device", fn);
    return FI_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                hipGetErrorString(e));
      return FI_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FI_OK;
}

}  // namespace

extern "C" int fi_paged_attention_fwd(const void* q, int64_t q_sb, int64_t q_sh,
                                      const void* k_cache, const void* v_cache,
                                      int64_t num_pool_blocks, int64_t block_size,
                                      int64_t num_kv_heads, const int32_t* block_table,
                                      int64_t bt_stride, int64_t max_blocks_per_seq,
                                      const int32_t* context_lens, int64_t num_tokens, void* o,
                                      int64_t o_sb, int64_t o_sh, int64_t batch,
                                      int64_t num_q_heads, int64_t head_dim, float sm_scale,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  fi::clear_error();
  return paged_fwd("fi_paged_attention_fwd", q, q_sb, q_sh, k_cache, v_cache, num_pool_blocks,
                   block_size, num_kv_heads, block_table, bt_stride, max_blocks_per_seq,
                   context_lens, num_tokens, o, o_sb, o_sh, batch, num_q_heads, head_dim,
                   sm_scale, workspace, workspace_bytes, stream);
}

extern "C" int fi_paged_attention_fwd_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                              const void* k_cache, const void* v_cache,
                                              int64_t num_pool_blocks, int64_t block_size,
                                              int64_t num_kv_heads, const int32_t* block_table,
                                              int64_t bt_stride, int64_t max_blocks_per_seq,
                                              const int32_t* context_lens, int64_t num_tokens,
                                              void* o, int64_t o_sb, int64_t o_sh,
                                              int64_t batch, int64_t num_q_heads,
                                              int64_t head_dim, float sm_scale, void* stream) {
  using namespace fi;
  static const char* fn = "fi_paged_attention_fwd_noalloc";
  clear_error();
  const size_t need = batch > 0 && num_tokens > 0
                          ? fi_paged_attention_workspace_size(batch, num_q_heads, num_kv_heads,
                                                              num_tokens, head_dim)
                          : 0;
  if (need > kScratchBytes) {
    set_error("%s: these sizes need %zu bytes of split-K scratch, more than the %zu bytes "
              "this entry point holds per device; use fi_paged_attention_fwd with a workspace",
              fn, need, kScratchBytes);
    return FI_ERR_UNSUPPORTED;
  }
  void* ws = nullptr;
  if (need) {
    const int rc = scratch_address(fn, &ws);
    if (rc != FI_OK) return rc;
  }
  return paged_fwd(fn, q, q_sb, q_sh, k_cache, v_cache, num_pool_blocks, block_size,
                   num_kv_heads, block_table, bt_stride, max_blocks_per_seq, context_lens,
                   num_tokens, o, o_sb, o_sh, batch, num_q_heads, head_dim, sm_scale, ws,
                   need ? kScratchBytes : 0, stream);
}
