// Causal prefill attention for gfx950 (FlashAttention-2 forward), GQA-native.
//
// Replaces _flash_attn_fwd (kernels/attention.py:8-77) and its launcher (:80-113).
// Same result — softmax(Q K^T * sm_scale, causal) V per query head, fp32 online
// softmax, fp16 output — but laid out for MI355X:
//   * a workgroup (4 waves, one per SIMD) owns 64 query positions of up to 3 query heads
//     that share one kv head, so a K/V tile staged in LDS feeds every head of the GQA
//     group and K/V are never expanded (the reference call site expands them,
//     model.py:110-111).  Two workgroups share a CU: the two waves on a SIMD belong to
//     different workgroups, so neither waits at the other's barriers;
//   * the grid covers (query tile, head group, batch) with the heaviest causal tiles
//     dispatched first, instead of one program walking a whole head (:34);
//   * S^T = K Q^T and O^T = V^T P^T run on v_mfma_f32_16x16x32_f16: the lane holding a
//     query column keeps its scores, P and O in registers with no shuffles between the
//     two products; K fragments are read from LDS as A operands and V^T fragments with
//     the LDS transpose read (ds_read_b64_tr_b16);
//   * 64-key K/V tiles are copied global->LDS by the buffer unit (no register staging),
//     double-buffered; each slice issues its share of the next tile's copy;
//   * the diagonal tile is processed first; when a pool is given, the workgroup that
//     owns a 64-token tile of K/V also copies it into the paged pool (the write of
//     model.py:176-183, any block size), so the scatter costs no extra read.
#include "common.h"

namespace fi {
namespace prefill {

constexpr int kWaves = 4;                        // one wave per SIMD; two workgroups per CU
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerWave = 16;                 // query positions per wave
constexpr int kQTile = kWaves * kRowsPerWave;    // query positions per workgroup (64)
constexpr int kKTile = 64;                       // keys per K/V tile (one pool block)
constexpr int kPoolBlock = 64;                   // block_size of the fused pool write
constexpr int kRowBytes = kHeadDim * 2;          // one K or V row in LDS (256 bytes)
constexpr int kTileBytes = kKTile * kRowBytes;   // 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;      // K tile + V tile (2 stages: 64 KiB)
constexpr int kOutOfRange = 0x7ffffff0;          // buffer offset past any tensor: loads give 0
constexpr int kBufferWord3 = 0x00020000;
constexpr float kLazyLog2 = 8.f;  // the reference max may lag the true max by 2^8

static_assert(kQTile == kKTile, "a query tile has exactly one diagonal key tile");
static_assert(kKTile % kPoolBlock == 0, "a key tile covers whole pool blocks");

struct Params {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int seq_len;
  int num_kv_heads;
  int group;         // query heads per kv head
  int hg_per_kv;     // workgroups per kv head (group / heads per workgroup)
  float scale_log2;  // |sm_scale| * log2(e)
  float lazy_raw;    // kLazyLog2 / scale_log2: slack of the reference max in raw units
  float lazy_log2;   // lazy_raw * scale_log2 (about kLazyLog2)
  uint32_t q_sign;   // 0x80008000 when sm_scale < 0: Q is negated instead of the scale
  int q_rows;        // rows of Q loaded: seq_len, or 0 when sm_scale == 0 (Q read as zeros)
  int num_q_tiles;
  int k_records;     // bytes addressable from one (batch, kv head) base of k
  int v_records;
  int k_row_bytes;   // k_ss * 2 (spans are checked to fit 31 bits)
  int v_row_bytes;
  half_t* k_cache;   // optional pool [num_pool_blocks, block_size, num_kv_heads, head_dim]
  half_t* v_cache;
  int64_t num_pool_blocks;
  int block_size;
  const int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
  int head_dim;      // D <= kHeadDim, a multiple of 8: tiles and fragments stay kHeadDim
  int d_chunks;      // wide, and the 16-byte chunks past D are loaded as zeros
};

// LDS tile layouts ("panels"): a K tile is 4 panels of 64 bytes per key (head_dim
// columns 32i..32i+31 in panel i), a V tile 8 panels of 32 bytes per key (columns
// 16dt..16dt+15 in panel dt).  Every MFMA fragment read then takes one base register
// per lane plus an immediate offset.  A K fragment read gives each 16-lane group 16
// consecutive keys at one 16-byte chunk; the four chunks of key r are stored
// XOR-permuted by (r >> 1) & 3.  Measured with an in-bounds probe of that read on gfx950:
// 4 LDS-active cycles per ds_read_b128 and no bank-conflict cycles, against 8 cycles (4 of
// them conflicts) with (r >> 2) & 3, with r & 3 or with no permutation.  A V^T fragment
// read (8 bytes, 32 lanes at a time) covers 8 consecutive keys x 32 bytes and is
// conflict-free as stored.  Byte offset of 16-byte chunk ch (0..15) of key row r:
constexpr int kKPanel = kKTile * 64;  // bytes per K panel
constexpr int kVPanel = kKTile * 32;  // bytes per V panel
__device__ __forceinline__ int k_off(int r, int ch) {
  return (ch >> 2) * kKPanel + r * 64 + (((ch & 3) ^ ((r >> 1) & 3)) << 4);
}
__device__ __forceinline__ int v_off(int r, int ch) {
  return (ch >> 1) * kVPanel + r * 32 + ((ch & 1) << 4);
}

// Issue the direct-to-LDS loads of this wave's share of the K/V tile at key k0 into
// `stage` (K at +0, V at +kTileBytes).  One instruction moves 64 lanes x 16 bytes to
// 1 KiB of consecutive LDS: for K, 16 keys of one panel (lane l: key l/4, chunk
// 4*panel + l%4); for V, 32 keys of one panel (lane l: key l/2, chunk 2*panel + l%2).
// Wave w's K instructions cover keys 16w..16w+15 in all four panels and its V
// instructions keys 32(w/2).. in four of the eight panels, so the lines a wave touches
// are reused across its own back-to-back instructions.  Keys past seq_len, or a tile
// past the end (k0 < 0), fetch zeros through the buffer bounds check.
template <int NW = kWaves>
__device__ __forceinline__ void issue_tile_part(const Params& p, __amdgpu_buffer_rsrc_t kr,
                                                __amdgpu_buffer_rsrc_t vr, char* stage, int k0,
                                                int w, int lane, int q) {
  typedef void __attribute__((address_space(3))) lds_void;
  constexpr int kPer = (kTileBytes / 1024) / NW;  // instructions per wave per tensor
  const int n = kPer * w + q;  // instruction index within the tile (uniform)
  {
    // slot l holds key row0 + l/4 at permuted position l%4: logical chunk
    // (l % 4) ^ ((l / 8) % 4) of the panel (see k_off; row0 is a multiple of 16)
    const int panel = n & 3, row0 = 16 * (n >> 2);
    const int key = k0 + row0 + (lane >> 2);
    const bool ok = k0 >= 0 && key < p.seq_len;
    const int ch = 4 * panel + ((lane & 3) ^ ((lane >> 3) & 3));
    const int off = ok && ch < p.d_chunks ? key * p.k_row_bytes + (ch << 4) : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        kr, (lds_void*)(stage + panel * kKPanel + row0 * 64), 16, off, 0, 0, 0);
  }
  {
    const int panel = n & 7, row0 = 32 * (n >> 3);
    const int key = k0 + row0 + (lane >> 1);
    const bool ok = k0 >= 0 && key < p.seq_len;
    const int ch = 2 * panel + (lane & 1);
    const int off = ok && ch < p.d_chunks ? key * p.v_row_bytes + (ch << 4) : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        vr, (lds_void*)(stage + kTileBytes + panel * kVPanel + row0 * 32), 16, off, 0, 0, 0);
  }
}
template <int NW = kWaves>
__device__ __forceinline__ void issue_tile(const Params& p, __amdgpu_buffer_rsrc_t kr,
                                           __amdgpu_buffer_rsrc_t vr, char* stage, int k0,
                                           int w, int lane) {
  constexpr int kPer = (kTileBytes / 1024) / NW;
  static_assert(kPer * NW * 1024 == kTileBytes, "tile split across waves");
#pragma unroll
  for (int q = 0; q < kPer; ++q) issue_tile_part<NW>(p, kr, vr, stage, k0, w, lane, q);
}
constexpr int kIssuePerTile = 2 * (kTileBytes / 1024) / kWaves;  // DMA instructions per wave per tile

// The diagonal tile (keys k0 .. k0 + 63, k0 a multiple of 64) is exactly one pool block:
// logical block k0 / 64 of the row, whose table entry `entry` the caller loaded (valid only
// when `row_ok`, i.e. that block is inside the table).  The entry is passed through an
// empty asm statement first, so its first use (and the compiler's wait for the load) stays
// here, after the caller's own waits, rather than next to the load.
__device__ __forceinline__ int64_t pool_block_base(const Params& p, bool row_ok, int entry,
                                                   int kvh) {
  asm volatile("" : "+v"(entry));
  entry = __builtin_amdgcn_readfirstlane(entry);
  if (!row_ok || entry < 0 || entry >= p.num_pool_blocks) return -1;
  return (int64_t)entry * kPoolBlock * p.num_kv_heads * p.head_dim + (int64_t)kvh * p.head_dim;
}

// Any other block size: lane r of every wave holds the table entry of row r of the diagonal
// tile (-1 when the row is past seq_len or the table), loaded by the caller.  The element
// offset of row `slot`'s chunk `ch` in the pool, or -1 when the row has no valid block.
// Every lane of the wave must call this (the entry comes from lane `slot` by ds_bpermute).
__device__ __forceinline__ int64_t pool_row_dst(const Params& p, int entry, int kvh, int k0,
                                                int slot, int ch) {
  const int e = __builtin_amdgcn_ds_bpermute(slot << 2, entry);
  if (e < 0 || e >= p.num_pool_blocks) return -1;
  const int tok = k0 + slot;
  const int64_t row = (int64_t)e * p.block_size + tok % p.block_size;
  return (row * p.num_kv_heads + kvh) * p.head_dim + 8 * ch;
}

// Copy the resident diagonal tile from LDS into the pool (kRows: any block size other
// than 64, one entry per row).
template <bool kRows, int NT = kThreads>
__device__ __forceinline__ void write_pool(const Params& p, const char* stage, bool row_ok,
                                           int entry, int kvh, int k0, int tid) {
  if (kRows) {
    asm volatile("" : "+v"(entry));  // the wait for the entries' loads stays here
#pragma unroll
    for (int j = 0; j < kKTile * 16 / NT; ++j) {
      const int f = NT * j + tid;
      const int slot = f >> 4, ch = f & 15;
      const int64_t dst = pool_row_dst(p, entry, kvh, k0, slot, ch);
      if (k0 + slot >= p.seq_len || ch >= p.d_chunks || dst < 0) continue;
      *(u32x4*)(p.k_cache + dst) = *(const u32x4*)(stage + k_off(slot, ch));
      *(u32x4*)(p.v_cache + dst) = *(const u32x4*)(stage + kTileBytes + v_off(slot, ch));
    }
    return;
  }
  const int64_t base = pool_block_base(p, row_ok, entry, kvh);
  if (base < 0) return;
  const int64_t row_stride = (int64_t)p.num_kv_heads * p.head_dim;
#pragma unroll
  for (int j = 0; j < kKTile * 16 / NT; ++j) {
    const int f = NT * j + tid;
    const int slot = f >> 4;  // row within the tile
    if (k0 + slot >= p.seq_len || (f & 15) >= p.d_chunks) continue;
    const int64_t dst = base + slot * row_stride + 8 * (f & 15);
    *(u32x4*)(p.k_cache + dst) = *(const u32x4*)(stage + k_off(slot, f & 15));
    *(u32x4*)(p.v_cache + dst) = *(const u32x4*)(stage + kTileBytes + v_off(slot, f & 15));
  }
}

// The same copy split by wave: wave w stores exactly the LDS bytes its own copy
// instructions of a later tile overwrite (K keys 16w..16w+15, all 256 bytes; V keys
// 32(w/2)..32(w/2)+31, head_dim columns 64(w%2)..64(w%2)+63; see issue_tile_part), so it
// may run after the tile's last barrier, just before this wave refills the stage.
__device__ __forceinline__ void write_pool_wave(const Params& p, const char* stage, bool row_ok,
                                                int entry, int kvh, int k0, int w, int lane) {
  static_assert(kWaves == 4 && kKTile == 64, "wave split of the pool copy");
  const int64_t base = pool_block_base(p, row_ok, entry, kvh);
  if (base < 0) return;
  const int64_t row_stride = (int64_t)p.num_kv_heads * p.head_dim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = 64 * j + lane;
    {
      const int slot = 16 * w + (f >> 4), ch = f & 15;
      if (k0 + slot < p.seq_len && ch < p.d_chunks)
        *(u32x4*)(p.k_cache + base + slot * row_stride + 8 * ch) =
            *(const u32x4*)(stage + k_off(slot, ch));
    }
    {
      const int slot = 32 * (w >> 1) + (f >> 3), ch = 8 * (w & 1) + (f & 7);
      if (k0 + slot < p.seq_len && ch < p.d_chunks)
        *(u32x4*)(p.v_cache + base + slot * row_stride + 8 * ch) =
            *(const u32x4*)(stage + kTileBytes + v_off(slot, ch));
    }
  }
}

// V^T MFMA fragment half: lane (col = i, g) receives keys key0 + j (j = 0..3) of head_dim
// column 16*dt + i, where key0 = row0 + 4g.  Lane i of each 16-lane group addresses row
// row0 + 4g + i/4, columns 16*dt + 4*(i%4)..+3 (ds_read_b64_tr_b16 hands element i%4 of
// lane 4j + i/4's 4-element chunk to lane i as element j).
__device__ __forceinline__ u32x2 vt_read(const char* vs, int row0, int dt, int col, int g) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const char* ptr = vs + dt * kVPanel + (row0 + 4 * g + (col >> 2)) * 32 + ((col & 3) << 3);
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s4 __attribute__((address_space(3)))*)ptr);
  return __builtin_bit_cast(u32x2, v);
}

// PV of half c of a resident tile: O^T += V^T P^T (slots 0..3 = keys 4g..4g+3,
// 4..7 = 16+4g..16+4g+3) in tiles 0..7, and the softmax denominator l in tile 8: an
// all-ones A operand puts sum_k p[k][q] (the fp16 values PV uses) in each of its rows.
// On the matrix core this costs one MFMA per head and slice; as VALU row sums
// (v_dot2_f32_f16) it took 12 instructions per slice that never overlap MFMA work.
template <int HPW>
__device__ __forceinline__ void pv_half8(const char* vs, int c, int col, int g,
                                         const half8 (&pf)[HPW], floatx4 (&acc)[HPW][9]) {
  // each V^T fragment is read one step ahead of its MFMAs, as in qk_slice
  auto frag = [&](int dt) {
    const u32x2 a0 = vt_read(vs, 32 * c, dt, col, g);
    const u32x2 a1 = vt_read(vs, 32 * c + 16, dt, col, g);
    return as_half8(u32x4{a0[0], a0[1], a1[0], a1[1]});
  };
  half8 vf = frag(0);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    half8 vn;
    if (dt + 1 < 8) vn = frag(dt + 1);
#pragma unroll
    for (int j = 0; j < HPW; ++j) acc[j][dt] = mfma16x16x32(vf, pf[j], acc[j][dt]);
    if (dt + 1 < 8) vf = vn;
  }
  const half8 ones = as_half8(u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
#pragma unroll
  for (int j = 0; j < HPW; ++j) acc[j][8] = mfma16x16x32(ones, pf[j], acc[j][8]);
}

// S^T = K Q^T for 32-key slice c of a resident K tile: s[j][t] holds keys
// 32c + 16t + 4g + r (tile-relative) for query column col of head j.  Each K fragment is
// read one step ahead of its MFMAs: read, wait, multiply in turn left every read's LDS
// latency exposed (the copies landing in LDS lengthen it), and the prefetch took the
// batch 4 x 4096 call from 404.7 to 384.9 us.
template <int HPW>
__device__ __forceinline__ void qk_slice(const char* ks, int c, int col, int g,
                                         const half8 (&qf)[HPW][4], floatx4 (&s)[HPW][2]) {
#pragma unroll
  for (int j = 0; j < HPW; ++j) s[j][0] = s[j][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  // fragment u = 4t + i: keys 32c + 16t + col, head_dim chunk panel i
  auto frag = [&](int u) {
    const int t = u >> 2, i = u & 3;
    return as_half8(*(const u32x4*)(ks + i * kKPanel + (32 * c + 16 * t + col) * 64 +
                                    ((g ^ ((col >> 1) & 3)) << 4)));
  };
  half8 cur = frag(0);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    half8 nxt;
    if (u + 1 < 8) nxt = frag(u + 1);
#pragma unroll
    for (int j = 0; j < HPW; ++j) s[j][u >> 2] = mfma16x16x32(cur, qf[j][u & 3], s[j][u >> 2]);
    if (u + 1 < 8) cur = nxt;
  }
}

// This lane's maximum over its 8 scores of each head.
template <int HPW>
__device__ __forceinline__ void lane_max(const floatx4 (&s)[HPW][2], float (&lmax)[HPW]) {
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    float x = fmaxf(fmaxf(fmaxf(s[j][0][0], s[j][0][1]), s[j][0][2]), s[j][0][3]);
    lmax[j] = fmaxf(fmaxf(fmaxf(fmaxf(x, s[j][1][0]), s[j][1][1]), s[j][1][2]), s[j][1][3]);
  }
}

// Online softmax with a lazily moved reference max m (raw score units):
// p = exp2(s*c2 - m*c2).  m only moves when some score exceeds it by more than
// kLazyLog2 in the log2 domain, so p <= 2^kLazyLog2 (exact in fp16, O and l in fp32) and
// the softmax is unchanged.  The running state is the threshold t = m + lazy_raw, so the
// test is one compare with no cross-lane step; when any lane's test fires (rare after
// the first slices), every head's row max is reduced across the column's four lanes
// and O and l (accumulator tiles 0..8) are rescaled (alpha == 1 for heads whose
// threshold stays).
template <int HPW>
__device__ __forceinline__ void maybe_move_max(const Params& p, const float (&lmax)[HPW],
                                               float (&t_run)[HPW], floatx4 (&acc)[HPW][9]) {
  bool move = false;
#pragma unroll
  for (int j = 0; j < HPW; ++j) move |= lmax[j] > t_run[j];
  if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const float t_old = t_run[j];
      const float rmax = row4_max(lmax[j]);
      const float t_new = rmax > t_old ? rmax + p.lazy_raw : t_old;
      const float alpha = fast_exp2((t_old - t_new) * p.scale_log2);
      t_run[j] = t_new;
#pragma unroll
      for (int dt = 0; dt < 9; ++dt) acc[j][dt] *= alpha;
    }
  }
}

// P = exp2(s*c2 - m*c2) rounded to fp16 (the PV operand).
template <int HPW>
__device__ __forceinline__ void softmax_exp(const Params& p, const floatx4 (&s)[HPW][2],
                                            const float (&t_run)[HPW], half8 (&pf)[HPW]) {
  const float c2 = p.scale_log2;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const float mc = __builtin_fmaf(t_run[j], c2, -p.lazy_log2);  // m * c2
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        pf[j][4 * t + r] = (half_t)fast_exp2(__builtin_fmaf(s[j][t][r], c2, -mc));
  }
}

// A tile on the diagonal: masked (key > position, key >= seq_len), slices wholly above
// this wave's last position skipped; one slice at a time.
template <int HPW>
__device__ __forceinline__ void consume_diag(const Params& p, const char* stage, int k0,
                                             int qpos, int wave_last, int col, int g,
                                             const half8 (&qf)[HPW][4], float (&m_run)[HPW],
                                             floatx4 (&acc)[HPW][9]) {
  const char* ks = stage;
  const char* vs = stage + kTileBytes;
#pragma unroll
  for (int c = 0; c < kKTile / 32; ++c) {
    if (k0 + 32 * c > wave_last) break;
    floatx4 s[HPW][2];
    qk_slice<HPW>(ks, c, col, g, qf, s);
#pragma unroll
    for (int j = 0; j < HPW; ++j)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 32 * c + 16 * t + 4 * g + r;
          if (key > qpos || key >= p.seq_len) s[j][t][r] = -__builtin_inff();
        }
    float lmax[HPW];
    lane_max<HPW>(s, lmax);
    maybe_move_max<HPW>(p, lmax, m_run, acc);
    half8 pf[HPW];
    softmax_exp<HPW>(p, s, m_run, pf);
    pv_half8<HPW>(vs, c, col, g, pf, acc);
  }
}


// A tile wholly below the diagonal: per 32-key slice, QK for every head of the group
// (each K fragment read once), the online softmax, then PV (each V^T fragment read
// once).  No masking.
template <int HPW>
__device__ __forceinline__ void consume_full(const Params& p, const char* stage, int col,
                                             int g, const half8 (&qf)[HPW][4],
                                             float (&m_run)[HPW], floatx4 (&acc)[HPW][9],
                                             __amdgpu_buffer_rsrc_t kr,
                                             __amdgpu_buffer_rsrc_t vr, char* nxt, int k0n,
                                             int w, int lane) {
  const char* ks = stage;
  const char* vs = stage + kTileBytes;
  constexpr int kPer = (kTileBytes / 1024) / kWaves;  // copy instruction pairs per wave
  constexpr int kPerSlice = kPer / (kKTile / 32);
  static_assert(kPerSlice * (kKTile / 32) == kPer, "copy instructions split evenly over slices");
#pragma unroll
  for (int c = 0; c < kKTile / 32; ++c) {
    // A uniform branch between slices (never taken) keeps the compiler from treating
    // the unrolled slices as one straight-line region, which otherwise overlaps them
    // far beyond the register file and spills.
    if (p.seq_len < 0) break;
    floatx4 s[HPW][2];
    qk_slice<HPW>(ks, c, col, g, qf, s);
    // this slice's share of the next tile's copy, issued while the QK MFMAs run (all
    // waves issuing a whole tile at once would queue behind each other)
#pragma unroll
    for (int q = 0; q < kPerSlice; ++q) issue_tile_part(p, kr, vr, nxt, k0n, w, lane, kPerSlice * c + q);
    float lmax[HPW];
    lane_max<HPW>(s, lmax);
    maybe_move_max<HPW>(p, lmax, m_run, acc);
    half8 pf[HPW];
    softmax_exp<HPW>(p, s, m_run, pf);
    pv_half8<HPW>(vs, c, col, g, pf, acc);
  }
}

// HPW: query heads per workgroup.  kRows: a fused pool write with a block size other than 64 (the diagonal tile then spans
// several pool blocks or part of one; it is written at the start, before the accumulators
// are live, as that write needs registers for per-row addresses).
template <int HPW, bool kRows>
__global__ __launch_bounds__(kThreads, 2) void fwd_kernel(Params p) {
  // two pipeline stages of one K tile + one V tile each (distinct objects, so the
  // compiler tracks their DMA writes separately)
  __shared__ __attribute__((aligned(16))) char st0[kStageBytes];
  __shared__ __attribute__((aligned(16))) char st1[kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int col = lane & 15;
  const int g = lane >> 4;

  const int qt = p.num_q_tiles - 1 - (int)blockIdx.y;  // heaviest tiles first
  const int q0 = qt * kQTile;
  const int hg_total = p.num_kv_heads * p.hg_per_kv;
  const int b = blockIdx.x / hg_total;
  const int hrem = blockIdx.x % hg_total;
  const int kvh = hrem / p.hg_per_kv;
  const int hsub = hrem % p.hg_per_kv;
  const int head0 = kvh * p.group + hsub * HPW;

  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.k + (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh), (short)0, p.k_records, kBufferWord3);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.v + (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh), (short)0, p.v_records, kBufferWord3);

  // Q^T fragments: column col = query position q0 + 16w + col; MFMA i takes
  // d = 32*i + 8*g + s in reduction slot 8*g + s (K fragments use the same map).
  const int qpos = q0 + kRowsPerWave * w + col;
  half8 qf[HPW][4];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const half_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(head0 + j) * p.q_sh +
                         (int64_t)(qpos < p.seq_len ? qpos : 0) * p.q_ss;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qpos < p.q_rows && 32 * i + 8 * g < p.head_dim) v = *(const u32x4*)(qrow + 32 * i + 8 * g);
      qf[j][i] = as_half8(v ^ p.q_sign);  // exact negation when sm_scale < 0
    }
  }

  float m_run[HPW];
  floatx4 acc[HPW][9];  // per head: O^T head_dim rows 16dt..16dt+15 (dt < 8), l (dt = 8)
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    m_run[j] = kNegBig;
#pragma unroll
    for (int dt = 0; dt < 9; ++dt) acc[j][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Key tiles: the diagonal tile (keys q0..q0+kKTile-1, this workgroup's own positions)
  // first, then tiles 0, 1, ... before it.
  const int n = qt + 1;
  auto key0 = [&](int idx) -> int {
    if (idx >= n) return -1;  // past the end: loads read zeros
    return (idx == 0 ? qt : idx - 1) * kKTile;
  };
  const bool pool = p.k_cache != nullptr && hsub == 0;
  // The pool block of the diagonal tile: logical block qt of row b (block_size 64).  Its
  // table entry is loaded right after the first copies go out and first used in the pool
  // write, so the load's latency hides under the first tile's.  With another block size
  // lane r loads the entry of the block holding position q0 + r instead.
  const bool pool_row = pool && qt < p.max_blocks_per_seq;
  const bool pool_rows = pool && kRows;
  int pool_entry = -1;
  const int wave_last = q0 + kRowsPerWave * w + kRowsPerWave - 1;  // last position of the wave

  // Two-stage pipeline over 128-key tiles (tile idx in stage idx % 2): while consuming
  // tile idx, copy tile idx+1 into the other stage (its last reader finished before the
  // previous barrier), then wait for this wave's copies and barrier.  Tile 0 is the
  // diagonal tile (masked; copied to the pool when one is given), the others lie wholly
  // below the diagonal.
  // Both stages are free at the start: the copies of tiles 0 and 1 go out back to back,
  // and the first wait covers tile 0 only (loads complete in issue order).
  issue_tile(p, kr, vr, st0, key0(0), w, lane);
  issue_tile(p, kr, vr, st1, key0(1), w, lane);
  if (pool_rows) {
    const int tok = q0 + lane;
    const int lb = tok / p.block_size;
    if (tok < p.seq_len && lb < p.max_blocks_per_seq)
      pool_entry = p.block_table[(int64_t)b * p.bt_stride + lb];
  } else if (pool_row) {
    pool_entry = p.block_table[(int64_t)b * p.bt_stride + qt];
  }
  wait_vmcnt<kIssuePerTile>();
  __builtin_amdgcn_s_barrier();
  // The pool copy of the diagonal tile: with a following tile, each wave stores its share
  // at the start of tile 1, just before refilling stage 0, so the stores drain under tile
  // 1's work instead of under this tile's closing wait.
  if (pool && (n == 1 || kRows)) write_pool<kRows>(p, st0, pool_row, pool_entry, kvh, key0(0), tid);
  consume_diag<HPW>(p, st0, key0(0), qpos, wave_last, col, g, qf, m_run, acc);
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
#define FI_PREFILL_STEP(IDX, CUR, NXT)                                                    \
  {                                                                                       \
    if (!kRows && pool && (IDX) == 1)                                                     \
      write_pool_wave(p, NXT, pool_row, pool_entry, kvh, key0(0), w, lane);              \
    consume_full<HPW>(p, CUR, col, g, qf, m_run, acc, kr, vr, NXT, key0((IDX) + 1),        \
                      w, lane);                                                           \
    wait_vmcnt<0>();                                                                      \
    __builtin_amdgcn_s_barrier();                                                         \
  }
  for (int idx = 1; idx < n; idx += 2) {
    FI_PREFILL_STEP(idx, st1, st0)
    if (idx + 1 >= n) break;
    FI_PREFILL_STEP(idx + 1, st0, st1)
  }
#undef FI_PREFILL_STEP

  // ---- normalise and store: lane holds O[qpos][16*dt + 4*g + r].  The row sums combine
  // the four lanes of a column (every lane takes part; rows past seq_len are never stored).
  // The rows go through this wave's own part of the tile stages, idle since the last
  // barrier, so that each store instruction writes four whole 256-byte rows (16 lanes x 16
  // bytes per row) rather than 32-byte pieces of sixteen rows: a workgroup's slot is held
  // until its last stores complete.  Staged rows are padded to 272 bytes so that the
  // sixteen rows of one write land in distinct banks.
  constexpr int kORow = 272;
  static_assert(kWaves == 4 && 2 * HPW * kRowsPerWave * kORow <= kStageBytes,
                "waves 0-1 stage their rows in st0, waves 2-3 in st1");
  char* ostage = (w < 2 ? st0 : st1) + (w & 1) * (HPW * kRowsPerWave * kORow);
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const float inv = 1.f / acc[j][8][0];  // every row of tile 8 holds the column's l
    char* orow = ostage + (j * kRowsPerWave + col) * kORow + 8 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *(half4*)(orow + 32 * dt) = to_half4(acc[j][dt] * inv);
  }
  wave_lds_sync();
  const int r4 = lane >> 4;   // row within each group of four read by one instruction
  const int c16 = lane & 15;  // 16-byte chunk of the row
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave / 4; ++rr) {
      const int rl = 4 * rr + r4;
      const u32x4 v = *(const u32x4*)(ostage + (j * kRowsPerWave + rl) * kORow + 16 * c16);
      const int pos = q0 + kRowsPerWave * w + rl;
      if (pos < p.seq_len && c16 < p.d_chunks)
        *(u32x4*)(p.o + (int64_t)b * p.o_sb + (int64_t)(head0 + j) * p.o_sh +
                  (int64_t)pos * p.o_ss + 8 * c16) = v;
    }
  }
}

static int heads_per_wg(int64_t group) {
  for (int h = 3; h >= 1; --h)
    if (group % h == 0) return h;
  return 1;
}

}  // namespace prefill
}  // namespace fi

extern "C" int fi_flash_attention_fwd(const void* q, const void* k, const void* v, void* o,
                                      int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                      int64_t seq_len, int64_t head_dim, int64_t q_sb,
                                      int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_sh,
                                      int64_t k_ss, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                      int64_t o_sb, int64_t o_sh, int64_t o_ss, float sm_scale,
                                      void* k_cache, void* v_cache, int64_t num_pool_blocks,
                                      int64_t block_size, const int32_t* block_table,
                                      int64_t bt_stride, int64_t max_blocks_per_seq,
                                      void* stream) {
  using namespace fi;
  using namespace fi::prefill;
  clear_error();
  if (!head_dim_ok(head_dim)) {
    set_error("fi_flash_attention_fwd: head_dim %lld not supported (a multiple of 8 up to %d)",
              (long long)head_dim, kHeadDim);
    return FI_ERR_UNSUPPORTED;
  }
  if (batch < 0 || seq_len < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0) {
    set_error("fi_flash_attention_fwd: invalid sizes (batch %lld, heads %lld/%lld, seq %lld)",
              (long long)batch, (long long)num_q_heads, (long long)num_kv_heads,
              (long long)seq_len);
    return FI_ERR_INVALID;
  }
  if (batch == 0 || seq_len == 0) return FI_OK;
  if (seq_len > (1 << 24) || batch > 65535) {
    set_error("fi_flash_attention_fwd: sizes too large");
    return FI_ERR_UNSUPPORTED;
  }
  if (!q || !k || !v || !o) {
    set_error("fi_flash_attention_fwd: null pointer");
    return FI_ERR_INVALID;
  }
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15u ||
      (q_sb | q_sh | q_ss | k_sb | k_sh | k_ss | v_sb | v_sh | v_ss | o_sb | o_sh | o_ss) % 8 !=
          0) {
    set_error("fi_flash_attention_fwd: rows must be 16-byte aligned (strides multiple of 8)");
    return FI_ERR_INVALID;
  }
  if (k_cache) {
    if (!v_cache || !block_table) {
      set_error("fi_flash_attention_fwd: pool write needs v_cache and block_table");
      return FI_ERR_INVALID;
    }
    if (block_size <= 0 || block_size > (1 << 20)) {
      set_error("fi_flash_attention_fwd: invalid pool block_size %lld", (long long)block_size);
      return FI_ERR_INVALID;
    }
    if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) {
      set_error("fi_flash_attention_fwd: pools must be 16-byte aligned");
      return FI_ERR_INVALID;
    }
  }

  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t q_tiles = (seq_len + kQTile - 1) / kQTile;
  // Several query heads per workgroup share each staged K/V tile, but make the grid that
  // many times smaller.  A grid below two workgroups per CU leaves slots idle for the whole
  // call: one head per workgroup is then faster (batch 1 x 512: 12.8 against 22.4 us;
  // batch 1 x 3072: 93 against 101 us; from two per CU up, several heads win).
  int hpw = heads_per_wg(group);
  if (hpw > 1 && batch * num_kv_heads * (group / hpw) * q_tiles <
                     2 * (int64_t)device_cu_count((hipStream_t)stream))
    hpw = 1;
  Params p;
  p.q = (const half_t*)q;
  p.k = (const half_t*)k;
  p.v = (const half_t*)v;
  p.o = (half_t*)o;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_sh = k_sh; p.k_ss = k_ss;
  p.v_sb = v_sb; p.v_sh = v_sh; p.v_ss = v_ss;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.seq_len = (int)seq_len;
  p.num_kv_heads = (int)num_kv_heads;
  p.group = (int)group;
  p.hg_per_kv = (int)(group / hpw);
  // A zero scale makes every valid score 0 (uniform weights over the causal keys).  The
  // kernel masks scores to -inf before scaling, and -inf * 0 is NaN, so that case runs with
  // unit scale on an all-zero Q instead: scores are exactly 0, masked ones -inf.
  const bool zero_scale = sm_scale == 0.f;
  p.scale_log2 = zero_scale ? kLog2e : (sm_scale < 0 ? -sm_scale : sm_scale) * kLog2e;
  p.q_sign = sm_scale < 0 ? 0x80008000u : 0u;
  p.q_rows = zero_scale ? 0 : (int)seq_len;
  p.lazy_raw = p.scale_log2 > 0.f ? kLazyLog2 / p.scale_log2 : 0.f;
  p.lazy_log2 = p.lazy_raw * p.scale_log2;
  p.num_q_tiles = (int)q_tiles;
  p.k_cache = (half_t*)k_cache;
  p.v_cache = (half_t*)v_cache;
  p.num_pool_blocks = num_pool_blocks;
  p.block_size = (int)block_size;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;
  p.head_dim = (int)head_dim;
  p.d_chunks = (int)(head_dim / 8);
  const int64_t k_span = (seq_len - 1) * k_ss * 2 + head_dim * 2;
  const int64_t v_span = (seq_len - 1) * v_ss * 2 + head_dim * 2;
  if (k_ss <= 0 || v_ss <= 0 || k_span >= kOutOfRange || v_span >= kOutOfRange) {
    set_error("fi_flash_attention_fwd: one head's K/V rows must span < 2 GiB with positive strides");
    return FI_ERR_UNSUPPORTED;
  }
  p.k_records = (int)k_span;
  p.v_records = (int)v_span;
  p.k_row_bytes = (int)(k_ss * 2);
  p.v_row_bytes = (int)(v_ss * 2);

  const int64_t gx = batch * num_kv_heads * p.hg_per_kv;
  if (gx > 0x7fffffff || p.num_q_tiles > 65535) {
    set_error("fi_flash_attention_fwd: grid too large");
    return FI_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)gx, (unsigned)p.num_q_tiles);
  const dim3 block(kThreads);
  const bool rows = k_cache && block_size != kPoolBlock;
  const hipStream_t st = (hipStream_t)stream;
  switch (hpw * 2 + (rows ? 1 : 0)) {
    case 6: hipLaunchKernelGGL((fwd_kernel<3, false>), grid, block, 0, st, p); break;
    case 7: hipLaunchKernelGGL((fwd_kernel<3, true>), grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL((fwd_kernel<2, false>), grid, block, 0, st, p); break;
    case 5: hipLaunchKernelGGL((fwd_kernel<2, true>), grid, block, 0, st, p); break;
    case 3: hipLaunchKernelGGL((fwd_kernel<1, true>), grid, block, 0, st, p); break;
    default: hipLaunchKernelGGL((fwd_kernel<1, false>), grid, block, 0, st, p); break;
  }
  return check_launch("fi_flash_attention_fwd");
}
