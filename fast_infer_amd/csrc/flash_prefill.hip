// Causal prefill attention for gfx950 (FlashAttention-2 forward), GQA-native.
//
// Replaces _flash_attn_fwd (kernels/attention.py:8-77) and its launcher (:80-113).
// Same result — softmax(Q K^T * sm_scale, causal) V per query head, fp32 online
// softmax, fp16 output — but laid out for MI355X:
//   * a workgroup owns 64 query positions of all query heads that share one kv head
//     (up to 4), so a K/V tile staged in LDS feeds every head of the GQA group and K/V
//     are never expanded (the reference call site expands them, model.py:110-111);
//   * the grid covers (query tile, head group, batch) with the heaviest causal tiles
//     dispatched first, instead of one program walking a whole head (:34);
//   * S^T = K Q^T and O^T = V^T P^T run on v_mfma_f32_16x16x32_f16: the lane holding a
//     query column keeps its scores, P and O in registers with no shuffles between the
//     two products; K tiles are read from LDS as A fragments, V is transposed once per
//     tile while being staged into LDS (V^T rows);
//   * K/V tiles are double-buffered in LDS with the next tile's global loads in flight
//     during the current tile's MFMAs;
//   * the diagonal tile is processed first; when a pool is given, the workgroup that
//     owns a 64-token block of K/V also copies it into the paged pool (the write of
//     model.py:176-183), so the scatter costs no extra read.
#include "common.h"

namespace fi {
namespace prefill {

constexpr int kWaves = 4;
constexpr int kRowsPerWave = 16;                 // query positions per wave
constexpr int kQTile = kWaves * kRowsPerWave;    // query positions per workgroup
constexpr int kKTile = 64;                       // keys per K/V tile
constexpr int kKStride = kHeadDim + 8;           // fp16 per K row in LDS (bank padding)
constexpr int kVtStride = kKTile + 4;            // fp16 per V^T row in LDS (bank padding)
constexpr int kKHalfs = kKTile * kKStride;
constexpr int kVtHalfs = kHeadDim * kVtStride;
constexpr int kStageHalfs = kKHalfs + kVtHalfs;  // one buffer stage
constexpr int kSmemBytes = 2 * kStageHalfs * 2;
static_assert(kQTile == kKTile, "the diagonal tile must coincide with the query tile");

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
  int group;        // query heads per kv head
  int hg_per_kv;    // workgroups per kv head (group / heads per workgroup)
  float scale_log2; // sm_scale * log2(e)
  int num_q_tiles;
  half_t* k_cache;  // optional pool (block_size 64)
  half_t* v_cache;
  int64_t num_pool_blocks;
  const int32_t* block_table;
  int64_t bt_stride;
  int max_blocks_per_seq;
};

// Global->register staging of one 64-key K/V tile by the 256 threads of a workgroup.
struct TileRegs {
  u32x4 k[4];  // K chunk: key = k0 + (f >> 4), d = 8 * (f & 15), f = 256 * j + tid
  u32x4 v[4];  // V rows: key = k0 + 16 * w + 4 * kq + j, d = 8 * dc..8 * dc + 7
};

__device__ __forceinline__ void load_tile(const Params& p, const half_t* kh, const half_t* vh,
                                          int k0, int tid, int w, int dc, int kq, TileRegs& r) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = 256 * j + tid;
    const int key = k0 + (f >> 4);
    r.k[j] = key < p.seq_len ? *(const u32x4*)(kh + (int64_t)key * p.k_ss + 8 * (f & 15))
                             : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int key = k0 + 16 * w + 4 * kq + j;
    r.v[j] = key < p.seq_len ? *(const u32x4*)(vh + (int64_t)key * p.v_ss + 8 * dc)
                             : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void store_tile(half_t* stage, int tid, int w, int dc, int kq,
                                           const TileRegs& r) {
  half_t* ks = stage;
  half_t* vts = stage + kKHalfs;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = 256 * j + tid;
    *(u32x4*)(ks + (f >> 4) * kKStride + 8 * (f & 15)) = r.k[j];
  }
  // V^T: row d = 8*dc + e holds keys 16*w + 4*kq .. +3 (register transpose of 4x8).
#pragma unroll
  for (int e2 = 0; e2 < 4; ++e2) {
    const u32x2 lo = {pack_lo(r.v[0][e2], r.v[1][e2]), pack_lo(r.v[2][e2], r.v[3][e2])};
    const u32x2 hi = {pack_hi(r.v[0][e2], r.v[1][e2]), pack_hi(r.v[2][e2], r.v[3][e2])};
    *(u32x2*)(vts + (8 * dc + 2 * e2) * kVtStride + 16 * w + 4 * kq) = lo;
    *(u32x2*)(vts + (8 * dc + 2 * e2 + 1) * kVtStride + 16 * w + 4 * kq) = hi;
  }
}

// Copy the staged diagonal tile (keys k0..k0+63, one pool block) into the pool.
__device__ __forceinline__ void write_pool(const Params& p, int b, int kvh, int k0, int tid,
                                           int w, int dc, int kq, const TileRegs& r) {
  const int lb = k0 / kKTile;
  if (lb >= p.max_blocks_per_seq) return;
  const int64_t phys = p.block_table[(int64_t)b * p.bt_stride + lb];
  if (phys < 0 || phys >= p.num_pool_blocks) return;
  const int64_t row_stride = (int64_t)p.num_kv_heads * kHeadDim;
  const int64_t base = phys * kKTile * row_stride + (int64_t)kvh * kHeadDim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = 256 * j + tid;
    const int slot = f >> 4;
    if (k0 + slot < p.seq_len)
      *(u32x4*)(p.k_cache + base + slot * row_stride + 8 * (f & 15)) = r.k[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int slot = 16 * w + 4 * kq + j;
    if (k0 + slot < p.seq_len)
      *(u32x4*)(p.v_cache + base + slot * row_stride + 8 * dc) = r.v[j];
  }
}

template <int HPW>  // query heads per workgroup
__global__ __launch_bounds__(256) void fwd_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) char smem_raw[kSmemBytes];
  half_t* smem = (half_t*)smem_raw;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int col = lane & 15;
  const int g = lane >> 4;
  const int dc = lane >> 2;  // V loader: 8 head_dim values
  const int kq = lane & 3;   // V loader: 4 consecutive keys

  const int qt = p.num_q_tiles - 1 - (int)blockIdx.y;  // heaviest tiles first
  const int q0 = qt * kQTile;
  const int hg_total = p.num_kv_heads * p.hg_per_kv;
  const int b = blockIdx.x / hg_total;
  const int hrem = blockIdx.x % hg_total;
  const int kvh = hrem / p.hg_per_kv;
  const int hsub = hrem % p.hg_per_kv;
  const int head0 = kvh * p.group + hsub * HPW;

  const half_t* kh = p.k + (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh;
  const half_t* vh = p.v + (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh;

  // Q^T fragments: column col = query position q0 + 16w + col; MFMA i takes
  // d = 32*i + 8*g + s in reduction slot 8*g + s (the K fragment uses the same map).
  const int qpos = q0 + kRowsPerWave * w + col;
  half8 qf[HPW][4];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const half_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(head0 + j) * p.q_sh +
                         (int64_t)(qpos < p.seq_len ? qpos : 0) * p.q_ss;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qpos < p.seq_len) v = *(const u32x4*)(qrow + 32 * i + 8 * g);
      qf[j][i] = as_half8(v);
    }
  }

  float m_run[HPW], l_run[HPW];
  floatx4 acc[HPW][8];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    m_run[j] = kNegBig;
    l_run[j] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[j][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Tile order: the diagonal tile (index qt) first, then tiles 0 .. qt-1.
  const int n_tiles = qt + 1;
  TileRegs regs;
  load_tile(p, kh, vh, q0, tid, w, dc, kq, regs);
  if (p.k_cache && hsub == 0) write_pool(p, b, kvh, q0, tid, w, dc, kq, regs);
  store_tile(smem, tid, w, dc, kq, regs);
  __syncthreads();

  for (int idx = 0; idx < n_tiles; ++idx) {
    const bool diag = idx == 0;
    const int k0 = diag ? q0 : (idx - 1) * kKTile;
    const bool more = idx + 1 < n_tiles;
    if (more) load_tile(p, kh, vh, idx * kKTile, tid, w, dc, kq, regs);

    const half_t* ks = smem + (idx & 1) * kStageHalfs;
    const half_t* vts = ks + kKHalfs;

    // ---- S^T = K Q^T: s[j][t] holds keys k0 + 16t + 4g + r for query column col.
    floatx4 s[HPW][4];
#pragma unroll
    for (int j = 0; j < HPW; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) s[j][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half8 kf = as_half8(*(const u32x4*)(ks + (16 * t + col) * kKStride + 32 * i + 8 * g));
#pragma unroll
        for (int j = 0; j < HPW; ++j) s[j][t] = mfma16x16x32(kf, qf[j][i], s[j][t]);
      }
    }

    // ---- online softmax per head (log2 domain).
    half8 pf[HPW][2];
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      float tmax = kNegBig;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = s[j][t][r] * p.scale_log2;
          if (diag) {
            const int key = k0 + 16 * t + 4 * g + r;
            if (key > qpos || key >= p.seq_len) x = -__builtin_inff();
          }
          s[j][t][r] = x;
          tmax = fmaxf(tmax, x);
        }
      }
      tmax = row4_max(tmax);
      const float m_new = fmaxf(m_run[j], tmax);
      const float alpha = fast_exp2(m_run[j] - m_new);
      m_run[j] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = fast_exp2(s[j][t][r] - m_new);
          psum += e;
          pf[j][t >> 1][4 * (t & 1) + r] = (half_t)e;
        }
      }
      l_run[j] = l_run[j] * alpha + psum;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[j][dt] *= alpha;
    }

    // ---- O^T += V^T P^T over the two 32-key chunks.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const half_t* row = vts + (16 * dt + col) * kVtStride + 32 * c;
        const u32x2 a0 = *(const u32x2*)(row + 4 * g);
        const u32x2 a1 = *(const u32x2*)(row + 16 + 4 * g);
        const half8 vf = as_half8(u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
        for (int j = 0; j < HPW; ++j) acc[j][dt] = mfma16x16x32(vf, pf[j][c], acc[j][dt]);
      }
    }

    if (more) store_tile(smem + ((idx + 1) & 1) * kStageHalfs, tid, w, dc, kq, regs);
    __syncthreads();
  }

  // ---- normalise and store: lane holds O[qpos][16*dt + 4*g + r].  The row sums
  // combine lanes of the same column, which share qpos, so the branch is uniform
  // across every shuffle's partners.
  if (qpos < p.seq_len) {
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const float inv = 1.f / row4_sum(l_run[j]);
      half_t* orow = p.o + (int64_t)b * p.o_sb + (int64_t)(head0 + j) * p.o_sh +
                     (int64_t)qpos * p.o_ss + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *(half4*)(orow + 16 * dt) = to_half4(acc[j][dt] * inv);
    }
  }
}

static int heads_per_wg(int64_t group) {
  for (int h = 4; h >= 1; --h)
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
  if (head_dim != kHeadDim) {
    set_error("fi_flash_attention_fwd: head_dim %lld not supported (only %d)",
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
    if (block_size != kKTile) {
      set_error("fi_flash_attention_fwd: fused pool write needs block_size %d (got %lld)",
                kKTile, (long long)block_size);
      return FI_ERR_UNSUPPORTED;
    }
    if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) {
      set_error("fi_flash_attention_fwd: pools must be 16-byte aligned");
      return FI_ERR_INVALID;
    }
  }

  const int64_t group = num_q_heads / num_kv_heads;
  const int hpw = heads_per_wg(group);
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
  p.scale_log2 = sm_scale * kLog2e;
  p.num_q_tiles = (int)((seq_len + kQTile - 1) / kQTile);
  p.k_cache = (half_t*)k_cache;
  p.v_cache = (half_t*)v_cache;
  p.num_pool_blocks = num_pool_blocks;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.max_blocks_per_seq = (int)max_blocks_per_seq;

  const int64_t gx = batch * num_kv_heads * p.hg_per_kv;
  if (gx > 0x7fffffff || p.num_q_tiles > 65535) {
    set_error("fi_flash_attention_fwd: grid too large");
    return FI_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)gx, (unsigned)p.num_q_tiles);
  const dim3 block(kWaves * 64);
  switch (hpw) {
    case 4:
      hipLaunchKernelGGL(fwd_kernel<4>, grid, block, 0, (hipStream_t)stream, p);
      break;
    case 3:
      hipLaunchKernelGGL(fwd_kernel<3>, grid, block, 0, (hipStream_t)stream, p);
      break;
    case 2:
      hipLaunchKernelGGL(fwd_kernel<2>, grid, block, 0, (hipStream_t)stream, p);
      break;
    default:
      hipLaunchKernelGGL(fwd_kernel<1>, grid, block, 0, (hipStream_t)stream, p);
      break;
  }
  return check_launch("fi_flash_attention_fwd");
}
