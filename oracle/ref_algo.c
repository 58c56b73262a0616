/*
 * C restatement of the reference's attention programs — TEST INFRASTRUCTURE and the
 * CPU baseline ("port"); never linked into the product library.
 *
 * oracle_flash_fwd  : kernels/attention.py:80-113 + _flash_attn_fwd :8-77.  One
 *                     program per (batch, head) walks its Q tiles serially (:34) and,
 *                     for each, the causal K tiles (:47) with BLOCK_M = BLOCK_N =
 *                     max(16, min(32, next_pow2(seq_len))) (:95-96); fp32 scores (:55),
 *                     causal and bounds masks (:57-59), online softmax (:61-66),
 *                     PV accumulation (:68-70), fp16 store of acc / l (:74-77).
 *                     Query head h reads kv head h / (H / H_kv): identical to the
 *                     reference run on K/V expanded by repeat_interleave (model.py:110-111).
 * oracle_paged_fwd  : kernels/attention.py:191-233 + _paged_attention_kernel :116-188.
 *                     One program per (batch, query head): kv head = h / groups (:137-139),
 *                     loop over ceil(ctx / block_size) blocks through the block table
 *                     (:155-156), token mask (:158-160), fp32 dot (:168), online softmax
 *                     (:171-176), PV (:178-182), fp16 store (:186-188).  `ctx_lens`
 *                     (optional) gives each row its own length, which equals running
 *                     the reference once per row with num_tokens = ctx_b.
 *
 * Programs run in parallel with OpenMP (`nthreads`, 0 = runtime default).  All
 * arithmetic is fp32; fp16 <-> fp32 conversions are exact / round-to-nearest-even.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) /* inf or nan */
    return sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0);
  if (absx >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return sign | 0x7c00u;
  if (absx < 0x38800000u) { /* result subnormal or zero: value * 2^24, round half even */
    float a;
    memcpy(&a, &absx, 4);
    const float scaled = a * 16777216.0f; /* exact: power-of-two scaling */
    float r = nearbyintf(scaled);         /* default rounding mode: nearest-even */
    return sign | (uint16_t)r;
  }
  /* normal: keep 10 mantissa bits, round half to even on the 13 dropped bits */
  const uint32_t mant = absx & 0x7fffffu;
  const uint32_t exp = (absx >> 23) - 127 + 15;
  uint32_t h = (exp << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry into exp */
  return sign | (uint16_t)h;
}

static int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

int oracle_flash_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                     int B, int H, int Hkv, int S, int D,
                     int64_t q_sb, int64_t q_sh, int64_t q_ss,
                     int64_t k_sb, int64_t k_sh, int64_t k_ss,
                     int64_t v_sb, int64_t v_sh, int64_t v_ss,
                     int64_t o_sb, int64_t o_sh, int64_t o_ss,
                     float sm_scale, const int32_t* programs, int nprog, int nthreads) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || S <= 0 || D <= 0 || H % Hkv) return 1;
  const int G = H / Hkv;
  int bm = next_pow2(S);
  bm = bm < 32 ? bm : 32;
  bm = bm > 16 ? bm : 16;
  const int BM = bm, BN = bm;
  const int total = programs ? nprog : B * H;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  int fail = 0;
#pragma omp parallel
  {
    float* qt = (float*)malloc(sizeof(float) * BM * D);
    float* kt = (float*)malloc(sizeof(float) * BN * D);
    float* vt = (float*)malloc(sizeof(float) * BN * D);
    float* acc = (float*)malloc(sizeof(float) * BM * D);
    float* qk = (float*)malloc(sizeof(float) * BM * BN);
    float* m_i = (float*)malloc(sizeof(float) * BM);
    float* l_i = (float*)malloc(sizeof(float) * BM);
    if (!qt || !kt || !vt || !acc || !qk || !m_i || !l_i) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int pi = 0; pi < total; ++pi) {
        const int b = programs ? programs[2 * pi] : pi / H;
        const int h = programs ? programs[2 * pi + 1] : pi % H;
        const uint16_t* qh = q + b * q_sb + h * q_sh;
        const uint16_t* kh = k + b * k_sb + (h / G) * k_sh;
        const uint16_t* vh = v + b * v_sb + (h / G) * v_sh;
        uint16_t* oh = o + b * o_sb + h * o_sh;
        for (int start_m = 0; start_m < S; start_m += BM) {
          for (int r = 0; r < BM; ++r) {
            m_i[r] = -INFINITY;
            l_i[r] = 0.f;
            for (int d = 0; d < D; ++d) {
              acc[r * D + d] = 0.f;
              qt[r * D + d] = (start_m + r < S) ? h2f(qh[(start_m + r) * q_ss + d]) : 0.f;
            }
          }
          for (int start_n = 0; start_n < start_m + BM; start_n += BN) {
            for (int c = 0; c < BN; ++c)
              for (int d = 0; d < D; ++d) {
                const int n = start_n + c;
                kt[c * D + d] = n < S ? h2f(kh[n * k_ss + d]) : 0.f;
                vt[c * D + d] = n < S ? h2f(vh[n * v_ss + d]) : 0.f;
              }
            for (int r = 0; r < BM; ++r) {
              const int m = start_m + r;
              float rmax = -INFINITY;
              for (int c = 0; c < BN; ++c) {
                const int n = start_n + c;
                float s = 0.f;
                for (int d = 0; d < D; ++d) s += qt[r * D + d] * kt[c * D + d];
                s *= sm_scale;
                if (!(m >= n) || !(m < S && n < S)) s = -INFINITY;
                qk[r * BN + c] = s;
                rmax = s > rmax ? s : rmax;
              }
              const float m_new = m_i[r] > rmax ? m_i[r] : rmax;
              const float alpha = expf(m_i[r] - m_new);
              float psum = 0.f;
              for (int c = 0; c < BN; ++c) {
                const float p = expf(qk[r * BN + c] - m_new);
                qk[r * BN + c] = p;
                psum += p;
              }
              l_i[r] = l_i[r] * alpha + psum;
              for (int d = 0; d < D; ++d) {
                float a = acc[r * D + d] * alpha;
                for (int c = 0; c < BN; ++c) a += qk[r * BN + c] * vt[c * D + d];
                acc[r * D + d] = a;
              }
              m_i[r] = m_new;
            }
          }
          for (int r = 0; r < BM && start_m + r < S; ++r)
            for (int d = 0; d < D; ++d)
              oh[(start_m + r) * o_ss + d] = f2h(acc[r * D + d] / l_i[r]);
        }
      }
    }
    free(qt); free(kt); free(vt); free(acc); free(qk); free(m_i); free(l_i);
  }
  return fail ? 2 : 0;
}

int oracle_paged_fwd(const uint16_t* q, int64_t q_sb, int64_t q_sh,
                     const uint16_t* k_cache, const uint16_t* v_cache,
                     int num_pool_blocks, int block_size, int Hkv,
                     const int32_t* block_table, int64_t bt_stride,
                     const int32_t* ctx_lens, int num_tokens,
                     uint16_t* o, int64_t o_sb, int64_t o_sh,
                     int B, int H, int D, float sm_scale, int nthreads) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || D <= 0 || H % Hkv || block_size <= 0) return 1;
  const int groups = H / Hkv;
  const int64_t slot_stride = (int64_t)Hkv * D;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  int fail = 0;
#pragma omp parallel
  {
    float* qv = (float*)malloc(sizeof(float) * D);
    float* acc = (float*)malloc(sizeof(float) * D);
    float* sc = (float*)malloc(sizeof(float) * block_size);
    if (!qv || !acc || !sc) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int pi = 0; pi < B * H; ++pi) {
        const int b = pi / H, h = pi % H, kvh = h / groups;
        const int ntok = ctx_lens ? ctx_lens[b] : num_tokens;
        uint16_t* oh = o + b * o_sb + h * o_sh;
        if (ntok <= 0) {
          for (int d = 0; d < D; ++d) oh[d] = 0;
          continue;
        }
        for (int d = 0; d < D; ++d) {
          qv[d] = h2f(q[b * q_sb + h * q_sh + d]);
          acc[d] = 0.f;
        }
        float m_i = -INFINITY, l_i = 0.f;
        const int nblocks = (ntok + block_size - 1) / block_size;
        for (int blk = 0; blk < nblocks; ++blk) {
          const int phys = block_table[b * bt_stride + blk];
          if (phys < 0 || phys >= num_pool_blocks) {
#pragma omp atomic write
            fail = 3;
            break;
          }
          float bmax = -INFINITY;
          for (int s = 0; s < block_size; ++s) {
            float x = -INFINITY;
            if (blk * block_size + s < ntok) {
              const uint16_t* kr = k_cache + ((int64_t)phys * block_size + s) * slot_stride + kvh * D;
              float dot = 0.f;
              for (int d = 0; d < D; ++d) dot += qv[d] * h2f(kr[d]);
              x = dot * sm_scale;
            }
            sc[s] = x;
            bmax = x > bmax ? x : bmax;
          }
          const float m_new = m_i > bmax ? m_i : bmax;
          const float alpha = expf(m_i - m_new);
          float psum = 0.f;
          for (int s = 0; s < block_size; ++s) {
            sc[s] = expf(sc[s] - m_new);
            psum += sc[s];
          }
          l_i = l_i * alpha + psum;
          for (int d = 0; d < D; ++d) acc[d] *= alpha;
          for (int s = 0; s < block_size; ++s) {
            if (blk * block_size + s >= ntok) continue;
            const uint16_t* vr = v_cache + ((int64_t)phys * block_size + s) * slot_stride + kvh * D;
            const float p = sc[s];
            for (int d = 0; d < D; ++d) acc[d] += p * h2f(vr[d]);
          }
          m_i = m_new;
        }
        for (int d = 0; d < D; ++d) oh[d] = f2h(acc[d] / l_i);
      }
    }
    free(qv); free(acc); free(sc);
  }
  return fail;
}

/* fp16 <-> fp32 round trip helpers exposed for the oracle's own tests. */
void oracle_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f2h(x[i]);
}
void oracle_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = h2f(x[i]);
}
