/*
 * fd_oracle.c -- CPU restatement of vllm_fastdecode's split decode-attention
 * path. TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check and the
 * CPU-baseline leg of bench.py may load it, as the checker or as the timed CPU
 * baseline; the product path never calls it and has no CPU fallback.
 *
 * Functions and the reference code each one restates:
 *
 *   oracle_decode_attn_f64     float64 closed form of the partial
 *                              (fastdecode/cpu_ops.py:54-81, ref_decode_attn),
 *                              with the layout/edge conventions of
 *                              fastdecode/csrc/cpu_attn.cpp:298-411 (only the
 *                              first ceil(len/BS) table entries are read,
 *                              len == 0 -> out 0 / lse -inf, :324-331) and a
 *                              generic (block, head, token) stride so it also
 *                              reads vLLM's [B, BS, KVH, 2D] GPU tier.
 *   oracle_decode_attn_cpu_f32 fp32 two-pass algorithm of decode_attn_impl
 *                              (cpu_attn.cpp:298-411): OpenMP dynamic schedule
 *                              over (sequence, kv head), pre-scaled q (:334-339),
 *                              score pass (:342-366), max + exp-sum (:368-374),
 *                              P.V pass (:376-400), out = acc / sum and
 *                              lse = m + log(sum) (:401-407). Used as the CPU
 *                              baseline when the reference build is absent.
 *   oracle_merge_f64           merge_partials_torch (cpu_ops.py:93-113).
 *   oracle_cache_write         store_kv_impl (cpu_attn.cpp:413-431) with the
 *                              range check before any write (:506-510), and the
 *                              reshape_and_cache stand-in that skips slot < 0
 *                              (tests/test_plan_and_forward.py:88-95).
 *
 * Element types: 0 = fp16, 1 = bf16, 2 = fp32 (as the reference's dispatch,
 * cpu_attn.cpp:439-448). All strides are in elements.
 *
 * Pinning: see tests/test_oracle.py (reference build outputs, closed forms,
 * brute-force and invariant checks).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary16 -> binary32 (exact). */
static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

static float bf16_to_float(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

static inline float load_f(const void* p, int64_t i, int dt) {
  if (dt == 2) return ((const float*)p)[i];
  const uint16_t w = ((const uint16_t*)p)[i];
  return dt == 0 ? half_to_float(w) : bf16_to_float(w);
}

/* Merge inputs may also be float64 (dt 3): the oracle's own partials. */
static inline double load_d(const void* p, int64_t i, int dt) {
  if (dt == 3) return ((const double*)p)[i];
  return (double)load_f(p, i, dt);
}

int oracle_elem_size(int dt) { return dt == 3 ? 8 : dt == 2 ? 4 : 2; }

/* Converts n elements of dtype dt to float (helper for tests). */
void oracle_to_float(const void* src, int dt, int64_t n, float* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = load_f(src, i, dt);
}

/* Returns 0, or 2 when a needed table entry is outside [0, num_blocks) or a
 * length exceeds the table (the rows concerned are left NaN). */
int oracle_decode_attn_f64(const void* q, int64_t q_ss, int64_t q_sh, const void* k,
                           const void* v, int64_t sb, int64_t sh, int64_t st,
                           int64_t num_blocks, const int32_t* bt, int64_t bt_stride,
                           int32_t bt_width, const int32_t* lens, int n, int H, int KVH,
                           int D, int BS, double scale, int dt, double* out, double* lse,
                           int nthreads) {
  const int G = H / KVH;
  int status = 0;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads) reduction(| : status)
#endif
  for (int64_t task = 0; task < (int64_t)n * H; ++task) {
    const int i = (int)(task / H);
    const int h = (int)(task % H);
    const int kh = h / G;
    double* o = out + ((int64_t)i * H + h) * D;
    const int L = lens[i];
    if (L <= 0) {
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      lse[(int64_t)h * n + i] = -INFINITY;
      continue;
    }
    const int nb = (L + BS - 1) / BS;
    int bad = nb > bt_width;
    for (int b = 0; b < nb && !bad; ++b) {
      const int32_t id = bt[(int64_t)i * bt_stride + b];
      bad = id < 0 || id >= num_blocks;
    }
    if (bad) {
      for (int d = 0; d < D; ++d) o[d] = NAN;
      lse[(int64_t)h * n + i] = NAN;
      status |= 2;
      continue;
    }
    double* s = (double*)malloc(sizeof(double) * (size_t)L);
    double* qd = (double*)malloc(sizeof(double) * (size_t)D);
    for (int d = 0; d < D; ++d) qd[d] = load_f(q, (int64_t)i * q_ss + (int64_t)h * q_sh + d, dt);
    double m = -INFINITY;
    for (int t = 0; t < L; ++t) {
      const int64_t id = bt[(int64_t)i * bt_stride + t / BS];
      const int64_t base = id * sb + (int64_t)kh * sh + (int64_t)(t % BS) * st;
      double acc = 0.0;
      for (int d = 0; d < D; ++d) acc += qd[d] * (double)load_f(k, base + d, dt);
      s[t] = acc * scale;
      if (s[t] > m) m = s[t];
    }
    double sum = 0.0;
    for (int t = 0; t < L; ++t) {
      s[t] = exp(s[t] - m);
      sum += s[t];
    }
    for (int d = 0; d < D; ++d) o[d] = 0.0;
    for (int t = 0; t < L; ++t) {
      const int64_t id = bt[(int64_t)i * bt_stride + t / BS];
      const int64_t base = id * sb + (int64_t)kh * sh + (int64_t)(t % BS) * st;
      const double p = s[t] / sum;
      for (int d = 0; d < D; ++d) o[d] += p * (double)load_f(v, base + d, dt);
    }
    lse[(int64_t)h * n + i] = m + log(sum);
    free(s);
    free(qd);
  }
  return status;
}

/* fp32 two-pass restatement of decode_attn_impl for the host-tier layout
 * [C, KVH, BS, D] (contiguous). out is float [n, H, D], lse float [H, n]. */
void oracle_decode_attn_cpu_f32(const void* q, const void* kc, const void* vc,
                                const int32_t* bt, const int32_t* lens, int n, int H, int KVH,
                                int D, int BS, int W, float scale, int dt, float* out,
                                float* lse, int nthreads) {
  const int G = H / KVH;
  const int64_t head_stride = (int64_t)BS * D;
  const int64_t blk_stride = (int64_t)KVH * head_stride;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float* qf = (float*)malloc(sizeof(float) * (size_t)G * D);
    float* rowf = (float*)malloc(sizeof(float) * (size_t)D);
    float* acc = (float*)malloc(sizeof(float) * (size_t)G * D);
    float* mx = (float*)malloc(sizeof(float) * (size_t)G);
    float* sm = (float*)malloc(sizeof(float) * (size_t)G);
    float* scores = NULL;
    size_t cap = 0;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1) collapse(2)
#endif
    for (int i = 0; i < n; ++i) {
      for (int kh = 0; kh < KVH; ++kh) {
        const int len = lens[i];
        if (len <= 0) {
          for (int g = 0; g < G; ++g) {
            const int h = kh * G + g;
            for (int d = 0; d < D; ++d) out[((int64_t)i * H + h) * D + d] = 0.f;
            lse[(int64_t)h * n + i] = -INFINITY;
          }
          continue;
        }
        if ((size_t)G * len > cap) {
          cap = (size_t)G * len;
          scores = (float*)realloc(scores, sizeof(float) * cap);
        }
        for (int g = 0; g < G; ++g) {
          const int h = kh * G + g;
          for (int d = 0; d < D; ++d)
            qf[g * D + d] = load_f(q, ((int64_t)i * H + h) * D + d, dt) * scale;
        }
        /* pass 1: scores */
        for (int t = 0; t < len; ++t) {
          const int64_t blk = bt[(int64_t)i * W + t / BS];
          const int64_t base = blk * blk_stride + kh * head_stride + (int64_t)(t % BS) * D;
          for (int d = 0; d < D; ++d) rowf[d] = load_f(kc, base + d, dt);
          for (int g = 0; g < G; ++g) {
            float a = 0.f;
            const float* qg = qf + g * D;
            for (int d = 0; d < D; ++d) a += qg[d] * rowf[d];
            scores[(size_t)g * len + t] = a;
          }
        }
        /* softmax numerators */
        for (int g = 0; g < G; ++g) {
          float* sg = scores + (size_t)g * len;
          float m = -INFINITY;
          for (int t = 0; t < len; ++t) m = sg[t] > m ? sg[t] : m;
          float s = 0.f;
          for (int t = 0; t < len; ++t) {
            sg[t] = expf(sg[t] - m);
            s += sg[t];
          }
          mx[g] = m;
          sm[g] = s;
        }
        /* pass 2: acc = p . v */
        memset(acc, 0, sizeof(float) * (size_t)G * D);
        for (int t = 0; t < len; ++t) {
          const int64_t blk = bt[(int64_t)i * W + t / BS];
          const int64_t base = blk * blk_stride + kh * head_stride + (int64_t)(t % BS) * D;
          for (int d = 0; d < D; ++d) rowf[d] = load_f(vc, base + d, dt);
          for (int g = 0; g < G; ++g) {
            const float p = scores[(size_t)g * len + t];
            float* ag = acc + g * D;
            for (int d = 0; d < D; ++d) ag[d] += p * rowf[d];
          }
        }
        for (int g = 0; g < G; ++g) {
          const int h = kh * G + g;
          const float inv = 1.f / sm[g];
          for (int d = 0; d < D; ++d) out[((int64_t)i * H + h) * D + d] = acc[g * D + d] * inv;
          lse[(int64_t)h * n + i] = mx[g] + logf(sm[g]);
        }
      }
    }
    free(qf);
    free(rowf);
    free(acc);
    free(mx);
    free(sm);
    free(scores);
  }
}

/* out[i,h,:] = o_a * w_a + o_b * w_b in float64 with the torch rule:
 * +inf lse -> -inf; both empty -> m = 0, weights' sum = 1 (out = 0).
 * o_* [n, H, D] contiguous of dtype a_dt / b_dt (fp16, bf16, fp32 or
 * float64); lse_* float64 [H, n]. */
void oracle_merge_f64(const void* o_a, int a_dt, const double* lse_a, const void* o_b, int b_dt,
                      const double* lse_b, int n, int H, int D, double* out, double* out_lse) {
  for (int i = 0; i < n; ++i) {
    for (int h = 0; h < H; ++h) {
      double la = lse_a[(int64_t)h * n + i], lb = lse_b[(int64_t)h * n + i];
      if (la == INFINITY) la = -INFINITY;
      if (lb == INFINITY) lb = -INFINITY;
      double m = la > lb ? la : lb;
      const int both_empty = m == -INFINITY;
      if (both_empty) m = 0.0;
      const double wa0 = exp(la - m), wb0 = exp(lb - m);
      const double tot = both_empty ? 1.0 : wa0 + wb0;
      const double wa = wa0 / tot, wb = wb0 / tot;
      const int64_t base = ((int64_t)i * H + h) * D;
      for (int d = 0; d < D; ++d)
        out[base + d] = load_d(o_a, base + d, a_dt) * wa + load_d(o_b, base + d, b_dt) * wb;
      if (out_lse) out_lse[(int64_t)h * n + i] = both_empty ? -INFINITY : m + log(tot);
    }
  }
}

/* Slot-mapping write. key/value rows at j*key_st + g*key_sh (elements);
 * cache element offset of (block b, token t, head g) is
 * b*c_sb + t*c_st + g*c_sh. check_all != 0: store_kv semantics -- every
 * slot must be in [0, capacity) or nothing is written and 2 is returned.
 * check_all == 0: reshape_and_cache semantics -- slots < 0 and slots past
 * the cache are skipped; the latter are counted into *n_out_of_range. */
int oracle_cache_write(const void* key, int64_t key_st, int64_t key_sh, const void* value,
                       int64_t value_st, int64_t value_sh, void* kc, void* vc, int64_t c_sb,
                       int64_t c_st, int64_t c_sh, int64_t num_blocks, const int64_t* slots,
                       int T, int KVH, int D, int BS, int elt, int check_all,
                       int64_t* n_out_of_range) {
  const int64_t cap = num_blocks * BS;
  if (check_all) {
    for (int j = 0; j < T; ++j)
      if (slots[j] < 0 || slots[j] >= cap) return 2;
  }
  int64_t oor = 0;
  for (int j = 0; j < T; ++j) {
    const int64_t s = slots[j];
    if (s < 0) continue;
    if (s >= cap) {
      ++oor;
      continue;
    }
    const int64_t blk = s / BS, off = s % BS;
    for (int g = 0; g < KVH; ++g) {
      const int64_t dst = (blk * c_sb + off * c_st + (int64_t)g * c_sh) * elt;
      memcpy((char*)kc + dst, (const char*)key + ((int64_t)j * key_st + (int64_t)g * key_sh) * elt,
             (size_t)D * elt);
      memcpy((char*)vc + dst,
             (const char*)value + ((int64_t)j * value_st + (int64_t)g * value_sh) * elt,
             (size_t)D * elt);
    }
  }
  if (n_out_of_range) *n_out_of_range = oor;
  return 0;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
