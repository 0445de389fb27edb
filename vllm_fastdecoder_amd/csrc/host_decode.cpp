// Host-core partial decode attention over the host tier: the co-processing
// leg of the split step. The reference computes the whole host-tier partial
// on the host cores (fastdecode/csrc/cpu_attn.cpp:298-411, called at
// fastdecode/backend.py:343-351); here the GPU can also read that memory
// zero-copy, but the PCIe link (~56 GB/s) is slower than the host cores
// reading their own DRAM, so the fastest split step gives part of every row's
// host blocks to the cores and the rest to the GPU, runs both at once and
// merges the partials on the GPU.
//
// Same semantics and layouts as fd_paged_decode_partial: for every sequence i
// and query head h, the softmax-weighted sum of V over the lens[i] tokens of
// blocks block_table[i, 0 ..), natural-log LSE; lens <= 0 -> out 0, lse -inf;
// a length past the table or a block id outside the cache -> NaN row.
//
// Design: one work item per (sequence, kv head), handed out longest row first
// from an atomic counter to a persistent thread pool. Per block one online
// softmax step in fp32 for the item's query heads: the block's scores, one
// max / rescale per head, then P.V with the rescale folded into the
// accumulator load. AVX2 FMAs with enough independent accumulator chains per
// head group to cover the FMA latency, F16C / shift conversions of fp16 /
// bf16 rows, and exp2 from a degree-6 polynomial for 2^f on [-0.5, 0.5]
// (least-squares fit on Chebyshev nodes, relative error < 1e-7 in fp32) times
// 2^n assembled in the exponent field. The vector code is compiled for
// AVX2+FMA+F16C and entered only after a run-time check of the CPU.
#include <immintrin.h>
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/fdattn.h"
#include "fd_errors.h"

namespace fd {
namespace {

// ---------------------------------------------------------------- pool
// A persistent pool: run(n, f) calls f(w) for w = 0 .. n-1 on n threads (the
// caller is worker 0) and returns when all of them have returned.
class Pool {
 public:
  void run(int n, const std::function<void(int)>& f) {
    std::unique_lock<std::mutex> lk(mu_);
    grow(n - 1);
    job_ = &f;
    want_ = n - 1;
    active_ = n - 1;
    ++gen_;
    lk.unlock();
    cv_.notify_all();
    f(0);
    lk.lock();
    done_.wait(lk, [&] { return active_ == 0; });
    job_ = nullptr;
  }

  ~Pool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : threads_) t.join();
  }

 private:
  void grow(int want) {  // mu_ held
    while ((int)threads_.size() < want) {
      const int id = (int)threads_.size() + 1;
      threads_.emplace_back([this, id] { loop(id); });
    }
  }

  void loop(int id) {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      cv_.wait(lk, [&] { return stop_ || (gen_ != seen && job_ != nullptr); });
      if (stop_) return;
      seen = gen_;
      if (id > want_) continue;  // not part of this run
      const std::function<void(int)>* f = job_;
      lk.unlock();
      (*f)(id);
      lk.lock();
      if (--active_ == 0) done_.notify_one();
    }
  }

  std::mutex mu_;
  std::condition_variable cv_, done_;
  std::vector<std::thread> threads_;
  const std::function<void(int)>* job_ = nullptr;
  uint64_t gen_ = 0;
  int want_ = 0, active_ = 0;
  bool stop_ = false;
};

Pool& pool() {
  static Pool p;
  return p;
}

std::mutex g_call_mu;  // the pool serves one call at a time

struct HostArgs {
  const void* q;
  int64_t q_ss, q_sh;
  const void* k;
  const void* v;
  int64_t sb, sh, st, num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
  int32_t n, H, KVH, D, BS;
  float scale;
  int32_t dt;
  void* out;
  int64_t out_ss, out_sh;
  int32_t out_dt;
  float* lse;
  int64_t lse_sh;
};

// ---------------------------------------------------------------- scalar
float f16_to_f32(uint16_t h) {  // exact, portable
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  uint32_t u;
  if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    u = s | ((e + 112) << 23) | (m << 13);
  } else if (m == 0) {
    u = s;
  } else {  // subnormal: m * 2^-24
    float f = std::ldexp((float)m, -24);
    memcpy(&u, &f, 4);
    u |= s;
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float load1(const void* p, int64_t i, int dt) {
  if (dt == FD_F32) return static_cast<const float*>(p)[i];
  const uint16_t w = static_cast<const uint16_t*>(p)[i];
  if (dt == FD_F16) return f16_to_f32(w);
  const uint32_t u = (uint32_t)w << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------- vector
#pragma GCC push_options
#pragma GCC target("avx2,fma,f16c")

inline __m256 exp2_ps(__m256 x) {
  const __m256 lo = _mm256_set1_ps(-126.f);
  const __m256 tiny = _mm256_cmp_ps(x, lo, _CMP_LT_OQ);  // includes -inf
  // operand order keeps a NaN input NaN (min/max return the second operand)
  x = _mm256_max_ps(lo, _mm256_min_ps(_mm256_set1_ps(127.f), x));
  const __m256 n = _mm256_round_ps(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m256 f = _mm256_sub_ps(x, n);
  __m256 p = _mm256_set1_ps(1.533757683e-04f);
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(1.339986036e-03f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(9.618519534e-03f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(5.550328998e-02f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(2.402264661e-01f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(6.931472056e-01f));
  p = _mm256_fmadd_ps(p, f, _mm256_set1_ps(1.000000001e+00f));
  const __m256i e = _mm256_slli_epi32(_mm256_cvtps_epi32(n), 23);
  const __m256 r = _mm256_castsi256_ps(_mm256_add_epi32(_mm256_castps_si256(p), e));
  return _mm256_andnot_ps(tiny, r);
}

inline float exp2_1(float x) { return _mm256_cvtss_f32(exp2_ps(_mm256_set1_ps(x))); }

inline float hsum(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
  return _mm_cvtss_f32(s);
}

// 8 consecutive elements of storage type DT as fp32
template <int DT>
inline __m256 ld8(const void* p) {
  if constexpr (DT == FD_F32) {
    return _mm256_loadu_ps(static_cast<const float*>(p));
  } else if constexpr (DT == FD_F16) {
    return _mm256_cvtph_ps(_mm_loadu_si128(static_cast<const __m128i*>(p)));
  } else {
    const __m256i w = _mm256_cvtepu16_epi32(_mm_loadu_si128(static_cast<const __m128i*>(p)));
    return _mm256_castsi256_ps(_mm256_slli_epi32(w, 16));
  }
}

// Scratch of one worker.
struct Scratch {
  std::vector<float> q, acc, s;
};

// Online-softmax partial of query heads kh*Gr + g0 .. + G-1 (Gr = H / KVH) of
// sequence i over kv head kh. Returns false if the row is invalid (a length
// past its table or a block id outside the cache).
template <int DT, int G>
bool run_heads(const HostArgs& a, int i, int kh, int g0, Scratch& w) {
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  constexpr int U = G >= 4 ? 1 : 4 / G;   // score chains per head
  constexpr int CU = G >= 8 ? 1 : 8 / G;  // P.V chunks in flight
  const int D = a.D, BS = a.BS, Gr = a.H / a.KVH;
  const int D8 = D & ~7;
  const int L = a.lens[i];
  const int nb = (L + BS - 1) / BS;
  if (nb > a.bt_width) return false;
  w.q.resize((size_t)G * D);
  w.acc.assign((size_t)G * D, 0.f);
  w.s.resize((size_t)G * BS);
  float* qf = w.q.data();
  float* acc = w.acc.data();
  float* s = w.s.data();
  const float qs = a.scale * 1.4426950408889634f;  // scores in the log2 domain
  for (int g = 0; g < G; ++g) {
    const int64_t qb = (int64_t)i * a.q_ss + (int64_t)(kh * Gr + g0 + g) * a.q_sh;
    for (int d = 0; d < D; ++d) qf[g * D + d] = load1(a.q, qb + d, a.dt) * qs;
  }
  float m[G], l[G], alpha[G];
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
  }
  const char* kbase = static_cast<const char*>(a.k);
  const char* vbase = static_cast<const char*>(a.v);
  const int32_t* row_bt = a.bt + (int64_t)i * a.bt_stride;
  for (int b = 0; b < nb; ++b) {
    const int64_t bid = row_bt[b];
    if (bid < 0 || bid >= a.num_blocks) return false;
    const int ntok = std::min(BS, L - b * BS);
    const int64_t base = bid * a.sb + (int64_t)kh * a.sh;
    if (b + 1 < nb) {  // the next block's rows, while this one computes
      const int64_t nid = row_bt[b + 1];
      if (nid >= 0 && nid < a.num_blocks) {
        const int64_t nbase = nid * a.sb + (int64_t)kh * a.sh;
        for (int t = 0; t < BS; ++t)
          for (int off = 0; off < D * elt; off += 64) {
            _mm_prefetch(kbase + (nbase + (int64_t)t * a.st) * elt + off, _MM_HINT_T0);
            _mm_prefetch(vbase + (nbase + (int64_t)t * a.st) * elt + off, _MM_HINT_T0);
          }
      }
    }
    // scores
    for (int t = 0; t < ntok; ++t) {
      const char* kp = kbase + (base + (int64_t)t * a.st) * elt;
      __m256 c[G][U];
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < U; ++u) c[g][u] = _mm256_setzero_ps();
      int d = 0;
      for (; d + 8 * U <= D8; d += 8 * U)
        for (int u = 0; u < U; ++u) {
          const __m256 kv = ld8<DT>(kp + (d + 8 * u) * elt);
          for (int g = 0; g < G; ++g)
            c[g][u] = _mm256_fmadd_ps(_mm256_loadu_ps(qf + g * D + d + 8 * u), kv, c[g][u]);
        }
      for (; d < D8; d += 8) {
        const __m256 kv = ld8<DT>(kp + d * elt);
        for (int g = 0; g < G; ++g)
          c[g][0] = _mm256_fmadd_ps(_mm256_loadu_ps(qf + g * D + d), kv, c[g][0]);
      }
      for (int g = 0; g < G; ++g) {
        __m256 sum = c[g][0];
        for (int u = 1; u < U; ++u) sum = _mm256_add_ps(sum, c[g][u]);
        float sc = hsum(sum);
        for (int e = D8; e < D; ++e) sc += qf[g * D + e] * load1(kp, e, DT);
        s[g * BS + t] = sc;
      }
    }
    // one online-softmax step per head
    for (int g = 0; g < G; ++g) {
      float* sg = s + g * BS;
      float bmax = sg[0];
      for (int t = 1; t < ntok; ++t) bmax = std::max(bmax, sg[t]);
      const float mn = std::max(m[g], bmax);
      alpha[g] = m[g] == -INFINITY ? 0.f : exp2_1(m[g] - mn);
      const __m256 mv = _mm256_set1_ps(mn);
      __m256 ps = _mm256_setzero_ps();
      int t = 0;
      for (; t + 8 <= ntok; t += 8) {
        const __m256 p = exp2_ps(_mm256_sub_ps(_mm256_loadu_ps(sg + t), mv));
        _mm256_storeu_ps(sg + t, p);
        ps = _mm256_add_ps(ps, p);
      }
      float psum = hsum(ps);
      for (; t < ntok; ++t) {
        sg[t] = exp2_1(sg[t] - mn);
        psum += sg[t];
      }
      l[g] = l[g] * alpha[g] + psum;
      m[g] = mn;
    }
    // acc = acc * alpha + P.V
    const char* vb = vbase + base * elt;
    int d = 0;
    for (; d + 8 * CU <= D8; d += 8 * CU) {
      __m256 r[G][CU];
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < CU; ++u)
          r[g][u] = _mm256_mul_ps(_mm256_loadu_ps(acc + g * D + d + 8 * u), _mm256_set1_ps(alpha[g]));
      for (int t = 0; t < ntok; ++t) {
        const char* vp = vb + (int64_t)t * a.st * elt;
        for (int u = 0; u < CU; ++u) {
          const __m256 vv = ld8<DT>(vp + (d + 8 * u) * elt);
          for (int g = 0; g < G; ++g)
            r[g][u] = _mm256_fmadd_ps(_mm256_broadcast_ss(s + g * BS + t), vv, r[g][u]);
        }
      }
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < CU; ++u) _mm256_storeu_ps(acc + g * D + d + 8 * u, r[g][u]);
    }
    for (; d < D8; d += 8) {
      __m256 r[G];
      for (int g = 0; g < G; ++g)
        r[g] = _mm256_mul_ps(_mm256_loadu_ps(acc + g * D + d), _mm256_set1_ps(alpha[g]));
      for (int t = 0; t < ntok; ++t) {
        const __m256 vv = ld8<DT>(vb + ((int64_t)t * a.st + d) * elt);
        for (int g = 0; g < G; ++g)
          r[g] = _mm256_fmadd_ps(_mm256_broadcast_ss(s + g * BS + t), vv, r[g]);
      }
      for (int g = 0; g < G; ++g) _mm256_storeu_ps(acc + g * D + d, r[g]);
    }
    for (; d < D; ++d)
      for (int g = 0; g < G; ++g) {
        float x = acc[g * D + d] * alpha[g];
        for (int t = 0; t < ntok; ++t) x += s[g * BS + t] * load1(vb, (int64_t)t * a.st + d, DT);
        acc[g * D + d] = x;
      }
  }
  for (int g = 0; g < G; ++g) {
    const int h = kh * Gr + g0 + g;
    const float inv = 1.f / l[g];
    float* o = acc + g * D;
    for (int d = 0; d < D; ++d) o[d] *= inv;
    const int64_t ob = (int64_t)i * a.out_ss + (int64_t)h * a.out_sh;
    if (a.out_dt == FD_F32) {
      memcpy(static_cast<float*>(a.out) + ob, o, (size_t)D * 4);
    } else if (a.out_dt == FD_F16) {
      uint16_t* dst = static_cast<uint16_t*>(a.out) + ob;
      int d = 0;
      for (; d + 8 <= D; d += 8)
        _mm_storeu_si128(reinterpret_cast<__m128i*>(dst + d),
                         _mm256_cvtps_ph(_mm256_loadu_ps(o + d), _MM_FROUND_TO_NEAREST_INT));
      for (; d < D; ++d) dst[d] = _cvtss_sh(o[d], _MM_FROUND_TO_NEAREST_INT);
    } else {
      uint16_t* dst = static_cast<uint16_t*>(a.out) + ob;
      for (int d = 0; d < D; ++d) dst[d] = f32_to_bf16(o[d]);
    }
    a.lse[(int64_t)h * a.lse_sh + i] = (m[g] + std::log2(l[g])) * 0.6931471805599453f;
  }
  return true;
}

template <int DT>
bool run_heads_dt(const HostArgs& a, int i, int kh, int g0, int G, Scratch& w) {
  switch (G) {
    case 1: return run_heads<DT, 1>(a, i, kh, g0, w);
    case 2: return run_heads<DT, 2>(a, i, kh, g0, w);
    case 4: return run_heads<DT, 4>(a, i, kh, g0, w);
    default: return run_heads<DT, 8>(a, i, kh, g0, w);
  }
}

#pragma GCC pop_options

// Fills every query head of kv head kh of sequence i with (x, lse); x is 0
// or NaN.
void fill_item(const HostArgs& a, int i, int kh, float x, float lse) {
  const int Gr = a.H / a.KVH;
  for (int g = 0; g < Gr; ++g) {
    const int h = kh * Gr + g;
    const int64_t ob = (int64_t)i * a.out_ss + (int64_t)h * a.out_sh;
    for (int d = 0; d < a.D; ++d) {
      if (a.out_dt == FD_F32) {
        static_cast<float*>(a.out)[ob + d] = x;
      } else {  // 0, or the quiet NaN of the 16-bit format
        static_cast<uint16_t*>(a.out)[ob + d] =
            x == 0.f ? 0 : (a.out_dt == FD_F16 ? 0x7e00 : 0x7fc0);
      }
    }
    a.lse[(int64_t)h * a.lse_sh + i] = lse;
  }
}

// All query heads of (sequence i, kv head kh), in passes of at most 8 heads.
void run_item(const HostArgs& a, int i, int kh, Scratch& w) {
  if (a.lens[i] <= 0) return fill_item(a, i, kh, 0.f, -INFINITY);
  const int Gr = a.H / a.KVH;
  for (int g0 = 0; g0 < Gr;) {
    const int rest = Gr - g0;
    const int G = rest >= 8 ? 8 : rest >= 4 ? 4 : rest >= 2 ? 2 : 1;
    bool ok;
    if (a.dt == FD_F16) {
      ok = run_heads_dt<FD_F16>(a, i, kh, g0, G, w);
    } else if (a.dt == FD_BF16) {
      ok = run_heads_dt<FD_BF16>(a, i, kh, g0, G, w);
    } else {
      ok = run_heads_dt<FD_F32>(a, i, kh, g0, G, w);
    }
    if (!ok) return fill_item(a, i, kh, NAN, NAN);
    g0 += G;
  }
}

int default_threads() {
  const char* e = getenv("FASTDECODE_CPU_THREADS");
  if (e != nullptr && atoi(e) > 0) return atoi(e);
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) return std::max(1, CPU_COUNT(&set));
  return std::max(1u, std::thread::hardware_concurrency());
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" int fd_host_decode_threads(void) { return default_threads(); }

extern "C" int fd_host_decode_partial(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype, void* out, int64_t out_stride_seq,
    int64_t out_stride_head, int32_t out_dtype, float* lse, int64_t lse_stride_head,
    int32_t num_threads) {
  if (n < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_size <= 0 || head_size > 1024 || block_size <= 0 || block_size > 1024 ||
      bt_width < 0 || num_blocks < 0 || num_threads < 0)
    return set_error(FD_ERR_INVALID, "fd_host_decode_partial: bad sizes");
  if (kv_dtype != FD_F16 && kv_dtype != FD_BF16 && kv_dtype != FD_F32)
    return set_error(FD_ERR_INVALID, "fd_host_decode_partial: unsupported kv dtype %d", kv_dtype);
  if (out_dtype != kv_dtype && out_dtype != FD_F32)
    return set_error(FD_ERR_INVALID,
                     "fd_host_decode_partial: out dtype must be the kv dtype or fp32");
  if (!std::isfinite(scale))
    return set_error(FD_ERR_INVALID, "fd_host_decode_partial: scale is not finite");
  if (n == 0) return FD_OK;
  if (!q || !k_cache || !v_cache || !block_table || !lens || !out || !lse)
    return set_error(FD_ERR_INVALID, "fd_host_decode_partial: NULL pointer");
  if (bt_width > 0 && bt_stride < bt_width)
    return set_error(FD_ERR_INVALID, "fd_host_decode_partial: bt_stride < bt_width");
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma") ||
      !__builtin_cpu_supports("f16c"))
    return set_error(FD_ERR_UNSUPPORTED, "fd_host_decode_partial: the CPU lacks AVX2/FMA/F16C");
  const HostArgs a{q, q_stride_seq, q_stride_head, k_cache, v_cache, kv_stride_block,
                   kv_stride_head, kv_stride_token, num_blocks, block_table, bt_stride, bt_width,
                   lens, n, num_heads, num_kv_heads, head_size, block_size, scale, kv_dtype, out,
                   out_stride_seq, out_stride_head, out_dtype, lse, lse_stride_head};
  // work items (sequence, kv head), longest sequences first
  std::vector<int32_t> rows(n);
  for (int i = 0; i < n; ++i) rows[i] = i;
  std::stable_sort(rows.begin(), rows.end(), [&](int x, int y) { return lens[x] > lens[y]; });
  const int64_t items = (int64_t)n * num_kv_heads;
  const int nt = (int)std::max<int64_t>(
      1, std::min<int64_t>(num_threads > 0 ? num_threads : default_threads(), items));
  std::atomic<int64_t> next{0};
  std::lock_guard<std::mutex> call(g_call_mu);
  pool().run(nt, [&](int) {
    Scratch w;
    for (;;) {
      const int64_t it = next.fetch_add(1, std::memory_order_relaxed);
      if (it >= items) break;
      run_item(a, rows[it / num_kv_heads], (int)(it % num_kv_heads), w);
    }
  });
  return FD_OK;
}
