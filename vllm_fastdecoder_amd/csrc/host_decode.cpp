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
// Design: one work item per (sequence, group of adjacent kv heads), handed
// out longest row first from an atomic counter to a persistent thread pool;
// an item walks its row's blocks and, inside each block, its kv heads, whose
// runs lie side by side in the host tier, so each block is streamed in one
// piece of up to KVH * BS * D elements. Per (block, kv head) one online
// softmax step in fp32 for that head's query heads: the block's scores, one
// max / rescale per head, then P.V with the rescale folded into the
// accumulator load. Vector FMAs with enough independent accumulator chains
// per head group to cover the FMA latency, F16C / shift conversions of fp16 /
// bf16 rows, and exp2 from a degree-6 polynomial for 2^f on [-0.5, 0.5]
// (least-squares fit on Chebyshev nodes, relative error < 1e-7 in fp32) times
// 2^n assembled in the exponent field. One kernel body
// (host_decode_kernel.h) is compiled for AVX-512 with bf16 pair dot products
// (bf16 KV scores by vdpbf16ps on the raw q and K rows, the scale applied to
// the dot), plain AVX-512 (16 lanes) and AVX2 (8 lanes); the widest one the
// CPU supports is picked at run time, and the rest of the library is built
// for baseline x86-64.
#include <immintrin.h>
#include <sched.h>
#include <unistd.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <exception>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/fdattn.h"
#include "fd_errors.h"
#include "host_decode.h"

namespace fd {
namespace {

// ---------------------------------------------------------------- pool
// A persistent pool: run(n, f) calls f(w) for w = 0 .. n-1 on n threads (the
// caller is worker 0) and returns when all of them have returned. The first
// exception any of them throws (no memory for its scratch, say) is rethrown
// on the caller's thread once all have returned.
class Pool {
 public:
  void run(int n, const std::function<void(int)>& f) {
    std::unique_lock<std::mutex> lk(mu_);
    grow(n - 1);
    job_ = &f;
    want_ = n - 1;
    active_ = n - 1;
    error_ = nullptr;
    ++gen_;
    lk.unlock();
    cv_.notify_all();
    std::exception_ptr mine;
    try {
      f(0);
    } catch (...) {
      mine = std::current_exception();
    }
    lk.lock();
    done_.wait(lk, [&] { return active_ == 0; });
    job_ = nullptr;
    std::exception_ptr e = mine ? mine : error_;
    error_ = nullptr;
    lk.unlock();
    if (e) std::rethrow_exception(e);
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
      std::exception_ptr e;
      try {
        (*f)(id);
      } catch (...) {
        e = std::current_exception();
      }
      lk.lock();
      if (e && !error_) error_ = e;
      if (--active_ == 0) done_.notify_one();
    }
  }

  std::mutex mu_;
  std::condition_variable cv_, done_;
  std::vector<std::thread> threads_;
  const std::function<void(int)>* job_ = nullptr;
  std::exception_ptr error_;  // the first exception of a worker in the current run
  uint64_t gen_ = 0;
  int want_ = 0, active_ = 0;
  bool stop_ = false;
};

// The pool and the lock that serialises calls on it, per process: a child
// forked from a process that used them gets new ones (the parent's worker
// threads do not exist in the child, and the lock may have been held at the
// fork). The parent's objects are left alone in the child, never destroyed.
struct PoolState {
  pid_t pid;
  Pool pool;
  std::mutex call_mu;
  explicit PoolState(pid_t p) : pid(p) {}
};

PoolState& pool_state() {
  static std::atomic<PoolState*> state{nullptr};
  static std::mutex create_mu;  // taken only to create the state of a process
  const pid_t me = getpid();
  PoolState* st = state.load(std::memory_order_acquire);
  if (st != nullptr && st->pid == me) return *st;
  std::lock_guard<std::mutex> lk(create_mu);
  st = state.load(std::memory_order_acquire);
  if (st == nullptr || st->pid != me) {
    st = new PoolState(me);  // intentionally never freed (lives for the process)
    state.store(st, std::memory_order_release);
  }
  return *st;
}

// How many (block, kv head) runs past the one being reduced the host-core
// kernel prefetches (spread over that run's score loop).
constexpr int kAheadRuns = 1;

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

// Scratch of one worker.
struct Scratch {
  std::vector<float> q, acc, s, m, l;
  std::vector<uint16_t> qh;
};

// exp2 for x <= 127: 2^x = 2^n * 2^f with n = round(x), |f| <= 1/2, 2^f from
// the polynomial below, 2^n added into the exponent field; x < -126
// (including -inf) gives 0 and NaN stays NaN (operand order of min/max).
#define FD_EXP2_POLY(fma, set1, f)                        \
  fma(fma(fma(fma(fma(fma(set1(1.533757683e-04f), f,      \
                          set1(1.339986036e-03f)), f,     \
                      set1(9.618519534e-03f)), f,         \
                  set1(5.550328998e-02f)), f,             \
              set1(2.402264661e-01f)), f,                 \
          set1(6.931472056e-01f)), f,                     \
      set1(1.000000001e+00f))

// ---------------------------------------------------------------- AVX2
#pragma GCC push_options
#pragma GCC target("avx2,fma,f16c")
namespace isa_avx2 {

struct V {
  using T = __m256;
  static constexpr int W = 8;
  static constexpr int kAcc = 8;  // P.V accumulators kept live (16 registers)
  static constexpr bool kBf16Dot = false;
  static __m256i ld_bf16x32(const void*) { return _mm256_setzero_si256(); }  // unused
  static T dot_bf16(T c, __m256i, __m256i) { return c; }                     // unused
  static T zero() { return _mm256_setzero_ps(); }
  static T set1(float x) { return _mm256_set1_ps(x); }
  static T load(const float* p) { return _mm256_loadu_ps(p); }
  static void store(float* p, T x) { _mm256_storeu_ps(p, x); }
  static T bcast(const float* p) { return _mm256_broadcast_ss(p); }
  static T add(T a, T b) { return _mm256_add_ps(a, b); }
  static T sub(T a, T b) { return _mm256_sub_ps(a, b); }
  static T mul(T a, T b) { return _mm256_mul_ps(a, b); }
  static T max(T a, T b) { return _mm256_max_ps(a, b); }
  // 2W bf16 at p as fp32: even-indexed elements in `ev`, odd in `od`
  static void ld_bf16_eo(const void* p, T& ev, T& od) {
    const __m256i x = _mm256_loadu_si256(static_cast<const __m256i*>(p));
    ev = _mm256_castsi256_ps(_mm256_slli_epi32(x, 16));
    od = _mm256_castsi256_ps(_mm256_and_si256(x, _mm256_set1_epi32((int)0xFFFF0000u)));
  }
  static float hmax(T v) {
    __m128 x = _mm_max_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    x = _mm_max_ps(x, _mm_movehl_ps(x, x));
    x = _mm_max_ss(x, _mm_shuffle_ps(x, x, 0x55));
    return _mm_cvtss_f32(x);
  }
  static T fma(T a, T b, T c) { return _mm256_fmadd_ps(a, b, c); }
  // o[0..3] = horizontal sums of a, b, c, d
  static void hsum4(T a, T b, T c, T d, float* o) {
    const T ab = _mm256_add_ps(_mm256_unpacklo_ps(a, b), _mm256_unpackhi_ps(a, b));
    const T cd = _mm256_add_ps(_mm256_unpacklo_ps(c, d), _mm256_unpackhi_ps(c, d));
    const T s = _mm256_add_ps(_mm256_shuffle_ps(ab, cd, 0x44), _mm256_shuffle_ps(ab, cd, 0xEE));
    _mm_storeu_ps(o, _mm_add_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1)));
  }
  static float hsum(T v) {
    __m128 x = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    x = _mm_add_ps(x, _mm_movehl_ps(x, x));
    x = _mm_add_ss(x, _mm_shuffle_ps(x, x, 0x55));
    return _mm_cvtss_f32(x);
  }
  static T exp2(T x) {
    const T lo = set1(-126.f);
    const T tiny = _mm256_cmp_ps(x, lo, _CMP_LT_OQ);
    x = _mm256_max_ps(lo, _mm256_min_ps(set1(127.f), x));
    const T n = _mm256_round_ps(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    const T f = sub(x, n);
    const T p = FD_EXP2_POLY(fma, set1, f);
    const __m256i e = _mm256_slli_epi32(_mm256_cvtps_epi32(n), 23);
    return _mm256_andnot_ps(tiny, _mm256_castsi256_ps(_mm256_add_epi32(_mm256_castps_si256(p), e)));
  }
  static float exp2_1(float x) { return _mm256_cvtss_f32(exp2(set1(x))); }
  template <int DT>
  static T ld(const void* p) {  // 8 storage elements -> fp32
    if constexpr (DT == FD_F32) {
      return _mm256_loadu_ps(static_cast<const float*>(p));
    } else if constexpr (DT == FD_F16) {
      return _mm256_cvtph_ps(_mm_loadu_si128(static_cast<const __m128i*>(p)));
    } else {
      const __m256i w = _mm256_cvtepu16_epi32(_mm_loadu_si128(static_cast<const __m128i*>(p)));
      return _mm256_castsi256_ps(_mm256_slli_epi32(w, 16));
    }
  }
};

#include "host_decode_kernel.h"

}  // namespace isa_avx2
#pragma GCC pop_options

// ---------------------------------------------------------------- AVX-512
#pragma GCC push_options
#pragma GCC target("avx512f,avx2,fma,f16c")
namespace isa_avx512 {

struct V512 {
  using T = __m512;
  static constexpr int W = 16;
  static constexpr int kAcc = 16;  // P.V accumulators kept live (32 registers)
  static constexpr bool kBf16Dot = false;
  static __m512i ld_bf16x32(const void*) { return _mm512_setzero_si512(); }  // unused
  static T dot_bf16(T c, __m512i, __m512i) { return c; }                     // unused
  static T zero() { return _mm512_setzero_ps(); }
  static T set1(float x) { return _mm512_set1_ps(x); }
  static T load(const float* p) { return _mm512_loadu_ps(p); }
  static void store(float* p, T x) { _mm512_storeu_ps(p, x); }
  static T bcast(const float* p) { return _mm512_set1_ps(*p); }
  static T add(T a, T b) { return _mm512_add_ps(a, b); }
  static T sub(T a, T b) { return _mm512_sub_ps(a, b); }
  static T mul(T a, T b) { return _mm512_mul_ps(a, b); }
  static T max(T a, T b) { return _mm512_max_ps(a, b); }
  // 2W bf16 at p as fp32: even-indexed elements in `ev`, odd in `od`
  static void ld_bf16_eo(const void* p, T& ev, T& od) {
    const __m512i x = _mm512_loadu_si512(p);
    ev = _mm512_castsi512_ps(_mm512_slli_epi32(x, 16));
    od = _mm512_castsi512_ps(_mm512_and_si512(x, _mm512_set1_epi32((int)0xFFFF0000u)));
  }
  static float hmax(T v) { return _mm512_reduce_max_ps(v); }
  static T fma(T a, T b, T c) { return _mm512_fmadd_ps(a, b, c); }
  // o[0..3] = horizontal sums of a, b, c, d
  static void hsum4(T a, T b, T c, T d, float* o) {
    const T ab = _mm512_add_ps(_mm512_unpacklo_ps(a, b), _mm512_unpackhi_ps(a, b));
    const T cd = _mm512_add_ps(_mm512_unpacklo_ps(c, d), _mm512_unpackhi_ps(c, d));
    const T s = _mm512_add_ps(_mm512_shuffle_ps(ab, cd, 0x44), _mm512_shuffle_ps(ab, cd, 0xEE));
    const __m256 y = _mm256_add_ps(_mm512_castps512_ps256(s),
                                   _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(s), 1)));
    _mm_storeu_ps(o, _mm_add_ps(_mm256_castps256_ps128(y), _mm256_extractf128_ps(y, 1)));
  }
  static float hsum(T v) {
    __m256 y = _mm256_add_ps(_mm512_castps512_ps256(v),
                             _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(v), 1)));
    __m128 x = _mm_add_ps(_mm256_castps256_ps128(y), _mm256_extractf128_ps(y, 1));
    x = _mm_add_ps(x, _mm_movehl_ps(x, x));
    x = _mm_add_ss(x, _mm_shuffle_ps(x, x, 0x55));
    return _mm_cvtss_f32(x);
  }
  static T exp2(T x) {
    const T lo = set1(-126.f);
    const __mmask16 keep = _mm512_cmp_ps_mask(x, lo, _CMP_NLT_UQ);  // not (x < -126)
    x = _mm512_max_ps(lo, _mm512_min_ps(set1(127.f), x));
    const T n = _mm512_roundscale_ps(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    const T f = sub(x, n);
    const T p = FD_EXP2_POLY(fma, set1, f);
    const __m512i e = _mm512_slli_epi32(_mm512_cvtps_epi32(n), 23);
    return _mm512_maskz_mov_ps(keep,
                               _mm512_castsi512_ps(_mm512_add_epi32(_mm512_castps_si512(p), e)));
  }
  static float exp2_1(float x) { return _mm512_cvtss_f32(exp2(set1(x))); }
  template <int DT>
  static T ld(const void* p) {  // 16 storage elements -> fp32
    if constexpr (DT == FD_F32) {
      return _mm512_loadu_ps(static_cast<const float*>(p));
    } else if constexpr (DT == FD_F16) {
      return _mm512_cvtph_ps(_mm256_loadu_si256(static_cast<const __m256i*>(p)));
    } else {
      const __m512i w = _mm512_cvtepu16_epi32(_mm256_loadu_si256(static_cast<const __m256i*>(p)));
      return _mm512_castsi512_ps(_mm512_slli_epi32(w, 16));
    }
  }
};

using V = V512;

#include "host_decode_kernel.h"

}  // namespace isa_avx512
#pragma GCC pop_options

// ------------------------------------------------ AVX-512 with BF16 dot products
#pragma GCC push_options
#pragma GCC target("avx512f,avx512bf16,avx2,fma,f16c")
namespace isa_avx512bf16 {

struct V : isa_avx512::V512 {
  static constexpr bool kBf16Dot = true;  // scores of bf16 KV by vdpbf16ps
  static __m512bh ld_bf16x32(const void* p) {
    return (__m512bh)_mm512_loadu_si512(p);
  }
  static T dot_bf16(T c, __m512bh a, __m512bh b) { return _mm512_dpbf16_ps(c, a, b); }
};

#include "host_decode_kernel.h"

}  // namespace isa_avx512bf16
#pragma GCC pop_options

// ------------------------------------------------ plain streaming read (measurement)
#pragma GCC push_options
#pragma GCC target("avx2")
namespace read_avx2 {

// XOR of the 64-bit words in bytes [lo, hi) of p (64-byte aligned, hi - lo a
// multiple of 64), read as four interleaved streams over its four quarters
// (each step takes 128 bytes of every stream with 32-byte loads), every line
// prefetched kAhead bytes before its load. One stream per core with the
// hardware prefetchers alone, or with a software prefetch, read the host's
// DRAM at about half its rate on some hosts (202 against 403 GB/s on 16
// cores); two to eight streams per core, or the host-core kernel's own
// pattern (K and V runs of adjacent kv heads, the next ones prefetched),
// reach it.
uint64_t xor_lines(const char* p, size_t lo, size_t hi) {
  constexpr int kStreams = 4;
  constexpr size_t kAhead = 4096;
  const size_t lines = (hi - lo) / 64;
  const size_t len = lines / kStreams * 64;  // bytes of each stream (the rest: a tail)
  __m256i acc[kStreams][2];
  for (int k = 0; k < kStreams; ++k) acc[k][0] = acc[k][1] = _mm256_setzero_si256();
  size_t o = 0;
  for (; o + 128 <= len; o += 128) {
    for (int k = 0; k < kStreams; ++k) {
      const char* q = p + lo + k * len + o;
      if (o + kAhead + 128 <= len) {
        _mm_prefetch(q + kAhead, _MM_HINT_T0);
        _mm_prefetch(q + kAhead + 64, _MM_HINT_T0);
      }
      const __m256i* v = reinterpret_cast<const __m256i*>(q);
      acc[k][0] = _mm256_xor_si256(acc[k][0], _mm256_xor_si256(_mm256_load_si256(v),
                                                                _mm256_load_si256(v + 1)));
      acc[k][1] = _mm256_xor_si256(acc[k][1], _mm256_xor_si256(_mm256_load_si256(v + 2),
                                                                _mm256_load_si256(v + 3)));
    }
  }
  __m256i x = _mm256_setzero_si256();
  for (int k = 0; k < kStreams; ++k) {
    if (o < len) {  // each stream's last 64-byte line (len an odd number of lines)
      const __m256i* v = reinterpret_cast<const __m256i*>(p + lo + k * len + o);
      x = _mm256_xor_si256(x, _mm256_xor_si256(_mm256_load_si256(v), _mm256_load_si256(v + 1)));
    }
    x = _mm256_xor_si256(x, _mm256_xor_si256(acc[k][0], acc[k][1]));
  }
  for (size_t t = lo + kStreams * len; t < hi; t += 64) {  // lines past the four streams
    const __m256i* v = reinterpret_cast<const __m256i*>(p + t);
    x = _mm256_xor_si256(x, _mm256_xor_si256(_mm256_load_si256(v), _mm256_load_si256(v + 1)));
  }
  return (uint64_t)_mm256_extract_epi64(x, 0) ^ (uint64_t)_mm256_extract_epi64(x, 1) ^
         (uint64_t)_mm256_extract_epi64(x, 2) ^ (uint64_t)_mm256_extract_epi64(x, 3);
}

}  // namespace read_avx2
#pragma GCC pop_options

// Vector width the kernel uses on this CPU: 512 (AVX-512F) or 256 (AVX2),
// 0 if neither is available. FASTDECODE_CPU_ISA=avx2 keeps to AVX2.
int isa_bits() {
  __builtin_cpu_init();
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma") ||
      !__builtin_cpu_supports("f16c"))
    return 0;
  const char* e = getenv("FASTDECODE_CPU_ISA");
  if (e != nullptr && strcmp(e, "avx2") == 0) return 256;
  return __builtin_cpu_supports("avx512f") ? 512 : 256;
}

// The AVX-512 body with bf16 pair dot products, where the CPU has them
// (FASTDECODE_CPU_ISA=avx512 keeps to plain AVX-512).
bool use_bf16_dot() {
  const char* e = getenv("FASTDECODE_CPU_ISA");
  if (e != nullptr && strcmp(e, "avx512") == 0) return false;
  return __builtin_cpu_supports("avx512bf16");
}

// Fills every query head of kv heads kh0 .. kh0 + nkh - 1 of sequence i with
// (x, lse); x is 0 or NaN.
void fill_item(const HostArgs& a, int i, int kh0, int nkh, float x, float lse) {
  const int Gr = a.H / a.KVH;
  for (int h = kh0 * Gr; h < (kh0 + nkh) * Gr; ++h) {
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

// All query heads of kv heads kh0 .. kh0 + nkh - 1 of sequence i, in passes of
// at most 8 query heads per kv head.
void run_item(const HostArgs& a, int i, int kh0, int nkh, int bits, Scratch& w) {
  if (a.lens[i] <= 0) return fill_item(a, i, kh0, nkh, 0.f, -INFINITY);
  const int Gr = a.H / a.KVH;
  for (int g0 = 0; g0 < Gr;) {
    const int rest = Gr - g0;
    const int G = rest >= 8 ? 8 : rest >= 4 ? 4 : rest >= 2 ? 2 : 1;
    const bool ok = bits == 513   ? isa_avx512bf16::run_group(a, i, kh0, nkh, g0, G, w)
                    : bits == 512 ? isa_avx512::run_group(a, i, kh0, nkh, g0, G, w)
                                  : isa_avx2::run_group(a, i, kh0, nkh, g0, G, w);
    if (!ok) return fill_item(a, i, kh0, nkh, NAN, NAN);
    g0 += G;
  }
}

// Kv heads per work item: the most (a power of two up to every kv head) that
// still leaves kItemsPerThread items per worker, so that the longest-first
// hand-out keeps the workers' finishing times close. More heads per item
// stream longer pieces of each block (run_heads). Measured on the vicuna-7b
// host tier (n = 128, 32 kv heads, 16 Zen 5 cores): 273 GB/s with one kv head
// per item, 290 / 344 / 375 / 380 GB/s with 4 / 8 / 16 / 32 (8 items per
// worker), against 416-424 GB/s for a plain read of the whole tier.
constexpr int kItemsPerThread = 8;
int item_heads(int n, int kvh, int threads) {
  int hg = 1;
  while (hg * 2 <= kvh && (int64_t)n * ((kvh + hg * 2 - 1) / (hg * 2)) >=
                              (int64_t)kItemsPerThread * threads)
    hg *= 2;
  return hg;
}

std::atomic<int> g_threads{0};  // set by fd_host_set_threads; 0 = the default below

int default_threads() {
  const int set_n = g_threads.load(std::memory_order_relaxed);
  if (set_n > 0) return set_n;
  const char* e = getenv("FASTDECODE_CPU_THREADS");
  if (e != nullptr && atoi(e) > 0) return std::min(atoi(e), FD_HOST_MAX_THREADS);
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) return std::max(1, CPU_COUNT(&set));
  return std::max(1u, std::thread::hardware_concurrency());
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" int fd_host_decode_threads(void) { return default_threads(); }

extern "C" int fd_share_host_blocks(const int32_t* host_bt, int64_t bt_stride, int32_t bt_width,
                                    const int32_t* host_lens, int32_t n, int32_t block_size,
                                    double cpu_fraction, int32_t* gpu_lens, int32_t* cpu_bt,
                                    int64_t cpu_bt_stride, int32_t* cpu_lens,
                                    int32_t* cpu_width) {
  if (n < 0 || bt_width < 0 || block_size <= 0 || !(cpu_fraction >= 0.0 && cpu_fraction <= 1.0))
    return set_error(FD_ERR_INVALID, "fd_share_host_blocks: bad sizes or fraction");
  if (n > 0 && (!host_lens || !gpu_lens || !cpu_lens || (bt_width > 0 && (!host_bt || !cpu_bt))))
    return set_error(FD_ERR_INVALID, "fd_share_host_blocks: NULL pointer");
  if (n > 0 && (bt_stride < bt_width || cpu_bt_stride < bt_width))
    return set_error(FD_ERR_INVALID, "fd_share_host_blocks: row stride below the table width");
  int32_t wc = 0;
  for (int32_t r = 0; r < n; ++r) {
    const int64_t len = std::max<int32_t>(host_lens[r], 0);
    const int64_t nb = (len + block_size - 1) / block_size;
    if (nb > bt_width)
      return set_error(FD_ERR_INVALID, "fd_share_host_blocks: row %d needs %lld blocks > width %d",
                       r, (long long)nb, bt_width);
    const int64_t k = std::min<int64_t>((int64_t)std::floor((double)nb * cpu_fraction + 0.5), nb);
    const int64_t j0 = nb - k;
    gpu_lens[r] = (int32_t)(k > 0 ? j0 * block_size : len);
    cpu_lens[r] = (int32_t)(len - gpu_lens[r]);
    if (bt_width > 0) {
      int32_t* dst = cpu_bt + (int64_t)r * cpu_bt_stride;
      if (k > 0) memcpy(dst, host_bt + (int64_t)r * bt_stride + j0, (size_t)k * 4);
      if (bt_width > k) memset(dst + k, 0, (size_t)(bt_width - k) * 4);
    }
    wc = std::max<int32_t>(wc, (int32_t)k);
  }
  if (cpu_width) *cpu_width = wc;
  return FD_OK;
}

extern "C" int fd_host_set_threads(int32_t n) {
  if (n > FD_HOST_MAX_THREADS)
    return set_error(FD_ERR_INVALID, "fd_host_set_threads: %d threads (at most %d)", n,
                     FD_HOST_MAX_THREADS);
  g_threads.store(n > 0 ? n : 0, std::memory_order_relaxed);
  return FD_OK;
}

extern "C" int fd_host_store_kv(const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                                void* k_cache, void* v_cache, int64_t cache_stride_block,
                                int64_t cache_stride_head, int64_t cache_stride_token,
                                int64_t num_blocks, const int64_t* slots, int64_t m,
                                int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                                int32_t dtype) {
  if (m < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks < 0)
    return set_error(FD_ERR_INVALID, "fd_host_store_kv: bad sizes");
  if (dtype != FD_F16 && dtype != FD_BF16 && dtype != FD_F32)
    return set_error(FD_ERR_INVALID, "fd_host_store_kv: unsupported dtype %d", dtype);
  if (m == 0) return FD_OK;
  if (!k || !v || !k_cache || !v_cache || !slots)
    return set_error(FD_ERR_INVALID, "fd_host_store_kv: NULL pointer");
  const int64_t capacity = num_blocks * block_size;
  for (int64_t j = 0; j < m; ++j)  // every slot before any write
    if (slots[j] < 0 || slots[j] >= capacity)
      return set_error(FD_ERR_RANGE, "CPU slot out of range: %lld", (long long)slots[j]);
  const size_t elt = dtype == FD_F32 ? 4 : 2, row = elt * (size_t)head_size;
  for (int64_t j = 0; j < m; ++j) {
    const int64_t blk = slots[j] / block_size, off = slots[j] % block_size;
    for (int kh = 0; kh < num_kv_heads; ++kh) {
      const int64_t dst = blk * cache_stride_block + kh * cache_stride_head + off * cache_stride_token;
      memcpy(static_cast<char*>(k_cache) + dst * elt,
             static_cast<const char*>(k) + (j * k_stride_tok + kh * k_stride_head) * elt, row);
      memcpy(static_cast<char*>(v_cache) + dst * elt,
             static_cast<const char*>(v) + (j * v_stride_tok + kh * v_stride_head) * elt, row);
    }
  }
  return FD_OK;
}

extern "C" int fd_host_decode_isa(void) { return isa_bits(); }

// Plain multi-threaded read of a host buffer on the pool that runs the
// host-core kernel: 1 MiB chunks handed out from an atomic counter, each
// read as four interleaved prefetched streams of 32-byte loads into XOR
// chains (no other work per byte; 64-bit words where AVX2 is missing), so the
// rate is the cores' DRAM read rate for a streamed buffer. The XOR of all
// words comes back as a checksum (order independent).
extern "C" int fd_host_stream_read(const void* src, size_t bytes, int32_t num_threads,
                                   uint64_t* checksum) {
  return guarded("fd_host_stream_read", [&]() -> int {
    if (bytes % 64 != 0 || num_threads < 0 || num_threads > FD_HOST_MAX_THREADS)
      return set_error(FD_ERR_INVALID, "fd_host_stream_read: bytes %% 64 != 0 or bad thread count");
    if (bytes > 0 && (src == nullptr || reinterpret_cast<uintptr_t>(src) % 64 != 0))
      return set_error(FD_ERR_INVALID, "fd_host_stream_read: NULL or unaligned (64 B) source");
    if (checksum == nullptr) return set_error(FD_ERR_INVALID, "fd_host_stream_read: NULL checksum");
    *checksum = 0;
    if (bytes == 0) return FD_OK;
    constexpr size_t kChunk = 1 << 20;
    const int64_t chunks = (int64_t)((bytes + kChunk - 1) / kChunk);
    const int nt = (int)std::max<int64_t>(
        1, std::min<int64_t>(num_threads > 0 ? num_threads : default_threads(), chunks));
    std::atomic<int64_t> next{0};
    std::atomic<uint64_t> total{0};
    const uint64_t* words = static_cast<const uint64_t*>(src);
    const bool avx2 = isa_bits() != 0;
    PoolState& ps = pool_state();
    std::lock_guard<std::mutex> call(ps.call_mu);
    ps.pool.run(nt, [&](int) {
      uint64_t x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (;;) {
        const int64_t c = next.fetch_add(1, std::memory_order_relaxed);
        if (c >= chunks) break;
        const size_t lo = (size_t)c * kChunk;
        const size_t hi = std::min(bytes, (size_t)(c + 1) * kChunk);
        if (avx2) {
          x[0] ^= read_avx2::xor_lines(static_cast<const char*>(src), lo, hi);
          continue;
        }
        for (size_t w = lo / 8; w < hi / 8; w += 8)
          for (int j = 0; j < 8; ++j) x[j] ^= words[w + j];
      }
      total.fetch_xor(x[0] ^ x[1] ^ x[2] ^ x[3] ^ x[4] ^ x[5] ^ x[6] ^ x[7],
                      std::memory_order_relaxed);
    });
    *checksum = total.load(std::memory_order_relaxed);
    return FD_OK;
  });
}

namespace fd {

// fd_host_decode_partial's argument checks (shared with the background form
// in host_async.hip, which checks before it queues a call).
int host_decode_check(const void* q, const void* k_cache, const void* v_cache, int64_t num_blocks,
                      const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
                      const int32_t* lens, int32_t n, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_size, int32_t block_size, float scale, int32_t kv_dtype,
                      void* out, int32_t out_dtype, float* lse, int32_t num_threads) {
  if (n < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_size <= 0 || head_size > 1024 || block_size <= 0 || block_size > 1024 ||
      bt_width < 0 || num_blocks < 0 || num_threads < 0 || num_threads > FD_HOST_MAX_THREADS)
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
  if (isa_bits() == 0)
    return set_error(FD_ERR_UNSUPPORTED, "fd_host_decode_partial: the CPU lacks AVX2/FMA/F16C");
  return FD_OK;
}

}  // namespace fd

extern "C" int fd_host_decode_partial(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype, void* out, int64_t out_stride_seq,
    int64_t out_stride_head, int32_t out_dtype, float* lse, int64_t lse_stride_head,
    int32_t num_threads) {
  return guarded("fd_host_decode_partial", [&]() -> int {
    const int rc = host_decode_check(q, k_cache, v_cache, num_blocks, block_table, bt_stride,
                                     bt_width, lens, n, num_heads, num_kv_heads, head_size,
                                     block_size, scale, kv_dtype, out, out_dtype, lse, num_threads);
    if (rc != FD_OK || n == 0) return rc;
    int bits = isa_bits();
    if (bits == 512 && use_bf16_dot()) bits = 513;  // internal tag of the bf16-dot body
    const HostArgs a{q, q_stride_seq, q_stride_head, k_cache, v_cache, kv_stride_block,
                     kv_stride_head, kv_stride_token, num_blocks, block_table, bt_stride, bt_width,
                     lens, n, num_heads, num_kv_heads, head_size, block_size, scale, kv_dtype, out,
                     out_stride_seq, out_stride_head, out_dtype, lse, lse_stride_head};
    // work items (sequence, group of hg adjacent kv heads), longest sequences first
    std::vector<int32_t> rows(n);
    for (int i = 0; i < n; ++i) rows[i] = i;
    std::stable_sort(rows.begin(), rows.end(), [&](int x, int y) { return lens[x] > lens[y]; });
    const int want = num_threads > 0 ? num_threads : default_threads();
    const int hg = item_heads(n, num_kv_heads, want);
    const int groups = (num_kv_heads + hg - 1) / hg;
    const int64_t items = (int64_t)n * groups;
    const int nt = (int)std::max<int64_t>(1, std::min<int64_t>(want, items));
    std::atomic<int64_t> next{0};
    PoolState& ps = pool_state();
    std::lock_guard<std::mutex> call(ps.call_mu);
    ps.pool.run(nt, [&](int) {
      Scratch w;
      for (;;) {
        const int64_t it = next.fetch_add(1, std::memory_order_relaxed);
        if (it >= items) break;
        const int kh0 = (int)(it % groups) * hg;
        run_item(a, rows[it / groups], kh0, std::min(hg, num_kv_heads - kh0), bits, w);
      }
    });
    return FD_OK;
  });
}
