// Shared device code of the two tiled decode kernels (decode_valu.hip and
// decode_mfma.hip): launch parameters, task decomposition, the K/V stream
// helpers and the cross-wave merge.
//
// Semantics follow the reference's host-tier kernel decode_attn
// (fastdecode/csrc/cpu_attn.cpp:298-411) and the GPU-tier FlashAttention
// decode call it is merged with (fastdecode/backend.py:305-316): for every
// (sequence i, query head h) the softmax-weighted sum of V over the tokens of
// the listed blocks, plus the natural-log LSE of the scaled scores, with
// out = 0 and lse = -inf for an empty row (cpu_attn.cpp:324-331).
//
// A launch covers one KV tier (a partial, as in the reference) or two: the
// fused split path walks a row's HBM-tier blocks and then its host-tier
// blocks as one list, so the tier merge of backend.py:354-356 happens inside
// the kernel. Each tier has its own cache pointers, strides, block table and
// lengths; the tier of a block is wave-uniform.
//
// Work decomposition (memory-bound design):
//   * a task = (sequence, kv head, range of up to `split_blocks` blocks) is
//     one 256-thread workgroup; its 4 wavefronts take the range's blocks
//     round-robin and each keeps its own softmax state, merged once through
//     LDS at the end. Longer rows are split and a small combine kernel merges
//     the split partials;
//   * the next block's K and V are in flight (register double buffer) while
//     the current block is reduced; 16-byte buffer loads with a non-temporal
//     hint (each byte is read once);
//   * the G = H/KVH query heads of a kv head share every K/V load.
#pragma once

#include <string.h>

#include <atomic>
#include <type_traits>

#include "fd_common.h"

namespace fd {

constexpr int kTileTokens = 16;         // tokens per block in the tiled kernels
constexpr int kWavesPerTask = 4;        // wavefronts sharing one task
constexpr int kMaxWaveBlocks = kWave;   // a wave's block ids of a task fit one VGPR
constexpr int kMaxSplitBlocks = kWavesPerTask * kMaxWaveBlocks;
constexpr int kMaxDevices = 64;         // per-device launch settings cached
constexpr int kMaxHeadGroup = 512;      // largest H / KVH the tiled kernels take (in passes)
constexpr int kMaxBlockSize = 1024;     // largest cache block size they take (16-token tiles)

// One KV tier as the tiled kernels see it (16-bit elements).
struct TierParams {
  const uint16_t* k;
  const uint16_t* v;
  int64_t sb, sh, st;  // element strides: block, head, token
  int64_t num_blocks;
  uint32_t run_bytes;    // extent of one (block, head) run: (15 * st + D) elements
  uint32_t k_run_bytes;  // extent of the K resource: run_bytes, or the K + V run if kv_adj
  bool kv_adj;           // V follows K in every token row (v == k + D): one load reads both
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
};

struct TiledParams {
  const uint16_t* q;
  int64_t q_ss, q_sh;
  TierParams tier[2];    // tier[1] is read by two-tier launches only
  const int32_t* order;  // optional processing order of the sequences
  int32_t n, H, KVH;
  int32_t D;       // head size (<= the kernel's D; lanes past it only stand by)
  int32_t BS;      // cache block size: tpb 16-token tiles, each handled as a kernel block
  int32_t tpb;     // tiles per cache block (BS / 16)
  int32_t hpk;     // query heads per kv head (H / KVH)
  int32_t passes;  // head groups per kv head: ceil(hpk / the kernel's G)
  float scale_log2;  // softmax scale * log2(e)
  void* out;
  int64_t out_ss, out_sh;
  bool out_f32;
  float* lse;
  int64_t lse_sh;
  float* part_o;    // [n, H, S, D] fp32 (normalised partial outputs)
  float* part_lse;  // [n, H, S] fp32 (natural-log LSE of each partial)
  int32_t S;        // max splits per (sequence, kv head)
  int32_t split_blocks;
  int32_t wave_blocks;  // blocks per working wave (0: every wave works; wave_blocks())
  bool xcd_group;   // adjacent kv heads of a row on one XCD (xcd_task)
  uint64_t* timeline;  // measurement only: kTimelineSlots stamps per workgroup (NULL: none)
};

// Time stamps of one workgroup in a timeline launch (s_memrealtime, 100 MHz):
// task start, wave 0's block ids in registers, each wave's end of its block
// loop, the end of the task, and a word with the task's block count (bits
// 0-15), working waves (16-23) and sequence (32-63).
constexpr int kTimelineSlots = 8;
enum TimelineSlot { kTlStart = 0, kTlIds = 1, kTlLoop0 = 2, kTlEnd = 6, kTlInfo = 7 };

// Launchers of the kernel families (decode_valu.hip, decode_mfma.hip,
// decode_mm.hip, decode_f32.hip).
hipError_t launch_valu(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                       int D, int G, bool two_tiers, hipStream_t s);
hipError_t launch_mfma(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                       int D, int G, bool two_tiers, hipStream_t s);
hipError_t launch_mm(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                     int D, bool two_tiers, hipStream_t s);
hipError_t launch_f32(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int D, int G,
                      bool two_tiers, hipStream_t s);

// Dynamic LDS that caps `kernel` at `wgs` workgroups per CU (decode_partial.hip).
unsigned cap_lds(const void* kernel, int wgs, std::atomic<int>* cache);
// Workgroups of `kernel` one CU holds at once without a cap, 0 if unknown
// (decode_partial.hip).
int natural_wgs_per_cu(const void* kernel, std::atomic<int>* cache);

// Launches `Kernel` with the occupancy cap when the plan asks for it. The
// kernel is a template argument so that each kernel has its own settings
// cache: the reserve depends on the kernel's static LDS (every kernel here
// has the type void(TiledParams), so a cache keyed by the pointer's type
// would hand the first kernel's reserve to all the others). A plan with an
// occupancy query launches nothing: it only reports the kernel's occupancy.
template <void (*Kernel)(TiledParams)>
hipError_t launch_capped(const TiledParams& tp, unsigned tasks, const SplitPlan& sp,
                         hipStream_t s) {
  if (sp.occupancy_query != nullptr) {
    static std::atomic<int> occupancy[kMaxDevices] = {};
    *sp.occupancy_query = natural_wgs_per_cu(reinterpret_cast<const void*>(Kernel), occupancy);
    return hipSuccess;
  }
  static std::atomic<int> cache[kMaxDevices] = {};
  const unsigned lds =
      sp.wg_cap > 0 ? cap_lds(reinterpret_cast<const void*>(Kernel), sp.wg_cap, cache) : 0;
  hipLaunchKernelGGL(Kernel, dim3(tasks), dim3(kWave * kWavesPerTask), lds, s, tp);
  return hipGetLastError();
}

// ---------------------------------------------------------------- loads

// 16 bytes of 16-bit elements (8 values).
struct Vec8 {
  uint32_t w[4];
};

__device__ __forceinline__ Vec8 ld16(const uint16_t* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  return Vec8{{u.x, u.y, u.z, u.w}};
}

// Buffer resource over `bytes` bytes at `base` (gfx9 raw buffer, dword data
// format); loads past `bytes` return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base,
                                                           uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Cache policy of the KV stream: non-temporal (each byte is read once; the
// hint keeps the stream from displacing other lines). Measured +7.6 % at the
// vicuna-7b shape over the default policy.
constexpr int kKvLoadPolicy = 2;
// The default policy, for loads whose cache lines are read again soon by
// another load: a line split between two loads of one wave (the matrix-core
// kernel's K column slices at head sizes other than 64 and 128) or between
// the runs of neighbouring heads (K + V runs of 4D bytes that are not whole
// lines in vLLM's layout, e.g. D = 80). There, non-temporal lines are often
// gone before their second reader comes and are fetched twice.
constexpr int kKvLoadKeep = 0;

// 16 bytes at byte `off` (per lane) + `soff` (wave-uniform) of the resource.
template <int POL = kKvLoadPolicy>
__device__ __forceinline__ Vec8 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                            uint32_t soff = 0) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, POL);
  return Vec8{{(uint32_t)u[0], (uint32_t)u[1], (uint32_t)u[2], (uint32_t)u[3]}};
}

// Loads that read K and V of a token together (a kv_adj tier) leave K and V
// interleaved in each pair of loads x, y. At D = 128 (16-lane rows, two
// tokens per load) x = [K a, V a, K b, V b] and y = [K c, V c, K d, V d]; one
// v_permlane16_swap per dword regroups them into x = [K a, K c, K b, K d] and
// y = [V a, V c, V b, V d], the layout of separate K and V loads. At D = 256
// (one token per load) v_permlane32_swap does the same with 32-lane halves:
// x = [K a, V a], y = [K c, V c] -> x = [K a, K c], y = [V a, V c].
template <int D>
__device__ __forceinline__ void split_kv(Vec8& x, Vec8& y) {
  static_assert(D == 128 || D == 256, "K and V halves of 16 or 32 lanes");
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (D == 128) {
      const auto r = __builtin_amdgcn_permlane16_swap(x.w[e], y.w[e], false, false);
      x.w[e] = r[0];
      y.w[e] = r[1];
    } else {
      const auto r = __builtin_amdgcn_permlane32_swap(x.w[e], y.w[e], false, false);
      x.w[e] = r[0];
      y.w[e] = r[1];
    }
  }
}

// 16 bytes at `p` through a global load with the non-temporal hint (the
// same cache policy as kKvLoadPolicy). Callers keep `p` inside the cache.
__device__ __forceinline__ Vec8 global_ld16(const char* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return Vec8{{u[0], u[1], u[2], u[3]}};
}

template <typename T>
__device__ __forceinline__ float dot8(const Vec8& a, const Vec8& b, float acc) {
  acc = dot2(T{}, a.w[0], b.w[0], acc);
  acc = dot2(T{}, a.w[1], b.w[1], acc);
  acc = dot2(T{}, a.w[2], b.w[2], acc);
  acc = dot2(T{}, a.w[3], b.w[3], acc);
  return acc;
}

template <typename T>
__device__ __forceinline__ void axpy8(float p, const Vec8& v, float* acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc[2 * e] = __builtin_fmaf(p, lo_f32(T{}, v.w[e]), acc[2 * e]);
    acc[2 * e + 1] = __builtin_fmaf(p, hi_f32(T{}, v.w[e]), acc[2 * e + 1]);
  }
}

// Writes 8 consecutive outputs starting at element `off` of `out` (fp32
// when `f32` is set or the KV is fp32, else the 16-bit KV type).
template <typename T>
__device__ __forceinline__ void store8(void* out, int64_t off, bool f32, const float* o) {
  if (std::is_same<T, F32>::value || f32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(out) + off);
    p[0] = make_float4(o[0], o[1], o[2], o[3]);
    p[1] = make_float4(o[4], o[5], o[6], o[7]);
  } else if constexpr (!std::is_same<T, F32>::value) {
    uint4 u;
    u.x = to_out(T{}, o[0]) | (uint32_t(to_out(T{}, o[1])) << 16);
    u.y = to_out(T{}, o[2]) | (uint32_t(to_out(T{}, o[3])) << 16);
    u.z = to_out(T{}, o[4]) | (uint32_t(to_out(T{}, o[5])) << 16);
    u.w = to_out(T{}, o[6]) | (uint32_t(to_out(T{}, o[7])) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + off) = u;
  }
}

// ---------------------------------------------------------------- tasks

// One task of a tiled launch: (sequence i, kv head kh, split) and the range
// [b_begin, b_end) of the row's nb blocks it covers. With two tiers the row's
// blocks are tier 0's nba blocks followed by tier 1's.
struct Task {
  int i, kh, split;
  int h0;      // first query head of the task: kh * hpk + its head group * G
  int gcount;  // query heads of the task (<= G; the kernel's other head slots
               // repeat the last one and write nothing)
  int la, lb;  // tokens of the row in tier 0 / tier 1 (<= 0: none)
  int nba, nb;
  int b_begin, b_end, nsplit;
  bool range_bad;  // a length needs more blocks than its table has
};

// blockIdx.x -> task: kv head fastest, then head group (one unless a kv head
// has more query heads than the kernel's G), then sequence (in the caller's order
// when one is given, e.g. longest rows first so the last workgroups dispatched
// are short ones), split slowest. Split-major order matters on this GPU:
// workgroups are dealt round-robin to the XCDs and, inside an XCD, to its
// shader engines, so interleaving each row's splits (most of whose later
// splits are empty) would hand the empty workgroups to a fixed half of the
// engines and idle them; split-major keeps the empty ones together at the end.
// False when the workgroup has nothing to do: an order entry outside [0, n),
// or a split past the row's last block.
// Workgroups are dealt round-robin to the GPU's 8 XCDs, each with its own
// L2. With p.xcd_group set, within every 32 consecutive workgroups XCD x
// receives four (dispatch rounds 0-3) and they take logical tasks 4x .. 4x+3
// of the 32, i.e. four adjacent kv heads of one row. Where a token's K + V
// runs of adjacent heads share 128-byte lines (2 D elements of 2 bytes, not
// a multiple of 128 bytes: D = 80, 112, ...), the shared lines are then read
// by tasks of one XCD at about the same time (four heads span 16 D bytes,
// always whole lines); measured +2-3 % at D = 80 / 96 / 112, but -0.7 % at
// D = 128 and -3 % on small batches, so the host sets the flag only for
// head sizes that are not multiples of 64. A trailing partial group of 32
// keeps the identity order; the longest-first row order holds at a
// granularity of 32 workgroups.
constexpr int kXcds = 8;
constexpr int kXcdHeads = 4;
__device__ __forceinline__ int xcd_task(int b, int tasks) {
  constexpr int kGroup = kXcds * kXcdHeads;
  const int g = b / kGroup, r = b % kGroup;
  return (g + 1) * kGroup <= tasks ? g * kGroup + kXcdHeads * (r % kXcds) + r / kXcds : b;
}

template <int G, bool TWO>
__device__ __forceinline__ bool decode_task(const TiledParams& p, Task& t) {
  const int task = p.xcd_group ? xcd_task(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  t.kh = task % p.KVH;
  int rest = task / p.KVH;
  // a kv head with more than G query heads is done in passes of up to G
  // heads, each its own task over the same blocks
  const int pass = rest % p.passes;
  rest /= p.passes;
  t.h0 = t.kh * p.hpk + pass * G;
  t.gcount = min(G, p.hpk - pass * G);
  t.split = rest / p.n;
  int i = rest % p.n;
  if (p.order != nullptr) {
    i = p.order[i];
    if ((unsigned)i >= (unsigned)p.n) return false;
  }
  t.i = i;
  t.la = p.tier[0].lens[i];
  t.lb = TWO ? p.tier[1].lens[i] : 0;
  t.nba = t.la > 0 ? (t.la + kTileTokens - 1) / kTileTokens : 0;
  const int nbb = t.lb > 0 ? (t.lb + kTileTokens - 1) / kTileTokens : 0;
  t.nb = t.nba + nbb;
  t.b_begin = t.split * p.split_blocks;
  if (t.split > 0 && t.b_begin >= t.nb) return false;
  t.b_end = min(t.nb, t.b_begin + p.split_blocks);
  t.nsplit = t.nb > 0 ? (t.nb + p.split_blocks - 1) / p.split_blocks : 1;
  t.range_bad = t.la > p.tier[0].bt_width * p.BS || (TWO && t.lb > p.tier[1].bt_width * p.BS);
  return true;
}

// Valid tokens of the row's block u (< 16 only for the last block of a tier).
template <bool TWO>
__device__ __forceinline__ int block_tokens(const Task& t, int u) {
  if (TWO && u >= t.nba) return min(kTileTokens, t.lb - (u - t.nba) * kTileTokens);
  return min(kTileTokens, t.la - u * kTileTokens);
}

// Empty row (out = 0, lse = -inf) or a length past its table (NaN), written
// by one wave of split 0.
template <typename T, int D, int G>
__device__ __forceinline__ void write_empty(const TiledParams& p, const Task& t, int lane) {
  constexpr int LPT = D / 8;
  if (lane >= LPT || lane * 8 >= p.D) return;
  const float fill = t.range_bad ? qnan() : 0.f;
  for (int g = 0; g < t.gcount; ++g) {  // gcount <= G
    const int h = t.h0 + g;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fill;
    store8<T>(p.out, (int64_t)t.i * p.out_ss + (int64_t)h * p.out_sh + lane * 8, p.out_f32, o);
    if (lane == 0) p.lse[(int64_t)h * p.lse_sh + t.i] = t.range_bad ? qnan() : neg_inf();
  }
}

// A wave's blocks of its task are b_begin + wave + s k, s = the task's
// working waves (4 unless p.wave_blocks says fewer). Their ids are read
// once, one per lane (at most 64), range-checked together against their
// tier's cache and later picked with v_readlane; a bad id is replaced by 0
// (every read stays inside the cache) and flags the row. The wave's blocks
// from index k1 on are in tier 1.
struct WaveBlocks {
  int first;   // the wave's first block index in the row
  int stride;  // block index step between the wave's blocks (the task's working waves)
  int nw;      // blocks of this wave
  int k1;      // first of the wave's blocks in tier 1 (>= nw: none)
  int my_bid;  // lane k: id of the cache block holding the wave's k-th tile
  int my_sub;  // lane k: that tile's index inside its cache block (0 when BS = 16)
  bool bad;
};

// With p.wave_blocks > 0 a task works with as many of its waves as give
// each about that many blocks (at least one, at most four); the rest only
// take part in the merge. A short row then keeps fewer blocks in flight than
// a long one.
template <bool TWO>
__device__ __forceinline__ WaveBlocks wave_blocks(const TiledParams& p, const Task& t, int wave,
                                                  int lane) {
  WaveBlocks w;
  int ws = kWavesPerTask;
  if (p.wave_blocks > 0) {
    // (each wave's block ids fit its 64 lanes: nblk <= split_blocks <= 256)
    const int nblk = t.b_end - t.b_begin;
    ws = max((nblk + p.wave_blocks - 1) / p.wave_blocks,
             (nblk + kMaxWaveBlocks - 1) / kMaxWaveBlocks);
    ws = min(kWavesPerTask, max(1, ws));
  }
  w.stride = ws;
  w.first = t.b_begin + wave;
  w.nw = wave < ws && w.first < t.b_end ? (t.b_end - w.first + ws - 1) / ws : 0;
  w.k1 = TWO ? (t.nba > w.first ? (t.nba - w.first + ws - 1) / ws : 0) : w.nw;
  int bid = 0, sub = 0;
  bool my_bad = false;
  if (lane < w.nw) {
    // tile u of the row: tile u % tpb of the row's cache block u / tpb
    const int u = w.first + ws * lane;
    if (TWO && u >= t.nba) {
      const TierParams& tp = p.tier[1];
      const int ut = u - t.nba;
      bid = tp.bt[(int64_t)t.i * tp.bt_stride + ut / p.tpb];
      sub = ut % p.tpb;
      my_bad = bid < 0 || (int64_t)bid >= tp.num_blocks;
    } else {
      const TierParams& tp = p.tier[0];
      bid = tp.bt[(int64_t)t.i * tp.bt_stride + u / p.tpb];
      sub = u % p.tpb;
      my_bad = bid < 0 || (int64_t)bid >= tp.num_blocks;
    }
  }
  w.bad = __ballot(my_bad) != 0;
  w.my_bid = my_bad ? 0 : bid;
  w.my_sub = my_bad ? 0 : sub;
  return w;
}

// Per-wave softmax states (log2-domain max, sum, unnormalised accumulator)
// for the cross-wave merge.
template <int D, int G>
struct WaveStates {
  float acc[kWavesPerTask][G][D];
  float m[kWavesPerTask][G];
  float l[kWavesPerTask][G];
  int bad[kWavesPerTask];
};

// Folds the TPW = 64 / LPT lane-rows of a wave (each with its own softmax
// state per head: log2-domain max m, sum l, accumulator of its 8 dims) into
// the wave's state and publishes it in `ws` for finish_task.
template <int D, int G>
__device__ __forceinline__ void publish_wave_state(WaveStates<D, G>& ws, int wave, int lane,
                                                   const float* m, const float* l,
                                                   const float (*acc)[8], bool bad) {
  constexpr int LPT = D / 8;
  const int chunk = lane % LPT;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = m[g];
    if constexpr (LPT < kWave) M = xor_max<LPT>(M);
    const float Ms = M == neg_inf() ? 0.f : M;
    const float w = fast_exp2(m[g] - Ms);
    float lt = l[g] * w;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = acc[g][e] * w;
    if constexpr (LPT < kWave) {
      lt = xor_sum<LPT>(lt);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = xor_sum<LPT>(o[e]);
    }
    if (lane < LPT) {
      float4* dst = reinterpret_cast<float4*>(&ws.acc[wave][g][chunk * 8]);
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (lane == 0) {
      ws.m[wave][g] = M;
      ws.l[wave][g] = lt;
    }
  }
  if (lane == 0) ws.bad[wave] = bad ? 1 : 0;
}

// Wave 0, after the workgroup barrier: merges the waves' states with the
// log-sum-exp rule and writes the final result (one split) or this split's
// partial for the combine pass.
template <typename T, int D, int G>
__device__ __forceinline__ void finish_task(const TiledParams& p, const Task& t,
                                            const WaveStates<D, G>& ws, int lane) {
  constexpr int LPT = D / 8;
  const int chunk = lane % LPT;
  bool bad = false;
#pragma unroll
  for (int w = 0; w < kWavesPerTask; ++w) bad |= ws.bad[w] != 0;
  const bool write_final = t.nsplit == 1;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = ws.m[0][g];
#pragma unroll
    for (int w = 1; w < kWavesPerTask; ++w) M = fmaxf(M, ws.m[w][g]);
    const float Ms = M == neg_inf() ? 0.f : M;
    float lt = 0.f;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
    // every lane reads its chunk's slice of every wave's state at once (lanes
    // past LPT repeat a chunk's reads and store nothing): the LDS reads issue
    // together instead of one wave's after another's
    float4 sa[kWavesPerTask], sb[kWavesPerTask];
#pragma unroll
    for (int w = 0; w < kWavesPerTask; ++w) {
      const float4* src = reinterpret_cast<const float4*>(&ws.acc[w][g][chunk * 8]);
      sa[w] = src[0];
      sb[w] = src[1];
    }
#pragma unroll
    for (int w = 0; w < kWavesPerTask; ++w) {
      const float sc = fast_exp2(ws.m[w][g] - Ms);  // 0 for a wave without blocks
      lt += sc * ws.l[w][g];
      o[0] += sc * sa[w].x;
      o[1] += sc * sa[w].y;
      o[2] += sc * sa[w].z;
      o[3] += sc * sa[w].w;
      o[4] += sc * sb[w].x;
      o[5] += sc * sb[w].y;
      o[6] += sc * sb[w].z;
      o[7] += sc * sb[w].w;
    }
    const float inv = 1.f / lt;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
    float lse_nat = (M + fast_log2(lt)) * kLn2;
    if (bad) {
      lse_nat = qnan();
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = qnan();
    }
    const int h = t.h0 + g;
    if (g < t.gcount && lane < LPT && chunk * 8 < p.D) {
      if (write_final) {
        store8<T>(p.out, (int64_t)t.i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8,
                  p.out_f32, o);
        if (lane == 0) p.lse[(int64_t)h * p.lse_sh + t.i] = lse_nat;
      } else {
        const int64_t pidx = ((int64_t)t.i * p.H + h) * p.S + t.split;
        store8<T>(p.part_o, pidx * p.D + chunk * 8, true, o);
        if (lane == 0) p.part_lse[pidx] = lse_nat;
      }
    }
  }
}

// Query head of the task's head slot g: slots past the task's heads repeat
// its last head (their results are never written).
__device__ __forceinline__ int task_head(const Task& t, int g) {
  return t.h0 + min(g, t.gcount - 1);
}

// The cache run of a wave's block k: K and V buffer resources over its
// (block, kv head) run in the tier it lies in, and that tier (wave-uniform;
// the kernel picks its per-lane offsets for the tier).
struct BlockSrc {
  __amdgpu_buffer_rsrc_t k, v;
  const char* kp;  // the K run's first byte (global loads of a kv_adj tier)
  bool t1;
};

template <bool TWO>
__device__ __forceinline__ BlockSrc block_src(const TiledParams& p, const WaveBlocks& wb, int kh,
                                              int k) {
  const bool t1 = TWO && k >= wb.k1;
  const int bid = __builtin_amdgcn_readlane(wb.my_bid, k);
  const int sub = __builtin_amdgcn_readlane(wb.my_sub, k);
  const TierParams& a = p.tier[0];
  const TierParams& b = p.tier[TWO ? 1 : 0];
  const int64_t base = (int64_t)bid * (t1 ? b.sb : a.sb) + (int64_t)kh * (t1 ? b.sh : a.sh) +
                       (int64_t)sub * kTileTokens * (t1 ? b.st : a.st);
  const uint32_t rb = t1 ? b.run_bytes : a.run_bytes;
  BlockSrc s;
  s.k = make_rsrc((t1 ? b.k : a.k) + base, t1 ? b.k_run_bytes : a.k_run_bytes);
  s.v = make_rsrc((t1 ? b.v : a.v) + base, rb);
  s.kp = reinterpret_cast<const char*>((t1 ? b.k : a.k) + base);
  s.t1 = t1;
  return s;
}

}  // namespace fd
