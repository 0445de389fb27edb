// Paged partial decode attention for gfx950.
//
// Semantics follow the reference's host-tier kernel decode_attn
// (fastdecode/csrc/cpu_attn.cpp:298-411) and the GPU-tier FlashAttention
// decode call it is merged with (fastdecode/backend.py:305-316): for every
// (sequence i, query head h) the softmax-weighted sum of V over the tokens of
// the listed blocks, plus the natural-log LSE of the scaled scores, with
// out = 0 and lse = -inf for an empty row (cpu_attn.cpp:324-331).
//
// Work decomposition (memory-bound design):
//   * a task = (sequence, kv head, range of up to `split_blocks` blocks) is
//     one 256-thread workgroup; its 4 wavefronts take the range's blocks
//     round-robin and each keeps its own softmax state, merged once through
//     LDS at the end. At the vicuna-7b shape a task covers a whole sequence,
//     so no second pass is needed; longer rows are split and a small combine
//     kernel merges the split partials;
//   * a block of 16 tokens is read as 16-byte buffer loads: a token row of D
//     elements is spread over LPT = D/8 lanes, so one load instruction moves
//     64/LPT whole rows (1 KiB for D = 128) and the wave's lanes form
//     TPW = 64/LPT "rows" that each own a token of every load;
//   * the next block's K and V are in flight (register double buffer) while
//     the current block is reduced;
//   * q.k: v_dot2_f32_{f16,bf16} on packed pairs, then a DPP butterfly over
//     the LPT lanes of a token (fp32 throughout);
//   * online softmax in the exp2 domain, kept independently per lane-row
//     (no cross-row traffic in the main loop); rows, then waves, are merged at
//     the end with the log-sum-exp rule of the tier merge;
//   * the G = H/KVH query heads of a kv head share every K/V load.
#include <string.h>

#include <atomic>
#include <type_traits>

#include "fd_common.h"

namespace fd {

namespace {

constexpr int kTileTokens = 16;         // tokens per block in the tiled kernel
constexpr int kWavesPerTask = 4;        // wavefronts sharing one task
constexpr int kMaxWaveBlocks = kWave;   // a wave's block ids of a task fit one VGPR
constexpr int kMaxSplitBlocks = kWavesPerTask * kMaxWaveBlocks;
constexpr int kMaxDevices = 64;         // per-device launch settings cached

struct TiledParams {
  const uint16_t* q;
  int64_t q_ss, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sh, kv_st;
  int64_t num_blocks;
  uint32_t run_bytes;  // extent of one (block, head) run: (15 * kv_st + D) elements
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
  const int32_t* order;  // optional processing order of the sequences
  int32_t n, H, KVH;
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
};

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

// 16 bytes at byte `off` (per lane) + `soff` (wave-uniform) of the resource.
__device__ __forceinline__ Vec8 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                            uint32_t soff = 0) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, kKvLoadPolicy);
  return Vec8{{(uint32_t)u[0], (uint32_t)u[1], (uint32_t)u[2], (uint32_t)u[3]}};
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

// Writes 8 consecutive outputs starting at element `off` of `out`.
template <typename T>
__device__ __forceinline__ void store8(void* out, int64_t off, bool f32, const float* o) {
  if (f32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(out) + off);
    p[0] = make_float4(o[0], o[1], o[2], o[3]);
    p[1] = make_float4(o[4], o[5], o[6], o[7]);
  } else {
    uint4 u;
    u.x = from_f32(T{}, o[0]) | (uint32_t(from_f32(T{}, o[1])) << 16);
    u.y = from_f32(T{}, o[2]) | (uint32_t(from_f32(T{}, o[3])) << 16);
    u.z = from_f32(T{}, o[4]) | (uint32_t(from_f32(T{}, o[5])) << 16);
    u.w = from_f32(T{}, o[6]) | (uint32_t(from_f32(T{}, o[7])) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + off) = u;
  }
}

// ---------------------------------------------------------------- shared
// pieces of the two tiled kernels

// One task of a tiled launch: (sequence i, kv head kh, split) and the block
// range [b_begin, b_end) of the sequence's nb blocks it covers.
struct Task {
  int i, kh, split;
  int L, nb, b_begin, b_end, nsplit;
  bool range_bad;  // the length needs more blocks than the table has
};

// blockIdx.x -> task: kv head fastest, then sequence (in the caller's order
// when one is given, e.g. longest rows first so the last workgroups dispatched
// are short ones), split slowest. Split-major order matters on this GPU:
// workgroups are dealt round-robin to the XCDs and, inside an XCD, to its
// shader engines, so interleaving each row's splits (most of whose later
// splits are empty) would hand the empty workgroups to a fixed half of the
// engines and idle them; split-major keeps the empty ones together at the end.
// False when the workgroup has nothing to do: an order entry outside [0, n),
// or a split past the row's last block.
__device__ __forceinline__ bool decode_task(const TiledParams& p, Task& t) {
  const int task = blockIdx.x;
  t.kh = task % p.KVH;
  const int rest = task / p.KVH;
  t.split = rest / p.n;
  int i = rest % p.n;
  if (p.order != nullptr) {
    i = p.order[i];
    if ((unsigned)i >= (unsigned)p.n) return false;
  }
  t.i = i;
  t.L = p.lens[i];
  t.nb = t.L > 0 ? (t.L + kTileTokens - 1) / kTileTokens : 0;
  t.b_begin = t.split * p.split_blocks;
  if (t.split > 0 && t.b_begin >= t.nb) return false;
  t.b_end = min(t.nb, t.b_begin + p.split_blocks);
  t.nsplit = t.nb > 0 ? (t.nb + p.split_blocks - 1) / p.split_blocks : 1;
  t.range_bad = t.L > p.bt_width * kTileTokens;
  return true;
}

// Empty row (out = 0, lse = -inf) or a length past the table (NaN), written
// by one wave of split 0.
template <typename T, int D, int G>
__device__ __forceinline__ void write_empty(const TiledParams& p, const Task& t, int lane) {
  constexpr int LPT = D / 8;
  if (lane >= LPT) return;
  const float fill = t.range_bad ? qnan() : 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = t.kh * G + g;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fill;
    store8<T>(p.out, (int64_t)t.i * p.out_ss + (int64_t)h * p.out_sh + lane * 8, p.out_f32, o);
    if (lane == 0) p.lse[(int64_t)h * p.lse_sh + t.i] = t.range_bad ? qnan() : neg_inf();
  }
}

// A wave's blocks of its task are b_begin + wave + 4k. Their ids are read
// once, one per lane (at most 64), range-checked together and later picked
// with v_readlane; a bad id is replaced by 0 (every read stays inside the
// cache) and flags the row.
struct WaveBlocks {
  int first;   // the wave's first block index in the row
  int nw;      // blocks of this wave
  int my_bid;  // lane k: id of the wave's k-th block
  bool bad;
};

__device__ __forceinline__ WaveBlocks wave_blocks(const TiledParams& p, const Task& t, int wave,
                                                  int lane) {
  WaveBlocks w;
  w.first = t.b_begin + wave;
  w.nw = w.first < t.b_end ? (t.b_end - w.first + kWavesPerTask - 1) / kWavesPerTask : 0;
  int bid = lane < w.nw ? p.bt[(int64_t)t.i * p.bt_stride + w.first + kWavesPerTask * lane] : 0;
  const bool my_bad = lane < w.nw && (bid < 0 || (int64_t)bid >= p.num_blocks);
  w.bad = __ballot(my_bad) != 0;
  w.my_bid = my_bad ? 0 : bid;
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
#pragma unroll
    for (int w = 0; w < kWavesPerTask; ++w) {
      const float sc = fast_exp2(ws.m[w][g] - Ms);  // 0 for a wave without blocks
      lt += sc * ws.l[w][g];
      if (lane < LPT) {
        const float4* src = reinterpret_cast<const float4*>(&ws.acc[w][g][chunk * 8]);
        const float4 a = src[0];
        const float4 b = src[1];
        o[0] += sc * a.x;
        o[1] += sc * a.y;
        o[2] += sc * a.z;
        o[3] += sc * a.w;
        o[4] += sc * b.x;
        o[5] += sc * b.y;
        o[6] += sc * b.z;
        o[7] += sc * b.w;
      }
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
    const int h = t.kh * G + g;
    if (lane < LPT) {
      if (write_final) {
        store8<T>(p.out, (int64_t)t.i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8,
                  p.out_f32, o);
        if (lane == 0) p.lse[(int64_t)h * p.lse_sh + t.i] = lse_nat;
      } else {
        const int64_t pidx = ((int64_t)t.i * p.H + h) * p.S + t.split;
        store8<T>(p.part_o, pidx * D + chunk * 8, true, o);
        if (lane == 0) p.part_lse[pidx] = lse_nat;
      }
    }
  }
}

// ---------------------------------------------------------------- VALU kernel
// Tiled kernel: block_size == 16, D in {64, 128, 256}, G in {1, 2, 4, 8},
// 16-bit KV, every stride a multiple of 8 elements and 16-byte aligned bases.
// One workgroup (4 waves) per task; grid = n * KVH * S tasks.
template <typename T, int D, int G>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_tiled_kernel(TiledParams p) {
  constexpr int LPT = D / 8;                // lanes per token row
  constexpr int TPW = kWave / LPT;          // token rows per load instruction
  constexpr int STEPS = kTileTokens / TPW;  // loads per block per lane

  __shared__ WaveStates<D, G> ws;

  const int lane = threadIdx.x & (kWave - 1);
  // The wave index is uniform across the wave; readfirstlane keeps it (and all
  // indexing derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Task t;
  if (!decode_task(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<T, D, G>(p, t, lane);
    return;
  }
  const int i = t.i;
  const int L = t.L;

  const int row = lane / LPT;    // which token of each load this lane owns
  const int chunk = lane % LPT;  // which 8-element slice of the row

  // ---- query fragments (unscaled, native precision)
  Vec8 qf[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = t.kh * G + g;
    qf[g] = ld16(p.q + (int64_t)i * p.q_ss + (int64_t)h * p.q_sh + chunk * 8);
  }

  // Byte offset of this lane's 16 bytes for load step j inside one
  // (block, head) run; the same for every block, so the loop only moves the
  // wave-uniform block base held in a scalar buffer resource.
  uint32_t voff[STEPS];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    voff[j] = (uint32_t)(((int64_t)(j * TPW + row) * p.kv_st + chunk * 8) * 2);
  }
  const int64_t head_off = (int64_t)t.kh * p.kv_sh;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = neg_inf();
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  const WaveBlocks wb = wave_blocks(p, t, wave, lane);
  const int nw = wb.nw;
  // Element offset of this wave's k-th block for this kv head; wave-uniform.
  auto block_base = [&](int k) -> int64_t {
    const int bid = __builtin_amdgcn_readlane(wb.my_bid, k);
    return (int64_t)bid * p.kv_sb + head_off;
  };
  // Valid tokens of this wave's k-th block (< 16 only for the row's last block).
  auto block_tokens = [&](int k) -> int {
    return min(kTileTokens, L - (wb.first + kWavesPerTask * k) * kTileTokens);
  };

  Vec8 kb[2][STEPS], vb[2][STEPS];
  auto load_block = [&](int slot, int64_t base) {
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.k + base, p.run_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.v + base, p.run_bytes);
#pragma unroll
    for (int j = 0; j < STEPS; ++j) kb[slot][j] = buffer_ld16(kr, voff[j]);
#pragma unroll
    for (int j = 0; j < STEPS; ++j) vb[slot][j] = buffer_ld16(vr, voff[j]);
    // keep the prefetch at the top of the reduction that overlaps it
    __builtin_amdgcn_sched_barrier(0);
  };

  // Reduces one resident block; `ntok` < 16 only for the sequence's last block.
  auto compute_block = [&](int slot, int ntok) {
    float s[G][STEPS];
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s[g][j] = group_sum<LPT>(dot8<T>(qf[g], kb[slot][j], 0.f)) * p.scale_log2;
      }
    }
    if (ntok < kTileTokens) {
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        const bool valid = j * TPW + row < ntok;
#pragma unroll
        for (int g = 0; g < G; ++g) s[g][j] = valid ? s[g][j] : neg_inf();
        if (!valid) {
#pragma unroll
          for (int e = 0; e < 4; ++e) vb[slot][j].w[e] = 0u;  // stale V may be NaN
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mb = s[g][0];
#pragma unroll
      for (int j = 1; j < STEPS; ++j) mb = fmaxf(mb, s[g][j]);
      const float mn = fmaxf(m[g], mb);
      const float ms = mn == neg_inf() ? 0.f : mn;
      const float alpha = fast_exp2(m[g] - ms);
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        const float pj = fast_exp2(s[g][j] - ms);
        psum += pj;
        axpy8<T>(pj, vb[slot][j], acc[g]);
      }
      l[g] = l[g] * alpha + psum;
      m[g] = mn;
    }
  };

  // ---- main loop: two blocks per iteration, ping-ponging register buffers.
  // Loads inside the steady-state body are unconditional so the compiler's
  // wait counts only cover the block being reduced, never its successor.
  if (nw > 0) {
    int k = 0;
    load_block(0, block_base(0));
    for (; k + 2 < nw; k += 2) {
      load_block(1, block_base(k + 1));
      compute_block(0, block_tokens(k));
      load_block(0, block_base(k + 2));
      compute_block(1, block_tokens(k + 1));
    }
    if (k + 1 < nw) {
      load_block(1, block_base(k + 1));
      compute_block(0, block_tokens(k));
      compute_block(1, block_tokens(k + 1));
    } else {
      compute_block(0, block_tokens(k));
    }
  }

  // ---- merge the TPW lane-rows of each head into this wave's state, publish it
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = m[g];
#pragma unroll
    for (int x = LPT; x < kWave; x <<= 1) M = fmaxf(M, shfl_xor_f32(M, x));
    const float Ms = M == neg_inf() ? 0.f : M;
    const float w = fast_exp2(m[g] - Ms);
    float lt = l[g] * w;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = acc[g][e] * w;
#pragma unroll
    for (int x = LPT; x < kWave; x <<= 1) {
      lt += shfl_xor_f32(lt, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += shfl_xor_f32(o[e], x);
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
  if (lane == 0) ws.bad[wave] = wb.bad ? 1 : 0;
  __syncthreads();
  if (wave != 0) return;
  finish_task<T, D, G>(p, t, ws, lane);
}

// ---------------------------------------------------------------- MFMA kernel
// Grouped-query kernel (G = H/KVH in {4, 8}): the scores of a block come from
// the matrix cores, P.V stays on the VALU in fp32.
//
// Per 32 dims, one v_mfma_f32_16x16x32_{f16,bf16} computes
//   S^T[16 x 16] = K[16 x 32] . Qrep^T[32 x 16]
// whose 16 A rows are the block's 16 tokens and whose 16 B columns hold the G
// query heads of the kv head repeated 16/G times. In the gfx950 operand
// layout (A: lane l holds row l%16, dims 8*(l/16)..+7 of the step; B: lane l
// holds column l%16, the same dims; D: lane l holds rows 4*(l/16)..+3 of
// column l%16) the K operand is simply 16 bytes of token l%16's row, and lane
// l ends with the scores of tokens 4R..4R+3, R = l/16, for head (l%16) % G.
//
// Every 16-lane row R keeps its own softmax state per head (max and sum over
// the row's tokens 4R..4R+3 of every block), and its lanes also hold the V
// slices of exactly those tokens, so the block loop has no cross-row traffic:
// a head's block max is an in-lane max over 4 scores, and the probabilities
// reach the V lanes of the row through DPP row broadcasts. The running max is
// raised only when a block max exceeds it by more than kLazyRescale (log2
// units, so p <= 2^kLazyRescale), which after a row's first block is rare;
// the four rows are merged once at the end with the log-sum-exp rule. p is
// never rounded to 16 bits.
constexpr float kLazyRescale = 8.f;

template <typename T>
__device__ __forceinline__ f32x4 mfma_16x16x32(const Vec8& a, const Vec8& b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<F16>(const Vec8& a, const Vec8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<BF16>(const Vec8& a, const Vec8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Lane n of each 16-lane row, broadcast to the whole row (DPP row_newbcast;
// every source lane exists, so bound_ctrl never applies).
template <int n>
__device__ __forceinline__ float row_bcast(float x) {
  static_assert(n >= 0 && n < 16, "row_bcast: lane within a row");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + n, 0xF, 0xF, true));
}

// f(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Per-lane V mapping of a 16-lane row: TPL tokens x CPL 8-element slices.
template <int D>
struct VMap {
  static constexpr int CPL = D >= 256 ? D / 128 : 1;  // slices per lane
  static constexpr int TPL = D / 32 / CPL;            // tokens per lane
  static constexpr int LPS = 4 * TPL;                 // lanes sharing the same tokens
  static_assert(CPL * TPL * 16 * 8 == 4 * D, "VMap covers the row's 4 tokens");
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_mfma_kernel(TiledParams p) {
  static_assert(G == 4 || G == 8, "decode_mfma_kernel: G must be 4 or 8");
  using VM = VMap<D>;
  constexpr int CPL = VM::CPL, TPL = VM::TPL;
  constexpr int KS = D / 32;  // K: 32-dim matrix-core steps per row

  __shared__ WaveStates<D, G> ws;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Task t;
  if (!decode_task(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<T, D, G>(p, t, lane);
    return;
  }
  const int L = t.L;

  const int col = lane & 15;   // K: token row of the A operand; scores: head column
  const int R = lane >> 4;     // K: dims 8R..+7 of each step; scores, V: tokens 4R..4R+3
  const int hg = col % G;      // this lane's score head
  // V: tokens 4R + tsub .. +TPL-1, slices vchunk + 16h (h < CPL)
  const int tsub = (col / VM::LPS) * TPL;
  const int vchunk = col % VM::LPS;

  // B operand: query head hg, dims 8R + 32*ks .. +7 (unscaled)
  Vec8 qb[KS];
  {
    const uint16_t* qrow =
        p.q + (int64_t)t.i * p.q_ss + (int64_t)(t.kh * G + hg) * p.q_sh + R * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] = ld16(qrow + 32 * ks);
  }
  // Byte offsets inside one (block, head) run: K step ks at koff + 64*ks;
  // V token j, slice h at voff + j*kv_st*2 + 256*h (scalar parts).
  const uint32_t koff = (uint32_t)(((int64_t)col * p.kv_st + R * 8) * 2);
  const uint32_t voff = (uint32_t)(((int64_t)(4 * R + tsub) * p.kv_st + vchunk * 8) * 2);
  const uint32_t vtok = (uint32_t)(p.kv_st * 2);
  const int64_t head_off = (int64_t)t.kh * p.kv_sh;

  // m, l: row R's state for head hg (identical in the row's copies of hg);
  // acc: every head, this lane's V slices, over its tokens.
  float m = neg_inf(), l = 0.f, acc[G][CPL][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int h = 0; h < CPL; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][h][e] = 0.f;
    }
  }

  const WaveBlocks wb = wave_blocks(p, t, wave, lane);
  const int nw = wb.nw;
  auto block_base = [&](int k) -> int64_t {
    const int bid = __builtin_amdgcn_readlane(wb.my_bid, k);
    return (int64_t)bid * p.kv_sb + head_off;
  };
  auto block_tokens = [&](int k) -> int {
    return min(kTileTokens, L - (wb.first + kWavesPerTask * k) * kTileTokens);
  };

  // K is single-buffered (its registers are free once the block's matrix-core
  // steps have read them), V double-buffered: block k+1's K and V are issued
  // right after block k's scores and land while block k's softmax and P.V run.
  Vec8 kb[KS], vb[2][TPL][CPL];
  auto load_block = [&](int slot, int64_t base) {
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.k + base, p.run_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.v + base, p.run_bytes);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kb[ks] = buffer_ld16(kr, koff, 64 * ks);
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
#pragma unroll
      for (int h = 0; h < CPL; ++h) vb[slot][j][h] = buffer_ld16(vr, voff, j * vtok + 256 * h);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Scores of the resident K block (log2 domain, masked past ntok).
  auto block_scores = [&](int ntok, float* s) {
    f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sv = mfma_16x16x32<T>(kb[ks], qb[ks], sv);
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = sv[r] * p.scale_log2;
    if (ntok < kTileTokens) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = 4 * R + r < ntok ? s[r] : neg_inf();
    }
  };

  // Online softmax (lazy rescale) and P.V of one block whose scores are in s.
  auto block_update = [&](int slot, int ntok, float* s) {
    if (ntok < kTileTokens) {
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        if (4 * R + tsub + j >= ntok) {
#pragma unroll
          for (int h = 0; h < CPL; ++h) {
#pragma unroll
            for (int e = 0; e < 4; ++e) vb[slot][j][h].w[e] = 0u;  // stale V may be NaN
          }
        }
      }
    }
    const float bmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    const bool raise = bmax > m + kLazyRescale;  // false while both are -inf
    if (__ballot(raise) != 0) {
      const float mn = raise ? bmax : m;
      const float alpha = raise ? fast_exp2(m - mn) : 1.f;  // 0 on the row's first raise
      l *= alpha;
      m = mn;
      static_for<0, G>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        const float a = row_bcast<g>(alpha);
#pragma unroll
        for (int h = 0; h < CPL; ++h) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][h][e] *= a;
        }
      });
    }
    const float ms = m == neg_inf() ? 0.f : m;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = fast_exp2(s[r] - ms);  // now p
    l += (s[0] + s[1]) + (s[2] + s[3]);
    static_for<0, G>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        float pj;
        if constexpr (TPL == 4) {
          pj = row_bcast<g>(s[j]);
        } else {  // two tokens per lane: tokens tsub + j of the row
          const float lo = row_bcast<g>(s[j]);
          const float hi = row_bcast<g>(s[2 + j]);
          pj = tsub != 0 ? hi : lo;
        }
#pragma unroll
        for (int h = 0; h < CPL; ++h) axpy8<T>(pj, vb[slot][j][h], acc[g][h]);
      }
    });
  };

  // ---- main loop: two blocks per iteration (V slots ping-pong); loads in
  // the steady-state body are unconditional so the wait counts only cover
  // the block being reduced
  if (nw > 0) {
    float s[4];
    int k = 0;
    load_block(0, block_base(0));
    for (; k + 2 < nw; k += 2) {
      block_scores(block_tokens(k), s);
      load_block(1, block_base(k + 1));
      block_update(0, block_tokens(k), s);
      block_scores(block_tokens(k + 1), s);
      load_block(0, block_base(k + 2));
      block_update(1, block_tokens(k + 1), s);
    }
    block_scores(block_tokens(k), s);
    if (k + 1 < nw) {
      load_block(1, block_base(k + 1));
      block_update(0, block_tokens(k), s);
      block_scores(block_tokens(k + 1), s);
      block_update(1, block_tokens(k + 1), s);
    } else {
      block_update(0, block_tokens(k), s);
    }
  }

  // ---- merge the four rows into this wave's state. M: max over the rows of
  // head hg's running max; each row's sum and V slices are scaled by
  // exp2(m_row - M) and summed over the rows (and, for D = 64, over the two
  // token halves of a row).
  float M = fmaxf(m, shfl_xor_f32(m, 16));
  M = fmaxf(M, shfl_xor_f32(M, 32));
  const float Ms = M == neg_inf() ? 0.f : M;
  float lt = l * fast_exp2(m - Ms);  // 0 for a row that saw no token
  lt += shfl_xor_f32(lt, 16);
  lt += shfl_xor_f32(lt, 32);
  static_for<0, G>([&](auto gc) {
    constexpr int g = decltype(gc)::value;
    const float w = fast_exp2(row_bcast<g>(m) - row_bcast<g>(Ms));
#pragma unroll
    for (int h = 0; h < CPL; ++h) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = acc[g][h][e] * w;
#pragma unroll
      for (int x = VM::LPS; x < kWave; x <<= 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += shfl_xor_f32(o[e], x);
      }
      if (lane < VM::LPS) {
        float4* dst = reinterpret_cast<float4*>(&ws.acc[wave][g][(vchunk + 16 * h) * 8]);
        dst[0] = make_float4(o[0], o[1], o[2], o[3]);
        dst[1] = make_float4(o[4], o[5], o[6], o[7]);
      }
    }
  });
  if (lane < G) {  // lane g < G holds head g
    ws.m[wave][lane] = M;
    ws.l[wave][lane] = lt;
  }
  if (lane == 0) ws.bad[wave] = wb.bad ? 1 : 0;
  __syncthreads();
  if (wave != 0) return;
  finish_task<T, D, G>(p, t, ws, lane);
}

// Combines the split partials of every (sequence, head) whose sequence used
// more than one split: the N-way form of the log-sum-exp merge. One thread
// per 4 output elements; each thread reads the row's split LSEs (L1-shared
// with its neighbours) and its slice of every split's partial.
__global__ __launch_bounds__(256) void combine_splits_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ lens, int32_t n, int32_t H, int32_t D, int32_t S,
    int32_t split_blocks, int32_t block_size, int32_t bt_width, void* out, int64_t out_ss,
    int64_t out_sh, int32_t out_dt, float* lse, int64_t lse_sh) {
  const int per_row = D / 4;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (int64_t)n * H * per_row) return;
  const int c = (int)(tid % per_row);
  const int64_t pair = tid / per_row;
  const int i = (int)(pair / H);
  const int h = (int)(pair % H);
  const int L = lens[i];
  if (L > bt_width * block_size) return;  // range error: already NaN
  const int nb = L > 0 ? (L + block_size - 1) / block_size : 0;
  const int ns = (nb + split_blocks - 1) / split_blocks;
  if (ns <= 1) return;  // written directly by the partial kernel
  const float* pl = part_lse + pair * S;
  float M = neg_inf();
  for (int s = 0; s < ns; ++s) M = fmaxf(M, pl[s]);
  const float Ms = M == neg_inf() ? 0.f : M;
  float wsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4* po = reinterpret_cast<const float4*>(part_o + pair * S * D) + c;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) {
    const float w = __expf(pl[s] - Ms);
    const float4 x = po[(int64_t)s * (D / 4)];
    wsum += w;
    acc.x += w * x.x;
    acc.y += w * x.y;
    acc.z += w * x.z;
    acc.w += w * x.w;
  }
  const float inv = 1.f / wsum;
  const int64_t ob = (int64_t)i * out_ss + (int64_t)h * out_sh + c * 4;
  store_elem(out, ob + 0, out_dt, acc.x * inv);
  store_elem(out, ob + 1, out_dt, acc.y * inv);
  store_elem(out, ob + 2, out_dt, acc.z * inv);
  store_elem(out, ob + 3, out_dt, acc.w * inv);
  if (c == 0) lse[(int64_t)h * lse_sh + i] = Ms + __logf(wsum);
}

// Generic kernel: any head_size, block_size, group size and dtype (including
// fp32 KV). One wavefront per (sequence, query head); each lane owns
// elements d = lane + 64k. Correct for every layout, not tuned.
__global__ __launch_bounds__(kWave) void decode_generic_kernel(
    const void* q, int64_t q_ss, int64_t q_sh, const void* k, const void* v,
    int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t num_blocks,
    const int32_t* bt, int64_t bt_stride, int32_t bt_width, const int32_t* lens,
    int32_t n, int32_t H, int32_t KVH, int32_t D, int32_t BS, float scale,
    int32_t dt, void* out, int64_t out_ss, int64_t out_sh, int32_t out_dt,
    float* lse, int64_t lse_sh) {
  constexpr int kMaxPerLane = 8;  // D <= 512
  const int lane = threadIdx.x;
  const int i = blockIdx.x / H;
  const int h = blockIdx.x % H;
  const int kh = h / (H / KVH);
  const int L = lens[i];
  const int64_t obase = (int64_t)i * out_ss + (int64_t)h * out_sh;
  if (L <= 0 || L > bt_width * BS || num_blocks <= 0) {
    const float fill = L <= 0 ? 0.f : qnan();
    for (int d = lane; d < D; d += kWave) store_elem(out, obase + d, out_dt, fill);
    if (lane == 0) lse[(int64_t)h * lse_sh + i] = L <= 0 ? neg_inf() : qnan();
    return;
  }
  float qv[kMaxPerLane], acc[kMaxPerLane];
  const int64_t qbase = (int64_t)i * q_ss + (int64_t)h * q_sh;
#pragma unroll
  for (int r = 0; r < kMaxPerLane; ++r) {
    const int d = lane + r * kWave;
    qv[r] = d < D ? load_elem(q, qbase + d, dt) * scale : 0.f;
    acc[r] = 0.f;
  }
  float mrun = neg_inf(), lrun = 0.f;
  bool bad = false;
  for (int t = 0; t < L; ++t) {
    int64_t bid = bt[(int64_t)i * bt_stride + t / BS];
    const bool ok = bid >= 0 && bid < num_blocks;
    bad |= !ok;
    bid = ok ? bid : 0;
    const int64_t base = bid * kv_sb + (int64_t)kh * kv_sh + (int64_t)(t % BS) * kv_st;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < kMaxPerLane; ++r) {
      const int d = lane + r * kWave;
      if (d < D) s += qv[r] * load_elem(k, base + d, dt);
    }
    s = wave_sum(s);
    const float mn = fmaxf(mrun, s);
    const float alpha = __expf(mrun - mn);
    const float pt = __expf(s - mn);
    lrun = lrun * alpha + pt;
#pragma unroll
    for (int r = 0; r < kMaxPerLane; ++r) {
      const int d = lane + r * kWave;
      if (d < D) acc[r] = acc[r] * alpha + pt * load_elem(v, base + d, dt);
    }
    mrun = mn;
  }
  const float inv = 1.f / lrun;
#pragma unroll
  for (int r = 0; r < kMaxPerLane; ++r) {
    const int d = lane + r * kWave;
    if (d < D) store_elem(out, obase + d, out_dt, bad ? qnan() : acc[r] * inv);
  }
  if (lane == 0) lse[(int64_t)h * lse_sh + i] = bad ? qnan() : mrun + __logf(lrun);
}

// FD_SPLIT_BLOCKS=<n> forces n blocks per task (tuning and tests).
int split_blocks_override() {
  const char* e = getenv("FD_SPLIT_BLOCKS");
  return e ? atoi(e) : 0;
}

// FD_DECODE_KERNEL=valu keeps grouped-query calls on the VALU kernel
// (comparison and tests); the matrix-core kernel is the default for G >= 4.
bool valu_forced() {
  const char* e = getenv("FD_DECODE_KERNEL");
  return e != nullptr && strcmp(e, "valu") == 0;
}

// Dynamic LDS that leaves room for at most two workgroups of `kernel` per CU
// (the reservation is never touched), or 0 when the kernel's own LDS already
// keeps it there or the reservation would not fit one workgroup's limit.
// Measured on MI355X: with tasks of 32+ blocks, two workgroups per CU (8
// waves, one block in flight each) already saturate HBM, and fewer, faster
// workgroups shorten the drain at the end of the grid (+1 to +6 % over the
// natural 3-4 per CU); short tasks want the extra workgroups to hide their
// start-up latency, so they are left uncapped.
// `cache` holds the result + 1 per device (0 = not computed yet).
unsigned two_per_cu_lds(const void* kernel, std::atomic<int>* cache) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return (unsigned)(v - 1);
  int per_cu = 0, per_wg = 0;
  hipFuncAttributes fa{};
  v = 0;
  if (hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
          hipSuccess &&
      hipDeviceGetAttribute(&per_wg, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) ==
          hipSuccess &&
      hipFuncGetAttributes(&fa, kernel) == hipSuccess) {
    const int stat = (int)fa.sharedSizeBytes;
    const int need = per_cu / 3 + 1024;  // more than a third of the CU: two fit, three do not
    if (need > stat && need <= per_wg) v = need - stat;
  }
  cache[dev].store(v + 1, std::memory_order_relaxed);
  return (unsigned)v;
}

template <typename T, int D, int G>
hipError_t launch_tiled(const TiledParams& tp, unsigned tasks, const SplitPlan& sp,
                        hipStream_t s) {
  if constexpr (G >= 4) {
    if (sp.mfma) {
      static std::atomic<int> cache[kMaxDevices] = {};
      const void* k = reinterpret_cast<const void*>(&decode_mfma_kernel<T, D, G>);
      const unsigned lds = sp.cap_occupancy ? two_per_cu_lds(k, cache) : 0;
      hipLaunchKernelGGL((decode_mfma_kernel<T, D, G>), dim3(tasks),
                         dim3(kWave * kWavesPerTask), lds, s, tp);
      return hipGetLastError();
    }
  }
  static std::atomic<int> cache[kMaxDevices] = {};
  const void* k = reinterpret_cast<const void*>(&decode_tiled_kernel<T, D, G>);
  const unsigned lds = sp.cap_occupancy ? two_per_cu_lds(k, cache) : 0;
  hipLaunchKernelGGL((decode_tiled_kernel<T, D, G>), dim3(tasks), dim3(kWave * kWavesPerTask),
                     lds, s, tp);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dispatch_g(const TiledParams& tp, unsigned tasks, int G, const SplitPlan& sp,
                      hipStream_t s) {
  switch (G) {
    case 1: return launch_tiled<T, D, 1>(tp, tasks, sp, s);
    case 2: return launch_tiled<T, D, 2>(tp, tasks, sp, s);
    case 4: return launch_tiled<T, D, 4>(tp, tasks, sp, s);
    case 8: return launch_tiled<T, D, 8>(tp, tasks, sp, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t dispatch_d(const TiledParams& tp, unsigned tasks, int D, int G, const SplitPlan& sp,
                      hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<T, 64>(tp, tasks, G, sp, s);
    case 128: return dispatch_g<T, 128>(tp, tasks, G, sp, s);
    case 256: return dispatch_g<T, 256>(tp, tasks, G, sp, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

SplitPlan plan_decode(int32_t n, int32_t H, int32_t KVH, int32_t D, int32_t BS,
                      int32_t bt_width, int32_t kv_dtype, bool aligned) {
  SplitPlan sp{};
  const int G = KVH > 0 ? H / KVH : 0;
  sp.fast = aligned && BS == kTileTokens && (D == 64 || D == 128 || D == 256) &&
            (G == 1 || G == 2 || G == 4 || G == 8) &&
            (kv_dtype == FD_F16 || kv_dtype == FD_BF16);
  if (!sp.fast) {
    sp.split_blocks = bt_width > 0 ? bt_width : 1;
    sp.max_splits = 1;
    return sp;
  }
  sp.mfma = G >= 4 && !valu_forced();
  int sb = split_blocks_override();
  if (sb > kMaxSplitBlocks) sb = kMaxSplitBlocks;  // 64 block ids per wave
  if (sb <= 0) {
    // Tasks as long as possible (up to 64 blocks per wave: whole rows of up
    // to 4096 tokens) while the batch still supplies >= 2048 workgroups (8
    // per CU); shorter tasks otherwise, down to 4 blocks per wave. Each task
    // pays a start-up latency chain (row, table, first K/V) of a few
    // microseconds, so fewer, longer tasks win once the GPU is full.
    const int64_t pairs = (int64_t)n * KVH;
    sb = kMaxSplitBlocks;
    while (sb > 16 && pairs * ((bt_width + sb - 1) / sb) < 2048) sb /= 2;
  }
  sp.split_blocks = sb;
  sp.max_splits = bt_width > 0 ? (bt_width + sb - 1) / sb : 1;
  const char* cap = getenv("FD_WG_CAP");  // FD_WG_CAP=0: natural occupancy (tuning)
  sp.cap_occupancy = sb >= 32 && !(cap != nullptr && strcmp(cap, "0") == 0);
  return sp;
}

size_t decode_workspace_bytes(const SplitPlan& sp, int32_t n, int32_t H, int32_t D) {
  if (sp.max_splits <= 1) return 0;
  const size_t parts = (size_t)n * H * sp.max_splits;
  return parts * D * sizeof(float) + parts * sizeof(float) + 256;
}

int launch_decode(const DecodeArgs& a, const SplitPlan& sp, hipStream_t s) {
  if (a.n == 0) return FD_OK;
  if (!sp.fast) {
    hipLaunchKernelGGL(decode_generic_kernel, dim3((unsigned)a.n * a.H), dim3(kWave), 0, s,
                       a.q, a.q_ss, a.q_sh, a.k, a.v, a.kv_sb, a.kv_sh, a.kv_st,
                       a.num_blocks, a.bt, a.bt_stride, a.bt_width, a.lens, a.n, a.H,
                       a.KVH, a.D, a.BS, a.scale, a.kv_dtype, a.out, a.out_ss,
                       a.out_sh, a.out_dtype, a.lse, a.lse_sh);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? FD_OK : hip_error(e, "decode_generic_kernel launch");
  }
  TiledParams tp{};
  tp.q = static_cast<const uint16_t*>(a.q);
  tp.q_ss = a.q_ss;
  tp.q_sh = a.q_sh;
  tp.k = static_cast<const uint16_t*>(a.k);
  tp.v = static_cast<const uint16_t*>(a.v);
  tp.kv_sb = a.kv_sb;
  tp.kv_sh = a.kv_sh;
  tp.kv_st = a.kv_st;
  tp.num_blocks = a.num_blocks;
  tp.run_bytes = (uint32_t)(((int64_t)(kTileTokens - 1) * a.kv_st + a.D) * 2);
  tp.bt = a.bt;
  tp.bt_stride = a.bt_stride;
  tp.bt_width = a.bt_width;
  tp.lens = a.lens;
  tp.order = a.order;
  tp.n = a.n;
  tp.H = a.H;
  tp.KVH = a.KVH;
  tp.scale_log2 = a.scale * kLog2e;
  tp.out = a.out;
  tp.out_ss = a.out_ss;
  tp.out_sh = a.out_sh;
  tp.out_f32 = a.out_dtype == FD_F32;
  tp.lse = a.lse;
  tp.lse_sh = a.lse_sh;
  tp.S = sp.max_splits;
  tp.split_blocks = sp.split_blocks;
  const size_t parts = (size_t)a.n * a.H * sp.max_splits;
  if (sp.max_splits > 1) {
    char* ws = static_cast<char*>(a.workspace);
    tp.part_o = reinterpret_cast<float*>(ws);
    tp.part_lse = reinterpret_cast<float*>(ws + parts * a.D * sizeof(float));
  }
  const int64_t tasks = (int64_t)a.n * a.KVH * sp.max_splits;
  if (tasks > INT32_MAX) return set_error(FD_ERR_UNSUPPORTED, "decode: too many tasks");
  const int G = a.H / a.KVH;
  hipError_t e = a.kv_dtype == FD_F16
                    ? dispatch_d<F16>(tp, (unsigned)tasks, a.D, G, sp, s)
                    : dispatch_d<BF16>(tp, (unsigned)tasks, a.D, G, sp, s);
  if (e != hipSuccess) return hip_error(e, "decode_tiled_kernel launch");
  if (sp.max_splits > 1) {
    const int64_t threads = (int64_t)a.n * a.H * (a.D / 4);
    hipLaunchKernelGGL(combine_splits_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, s, tp.part_o, tp.part_lse, a.lens, a.n, a.H, a.D, sp.max_splits,
                       sp.split_blocks, kTileTokens, a.bt_width, a.out, a.out_ss, a.out_sh,
                       a.out_dtype, a.lse, a.lse_sh);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "combine_splits_kernel launch");
  }
  return FD_OK;
}

}  // namespace fd
