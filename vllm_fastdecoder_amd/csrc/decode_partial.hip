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
//   * one wavefront task = (sequence, kv head, range of `split_blocks`
//     blocks); four independent tasks share a 256-thread workgroup so a CU
//     can hold its full 32 waves;
//   * a block of 16 tokens is read as 16-byte vector loads: a token row of
//     D elements is spread over LPT = D/8 lanes, so one load instruction moves
//     64/LPT whole rows (1 KiB for D = 128) and the wave's lanes form
//     TPW = 64/LPT "rows" that each own a token of every load;
//   * the next block's K and V are in flight (register double buffer) while
//     the current block is reduced;
//   * q.k: v_dot2_f32_{f16,bf16} on packed pairs, then a DPP butterfly over
//     the LPT lanes of a token (fp32 throughout);
//   * online softmax in the exp2 domain, kept independently per lane-row
//     (no cross-row traffic in the main loop), rows and splits are merged once
//     at the end with the same log-sum-exp rule as the tier merge;
//   * the G = H/KVH query heads of a kv head share every K/V load.
// Splits of one (sequence, head) are combined by a second small kernel.
#include "fd_common.h"

namespace fd {

namespace {

constexpr int kTileTokens = 16;   // tokens per block in the tiled kernel
constexpr int kTasksPerGroup = 4; // independent wavefront tasks per workgroup
constexpr int kMaxSplitBlocks = kWave;  // a split's block ids fit one VGPR

struct TiledParams {
  const uint16_t* q;
  int64_t q_ss, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sh, kv_st;
  int64_t num_blocks;
  uint32_t run_bytes;  // extent of one (block, head) run: 15 * kv_st + D elements
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
  int32_t n, H, KVH;
  float scale_log2;  // softmax scale * log2(e)
  void* out;
  int64_t out_ss, out_sh;
  bool out_f32;
  float* lse;
  int64_t lse_sh;
  float* part_o;    // [n, H, S, D] fp32 (normalised partial outputs)
  float* part_lse;  // [n, H, S] fp32 (natural-log LSE of each partial)
  int32_t S;        // max splits per (sequence, head)
  int32_t split_blocks;
  int32_t tasks;    // n * KVH * S
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

__device__ __forceinline__ Vec8 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
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
__device__ __forceinline__ void store8(void* out, int64_t off, bool f32,
                                       const float* o) {
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

// Tiled kernel: block_size == 16, D in {64, 128, 256}, G in {1, 2, 4, 8},
// 16-bit KV, every stride a multiple of 8 elements and 16-byte aligned bases.
template <typename T, int D, int G>
__global__ __launch_bounds__(kWave * kTasksPerGroup) void decode_tiled_kernel(
    TiledParams p) {
  constexpr int LPT = D / 8;              // lanes per token row
  constexpr int TPW = kWave / LPT;        // token rows per load instruction
  constexpr int STEPS = kTileTokens / TPW;  // loads per block per lane

  const int lane = threadIdx.x & (kWave - 1);
  // The wave index is uniform across the wave; readfirstlane puts it (and all
  // task indexing derived from it) in scalar registers, so block-table and
  // length reads become scalar loads and block bases scalar adds.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int task = blockIdx.x * kTasksPerGroup + wave;
  if (task >= p.tasks) return;
  // task -> (kv head fastest, then split, then sequence)
  const int kh = task % p.KVH;
  const int rest = task / p.KVH;
  const int split = rest % p.S;
  const int i = rest / p.S;

  const int row = lane / LPT;  // which token of each load this lane owns
  const int chunk = lane % LPT;  // which 8-element slice of the row

  const int L = p.lens[i];
  const int nb = L > 0 ? (L + kTileTokens - 1) / kTileTokens : 0;
  const int b_begin = split * p.split_blocks;
  if (split > 0 && b_begin >= nb) return;  // nothing left for this split
  const int b_end = min(nb, b_begin + p.split_blocks);
  const int nsplit = nb > 0 ? (nb + p.split_blocks - 1) / p.split_blocks : 1;
  const bool range_bad = L > p.bt_width * kTileTokens;

  // ---- empty row or bad length: split 0 writes the final result directly
  if (nb == 0 || range_bad) {
    if (split > 0) return;
    if (chunk == lane) {  // lanes 0 .. LPT-1 write
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int h = kh * G + g;
        float o[8];
        const float fill = range_bad ? qnan() : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fill;
        store8<T>(p.out, (int64_t)i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8,
                  p.out_f32, o);
        if (chunk == 0) p.lse[(int64_t)h * p.lse_sh + i] = range_bad ? qnan() : neg_inf();
      }
    }
    return;
  }

  // ---- query fragments (unscaled, native precision)
  Vec8 qf[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = kh * G + g;
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
  const int64_t head_off = (int64_t)kh * p.kv_sh;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = neg_inf();
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  // The split's block ids, one per lane (split_blocks <= 64), read once and
  // range-checked together; the loop picks them with v_readlane.
  const int nblk = b_end - b_begin;
  int my_bid = lane < nblk ? p.bt[(int64_t)i * p.bt_stride + b_begin + lane] : 0;
  const bool my_bad = lane < nblk && (my_bid < 0 || (int64_t)my_bid >= p.num_blocks);
  const bool bad_block = __ballot(my_bad) != 0;
  my_bid = my_bad ? 0 : my_bid;  // keep every read inside the cache

  // Element offset of the split's b-th block for this kv head; wave-uniform.
  auto block_base = [&](int b) -> int64_t {
    const int bid = __builtin_amdgcn_readlane(my_bid, b - b_begin);
    return (int64_t)bid * p.kv_sb + head_off;
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
  int b = b_begin;
  load_block(0, block_base(b));
  for (; b + 2 < b_end; b += 2) {
    load_block(1, block_base(b + 1));
    compute_block(0, kTileTokens);  // never the last block of the sequence
    load_block(0, block_base(b + 2));
    compute_block(1, kTileTokens);
  }
  if (b + 1 < b_end) {
    load_block(1, block_base(b + 1));
    compute_block(0, kTileTokens);
    compute_block(1, min(kTileTokens, L - (b + 1) * kTileTokens));
  } else {
    compute_block(0, min(kTileTokens, L - b * kTileTokens));
  }

  // ---- merge the TPW lane-rows of each head, then write
  constexpr int kRowsMask = kWave - LPT;  // xor masks that cross rows
  const bool write_final = nsplit == 1;
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
    (void)kRowsMask;
    const float inv = 1.f / lt;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
    float lse_nat = (M + fast_log2(lt)) * kLn2;
    if (bad_block) {
      lse_nat = qnan();
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = qnan();
    }
    const int h = kh * G + g;
    if (lane < LPT) {
      if (write_final) {
        store8<T>(p.out, (int64_t)i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8,
                  p.out_f32, o);
        if (lane == 0) p.lse[(int64_t)h * p.lse_sh + i] = lse_nat;
      } else {
        const int64_t pidx = ((int64_t)i * p.H + h) * p.S + split;
        store8<T>(p.part_o, pidx * D + chunk * 8, true, o);
        if (lane == 0) p.part_lse[pidx] = lse_nat;
      }
    }
  }
}

// Combines the split partials of every (sequence, head) whose sequence used
// more than one split: the N-way form of the log-sum-exp merge.
__global__ __launch_bounds__(256) void combine_splits_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ lens, int32_t n, int32_t H, int32_t D, int32_t S,
    int32_t split_blocks, int32_t block_size, int32_t bt_width, void* out, int64_t out_ss,
    int64_t out_sh, int32_t out_dt, float* lse, int64_t lse_sh) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= (int64_t)n * H) return;
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
  for (int s = 0; s < ns; ++s) wsum += __expf(pl[s] - Ms);
  const float inv = 1.f / wsum;
  const float* po = part_o + pair * S * D;
  for (int d = lane; d < D; d += kWave) {
    float acc = 0.f;
    for (int s = 0; s < ns; ++s) acc += __expf(pl[s] - Ms) * po[(int64_t)s * D + d];
    store_elem(out, (int64_t)i * out_ss + (int64_t)h * out_sh + d, out_dt, acc * inv);
  }
  if (lane == 0) lse[(int64_t)h * lse_sh + i] = Ms + __logf(wsum);
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

// FD_SPLIT_BLOCKS=<n> forces n blocks per split task (tuning and tests).
int split_blocks_override() {
  const char* e = getenv("FD_SPLIT_BLOCKS");
  return e ? atoi(e) : 0;
}

template <typename T, int D, int G>
hipError_t launch_tiled(const TiledParams& tp, hipStream_t s) {
  const int groups = (tp.tasks + kTasksPerGroup - 1) / kTasksPerGroup;
  hipLaunchKernelGGL((decode_tiled_kernel<T, D, G>), dim3(groups),
                     dim3(kWave * kTasksPerGroup), 0, s, tp);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dispatch_g(const TiledParams& tp, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_tiled<T, D, 1>(tp, s);
    case 2: return launch_tiled<T, D, 2>(tp, s);
    case 4: return launch_tiled<T, D, 4>(tp, s);
    case 8: return launch_tiled<T, D, 8>(tp, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t dispatch_d(const TiledParams& tp, int D, int G, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<T, 64>(tp, G, s);
    case 128: return dispatch_g<T, 128>(tp, G, s);
    case 256: return dispatch_g<T, 256>(tp, G, s);
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
  int sb = split_blocks_override();
  if (sb > kMaxSplitBlocks) sb = kMaxSplitBlocks;  // one block id per lane
  if (sb <= 0) {
    // Enough wavefront tasks to cover every CU several times over, without
    // cutting a sequence into tiny pieces: 8 blocks (128 tokens) per task
    // unless the batch already supplies the parallelism.
    const int64_t pairs = (int64_t)n * KVH;
    sb = 8;
    while (sb < kMaxSplitBlocks && pairs * ((bt_width + 2 * sb - 1) / (2 * sb)) >= 32768) sb *= 2;
  }
  sp.split_blocks = sb;
  sp.max_splits = bt_width > 0 ? (bt_width + sb - 1) / sb : 1;
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
  if (tasks > INT32_MAX / 2) return set_error(FD_ERR_UNSUPPORTED, "decode: too many tasks");
  tp.tasks = (int32_t)tasks;
  const int G = a.H / a.KVH;
  hipError_t e = a.kv_dtype == FD_F16 ? dispatch_d<F16>(tp, a.D, G, s)
                                      : dispatch_d<BF16>(tp, a.D, G, s);
  if (e != hipSuccess) return hip_error(e, "decode_tiled_kernel launch");
  if (sp.max_splits > 1) {
    const int64_t pairs = (int64_t)a.n * a.H;
    hipLaunchKernelGGL(combine_splits_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0,
                       s, tp.part_o, tp.part_lse, a.lens, a.n, a.H, a.D, sp.max_splits,
                       sp.split_blocks, kTileTokens, a.bt_width, a.out, a.out_ss, a.out_sh,
                       a.out_dtype, a.lse, a.lse_sh);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "combine_splits_kernel launch");
  }
  return FD_OK;
}

}  // namespace fd
