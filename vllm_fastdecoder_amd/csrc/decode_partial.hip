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
#include "fd_common.h"

namespace fd {

namespace {

constexpr int kTileTokens = 16;         // tokens per block in the tiled kernel
constexpr int kWavesPerTask = 4;        // wavefronts sharing one task
constexpr int kMaxWaveBlocks = kWave;   // a wave's block ids of a task fit one VGPR
constexpr int kMaxSplitBlocks = kWavesPerTask * kMaxWaveBlocks;

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

__device__ __forceinline__ Vec8 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kKvLoadPolicy);
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

// Tiled kernel: block_size == 16, D in {64, 128, 256}, G in {1, 2, 4, 8},
// 16-bit KV, every stride a multiple of 8 elements and 16-byte aligned bases.
// One workgroup (4 waves) per task; grid = n * KVH * S tasks.
template <typename T, int D, int G>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_tiled_kernel(TiledParams p) {
  constexpr int LPT = D / 8;                // lanes per token row
  constexpr int TPW = kWave / LPT;          // token rows per load instruction
  constexpr int STEPS = kTileTokens / TPW;  // loads per block per lane

  // per-wave softmax states for the cross-wave merge (log2-domain max, sum,
  // unnormalised accumulator)
  __shared__ float s_acc[kWavesPerTask][G][D];
  __shared__ float s_m[kWavesPerTask][G];
  __shared__ float s_l[kWavesPerTask][G];
  __shared__ int s_bad[kWavesPerTask];

  const int lane = threadIdx.x & (kWave - 1);
  // The wave index is uniform across the wave; readfirstlane keeps it (and all
  // indexing derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int task = blockIdx.x;
  // task -> (kv head fastest, then split, then sequence)
  const int kh = task % p.KVH;
  const int rest = task / p.KVH;
  const int split = rest % p.S;
  int i = rest / p.S;
  if (p.order != nullptr) {
    // the caller's processing order (e.g. longest rows first, so the last
    // workgroups dispatched are short ones); an entry outside [0, n) is skipped
    i = p.order[i];
    if ((unsigned)i >= (unsigned)p.n) return;
  }

  const int row = lane / LPT;    // which token of each load this lane owns
  const int chunk = lane % LPT;  // which 8-element slice of the row

  const int L = p.lens[i];
  const int nb = L > 0 ? (L + kTileTokens - 1) / kTileTokens : 0;
  const int b_begin = split * p.split_blocks;
  if (split > 0 && b_begin >= nb) return;  // nothing left for this split (whole group)
  const int b_end = min(nb, b_begin + p.split_blocks);
  const int nsplit = nb > 0 ? (nb + p.split_blocks - 1) / p.split_blocks : 1;
  const bool range_bad = L > p.bt_width * kTileTokens;

  // ---- empty row or bad length: split 0, wave 0 writes the final result
  if (nb == 0 || range_bad) {
    if (split > 0 || wave > 0) return;
    if (lane < LPT) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int h = kh * G + g;
        float o[8];
        const float fill = range_bad ? qnan() : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fill;
        store8<T>(p.out, (int64_t)i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8, p.out_f32, o);
        if (lane == 0) p.lse[(int64_t)h * p.lse_sh + i] = range_bad ? qnan() : neg_inf();
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

  // This wave's blocks are b_begin + wave + 4k. Their ids are read once, one
  // per lane (at most 64), range-checked together and picked with v_readlane.
  const int first = b_begin + wave;
  const int nw = first < b_end ? (b_end - first + kWavesPerTask - 1) / kWavesPerTask : 0;
  int my_bid = lane < nw ? p.bt[(int64_t)i * p.bt_stride + first + kWavesPerTask * lane] : 0;
  const bool my_bad = lane < nw && (my_bid < 0 || (int64_t)my_bid >= p.num_blocks);
  const bool bad_block = __ballot(my_bad) != 0;
  my_bid = my_bad ? 0 : my_bid;  // keep every read inside the cache

  // Element offset of this wave's k-th block for this kv head; wave-uniform.
  auto block_base = [&](int k) -> int64_t {
    const int bid = __builtin_amdgcn_readlane(my_bid, k);
    return (int64_t)bid * p.kv_sb + head_off;
  };
  // Valid tokens of this wave's k-th block (< 16 only for the row's last block).
  auto block_tokens = [&](int k) -> int {
    return min(kTileTokens, L - (first + kWavesPerTask * k) * kTileTokens);
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
      float4* dst = reinterpret_cast<float4*>(&s_acc[wave][g][chunk * 8]);
      dst[0] = make_float4(o[0], o[1], o[2], o[3]);
      dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (lane == 0) {
      s_m[wave][g] = M;
      s_l[wave][g] = lt;
    }
  }
  if (lane == 0) s_bad[wave] = bad_block ? 1 : 0;
  __syncthreads();
  if (wave != 0) return;

  // ---- wave 0: merge the waves' states and write the final result or this
  // split's partial
  bool bad = false;
#pragma unroll
  for (int w = 0; w < kWavesPerTask; ++w) bad |= s_bad[w] != 0;
  const bool write_final = nsplit == 1;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kWavesPerTask; ++w) M = fmaxf(M, s_m[w][g]);
    const float Ms = M == neg_inf() ? 0.f : M;
    float lt = 0.f;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerTask; ++w) {
      const float sc = fast_exp2(s_m[w][g] - Ms);  // 0 for a wave without blocks
      lt += sc * s_l[w][g];
      if (lane < LPT) {
        const float4* src = reinterpret_cast<const float4*>(&s_acc[w][g][chunk * 8]);
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
    const int h = kh * G + g;
    if (lane < LPT) {
      if (write_final) {
        store8<T>(p.out, (int64_t)i * p.out_ss + (int64_t)h * p.out_sh + chunk * 8, p.out_f32, o);
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

template <typename T, int D, int G>
hipError_t launch_tiled(const TiledParams& tp, unsigned tasks, hipStream_t s) {
  hipLaunchKernelGGL((decode_tiled_kernel<T, D, G>), dim3(tasks), dim3(kWave * kWavesPerTask),
                     0, s, tp);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dispatch_g(const TiledParams& tp, unsigned tasks, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_tiled<T, D, 1>(tp, tasks, s);
    case 2: return launch_tiled<T, D, 2>(tp, tasks, s);
    case 4: return launch_tiled<T, D, 4>(tp, tasks, s);
    case 8: return launch_tiled<T, D, 8>(tp, tasks, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t dispatch_d(const TiledParams& tp, unsigned tasks, int D, int G, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<T, 64>(tp, tasks, G, s);
    case 128: return dispatch_g<T, 128>(tp, tasks, G, s);
    case 256: return dispatch_g<T, 256>(tp, tasks, G, s);
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
  if (sb > kMaxSplitBlocks) sb = kMaxSplitBlocks;  // 64 block ids per wave
  if (sb <= 0) {
    // Whole rows per workgroup (32 blocks per wave) while the batch alone
    // supplies >= 2048 workgroups (8 per CU); shorter tasks otherwise, down
    // to 4 blocks per wave.
    const int64_t pairs = (int64_t)n * KVH;
    sb = 128;
    while (sb > 16 && pairs * ((bt_width + sb - 1) / sb) < 2048) sb /= 2;
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
  hipError_t e = a.kv_dtype == FD_F16 ? dispatch_d<F16>(tp, (unsigned)tasks, a.D, G, s)
                                      : dispatch_d<BF16>(tp, (unsigned)tasks, a.D, G, s);
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
