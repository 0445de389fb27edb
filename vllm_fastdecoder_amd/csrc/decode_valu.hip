// VALU tiled decode kernel: MHA and small query groups (G = H/KVH in
// {1, 2, 4, 8}); the grouped-query default for G >= 4 is decode_mfma.hip.
//
//   * a block of 16 tokens is read as 16-byte buffer loads: a token row of D
//     elements is spread over LPT = D/8 lanes, so one load instruction moves
//     64/LPT whole rows (1 KiB for D = 128) and the wave's lanes form
//     TPW = 64/LPT "rows" that each own a token of every load;
//   * q.k: v_dot2_f32_{f16,bf16} on packed pairs, then a DPP butterfly over
//     the LPT lanes of a token (fp32 throughout);
//   * online softmax in the exp2 domain, kept independently per lane-row
//     (no cross-row traffic in the main loop); rows, then waves, are merged at
//     the end with the log-sum-exp rule of the tier merge.
#include "decode_tiled.h"

namespace fd {

namespace {

// block_size == 16, D in {64, 128, 256}, G in {1, 2, 4, 8}, 16-bit KV, every
// stride a multiple of 8 elements and 16-byte aligned bases. One workgroup
// (4 waves) per task; grid = n * KVH * S tasks. TWO: a second KV tier. ADJ:
// tier 0 keeps V right after K in each token row (vLLM's [B, BS, KVH, 2D]
// cache; D = 128 or 256), and each load reads whole K + V runs of its tokens
// (512 B at D = 128) instead of K and V rows in separate loads.
// TL: a measurement build that records p.timeline (fd_paged_decode_timeline);
// the production builds carry none of it.
template <typename T, int D, int G, bool TWO, bool ADJ, bool KEEP, bool TL = false>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_tiled_kernel(TiledParams p) {
  constexpr int LPT = D / 8;                // lanes per token row
  constexpr int TPW = kWave / LPT;          // token rows per load instruction
  constexpr int STEPS = kTileTokens / TPW;  // loads per block per lane
  static_assert(!ADJ || D == 128 || D == 256, "K + V loads pair 16- or 32-lane groups");

  __shared__ WaveStates<D, G> ws;

  const int lane = threadIdx.x & (kWave - 1);
  // The wave index is uniform across the wave; readfirstlane keeps it (and all
  // indexing derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // measurement build only: lane 0 of the wave that reaches a point records
  // the time
  auto stamp = [&](int slot) {
    if constexpr (TL) {
      if (lane == 0) {
        __builtin_amdgcn_sched_barrier(0);
        p.timeline[(int64_t)blockIdx.x * kTimelineSlots + slot] = __builtin_amdgcn_s_memrealtime();
      }
    }
  };
  if (wave == 0) stamp(kTlStart);
  Task t;
  if (!decode_task<G, TWO>(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<T, D, G>(p, t, lane);
    return;
  }
  const int i = t.i;

  const int row = lane / LPT;    // which token of each load this lane owns
  const int chunk = lane % LPT;  // which 8-element slice of the row
  // A head size below the kernel's D (e.g. 96 in the 128 kernel): lanes of
  // the slices past it hold a zero query, load their token's first slice
  // (in bounds, already fetched by the row's first lane) and are never stored.
  const bool lane_on = chunk * 8 < p.D;
  const int lchunk = lane_on ? chunk : 0;

  // ---- query fragments (unscaled, native precision)
  Vec8 qf[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = task_head(t, g);
    qf[g] = lane_on ? ld16(p.q + (int64_t)i * p.q_ss + (int64_t)h * p.q_sh + chunk * 8)
                    : Vec8{{0u, 0u, 0u, 0u}};
  }

  // Byte offset of this lane's 16 bytes inside one (block, head) run, per
  // tier; load step j adds j*step (a scalar operand). The same for every
  // block, so the loop only moves the wave-uniform base held in a scalar
  // buffer resource.
  const uint32_t off0 = (uint32_t)(((int64_t)row * p.tier[0].st + lchunk * 8) * 2);
  const uint32_t step0 = (uint32_t)((int64_t)TPW * p.tier[0].st * 2);
  uint32_t off1 = 0, step1 = 0;
  if constexpr (TWO) {
    off1 = (uint32_t)(((int64_t)row * p.tier[1].st + lchunk * 8) * 2);
    step1 = (uint32_t)((int64_t)TPW * p.tier[1].st * 2);
  }
  // ADJ: lanes [2 LPT c, 2 LPT c + LPT) read K and the next LPT lanes V of
  // token 2c of each load pair's first load, token 2c + 1 in its second
  // (c = lane / (2 LPT)); split_kv then restores the row-per-token layout.
  uint32_t off_kv = 0, st_bytes = 0;
  if constexpr (ADJ) {
    const int half = (lane / LPT) & 1;
    const int c = lane / (2 * LPT);
    off_kv = (uint32_t)(((int64_t)(2 * c) * p.tier[0].st + half * D + lchunk * 8) * 2);
    st_bytes = (uint32_t)(p.tier[0].st * 2);
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = neg_inf();
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  const WaveBlocks wb = wave_blocks<TWO>(p, t, wave, lane);
  const int nw = wb.nw;
  if (wave == 0) stamp(kTlIds);
  // the wave's block k read as K + V runs (tier 0 of an ADJ launch)
  auto adj_block = [&](int k) -> bool { return ADJ && !(TWO && k >= wb.k1); };

  Vec8 kb[2][STEPS], vb[2][STEPS];
  auto load_block = [&](int slot, int k) {
    const BlockSrc src = block_src<TWO>(p, wb, t.kh, k);
    if (adj_block(k)) {
      // global rather than buffer loads here: ~1 % faster for K + V runs
      // (and ~0.3 % slower for separate K and V rows), measured on MI355X;
      // every offset lies inside the block's run (k_run_bytes)
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        kb[slot][j] = global_ld16(src.kp + off_kv + j * step0);
        vb[slot][j] = global_ld16(src.kp + off_kv + j * step0 + st_bytes);
      }
    } else {
      const uint32_t off = src.t1 ? off1 : off0;
      const uint32_t step = src.t1 ? step1 : step0;
      constexpr int POL = KEEP ? kKvLoadKeep : kKvLoadPolicy;
#pragma unroll
      for (int j = 0; j < STEPS; ++j) kb[slot][j] = buffer_ld16<POL>(src.k, off, j * step);
#pragma unroll
      for (int j = 0; j < STEPS; ++j) vb[slot][j] = buffer_ld16<POL>(src.v, off, j * step);
    }
    // keep the prefetch at the top of the reduction that overlaps it
    __builtin_amdgcn_sched_barrier(0);
  };

  // Reduces the wave's resident block k (in `slot`); fewer than 16 valid
  // tokens only in a tier's last block.
  auto compute_block = [&](int slot, int k) {
    const int ntok = block_tokens<TWO>(t, wb.first + wb.stride * k);
    if constexpr (ADJ) {
      if (adj_block(k)) {
#pragma unroll
        for (int j = 0; j < STEPS; ++j) split_kv<D>(kb[slot][j], vb[slot][j]);
      }
    }
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
    load_block(0, 0);
    for (; k + 2 < nw; k += 2) {
      load_block(1, k + 1);
      compute_block(0, k);
      load_block(0, k + 2);
      compute_block(1, k + 1);
    }
    if (k + 1 < nw) {
      load_block(1, k + 1);
      compute_block(0, k);
      compute_block(1, k + 1);
    } else {
      compute_block(0, k);
    }
  }

  stamp(kTlLoop0 + wave);

  // ---- merge the TPW lane-rows of each head into this wave's state, publish it
  publish_wave_state<D, G>(ws, wave, lane, m, l, acc, wb.bad);
  __syncthreads();
  if (wave != 0) return;
  finish_task<T, D, G>(p, t, ws, lane);
  stamp(kTlEnd);
  if constexpr (TL) {
    if (lane == 0)
      p.timeline[(int64_t)blockIdx.x * kTimelineSlots + kTlInfo] =
          (uint64_t)(t.b_end - t.b_begin) | ((uint64_t)wb.stride << 16) |
          ((uint64_t)(uint32_t)t.i << 32);
  }
}

template <typename T, int D, int G, bool ADJ, bool KEEP>
hipError_t launch_mode(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, bool two,
                       hipStream_t s) {
  if (tp.timeline != nullptr)  // a timeline launch (single tier: fd_paged_decode_timeline)
    return two ? hipErrorInvalidValue
               : launch_capped<&decode_tiled_kernel<T, D, G, false, ADJ, KEEP, true>>(tp, tasks,
                                                                                      sp, s);
  return two ? launch_capped<&decode_tiled_kernel<T, D, G, true, ADJ, KEEP>>(tp, tasks, sp, s)
             : launch_capped<&decode_tiled_kernel<T, D, G, false, ADJ, KEEP>>(tp, tasks, sp, s);
}

template <typename T, int D, int G>
hipError_t launch_dg(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, bool two,
                     hipStream_t s) {
  if constexpr (D == 128 || D == 256) {
    if (tp.tier[0].kv_adj) return launch_mode<T, D, G, true, false>(tp, tasks, sp, two, s);
  }
  if constexpr (D == 128) {
    // head sizes run in the 128 build whose heads' K + V runs (4 D bytes in
    // vLLM's layout) are not whole lines: neighbouring heads share lines,
    // and the default policy keeps them for the second reader. Measured
    // (n = 128, MHA, bf16, L in [1024, 4096]): D = 72 / 80 / 112 at 5.56 /
    // 5.79 / 5.64 TB/s against 4.66 / 5.00 / 5.56 non-temporal; D = 96
    // (whole lines) 5.88 against 6.02, so it stays non-temporal.
    if (tp.D % 32 != 0) return launch_mode<T, D, G, false, true>(tp, tasks, sp, two, s);
  }
  return launch_mode<T, D, G, false, false>(tp, tasks, sp, two, s);
}

template <typename T, int D>
hipError_t launch_d(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int G, bool two,
                    hipStream_t s) {
  switch (G) {
    case 1: return launch_dg<T, D, 1>(tp, tasks, sp, two, s);
    case 2: return launch_dg<T, D, 2>(tp, tasks, sp, two, s);
    case 4: return launch_dg<T, D, 4>(tp, tasks, sp, two, s);
    case 8: return launch_dg<T, D, 8>(tp, tasks, sp, two, s);
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_t(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int D, int G,
                    bool two, hipStream_t s) {
  switch (D) {
    case 64: return launch_d<T, 64>(tp, tasks, sp, G, two, s);
    case 128: return launch_d<T, 128>(tp, tasks, sp, G, two, s);
    case 256: return launch_d<T, 256>(tp, tasks, sp, G, two, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_valu(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                       int D, int G, bool two_tiers, hipStream_t s) {
  return kv_dtype == FD_F16 ? launch_t<F16>(tp, tasks, sp, D, G, two_tiers, s)
                            : launch_t<BF16>(tp, tasks, sp, D, G, two_tiers, s);
}

}  // namespace fd
