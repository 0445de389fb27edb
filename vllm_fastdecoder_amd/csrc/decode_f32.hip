// Tiled decode kernel for fp32 KV caches, the third dtype of the reference's
// host-tier kernel (fastdecode/csrc/cpu_attn.cpp:439-448).
//
// The task decomposition, block-id checks, cross-wave merge, split partials
// and two-tier walk are the 16-bit kernels' (decode_tiled.h). What differs is
// the stream:
//   * a token row of D fp32 values is spread over LPT = D/8 lanes, 32 bytes
//     (two 16-byte loads) per lane, so one pair of load instructions moves
//     64/LPT whole rows (2 KiB at D = 128);
//   * each 16-token block is taken as two 8-token halves: a half holds as
//     many bytes as a whole 16-bit block (8 KiB of K + V at D = 128), so the
//     register double buffer (the next half in flight while the current one
//     is reduced) has the 16-bit kernel's size and bytes in flight;
//   * q.k and P.V are fp32 FMAs; the online softmax runs in the exp2 domain
//     per lane-row, as in decode_valu.hip.
// Tier strides, q strides and the run extents arrive in 16-bit words (twice
// the fp32 element counts), so the shared block-address code is unchanged.
#include "decode_tiled.h"

namespace fd {

namespace {

template <int D, int G, bool TWO, bool KEEP>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_f32_kernel(TiledParams p) {
  constexpr int LPT = D / 8;                // lanes per token row (8 values each)
  constexpr int TPW = kWave / LPT;          // token rows per pair of loads
  constexpr int HALF = kTileTokens / 2;     // tokens per half block
  constexpr int STEPS = HALF / TPW;         // load pairs per half block per lane
  static_assert(STEPS >= 1 && HALF % TPW == 0, "decode_f32_kernel: D in {64, 128, 256}");

  __shared__ WaveStates<D, G> ws;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Task t;
  if (!decode_task<G, TWO>(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<F32, D, G>(p, t, lane);
    return;
  }

  const int row = lane / LPT;    // which token of each load pair this lane owns
  const int chunk = lane % LPT;  // which 8-value slice of the row
  // a head size below the kernel's D: lanes past it hold a zero query and
  // load their token's first slice (in bounds), as in decode_valu.hip
  const bool lane_on = chunk * 8 < p.D;
  const int lchunk = lane_on ? chunk : 0;

  float qf[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane_on) {
      const float4* qp = reinterpret_cast<const float4*>(
          p.q + (int64_t)t.i * p.q_ss + (int64_t)task_head(t, g) * p.q_sh) + 2 * chunk;
      const float4 a = qp[0], b = qp[1];
      qf[g][0] = a.x, qf[g][1] = a.y, qf[g][2] = a.z, qf[g][3] = a.w;
      qf[g][4] = b.x, qf[g][5] = b.y, qf[g][6] = b.z, qf[g][7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[g][e] = 0.f;
    }
  }

  // Byte offsets inside one (block, head) run, per tier: this lane's first
  // 16 bytes; + 16 for its second; + j * step for load pair j; + half for
  // the block's second half (st in 16-bit words).
  const uint32_t off0 = (uint32_t)(((int64_t)row * p.tier[0].st + lchunk * 16) * 2);
  const uint32_t step0 = (uint32_t)((int64_t)TPW * p.tier[0].st * 2);
  const uint32_t half0 = (uint32_t)((int64_t)HALF * p.tier[0].st * 2);
  uint32_t off1 = 0, step1 = 0, half1 = 0;
  if constexpr (TWO) {
    off1 = (uint32_t)(((int64_t)row * p.tier[1].st + lchunk * 16) * 2);
    step1 = (uint32_t)((int64_t)TPW * p.tier[1].st * 2);
    half1 = (uint32_t)((int64_t)HALF * p.tier[1].st * 2);
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
  const int nu = 2 * wb.nw;  // half blocks of this wave: u = 2k + (second half)

  // head sizes below 128 run in the 128 build read with the default cache
  // policy (kKvLoadKeep). Measured (n = 128, MHA, L in [256, 2048]):
  // D = 72 / 80 / 96 / 112 at 5.95 / 5.91 / 5.87 / 5.84 TB/s against
  // 4.17 / 4.27 / 5.47 / 4.65 non-temporal; D = 128 reads 6.25 either way.
  constexpr int POL = KEEP ? kKvLoadKeep : kKvLoadPolicy;
  Vec8 kb[2][STEPS][2], vb[2][STEPS][2];
  auto load_half = [&](int slot, int u) {
    const BlockSrc src = block_src<TWO>(p, wb, t.kh, u >> 1);
    const uint32_t off = src.t1 ? off1 : off0;
    const uint32_t step = src.t1 ? step1 : step0;
    const uint32_t base = (u & 1) ? (src.t1 ? half1 : half0) : 0u;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      kb[slot][j][0] = buffer_ld16<POL>(src.k, off, base + j * step);
      kb[slot][j][1] = buffer_ld16<POL>(src.k, off + 16, base + j * step);
    }
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      vb[slot][j][0] = buffer_ld16<POL>(src.v, off, base + j * step);
      vb[slot][j][1] = buffer_ld16<POL>(src.v, off + 16, base + j * step);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Reduces the resident half block u (in `slot`); fewer than 8 valid tokens
  // only in a tier's last block.
  auto compute_half = [&](int slot, int u) {
    const int ntok = block_tokens<TWO>(t, wb.first + wb.stride * (u >> 1)) - HALF * (u & 1);
    if (ntok <= 0) return;  // the empty second half of a short last block
    float s[G][STEPS];
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d = __builtin_fmaf(qf[g][e], __uint_as_float(kb[slot][j][0].w[e]), d);
          d = __builtin_fmaf(qf[g][4 + e], __uint_as_float(kb[slot][j][1].w[e]), d);
        }
        s[g][j] = group_sum<LPT>(d) * p.scale_log2;
      }
    }
    if (ntok < HALF) {
#pragma unroll
      for (int j = 0; j < STEPS; ++j) {
        const bool valid = j * TPW + row < ntok;
#pragma unroll
        for (int g = 0; g < G; ++g) s[g][j] = valid ? s[g][j] : neg_inf();
        if (!valid) {
#pragma unroll
          for (int e = 0; e < 4; ++e) vb[slot][j][0].w[e] = vb[slot][j][1].w[e] = 0u;  // stale V may be NaN
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
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[g][e] = __builtin_fmaf(pj, __uint_as_float(vb[slot][j][0].w[e]), acc[g][e]);
          acc[g][4 + e] = __builtin_fmaf(pj, __uint_as_float(vb[slot][j][1].w[e]), acc[g][4 + e]);
        }
      }
      l[g] = l[g] * alpha + psum;
      m[g] = mn;
    }
  };

  // ---- main loop: two halves (one block) per iteration, ping-ponging the
  // register buffers; loads in the steady-state body are unconditional so
  // the wait counts only cover the half being reduced
  if (nu > 0) {
    int u = 0;
    load_half(0, 0);
    for (; u + 2 < nu; u += 2) {
      load_half(1, u + 1);
      compute_half(0, u);
      load_half(0, u + 2);
      compute_half(1, u + 1);
    }
    load_half(1, u + 1);  // nu is even: the last block's two halves
    compute_half(0, u);
    compute_half(1, u + 1);
  }

  publish_wave_state<D, G>(ws, wave, lane, m, l, acc, wb.bad);
  __syncthreads();
  if (wave != 0) return;
  finish_task<F32, D, G>(p, t, ws, lane);
}

template <int D, int G>
hipError_t launch_dg(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, bool two,
                     hipStream_t s) {
  if constexpr (D == 128) {
    if (tp.D != 128)
      return two ? launch_capped<&decode_f32_kernel<D, G, true, true>>(tp, tasks, sp, s)
                 : launch_capped<&decode_f32_kernel<D, G, false, true>>(tp, tasks, sp, s);
  }
  return two ? launch_capped<&decode_f32_kernel<D, G, true, false>>(tp, tasks, sp, s)
             : launch_capped<&decode_f32_kernel<D, G, false, false>>(tp, tasks, sp, s);
}

template <int D>
hipError_t launch_d(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int G, bool two,
                    hipStream_t s) {
  switch (G) {
    case 1: return launch_dg<D, 1>(tp, tasks, sp, two, s);
    case 2: return launch_dg<D, 2>(tp, tasks, sp, two, s);
    case 4: return launch_dg<D, 4>(tp, tasks, sp, two, s);
    case 8:
      if constexpr (D <= 128) return launch_dg<D, 8>(tp, tasks, sp, two, s);
      break;
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_f32(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int D, int G,
                      bool two_tiers, hipStream_t s) {
  switch (D) {
    case 64: return launch_d<64>(tp, tasks, sp, G, two_tiers, s);
    case 128: return launch_d<128>(tp, tasks, sp, G, two_tiers, s);
    case 256: return launch_d<256>(tp, tasks, sp, G, two_tiers, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fd
