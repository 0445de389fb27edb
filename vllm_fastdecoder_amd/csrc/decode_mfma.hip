// Matrix-core tiled decode kernel for grouped-query heads (G = H/KVH in
// {4, 8}): the scores of a block come from v_mfma_f32_16x16x32_{f16,bf16},
// P.V stays on the VALU in fp32.
#include "decode_tiled.h"

namespace fd {

namespace {

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

template <typename T, int D, int G, bool TWO>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_mfma_kernel(TiledParams p) {
  static_assert(G == 4 || G == 8, "decode_mfma_kernel: G must be 4 or 8");
  using VM = VMap<D>;
  constexpr int CPL = VM::CPL, TPL = VM::TPL;
  constexpr int KS = D / 32;  // K: 32-dim matrix-core steps per row

  __shared__ WaveStates<D, G> ws;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Task t;
  if (!decode_task<G, TWO>(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<T, D, G>(p, t, lane);
    return;
  }

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
        p.q + (int64_t)t.i * p.q_ss + (int64_t)task_head(t, hg) * p.q_sh + R * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] = ld16(qrow + 32 * ks);
  }
  // Byte offsets inside one (block, head) run, per tier: K step ks at
  // koff + 64*ks; V token j, slice h at voff + j*vtok + 256*h (scalar parts).
  const TierParams& t0 = p.tier[0];
  const uint32_t koff0 = (uint32_t)(((int64_t)col * t0.st + R * 8) * 2);
  const uint32_t voff0 = (uint32_t)(((int64_t)(4 * R + tsub) * t0.st + vchunk * 8) * 2);
  const uint32_t vtok0 = (uint32_t)(t0.st * 2);
  uint32_t koff1 = 0, voff1 = 0, vtok1 = 0;
  if constexpr (TWO) {
    const TierParams& t1 = p.tier[1];
    koff1 = (uint32_t)(((int64_t)col * t1.st + R * 8) * 2);
    voff1 = (uint32_t)(((int64_t)(4 * R + tsub) * t1.st + vchunk * 8) * 2);
    vtok1 = (uint32_t)(t1.st * 2);
  }

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

  const WaveBlocks wb = wave_blocks<TWO>(p, t, wave, lane);
  const int nw = wb.nw;
  auto ntok_of = [&](int k) -> int {
    return block_tokens<TWO>(t, wb.first + wb.stride * k);
  };

  // K is single-buffered (its registers are free once the block's matrix-core
  // steps have read them), V double-buffered: block k+1's K and V are issued
  // right after block k's scores and land while block k's softmax and P.V run.
  Vec8 kb[KS], vb[2][TPL][CPL];
  auto load_block = [&](int slot, int k) {
    const BlockSrc src = block_src<TWO>(p, wb, t.kh, k);
    const uint32_t koff = src.t1 ? koff1 : koff0;
    const uint32_t voff = src.t1 ? voff1 : voff0;
    const uint32_t vtok = src.t1 ? vtok1 : vtok0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kb[ks] = buffer_ld16(src.k, koff, 64 * ks);
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
#pragma unroll
      for (int h = 0; h < CPL; ++h) vb[slot][j][h] = buffer_ld16(src.v, voff, j * vtok + 256 * h);
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
    load_block(0, 0);
    for (; k + 2 < nw; k += 2) {
      block_scores(ntok_of(k), s);
      load_block(1, k + 1);
      block_update(0, ntok_of(k), s);
      block_scores(ntok_of(k + 1), s);
      load_block(0, k + 2);
      block_update(1, ntok_of(k + 1), s);
    }
    block_scores(ntok_of(k), s);
    if (k + 1 < nw) {
      load_block(1, k + 1);
      block_update(0, ntok_of(k), s);
      block_scores(ntok_of(k + 1), s);
      block_update(1, ntok_of(k + 1), s);
    } else {
      block_update(0, ntok_of(k), s);
    }
  }

  // ---- merge the four rows into this wave's state. M: max over the rows of
  // head hg's running max; each row's sum and V slices are scaled by
  // exp2(m_row - M) and summed over the rows (and, for D = 64, over the two
  // token halves of a row).
  const float M = xor_max<16>(m);
  const float Ms = M == neg_inf() ? 0.f : M;
  const float lt = xor_sum<16>(l * fast_exp2(m - Ms));  // 0 for a row that saw no token
  static_for<0, G>([&](auto gc) {
    constexpr int g = decltype(gc)::value;
    const float w = fast_exp2(row_bcast<g>(m) - row_bcast<g>(Ms));
#pragma unroll
    for (int h = 0; h < CPL; ++h) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = acc[g][h][e] * w;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = xor_sum<VM::LPS>(o[e]);
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

template <typename T, int D, int G>
hipError_t launch_dg(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, bool two,
                     hipStream_t s) {
  return two ? launch_capped<&decode_mfma_kernel<T, D, G, true>>(tp, tasks, sp, s)
             : launch_capped<&decode_mfma_kernel<T, D, G, false>>(tp, tasks, sp, s);
}

template <typename T, int D>
hipError_t launch_d(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int G, bool two,
                    hipStream_t s) {
  switch (G) {
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

hipError_t launch_mfma(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                       int D, int G, bool two_tiers, hipStream_t s) {
  return kv_dtype == FD_F16 ? launch_t<F16>(tp, tasks, sp, D, G, two_tiers, s)
                            : launch_t<BF16>(tp, tasks, sp, D, G, two_tiers, s);
}

}  // namespace fd
