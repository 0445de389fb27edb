// Decode kernel with both products on the matrix cores: CG groups of 16
// query heads of one kv head per task (CG = 1, 2 or 4; larger groups in
// passes of 16 CG), head sizes 32 to 128 in steps of 16 (CG = 4 up to 64).
// The planner gives it grouped-query launches, large MHA launches at D = 128
// (one real column of 16: the contraction is free next to the read, and its
// access pattern reads HBM a little faster there than the VALU kernel's) and,
// with CG > 1, groups of more than 16 heads (multi-query models): each pass
// re-reads the kv head's blocks, so wider tasks cut the bytes read.
//
// Per 16-token block of one kv head and each group of up to 16 of its query
// heads (the "columns"; spare columns repeat the task's last head and are
// never written), the groups sharing the block's K and V registers and its V
// staging:
//   scores  S[16 tokens x 16 columns] = K . Q^T: one v_mfma_f32_16x16x32 per
//           32 dims (the dims of a last step past D zero in both operands),
//           as in decode_mfma.hip; lane l ends with the scores of tokens
//           4R..4R+3 (R = l/16) for column l%16;
//   softmax per column in the exp2 domain: the block max over the 16 tokens
//           (an in-lane max of 4, then across the four 16-lane rows), a
//           running max raised only when a block max passes it by more than
//           kLazyRescale (so p <= 2^8), p = exp2(s - m);
//   P.V     O[16 columns x D] += P . V: one v_mfma_f32_16x16x16 per 16 dims.
//           Its A operand (lane l: row l%16, K = 4R..4R+3) is exactly the
//           lane's p values. P goes in as two 16-bit parts, p_hi = p rounded
//           and p_lo = (p - p_hi) rounded, so the products keep about 16 bits
//           of p (one part alone keeps 8 for bf16, 11 for fp16); fp16 p is
//           scaled by 2^7 first (p <= 2^15) so small weights stay normal.
//           The B operand needs 4 consecutive tokens of one dim per lane:
//           each wave writes its V block row-major to LDS (lane l of load j
//           carries 16-byte chunk 64 j + l of the block, so the loads stay
//           whole at any D) and reads it back with ds_read_b64_tr_b16.
//           That instruction (lane mapping checked on the GPU with an
//           in-bounds probe) gives lane 16g+i the element
//           i%4 of the 64-bit rows addressed by lanes 16g + i/4 + 4k,
//           k = 0..3; so with lane 16g+j addressing V[token 4g + j/4][dims
//           16c + 4(j%4) ..+3], lane 16g+i receives V[tokens 4g..4g+3][dim
//           16c + i], the B operand of dims 16c..16c+15.
// The output tile (lane l: columns 4R..4R+3, dim 16c + l%16) accumulates in
// fp32 over all of the wave's blocks; the waves of the task are merged once
// through LDS with the log-sum-exp rule.
//
// Against decode_mfma.hip (P.V on the VALU, 32*G FMAs per lane per block) the
// vector work per block no longer grows with the group: at G = 8 that kernel
// issues ~1.7x the VALU instructions of G = 4.
#include "decode_tiled.h"

namespace fd {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef s16x4 __attribute__((address_space(3))) * lds_s16x4_ptr;

constexpr int kCols = 16;           // query heads per column group
constexpr float kLazyRescale = 8.f;  // log2 units

template <typename T>
__device__ __forceinline__ f32x4 mfma_qk(const Vec8& a, const Vec8& b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_qk<F16>(const Vec8& a, const Vec8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_qk<BF16>(const Vec8& a, const Vec8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ f32x4 mfma_pv(s16x4 a, s16x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_pv<F16>(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                               __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_pv<BF16>(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// p split into its 16-bit rounding and the rounding of the remainder.
template <typename T>
__device__ __forceinline__ void split16(float x, short& hi, short& lo) {
  const uint16_t h = from_f32(T{}, x);
  hi = (short)h;
  lo = (short)from_f32(T{}, x - lo_f32(T{}, (uint32_t)h));
}

// LDS of one workgroup: the waves' V staging (two slots each) during the
// block loop, then the waves' states for the merge.
template <int D>
struct __align__(16) MmLds {  // 16-byte V rows, float4 merge reads
  static constexpr int kStage = 2 * kWavesPerTask * kTileTokens * D;  // 16-bit elements
  struct Merge {
    float acc[kWavesPerTask][kCols][D];
    float m[kWavesPerTask][kCols];
    float l[kWavesPerTask][kCols];
    int bad[kWavesPerTask];
  };
  union {
    uint16_t stage[kStage];
    Merge merge;
  };
};

template <typename T, int D, int CG, bool TWO>
__global__ __launch_bounds__(kWave * kWavesPerTask) void decode_mm_kernel(TiledParams p) {
  static_assert(D % 16 == 0 && D >= 32 && D <= 128, "decode_mm_kernel: D = 16 m, 32..128");
  static_assert(CG == 1 || CG == 2 || (CG == 4 && D <= 64), "decode_mm_kernel: CG 1, 2, 4");
  constexpr int COLS = kCols * CG;       // query heads per task
  constexpr int KS = (D + 31) / 32;      // scores: 32-dim matrix-core steps (the last
                                         // masked past D when D is not a multiple of 32)
  constexpr int NC = D / 16;             // P.V: 16-dim output chunks
  constexpr int CPT = D / 8;             // V: 16-byte chunks per token row
  constexpr int TC = kTileTokens * CPT;  // V: 16-byte chunks per block
  constexpr int NLD = (TC + kWave - 1) / kWave;  // V: loads per block (lane l of load j
                                                 // takes chunk 64 j + l, if < TC)
  constexpr float kPScale = std::is_same<T, F16>::value ? 128.f : 1.f;
  // K is read in 64-byte column slices, so most lines are read by two loads
  // of the wave; below 128 dims (64 aside) non-temporal lines were often
  // fetched twice. Measured (n = 128, 40/8 heads, bf16, L in [1024, 4096]):
  // the default policy reads D = 32 / 48 / 80 / 96 / 112 at 4.6 / 5.5 / 5.8 /
  // 5.8 / 5.9 TB/s against 3.9 / 3.7 / 4.7 / 5.5 / 5.2 non-temporal, and
  // D = 64 / 128 at 5.6 / 6.0 against 6.1 / 6.2.
  constexpr int POL = (D == 64 || D == 128) ? kKvLoadPolicy : kKvLoadKeep;

  __shared__ MmLds<D> lds;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Task t;
  if (!decode_task<COLS, TWO>(p, t)) return;
  if (t.nb == 0 || t.range_bad) {
    if (t.split == 0 && wave == 0) write_empty<T, D, COLS>(p, t, lane);
    return;
  }

  const int col = lane & 15;  // K: token row of the A operand; scores: column
  const int R = lane >> 4;    // K: dims 8R..+7 of each step; scores: tokens 4R..4R+3
  // K step ks covers dims 8R + 32 ks .. +7 of this lane; past D (the last step
  // when D is not a multiple of 32) both operands are zero
  auto k_dims_on = [&](int ks) { return 8 * R + 32 * ks < D; };

  // B operand of the scores of group g: column col's head, dims 8R + 32*ks .. +7
  Vec8 qb[CG][KS];
#pragma unroll
  for (int g = 0; g < CG; ++g) {
    const uint16_t* qrow =
        p.q + (int64_t)t.i * p.q_ss + (int64_t)task_head(t, kCols * g + col) * p.q_sh + R * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qb[g][ks] = k_dims_on(ks) ? ld16(qrow + 32 * ks) : Vec8{{0u, 0u, 0u, 0u}};
  }
  // V chunk of load j: c = 64 j + lane, token c / CPT, 16-byte slice c % CPT;
  // row-major in LDS it sits at element 8 c. Byte offsets inside one (block,
  // head) run, per tier: K step ks at koff + 64*ks, V load j at voff[j].
  int vtok[NLD];
  const TierParams& t0 = p.tier[0];
  const uint32_t koff0 = (uint32_t)(((int64_t)col * t0.st + R * 8) * 2);
  uint32_t voff0[NLD], voff1[NLD], koff1 = 0;
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int c = kWave * j + lane < TC ? kWave * j + lane : 0;  // spare lanes read chunk 0
    vtok[j] = kWave * j + lane < TC ? c / CPT : kTileTokens;     // and never store it
    voff0[j] = (uint32_t)(((int64_t)(c / CPT) * t0.st + (c % CPT) * 8) * 2);
    voff1[j] = 0;
  }
  if constexpr (TWO) {
    const TierParams& t1 = p.tier[1];
    koff1 = (uint32_t)(((int64_t)col * t1.st + R * 8) * 2);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int c = kWave * j + lane < TC ? kWave * j + lane : 0;
      voff1[j] = (uint32_t)(((int64_t)(c / CPT) * t1.st + (c % CPT) * 8) * 2);
    }
  }

  // This wave's V staging, two slots of [16 tokens][D]; the tr16 read of
  // chunk c by lane 16g+j starts at token 4g + j/4, dim 16c + 4(j%4).
  uint16_t* stage = lds.stage + (wave * 2) * kTileTokens * D;
  const int tr_off = (4 * R + (col >> 2)) * D + 4 * (col & 3);

  // Per group g: m[g], column col's running max (the same in the four rows);
  // l[g], the sum of p over this lane's tokens; acc[g][c], columns
  // 4R..4R+3, dim 16c + col.
  float m[CG], l[CG];
  f32x4 acc[CG][NC];
#pragma unroll
  for (int g = 0; g < CG; ++g) {
    m[g] = neg_inf();
    l[g] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[g][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const WaveBlocks wb = wave_blocks<TWO>(p, t, wave, lane);
  const int nw = wb.nw;
  auto ntok_of = [&](int k) -> int {
    return block_tokens<TWO>(t, wb.first + wb.stride * k);
  };

  // K and V double-buffered in registers: block k+1's loads are issued right
  // after block k's scores and land while block k's softmax and P.V run. (A
  // third slot, two blocks in flight, measured 0.5-4 % slower on most
  // shapes: HBM is already busy and the extra requests only queue.)
  Vec8 kb[2][KS], vb[2][NLD];
  auto load_block = [&](int slot, int k) {
    const BlockSrc src = block_src<TWO>(p, wb, t.kh, k);
    const uint32_t koff = src.t1 ? koff1 : koff0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kb[slot][ks] = buffer_ld16<POL>(src.k, koff, 64 * ks);
#pragma unroll
    for (int j = 0; j < NLD; ++j)
      vb[slot][j] = buffer_ld16<POL>(src.v, src.t1 ? voff1[j] : voff0[j]);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Scores of the K block in `slot` for every group (log2 domain, masked
  // past ntok).
  auto block_scores = [&](int slot, int ntok, float (*s)[4]) {
    f32x4 sv[CG];
#pragma unroll
    for (int g = 0; g < CG; ++g) sv[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // K past D (the next field of the row, or 0 past the run) times a zero
      // q could still be NaN: zero it too
      const Vec8 kv = (32 * (ks + 1) <= D || k_dims_on(ks)) ? kb[slot][ks] : Vec8{{0u, 0u, 0u, 0u}};
#pragma unroll
      for (int g = 0; g < CG; ++g) sv[g] = mfma_qk<T>(kv, qb[g][ks], sv[g]);
    }
#pragma unroll
    for (int g = 0; g < CG; ++g) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[g][r] = sv[g][r] * p.scale_log2;
    }
    // Short blocks (a tier's last) are masked under a branch with one column
    // group, whose full blocks then skip the selects (1-2 % at the
    // grouped-query and MHA shapes). With more groups the masking is done
    // with selects: the compiler's count of the wait states an MFMA result
    // needs before a VALU read falls short across that branch there (paths
    // of 1-5 of the 8 the 16x16x32 MFMA needs were found in the two-group
    // kernels' code, which read stale scores of the second group).
    if (CG == 1 && ntok >= kTileTokens) return;
#pragma unroll
    for (int g = 0; g < CG; ++g) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[g][r] = 4 * R + r < ntok ? s[g][r] : neg_inf();
    }
  };

  // Softmax and P.V of the wave's block k, whose scores are in s and V in
  // vb[slot] (staged through the LDS slot of k's parity).
  auto block_update = [&](int slot, int k, int ntok, float (*s)[4]) {
    uint16_t* st = stage + (k & 1) * kTileTokens * D;
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      if (TC % kWave == 0 || vtok[j] < kTileTokens) {  // a chunk of the block
        Vec8 x = vb[slot][j];
        if (ntok < kTileTokens && vtok[j] >= ntok) x = Vec8{{0u, 0u, 0u, 0u}};  // stale V may be NaN
        *reinterpret_cast<uint4*>(st + 8 * (kWave * j + lane)) =
            make_uint4(x.w[0], x.w[1], x.w[2], x.w[3]);
      }
    }
    s16x4 phi[CG], plo[CG];
#pragma unroll
    for (int g = 0; g < CG; ++g) {
      float bmax = fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3]));
      bmax = xor_max<16>(bmax);
      const bool raise = bmax > m[g] + kLazyRescale;  // false while both are -inf
      if (__ballot(raise) != 0) {
        const float mn = raise ? bmax : m[g];
        const float alpha = raise ? fast_exp2(m[g] - mn) : 1.f;  // 0 on the column's first raise
        l[g] *= alpha;
        m[g] = mn;
        // acc row e holds column 4R + e, whose alpha lane 4R + e holds
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = __shfl(alpha, 4 * R + e, kWave);
#pragma unroll
          for (int c = 0; c < NC; ++c) acc[g][c][e] *= a;
        }
      }
      const float ms = m[g] == neg_inf() ? 0.f : m[g];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = fast_exp2(s[g][r] - ms);
        l[g] += pr;
        short h, lo;
        split16<T>(pr * kPScale, h, lo);
        phi[g][r] = h;
        plo[g][r] = lo;
      }
    }
    // the block's V rows are in LDS before any lane reads them transposed
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const s16x4 bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + tr_off + 16 * c));
#pragma unroll
      for (int g = 0; g < CG; ++g) {
        acc[g][c] = mfma_pv<T>(phi[g], bv, acc[g][c]);
        acc[g][c] = mfma_pv<T>(plo[g], bv, acc[g][c]);
      }
    }
  };

  // ---- main loop: two blocks per iteration (block k in slot k % 2); loads
  // in the steady-state body are unconditional so the wait counts only cover
  // the block being reduced
  if (nw > 0) {
    float s[CG][4];
    int k = 0;
    load_block(0, 0);
    for (; k + 2 < nw; k += 2) {
      block_scores(0, ntok_of(k), s);
      load_block(1, k + 1);
      block_update(0, k, ntok_of(k), s);
      block_scores(1, ntok_of(k + 1), s);
      load_block(0, k + 2);
      block_update(1, k + 1, ntok_of(k + 1), s);
    }
    block_scores(0, ntok_of(k), s);
    if (k + 1 < nw) {
      load_block(1, k + 1);
      block_update(0, k, ntok_of(k), s);
      block_scores(1, ntok_of(k + 1), s);
      block_update(1, k + 1, ntok_of(k + 1), s);
    } else {
      block_update(0, k, ntok_of(k), s);
    }
  }

  // ---- merge, one column group at a time through the LDS (the V staging
  // reused): each wave's column sums over its four rows (they share m) and
  // its output tile, unscaled from the fp16 pre-scale; then wave w finishes
  // columns w, w+4, w+8, w+12 of the group, each over LPC lanes of 8 dims
  constexpr int LPC = D / 8;           // lanes per column
  constexpr int CPP = kWave / LPC;     // columns per pass of the wave
  auto& mg = lds.merge;
  const bool write_final = t.nsplit == 1;
#pragma unroll
  for (int g = 0; g < CG; ++g) {
    const float lt = xor_sum<16>(l[g]);
    __syncthreads();  // the V staging (g = 0) or the previous group's merge is done
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        mg.acc[wave][4 * R + e][16 * c + col] = acc[g][c][e] * (1.f / kPScale);
    }
    if (lane < kCols) {
      mg.m[wave][lane] = m[g];
      mg.l[wave][lane] = lt;
    }
    if (lane == 0) mg.bad[wave] = wb.bad ? 1 : 0;
    __syncthreads();

    bool bad = false;
#pragma unroll
    for (int w = 0; w < kWavesPerTask; ++w) bad |= mg.bad[w] != 0;
#pragma unroll
    for (int pass = 0; pass < (4 + CPP - 1) / CPP; ++pass) {
      const int q = pass * CPP + lane / LPC;  // which of the wave's 4 columns
      if (q >= 4) break;
      const int cc = wave + 4 * q;
      const int d0 = (lane % LPC) * 8;
      float M = mg.m[0][cc];
#pragma unroll
      for (int w = 1; w < kWavesPerTask; ++w) M = fmaxf(M, mg.m[w][cc]);
      const float Ms = M == neg_inf() ? 0.f : M;
      float ltot = 0.f, o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
      for (int w = 0; w < kWavesPerTask; ++w) {
        const float sc = fast_exp2(mg.m[w][cc] - Ms);  // 0 for a wave without blocks
        ltot += sc * mg.l[w][cc];
        const float4 a = *reinterpret_cast<const float4*>(&mg.acc[w][cc][d0]);
        const float4 b = *reinterpret_cast<const float4*>(&mg.acc[w][cc][d0 + 4]);
        o[0] += sc * a.x;
        o[1] += sc * a.y;
        o[2] += sc * a.z;
        o[3] += sc * a.w;
        o[4] += sc * b.x;
        o[5] += sc * b.y;
        o[6] += sc * b.z;
        o[7] += sc * b.w;
      }
      const float inv = 1.f / ltot;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= inv;
      float lse_nat = (M + fast_log2(ltot)) * kLn2;
      if (bad) {
        lse_nat = qnan();
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = qnan();
      }
      const int hc = kCols * g + cc;  // the task's head slot
      if (hc < t.gcount && d0 < p.D) {
        const int h = t.h0 + hc;
        if (write_final) {
          store8<T>(p.out, (int64_t)t.i * p.out_ss + (int64_t)h * p.out_sh + d0, p.out_f32, o);
          if (d0 == 0) p.lse[(int64_t)h * p.lse_sh + t.i] = lse_nat;
        } else {
          const int64_t pidx = ((int64_t)t.i * p.H + h) * p.S + t.split;
          store8<T>(p.part_o, pidx * p.D + d0, true, o);
          if (d0 == 0) p.part_lse[pidx] = lse_nat;
        }
      }
    }
  }
}

template <typename T, int D, int CG>
hipError_t launch_dc(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, bool two,
                     hipStream_t s) {
  return two ? launch_capped<&decode_mm_kernel<T, D, CG, true>>(tp, tasks, sp, s)
             : launch_capped<&decode_mm_kernel<T, D, CG, false>>(tp, tasks, sp, s);
}

template <typename T, int D>
hipError_t launch_d(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int cg, bool two,
                    hipStream_t s) {
  switch (cg) {
    case 1: return launch_dc<T, D, 1>(tp, tasks, sp, two, s);
    case 2: return launch_dc<T, D, 2>(tp, tasks, sp, two, s);
    case 4:
      if constexpr (D <= 64) return launch_dc<T, D, 4>(tp, tasks, sp, two, s);
      break;
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_t(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int D, int cg,
                    bool two, hipStream_t s) {
  switch (D) {
    case 32: return launch_d<T, 32>(tp, tasks, sp, cg, two, s);
    case 48: return launch_d<T, 48>(tp, tasks, sp, cg, two, s);
    case 64: return launch_d<T, 64>(tp, tasks, sp, cg, two, s);
    case 80: return launch_d<T, 80>(tp, tasks, sp, cg, two, s);
    case 96: return launch_d<T, 96>(tp, tasks, sp, cg, two, s);
    case 112: return launch_d<T, 112>(tp, tasks, sp, cg, two, s);
    case 128: return launch_d<T, 128>(tp, tasks, sp, cg, two, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_mm(const TiledParams& tp, unsigned tasks, const SplitPlan& sp, int kv_dtype,
                     int D, bool two_tiers, hipStream_t s) {
  const int cg = sp.kernel_g / kCols;  // column groups of 16 heads per task
  return kv_dtype == FD_F16 ? launch_t<F16>(tp, tasks, sp, D, cg, two_tiers, s)
                            : launch_t<BF16>(tp, tasks, sp, D, cg, two_tiers, s);
}

}  // namespace fd
