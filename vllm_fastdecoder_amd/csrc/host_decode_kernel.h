// Body of the host-core decode kernel, compiled once per vector ISA.
//
// host_decode.cpp includes this file several times, each time inside a
// `#pragma GCC target` region and a namespace that defines `V`, the vector
// traits of that ISA (width W, fp32 arithmetic, conversions of W storage
// elements, exp2). No include guard on purpose.
//
// Needs, from the including namespace: V, HostArgs, Scratch, load1,
// f32_to_bf16.

// acc[g][d0 .. d0 + W*CU) = acc * alpha[g] + sum_t s[g][t] * V[t][...] for as
// many whole groups of CU chunks as fit below DW, advancing d; the rest goes
// to groups of CU / 2, and so on. The G*CU accumulators stay in registers.
// PERM (bf16 V): each 2W-element load is split into its even- and
// odd-indexed elements by one shift and one mask, so acc holds every 2W span
// as [even elements, odd elements]; run_heads restores the order at the end.
// The same products in the same order: results equal the plain layout's.
template <int DT, int G, int CU, bool PERM = false>
__attribute__((always_inline)) inline void pv_groups(float* acc, const float* s, const float* alpha, const char* vb,
                      int64_t st, int D, int DW, int BS, int ntok, int& d) {
  using T = typename V::T;
  constexpr int W = V::W;
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  for (; d + W * CU <= DW; d += W * CU) {
    T r[G][CU];
    for (int g = 0; g < G; ++g)
      for (int u = 0; u < CU; ++u)
        r[g][u] = V::mul(V::load(acc + g * D + d + W * u), V::set1(alpha[g]));
    for (int t = 0; t < ntok; ++t) {
      const char* vp = vb + (int64_t)t * st * elt;
      T p[G];
      for (int g = 0; g < G; ++g) p[g] = V::bcast(s + g * BS + t);
      if constexpr (PERM && CU % 2 == 0) {
        for (int u = 0; u < CU; u += 2) {
          T ev, od;
          V::ld_bf16_eo(vp + (d + W * u) * elt, ev, od);
          for (int g = 0; g < G; ++g) {
            r[g][u] = V::fma(p[g], ev, r[g][u]);
            r[g][u + 1] = V::fma(p[g], od, r[g][u + 1]);
          }
        }
      } else {
        for (int u = 0; u < CU; ++u) {
          const T vv = V::template ld<DT>(vp + (d + W * u) * elt);
          for (int g = 0; g < G; ++g) r[g][u] = V::fma(p[g], vv, r[g][u]);
        }
      }
    }
    for (int g = 0; g < G; ++g)
      for (int u = 0; u < CU; ++u) V::store(acc + g * D + d + W * u, r[g][u]);
  }
  if constexpr (CU > 1) pv_groups<DT, G, CU / 2, PERM>(acc, s, alpha, vb, st, D, DW, BS, ntok, d);
}

// s[g * BS] = q[g] . K row at kp for the G heads, with U independent
// accumulator chains per head; every loop over heads and chains is unrolled so
// the G*U accumulators stay in registers.
template <int DT, int G, int U>
__attribute__((always_inline)) inline void score_token(const char* kp, const float* qf,
                                                       const uint16_t* qh, float qs, int D, int DW,
                                                       float* s, int BS) {
  using T = typename V::T;
  constexpr int W = V::W;
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  if constexpr (V::kBf16Dot && DT == FD_BF16) {
    if (D % 32 == 0) {  // bf16 pair dot products on the raw q and K rows
      constexpr int UB = U > 4 ? 4 : U;
      T c[G][UB];
#pragma GCC unroll 64
      for (int j = 0; j < G * UB; ++j) c[j / UB][j % UB] = V::zero();
      int d = 0;
      for (; d + 32 * UB <= D; d += 32 * UB) {
#pragma GCC unroll 16
        for (int u = 0; u < UB; ++u) {
          const auto kv = V::ld_bf16x32(kp + (d + 32 * u) * 2);
#pragma GCC unroll 16
          for (int g = 0; g < G; ++g) c[g][u] = V::dot_bf16(c[g][u], V::ld_bf16x32(qh + g * D + d + 32 * u), kv);
        }
      }
      for (; d < D; d += 32) {
        const auto kv = V::ld_bf16x32(kp + d * 2);
#pragma GCC unroll 16
        for (int g = 0; g < G; ++g) c[g][0] = V::dot_bf16(c[g][0], V::ld_bf16x32(qh + g * D + d), kv);
      }
#pragma GCC unroll 16
      for (int g = 0; g < G; ++g) {
#pragma GCC unroll 16
        for (int step = 1; step < UB; step *= 2)
#pragma GCC unroll 16
          for (int u = 0; u + step < UB; u += 2 * step) c[g][u] = V::add(c[g][u], c[g][u + step]);
        s[g * BS] = V::hsum(c[g][0]) * qs;
      }
      return;
    }
  }
  T c[G][U];
#pragma GCC unroll 64
  for (int j = 0; j < G * U; ++j) c[j / U][j % U] = V::zero();
  int d = 0;
  for (; d + W * U <= DW; d += W * U) {
#pragma GCC unroll 16
    for (int u = 0; u < U; ++u) {
      const T kv = V::template ld<DT>(kp + (d + W * u) * elt);
#pragma GCC unroll 16
      for (int g = 0; g < G; ++g)
        c[g][u] = V::fma(V::load(qf + g * D + d + W * u), kv, c[g][u]);
    }
  }
  for (; d < DW; d += W) {
    const T kv = V::template ld<DT>(kp + d * elt);
#pragma GCC unroll 16
    for (int g = 0; g < G; ++g) c[g][0] = V::fma(V::load(qf + g * D + d), kv, c[g][0]);
  }
#pragma GCC unroll 16
  for (int g = 0; g < G; ++g) {
#pragma GCC unroll 16
    for (int step = 1; step < U; step *= 2)  // pairwise sum of the chains
#pragma GCC unroll 16
      for (int u = 0; u + step < U; u += 2 * step) c[g][u] = V::add(c[g][u], c[g][u + step]);
    float sc = V::hsum(c[g][0]);
    for (int e = DW; e < D; ++e) sc += qf[g * D + e] * load1(kp, e, DT);
    s[g * BS] = sc;
  }
}

// Scores of TT consecutive tokens (rows kp, kp + st_b, ...) for the G heads:
// s[g * BS + t], t < TT. The G * TT dot products are independent accumulator
// chains, reduced four at a time (V::hsum4) instead of one horizontal sum
// per (head, token).
template <int DT, int G, int TT>
__attribute__((always_inline)) inline void score_tokens(const char* kp, int64_t st_b,
                                                        const float* qf, const uint16_t* qh,
                                                        float qs, int D, int DW, float* s,
                                                        int BS) {
  using T = typename V::T;
  constexpr int W = V::W;
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  static_assert((G * TT) % 4 == 0, "sums are reduced four at a time");
  alignas(16) float r[G * TT];
  if constexpr (V::kBf16Dot && DT == FD_BF16) {
    if (D % 32 == 0) {
      T c[G][TT];
#pragma GCC unroll 64
      for (int j = 0; j < G * TT; ++j) c[j / TT][j % TT] = V::zero();
      for (int d = 0; d < D; d += 32) {
        decltype(V::ld_bf16x32(kp)) kv[TT];
#pragma GCC unroll 16
        for (int t = 0; t < TT; ++t) kv[t] = V::ld_bf16x32(kp + t * st_b + d * 2);
#pragma GCC unroll 16
        for (int g = 0; g < G; ++g) {
          const auto qv = V::ld_bf16x32(qh + g * D + d);
#pragma GCC unroll 16
          for (int t = 0; t < TT; ++t) c[g][t] = V::dot_bf16(c[g][t], qv, kv[t]);
        }
      }
#pragma GCC unroll 64
      for (int j = 0; j < G * TT; j += 4)
        V::hsum4(c[j / TT][j % TT], c[(j + 1) / TT][(j + 1) % TT], c[(j + 2) / TT][(j + 2) % TT],
                 c[(j + 3) / TT][(j + 3) % TT], r + j);
#pragma GCC unroll 64
      for (int j = 0; j < G * TT; ++j) s[(j / TT) * BS + j % TT] = r[j] * qs;
      return;
    }
  }
  constexpr int U = G * TT >= 8 ? 1 : 8 / (G * TT);
  T c[G][TT][U];
#pragma GCC unroll 64
  for (int j = 0; j < G * TT * U; ++j) c[j / (TT * U)][(j / U) % TT][j % U] = V::zero();
  int d = 0;
  for (; d + W * U <= DW; d += W * U) {
#pragma GCC unroll 16
    for (int u = 0; u < U; ++u) {
      T kv[TT];
#pragma GCC unroll 16
      for (int t = 0; t < TT; ++t) kv[t] = V::template ld<DT>(kp + t * st_b + (d + W * u) * elt);
#pragma GCC unroll 16
      for (int g = 0; g < G; ++g) {
        const T qv = V::load(qf + g * D + d + W * u);
#pragma GCC unroll 16
        for (int t = 0; t < TT; ++t) c[g][t][u] = V::fma(qv, kv[t], c[g][t][u]);
      }
    }
  }
  for (; d < DW; d += W) {
#pragma GCC unroll 16
    for (int t = 0; t < TT; ++t) {
      const T kv = V::template ld<DT>(kp + t * st_b + d * elt);
#pragma GCC unroll 16
      for (int g = 0; g < G; ++g) c[g][t][0] = V::fma(V::load(qf + g * D + d), kv, c[g][t][0]);
    }
  }
#pragma GCC unroll 16
  for (int g = 0; g < G; ++g)
#pragma GCC unroll 16
    for (int t = 0; t < TT; ++t)
#pragma GCC unroll 16
      for (int step = 1; step < U; step *= 2)
#pragma GCC unroll 16
        for (int u = 0; u + step < U; u += 2 * step) c[g][t][u] = V::add(c[g][t][u], c[g][t][u + step]);
#pragma GCC unroll 64
  for (int j = 0; j < G * TT; j += 4)
    V::hsum4(c[j / TT][j % TT][0], c[(j + 1) / TT][(j + 1) % TT][0],
             c[(j + 2) / TT][(j + 2) % TT][0], c[(j + 3) / TT][(j + 3) % TT][0], r + j);
  for (int j = 0; j < G * TT; ++j) {
    const int g = j / TT, t = j % TT;
    float sc = r[j];
    for (int e = DW; e < D; ++e) sc += qf[g * D + e] * load1(kp + t * st_b, e, DT);
    s[g * BS + t] = sc;
  }
}

// Online-softmax partials of query heads g0 .. g0 + G - 1 of each of the kv
// heads kh0 .. kh0 + nkh - 1 (query head kh * Gr + g0 + g, Gr = H / KVH) of
// sequence i. Blocks are the outer loop and the item's kv heads the inner
// one: in the host tier's [C, KVH, BS, D] layout the runs of adjacent kv heads
// of a block are adjacent, so one item streams nkh * BS * D elements of K and
// of V per block in one piece instead of one head's run (measured on the
// host tier of the vicuna-7b split: a plain read of 4 KiB runs per block
// reaches ~80 % of the cores' rate for whole blocks). Each (block, kv head)
// step is one online-softmax step of that head's G query heads. Returns false
// if the row is invalid (a length past its table or a block id outside the
// cache).
template <int DT, int G>
bool run_heads(const HostArgs& a, int i, int kh0, int nkh, int g0, Scratch& w) {
  using T = typename V::T;
  constexpr int W = V::W;
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  constexpr int U = G >= 8 ? 1 : 8 / G;   // score chains per head (>= 8 in all)
  constexpr int CU = G >= V::kAcc ? 1 : V::kAcc / G;  // P.V chunks in flight
  constexpr int TT0 = V::kAcc / G < 4 ? V::kAcc / G : 4;  // tokens scored together
  constexpr int TT = (G * TT0) % 4 == 0 ? TT0 : 1;
  const int D = a.D, BS = a.BS, Gr = a.H / a.KVH;
  const int DW = D - D % W;
  // bf16 V: P.V on even / odd halves of 2W-element loads (D a multiple of 2W,
  // and each P.V group an even number of W chunks: CU >= 2 at every level)
  constexpr bool kPermOk = DT == FD_BF16 && CU >= 2;
  const bool perm = kPermOk && D % (2 * W) == 0 && (D / W) % 2 == 0;
  const int L = a.lens[i];
  const int nb = (L + BS - 1) / BS;
  if (nb > a.bt_width) return false;
  const int GH = nkh * G;  // query heads of the item
  w.q.resize((size_t)GH * D);
  w.acc.assign((size_t)GH * D, 0.f);
  w.s.resize((size_t)G * BS);
  w.m.assign((size_t)GH, -INFINITY);
  w.l.assign((size_t)GH, 0.f);
  float* s = w.s.data();
  const float qs = a.scale * 1.4426950408889634f;  // scores in the log2 domain
  for (int j = 0; j < nkh; ++j)
    for (int g = 0; g < G; ++g) {
      const int64_t qb = (int64_t)i * a.q_ss + (int64_t)((kh0 + j) * Gr + g0 + g) * a.q_sh;
      float* qd = w.q.data() + (size_t)(j * G + g) * D;
      for (int d = 0; d < D; ++d) qd[d] = load1(a.q, qb + d, a.dt) * qs;
    }
  const uint16_t* qh_all = nullptr;  // the raw bf16 q rows, for the pair dot products
  if constexpr (V::kBf16Dot && DT == FD_BF16) {
    w.qh.resize((size_t)GH * D);
    for (int j = 0; j < nkh; ++j)
      for (int g = 0; g < G; ++g) {
        const int64_t qb = (int64_t)i * a.q_ss + (int64_t)((kh0 + j) * Gr + g0 + g) * a.q_sh;
        memcpy(w.qh.data() + (size_t)(j * G + g) * D, static_cast<const uint16_t*>(a.q) + qb,
               (size_t)D * 2);
      }
    qh_all = w.qh.data();
  }
  const char* kbase = static_cast<const char*>(a.k);
  const char* vbase = static_cast<const char*>(a.v);
  const int32_t* row_bt = a.bt + (int64_t)i * a.bt_stride;
  // the item's (block, kv head) runs in the order read: r = b * nkh + j
  const int64_t runs = (int64_t)nb * nkh;
  auto run_base = [&](int64_t r) -> int64_t {  // -1 past the row or at a bad id
    if (r >= runs) return -1;
    const int64_t id = row_bt[r / nkh];
    if (id < 0 || id >= a.num_blocks) return -1;
    return id * a.sb + (int64_t)(kh0 + r % nkh) * a.sh;
  };
  for (int b = 0; b < nb; ++b) {
    const int64_t bid = row_bt[b];
    if (bid < 0 || bid >= a.num_blocks) return false;
    const int ntok = std::min(BS, L - b * BS);
    for (int j = 0; j < nkh; ++j) {
      const int kh = kh0 + j;
      const int64_t base = bid * a.sb + (int64_t)kh * a.sh;
      // the run read kAheadRuns after this one, prefetched a few rows at a
      // time below
      const int64_t nbase = run_base((int64_t)b * nkh + j + kAheadRuns);
      int pf = 0;  // next row of that run to prefetch
      auto prefetch_rows = [&](int upto) {
        if (nbase < 0) return;
        for (; pf < upto && pf < BS; ++pf)
          for (int off = 0; off < D * elt; off += 64) {
            _mm_prefetch(kbase + (nbase + (int64_t)pf * a.st) * elt + off, _MM_HINT_T0);
            _mm_prefetch(vbase + (nbase + (int64_t)pf * a.st) * elt + off, _MM_HINT_T0);
          }
      };
      const float* qf = w.q.data() + (size_t)j * G * D;
      const uint16_t* qh = qh_all != nullptr ? qh_all + (size_t)j * G * D : nullptr;
      float* acc = w.acc.data() + (size_t)j * G * D;
      float* mj = w.m.data() + j * G;
      float* lj = w.l.data() + j * G;
      float alpha[G];
      // scores, TT tokens at a time where the accumulators fit
      int t0 = 0;
      if constexpr (TT >= 2) {
        for (; t0 + TT <= ntok; t0 += TT) {
          // half the next run's rows over the score loop, the rest below:
          // measured best on Zen 5 against TT rows per group or one per group
          prefetch_rows(pf + (TT + 1) / 2);
          score_tokens<DT, G, TT>(kbase + (base + (int64_t)t0 * a.st) * elt, a.st * elt, qf, qh,
                                  qs, D, DW, s + t0, BS);
        }
      }
      prefetch_rows(BS);
      for (int t = t0; t < ntok; ++t)
        score_token<DT, G, U>(kbase + (base + (int64_t)t * a.st) * elt, qf, qh, qs, D, DW,
                              s + t, BS);
      // one online-softmax step per head
      for (int g = 0; g < G; ++g) {
        float* sg = s + g * BS;
        float bmax = -INFINITY;
        {
          int t = 0;
          if (ntok >= W) {
            T mx = V::load(sg);
            for (t = W; t + W <= ntok; t += W) mx = V::max(mx, V::load(sg + t));
            bmax = V::hmax(mx);
          }
          for (; t < ntok; ++t) bmax = std::max(bmax, sg[t]);
        }
        const float mn = std::max(mj[g], bmax);
        alpha[g] = mj[g] == -INFINITY ? 0.f : V::exp2_1(mj[g] - mn);
        const T mv = V::set1(mn);
        T ps = V::zero();
        int t = 0;
        for (; t + W <= ntok; t += W) {
          const T p = V::exp2(V::sub(V::load(sg + t), mv));
          V::store(sg + t, p);
          ps = V::add(ps, p);
        }
        float psum = V::hsum(ps);
        for (; t < ntok; ++t) {
          sg[t] = V::exp2_1(sg[t] - mn);
          psum += sg[t];
        }
        lj[g] = lj[g] * alpha[g] + psum;
        mj[g] = mn;
      }
      // acc = acc * alpha + P.V, CU chunks of W columns at a time, then
      // halving groups for what is left
      const char* vb = vbase + base * elt;
      int d = 0;
      if (perm)
        pv_groups<DT, G, CU, true>(acc, s, alpha, vb, a.st, D, DW, BS, ntok, d);
      else
        pv_groups<DT, G, CU>(acc, s, alpha, vb, a.st, D, DW, BS, ntok, d);
      for (; d < D; ++d)
        for (int g = 0; g < G; ++g) {
          float x = acc[g * D + d] * alpha[g];
          for (int t = 0; t < ntok; ++t) x += s[g * BS + t] * load1(vb, (int64_t)t * a.st + d, DT);
          acc[g * D + d] = x;
        }
    }
  }
  for (int j = 0; j < nkh; ++j)
    for (int g = 0; g < G; ++g) {
      const int h = (kh0 + j) * Gr + g0 + g;
      const float lh = w.l[j * G + g];
      const float inv = 1.f / lh;
      float* o = w.acc.data() + (size_t)(j * G + g) * D;
      if (perm) {  // back from the even / odd layout of each 2W span
        float tmp[2 * W];
        for (int d0 = 0; d0 < D; d0 += 2 * W) {
          for (int e = 0; e < W; ++e) {
            tmp[2 * e] = o[d0 + e];
            tmp[2 * e + 1] = o[d0 + W + e];
          }
          memcpy(o + d0, tmp, sizeof(tmp));
        }
      }
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
      a.lse[(int64_t)h * a.lse_sh + i] = (w.m[j * G + g] + std::log2(lh)) * 0.6931471805599453f;
    }
  return true;
}

template <int DT>
bool run_heads_dt(const HostArgs& a, int i, int kh0, int nkh, int g0, int G, Scratch& w) {
  switch (G) {
    case 1: return run_heads<DT, 1>(a, i, kh0, nkh, g0, w);
    case 2: return run_heads<DT, 2>(a, i, kh0, nkh, g0, w);
    case 4: return run_heads<DT, 4>(a, i, kh0, nkh, g0, w);
    default: return run_heads<DT, 8>(a, i, kh0, nkh, g0, w);
  }
}

// Query heads g0 .. g0 + G - 1 (G in {1, 2, 4, 8}) of each kv head kh0 ..
// kh0 + nkh - 1 of sequence i.
bool run_group(const HostArgs& a, int i, int kh0, int nkh, int g0, int G, Scratch& w) {
  if (a.dt == FD_F16) return run_heads_dt<FD_F16>(a, i, kh0, nkh, g0, G, w);
  if (a.dt == FD_BF16) return run_heads_dt<FD_BF16>(a, i, kh0, nkh, g0, G, w);
  return run_heads_dt<FD_F32>(a, i, kh0, nkh, g0, G, w);
}
