// Body of the host-core decode kernel, compiled once per vector ISA.
//
// host_decode.cpp includes this file several times, each time inside a
// `#pragma GCC target` region and a namespace that defines `V`, the vector
// traits of that ISA (width W, fp32 arithmetic, conversions of W storage
// elements, exp2). No include guard on purpose.
//
// Needs, from the including namespace: V, HostArgs, Scratch, load1,
// f32_to_bf16, kPrefetchBlocks.

// Online-softmax partial of query heads kh*Gr + g0 .. + G-1 (Gr = H / KVH) of
// sequence i over kv head kh. Returns false if the row is invalid (a length
// past its table or a block id outside the cache).
template <int DT, int G>
bool run_heads(const HostArgs& a, int i, int kh, int g0, Scratch& w) {
  using T = typename V::T;
  constexpr int W = V::W;
  constexpr int elt = DT == FD_F32 ? 4 : 2;
  constexpr int U = G >= 4 ? 1 : 4 / G;   // score chains per head
  constexpr int CU = G >= 8 ? 1 : 8 / G;  // P.V chunks in flight
  const int D = a.D, BS = a.BS, Gr = a.H / a.KVH;
  const int DW = D - D % W;
  const int L = a.lens[i];
  const int nb = (L + BS - 1) / BS;
  if (nb > a.bt_width) return false;
  w.q.resize((size_t)G * D);
  w.acc.assign((size_t)G * D, 0.f);
  w.s.resize((size_t)G * BS);
  float* qf = w.q.data();
  float* acc = w.acc.data();
  float* s = w.s.data();
  const float qs = a.scale * 1.4426950408889634f;  // scores in the log2 domain
  for (int g = 0; g < G; ++g) {
    const int64_t qb = (int64_t)i * a.q_ss + (int64_t)(kh * Gr + g0 + g) * a.q_sh;
    for (int d = 0; d < D; ++d) qf[g * D + d] = load1(a.q, qb + d, a.dt) * qs;
  }
  float m[G], l[G], alpha[G];
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
  }
  const char* kbase = static_cast<const char*>(a.k);
  const char* vbase = static_cast<const char*>(a.v);
  const int32_t* row_bt = a.bt + (int64_t)i * a.bt_stride;
  for (int b = 0; b < nb; ++b) {
    const int64_t bid = row_bt[b];
    if (bid < 0 || bid >= a.num_blocks) return false;
    const int ntok = std::min(BS, L - b * BS);
    const int64_t base = bid * a.sb + (int64_t)kh * a.sh;
    if (b + kPrefetchBlocks < nb) {  // a later block's rows, while this one computes
      const int64_t nid = row_bt[b + kPrefetchBlocks];
      if (nid >= 0 && nid < a.num_blocks) {
        const int64_t nbase = nid * a.sb + (int64_t)kh * a.sh;
        for (int t = 0; t < BS; ++t)
          for (int off = 0; off < D * elt; off += 64) {
            _mm_prefetch(kbase + (nbase + (int64_t)t * a.st) * elt + off, _MM_HINT_T0);
            _mm_prefetch(vbase + (nbase + (int64_t)t * a.st) * elt + off, _MM_HINT_T0);
          }
      }
    }
    // scores
    for (int t = 0; t < ntok; ++t) {
      const char* kp = kbase + (base + (int64_t)t * a.st) * elt;
      T c[G][U];
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < U; ++u) c[g][u] = V::zero();
      int d = 0;
      for (; d + W * U <= DW; d += W * U)
        for (int u = 0; u < U; ++u) {
          const T kv = V::template ld<DT>(kp + (d + W * u) * elt);
          for (int g = 0; g < G; ++g)
            c[g][u] = V::fma(V::load(qf + g * D + d + W * u), kv, c[g][u]);
        }
      for (; d < DW; d += W) {
        const T kv = V::template ld<DT>(kp + d * elt);
        for (int g = 0; g < G; ++g) c[g][0] = V::fma(V::load(qf + g * D + d), kv, c[g][0]);
      }
      for (int g = 0; g < G; ++g) {
        T sum = c[g][0];
        for (int u = 1; u < U; ++u) sum = V::add(sum, c[g][u]);
        float sc = V::hsum(sum);
        for (int e = DW; e < D; ++e) sc += qf[g * D + e] * load1(kp, e, DT);
        s[g * BS + t] = sc;
      }
    }
    // one online-softmax step per head
    for (int g = 0; g < G; ++g) {
      float* sg = s + g * BS;
      float bmax = sg[0];
      for (int t = 1; t < ntok; ++t) bmax = std::max(bmax, sg[t]);
      const float mn = std::max(m[g], bmax);
      alpha[g] = m[g] == -INFINITY ? 0.f : V::exp2_1(m[g] - mn);
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
      l[g] = l[g] * alpha[g] + psum;
      m[g] = mn;
    }
    // acc = acc * alpha + P.V
    const char* vb = vbase + base * elt;
    int d = 0;
    for (; d + W * CU <= DW; d += W * CU) {
      T r[G][CU];
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < CU; ++u)
          r[g][u] = V::mul(V::load(acc + g * D + d + W * u), V::set1(alpha[g]));
      for (int t = 0; t < ntok; ++t) {
        const char* vp = vb + (int64_t)t * a.st * elt;
        for (int u = 0; u < CU; ++u) {
          const T vv = V::template ld<DT>(vp + (d + W * u) * elt);
          for (int g = 0; g < G; ++g) r[g][u] = V::fma(V::bcast(s + g * BS + t), vv, r[g][u]);
        }
      }
      for (int g = 0; g < G; ++g)
        for (int u = 0; u < CU; ++u) V::store(acc + g * D + d + W * u, r[g][u]);
    }
    for (; d < DW; d += W) {
      T r[G];
      for (int g = 0; g < G; ++g) r[g] = V::mul(V::load(acc + g * D + d), V::set1(alpha[g]));
      for (int t = 0; t < ntok; ++t) {
        const T vv = V::template ld<DT>(vb + ((int64_t)t * a.st + d) * elt);
        for (int g = 0; g < G; ++g) r[g] = V::fma(V::bcast(s + g * BS + t), vv, r[g]);
      }
      for (int g = 0; g < G; ++g) V::store(acc + g * D + d, r[g]);
    }
    for (; d < D; ++d)
      for (int g = 0; g < G; ++g) {
        float x = acc[g * D + d] * alpha[g];
        for (int t = 0; t < ntok; ++t) x += s[g * BS + t] * load1(vb, (int64_t)t * a.st + d, DT);
        acc[g * D + d] = x;
      }
  }
  for (int g = 0; g < G; ++g) {
    const int h = kh * Gr + g0 + g;
    const float inv = 1.f / l[g];
    float* o = acc + g * D;
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
    a.lse[(int64_t)h * a.lse_sh + i] = (m[g] + std::log2(l[g])) * 0.6931471805599453f;
  }
  return true;
}

template <int DT>
bool run_heads_dt(const HostArgs& a, int i, int kh, int g0, int G, Scratch& w) {
  switch (G) {
    case 1: return run_heads<DT, 1>(a, i, kh, g0, w);
    case 2: return run_heads<DT, 2>(a, i, kh, g0, w);
    case 4: return run_heads<DT, 4>(a, i, kh, g0, w);
    default: return run_heads<DT, 8>(a, i, kh, g0, w);
  }
}

// Query heads g0 .. g0 + G - 1 (G in {1, 2, 4, 8}) of (sequence i, kv head kh).
bool run_group(const HostArgs& a, int i, int kh, int g0, int G, Scratch& w) {
  if (a.dt == FD_F16) return run_heads_dt<FD_F16>(a, i, kh, g0, G, w);
  if (a.dt == FD_BF16) return run_heads_dt<FD_BF16>(a, i, kh, g0, G, w);
  return run_heads_dt<FD_F32>(a, i, kh, g0, G, w);
}
