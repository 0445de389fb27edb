// Log-sum-exp merge of two attention partials (GPU tier + host tier).
//
// Rule of the reference's merge_partials_torch (fastdecode/cpu_ops.py:93-113),
// which restates vLLM's merge_attn_states as called at
// fastdecode/backend.py:53-55,354-355:
//   +inf LSE means "empty" and is treated as -inf (cpu_ops.py:102-103);
//   m = max(lse_a, lse_b), with m = 0 when both are empty (:104-106);
//   w = exp(lse - m), normalised by their sum, which is 1 when both are
//   empty (:107-110); out = o_a * w_a + o_b * w_b in fp32 (:111-113).
//
// One thread per 4 consecutive elements of a (sequence, head) row; the two
// LSE values are read once per thread (they are L2-broadcast within a row).
// Pure streaming work: 2 reads + 1 write of [n, H, D] plus the LSEs.
#include "fd_common.h"

namespace fd {

namespace {

constexpr int kVec = 4;

__device__ __forceinline__ void load4(const void* p, int64_t off, int dt, bool vec,
                                      float* x) {
  if (vec && dt == FD_F32) {
    const float4 u = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + off);
    x[0] = u.x;
    x[1] = u.y;
    x[2] = u.z;
    x[3] = u.w;
  } else if (vec) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + off);
    if (dt == FD_F16) {
      x[0] = lo_f32(F16{}, u.x);
      x[1] = hi_f32(F16{}, u.x);
      x[2] = lo_f32(F16{}, u.y);
      x[3] = hi_f32(F16{}, u.y);
    } else {
      x[0] = lo_f32(BF16{}, u.x);
      x[1] = hi_f32(BF16{}, u.x);
      x[2] = lo_f32(BF16{}, u.y);
      x[3] = hi_f32(BF16{}, u.y);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kVec; ++e) x[e] = load_elem(p, off + e, dt);
  }
}

__device__ __forceinline__ void store4(void* p, int64_t off, int dt, bool vec,
                                       const float* x) {
  if (vec && dt == FD_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + off) =
        make_float4(x[0], x[1], x[2], x[3]);
  } else if (vec) {
    uint2 u;
    if (dt == FD_F16) {
      u.x = to_out(F16{}, x[0]) | (uint32_t(to_out(F16{}, x[1])) << 16);
      u.y = to_out(F16{}, x[2]) | (uint32_t(to_out(F16{}, x[3])) << 16);
    } else {
      u.x = to_out(BF16{}, x[0]) | (uint32_t(to_out(BF16{}, x[1])) << 16);
      u.y = to_out(BF16{}, x[2]) | (uint32_t(to_out(BF16{}, x[3])) << 16);
    }
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + off) = u;
  } else {
#pragma unroll
    for (int e = 0; e < kVec; ++e) store_elem(p, off + e, dt, x[e]);
  }
}

// vec: every row start is 4-element aligned in all three tensors (checked on
// the host), so 4 elements move as one 8- or 16-byte access.
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a, bool vec) {
  const int per_row = a.D / kVec;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.n * a.H * per_row;
  if (tid >= total) return;
  const int c = (int)(tid % per_row);
  const int64_t rowid = tid / per_row;
  const int h = (int)(rowid % a.H);
  const int i = (int)(rowid / a.H);
  const int d = c * kVec;

  float la = a.lse_a[(int64_t)h * a.lse_a_sh + i];
  float lb = a.lse_b[(int64_t)h * a.lse_b_sh + i];
  const float pinf = __builtin_huge_valf();
  la = la == pinf ? neg_inf() : la;
  lb = lb == pinf ? neg_inf() : lb;
  float m = fmaxf(la, lb);
  const bool both_empty = m == neg_inf();
  m = both_empty ? 0.f : m;
  const float ea = __expf(la - m);
  const float eb = __expf(lb - m);
  float tot = ea + eb;
  tot = both_empty ? 1.f : tot;
  const float wa = ea / tot;
  const float wb = eb / tot;

  float xa[kVec], xb[kVec], y[kVec];
  load4(a.a, (int64_t)i * a.a_ss + (int64_t)h * a.a_sh + d, a.a_dt, vec, xa);
  load4(a.b, (int64_t)i * a.b_ss + (int64_t)h * a.b_sh + d, a.b_dt, vec, xb);
#pragma unroll
  for (int e = 0; e < kVec; ++e) y[e] = xa[e] * wa + xb[e] * wb;
  store4(a.out, (int64_t)i * a.out_ss + (int64_t)h * a.out_sh + d, a.out_dt, vec, y);
  if (a.out_lse != nullptr && c == 0) {
    a.out_lse[(int64_t)h * a.out_lse_sh + i] = both_empty ? neg_inf() : m + __logf(tot);
  }
}

// Scalar tail for head sizes that are not a multiple of 4.
__global__ __launch_bounds__(256) void merge_scalar_kernel(MergeArgs a) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.n * a.H * a.D;
  if (tid >= total) return;
  const int d = (int)(tid % a.D);
  const int64_t rowid = tid / a.D;
  const int h = (int)(rowid % a.H);
  const int i = (int)(rowid / a.H);
  float la = a.lse_a[(int64_t)h * a.lse_a_sh + i];
  float lb = a.lse_b[(int64_t)h * a.lse_b_sh + i];
  const float pinf = __builtin_huge_valf();
  la = la == pinf ? neg_inf() : la;
  lb = lb == pinf ? neg_inf() : lb;
  float m = fmaxf(la, lb);
  const bool both_empty = m == neg_inf();
  m = both_empty ? 0.f : m;
  const float ea = __expf(la - m);
  const float eb = __expf(lb - m);
  float tot = ea + eb;
  tot = both_empty ? 1.f : tot;
  const float y = load_elem(a.a, (int64_t)i * a.a_ss + (int64_t)h * a.a_sh + d, a.a_dt) * (ea / tot) +
                  load_elem(a.b, (int64_t)i * a.b_ss + (int64_t)h * a.b_sh + d, a.b_dt) * (eb / tot);
  store_elem(a.out, (int64_t)i * a.out_ss + (int64_t)h * a.out_sh + d, a.out_dt, y);
  if (a.out_lse != nullptr && d == 0) {
    a.out_lse[(int64_t)h * a.out_lse_sh + i] = both_empty ? neg_inf() : m + __logf(tot);
  }
}

bool aligned4(const void* p, int dt, int64_t s1, int64_t s2) {
  const int64_t bytes = (int64_t)kVec * dtype_size(dt);
  return reinterpret_cast<uintptr_t>(p) % bytes == 0 && s1 % kVec == 0 && s2 % kVec == 0;
}

}  // namespace

int launch_merge(const MergeArgs& a, hipStream_t s) {
  if (a.n == 0 || a.H == 0 || a.D == 0) return FD_OK;
  if (a.D % kVec == 0) {
    const bool vec = aligned4(a.out, a.out_dt, a.out_ss, a.out_sh) &&
                     aligned4(a.a, a.a_dt, a.a_ss, a.a_sh) &&
                     aligned4(a.b, a.b_dt, a.b_ss, a.b_sh);
    const int64_t total = (int64_t)a.n * a.H * (a.D / kVec);
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       a, vec);
  } else {
    const int64_t total = (int64_t)a.n * a.H * a.D;
    hipLaunchKernelGGL(merge_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, a);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FD_OK : hip_error(e, "merge kernel launch");
}

}  // namespace fd
