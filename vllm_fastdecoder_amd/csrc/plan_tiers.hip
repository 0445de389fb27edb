// Device-side tier split of a decode step: the part of the reference's
// per-step planner (fastdecode/plan.py:103-199) that the decode path needs,
// computed on the GPU so the step needs no device-to-host copy.
//
// For every row r (one request):
//   * its valid block ids bt[r, 0 .. ceil(L_r / BS)) are split, in order, into
//     the HBM tier (id < G) and the host tier (id >= G, stored as id - G): the
//     stable per-tier compaction of plan.py:82-100, zero-padded to the output
//     width;
//   * each tier's token count adds the tokens its blocks hold (BS per block,
//     L - (nb-1)*BS for the row's last block): plan.py:165-170;
//   * a host id >= G + C (past the host tier) is counted into *error_count,
//     the device-side counterpart of the planner's RuntimeError
//     (plan.py:135-140); the decode kernels also turn such a row into NaN.
// For every token t the slot mapping is split too (plan.py:150-152): a host
// slot (>= G*BS) becomes -1 in gpu_slots and slot - G*BS in host_slots; any
// other slot (negative padding included) keeps its value in gpu_slots and is
// -1 in host_slots. A host slot past the host tier (>= (G+C)*BS) is counted
// into *error_count too: the host-tier store_kv's range check
// (cpu_attn.cpp:506-510), made before any write of the step.
#include "fd_common.h"

namespace fd {

namespace {

// One wave per row, 64 blocks per pass: ballots give each tier's block
// positions (mbcnt = number of set lanes below), a wave sum the token counts.
__global__ __launch_bounds__(kWave) void plan_rows_kernel(PlanTiersArgs a) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  const int L = a.seq_lens[r];
  int nb = L > 0 ? (L + a.BS - 1) / a.BS : 0;
  const int last = L - (nb - 1) * a.BS;
  // a length past the table is not read: the row gets an HBM length past its
  // table, which the decode kernels turn into NaN, and counts as an error
  const bool too_long = nb > a.bt_width;
  if (too_long) nb = 0;
  const int32_t* bt = a.bt + (int64_t)r * a.bt_stride;
  int32_t* og = a.gpu_bt + (int64_t)r * a.out_stride;
  int32_t* oc = a.cpu_bt + (int64_t)r * a.out_stride;
  int ng = 0, nc = 0, tg = 0, tc = 0, bad = too_long ? 1 : 0;
  for (int base = 0; base < nb; base += kWave) {
    const int j = base + lane;
    const bool valid = j < nb;
    const int id = valid ? bt[j] : 0;
    const bool host = valid && id >= a.G;
    const bool hbm = valid && !host;
    const uint64_t mh = __ballot(hbm);
    const uint64_t mc = __ballot(host);
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    if (hbm) og[ng + __popcll(mh & below)] = id;
    if (host) oc[nc + __popcll(mc & below)] = id - a.G;
    const int ntok = j == nb - 1 ? last : a.BS;
    int sg = hbm ? ntok : 0;
    int sc = host ? ntok : 0;
    for (int x = kWave / 2; x >= 1; x >>= 1) {
      sg += __shfl_xor(sg, x, kWave);
      sc += __shfl_xor(sc, x, kWave);
    }
    tg += sg;
    tc += sc;
    ng += __popcll(mh);
    nc += __popcll(mc);
    bad += __popcll(__ballot(host && (int64_t)id >= (int64_t)a.G + a.C));
  }
  for (int j = ng + lane; j < a.out_width; j += kWave) og[j] = 0;
  for (int j = nc + lane; j < a.out_width; j += kWave) oc[j] = 0;
  if (lane == 0) {
    a.gpu_lens[r] = too_long ? a.out_width * a.BS + 1 : tg;
    a.cpu_lens[r] = tc;
    if (bad != 0 && a.error_count != nullptr) atomicAdd(a.error_count, bad);
  }
}

__global__ __launch_bounds__(256) void plan_slots_kernel(const int64_t* __restrict__ slots,
                                                         int32_t n, int64_t hbm_slots,
                                                         int64_t host_cap,
                                                         int64_t* __restrict__ gpu_slots,
                                                         int64_t* __restrict__ host_slots,
                                                         int32_t* __restrict__ error_count) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int64_t s = slots[t];
  const bool on_host = s >= hbm_slots;
  gpu_slots[t] = on_host ? -1 : s;
  host_slots[t] = on_host ? s - hbm_slots : -1;
  if (on_host && s - hbm_slots >= host_cap && error_count != nullptr) atomicAdd(error_count, 1);
}

}  // namespace

int launch_plan_tiers(const PlanTiersArgs& a, hipStream_t s) {
  if (a.n_rows > 0) {
    hipLaunchKernelGGL(plan_rows_kernel, dim3((unsigned)a.n_rows), dim3(kWave), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "plan_rows_kernel launch");
  }
  if (a.n_tokens > 0) {
    hipLaunchKernelGGL(plan_slots_kernel, dim3((unsigned)((a.n_tokens + 255) / 256)), dim3(256),
                       0, s, a.slots, a.n_tokens, (int64_t)a.G * a.BS, a.C * a.BS,
                       a.gpu_slots, a.host_slots, a.error_count);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "plan_slots_kernel launch");
  }
  return FD_OK;
}

}  // namespace fd
