// Paged decode attention: planning, the generic kernel, the split combine
// and the launcher. The tiled kernels live in decode_valu.hip and
// decode_mfma.hip (shared code in decode_tiled.h).
#include <algorithm>

#include "decode_tiled.h"

extern char** environ;  // the process environment (POSIX)

namespace fd {

namespace {

// Combines the split partials of every (sequence, head) whose row used more
// than one task: the N-way form of the log-sum-exp merge. One thread per 4
// output elements; each thread reads the row's split LSEs (L1-shared with its
// neighbours) and its slice of every split's partial. The reads go out
// kSplitChunk splits at a time, all in flight together, and the first
// chunk's with the row lengths' (the workspace holds S splits per pair, so
// they are in bounds before the row's split count is known): a launch of a
// few rows is a chain of dependent memory round trips, and a loop issuing
// one split's read per iteration made it one per split. Batched, split
// launches of 1-8 rows take 0.6-0.8 us less. Splits are summed in index order.
constexpr int kSplitChunk = 8;

__global__ __launch_bounds__(256) void combine_splits_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ lens_a, const int32_t* __restrict__ lens_b, int32_t width_a,
    int32_t width_b, int32_t n, int32_t H, int32_t D, int32_t S, int32_t split_blocks,
    int32_t block_size, void* out, int64_t out_ss, int64_t out_sh, int32_t out_dt, float* lse,
    int64_t lse_sh) {
  const int per_row = D / 4;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (int64_t)n * H * per_row) return;
  const int c = (int)(tid % per_row);
  const int64_t pair = tid / per_row;
  const int i = (int)(pair / H);
  const int h = (int)(pair % H);
  const float* pl = part_lse + pair * S;
  const float4* po = reinterpret_cast<const float4*>(part_o + pair * S * D) + c;
  float l0[kSplitChunk];
  float4 o0[kSplitChunk];
#pragma unroll
  for (int u = 0; u < kSplitChunk; ++u) {
    l0[u] = u < S ? pl[u] : neg_inf();
    o0[u] = u < S ? po[(int64_t)u * per_row] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int La = lens_a[i];
  const int Lb = lens_b != nullptr ? lens_b[i] : 0;
  if (La > width_a * block_size || Lb > width_b * block_size) return;  // range error: NaN
  const int nb = (La > 0 ? (La + block_size - 1) / block_size : 0) +
                 (Lb > 0 ? (Lb + block_size - 1) / block_size : 0);
  const int ns = (nb + split_blocks - 1) / split_blocks;
  if (ns <= 1) return;  // written directly by the partial kernel
  float M = neg_inf();
  for (int s0 = 0; s0 < ns; s0 += kSplitChunk) {
    float v[kSplitChunk];
#pragma unroll
    for (int u = 0; u < kSplitChunk; ++u)
      v[u] = s0 == 0 ? l0[u] : (s0 + u < ns ? pl[s0 + u] : neg_inf());
#pragma unroll
    for (int u = 0; u < kSplitChunk; ++u)
      if (s0 + u < ns) M = fmaxf(M, v[u]);
  }
  const float Ms = M == neg_inf() ? 0.f : M;
  float wsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += kSplitChunk) {
    float lv[kSplitChunk];
    float4 ov[kSplitChunk];
#pragma unroll
    for (int u = 0; u < kSplitChunk; ++u) {
      const bool on = s0 + u < ns;
      lv[u] = s0 == 0 ? l0[u] : (on ? pl[s0 + u] : neg_inf());
      ov[u] = s0 == 0 ? o0[u] : (on ? po[(int64_t)(s0 + u) * per_row] : make_float4(0.f, 0.f, 0.f, 0.f));
    }
#pragma unroll
    for (int u = 0; u < kSplitChunk; ++u) {
      if (s0 + u < ns) {
        const float w = __expf(lv[u] - Ms);
        const float4 x = ov[u];
        wsum += w;
        acc.x += w * x.x;
        acc.y += w * x.y;
        acc.z += w * x.z;
        acc.w += w * x.w;
      }
    }
  }
  const float inv = 1.f / wsum;
  const int64_t ob = (int64_t)i * out_ss + (int64_t)h * out_sh + c * 4;
  store_elem(out, ob + 0, out_dt, acc.x * inv);
  store_elem(out, ob + 1, out_dt, acc.y * inv);
  store_elem(out, ob + 2, out_dt, acc.z * inv);
  store_elem(out, ob + 3, out_dt, acc.w * inv);
  if (c == 0) lse[(int64_t)h * lse_sh + i] = Ms + __logf(wsum);
}

struct GenericParams {
  const void* q;
  int64_t q_ss, q_sh;
  KvTier tier[2];
  int32_t ntiers;
  int32_t H, KVH, D, BS;
  float scale;
  int32_t dt;
  void* out;
  int64_t out_ss, out_sh;
  int32_t out_dt;
  float* lse;
  int64_t lse_sh;
};

// Generic kernel: any head_size, block_size, group size and dtype (including
// fp32 KV), one or two tiers. One wavefront per (sequence, query head); each
// lane owns elements d = lane + 64k. Correct for every layout, not tuned.
__global__ __launch_bounds__(kWave) void decode_generic_kernel(GenericParams p) {
  constexpr int kMaxPerLane = 8;  // D <= 512
  const int lane = threadIdx.x;
  const int i = blockIdx.x / p.H;
  const int h = blockIdx.x % p.H;
  const int kh = h / (p.H / p.KVH);
  const int D = p.D;
  int len[2] = {p.tier[0].lens[i], p.ntiers > 1 ? p.tier[1].lens[i] : 0};
  bool bad = false;
  for (int t = 0; t < 2; ++t) {
    if (len[t] > 0 && (len[t] > p.tier[t].bt_width * p.BS || p.tier[t].num_blocks <= 0))
      bad = true;
    len[t] = len[t] > 0 ? len[t] : 0;
  }
  const int L = len[0] + len[1];
  const int64_t obase = (int64_t)i * p.out_ss + (int64_t)h * p.out_sh;
  if (L == 0 || bad) {
    const float fill = bad ? qnan() : 0.f;
    for (int d = lane; d < D; d += kWave) store_elem(p.out, obase + d, p.out_dt, fill);
    if (lane == 0) p.lse[(int64_t)h * p.lse_sh + i] = bad ? qnan() : neg_inf();
    return;
  }
  float qv[kMaxPerLane], acc[kMaxPerLane];
  const int64_t qbase = (int64_t)i * p.q_ss + (int64_t)h * p.q_sh;
#pragma unroll
  for (int r = 0; r < kMaxPerLane; ++r) {
    const int d = lane + r * kWave;
    qv[r] = d < D ? load_elem(p.q, qbase + d, p.dt) * p.scale : 0.f;
    acc[r] = 0.f;
  }
  float mrun = neg_inf(), lrun = 0.f;
  for (int t = 0; t < L; ++t) {
    const int tier = t < len[0] ? 0 : 1;
    const int tt = tier == 0 ? t : t - len[0];
    const KvTier& kt = p.tier[tier];
    int64_t bid = kt.bt[(int64_t)i * kt.bt_stride + tt / p.BS];
    const bool ok = bid >= 0 && bid < kt.num_blocks;
    bad |= !ok;
    bid = ok ? bid : 0;
    const int64_t base = bid * kt.sb + (int64_t)kh * kt.sh + (int64_t)(tt % p.BS) * kt.st;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < kMaxPerLane; ++r) {
      const int d = lane + r * kWave;
      if (d < D) s += qv[r] * load_elem(kt.k, base + d, p.dt);
    }
    s = wave_sum(s);
    const float mn = fmaxf(mrun, s);
    const float alpha = __expf(mrun - mn);
    const float pt = __expf(s - mn);
    lrun = lrun * alpha + pt;
#pragma unroll
    for (int r = 0; r < kMaxPerLane; ++r) {
      const int d = lane + r * kWave;
      if (d < D) acc[r] = acc[r] * alpha + pt * load_elem(kt.v, base + d, p.dt);
    }
    mrun = mn;
  }
  const float inv = 1.f / lrun;
#pragma unroll
  for (int r = 0; r < kMaxPerLane; ++r) {
    const int d = lane + r * kWave;
    if (d < D) store_elem(p.out, obase + d, p.out_dt, bad ? qnan() : acc[r] * inv);
  }
  if (lane == 0) p.lse[(int64_t)h * p.lse_sh + i] = bad ? qnan() : mrun + __logf(lrun);
}

// The planner's tuning variables (comparison runs and tests), found in one
// pass over the environment per plan rather than one getenv each (seven per
// launch cost ~0.5 us of host time with ~90 variables set):
//   FD_SPLIT_BLOCKS=<n>  n blocks per task;
//   FD_KV_ADJ=0          separate K and V loads where V follows K;
//   FD_DECODE_KERNEL=valu | mfma | mm  a kernel family where it applies: the
//                        VALU kernel, the one with only the scores on the
//                        matrix cores (4+ query heads per kv head), the one
//                        with P.V there too (D <= 128);
//   FD_WAVE_BLOCKS=<b>   blocks per working wave (0: every wave works);
//   FD_WG_CAP=<k>        at most k workgroups per CU (0: no cap).
// Like getenv, the first definition of a name counts.
struct Tuning {
  const char* split_blocks = nullptr;
  const char* kv_adj = nullptr;
  const char* kernel = nullptr;
  const char* wave_blocks = nullptr;
  const char* wg_cap = nullptr;

  bool kernel_forced(const char* name) const {
    return kernel != nullptr && strcmp(kernel, name) == 0;
  }
};

Tuning read_tuning() {
  Tuning t;
  // the value of `entry` if it defines `name` (entry past its "FD_"), else null
  auto value = [](const char* entry, const char* name) -> const char* {
    const size_t k = strlen(name);
    return strncmp(entry, name, k) == 0 && entry[k] == '=' ? entry + k + 1 : nullptr;
  };
  for (char** e = environ; e != nullptr && *e != nullptr; ++e) {
    const char* s = *e;
    if (s[0] != 'F' || s[1] != 'D' || s[2] != '_') continue;
    s += 3;
    const char* v;
    if (!t.split_blocks && (v = value(s, "SPLIT_BLOCKS"))) t.split_blocks = v;
    else if (!t.kv_adj && (v = value(s, "KV_ADJ"))) t.kv_adj = v;
    else if (!t.kernel && (v = value(s, "DECODE_KERNEL"))) t.kernel = v;
    else if (!t.wave_blocks && (v = value(s, "WAVE_BLOCKS"))) t.wave_blocks = v;
    else if (!t.wg_cap && (v = value(s, "WG_CAP"))) t.wg_cap = v;
  }
  return t;
}

}  // namespace

// Compute units of the current device (cached per device; 0 if unknown).
static int device_cus() {
  static std::atomic<int> cache[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  const int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v - 1;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 0;
  cache[dev].store(cus + 1, std::memory_order_relaxed);
  return cus;
}

// LDS of the current device: per CU and the most one workgroup may take
// (cached per device; 0 if unknown).
static void device_lds(int dev, int* per_cu, int* per_wg) {
  static std::atomic<int> cu_cache[kMaxDevices] = {}, wg_cache[kMaxDevices] = {};
  int cu = cu_cache[dev].load(std::memory_order_relaxed) - 1;
  int wg = wg_cache[dev].load(std::memory_order_relaxed) - 1;
  if (cu < 0 || wg < 0) {
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
            hipSuccess ||
        hipDeviceGetAttribute(&wg, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      cu = wg = 0;
    cu_cache[dev].store(cu + 1, std::memory_order_relaxed);
    wg_cache[dev].store(wg + 1, std::memory_order_relaxed);
  }
  *per_cu = cu;
  *per_wg = wg;
}

// Dynamic LDS that leaves room for at most `wgs` workgroups of `kernel` per
// CU (the reservation is never touched), or 0 when the kernel's own LDS
// already keeps it there or the reservation would not fit one workgroup's
// limit. Measured on MI355X: with tasks of 32+ blocks, two workgroups per CU
// (8 waves, one block in flight each) already saturate HBM, and the fewer
// concurrent streams read faster (+1 to +6 % over the natural 3-4 per CU);
// short tasks want the extra workgroups to hide their start-up latency, so
// they are left uncapped. `cache` holds the kernel's static LDS + 1 per
// device (0 = not read yet).
unsigned cap_lds(const void* kernel, int wgs, std::atomic<int>* cache) {
  int dev = 0;
  if (wgs <= 0 || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int stat = cache[dev].load(std::memory_order_relaxed) - 1;
  if (stat < 0) {
    hipFuncAttributes fa{};
    // unknown: as if the kernel's own LDS already capped it (no reservation)
    stat = hipFuncGetAttributes(&fa, kernel) == hipSuccess ? (int)fa.sharedSizeBytes : 1 << 30;
    cache[dev].store(stat + 1, std::memory_order_relaxed);
  }
  int per_cu = 0, per_wg = 0;
  device_lds(dev, &per_cu, &per_wg);
  // more than 1 / (wgs + 1) of the CU: wgs workgroups fit, one more does not
  const int need = per_cu / (wgs + 1) + 1024;
  return per_cu > 0 && need > stat && need <= per_wg ? (unsigned)(need - stat) : 0u;
}

int natural_wgs_per_cu(const void* kernel, std::atomic<int>* cache) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  const int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v - 1;
  int wgs = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wgs, kernel, kWave * kWavesPerTask, 0) !=
      hipSuccess)
    wgs = 0;
  cache[dev].store(wgs + 1, std::memory_order_relaxed);
  return wgs;
}

namespace {

// The tiled kernel family the plan selects, for a launch or (with the plan's
// occupancy query set) for its occupancy.
hipError_t dispatch_tiled(const TiledParams& tp, unsigned tasks, const SplitPlan& sp,
                          int32_t kv_dtype, int32_t D, bool two, hipStream_t s) {
  const int G = sp.kernel_g;  // the kernel's head slots per task
  return kv_dtype == FD_F32 ? launch_f32(tp, tasks, sp, sp.kernel_d, G, two, s)
         : sp.mm            ? launch_mm(tp, tasks, sp, kv_dtype, D, two, s)
         : sp.mfma          ? launch_mfma(tp, tasks, sp, kv_dtype, D, G, two, s)
                            : launch_valu(tp, tasks, sp, kv_dtype, sp.kernel_d, G, two, s);
}

// Workgroups per CU of the (single-tier, separate K / V loads) kernel the
// plan selects; 0 when no device answers.
int tiled_wgs_per_cu(const SplitPlan& sp, int32_t kv_dtype, int32_t D) {
  SplitPlan q = sp;
  int wgs = 0;
  q.occupancy_query = &wgs;
  TiledParams tp{};
  tp.D = D;
  return dispatch_tiled(tp, 0, q, kv_dtype, D, false, nullptr) == hipSuccess ? wgs : 0;
}

// ---------------------------------------------------------------- row cuts
// The windows in which the plan departs from the launch-time model below
// (model_split_blocks: whole rows unless few long rows need splitting), all
// in this block. A "row" is a (sequence, kv head, head-group pass) of the
// launch; rows per CU = rows / the device's CUs; fill = the rows' mean
// length over the table width, from the caller's token total (0: unknown).
// Row windows are open below and closed above (lo < rows per CU <= hi),
// fill windows closed below. tests/test_plan_info.py pins both sides of
// every boundary.
//
//   plan          kernel            D      rows per CU   fill          tasks
//   slot fill     mm, 16 heads      any    (0, 1.5]      (0, 0.8)      3 WGs/CU, 65-130 % filled, <= 8 per row
//   quarter rows  VALU or mm        128    (1.0, 1.3]    any           4 per row of the table, 3 WGs/CU
//   quarter rows  VALU or mm        64     (1.0, 1.3]    [0.95, 1]     4 per row, 3 WGs/CU
//   half rows     VALU or mm        128    (2.0, 2.6]    [0.8, 1]      2 per row, 3 WGs/CU
//   half rows     VALU or mm        64     (2.0, 2.6]    [0.95, 1]     2 per row, 3 WGs/CU
//   wave blocks   VALU              128    tasks <= CUs  any           a task's waves work by row length
//
// Why each window (measured on MI355X, bf16 unless stated, HIP graph replay,
// the same call with and without the plan):
//   * slot fill: the matrix-core kernel's per-block chain (scores MFMAs, the
//     cross-row max, the LDS round trip of V, the P.V MFMAs) makes one
//     workgroup a slow stream, so uneven rows leave the CUs holding the
//     longest ones working long after the rest; three workgroups per CU,
//     each with a share, end together. 8 / 1 heads, batch 256, rows of
//     U[1024, 4096]: 67.4 -> 61.7 us; +8 to +17 % over 17 shapes of rows of
//     U[L/4, L] and U[L/16, L]. Equal rows lose under it (86.7 -> 101.2 us at
//     4096 tokens: a second round of whole tasks), so it needs the total.
//     Past 1.5 rows per CU mixed rows balance by themselves (-3 to -6 % split
//     at two per CU); a cut into one task per row would drop the model's
//     two-per-CU cap (-9 to -12 %), so a fill always splits.
//   * quarter rows: with whole rows, the rows past one per CU land as second
//     workgroups on CUs that already stream one, and those CUs take about
//     twice as long. 8 / 1 heads at 272 rows of 4096 tokens 136.4 -> 104.2 us;
//     MHA (VALU) at 288 rows 121.6 -> 100.2 us; the gain is gone by about 1.5
//     rows per CU. At D = 64 quarters lost on near-full rows of mixed length
//     (fill 0.8-0.9: up to -20 %) and gained 10-20 % on equal ones, hence the
//     0.95 fill there.
//   * half rows: the same effect past two rows per CU under the two-per-CU
//     cap, for full rows only (8 / 1 heads, 528-640 rows of 4096 tokens:
//     216.1 / 264.9 / 278.0 -> 196.3 / 205.8 / 210.1 us); rows of mixed length
//     balance by themselves and lose 3-11 % split.
//   * wave blocks: see plan_decode.
constexpr int kFillPerCu = 3;            // workgroups per CU the cut plans run at
constexpr int32_t kMinFillBlocks = 16;   // smallest task a cut makes (16-token tiles)
constexpr int32_t kMaxFillSplits = 8;    // slot fill: at most this many tasks per row
constexpr double kMaxFillRows = 0.8;     // slot fill: mean fill below this (rows uneven)
constexpr int kMaxFillRowsPerCu10 = 15;  // slot fill: at most 1.5 rows per CU (in tenths)
constexpr double kMinFillSlots = 0.65;   // slot fill: expected tasks as a share of the
constexpr double kMaxFillSlots = 1.3;    // three-per-CU slots, at least / at most

// The quarter- and half-row windows of the table above.
struct RowCut {
  int32_t head_size;  // the head size the window applies to
  int lo10, hi10;     // lo10 / 10 < rows per CU <= hi10 / 10
  double fill_lo;     // mean fill >= fill_lo (0: the total may be unknown)
  int32_t parts;      // a row of the table's width is cut into this many tasks
};
constexpr RowCut kRowCuts[] = {
    {128, 10, 13, 0.0, 4},
    {64, 10, 13, 0.95, 4},
    {128, 20, 26, 0.8, 2},
    {64, 20, 26, 0.95, 2},
};

// Tasks a launch is expected to run with S tasks per full row when its rows
// fill `fill` of the table width on average (a row of fill x has ceil(x S)
// tasks; about fill * S + 1/2 per row).
double expected_tasks(int32_t n, int32_t kv_tasks, int64_t S, double fill) {
  return (double)n * kv_tasks * (S <= 1 ? 1.0 : std::min((double)S, fill * S + 0.5));
}

// Whether the slot fill's window holds: uneven rows (fill known and below
// 0.8) on the one-column-group matrix-core kernel, at up to 1.5 rows per CU.
bool slot_fill_window(const SplitPlan& sp, int64_t rows, int cus, double fill) {
  return fill > 0.0 && fill < kMaxFillRows && sp.mm && sp.kernel_g == 16 && cus > 0 &&
         rows * 10 <= (int64_t)kMaxFillRowsPerCu10 * cus;
}

// The slot fill: blocks per task such that the expected tasks make 65-130 %
// of one round of three workgroups per CU and no row splits more than eight
// ways, or 0 when no task size that splits rows does; the coarsest such size
// wins. (Past one round the few extra tasks are short ones: at 1.05-1.27
// rounds split tasks still beat the model's whole rows by 14-32 %.)
int32_t fill_split_blocks(int32_t n, int32_t kv_tasks, int32_t wt, int64_t slots, double fill) {
  const int64_t W = wt > 0 ? wt : 1;
  for (int32_t sb = kMaxSplitBlocks; sb >= kMinFillBlocks; sb /= 2) {
    const int64_t S = (W + sb - 1) / sb;
    if (S > kMaxFillSplits) break;
    const double tasks = expected_tasks(n, kv_tasks, S, fill);
    if (tasks > kMaxFillSlots * (double)slots) break;  // finer sizes only add tasks
    if (S > 1 && tasks > kMinFillSlots * (double)slots) return sb;
  }
  return 0;
}

// Quarter and half rows (kRowCuts) on the 16-bit VALU and matrix-core
// kernels: the task size (a power of two >= 16 tiles, at most the table
// width over the window's parts) of the first window that holds, or 0.
int32_t quarter_row_blocks(int32_t n, int32_t kv_tasks, int32_t D, bool f32, bool mfma,
                           int cus, int32_t wt, double fill) {
  const int64_t rows = (int64_t)n * kv_tasks;
  if (f32 || mfma || cus <= 0 || wt < 4 * kMinFillBlocks) return 0;
  for (const RowCut& c : kRowCuts) {
    if (c.head_size != D || fill < c.fill_lo || rows * 10 <= (int64_t)c.lo10 * cus ||
        rows * 10 > (int64_t)c.hi10 * cus)
      continue;
    int32_t q = kMinFillBlocks;
    while (q * 2 <= wt / c.parts) q *= 2;
    return q;
  }
  return 0;
}

}  // namespace

// Blocks per task (16 .. 256) from a launch-time model. Only the shapes are
// known on the host (row lengths live on the device), so rows are taken as
// bt_width blocks at most and half of that on average. For sb blocks per
// task (S = ceil(W / sb) tasks per row):
//   T(sb) = max(longest task bytes / per-workgroup stream rate,
//               (KV bytes + split partials) / min(HBM rate, tasks * that rate))
//           + the combine launch when rows split (S > 1).
// One workgroup streams ~50 GB/s when a block of one kv head holds 8 KiB of
// K and V (D = 128 at 16 bits; its waves keep a block each in flight) and
// proportionally less for smaller blocks (D = 64: ~25 GB/s), the GPU
// ~6 TB/s, and the split costs a second launch of ~8 us: so short, few rows
// run unsplit (one launch), few long rows split until enough tasks keep HBM
// busy. The constants were fitted to measured launches of MHA and GQA-4
// shapes at D = 128 (batch 1-64, 128-16k tokens), where the choice lands
// within 4 % of the best split size; the per-block scaling to a sweep of
// small-kv-head shapes (8/1, 12/2, 14/2 at D = 64, 28/4, 32/8, 71/1 at D = 64;
// batch 32-256, 1-4k tokens), where it cut the mean excess over the best
// fixed size from 7.4 % to 0.7 % (D = 64 rows were split too little).
int32_t model_split_blocks(int32_t n, int32_t H, int32_t KVH, int32_t D, int32_t BS,
                           int32_t bt_width, int32_t elt) {
  constexpr double kWgRate = 50e9, kWgBlock = 8192.0, kHbmRate = 6e12, kCombine = 8e-6,
                   kFill = 0.5;
  const int64_t W = bt_width > 0 ? bt_width : 1;
  const double blk = (double)BS * 2.0 * D * elt;  // K and V of one block, one kv head
  const double wg_rate = kWgRate * std::min(1.0, blk / kWgBlock);
  int32_t best = kMaxSplitBlocks;
  double best_t = 0.0;
  for (int32_t sb = kMaxSplitBlocks; sb >= 16; sb /= 2) {
    const int64_t S = (W + sb - 1) / sb;
    const bool split = S > 1;
    const double tasks = (double)n * KVH * std::max(1.0, S * kFill);
    const double longest = (double)std::min<int64_t>(W, sb) * blk;
    const double kv = (double)n * W * kFill * KVH * blk;
    const double part = split ? (double)n * H * S * kFill * D * 8.0 : 0.0;
    const double t = std::max(longest / wg_rate, (kv + part) / std::min(kHbmRate, tasks * wg_rate)) +
                     (split ? kCombine : 0.0);
    if (sb == kMaxSplitBlocks || t < best_t) {
      best = sb;
      best_t = t;
    }
  }
  return best;
}

SplitPlan plan_decode(int32_t n, int32_t H, int32_t KVH, int32_t D, int32_t BS,
                      int32_t bt_width, int32_t kv_dtype, bool aligned, bool matrix,
                      double fill) {
  SplitPlan sp{};
  sp.passes = 1;
  const int G = KVH > 0 ? H / KVH : 0;
  // The tiled kernels are built for 1, 2, 4 or 8 query heads per task (16 on
  // the matrix-core P.V kernel): a group of 3 runs in a 4-head kernel, of 5-7
  // in an 8-head one (the spare head slots repeat a real head and write
  // nothing), and more heads per kv head than a task holds run as passes,
  // each re-reading the blocks.
  const bool f32 = kv_dtype == FD_F32;
  // (fp32 KV at D > 128: passes of 4, its 8-head kernel would spill)
  sp.kernel_g = G <= 1 ? 1 : G == 2 ? 2 : (G <= 4 || (f32 && D > 128)) ? 4 : 8;
  // head sizes are built for 64, 128 and 256; any other multiple of 8 up to
  // 256 runs in the next larger one on the VALU kernel (its spare lanes idle)
  sp.kernel_d = D <= 64 ? 64 : D <= 128 ? 128 : 256;
  // cache blocks of 16 * m tokens are m 16-token tiles to the tiled kernels
  sp.fast = aligned && BS % kTileTokens == 0 && BS <= kMaxBlockSize && D % 8 == 0 && D >= 8 &&
            D <= 256 && G >= 1 &&
            G <= kMaxHeadGroup && (kv_dtype == FD_F16 || kv_dtype == FD_BF16 || f32);
  if (!sp.fast) {
    sp.split_blocks = bt_width > 0 ? bt_width : 1;
    sp.max_splits = 1;
    return sp;
  }
  const Tuning tune = read_tuning();
  sp.no_kv_adj = tune.kv_adj != nullptr && strcmp(tune.kv_adj, "0") == 0;
  // tasks, splits and the model count 16-token tiles (BS / 16 per block)
  const int64_t tiles = (int64_t)(bt_width > 0 ? bt_width : 0) * (BS / kTileTokens);
  const int32_t wt = (int32_t)std::min<int64_t>(tiles, INT32_MAX);
  // Kernel family (one box, vLLM layout, rows longest first, D = 128):
  //   * 4 and more query heads per kv head take the kernel with both
  //     products on the matrix cores at D <= 128 (16 query heads per task),
  //     the one with only the scores there at D = 256. At n = 64 / 256, 8 kv
  //     heads, bf16: G = 4 5.88 / 6.81 TB/s against 5.76 / 6.75 (scores
  //     only) and 5.67 / 6.79 (VALU); G = 8 5.48 / 6.64 against 4.88 / 6.12
  //     and 2.86 / 3.08.
  //   * MHA at D = 128 takes it too on large launches: with >= 8 tasks per
  //     CU and rows that may reach 1,024 tokens it reads 0.5-1.3 % faster
  //     than the VALU kernel (n = 64-256 x 32 heads, fp16 / bf16, L in
  //     [256, 2048] or [1024, 4096]); with fewer tasks its longer per-block
  //     chain loses (n = 32: -3 %), and so it does on short rows (L <= 512:
  //     -1 %). G = 2 / 3 and D = 64 stay on the VALU kernel (G = 2, n = 128:
  //     6.79 against 6.74 TB/s; MHA D = 64: 6.50 against 6.03).
  //   * other head sizes: the P.V-on-MFMA kernel is built for every multiple
  //     of 16 from 32 to 128 (the q.K-only one for 64, 128 and 256 only). At
  //     D = 32 / 48 / 80 / 96 / 112 (n = 128, L in [256, 2048], bf16) it
  //     takes groups of 8 at 3.69 / 3.51 / 4.45 / 5.22 / 4.88 TB/s against
  //     1.80 / 2.63 / 1.99 / 2.39 / 2.78 on the VALU kernel; groups of 4 gain
  //     where D is a multiple of 32 (D = 32: 3.67 against 3.05; D = 96 ties)
  //     and tie or lose where the last q.K step is half empty (48 / 80 / 112:
  //     3.48 / 4.43 / 4.86 against 3.53 / 4.47 / 5.22), so there it takes
  //     groups of 5 and more. MHA at these sizes loses 5-25 % and stays on the
  //     VALU kernel. (K + V runs of 320 or 448 bytes straddle cache lines;
  //     both kernels read those sizes slower.)
  const bool matrix_ok = matrix && !f32 && !tune.kernel_forced("valu");
  const int cus = device_cus();
  const bool big_mha = G == 1 && D == 128 && cus > 0 && (int64_t)n * KVH >= 8LL * cus &&
                       wt >= 1024 / kTileTokens;
  const bool mm_g = D % 32 == 0 ? G >= 4 : G >= 5;
  sp.mfma = matrix_ok && G >= 4 && D == sp.kernel_d;
  sp.mm = matrix_ok && D % 16 == 0 && D >= 32 && D <= 128 &&
          (tune.kernel_forced("mm") || ((mm_g || big_mha) && !tune.kernel_forced("mfma")));
  if (sp.mm) {
    sp.mfma = false;
    // more than 16 heads per kv head (multi-query models): tasks of two or
    // four groups of 16 columns (four up to D = 64, where the registers
    // allow), so fewer passes re-read the blocks
    const int cg = G <= 16 ? 1 : (G <= 32 || D > 64) ? 2 : 4;
    sp.kernel_g = 16 * cg;
  }
  sp.passes = (G + sp.kernel_g - 1) / sp.kernel_g;
  int sb = tune.split_blocks ? atoi(tune.split_blocks) : 0;
  if (sb > kMaxSplitBlocks) sb = kMaxSplitBlocks;  // 64 block ids per wave
  // each pass streams the blocks once more: count it as that many kv heads
  const int32_t kv_tasks = KVH * sp.passes;
  const int elt = f32 ? 4 : 2;
  bool filled = false;
  if (sb <= 0 && slot_fill_window(sp, (int64_t)n * kv_tasks, cus, fill)) {
    sb = fill_split_blocks(n, kv_tasks, wt, (int64_t)kFillPerCu * cus, fill);
    filled = sb > 0;
  }
  bool quartered = false;
  if (sb <= 0) {
    sb = model_split_blocks(n, H, kv_tasks, D, kTileTokens, wt, elt);
    const int32_t q = quarter_row_blocks(n, kv_tasks, D, f32, sp.mfma, cus, wt, fill);
    if (q > 0 && q < sb) {
      sb = q;
      quartered = true;
    }
  }
  sp.split_blocks = sb;
  sp.max_splits = wt > 0 ? (wt + sb - 1) / sb : 1;
  // The slot fill and quarter rows run at three workgroups per CU (a cap
  // where the kernel would hold more; its own occupancy where that is three).
  sp.wg_cap = filled || quartered
                  ? (tiled_wgs_per_cu(sp, kv_dtype, D) > kFillPerCu ? kFillPerCu : 0)
                  : sb >= 32 ? 2 : 0;
  // Working waves by row length: in a launch of at most one task per CU on
  // the VALU kernel at D = 128 (small batches), a task's four waves work
  // only as far as its range holds a quarter of the longest task's blocks
  // each; a task of half that works with two waves, and so on. One CU keeps
  // at most about 64 KiB of reads in flight (one task's four waves with two
  // 8 KiB blocks each), so the CUs that hold the longest rows of a batch of
  // mixed lengths stream no faster than that allows and finish last; the
  // short rows, with fewer blocks in flight, leave them a larger share of
  // HBM while all rows stream. Measured on MI355X (n = 8, 32 heads, rows of
  // U[128, 1024] tokens, HIP graph replay): 16.7 -> 15.9 us. (Sixteen waves
  // per task, four times the blocks in flight per CU, were slower: 17.3 us.)
  const int64_t launch_tasks = (int64_t)n * kv_tasks * sp.max_splits;
  if (!sp.mm && !sp.mfma && !f32 && D == 128 && cus > 0 && launch_tasks <= cus) {
    const int32_t longest = std::min(sb, wt > 0 ? wt : 1);
    sp.wave_blocks = (longest + kWavesPerTask - 1) / kWavesPerTask;
  }
  if (tune.wave_blocks != nullptr) sp.wave_blocks = std::max(0, atoi(tune.wave_blocks));
  if (tune.wg_cap != nullptr && *tune.wg_cap != 0) sp.wg_cap = std::max(0, atoi(tune.wg_cap));
  return sp;
}

size_t fill_workspace_bound(const SplitPlan& sp, int32_t n, int32_t H, int32_t KVH, int32_t D,
                            int32_t BS, int32_t bt_width, int32_t kv_dtype) {
  const int cus = device_cus();
  if (!sp.fast || cus <= 0 || BS % kTileTokens != 0 || bt_width <= 0) return 0;
  const int64_t wt64 = (int64_t)bt_width * (BS / kTileTokens);
  const int32_t wt = (int32_t)std::min<int64_t>(wt64, INT32_MAX);
  int64_t most = 0;
  // the slot fill: at most kMaxFillSplits tasks per row
  if (sp.mm && sp.kernel_g == 16)
    most = std::min<int64_t>(kMaxFillSplits, (wt64 + kMinFillBlocks - 1) / kMinFillBlocks);
  // half rows for full rows (quarter_row_blocks given a total)
  const int32_t half = quarter_row_blocks(n, KVH * sp.passes, D, kv_dtype == FD_F32, sp.mfma, cus,
                                          wt, 1.0);
  if (half > 0) most = std::max<int64_t>(most, (wt64 + half - 1) / half);
  if (most <= 1) return 0;
  SplitPlan b = sp;
  b.max_splits = (int32_t)most;
  return decode_workspace_bytes(b, n, H, D);
}

size_t decode_workspace_bytes(const SplitPlan& sp, int32_t n, int32_t H, int32_t D) {
  if (sp.max_splits <= 1) return 0;
  const size_t parts = (size_t)n * H * sp.max_splits;
  return parts * D * sizeof(float) + parts * sizeof(float) + 256;
}

int launch_decode(const DecodeArgs& a, const SplitPlan& sp, hipStream_t s) {
  if (a.n == 0) return FD_OK;
  if (a.timeline != nullptr && (!sp.fast || sp.mm || sp.mfma || a.kv_dtype == FD_F32))
    return set_error(FD_ERR_UNSUPPORTED,
                     "decode_timeline: the launch takes another kernel than the 16-bit VALU one");
  const bool two = a.ntiers > 1;
  if (!sp.fast) {
    GenericParams gp{};
    gp.q = a.q;
    gp.q_ss = a.q_ss;
    gp.q_sh = a.q_sh;
    gp.tier[0] = a.tier[0];
    gp.tier[1] = two ? a.tier[1] : a.tier[0];
    gp.ntiers = two ? 2 : 1;
    gp.H = a.H;
    gp.KVH = a.KVH;
    gp.D = a.D;
    gp.BS = a.BS;
    gp.scale = a.scale;
    gp.dt = a.kv_dtype;
    gp.out = a.out;
    gp.out_ss = a.out_ss;
    gp.out_sh = a.out_sh;
    gp.out_dt = a.out_dtype;
    gp.lse = a.lse;
    gp.lse_sh = a.lse_sh;
    if ((int64_t)a.n * a.H > INT32_MAX)
      return set_error(FD_ERR_UNSUPPORTED, "decode: too many (sequence, head) pairs");
    hipLaunchKernelGGL(decode_generic_kernel, dim3((unsigned)((int64_t)a.n * a.H)), dim3(kWave),
                       0, s, gp);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? FD_OK : hip_error(e, "decode_generic_kernel launch");
  }
  // the tiled kernels address q and the caches in 16-bit words: an fp32
  // element is two of them
  const bool f32 = a.kv_dtype == FD_F32;
  const int64_t ew = f32 ? 2 : 1;
  TiledParams tp{};
  tp.q = static_cast<const uint16_t*>(a.q);
  tp.q_ss = a.q_ss * ew;
  tp.q_sh = a.q_sh * ew;
  for (int t = 0; t < 2; ++t) {
    const KvTier& kt = a.tier[two ? t : 0];
    TierParams& tt = tp.tier[t];
    tt.k = static_cast<const uint16_t*>(kt.k);
    tt.v = static_cast<const uint16_t*>(kt.v);
    tt.sb = kt.sb * ew;
    tt.sh = kt.sh * ew;
    tt.st = kt.st * ew;
    tt.num_blocks = kt.num_blocks;
    tt.run_bytes = (uint32_t)(((int64_t)(kTileTokens - 1) * kt.st + a.D) * 2 * ew);
    // vLLM's cache keeps a token's V right after its K (v == k + D): the VALU
    // kernel then reads both in one load (16-bit tier 0 only; the host tier
    // of a split keeps separate K and V tensors).
    tt.kv_adj = t == 0 && !f32 && (a.D == 128 || a.D == 256) && !sp.no_kv_adj &&
                static_cast<const char*>(kt.v) == static_cast<const char*>(kt.k) + (int64_t)a.D * 2;
    tt.k_run_bytes = tt.run_bytes + (tt.kv_adj ? (uint32_t)a.D * 2 : 0u);
    tt.bt = kt.bt;
    tt.bt_stride = kt.bt_stride;
    tt.bt_width = kt.bt_width;
    tt.lens = kt.lens;
  }
  // in a launch of at most one task per CU (working waves by row length) every
  // task starts at once, so the dispatch order changes nothing; without it a
  // task's first dependent load (its row's place in the order) goes away
  tp.order = sp.wave_blocks > 0 ? nullptr : a.order;
  tp.n = a.n;
  tp.H = a.H;
  tp.KVH = a.KVH;
  tp.D = a.D;
  tp.BS = a.BS;
  tp.tpb = a.BS / kTileTokens;
  tp.hpk = a.H / a.KVH;
  tp.passes = sp.passes;
  tp.scale_log2 = a.scale * kLog2e;
  tp.out = a.out;
  tp.out_ss = a.out_ss;
  tp.out_sh = a.out_sh;
  tp.out_f32 = a.out_dtype == FD_F32;
  tp.lse = a.lse;
  tp.lse_sh = a.lse_sh;
  tp.S = sp.max_splits;
  tp.split_blocks = sp.split_blocks;
  tp.wave_blocks = sp.wave_blocks;
  tp.xcd_group = a.D % 64 != 0;
  tp.timeline = a.timeline;
  const size_t parts = (size_t)a.n * a.H * sp.max_splits;
  if (sp.max_splits > 1) {
    char* ws = static_cast<char*>(a.workspace);
    tp.part_o = reinterpret_cast<float*>(ws);
    tp.part_lse = reinterpret_cast<float*>(ws + parts * a.D * sizeof(float));
  }
  const int64_t tasks = (int64_t)a.n * a.KVH * sp.passes * sp.max_splits;
  if (tasks > INT32_MAX) return set_error(FD_ERR_UNSUPPORTED, "decode: too many tasks");
  if (a.timeline != nullptr && tasks > a.timeline_tasks)
    return set_error(FD_ERR_INVALID, "decode_timeline: %lld workgroups, room for %lld",
                     (long long)tasks, (long long)a.timeline_tasks);
  hipError_t e = dispatch_tiled(tp, (unsigned)tasks, sp, a.kv_dtype, a.D, two, s);
  if (e != hipSuccess) return hip_error(e, "decode kernel launch");
  if (sp.max_splits > 1) {
    const int64_t threads = (int64_t)a.n * a.H * (a.D / 4);
    hipLaunchKernelGGL(combine_splits_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, s, tp.part_o, tp.part_lse, a.tier[0].lens,
                       two ? a.tier[1].lens : nullptr, a.tier[0].bt_width * tp.tpb,
                       two ? a.tier[1].bt_width * tp.tpb : 0, a.n, a.H, a.D, sp.max_splits,
                       sp.split_blocks, kTileTokens, a.out, a.out_ss, a.out_sh, a.out_dtype, a.lse,
                       a.lse_sh);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "combine_splits_kernel launch");
  }
  return FD_OK;
}

}  // namespace fd
