// extern "C" entry points of libfdattn.so: argument validation on the host,
// error reporting, pinned host memory, then the kernel launchers.
//
// Every check runs before any launch, so a rejected call writes nothing
// (the contract of fastdecode/csrc/cpu_attn.cpp:433-477 and :495-510, where
// TORCH_CHECK raises before the kernel runs).
#include <algorithm>
#include <mutex>
#include <unordered_map>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "fd_common.h"

namespace fd {

namespace {
thread_local char g_err[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_error(hipError_t e, const char* what) {
  return set_error(FD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {

bool valid_dtype(int dt) { return dt == FD_F16 || dt == FD_BF16 || dt == FD_F32; }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Whether p points into pinned host memory, which the GPU reads over the link.
// The answer for each recently seen pointer is kept per thread (a lookup
// costs ~1 us; a layer's caches keep their addresses), and a stale entry
// after a free can only change which of two correct kernels runs.
bool in_host_memory(const void* p) {
  struct Entry {
    const void* p;
    bool host;
  };
  constexpr int kEntries = 128;
  static thread_local Entry cache[kEntries] = {};
  static thread_local int next = 0;
  for (const Entry& e : cache)
    if (e.p == p) return e.host;
  hipPointerAttribute_t attr{};
  const hipError_t rc = hipPointerGetAttributes(&attr, p);
  if (rc != hipSuccess) (void)hipGetLastError();  // an unknown pointer leaves no error behind
  const bool host = rc == hipSuccess && attr.type == hipMemoryTypeHost;
  cache[next] = {p, host};
  next = (next + 1) % kEntries;
  return host;
}

// Blocks made by fd_host_alloc and the device that was current then: the
// device whose queued work fd_host_free waits for.
std::mutex g_host_mu;
std::unordered_map<void*, int>& host_blocks() {
  static auto* m = new std::unordered_map<void*, int>();  // outlives static destructors
  return *m;
}

// Mean fill of the table by the rows, from the caller's token total: the
// rows' tokens over n * width * block_size, at most 1 (0: unknown).
double row_fill(int64_t total_tokens, int32_t n, int64_t width, int32_t block_size) {
  if (total_tokens <= 0 || n <= 0 || width <= 0) return 0.0;
  const double cap = (double)n * (double)width * block_size;
  return std::min(1.0, (double)total_tokens / cap);
}

// Validates a decode call over a.ntiers tiers (tiers already filled in),
// completes `a` and launches it. Every check runs before the launch.
// total_tokens: the rows' token total when the caller knows it (0: unknown);
// it only steers the task sizes, never the results.
int run_decode(DecodeArgs& a, const char* who, const void* q, int64_t q_stride_seq,
               int64_t q_stride_head, const int32_t* row_order, int32_t n, int32_t num_heads,
               int32_t num_kv_heads, int32_t head_size, int32_t block_size, float scale,
               int32_t kv_dtype, void* out, int64_t out_stride_seq, int64_t out_stride_head,
               int32_t out_dtype, float* lse, int64_t lse_stride_head, void* workspace,
               size_t workspace_bytes, void* stream, int64_t total_tokens = 0) {
  if (n < 0) return set_error(FD_ERR_INVALID, "%s: n must be >= 0 (got %d)", who, n);
  if (total_tokens < 0)
    return set_error(FD_ERR_INVALID, "%s: total_tokens must be >= 0 (got %lld)", who,
                     (long long)total_tokens);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return set_error(FD_ERR_INVALID,
                     "%s: num_heads must be a multiple of num_kv_heads (%d, %d)", who, num_heads,
                     num_kv_heads);
  if (head_size <= 0 || head_size > 512)
    return set_error(FD_ERR_UNSUPPORTED, "%s: head_size %d outside 1..512", who, head_size);
  if (block_size <= 0) return set_error(FD_ERR_INVALID, "%s: block_size must be > 0", who);
  if (kv_dtype != FD_F16 && kv_dtype != FD_BF16 && kv_dtype != FD_F32)
    return set_error(FD_ERR_INVALID, "%s: unsupported kv dtype %d", who, kv_dtype);
  if (out_dtype != kv_dtype && out_dtype != FD_F32)
    return set_error(FD_ERR_INVALID, "%s: out dtype must equal the kv dtype or be fp32", who);
  if (!std::isfinite(scale)) return set_error(FD_ERR_INVALID, "%s: scale is not finite", who);
  int64_t width = 0;
  for (int t = 0; t < a.ntiers; ++t) {
    if (a.tier[t].bt_width < 0 || a.tier[t].num_blocks < 0)
      return set_error(FD_ERR_INVALID, "%s: negative size (tier %d)", who, t);
    width += a.tier[t].bt_width;
  }
  if (width > INT32_MAX) return set_error(FD_ERR_UNSUPPORTED, "%s: table too wide", who);
  if (n == 0) return FD_OK;
  if (!q || !out || !lse) return set_error(FD_ERR_INVALID, "%s: NULL tensor pointer", who);
  for (int t = 0; t < a.ntiers; ++t) {
    const KvTier& kt = a.tier[t];
    if (!kt.k || !kt.v || !kt.bt || !kt.lens)
      return set_error(FD_ERR_INVALID, "%s: NULL tensor pointer (tier %d)", who, t);
    if (kt.bt_width > 0 && kt.bt_stride < kt.bt_width)
      return set_error(FD_ERR_INVALID, "%s: bt_stride %lld < bt_width %d (tier %d)", who,
                       (long long)kt.bt_stride, kt.bt_width, t);
  }

  // An empty cache goes to the generic kernel, which never reads it.
  bool aligned = aligned16(q) && aligned16(out) && q_stride_seq % 8 == 0 &&
                 q_stride_head % 8 == 0 && out_stride_seq % 8 == 0 && out_stride_head % 8 == 0;
  for (int t = 0; t < a.ntiers; ++t) {
    const KvTier& kt = a.tier[t];
    aligned = aligned && kt.num_blocks > 0 && aligned16(kt.k) && aligned16(kt.v) &&
              kt.sb % 8 == 0 && kt.sh % 8 == 0 && kt.st % 8 == 0 &&
              // one (block, head) run must be addressable by a 32-bit offset
              ((int64_t)(block_size - 1) * kt.st + head_size) * (kv_dtype == FD_F32 ? 4 : 2) <
                  (1ll << 31);
  }
  const double fill = row_fill(total_tokens, n, width, block_size);
  SplitPlan sp = plan_decode(n, num_heads, num_kv_heads, head_size, block_size,
                             (int32_t)width, kv_dtype, aligned, true, fill);
  // Over the link the matrix-core kernels' K tiles (16 token rows of 16 bytes
  // per lane group) read slower than the VALU kernel's whole rows (measured
  // on a GQA-4 host tier: 47.9 against 55.9 GB/s; in HBM the two are within
  // 3 %), so launches that read pinned host memory take the VALU kernel.
  bool host = false;
  for (int t = 0; (sp.mfma || sp.mm) && t < a.ntiers; ++t) host = host || in_host_memory(a.tier[t].k);
  if (host)
    sp = plan_decode(n, num_heads, num_kv_heads, head_size, block_size, (int32_t)width, kv_dtype,
                     aligned, false, fill);
  const size_t need = decode_workspace_bytes(sp, n, num_heads, head_size);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
    return set_error(FD_ERR_WORKSPACE,
                     "%s: workspace of %zu bytes (16-byte aligned) required, got %zu", who, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);

  a.q = q;
  a.q_ss = q_stride_seq;
  a.q_sh = q_stride_head;
  a.order = row_order;
  a.n = n;
  a.H = num_heads;
  a.KVH = num_kv_heads;
  a.D = head_size;
  a.BS = block_size;
  a.scale = scale;
  a.kv_dtype = kv_dtype;
  a.out = out;
  a.out_ss = out_stride_seq;
  a.out_sh = out_stride_head;
  a.out_dtype = out_dtype;
  a.lse = lse;
  a.lse_sh = lse_stride_head;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return launch_decode(a, sp, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" {

const char* fd_last_error(void) { return g_err; }

int fd_abi_version(void) { return 12; }

int fd_paged_decode_workspace_size(int32_t n, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_size, int32_t block_size, int32_t bt_width,
                                   size_t* bytes) {
  if (bytes == nullptr) return set_error(FD_ERR_INVALID, "workspace_size: bytes is NULL");
  if (n < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 ||
      bt_width < 0)
    return set_error(FD_ERR_INVALID, "workspace_size: bad sizes");
  // The aligned fast path is the only one that needs workspace; size for
  // every kernel it may take (the kernels' head passes and the fp32 stream
  // may split rows differently): 16-bit KV with or without the matrix-core
  // kernels (a tier in pinned host memory takes the VALU kernel), fp32 KV.
  size_t most = 0;
  const int32_t dts[3] = {FD_F16, FD_F16, FD_F32};
  for (int c = 0; c < 3; ++c) {
    const SplitPlan sp = plan_decode(n, num_heads, num_kv_heads, head_size, block_size, bt_width,
                                     dts[c], true, c == 0);
    most = std::max(most, decode_workspace_bytes(sp, n, num_heads, head_size));
    // what a token total may make of it (fd_paged_decode_partial_hint)
    most = std::max(most, fill_workspace_bound(sp, n, num_heads, num_kv_heads, head_size,
                                               block_size, bt_width, dts[c]));
  }
  *bytes = most;
  return FD_OK;
}

int fd_decode_plan_info(int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                        int32_t block_size, int32_t bt_width, int32_t kv_dtype, int32_t aligned,
                        int32_t host_tier, int64_t total_tokens, FdDecodePlan* plan) {
  if (plan == nullptr) return set_error(FD_ERR_INVALID, "plan_info: plan is NULL");
  if (n < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_size <= 0 || block_size <= 0 || bt_width < 0 || total_tokens < 0)
    return set_error(FD_ERR_INVALID, "plan_info: bad sizes");
  const double fill = row_fill(total_tokens, n, bt_width, block_size);
  if (kv_dtype != FD_F16 && kv_dtype != FD_BF16 && kv_dtype != FD_F32)
    return set_error(FD_ERR_INVALID, "plan_info: unsupported kv dtype %d", kv_dtype);
  // the same two-step choice as run_decode: a tier in pinned host memory
  // re-plans 16-bit launches without the matrix-core kernels
  SplitPlan sp = plan_decode(n, num_heads, num_kv_heads, head_size, block_size, bt_width, kv_dtype,
                             aligned != 0, true, fill);
  if (host_tier != 0 && (sp.mfma || sp.mm))
    sp = plan_decode(n, num_heads, num_kv_heads, head_size, block_size, bt_width, kv_dtype,
                     aligned != 0, false, fill);
  plan->kernel = !sp.fast ? FD_KERNEL_GENERIC
                 : kv_dtype == FD_F32 ? FD_KERNEL_F32
                 : sp.mm ? FD_KERNEL_MM
                 : sp.mfma ? FD_KERNEL_MFMA
                           : FD_KERNEL_VALU;
  plan->heads_per_task = sp.fast ? sp.kernel_g : 1;
  plan->passes = sp.fast ? sp.passes : 1;
  plan->split_blocks = sp.split_blocks;
  plan->max_splits = sp.max_splits;
  plan->wg_cap = sp.fast ? sp.wg_cap : 0;
  plan->wave_blocks = sp.fast ? sp.wave_blocks : 0;
  return FD_OK;
}

int fd_paged_decode_partial(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                            const void* k_cache, const void* v_cache, int64_t kv_stride_block,
                            int64_t kv_stride_head, int64_t kv_stride_token, int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
                            const int32_t* lens, const int32_t* row_order, int32_t n,
                            int32_t num_heads,
                            int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                            float scale, int32_t kv_dtype, void* out, int64_t out_stride_seq,
                            int64_t out_stride_head, int32_t out_dtype, float* lse,
                            int64_t lse_stride_head, void* workspace, size_t workspace_bytes,
                            void* stream) {
  DecodeArgs a{};
  a.tier[0] = KvTier{k_cache, v_cache, kv_stride_block, kv_stride_head, kv_stride_token,
                     num_blocks, block_table, bt_stride, bt_width, lens};
  a.ntiers = 1;
  return run_decode(a, "decode", q, q_stride_seq, q_stride_head, row_order, n, num_heads,
                    num_kv_heads, head_size, block_size, scale, kv_dtype, out, out_stride_seq,
                    out_stride_head, out_dtype, lse, lse_stride_head, workspace,
                    workspace_bytes, stream);
}

int fd_paged_decode_partial_hint(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head,
    int64_t kv_stride_token, int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
    int32_t bt_width, const int32_t* lens, const int32_t* row_order, int32_t n,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_size, int32_t block_size, float scale,
    int32_t kv_dtype, void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype, float* lse, int64_t lse_stride_head, void* workspace,
    size_t workspace_bytes, void* stream, int64_t total_tokens) {
  DecodeArgs a{};
  a.tier[0] = KvTier{k_cache, v_cache, kv_stride_block, kv_stride_head, kv_stride_token,
                     num_blocks, block_table, bt_stride, bt_width, lens};
  a.ntiers = 1;
  return run_decode(a, "decode", q, q_stride_seq, q_stride_head, row_order, n, num_heads,
                    num_kv_heads, head_size, block_size, scale, kv_dtype, out, out_stride_seq,
                    out_stride_head, out_dtype, lse, lse_stride_head, workspace,
                    workspace_bytes, stream, total_tokens);
}

int fd_paged_decode_timeline(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head,
    int64_t kv_stride_token, int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
    int32_t bt_width, const int32_t* lens, const int32_t* row_order, int32_t n,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_size, int32_t block_size, float scale,
    int32_t kv_dtype, void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype, float* lse, int64_t lse_stride_head, void* workspace,
    size_t workspace_bytes, void* stream, uint64_t* timeline, int64_t timeline_workgroups) {
  if (timeline == nullptr || timeline_workgroups <= 0 || !aligned16(timeline))
    return set_error(FD_ERR_INVALID,
                     "decode_timeline: timeline must be a 16-byte aligned device buffer of at "
                     "least one workgroup");
  DecodeArgs a{};
  a.tier[0] = KvTier{k_cache, v_cache, kv_stride_block, kv_stride_head, kv_stride_token,
                     num_blocks, block_table, bt_stride, bt_width, lens};
  a.ntiers = 1;
  a.timeline = timeline;
  a.timeline_tasks = timeline_workgroups;
  return run_decode(a, "decode_timeline", q, q_stride_seq, q_stride_head, row_order, n,
                    num_heads, num_kv_heads, head_size, block_size, scale, kv_dtype, out,
                    out_stride_seq, out_stride_head, out_dtype, lse, lse_stride_head, workspace,
                    workspace_bytes, stream);
}

int fd_split_decode(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                    const fd_kv_tier* hbm, const fd_kv_tier* host, const int32_t* row_order,
                    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                    int32_t block_size, float scale, int32_t kv_dtype, void* out,
                    int64_t out_stride_seq, int64_t out_stride_head, int32_t out_dtype,
                    float* lse, int64_t lse_stride_head, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (hbm == nullptr || host == nullptr)
    return set_error(FD_ERR_INVALID, "split_decode: NULL tier descriptor");
  DecodeArgs a{};
  const fd_kv_tier* tiers[2] = {hbm, host};
  for (int t = 0; t < 2; ++t) {
    const fd_kv_tier& d = *tiers[t];
    a.tier[t] = KvTier{d.k_cache, d.v_cache, d.stride_block, d.stride_head, d.stride_token,
                       d.num_blocks, d.block_table, d.bt_stride, d.bt_width, d.lens};
  }
  a.ntiers = 2;
  return run_decode(a, "split_decode", q, q_stride_seq, q_stride_head, row_order, n, num_heads,
                    num_kv_heads, head_size, block_size, scale, kv_dtype, out, out_stride_seq,
                    out_stride_head, out_dtype, lse, lse_stride_head, workspace,
                    workspace_bytes, stream);
}

int fd_plan_tiers(const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
                  const int32_t* seq_lens, int32_t n_rows, int32_t num_gpu_blocks,
                  int64_t num_cpu_blocks, int32_t block_size, int32_t* gpu_block_table,
                  int32_t* cpu_block_table, int64_t out_stride, int32_t out_width,
                  int32_t* gpu_lens, int32_t* cpu_lens, const int64_t* slot_mapping,
                  int32_t n_tokens, int64_t* gpu_slot_mapping, int64_t* host_slot_mapping,
                  int32_t* error_count, void* stream) {
  if (n_rows < 0 || n_tokens < 0 || bt_width < 0 || num_gpu_blocks < 0 || num_cpu_blocks < 0 ||
      block_size <= 0)
    return set_error(FD_ERR_INVALID, "plan_tiers: bad sizes");
  if (n_rows > 0) {
    if (!block_table || !seq_lens || !gpu_block_table || !cpu_block_table || !gpu_lens ||
        !cpu_lens)
      return set_error(FD_ERR_INVALID, "plan_tiers: NULL row pointer");
    if (bt_width > 0 && bt_stride < bt_width)
      return set_error(FD_ERR_INVALID, "plan_tiers: bt_stride < bt_width");
    if (out_width < bt_width || out_stride < out_width)
      return set_error(FD_ERR_INVALID, "plan_tiers: output tables narrower than the input");
  }
  if (n_tokens > 0 && (!slot_mapping || !gpu_slot_mapping || !host_slot_mapping))
    return set_error(FD_ERR_INVALID, "plan_tiers: NULL slot pointer");
  PlanTiersArgs a{};
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.bt_width = bt_width;
  a.seq_lens = seq_lens;
  a.n_rows = n_rows;
  a.G = num_gpu_blocks;
  a.C = num_cpu_blocks;
  a.BS = block_size;
  a.gpu_bt = gpu_block_table;
  a.cpu_bt = cpu_block_table;
  a.out_stride = out_stride;
  a.out_width = out_width;
  a.gpu_lens = gpu_lens;
  a.cpu_lens = cpu_lens;
  a.slots = slot_mapping;
  a.n_tokens = n_tokens;
  a.gpu_slots = gpu_slot_mapping;
  a.host_slots = host_slot_mapping;
  a.error_count = error_count;
  return launch_plan_tiers(a, static_cast<hipStream_t>(stream));
}

int fd_merge_attn_states(void* out, int64_t out_stride_seq, int64_t out_stride_head,
                         int32_t out_dtype, const void* o_a, int64_t a_stride_seq,
                         int64_t a_stride_head, int32_t a_dtype, const float* lse_a,
                         int64_t lse_a_stride_head, const void* o_b, int64_t b_stride_seq,
                         int64_t b_stride_head, int32_t b_dtype, const float* lse_b,
                         int64_t lse_b_stride_head, float* out_lse,
                         int64_t out_lse_stride_head, int32_t n, int32_t num_heads,
                         int32_t head_size, void* stream) {
  if (n < 0 || num_heads < 0 || head_size < 0)
    return set_error(FD_ERR_INVALID, "merge: negative size");
  if (!valid_dtype(out_dtype) || !valid_dtype(a_dtype) || !valid_dtype(b_dtype))
    return set_error(FD_ERR_INVALID, "merge: unsupported dtype");
  if ((int64_t)n * num_heads * head_size == 0) return FD_OK;
  if (!out || !o_a || !lse_a || !o_b || !lse_b)
    return set_error(FD_ERR_INVALID, "merge: NULL tensor pointer");
  MergeArgs a{};
  a.out = out;
  a.out_ss = out_stride_seq;
  a.out_sh = out_stride_head;
  a.out_dt = out_dtype;
  a.a = o_a;
  a.a_ss = a_stride_seq;
  a.a_sh = a_stride_head;
  a.a_dt = a_dtype;
  a.lse_a = lse_a;
  a.lse_a_sh = lse_a_stride_head;
  a.b = o_b;
  a.b_ss = b_stride_seq;
  a.b_sh = b_stride_head;
  a.b_dt = b_dtype;
  a.lse_b = lse_b;
  a.lse_b_sh = lse_b_stride_head;
  a.out_lse = out_lse;
  a.out_lse_sh = out_lse_stride_head;
  a.n = n;
  a.H = num_heads;
  a.D = head_size;
  return launch_merge(a, static_cast<hipStream_t>(stream));
}

int fd_reshape_and_cache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                         const void* value, int64_t value_stride_tok,
                         int64_t value_stride_head, void* k_cache, void* v_cache,
                         int64_t cache_stride_block, int64_t cache_stride_token,
                         int64_t cache_stride_head, int64_t num_blocks,
                         const int64_t* slot_mapping, int32_t num_tokens,
                         int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                         int32_t dtype, int32_t* error_count, const int32_t* write_gate,
                         void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 ||
      num_blocks < 0)
    return set_error(FD_ERR_INVALID, "reshape_and_cache: bad sizes");
  if (!valid_dtype(dtype)) return set_error(FD_ERR_INVALID, "reshape_and_cache: bad dtype");
  if (num_tokens == 0) return FD_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return set_error(FD_ERR_INVALID, "reshape_and_cache: NULL tensor pointer");
  CacheWriteArgs a{};
  a.key = key;
  a.key_st = key_stride_tok;
  a.key_sh = key_stride_head;
  a.value = value;
  a.value_st = value_stride_tok;
  a.value_sh = value_stride_head;
  a.kc = k_cache;
  a.vc = v_cache;
  a.c_sb = cache_stride_block;
  a.c_st = cache_stride_token;
  a.c_sh = cache_stride_head;
  a.num_blocks = num_blocks;
  a.slots = slot_mapping;
  a.T = num_tokens;
  a.KVH = num_kv_heads;
  a.D = head_size;
  a.BS = block_size;
  a.elt = dtype_size(dtype);
  a.err = error_count;
  a.gate = write_gate;
  if (write_gate != nullptr && write_gate == error_count)
    return set_error(FD_ERR_INVALID, "reshape_and_cache: write_gate and error_count must differ");
  return launch_cache_write(a, static_cast<hipStream_t>(stream));
}

int fd_check_slots(const int64_t* slots, int64_t m, int64_t capacity, int64_t* first_bad) {
  if (m < 0) return set_error(FD_ERR_INVALID, "check_slots: negative count");
  if (m > 0 && slots == nullptr) return set_error(FD_ERR_INVALID, "check_slots: NULL slots");
  for (int64_t j = 0; j < m; ++j) {
    if (slots[j] < 0 || slots[j] >= capacity) {
      if (first_bad) *first_bad = j;
      return set_error(FD_ERR_RANGE, "host-tier slot out of range: %lld (capacity %lld)",
                       (long long)slots[j], (long long)capacity);
    }
  }
  return FD_OK;
}

int fd_host_alloc(size_t bytes, void** host_ptr) {
  if (host_ptr == nullptr) return set_error(FD_ERR_INVALID, "host_alloc: host_ptr is NULL");
  *host_ptr = nullptr;
  if (bytes == 0) bytes = 16;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "host_alloc: hipGetDevice");
  unsigned flags = hipHostMallocMapped | hipHostMallocPortable;
  const char* nc = getenv("FD_HOST_NONCOHERENT");
  if (nc != nullptr && nc[0] == '1') flags |= hipHostMallocNonCoherent;
  e = hipHostMalloc(host_ptr, bytes, flags);
  if (e != hipSuccess) return hip_error(e, "hipHostMalloc");
  const int rc = guarded("host_alloc", [&]() -> int {
    std::lock_guard<std::mutex> lock(g_host_mu);
    host_blocks()[*host_ptr] = dev;
    return FD_OK;
  });
  if (rc != FD_OK) {  // not recorded (no memory for the entry): give the block back
    (void)hipHostFree(*host_ptr);
    *host_ptr = nullptr;
  }
  return rc;
}

int fd_host_free(void* host_ptr) {
  if (host_ptr == nullptr) return FD_OK;
  int dev = 0;
  {
    std::lock_guard<std::mutex> lock(g_host_mu);
    const auto it = host_blocks().find(host_ptr);
    if (it == host_blocks().end())
      return set_error(FD_ERR_INVALID, "host_free: %p was not allocated by fd_host_alloc",
                       host_ptr);
    dev = it->second;
  }
  // Kernels still enqueued on the tier's device may read or write the block
  // over the link: let them finish first (freeing is rare: a tier's
  // teardown). Only that device is waited for: a process that also reaches
  // the block from other devices synchronises them itself. If the wait fails
  // (e.g. a stream capture is under way), the block is not freed: a leak,
  // never a free under running kernels.
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_error(e, "host_free: hipGetDevice");
  e = dev == cur ? hipSuccess : hipSetDevice(dev);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  const hipError_t back = dev == cur ? hipSuccess : hipSetDevice(cur);
  if (e != hipSuccess) return hip_error(e, "host_free: waiting for the device's work (block kept)");
  if (back != hipSuccess) return hip_error(back, "host_free: hipSetDevice (block kept)");
  e = hipHostFree(host_ptr);
  if (e != hipSuccess) return hip_error(e, "hipHostFree");
  std::lock_guard<std::mutex> lock(g_host_mu);
  host_blocks().erase(host_ptr);
  return FD_OK;
}

int fd_host_device_pointer(void* host_ptr, void** device_ptr) {
  if (host_ptr == nullptr || device_ptr == nullptr)
    return set_error(FD_ERR_INVALID, "host_device_pointer: NULL argument");
  const hipError_t e = hipHostGetDevicePointer(device_ptr, host_ptr, 0);
  return e == hipSuccess ? FD_OK : hip_error(e, "hipHostGetDevicePointer");
}

int fd_stream_copy(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes % 16 != 0) return set_error(FD_ERR_INVALID, "stream_copy: bytes %% 16 != 0");
  if (bytes == 0) return FD_OK;
  if (!dst || !src || !aligned16(dst) || !aligned16(src))
    return set_error(FD_ERR_INVALID, "stream_copy: NULL or unaligned pointer");
  return launch_stream_copy(dst, src, bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
