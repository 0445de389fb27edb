// Allocation-free variant of the paged partial decode entry point.
//
// fd_paged_decode_partial takes its split workspace (the fp32 partials of
// rows longer than one task) from the caller. Callers that cannot allocate
// device memory at all (code under stream capture, tight serving loops)
// call fd_paged_decode_partial_noalloc instead: the same kernels, with the
// workspace taken from `scratch`, a fixed-size array in device memory that
// each GPU holds for the life of the process.
//
// `scratch` is a __device__ symbol: in host code its name is only a host-side
// stand-in, so its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept; launches take that
// address, never the symbol. The kernels write every split partial before
// the combine reads it, so the array needs no clearing between calls. Calls
// that overlap on one GPU (other streams, other threads) share the array and
// race; calls on one stream run in order.
#include <atomic>
#include <mutex>

#include "fd_common.h"

namespace {

constexpr size_t kScratchBytes = (size_t)FD_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch[kMaxScratchDevices] = {};
std::mutex g_scratch_lock;

// Device address of the current device's `scratch`, looked up on the first
// call on that device.
int scratch_address(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fd::hip_error(e, "decode_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fd::set_error(FD_ERR_UNSUPPORTED, "decode_noalloc: device %d beyond %d devices", dev,
                         kMaxScratchDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_lock);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return fd::hip_error(e, "decode_noalloc: hipGetSymbolAddress");
      if (p == nullptr)
        return fd::set_error(FD_ERR_HIP, "decode_noalloc: scratch has no device address");
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return FD_OK;
}

}  // namespace

extern "C" int fd_paged_decode_partial_noalloc(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, const int32_t* row_order, int32_t n, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_size, int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head, int32_t out_dtype, float* lse,
    int64_t lse_stride_head, void* stream) {
  // The size query plans for the fast kernels, the only ones with split
  // partials, so it bounds what the call below can need; it is pure host code.
  size_t need = 0;
  if (n > 0 && num_heads > 0 && num_kv_heads > 0 && head_size > 0 && block_size > 0 &&
      bt_width >= 0) {
    const int rc = fd_paged_decode_workspace_size(n, num_heads, num_kv_heads, head_size,
                                                  block_size, bt_width, &need);
    if (rc != FD_OK) return rc;
  }
  if (need > kScratchBytes)
    return fd::set_error(FD_ERR_WORKSPACE,
                         "decode_noalloc: these sizes need %zu bytes of split workspace, more "
                         "than the %zu-byte scratch of the allocation-free entry point; call "
                         "fd_paged_decode_partial with a workspace instead",
                         need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != FD_OK) return rc;
  }
  return fd_paged_decode_partial(q, q_stride_seq, q_stride_head, k_cache, v_cache,
                                 kv_stride_block, kv_stride_head, kv_stride_token, num_blocks,
                                 block_table, bt_stride, bt_width, lens, row_order, n, num_heads,
                                 num_kv_heads, head_size, block_size, scale, kv_dtype, out,
                                 out_stride_seq, out_stride_head, out_dtype, lse, lse_stride_head,
                                 ws, need > 0 ? kScratchBytes : 0, stream);
}
