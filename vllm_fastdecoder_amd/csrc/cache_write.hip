// reshape_and_cache: scatter this step's K/V rows into a paged cache by slot.
//
// One kernel for both tiers of the reference:
//   * HBM tier: vLLM's reshape_and_cache_flash (fastdecode/backend.py:270-273),
//     cache view [num_blocks, block_size, kv_heads, D] of the interleaved
//     [.., 2D] K/V cache, slots < 0 skipped (plan.py:152 marks host-tier slots
//     -1; the reference's CPU stand-in skips them,
//     tests/test_plan_and_forward.py:88-95);
//   * host tier: store_kv (fastdecode/csrc/cpu_attn.cpp:413-431), cache
//     [C, kv_heads, block_size, D] in pinned host memory written zero-copy.
// The copy is bit-exact: bytes move unchanged, 16 at a time when every row
// start is 16-byte aligned. A slot past the cache is never written; it is
// counted into an optional device error counter instead. An optional write
// gate (a device counter written by earlier work on the stream, e.g. the
// tier planner's error count) stops the whole launch when it is non-zero,
// so a step whose slots were found bad writes nothing (cpu_attn.cpp:506-510
// checks every slot before any write).
#include "fd_common.h"

namespace fd {

namespace {

// One thread moves one VEC-byte piece of one (token, head) row of K and the
// same piece of V.
template <int VEC>
__global__ __launch_bounds__(256) void cache_write_kernel(CacheWriteArgs a) {
  const int row_bytes = a.D * a.elt;
  const int pieces = row_bytes / VEC;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.T * a.KVH * pieces;
  if (tid >= total) return;
  if (a.gate != nullptr && *a.gate != 0) return;
  const int c = (int)(tid % pieces);
  const int64_t rowid = tid / pieces;
  const int g = (int)(rowid % a.KVH);
  const int j = (int)(rowid / a.KVH);
  const int64_t slot = a.slots[j];
  if (slot < 0) return;
  if (slot >= a.num_blocks * a.BS) {
    if (a.err != nullptr && g == 0 && c == 0) atomicAdd(a.err, 1);
    return;
  }
  const int64_t blk = slot / a.BS;
  const int64_t off = slot % a.BS;
  const int64_t dst = (blk * a.c_sb + off * a.c_st + (int64_t)g * a.c_sh) * a.elt + (int64_t)c * VEC;
  const int64_t srck = ((int64_t)j * a.key_st + (int64_t)g * a.key_sh) * a.elt + (int64_t)c * VEC;
  const int64_t srcv = ((int64_t)j * a.value_st + (int64_t)g * a.value_sh) * a.elt + (int64_t)c * VEC;
  using V = typename std::conditional<
      VEC == 16, uint4,
      typename std::conditional<VEC == 8, uint2,
                                typename std::conditional<VEC == 4, uint32_t, uint16_t>::type>::type>::type;
  *reinterpret_cast<V*>(static_cast<char*>(a.kc) + dst) =
      *reinterpret_cast<const V*>(static_cast<const char*>(a.key) + srck);
  *reinterpret_cast<V*>(static_cast<char*>(a.vc) + dst) =
      *reinterpret_cast<const V*>(static_cast<const char*>(a.value) + srcv);
}

template <int VEC>
hipError_t launch(const CacheWriteArgs& a, hipStream_t s) {
  const int64_t pieces = (int64_t)a.D * a.elt / VEC;
  const int64_t total = (int64_t)a.T * a.KVH * pieces;
  hipLaunchKernelGGL((cache_write_kernel<VEC>), dim3((unsigned)((total + 255) / 256)), dim3(256),
                     0, s, a);
  return hipGetLastError();
}

bool fits(int vec, const CacheWriteArgs& a) {
  const int64_t eb = a.elt;
  auto ok = [&](const void* p, int64_t s1, int64_t s2, int64_t s3) {
    return reinterpret_cast<uintptr_t>(p) % vec == 0 && (s1 * eb) % vec == 0 &&
           (s2 * eb) % vec == 0 && (s3 * eb) % vec == 0;
  };
  return ((int64_t)a.D * eb) % vec == 0 && ok(a.key, a.key_st, a.key_sh, 0) &&
         ok(a.value, a.value_st, a.value_sh, 0) && ok(a.kc, a.c_sb, a.c_st, a.c_sh) &&
         ok(a.vc, a.c_sb, a.c_st, a.c_sh);
}

}  // namespace

int launch_cache_write(const CacheWriteArgs& a, hipStream_t s) {
  if (a.T == 0 || a.KVH == 0 || a.D == 0) return FD_OK;
  hipError_t e;
  if (fits(16, a)) {
    e = launch<16>(a, s);
  } else if (fits(8, a)) {
    e = launch<8>(a, s);
  } else if (fits(4, a)) {
    e = launch<4>(a, s);
  } else {
    e = launch<2>(a, s);
  }
  return e == hipSuccess ? FD_OK : hip_error(e, "cache_write_kernel launch");
}

// ------------------------------------------------------------ stream copy
namespace {
__global__ __launch_bounds__(256) void stream_copy_kernel(uint4* __restrict__ dst,
                                                          const uint4* __restrict__ src,
                                                          int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n16; idx += stride) {
    dst[idx] = src[idx];
  }
}
}  // namespace

int launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
  const int64_t n16 = (int64_t)(bytes / 16);
  if (n16 == 0) return FD_OK;
  const int64_t want = (n16 + 255) / 256;
  const unsigned grid = (unsigned)(want < 256 * 64 ? want : 256 * 64);
  hipLaunchKernelGGL(stream_copy_kernel, dim3(grid), dim3(256), 0, s,
                     static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FD_OK : hip_error(e, "stream_copy_kernel launch");
}

}  // namespace fd
