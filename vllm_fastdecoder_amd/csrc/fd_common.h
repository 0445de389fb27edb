// Shared helpers for the gfx950 split decode-attention kernels: element
// conversions, 64-lane wavefront reductions, error reporting and launch
// bookkeeping used by every translation unit of libfdattn.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdattn.h"
#include "fd_errors.h"

namespace fd {

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors
// Converts a failed HIP call into FD_ERR_HIP with the runtime's message.
int hip_error(hipError_t e, const char* what);

inline int dtype_size(int dt) {
  return dt == FD_F32 ? 4 : (dt == FD_F16 || dt == FD_BF16) ? 2 : 0;
}

// ---------------------------------------------------------------- types
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
// matrix-core operand / accumulator vectors
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Storage tags for 16-bit KV elements. Both are moved around as raw 16-bit
// words; only the arithmetic below differs.
struct F16 {
  static constexpr int kCode = FD_F16;
};
struct BF16 {
  static constexpr int kCode = FD_BF16;
};
// fp32 KV (its outputs are always fp32).
struct F32 {
  static constexpr int kCode = FD_F32;
};

// Low / high 16-bit element of a packed 32-bit word as fp32.
__device__ __forceinline__ float lo_f32(F16, uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).x;
}
__device__ __forceinline__ float hi_f32(F16, uint32_t w) {
  return (float)__builtin_bit_cast(half2_t, w).y;
}
__device__ __forceinline__ float lo_f32(BF16, uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float hi_f32(BF16, uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}

// acc + a.lo*b.lo + a.hi*b.hi with fp32 accumulation (v_dot2_f32_{f16,bf16}).
__device__ __forceinline__ float dot2(F16, uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                __builtin_bit_cast(half2_t, b), acc, false);
}
__device__ __forceinline__ float dot2(BF16, uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                         __builtin_bit_cast(bf162_t, b), acc,
                                         false);
}

// fp32 -> 16-bit storage, round to nearest even.
__device__ __forceinline__ uint16_t from_f32(F16, float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ uint16_t from_f32(BF16, float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// A result in fp32 -> 16-bit output, rounded twice: to fp32 first (a product
// computed before the call is an fp32 value), then to nearest even in the
// 16-bit type, as the reference's from_float does (static_cast<T>(src * mul),
// fastdecode/csrc/cpu_attn.cpp:76-78). The empty asm keeps the compiler from
// fusing a preceding multiply into the conversion: a mixed-precision FMA with
// a 16-bit result rounds the exact product once, which differs in the last
// bit now and then, and would make outputs depend on which code path wrote
// them.
__device__ __forceinline__ uint16_t to_out(F16, float x) {
  asm("" : "+v"(x));
  return from_f32(F16{}, x);
}
__device__ __forceinline__ uint16_t to_out(BF16, float x) {
  asm("" : "+v"(x));
  return from_f32(BF16{}, x);
}

// Generic scalar load/store by runtime dtype (used by the slow paths).
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dt) {
  if (dt == FD_F32) return static_cast<const float*>(p)[i];
  const uint16_t w = static_cast<const uint16_t*>(p)[i];
  return dt == FD_F16 ? (float)__builtin_bit_cast(_Float16, w)
                      : __uint_as_float(static_cast<uint32_t>(w) << 16);
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dt, float x) {
  if (dt == FD_F32) {
    static_cast<float*>(p)[i] = x;
  } else if (dt == FD_F16) {
    static_cast<uint16_t*>(p)[i] = to_out(F16{}, x);
  } else {
    static_cast<uint16_t*>(p)[i] = to_out(BF16{}, x);
  }
}

// ---------------------------------------------------------------- DPP
// DPP control words (GCN/CDNA "data parallel primitives" operand modifiers).
constexpr int kDppQuadXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;   // lane i <- lane 7-i in each 8
constexpr int kDppRowMirror = 0x140;       // lane i <- lane 15-i in each 16

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl,
                                         0xF, 0xF, false));
}

// Sum over aligned groups of kLanes consecutive lanes (4, 8, 16 or 32); every
// lane of a group receives the group's sum. The butterfly uses quad
// permutes and row mirrors, so each step is one v_add_f32 with a DPP operand;
// the 32-lane step crosses DPP rows with a ds_swizzle.
template <int kLanes>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(kLanes == 4 || kLanes == 8 || kLanes == 16 || kLanes == 32,
                "group_sum: unsupported group");
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  if constexpr (kLanes >= 8) x += dpp<kDppRowHalfMirror>(x);
  if constexpr (kLanes >= 16) x += dpp<kDppRowMirror>(x);
  if constexpr (kLanes >= 32) {
    // swizzle bitmask mode: and_mask=0x1f, or_mask=0, xor_mask=0x10
    x += __builtin_bit_cast(
        float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
  }
  return x;
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) {
  return __shfl_xor(x, mask, kWave);
}

// x and the value of the lane at lane ^ kMask (kMask = 8, 16 or 32) as the
// pair (a, b), in an order that depends on the lane: a commutative op of the
// two is op(x, partner) on every lane. VALU only, no LDS round trip (a
// __shfl_xor is a ds_bpermute): kMask = 8 is a DPP row rotate by 8 (the xor-8
// partner inside a 16-lane row); 16 and 32 are gfx950's v_permlane16_swap /
// v_permlane32_swap with x as both operands, which leave [x0, x0, x2, x2]
// and [x1, x1, x3, x3] (16-lane rows), or [lo, lo] and [hi, hi] (32-lane
// halves).
constexpr int kDppRowRor8 = 0x128;  // lane i <- lane (i + 8) % 16 in each 16

template <int kMask>
__device__ __forceinline__ void xor_pair(float x, float& a, float& b) {
  static_assert(kMask == 8 || kMask == 16 || kMask == 32, "xor_pair: unsupported mask");
  if constexpr (kMask == 8) {
    a = x;
    b = dpp<kDppRowRor8>(x);
  } else {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if constexpr (kMask == 16) {
      const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      a = __builtin_bit_cast(float, (uint32_t)r[0]);
      b = __builtin_bit_cast(float, (uint32_t)r[1]);
    } else {
      const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      a = __builtin_bit_cast(float, (uint32_t)r[0]);
      b = __builtin_bit_cast(float, (uint32_t)r[1]);
    }
  }
}

// Sum / max over the lanes that differ from this one in the bits kFrom,
// 2 kFrom, .. 32 of the lane index (kFrom = 8, 16 or 32): every lane of such
// a group receives the group's result.
template <int kFrom>
__device__ __forceinline__ float xor_sum(float x) {
  float a, b;
  xor_pair<kFrom>(x, a, b);
  x = a + b;
  if constexpr (kFrom < 32) x = xor_sum<2 * kFrom>(x);
  return x;
}
template <int kFrom>
__device__ __forceinline__ float xor_max(float x) {
  float a, b;
  xor_pair<kFrom>(x, a, b);
  x = fmaxf(a, b);
  if constexpr (kFrom < 32) x = xor_max<2 * kFrom>(x);
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
  for (int m = 32; m >= 1; m >>= 1) x += shfl_xor_f32(x, m);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, shfl_xor_f32(x, m));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }
__device__ __forceinline__ float qnan() { return __builtin_nanf(""); }

// ---------------------------------------------------------------- launchers
// Implemented in decode_partial.hip / merge.hip / cache_write.hip; the C ABI
// in capi.hip validates arguments and then calls these.
// One KV tier of a decode call: its own cache, strides, table and lengths.
struct KvTier {
  const void* k;
  const void* v;
  int64_t sb, sh, st;  // element strides: block, head, token
  int64_t num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
};

// A decode call over one tier (a partial) or two (the fused split path: each
// row's tier-0 blocks, then its tier-1 blocks, as one list).
struct DecodeArgs {
  const void* q;
  int64_t q_ss, q_sh;
  KvTier tier[2];
  int32_t ntiers;
  const int32_t* order;  // optional sequence processing order (may be NULL)
  int32_t n, H, KVH, D, BS;
  float scale;
  int32_t kv_dtype;
  void* out;
  int64_t out_ss, out_sh;
  int32_t out_dtype;
  float* lse;
  int64_t lse_sh;
  void* workspace;
  size_t workspace_bytes;
  // measurement only (fd_paged_decode_timeline): per-workgroup time stamps
  // of a VALU-kernel launch, kTimelineSlots words per workgroup; NULL in
  // every other call
  uint64_t* timeline;
  int64_t timeline_tasks;
};

// Split plan of one decode call: blocks per split and the split count.
struct SplitPlan {
  int32_t split_blocks;  // blocks handled by one wavefront task
  int32_t max_splits;    // ceil(bt_width / split_blocks)
  bool fast;             // the tiled kernel applies (else the generic one)
  bool mfma;             // grouped-query scores on the matrix cores (G >= 4 at D = 256)
  bool mm;               // scores and P.V on the matrix cores (G >= 4, D <= 128)
  int32_t wg_cap;        // workgroups per CU the launch allows at most (0: the kernel's own
                         // occupancy); enforced by reserving LDS
  int32_t kernel_g;      // head slots per task of the tiled kernel: 1, 2, 4, 8, 16, 32 or 64
  int32_t kernel_d;      // head size the tiled kernel is built for: 64, 128 or 256
  int32_t passes;        // tasks per (sequence, kv head, block range): ceil((H / KVH) /
                         // kernel_g), each over the same blocks
  int32_t wave_blocks;   // blocks per working wave of a task (0: every wave works)
  bool no_kv_adj;        // separate K and V loads even where V follows K (FD_KV_ADJ=0)
  int* occupancy_query;  // planner only: when set, the tiled launchers store the selected
                         // kernel's workgroups per CU there instead of launching it
};

// matrix: the matrix-core kernels may be used (false when a tier lies in
// pinned host memory, which the VALU kernel reads faster over the link).
// fill: the rows' mean length over bt_width * BS when the caller knows it
// (0: unknown).
SplitPlan plan_decode(int32_t n, int32_t H, int32_t KVH, int32_t D, int32_t BS,
                      int32_t bt_width, int32_t kv_dtype, bool aligned, bool matrix = true,
                      double fill = 0.0);
size_t decode_workspace_bytes(const SplitPlan& sp, int32_t n, int32_t H,
                              int32_t D);
// Workspace a plan of these sizes may need whatever the rows' token total
// (the slot fill, half rows), 0 when neither can apply to it.
size_t fill_workspace_bound(const SplitPlan& sp, int32_t n, int32_t H, int32_t KVH, int32_t D,
                            int32_t BS, int32_t bt_width, int32_t kv_dtype);
int launch_decode(const DecodeArgs& a, const SplitPlan& sp, hipStream_t s);

struct MergeArgs {
  void* out;
  int64_t out_ss, out_sh;
  int32_t out_dt;
  const void* a;
  int64_t a_ss, a_sh;
  int32_t a_dt;
  const float* lse_a;
  int64_t lse_a_sh;
  const void* b;
  int64_t b_ss, b_sh;
  int32_t b_dt;
  const float* lse_b;
  int64_t lse_b_sh;
  float* out_lse;
  int64_t out_lse_sh;
  int32_t n, H, D;
};
int launch_merge(const MergeArgs& a, hipStream_t s);

struct CacheWriteArgs {
  const void* key;
  int64_t key_st, key_sh;
  const void* value;
  int64_t value_st, value_sh;
  void* kc;
  void* vc;
  int64_t c_sb, c_st, c_sh;
  int64_t num_blocks;
  const int64_t* slots;
  int32_t T, KVH, D, BS;
  int32_t elt;  // element size in bytes
  int32_t* err;
  const int32_t* gate;  // nothing is written when *gate != 0 (may be NULL)
};
int launch_cache_write(const CacheWriteArgs& a, hipStream_t s);

int launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s);

// Device-side tier split of a decode step (plan_tiers.hip).
struct PlanTiersArgs {
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* seq_lens;
  int32_t n_rows;
  int32_t G;  // HBM blocks: ids < G are in HBM
  int64_t C;  // host blocks: ids in [G, G + C)
  int32_t BS;
  int32_t* gpu_bt;
  int32_t* cpu_bt;
  int64_t out_stride;
  int32_t out_width;
  int32_t* gpu_lens;
  int32_t* cpu_lens;
  const int64_t* slots;
  int32_t n_tokens;
  int64_t* gpu_slots;
  int64_t* host_slots;
  int32_t* error_count;
};
int launch_plan_tiers(const PlanTiersArgs& a, hipStream_t s);

}  // namespace fd
