// Internal interface between the host-core kernel (host_decode.cpp) and its
// background form (host_async.hip); both are parts of libfdattn.so.
#pragma once

#include <stdint.h>

namespace fd {

// The argument checks of fd_host_decode_partial: FD_OK, or an error code
// with its message recorded for fd_last_error().
int host_decode_check(const void* q, const void* k_cache, const void* v_cache, int64_t num_blocks,
                      const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
                      const int32_t* lens, int32_t n, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_size, int32_t block_size, float scale, int32_t kv_dtype,
                      void* out, int32_t out_dtype, float* lse, int32_t num_threads);

}  // namespace fd
