// Error reporting shared by the HIP translation units and the host-only C++
// ones of libfdattn.so (this header needs no HIP runtime).
#pragma once

namespace fd {

// Records a printf-style message for fd_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace fd
