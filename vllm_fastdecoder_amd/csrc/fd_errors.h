// Error reporting shared by the HIP translation units and the host-only C++
// ones of libfdattn.so (this header needs no HIP runtime).
#pragma once

#include <exception>

#include "../../include/fdattn.h"

namespace fd {

// Records a printf-style message for fd_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// f() for an extern "C" entry point whose host code allocates or starts
// threads: a C++ exception (no memory, no thread) comes back as
// FD_ERR_RESOURCE instead of crossing the C ABI.
template <typename F>
int guarded(const char* who, F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    return set_error(FD_ERR_RESOURCE, "%s: %s", who, e.what());
  } catch (...) {
    return set_error(FD_ERR_RESOURCE, "%s: unknown C++ exception", who);
  }
}

}  // namespace fd
