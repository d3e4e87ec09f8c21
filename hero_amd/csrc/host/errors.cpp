// errors.cpp -- thread-local last-error message and HIP status checks.
#include "hero/errors.hpp"

#include "hero_kernels.h"

namespace hero {

namespace {
thread_local std::string tl_message;
}

void set_last_error(const std::string& message) { tl_message = message; }
const char* last_error_message() { return tl_message.c_str(); }

void hip_check(hipError_t status, const char* what) {
    if (status == hipSuccess) return;
    const int code = status == hipErrorOutOfMemory ? HERO_ENOMEM : HERO_EHIP;
    throw Error(code, std::string(what) + ": " + hipGetErrorString(status));
}

void check_launch(const char* what) { hip_check(hipGetLastError(), what); }

}  // namespace hero
