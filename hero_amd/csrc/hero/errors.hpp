// errors.hpp -- error plumbing between C++ internals and the C ABI.
// Internals throw hero::Error; every extern "C" entry point runs inside
// guard(), which converts the exception into a status code and a
// thread-local message for hero_last_error().
#pragma once
#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace hero {

class Error : public std::runtime_error {
public:
    Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

void set_last_error(const std::string& message);
const char* last_error_message();

// HIP status -> exception
void hip_check(hipError_t status, const char* what);
// the status of the launch just enqueued
void check_launch(const char* what);

template <class F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code();
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return 4;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return 1;
    }
}

}  // namespace hero
