// sjh_host.hpp -- host-side error helpers shared by the launchers and engine.
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace sjh {

[[noreturn]] inline void fail(const std::string& what) {
  throw std::runtime_error("snapjudge HIP: " + what);
}

// A caller's argument the call cannot serve (the C ABI returns SJH_E_INVALID).
struct ArgError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
[[noreturn]] inline void fail_arg(const std::string& what) {
  throw ArgError("snapjudge HIP: " + what);
}

inline void require(bool ok, const char* what) {
  if (!ok) fail(what);
}

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

inline void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(std::string("launch ") + what + ": " + hipGetErrorString(e));
}

}  // namespace sjh
