// Shared helpers for the boundflow HIP library (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdarg>

namespace bf {

// Status codes returned by every extern "C" entry point.
enum Status : int {
  BF_OK = 0,
  BF_EINVAL = 1,    // bad shape / null pointer / unsupported option
  BF_ELAUNCH = 2,   // kernel launch failed
  BF_ERANGE = 3,    // size exceeds a documented limit
};

void set_error(const char* fmt, ...);

#define BF_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      ::bf::set_error(__VA_ARGS__);      \
      return ::bf::BF_EINVAL;            \
    }                                    \
  } while (0)

#define BF_LAUNCH_CHECK(what)                                                       \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::bf::set_error("%s: launch failed: %s", what, hipGetErrorString(_e));        \
      return ::bf::BF_ELAUNCH;                                                      \
    }                                                                               \
  } while (0)

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// fp32 machine epsilon, the clamp used by the reference relaxation denominator
// (torch.finfo(float32).eps, boundflow/runtime/crown_ibp.py:750).
constexpr float kF32Eps = 1.1920928955078125e-07f;

// ReLU relaxation of one neuron with pre-activation box [l, u]
// (boundflow/runtime/crown_ibp.py:722-758).  Stable-active: identity.
// Stable-inactive (also l == u == 0): zero.  Ambiguous: upper chord
// a = u / max(u - l, eps), intercept -l * a; lower slope 0 unless an alpha
// override (already clamped to [0, 1]) is supplied.
struct Relax {
  float au, bu, al, bl;
};

__device__ __forceinline__ Relax relu_relax(float l, float u, bool has_alpha, float alpha) {
  Relax r;
  const bool pos = l >= 0.f;
  const bool neg = u <= 0.f;
  if (neg) {
    r.au = 0.f; r.bu = 0.f; r.al = 0.f; r.bl = 0.f;
  } else if (pos) {
    r.au = 1.f; r.bu = 0.f; r.al = 1.f; r.bl = 0.f;
  } else {
    float denom = fmaxf(u - l, kF32Eps);
    float a = u / denom;
    r.au = a;
    r.bu = -l * a;
    r.al = has_alpha ? alpha : 0.f;
    r.bl = 0.f;
  }
  return r;
}

__device__ __forceinline__ float clamp01(float x) { return fminf(fmaxf(x, 0.f), 1.f); }

}  // namespace bf
