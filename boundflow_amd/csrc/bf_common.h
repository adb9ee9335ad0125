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

// Sum over the 64 lanes of a wave in a fixed order (pairs, quads, half rows and
// rows of 16 by DPP, then the row broadcasts that gather the total in lane 63),
// returned to every lane.  Cheaper than a butterfly of ds_bpermute shuffles.
__device__ __forceinline__ float wave_sum(float v) {
  v += __builtin_amdgcn_update_dpp(0.f, v, 0xb1, 0xf, 0xf, false);    // quad_perm [1, 0, 3, 2]
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x4e, 0xf, 0xf, false);    // quad_perm [2, 3, 0, 1]
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x141, 0xf, 0xf, false);   // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x140, 0xf, 0xf, false);   // row_mirror
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x142, 0xa, 0xf, false);   // row_bcast:15 into rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x143, 0xc, 0xf, false);   // row_bcast:31 into rows 2 and 3
  // readlane moves 32-bit integers: the float travels as its bit pattern
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over the 64 lanes of a wave of values >= 0, by the DPP steps of wave_sum with
// max in place of the sum (a lane a step leaves unwritten reads 0, the identity of
// the max of non-negative values), returned to every lane.
__device__ __forceinline__ float wave_max_nonneg(float v) {
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0xb1, 0xf, 0xf, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0x4e, 0xf, 0xf, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0x141, 0xf, 0xf, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0x140, 0xf, 0xf, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0x142, 0xa, 0xf, false));
  v = fmaxf(v, __builtin_amdgcn_update_dpp(0.f, v, 0x143, 0xc, 0xf, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// m / d for 0 <= m, d > 0, in 32-bit arithmetic when both fit (uniform over a launch)
__device__ __forceinline__ int64_t div_rows(int64_t m, int64_t d, bool fits32) {
  return fits32 ? (int64_t)((uint32_t)m / (uint32_t)d) : m / d;
}

}  // namespace bf
