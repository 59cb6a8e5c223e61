// Shared helpers for the deflated-Muon polar-path HIP library (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// status codes returned by every entry point (0 = success)
enum {
  DMH_OK = 0,
  DMH_EINVAL = 1,     // bad shape / argument
  DMH_EWORKSPACE = 2, // workspace too small
  DMH_ELAUNCH = 3,    // a HIP call or launch failed
};

namespace dmh {

void set_error(const char* fmt, ...);

// Round-to-nearest-even fp32 -> bf16 (clang lowers the cast to the gfx950
// v_cvt_pk_bf16_f32 instruction).
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }
__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }

// Map a hardware workgroup id to a logical tile id so that each XCD (the
// dispatcher deals workgroups round-robin over the 8 XCDs) works on a
// contiguous range of logical tiles and shares their operands in its L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int NXCD = 8;
  const int q = nblocks / NXCD, rem = nblocks % NXCD;
  const int xcd = bid % NXCD, slot = bid / NXCD;
  return xcd * q + (xcd < rem ? xcd : rem) + slot;
}

inline int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

}  // namespace dmh

#define DMH_CHECK_LAUNCH(what)                                              \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess) {                                                 \
      dmh::set_error("%s: %s", what, hipGetErrorString(_e));                \
      return DMH_ELAUNCH;                                                   \
    }                                                                       \
  } while (0)
