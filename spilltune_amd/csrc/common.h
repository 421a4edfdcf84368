// Shared device/host helpers for the SpillTune MI355X (gfx950) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/spilltune_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// 16-entry fp32 codebook passed by value as a kernel argument.
struct Lut16 {
  float v[16];
};

namespace st {

// ---- error reporting (thread-local, read through st_last_error) ----
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- bf16 helpers ----
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Two fp32 -> packed bf16x2 (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return (uint16_t)(pack_bf16x2(x, 0.0f) & 0xffffu);
}
// round an fp32 value through bf16 and back (models a bf16 tensor op result)
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// XCD-aware block remap: consecutive logical tiles land on the same XCD so they
// share that XCD's L2 (blocks are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  if (nb % 8 != 0) return b;
  return (b % 8) * (nb / 8) + b / 8;
}

}  // namespace st

#define ST_CHECK_ARG(cond, ...)                           \
  do {                                                    \
    if (!(cond)) return st::fail(ST_EINVAL, __VA_ARGS__); \
  } while (0)
