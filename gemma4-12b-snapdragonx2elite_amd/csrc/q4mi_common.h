// Shared helpers for libq4mi: status/error plumbing, vector types, launch
// checks. gfx950 (CDNA4) only; wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>
#include <type_traits>

#include "../../include/q4mi.h"

namespace q4 {

constexpr int BLK = 32;     // K elements per scale block
constexpr int PANEL = 64;   // rows per device panel (one wave64, lane = row)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

void set_error(const char* fmt, ...);
void clear_error();

__host__ __device__ inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }
__host__ __device__ inline int pad_rows(int N) { return ceil_div(N, PANEL) * PANEL; }

// Status helpers used by every extern "C" entry point.
#define Q4_ARG(cond, ...)                 \
  do {                                    \
    if (!(cond)) {                        \
      ::q4::set_error(__VA_ARGS__);       \
      return Q4_ERR_ARG;                  \
    }                                     \
  } while (0)

#define Q4_HIP(call)                                                        \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess) {                                                 \
      ::q4::set_error("%s failed: %s", #call, hipGetErrorString(e_));       \
      return Q4_ERR_HIP;                                                    \
    }                                                                       \
  } while (0)

// Check the launch that was just enqueued.
#define Q4_LAUNCHED(name)                                                   \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess) {                                                 \
      ::q4::set_error("launch of %s failed: %s", name, hipGetErrorString(e_)); \
      return Q4_ERR_HIP;                                                    \
    }                                                                       \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers -------------------------------------------------------

// Index of (row n, block b) in the panel-64 order shared by codes and scales.
__device__ __host__ inline long panel_index(int n, int b, int nblk) {
  return ((long)(n / PANEL) * nblk + b) * PANEL + (n % PANEL);
}

// Nibble position of element e (0..7) within a device word.
__device__ __host__ constexpr int nib_pos(int e) { return (e & 1) * 4 + (e >> 1); }

__device__ inline float h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ inline uint16_t f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Round an fp32 value that is the result of an fp32 operation to fp16.
// The empty asm pins the fp32 rounding of that operation: without it the
// compiler may fold "fp32 multiply, then fp16 convert" into one
// mixed-precision instruction that rounds the exact product straight to
// fp16, which differs from numpy's two roundings at fp16 half-way points.
__device__ inline uint16_t f2h_after_f32(float f) {
  asm volatile("" : "+v"(f));
  return f2h(f);
}

// e4m3fn byte -> f16 bits holding value * 2^-8 (exact for every code): the
// 7 magnitude bits land in the f16 exponent/mantissa fields, so the e4m3
// bias (7) becomes the f16 bias (15) and subnormals stay subnormal.
__device__ inline uint16_t e4m3_to_h_scaled(uint32_t b) {
  return (uint16_t)(((b & 0x80u) << 8) | ((b & 0x7Fu) << 7));
}

}  // namespace q4
