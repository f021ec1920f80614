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
typedef unsigned v2u __attribute__((ext_vector_type(2)));

void set_error(const char* fmt, ...);
void clear_error();
// Plan override of a Q4_TUNE_* knob (q4_tune_set), -1 when none.
int tune_value(int knob);

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

// ---- inline-asm memory operations ------------------------------------------
// Loads issued through asm are invisible to the compiler's wait-count
// tracking: the kernel waits for them with explicit s_waitcnt vmcnt(n), the
// count fixed by the issue order (vector memory loads return in order), and
// pins the registers a wait covers (an empty asm that reads and writes them)
// so no use of a loaded value is scheduled above its wait. Volatile asm
// statements keep their relative order; the direct-to-LDS load also
// clobbers memory, so LDS accesses stay on their side of it.

// 16 bytes per lane from global memory into LDS at lds_dst + 16 * lane
// (lds_dst wave-uniform).
__device__ inline void dma16(const void* gptr, const void* lds_dst) {
  const unsigned l = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(l) : "memory");
}
__device__ inline v4u ld16(const void* p) {
  v4u r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
__device__ inline v2u ld8(const void* p) {
  v2u r;
  asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
// Uniform base (SGPR pair) + per-lane 32-bit byte offset + immediate byte
// offset OFF (-4096 .. 4095), streaming (read-once data).
template <int OFF>
__device__ inline uint32_t ld4_so_nt(const void* sbase, uint32_t voff) {
  uint32_t r;
  asm volatile("global_load_dword %0, %1, %2 offset:%3 nt" : "=v"(r) : "v"(voff), "s"(sbase), "n"(OFF));
  return r;
}
template <int OFF>
__device__ inline uint32_t ld2_so_off(const void* sbase, uint32_t voff) {
  uint32_t r;
  asm volatile("global_load_ushort %0, %1, %2 offset:%3" : "=v"(r) : "v"(voff), "s"(sbase), "n"(OFF));
  return r;
}
template <int OFF>
__device__ inline uint32_t ld1_so_off(const void* sbase, uint32_t voff) {
  uint32_t r;
  asm volatile("global_load_ubyte %0, %1, %2 offset:%3" : "=v"(r) : "v"(voff), "s"(sbase), "n"(OFF));
  return r;
}
// (a & m) | c in one VALU operation. v_and_or_b32 takes no literal
// constants and reads at most one SGPR: m comes in an SGPR, c in a VGPR
// (both loop-invariant, so they are set up once).
__device__ inline uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
  return r;
}
__device__ inline uint32_t ld2(const void* p) {
  uint32_t r;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
__device__ inline uint32_t ld1(const void* p) {
  uint32_t r;
  asm volatile("global_load_ubyte %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
// Uniform base (SGPR pair) + per-lane 32-bit byte offset: one VGPR per
// address instead of two.
__device__ inline v4u ld16_so(const void* sbase, uint32_t voff) {
  v4u r;
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(r) : "v"(voff), "s"(sbase));
  return r;
}
__device__ inline v2u ld8_so(const void* sbase, uint32_t voff) {
  v2u r;
  asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(r) : "v"(voff), "s"(sbase));
  return r;
}
__device__ inline uint32_t ld2_so(const void* sbase, uint32_t voff) {
  uint32_t r;
  asm volatile("global_load_ushort %0, %1, %2" : "=v"(r) : "v"(voff), "s"(sbase));
  return r;
}
// Direct-to-LDS load at uniform base + per-lane offset (lds_dst as dma16).
__device__ inline void dma16_so(const void* sbase, uint32_t voff, const void* lds_dst) {
  const unsigned l = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(l)
               : "memory");
}
// Streaming (non-temporal) variants for data read exactly once.
__device__ inline v4u ld16_nt(const void* p) {
  v4u r;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(r) : "v"(p));
  return r;
}
// Cross-lane reductions on VALU (DPP row operations and gfx950's
// permlane swaps) instead of LDS-routed shuffles: every lane of the group
// ends with the same bits. Pair order (per lane): quad xor 1, quad xor 2,
// 8-lane mirror, 16-lane mirror, then rows 0+1 / 2+3 (permlane16 swap),
// then halves (permlane32 swap).
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_MIRROR8 = 0x141, DPP_MIRROR16 = 0x140;
template <bool MAX>
__device__ inline float red_op(float a, float b) {
  if constexpr (MAX) return fmaxf(a, b);
  else return a + b;
}
template <bool MAX>
__device__ inline float reduce8(float v) {
  v = red_op<MAX>(v, dpp_f<DPP_XOR1>(v));
  v = red_op<MAX>(v, dpp_f<DPP_XOR2>(v));
  return red_op<MAX>(v, dpp_f<DPP_MIRROR8>(v));
}
template <bool MAX>
__device__ inline float reduce16(float v) {
  v = reduce8<MAX>(v);
  return red_op<MAX>(v, dpp_f<DPP_MIRROR16>(v));
}
template <bool MAX>
__device__ inline float reduce32(float v) {
  v = reduce16<MAX>(v);
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return red_op<MAX>(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
template <bool MAX>
__device__ inline float reduce64(float v) {
  v = reduce32<MAX>(v);
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return red_op<MAX>(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Sum (or max) over lanes l, l + R, l + 2R, .. (R = 8, 16, 32, 64), valid
// in lanes l < R (with R = 16 or 32, in every lane): the xor-8, xor-16,
// xor-32 pairings of a shuffle loop, each own + partner (so the bits equal
// those of that loop), on VALU: DPP row rotate by 8 within 16 lanes, then
// the permlane16 and permlane32 swaps.
template <int R, bool MAX = false>
__device__ inline float slot_reduce(float v) {
  static_assert(R == 8 || R == 16 || R == 32 || R == 64, "slot width");
  if constexpr (R <= 8) v = red_op<MAX>(v, dpp_f<0x128>(v));  // row_ror:8 = lane ^ 8 within 16
  if constexpr (R <= 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = red_op<MAX>(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  if constexpr (R <= 32) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = red_op<MAX>(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  return v;
}
template <int R>
__device__ inline float slot_sum(float v) { return slot_reduce<R, false>(v); }

template <int N>
__device__ inline void vmwait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline void lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <class T>
__device__ inline void pin(T& v) {
  asm volatile("" : "+v"(v));
}

// f(std::integral_constant<int, I>) for I = B .. E-1, unrolled at compile
// time (wait counts and register indices must be constants).
// tanh-form GELU with the reference's operation order (vk/gelumul.comp:8):
// 0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3))), each product and
// sum rounded once.
__device__ inline float gelu_tanh(float x) {
  const float inner = __fmul_rn(0.7978845608028654f, __fadd_rn(x, __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x)));
  return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}

// KV-cache slot of position pos: a ring of `window` slots for sliding
// layers, the position itself for global ones (window 0).
__device__ inline int kv_slot(uint32_t pos, int window) { return window > 0 ? (int)(pos % (uint32_t)window) : (int)pos; }
// Keys the token at pos attends: pos + 1, at most the ring, at most the cache.
__device__ inline int att_len(uint32_t pos, int window, int stride) {
  const long T = window > 0 ? min((long)pos + 1, (long)window) : (long)pos + 1;
  return (int)min(T, (long)stride);
}

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// RMS norm factor 1 / sqrt(mean(x^2) + eps) from a sum of squares over D
// elements (vk/rmsnorm.comp:8-12, vk/normadd.comp:8-12)
constexpr float NORM_EPS = 1e-6f;
__device__ inline float inv_rms(float sumsq, int D) { return 1.0f / sqrtf(sumsq / (float)D + NORM_EPS); }

// W4A16 GEMM into fp32 split-K partials [split][M][N] at every split
// (split 1 included) for a caller that reduces them itself (gemm.hip):
// w4a16_partials_bytes is the workspace it needs, *split_out the split it
// used; returns Q4_OK or an error (set).
size_t w4a16_partials_bytes(int M, int N, int K);
int w4a16_partials(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M, int N, int K, void* ws,
                   size_t ws_bytes, hipStream_t st, int* split_out);

}  // namespace q4
