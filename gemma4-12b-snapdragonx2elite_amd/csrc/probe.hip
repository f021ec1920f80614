// Measurement probes: the ceilings the quantized kernels are judged against,
// measured on the part itself instead of quoted from a data sheet.
//
//  * stream_read_kernel: the fastest plain streaming read this build knows
//    (16-byte nontemporal loads, U per lane always in flight, explicit wait
//    counts, as in the decode GEMV), over a buffer of any size. Timed in a
//    graph over distinct buffers, it is the achievable-bandwidth ceiling
//    for a dependent launch that reads that many bytes once: the
//    counterpart of the reference's streaming-read microbenchmark
//    (benchmarks/microbench_bw.py:26-35). Optionally each workgroup, after
//    its own share, reads the first bytes that the same workgroup of the
//    next launch will read (a cross-launch prefetch into its XCD's L2), or
//    every unit load takes a 2-byte companion load (the GEMV's scales).
//  * mfma_loop_kernel: back-to-back independent int8 (32x32x32) or f16
//    (32x32x16) MFMAs on registers, with the shader clock (s_memtime)
//    and the constant wall clock (s_memrealtime) read at both ends of the
//    loop: the matrix-core ceiling and the clock the chip actually runs at
//    under that load (the counterpart of the reference's raw cooperative-
//    matrix probes, vk/coopgemm_i8.comp with benchmarks/coopgemm_i8.py:85).
#include "q4mi_common.h"

namespace q4 {

typedef int v16i_p __attribute__((ext_vector_type(16)));
typedef float v16f_p __attribute__((ext_vector_type(16)));

constexpr int PROBE_THREADS = 256;
constexpr uint32_t PROBE_MAGIC = 0x9E3779B9u;   // a store only if the data hash equals it

// One workgroup streams `per` units (16 bytes) of its own contiguous chunk
// (CHUNK) or every G-th 4 KB row of the buffer (grid-strided); lane t reads
// unit t of each 256-unit row. U loads per lane stay in flight: unit i's
// registers are refilled with unit i + U right after use. Indices past the
// buffer are clamped (re-read, not counted). SC: every unit load has a
// 2-byte companion load at unit index * 2 of `comp` (n16 * 2 bytes), the
// access pattern of the GEMV's block scales (1/8 of the bytes, one load per
// unit), so the pair of probes prices the scale loads.
template <int U, bool CHUNK, bool SC>
__global__ void __launch_bounds__(PROBE_THREADS)
stream_read_kernel(const uint8_t* __restrict__ buf, long n16, long per_rows, const uint8_t* __restrict__ next,
                   long next_n16, long pf_rows, const uint8_t* __restrict__ comp, uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(16))) uint32_t pf_lds[PROBE_THREADS * 4];
  constexpr int LPU = SC ? 2 : 1;  // loads per unit
  const int t = threadIdx.x;
  const long G = gridDim.x, w = blockIdx.x;
  auto unit = [&](long i) -> long {   // unit of row i of this workgroup
    const long row = CHUNK ? w * per_rows + i : i * G + w;
    return row * PROBE_THREADS + t;
  };
  const long last = n16 - 1;
  uint32_t acc = 0;
  v4u r[U];
  uint32_t c[U];
  // the companion load writes its ring slot in place (an in-out operand): an
  // output-only asm result may be copied by the register allocator while the
  // load is still in flight, and the landing load then overwrites a register
  // that holds something else by then
  auto issue = [&](int k, long j) {
    const long u = min(unit(j < per_rows ? j : per_rows - 1), last);
    r[k] = ld16_nt(buf + u * 16);
    if constexpr (SC) asm volatile("global_load_ushort %0, %1, off" : "+v"(c[k]) : "v"(comp + u * 2));
  };
  // a companion value is consumed by an ordered (volatile) instruction right
  // after its wait, so it is dead before the same slot's next load: the
  // compiler cannot sink its use below that load and keep two copies
  auto take = [&](int k) {
    pin(r[k]);
    uint32_t v = (r[k][0] + r[k][1]) ^ (r[k][2] + r[k][3]);
    if constexpr (SC) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(v) : "v"(c[k]));
    return v;
  };
#pragma unroll
  for (int k = 0; k < U; ++k) issue(k, k);
  const long rounds = (per_rows + U - 1) / U;
  long i = 0;
  for (long rd = 1; rd < rounds; ++rd) {
    static_for<0, U>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      vmwait<LPU * (U - 1)>();
      acc ^= take(k);
      issue(k, i + k + U);
    });
    i += U;
  }
  static_for<0, U>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    vmwait<LPU * (U - 1 - k)>();
    const uint32_t v = take(k);
    if (i + k < per_rows) acc ^= v;
  });
  // the first rows this workgroup's successor (same index, next launch,
  // same XCD) reads, with ordinary (L2-allocating) direct-to-LDS loads: no
  // registers, all in flight at once, the LDS copy is never read
  if (pf_rows > 0) {
    const uint32_t* dst = pf_lds + (t >> 6) * 256;
    for (long p = 0; p < pf_rows; ++p) dma16(next + min(unit(p), next_n16 - 1) * 16, dst);
    vmwait<0>();
  }
  if (acc == PROBE_MAGIC) sink[w] = acc;
}

// iters rounds of four independent MFMAs per wave; clocks[2 b] = shader
// clock cycles, clocks[2 b + 1] = wall-clock ticks of workgroup b's wave 0.
// RND: every MFMA takes another of 8 A and 8 B fragments per lane, read from
// `operands` at the start (random bytes: the operand bits toggle as real
// data does, and the chip's clock under that load is the one a GEMM sees);
// otherwise the same fragments every time.
template <bool I8, bool RND>
__global__ void __launch_bounds__(PROBE_THREADS)
mfma_loop_kernel(int iters, const v4i* __restrict__ operands, unsigned long long* __restrict__ clocks,
                 int* __restrict__ sink) {
  const int t = threadIdx.x;
  v16i_p ai[4];
  v16f_p af[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    for (int e = 0; e < 16; ++e) {
      ai[j][e] = 0;
      af[j][e] = 0.0f;
    }
  }
  v4i a[8], b[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if constexpr (RND) {
      a[k] = operands[(2 * k) * PROBE_THREADS + t];
      b[k] = operands[(2 * k + 1) * PROBE_THREADS + t];
    } else {
      a[k] = v4i{t, t * 3 + 1, t ^ 0x55, t + 7};
      b[k] = v4i{t * 5, t + 11, t ^ 0x33, t * 7 + 2};
    }
  }
  __syncthreads();
  const unsigned long long c0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; i += 8) {
    static_for<0, 8>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i& x = a[(u + j) & 7];
        const v4i& y = b[(3 * u + j) & 7];
        if constexpr (I8) ai[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, ai[j], 0, 0, 0);
        else af[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, x), __builtin_bit_cast(v8h, y),
                                                            af[j], 0, 0, 0);
      }
    });
  }
  int s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    for (int e = 0; e < 16; ++e) s += I8 ? ai[j][e] : (int)af[j][e];
  const unsigned long long c1 = clock64(), r1 = wall_clock64();
  if (t == 0) {
    clocks[2 * blockIdx.x] = c1 - c0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
  if (s == (int)PROBE_MAGIC) sink[blockIdx.x] = s;
}

typedef void (*stream_fn)(const uint8_t*, long, long, const uint8_t*, long, long, const uint8_t*, uint32_t*);
template <bool C, bool SC>
static stream_fn pick_stream_c(int U) {
  return U == 4 ? stream_read_kernel<4, C, SC> : U == 8 ? stream_read_kernel<8, C, SC> : stream_read_kernel<16, C, SC>;
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_probe_stream_read(const void* buf, size_t bytes, int wgs, int units, int chunked, const void* next,
                         size_t next_bytes, size_t prefetch_bytes, const void* comp, size_t comp_bytes,
                         uint32_t* sink, size_t sink_bytes, void* stream) {
  clear_error();
  Q4_ARG(buf && sink, "null pointer");
  Q4_ARG(bytes >= 16 && bytes % 16 == 0 && ((uintptr_t)buf & 15) == 0, "buffer must be 16-byte aligned and sized");
  Q4_ARG(wgs >= 1 && wgs <= 65536, "bad workgroup count %d", wgs);
  Q4_ARG(units == 4 || units == 8 || units == 16, "units in flight must be 4, 8 or 16 (got %d)", units);
  Q4_ARG(sink_bytes >= (size_t)wgs * sizeof(uint32_t), "sink needs %d words", wgs);
  const long n16 = (long)(bytes / 16);
  const long rows = (n16 + PROBE_THREADS - 1) / PROBE_THREADS;
  const long per_rows = (rows + wgs - 1) / wgs;
  long pf_rows = 0, next_n16 = n16;
  if (next && prefetch_bytes) {
    Q4_ARG(((uintptr_t)next & 15) == 0 && next_bytes >= 16, "next buffer must be 16-byte aligned and sized");
    // rows of the successor's own share (it reads a buffer laid out like this one); reads clamp to next_bytes
    pf_rows = (long)(prefetch_bytes / 16 / PROBE_THREADS) / wgs;
    if (pf_rows > per_rows) pf_rows = per_rows;
    next_n16 = (long)(next_bytes / 16);
  }
  if (comp) {
    Q4_ARG(comp_bytes >= (size_t)n16 * 2 && ((uintptr_t)comp & 1) == 0, "companion buffer needs bytes / 8 (%ld)",
           n16 * 2);
    Q4_ARG(pf_rows == 0, "companion loads and successor prefetch are separate probes");
  }
  const stream_fn fn = comp ? (chunked ? pick_stream_c<true, true>(units) : pick_stream_c<false, true>(units))
                            : (chunked ? pick_stream_c<true, false>(units) : pick_stream_c<false, false>(units));
  hipLaunchKernelGGL(fn, dim3(wgs), dim3(PROBE_THREADS), 0, as_stream(stream), reinterpret_cast<const uint8_t*>(buf),
                     n16, per_rows, reinterpret_cast<const uint8_t*>(pf_rows ? next : buf), next_n16, pf_rows,
                     reinterpret_cast<const uint8_t*>(comp), sink);
  Q4_LAUNCHED("stream_read");
  return Q4_OK;
}

int q4_probe_mfma(int kind, int wgs, int iters, const void* operands, size_t operand_bytes,
                  unsigned long long* clocks, size_t clocks_bytes, int* sink, size_t sink_bytes, void* stream) {
  clear_error();
  Q4_ARG(clocks && sink, "null pointer");
  Q4_ARG(clocks_bytes >= (size_t)wgs * 16 && sink_bytes >= (size_t)wgs * 4, "clocks need 2 and sink 1 word per workgroup");
  Q4_ARG(kind == 0 || kind == 1, "kind 0 (int8 32x32x32) or 1 (f16 32x32x16), got %d", kind);
  Q4_ARG(wgs >= 1 && wgs <= 65536 && iters >= 8 && iters % 8 == 0, "bad probe size wgs=%d iters=%d (a multiple of 8)",
         wgs, iters);
  Q4_ARG(!operands || (operand_bytes >= (size_t)16 * PROBE_THREADS * 16 && ((uintptr_t)operands & 15) == 0),
         "operands: 64 KB, 16-byte aligned (or NULL)");
  const v4i* ops = reinterpret_cast<const v4i*>(operands);
  void (*fn)(int, const v4i*, unsigned long long*, int*) =
      kind == 0 ? (ops ? mfma_loop_kernel<true, true> : mfma_loop_kernel<true, false>)
                : (ops ? mfma_loop_kernel<false, true> : mfma_loop_kernel<false, false>);
  hipLaunchKernelGGL(fn, dim3(wgs), dim3(PROBE_THREADS), 0, as_stream(stream), iters, ops, clocks, sink);
  Q4_LAUNCHED("mfma_loop");
  return Q4_OK;
}

int q4_probe_wall_clock_khz(int* khz) {
  clear_error();
  Q4_ARG(khz, "null pointer");
  int dev = 0;
  Q4_HIP(hipGetDevice(&dev));
  Q4_HIP(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev));
  return Q4_OK;
}

}  // extern "C"
