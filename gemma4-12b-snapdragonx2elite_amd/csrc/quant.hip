// Weight preparation on the GPU (load time): the int4 block quantizer, the
// e4m3 scale lift, the W8A8 int8 fold, the W4A8 ratio and the repacks from
// the reference engine's storage layouts into the panel-64 device layout.
//
// Arithmetic follows the reference quantizer quant() (src/vk_engine.py:125-159)
// operation for operation: IEEE fp32 divides (__fdiv_rn), products rounded
// once (__fmul_rn), round-half-to-even (rintf), RNE narrowing to fp16. The
// outputs are bit-identical to the numpy quantizer.
#include "q4mi_common.h"

namespace q4 {

// ---- int4 block quantizer (src/vk_engine.py:126-131) ---------------------
// One thread per (row, block) unit, lanes along rows, so the panel-64 unit
// and scale stores of a wave are contiguous.
__global__ void quantize_kernel(const float* __restrict__ W, int N, int K, int nblk,
                                uint4* __restrict__ wq, uint16_t* __restrict__ sc16,
                                float* __restrict__ sc32) {
  long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long units = (long)pad_rows(N) * nblk;
  if (u >= units) return;
  int r = (int)(u % PANEL);
  long pb = u / PANEL;
  int b = (int)(pb % nblk);
  int n = (int)(pb / nblk) * PANEL + r;
  if (n >= N) {  // padded row: code 8 (= weight 0), scale 0
    wq[u] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
    sc16[u] = 0;
    return;
  }
  const float4* src = reinterpret_cast<const float4*>(W + (long)n * K + (long)b * BLK);
  float v[BLK];
#pragma unroll
  for (int i = 0; i < BLK / 4; ++i) {
    float4 t = src[i];
    v[4 * i + 0] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < BLK; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float sc = fmaxf(__fdiv_rn(amax, 7.0f), 1e-8f);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < BLK; ++k) {
    float c = rintf(__fdiv_rn(v[k], sc)) + 8.0f;
    c = fminf(fmaxf(c, 0.0f), 15.0f);
    w[k >> 3] |= ((uint32_t)c & 15u) << (4 * nib_pos(k & 7));
  }
  wq[u] = make_uint4(w[0], w[1], w[2], w[3]);
  sc16[u] = f2h_after_f32(sc);
  if (sc32) sc32[(long)n * nblk + b] = sc;
}

// ---- e4m3 scale lift (src/vk_engine.py:133-137) ---------------------------
__global__ void absmax_bits_kernel(const float* __restrict__ x, long n, uint32_t* __restrict__ out) {
  float m = 0.0f;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    m = fmaxf(m, fabsf(x[i]));
  m = reduce64<true>(m);
  if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));  // m >= 0: bit order == value order
}

// float32 in [0, 448] -> e4m3fn byte, round-half-to-even. Normal band:
// round the fp32 bit pattern at mantissa bit 20 (keeping 3 mantissa bits)
// and rebias the exponent from 127 to 7; a rounding carry moves into the
// exponent by itself. Subnormal band (< 2^-6): the value in units of 2^-9,
// rounded to even (code 8 is the smallest normal, 2^-6).
__device__ inline uint32_t e4m3_encode_pos(float v) {
  if (v < 0.015625f) return (uint32_t)rintf(v * 512.0f);
  uint32_t bits = __float_as_uint(v);
  uint32_t r = (bits + 0x7FFFFu + ((bits >> 20) & 1u)) >> 20;
  return r - (120u << 3);
}

__device__ inline int lift_shift(const uint32_t* maxbits) {
  float mx = __uint_as_float(*maxbits);
  if (!(mx > 0.0f)) return 0;
  int e;
  frexp(256.0 / (double)mx, &e);  // 256/mx = f * 2^e, f in [0.5, 1): floor(log2) = e - 1
  return e - 1;
}

__global__ void e4m3_lift_kernel(const float* __restrict__ sc32, int N, int nblk, const uint32_t* __restrict__ maxbits,
                                 uint8_t* __restrict__ sc8, float* __restrict__ inv_out) {
  long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long units = (long)pad_rows(N) * nblk;
  const int shift = lift_shift(maxbits);
  if (u == 0 && inv_out) *inv_out = ldexpf(1.0f, -shift);
  if (u >= units) return;
  int r = (int)(u % PANEL);
  long pb = u / PANEL;
  int b = (int)(pb % nblk);
  int n = (int)(pb / nblk) * PANEL + r;
  if (n >= N) { sc8[u] = 0; return; }
  const float p2 = __int_as_float((shift + 127) << 23);  // 2^shift, exact
  float v = __fmul_rn(sc32[(long)n * nblk + b], p2);
  v = fminf(fmaxf(v, 0.0f), 448.0f);
  sc8[u] = (uint8_t)e4m3_encode_pos(v);
}

// ---- W8A8 fold (src/vk_engine.py:152-157) --------------------------------
// One workgroup per weight row.
__device__ inline void unit_codes(uint4 unit, float* qm8) {
  uint32_t w[4] = {unit.x, unit.y, unit.z, unit.w};
#pragma unroll
  for (int k = 0; k < BLK; ++k) qm8[k] = (float)(int)((w[k >> 3] >> (4 * nib_pos(k & 7))) & 15u) - 8.0f;
}

__global__ void __launch_bounds__(256) w8_fold_kernel(const uint4* __restrict__ wq, const float* __restrict__ sc32,
                                                      int N, int K, int nblk, int8_t* __restrict__ W8,
                                                      float* __restrict__ sw32, uint16_t* __restrict__ sw16) {
  __shared__ float red[4];
  const int n = blockIdx.x;
  float amax = 0.0f;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    float q[BLK];
    unit_codes(wq[panel_index(n, b, nblk)], q);
    const float s = sc32[(long)n * nblk + b];
#pragma unroll
    for (int k = 0; k < BLK; ++k) amax = fmaxf(amax, fabsf(__fmul_rn(q[k], s)));
  }
  amax = reduce64<true>(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sw = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
  if (threadIdx.x == 0) {
    if (sw32) sw32[n] = sw;
    if (sw16) sw16[n] = f2h_after_f32(sw);
  }
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    float q[BLK];
    unit_codes(wq[panel_index(n, b, nblk)], q);
    const float s = sc32[(long)n * nblk + b];
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = rintf(__fdiv_rn(__fmul_rn(q[4 * j + e], s), sw));
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        word |= ((uint32_t)(int)v & 0xFFu) << (8 * e);
      }
      o[j] = word;
    }
    uint4* dst = reinterpret_cast<uint4*>(W8 + (long)n * K + (long)b * BLK);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// ---- W4A8 ratio (benchmarks/coopgemm_w4a8.py:84) --------------------------
__global__ void w4a8_ratio_kernel(const float* __restrict__ sc32, const float* __restrict__ sw32, int N, int nblk,
                                  uint16_t* __restrict__ ratio) {
  long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long units = (long)pad_rows(N) * nblk;
  if (u >= units) return;
  int r = (int)(u % PANEL);
  long pb = u / PANEL;
  int b = (int)(pb % nblk);
  int n = (int)(pb / nblk) * PANEL + r;
  ratio[u] = (n < N) ? f2h_after_f32(__fdiv_rn(sc32[(long)n * nblk + b], sw32[n])) : (uint16_t)0;
}

// ---- repacks from the reference layouts ----------------------------------
__global__ void repack_ref_kernel(const uint32_t* __restrict__ wp, const uint16_t* __restrict__ sc_ref, int N, int K,
                                  int nblk, uint4* __restrict__ wq, uint16_t* __restrict__ sc_dev) {
  long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long units = (long)pad_rows(N) * nblk;
  if (u >= units) return;
  int r = (int)(u % PANEL);
  long pb = u / PANEL;
  int b = (int)(pb % nblk);
  int n = (int)(pb / nblk) * PANEL + r;
  if (n >= N) {
    if (wq) wq[u] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
    if (sc_dev) sc_dev[u] = 0;
    return;
  }
  if (wq) {
    const int n8 = N / 8, shift = 4 * (n % 8);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < BLK; ++k) {
      uint32_t q = (wp[(long)(b * BLK + k) * n8 + n / 8] >> shift) & 15u;
      w[k >> 3] |= q << (4 * nib_pos(k & 7));
    }
    wq[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (sc_dev) sc_dev[u] = sc_ref[(long)b * N + n];
}

__global__ void repack_e4m3_ref_kernel(const uint8_t* __restrict__ sc_ref, int N, int nblk, uint8_t* __restrict__ sc_dev) {
  long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long units = (long)pad_rows(N) * nblk;
  if (u >= units) return;
  int r = (int)(u % PANEL);
  long pb = u / PANEL;
  int b = (int)(pb % nblk);
  int n = (int)(pb / nblk) * PANEL + r;
  sc_dev[u] = (n < N) ? sc_ref[(long)b * N + n] : (uint8_t)0;
}

__global__ void transpose_i8_kernel(const int8_t* __restrict__ src, int rows, int cols, int8_t* __restrict__ dst) {
  // src [rows][cols] -> dst [cols][rows]; 64x64 tiles through LDS.
  __shared__ int8_t tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
    int r = i / 64, c = i % 64;
    if (r0 + r < rows && c0 + c < cols) tile[r][c] = src[(long)(r0 + r) * cols + c0 + c];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
    int c = i / 64, r = i % 64;
    if (r0 + r < rows && c0 + c < cols) dst[(long)(c0 + c) * rows + r0 + r] = tile[r][c];
  }
}

// Two panel-64 matrices A, B (N rows each, N % 32 == 0) -> one of 2N rows
// with row 2i = A row i and row 2i + 1 = B row i, units and scales (sb
// bytes each) moved as they are. One thread per output (row, block) unit.
__global__ void interleave_rows_kernel(const uint4* __restrict__ wa, const uint8_t* __restrict__ sa,
                                       const uint4* __restrict__ wb, const uint8_t* __restrict__ sbp, int nblk,
                                       int sbytes, uint4* __restrict__ wo, uint8_t* __restrict__ so, long units) {
  const long u = (long)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int r64 = (int)(u % PANEL);
  const long pb = u / PANEL;  // panel * nblk + block
  const int b = (int)(pb % nblk);
  const int n2 = (int)(pb / nblk) * PANEL + r64;  // output row
  const int n = n2 >> 1;
  const long src = ((long)(n / PANEL) * nblk + b) * PANEL + n % PANEL;
  const bool odd = n2 & 1;
  wo[u] = odd ? wb[src] : wa[src];
  const uint8_t* sp = (odd ? sbp : sa) + src * sbytes;
  for (int i = 0; i < sbytes; ++i) so[u * sbytes + i] = sp[i];
}

static int check_wk(int N, int K) {
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  Q4_ARG((long)N * K < (1L << 40), "matrix too large");
  return Q4_OK;
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_quantize(const float* W, int N, int K, uint32_t* wq, uint16_t* sc16, float* sc32, void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(W && wq && sc16, "null pointer");
  Q4_ARG(((uintptr_t)W & 15) == 0 && ((uintptr_t)wq & 15) == 0, "W and wq must be 16-byte aligned");
  const int nblk = K / BLK;
  long units = (long)pad_rows(N) * nblk;
  hipLaunchKernelGGL(quantize_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream), W, N, K, nblk,
                     reinterpret_cast<uint4*>(wq), sc16, sc32);
  Q4_LAUNCHED("quantize");
  return Q4_OK;
}

int q4_scales_e4m3(const float* sc32, int N, int K, uint8_t* sc8, float* inv_dev, uint32_t* work, void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(sc32 && sc8 && work, "null pointer");
  const int nblk = K / BLK;
  long n = (long)N * nblk;
  Q4_HIP(hipMemsetAsync(work, 0, sizeof(uint32_t), as_stream(stream)));
  int grid = ceil_div(n, 256);
  if (grid > 1024) grid = 1024;
  hipLaunchKernelGGL(absmax_bits_kernel, dim3(grid), dim3(256), 0, as_stream(stream), sc32, n, work);
  Q4_LAUNCHED("absmax_bits");
  long units = (long)pad_rows(N) * nblk;
  hipLaunchKernelGGL(e4m3_lift_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream), sc32, N, nblk,
                     work, sc8, inv_dev);
  Q4_LAUNCHED("e4m3_lift");
  return Q4_OK;
}

int q4_w8_fold(const uint32_t* wq, const float* sc32, int N, int K, int8_t* W8, float* sw32, uint16_t* sw16,
               void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(wq && sc32 && W8, "null pointer");
  Q4_ARG(((uintptr_t)W8 & 15) == 0 && ((uintptr_t)wq & 15) == 0, "W8 and wq must be 16-byte aligned");
  hipLaunchKernelGGL(w8_fold_kernel, dim3(N), dim3(256), 0, as_stream(stream), reinterpret_cast<const uint4*>(wq),
                     sc32, N, K, K / BLK, W8, sw32, sw16);
  Q4_LAUNCHED("w8_fold");
  return Q4_OK;
}

int q4_w4a8_ratio(const float* sc32, const float* sw32, int N, int K, uint16_t* ratio, void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(sc32 && sw32 && ratio, "null pointer");
  const int nblk = K / BLK;
  long units = (long)pad_rows(N) * nblk;
  hipLaunchKernelGGL(w4a8_ratio_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream), sc32, sw32, N,
                     nblk, ratio);
  Q4_LAUNCHED("w4a8_ratio");
  return Q4_OK;
}

int q4_repack_ref(const uint32_t* wp, const uint16_t* sc_ref, int N, int K, uint32_t* wq, uint16_t* sc_dev,
                  void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(N % 8 == 0, "reference layout needs N %% 8 == 0 (N=%d)", N);
  Q4_ARG((wp != nullptr) == (wq != nullptr), "wp and wq must both be given or both be NULL");
  Q4_ARG((sc_ref != nullptr) == (sc_dev != nullptr), "sc_ref and sc_dev must both be given or both be NULL");
  Q4_ARG(((uintptr_t)wq & 15) == 0, "wq must be 16-byte aligned");
  const int nblk = K / BLK;
  long units = (long)pad_rows(N) * nblk;
  hipLaunchKernelGGL(repack_ref_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream), wp, sc_ref, N, K,
                     nblk, reinterpret_cast<uint4*>(wq), sc_dev);
  Q4_LAUNCHED("repack_ref");
  return Q4_OK;
}

int q4_interleave_rows(const uint32_t* wa, const void* sa, const uint32_t* wb, const void* sb, int N, int K,
                       int scale_bytes, uint32_t* wout, void* sout, void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(wa && sa && wb && sb && wout && sout, "null pointer");
  Q4_ARG(N % 32 == 0, "interleaving needs N %% 32 == 0 (got N=%d)", N);
  Q4_ARG(scale_bytes == 1 || scale_bytes == 2, "scale_bytes must be 1 or 2");
  Q4_ARG(((uintptr_t)wa & 15) == 0 && ((uintptr_t)wb & 15) == 0 && ((uintptr_t)wout & 15) == 0,
         "weight words must be 16-byte aligned");
  const int nblk = K / BLK;
  const long units = (long)2 * N * nblk;
  hipLaunchKernelGGL(interleave_rows_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4*>(wa), reinterpret_cast<const uint8_t*>(sa),
                     reinterpret_cast<const uint4*>(wb), reinterpret_cast<const uint8_t*>(sb), nblk, scale_bytes,
                     reinterpret_cast<uint4*>(wout), reinterpret_cast<uint8_t*>(sout), units);
  Q4_LAUNCHED("interleave_rows");
  return Q4_OK;
}

int q4_repack_e4m3_ref(const uint8_t* sc_ref, int N, int K, uint8_t* sc_dev, void* stream) {
  clear_error();
  if (int st = check_wk(N, K)) return st;
  Q4_ARG(sc_ref && sc_dev, "null pointer");
  const int nblk = K / BLK;
  long units = (long)pad_rows(N) * nblk;
  hipLaunchKernelGGL(repack_e4m3_ref_kernel, dim3(ceil_div(units, 256)), dim3(256), 0, as_stream(stream), sc_ref, N,
                     nblk, sc_dev);
  Q4_LAUNCHED("repack_e4m3_ref");
  return Q4_OK;
}

int q4_repack_w8_ref(const int8_t* w8_kn, int N, int K, int8_t* w8_nk, void* stream) {
  clear_error();
  Q4_ARG(N > 0 && K > 0, "bad shape N=%d K=%d", N, K);
  Q4_ARG(w8_kn && w8_nk, "null pointer");
  dim3 grid(ceil_div(N, 64), ceil_div(K, 64));
  hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, as_stream(stream), w8_kn, K, N, w8_nk);
  Q4_LAUNCHED("repack_w8_ref");
  return Q4_OK;
}

}  // extern "C"
