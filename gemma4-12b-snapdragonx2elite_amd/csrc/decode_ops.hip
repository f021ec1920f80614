// Decode-token ops between the GEMVs, for gfx950: rmsnorm, normadd, gelumul,
// prepkv (k/v norm + RoPE into the fp16 KV cache) and decode attention.
//
// Replaces vk/rmsnorm.comp, vk/normadd.comp, vk/gelumul.comp,
// vk/prepkv.comp and vk/attn.comp of the reference engine (recorded per
// layer at src/vk_engine.py:277-287). Activations are fp32 as in the
// reference; the KV cache is fp16 [nkv][stride][hd].
//
// Design:
//  * The norms are one workgroup of 1024 threads over the whole vector
//    (3840 elements: ~4 per thread): wave xor-shuffle sums, then the 16 wave
//    sums in a fixed order, so every thread holds the same bit-identical
//    inverse norm.
//  * The token position is read from device memory (dyn[0]) inside the
//    kernels, so a captured graph replays every token without updates (the
//    reference's DYN uniform buffer, src/vk_engine.py:306-310).
//  * Attention is split along the cached keys (flash-decoding): workgroup
//    (head group, split) serves up to 4 query heads of one KV head over 32
//    keys (8 per wave), with every K and V row it needs in flight from the
//    start; a second kernel merges the splits' (max, sum, accumulator)
//    triples. The grid covers the cache capacity and splits past the current
//    length exit at once, so the launch shape does not depend on the
//    position; a 1024-key window of 8 KV heads with 2 query heads each is
//    256 workgroups. Per-head vector work (q/k norms, RoPE) runs once per
//    wave in row layout (EPL elements per lane: 64-lane sums, the RoPE
//    partner from lane l ^ 32), not once per key row: the kernel is bound by
//    VALU issue and latency, not by its 8 MB of reads.
#include "q4mi_common.h"

namespace q4 {

constexpr int NORM_THREADS = 1024;
constexpr int ATT_THREADS = 256;
constexpr int ATT_KPW = 8;        // keys per wave of an attention split (one K row per 8 lanes)
constexpr int ATT_HPW = 4;        // query heads per attention workgroup (at most)
constexpr int ATT_MAX_HD = 512;   // head dims up to 512 (global layers)


// Sum over the workgroup, identical in every thread. red: blockDim/64 floats.
__device__ inline float block_sum(float v, float* red) {
  v = reduce64<false>(v);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}
__device__ inline float block_max(float v, float* red) {
  v = reduce64<true>(v);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
  return m;
}

// Elements of a norm kernel: thread t holds elements t + NORM_THREADS r,
// r < NORM_PER, in registers (every operand is loaded before the first
// reduction, so the kernel makes one memory round trip, not one per
// dependent step); longer vectors take a second, plain loop.
constexpr int NORM_PER = 4;

template <int YT>
__device__ inline void store_y(void* y, int i, float v) {
  if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(y)[i] = f2h(v);
  else reinterpret_cast<float*>(y)[i] = v;
}

// y = (x * inv) * w   (vk/rmsnorm.comp:8-12); y fp32 or fp16
// Row blockIdx.x of [rows][D] x and y (one row for the decode token).
template <int YT>
__global__ void __launch_bounds__(NORM_THREADS) rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               void* __restrict__ y, int D) {
  __shared__ float red[NORM_THREADS / 64];
  const int t = threadIdx.x;
  x += (long)blockIdx.x * D;
  y = reinterpret_cast<char*>(y) + (long)blockIdx.x * D * (YT == Q4_DT_F16 ? 2 : 4);
  float xv[NORM_PER], wv[NORM_PER];
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) {
    const int i = t + NORM_THREADS * r;
    xv[r] = i < D ? x[i] : 0.0f;
    wv[r] = i < D ? w[i] : 0.0f;
  }
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) s = fmaf(xv[r], xv[r], s);
  for (int i = t + NORM_THREADS * NORM_PER; i < D; i += NORM_THREADS) s = fmaf(x[i], x[i], s);
  const float inv = inv_rms(block_sum(s, red), D);
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) {
    const int i = t + NORM_THREADS * r;
    if (i < D) store_y<YT>(y, i, __fmul_rn(__fmul_rn(xv[r], inv), wv[r]));
  }
  for (int i = t + NORM_THREADS * NORM_PER; i < D; i += NORM_THREADS)
    store_y<YT>(y, i, __fmul_rn(__fmul_rn(x[i], inv), w[i]));
}

// h = (h + (x * inv) * w) * sc   (vk/normadd.comp:8-12); with FUSE, then
// y = (h * inv2) * w2, the rmsnorm the reference records next on the new h
// (src/vk_engine.py:242-243 and :248-249 followed by the next layer's :231
// or the final norm :250), in the same workgroup: h never leaves registers.
// Row blockIdx.x of [rows][D] x, h and y; x fp32 or fp16 (a prefill GEMM's
// output, whose fp32 value the reference's up-cast gives exactly).
// XT_SPLITK: x is a W4A16 GEMM's fp32 split-K partials [split][rows][D]
// (stride ps between splits); the value is that GEMM's fp16 output, f16 of
// the sum in split order (its split-K reduce), taken without the round trip
// through memory.
constexpr int XT_SPLITK = 2;
template <int XT>
__device__ inline float ld_act(const void* x, long i, int split = 1, long ps = 0) {
  if constexpr (XT == Q4_DT_F16) {
    return h2f(reinterpret_cast<const uint16_t*>(x)[i]);
  } else if constexpr (XT == XT_SPLITK) {
    const float* p = reinterpret_cast<const float*>(x) + i;
    float v = p[0];
    for (int s = 1; s < split; ++s) v += p[(long)s * ps];
    return h2f(f2h(v));
  } else {
    return reinterpret_cast<const float*>(x)[i];
  }
}
template <bool FUSE, int YT, int XT = Q4_DT_F32>
__global__ void __launch_bounds__(NORM_THREADS) normadd_kernel(const void* __restrict__ xin, const float* __restrict__ w,
                                                               float* __restrict__ h, int D, float sc,
                                                               const float* __restrict__ w2, void* __restrict__ y,
                                                               int split = 1, long ps = 0) {
  __shared__ float red[NORM_THREADS / 64];
  const int t = threadIdx.x;
  const void* x = reinterpret_cast<const char*>(xin) + (long)blockIdx.x * D * (XT == Q4_DT_F16 ? 2 : 4);
  h += (long)blockIdx.x * D;
  if constexpr (FUSE) y = reinterpret_cast<char*>(y) + (long)blockIdx.x * D * (YT == Q4_DT_F16 ? 2 : 4);
  float xv[NORM_PER], wv[NORM_PER], hv[NORM_PER], w2v[NORM_PER];
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) {
    const int i = t + NORM_THREADS * r;
    if constexpr (XT == XT_SPLITK) xv[r] = i < D ? reinterpret_cast<const float*>(x)[i] : 0.0f;
    else xv[r] = i < D ? ld_act<XT>(x, i) : 0.0f;
    wv[r] = i < D ? w[i] : 0.0f;
    hv[r] = i < D ? h[i] : 0.0f;
    if constexpr (FUSE) w2v[r] = i < D ? w2[i] : 0.0f;
  }
  if constexpr (XT == XT_SPLITK) {
    // the other splits, SB at a time with all their loads in flight, added in split order
    constexpr int SB = 8;
    const float* p = reinterpret_cast<const float*>(x);
    for (int s0 = 1; s0 < split; s0 += SB) {
      float tv[SB][NORM_PER];
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int r = 0; r < NORM_PER; ++r) {
          const int i = t + NORM_THREADS * r;
          tv[u][r] = p[(long)min(s0 + u, split - 1) * ps + min(i, D - 1)];  // (clamped; unused past the ends)
        }
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (s0 + u < split) {
#pragma unroll
          for (int r = 0; r < NORM_PER; ++r)
            if (t + NORM_THREADS * r < D) xv[r] += tv[u][r];
        }
    }
#pragma unroll
    for (int r = 0; r < NORM_PER; ++r) xv[r] = h2f(f2h(xv[r]));
  }
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) s = fmaf(xv[r], xv[r], s);
  for (int i = t + NORM_THREADS * NORM_PER; i < D; i += NORM_THREADS) {
    const float v = ld_act<XT>(x, i, split, ps);
    s = fmaf(v, v, s);
  }
  const float inv = inv_rms(block_sum(s, red), D);
  float s2 = 0.0f;
#pragma unroll
  for (int r = 0; r < NORM_PER; ++r) {
    const int i = t + NORM_THREADS * r;
    hv[r] = __fmul_rn(__fadd_rn(hv[r], __fmul_rn(__fmul_rn(xv[r], inv), wv[r])), sc);
    if (i < D) h[i] = hv[r];
    s2 = fmaf(hv[r], hv[r], s2);  // padding elements are 0
  }
  for (int i = t + NORM_THREADS * NORM_PER; i < D; i += NORM_THREADS) {
    const float v = __fmul_rn(__fadd_rn(h[i], __fmul_rn(__fmul_rn(ld_act<XT>(x, i, split, ps), inv), w[i])), sc);
    h[i] = v;
    s2 = fmaf(v, v, s2);
  }
  if constexpr (FUSE) {
    const float inv2 = inv_rms(block_sum(s2, red), D);
#pragma unroll
    for (int r = 0; r < NORM_PER; ++r) {
      const int i = t + NORM_THREADS * r;
      if (i < D) store_y<YT>(y, i, __fmul_rn(__fmul_rn(hv[r], inv2), w2v[r]));
    }
    // (the tail was written to h by this thread above; it rereads its own writes)
    for (int i = t + NORM_THREADS * NORM_PER; i < D; i += NORM_THREADS)
      store_y<YT>(y, i, __fmul_rn(__fmul_rn(h[i], inv2), w2[i]));
  }
}

// out = gelu_tanh(gate) * up   (vk/gelumul.comp:7-8); out fp32 or fp16,
// gate/up fp32 or fp16 (prefill GEMM outputs)
template <int YT, int GT = Q4_DT_F32>
__global__ void __launch_bounds__(256) gelumul_kernel(const void* __restrict__ gate, const void* __restrict__ up,
                                                      void* __restrict__ out, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = __fmul_rn(gelu_tanh(ld_act<GT>(gate, i)), ld_act<GT>(up, i));
  if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(out)[i] = f2h(v);
  else reinterpret_cast<float*>(out)[i] = v;
}

// One head vector of hd (<= 512) fp32 values in LDS `v`: normalise (times
// weight w unless null) and, when cs/sn are given, rotate-half RoPE into
// `o`. Threads handle elements t and t + 256.
__device__ inline void norm_rope_head(float* v, float* o, const float* __restrict__ w, const float* __restrict__ cs,
                                      const float* __restrict__ sn, int hd, float* red) {
  const int t = threadIdx.x;
  float s = 0.0f;
  for (int i = t; i < hd; i += ATT_THREADS) s = fmaf(v[i], v[i], s);
  const float inv = inv_rms(block_sum(s, red), hd);
  for (int i = t; i < hd; i += ATT_THREADS) v[i] = w ? __fmul_rn(__fmul_rn(v[i], inv), w[i]) : __fmul_rn(v[i], inv);
  __syncthreads();
  if (cs) {
    const int hf = hd >> 1;
    for (int i = t; i < hd; i += ATT_THREADS) {
      const float r = i < hf ? -v[i + hf] : v[i - hf];
      o[i] = __fadd_rn(__fmul_rn(v[i], cs[i]), __fmul_rn(r, sn[i]));
    }
    __syncthreads();
  }
}


// K and V of KV head blockIdx.x into slot(pos)   (vk/prepkv.comp:16-30)
__global__ void __launch_bounds__(ATT_THREADS) prepkv_kernel(const float* __restrict__ qkv, const float* __restrict__ knw,
                                                             const float* __restrict__ cs, const float* __restrict__ sn,
                                                             uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int hd,
                                                             int koff, int voff, int stride, int window,
                                                             const uint32_t* __restrict__ dyn) {
  __shared__ float hv[ATT_MAX_HD], ro[ATT_MAX_HD], red[ATT_THREADS / 64];
  const int kvh = blockIdx.x, t = threadIdx.x;
  const int slot = kv_slot(dyn[0], window);
  if (slot >= stride) return;  // position past a global layer's cache: nothing to write
  const long o = ((long)kvh * stride + slot) * hd;
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = qkv[koff + kvh * hd + i];
  __syncthreads();
  norm_rope_head(hv, ro, knw, cs, sn, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) kc[o + i] = f2h(ro[i]);
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = qkv[voff + kvh * hd + i];
  __syncthreads();
  norm_rope_head(hv, ro, nullptr, nullptr, nullptr, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) vc[o + i] = f2h(hv[i]);
}

// Row layout of one head vector of HD = 64 EPL fp32 values over a wave:
// lane l holds elements EPL l .. EPL l + EPL - 1. The rotate-half partner
// of element i (i +- HD / 2) is the same element slot of lane l +- 32.
template <int EPL>
__device__ inline void ld_row(const float* __restrict__ p, float (&v)[EPL]) {
  const float* q = p + EPL * (threadIdx.x & 63);
  if constexpr (EPL >= 4) {
#pragma unroll
    for (int c = 0; c < EPL / 4; ++c) {
      const float4 f = *reinterpret_cast<const float4*>(q + 4 * c);
      v[4 * c] = f.x;
      v[4 * c + 1] = f.y;
      v[4 * c + 2] = f.z;
      v[4 * c + 3] = f.w;
    }
  } else if constexpr (EPL == 2) {
    const float2 f = *reinterpret_cast<const float2*>(q);
    v[0] = f.x;
    v[1] = f.y;
  } else {
    v[0] = q[0];
  }
}

// Sum of squares over the wave, the same bits in every lane: each lane's
// elements in order, then the 64-lane pairing levels of reduce64.
template <int EPL>
__device__ inline float row_sumsq(const float (&v)[EPL]) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) s = fmaf(v[e], v[e], s);
  return reduce64<false>(s);
}

// x <- RoPE((x * inv(x)) * w) for a row-layout vector (the arithmetic of
// norm_rope_head per element; the partner comes from lane l ^ 32).
template <int EPL>
__device__ inline void row_norm_rope(float (&x)[EPL], const float (&w)[EPL], const float (&cs)[EPL],
                                     const float (&sn)[EPL]) {
  constexpr int HD = 64 * EPL;
  const float inv = inv_rms(row_sumsq<EPL>(x), HD);
  const bool lo = (threadIdx.x & 63) < 32;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float y = __fmul_rn(__fmul_rn(x[e], inv), w[e]);
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    const float pr = __uint_as_float(lo ? p[1] : p[0]);
    x[e] = __fadd_rn(__fmul_rn(y, cs[e]), __fmul_rn(lo ? -pr : pr, sn[e]));
  }
}

// This token's K (k-norm with weight, RoPE) and V (v-norm) of one KV head in
// row layout, rounded to fp16 as the cache holds them. Each value is rounded
// to fp32 before the fp16 conversion (two roundings, as the reference's
// float16_t(v * inv)). prepkv_row_kernel and the attention with prepkv
// folded in both use this, so their cache rows are the same bits.
template <int EPL>
__device__ inline void fresh_kv(float (&k)[EPL], const float (&v)[EPL], const float (&knw)[EPL],
                                const float (&cs)[EPL], const float (&sn)[EPL], uint16_t (&kb)[EPL],
                                uint16_t (&vb)[EPL]) {
  constexpr int HD = 64 * EPL;
  row_norm_rope<EPL>(k, knw, cs, sn);
#pragma unroll
  for (int e = 0; e < EPL; ++e) kb[e] = f2h_after_f32(k[e]);
  const float iv = inv_rms(row_sumsq<EPL>(v), HD);
#pragma unroll
  for (int e = 0; e < EPL; ++e) vb[e] = f2h_after_f32(__fmul_rn(v[e], iv));
}

// prepkv for the attention's head dims (64 EPL): one wave per KV head
// (vk/prepkv.comp:16-30).
template <int EPL>
__global__ void __launch_bounds__(64) prepkv_row_kernel(const float* __restrict__ qkv, const float* __restrict__ knw,
                                                        const float* __restrict__ cs, const float* __restrict__ sn,
                                                        uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                        int koff, int voff, int stride, int window,
                                                        const uint32_t* __restrict__ dyn) {
  constexpr int HD = 64 * EPL;
  const int kvh = blockIdx.x, lane = threadIdx.x;
  const int slot = kv_slot(dyn[0], window);
  if (slot >= stride) return;
  float k[EPL], v[EPL], w[EPL], c[EPL], sv[EPL];
  ld_row<EPL>(qkv + koff + kvh * HD, k);
  ld_row<EPL>(qkv + voff + kvh * HD, v);
  ld_row<EPL>(knw, w);
  ld_row<EPL>(cs, c);
  ld_row<EPL>(sn, sv);
  uint16_t kb[EPL], vb[EPL];
  fresh_kv<EPL>(k, v, w, c, sv, kb, vb);
  const long o = ((long)kvh * stride + slot) * HD;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    kc[o + EPL * lane + e] = kb[e];
    vc[o + EPL * lane + e] = vb[e];
  }
}

// Prefill: K and V of KV head blockIdx.x of token blockIdx.y (position
// dyn[0] + token) into the token's slot, with the token's cos/sin row
// (vk/pre_prepkv.comp:18-32). k, v: [M][ld] rows of fp32 or fp16 (the
// prefill GEMM outputs; v == k for k == v layers). Tokens write in parallel:
// when a chunk wraps a ring, two tokens share a slot and the later one must
// win, so only the last token of each slot writes (the reference runs its
// tokens in parallel too and leaves that race to the hardware).
template <int KT>
__global__ void __launch_bounds__(ATT_THREADS) pre_prepkv_kernel(const void* __restrict__ k, const void* __restrict__ v,
                                                                 int ld, const float* __restrict__ knw,
                                                                 const float* __restrict__ cosM,
                                                                 const float* __restrict__ sinM, uint16_t* __restrict__ kc,
                                                                 uint16_t* __restrict__ vc, int hd, int stride,
                                                                 int window, int M, const uint32_t* __restrict__ dyn) {
  __shared__ float hv[ATT_MAX_HD], ro[ATT_MAX_HD], red[ATT_THREADS / 64];
  const int kvh = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  if (window > 0 && m + window < M) return;  // a later token of the chunk takes this slot
  const uint32_t pos = dyn[0] + (uint32_t)m;
  const int slot = kv_slot(pos, window);
  if (slot >= stride) return;  // position past a global layer's cache: nothing to write
  const long o = ((long)kvh * stride + slot) * hd;
  const long r = (long)m * ld + (long)kvh * hd;
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = ld_act<KT>(k, r + i);
  __syncthreads();
  norm_rope_head(hv, ro, knw, cosM + (long)m * hd, sinM + (long)m * hd, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) kc[o + i] = f2h(ro[i]);
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = ld_act<KT>(v, r + i);
  __syncthreads();
  norm_rope_head(hv, ro, nullptr, nullptr, nullptr, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) vc[o + i] = f2h(hv[i]);
}

// The stacked q/k/v GEMM's split-K reduce and the prepkv after it in one
// launch, from fp32 partials P [split][M][N] (N = nq + nk (+ nk), row m of
// split s at s ps + m N): blocks x < QB sum 1024 q columns of token
// blockIdx.y in split order and store them as fp16 (the GEMM's output) at
// q + m ldq; block QB + h takes KV head h: its k and v columns, summed and
// rounded the same way, then pre_prepkv_kernel's arithmetic into the
// caches. The split sums run SB splits at a time with every load in flight.
constexpr int QKV_QCOLS = 4 * ATT_THREADS;
template <int SB = 8>
__device__ inline float split_sum_f16(const float* p, int split, long ps) {
  float v = p[0];
  for (int s0 = 1; s0 < split; s0 += SB) {
    float t[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) t[u] = p[(long)min(s0 + u, split - 1) * ps];
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (s0 + u < split) v += t[u];
  }
  return h2f(f2h(v));
}
__global__ void __launch_bounds__(ATT_THREADS) pre_qkv_prepkv_kernel(
    const float* __restrict__ P, int split, long ps, int N, int nq, int kvoff, int voff, uint16_t* __restrict__ q,
    int ldq, const float* __restrict__ knw, const float* __restrict__ cosM, const float* __restrict__ sinM,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int hd, int stride, int window, int M,
    const uint32_t* __restrict__ dyn) {
  __shared__ float hv[ATT_MAX_HD], ro[ATT_MAX_HD], red[ATT_THREADS / 64];
  const int QB = (nq + QKV_QCOLS - 1) / QKV_QCOLS;
  const int m = blockIdx.y, t = threadIdx.x;
  const float* row = P + (long)m * N;
  if ((int)blockIdx.x < QB) {
    const int c = blockIdx.x * QKV_QCOLS + 4 * t;
    if (c >= nq) return;
    v4f a = *reinterpret_cast<const v4f*>(row + c);
    constexpr int SB = 8;
    for (int s0 = 1; s0 < split; s0 += SB) {
      v4f tv[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) tv[u] = *reinterpret_cast<const v4f*>(row + (long)min(s0 + u, split - 1) * ps + c);
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (s0 + u < split) a += tv[u];
    }
    *reinterpret_cast<ushort4*>(q + (long)m * ldq + c) = make_ushort4(f2h(a.x), f2h(a.y), f2h(a.z), f2h(a.w));
    return;
  }
  const int kvh = blockIdx.x - QB;
  if (window > 0 && m + window < M) return;  // a later token of the chunk takes this slot
  const uint32_t pos = dyn[0] + (uint32_t)m;
  const int slot = kv_slot(pos, window);
  if (slot >= stride) return;  // position past a global layer's cache: nothing to write
  const long o = ((long)kvh * stride + slot) * hd;
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = split_sum_f16(row + kvoff + kvh * hd + i, split, ps);
  __syncthreads();
  norm_rope_head(hv, ro, knw, cosM + (long)m * hd, sinM + (long)m * hd, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) kc[o + i] = f2h(ro[i]);
  for (int i = t; i < hd; i += ATT_THREADS) hv[i] = split_sum_f16(row + voff + kvh * hd + i, split, ps);
  __syncthreads();
  norm_rope_head(hv, ro, nullptr, nullptr, nullptr, hd, red);
  for (int i = t; i < hd; i += ATT_THREADS) vc[o + i] = f2h(hv[i]);
}


// Loads of E halves (E = 1, 2, 4, 8) as one 2/4/8/16-byte access.
template <int E>
struct HalfVec {
  uint16_t h[E];
};
template <int E>
__device__ inline HalfVec<E> ld_halves(const uint16_t* p) {
  HalfVec<E> r;
  if constexpr (E == 8) {
    const v4u u = *reinterpret_cast<const v4u*>(p);
    __builtin_memcpy(r.h, &u, 16);
  } else if constexpr (E == 4) {
    const v2u u = *reinterpret_cast<const v2u*>(p);
    __builtin_memcpy(r.h, &u, 8);
  } else if constexpr (E == 2) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    __builtin_memcpy(r.h, &u, 4);
  } else {
    r.h[0] = *p;
  }
  return r;
}

// The token position dyn[0] as a vector load, made uniform afterwards: it
// then lands in order with the kernel's other vector loads. As a scalar
// load it shares lgkmcnt with the kernel-argument loads issued after it,
// and their wait would put its round trip before every later load.
__device__ inline uint32_t load_pos(const uint32_t* dyn) {
  return __builtin_amdgcn_readfirstlane(__hip_atomic_load(dyn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Decode attention, split along the keys (vk/attn.comp:18-53,
// flash-decoding). Workgroup (g, s): head group g = hpw query heads of one
// KV head (they share that KV head's rows, so the rows are read once for all
// of them) and keys [KCH s, KCH (s + 1)) of the current length, KCH = 8 NW
// for NW waves; wave w takes 8 of those keys. Every global load is issued first, none of them
// waiting for the position: the wave's K rows (8 lanes per row, lane c8
// reading 16-byte chunks c8, c8 + 8, ..: 128 contiguous bytes per row and
// load), its V rows (one coalesced row per key, lane l owning elements
// EPL l ..; rows clamped to the cache, rows past the length masked), and in
// row layout (EPL elements per lane) the raw q of the group's heads, the
// q-norm weight and the RoPE row (and this token's raw k, v and k-norm
// weight). Each wave normalises and rotates the q heads in row layout (a
// 64-lane sum, the RoPE partner from lane l ^ 32) and hands them to its K
// layout through its own LDS area (no barrier); the score of each head
// comes from the same K registers (8-lane sums). Two barriers: after the
// scores (every wave takes the split's softmax per head from LDS: m, l, and
// the p of its own keys by lane broadcast) and after the waves' p V
// partials. Per head the split's maximum m, sum l of exp(s - m) and
// unnormalised p V go to the workspace for attn_merge_kernel. Splits past
// the length exit at once (the grid covers the cache depth, so a captured
// graph replays every position).
//
// With PREP (prepkv folded in, vk/prepkv.comp:16-30): the split holding this
// token's slot forms its K and V with fresh_kv (the same bits as
// prepkv_row_kernel), uses them for that key in place of the cache row, and
// the first head group of each KV head writes them to the cache for the
// next tokens; no other workgroup reads that row.
template <int EPL, bool PREP, int NW>
__global__ void __launch_bounds__(64 * NW)
attn_split_kernel(const float* __restrict__ qkv, const float* __restrict__ qnw, const float* __restrict__ cs,
                  const float* __restrict__ sn, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int stride,
                  int window, int qoff, int grp, int hpw, const uint32_t* __restrict__ dyn, float* __restrict__ part,
                  int nsplit, const float* __restrict__ knw, int koff, int voff) {
  constexpr int HD = 64 * EPL, KPW = ATT_KPW, KCH = KPW * NW, NT = 64 * NW;  // keys per split, threads
  constexpr int KPL = KCH / 32;  // keys per lane in the softmax (32 lanes per head)
  constexpr int NR = PREP ? ATT_HPW + 1 : ATT_HPW;  // row-layout vectors handed to the K layout: q heads (, k)
  static_assert(KCH % 32 == 0, "whole softmax lanes");
  __shared__ __attribute__((aligned(16))) float rows[NW][NR][HD];
  __shared__ float ps[ATT_HPW][KCH];
  __shared__ float accp[NW][ATT_HPW][HD];
  const int g = blockIdx.x, sp = blockIdx.y, t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int gpk = grp / hpw;  // head groups per KV head
  const int kvh = g / gpk, h0 = g * hpw;
  const int j0 = sp * KCH;
  const long kv0 = (long)kvh * stride * HD;
  const int kk = lane >> 3, c8 = lane & 7;
  const int key = KPW * wave + kk;  // this lane's K row within the split

  // (1) every global load of the split, in the order their data is used:
  //     the position, the row-layout vectors of step (2), then the K and V
  //     rows, so that step (2) runs while the cache rows are still in
  //     flight. A split past the current length runs through with every key
  //     masked (n <= 0) instead of leaving early: a branch on the position
  //     here lets the compiler sink the vector loads below it, behind the
  //     position's round trip.
  const uint32_t pos = load_pos(dyn);
  float q[ATT_HPW][EPL], wq[EPL], cr[EPL], sr[EPL], kr[EPL], vr[EPL], wk[EPL];
#pragma unroll
  for (int h = 0; h < ATT_HPW; ++h)
    if (h < hpw) ld_row<EPL>(qkv + qoff + (h0 + h) * HD, q[h]);
  ld_row<EPL>(qnw, wq);
  ld_row<EPL>(cs, cr);
  ld_row<EPL>(sn, sr);
  if constexpr (PREP) {
    ld_row<EPL>(qkv + koff + kvh * HD, kr);
    ld_row<EPL>(qkv + voff + kvh * HD, vr);
    ld_row<EPL>(knw, wk);
  }
  v4u ku[EPL];
  {
    const int j = min(j0 + key, stride - 1);
#pragma unroll
    for (int m = 0; m < EPL; ++m)
      ku[m] = *reinterpret_cast<const v4u*>(kc + kv0 + (long)j * HD + 8 * (c8 + 8 * m));
  }
  HalfVec<EPL> vv[KPW];
#pragma unroll
  for (int k = 0; k < KPW; ++k) {
    const int j = min(j0 + KPW * wave + k, stride - 1);
    vv[k] = ld_halves<EPL>(vc + kv0 + (long)j * HD + EPL * lane);
  }
  const int T = att_len(pos, window, stride);
  const int n = min(KCH, T - j0);  // <= 0 past the current length: the merge reads only the live splits
  const int slot = kv_slot(pos, window);
  const bool fresh_split = PREP && slot < stride && slot >= j0 && slot < j0 + n;  // workgroup-uniform
  const int kslot = fresh_split ? slot - j0 : -1;

  // (2) q heads in row layout -> this wave's LDS rows; with the fresh slot
  //     in this split, this token's K and V (K also through the LDS rows)
  float(*rw)[HD] = rows[wave];
#pragma unroll
  for (int h = 0; h < ATT_HPW; ++h) {
    if (h >= hpw) break;
    row_norm_rope<EPL>(q[h], wq, cr, sr);
#pragma unroll
    for (int e = 0; e < EPL; ++e) rw[h][EPL * lane + e] = q[h][e];
  }
  float vnew[EPL];
  if constexpr (PREP) {
    if (fresh_split) {
      uint16_t kb[EPL], vb[EPL];
      fresh_kv<EPL>(kr, vr, wk, cr, sr, kb, vb);
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        rw[ATT_HPW][EPL * lane + e] = h2f(kb[e]);
        vnew[e] = h2f(vb[e]);
      }
      if (g % gpk == 0 && wave == 0) {
        const long o = ((long)kvh * stride + slot) * HD;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          kc[o + EPL * lane + e] = kb[e];
          vc[o + EPL * lane + e] = vb[e];
        }
      }
    }
  }
  // (the wave reads back what it wrote: its LDS operations run in order)
  __builtin_amdgcn_wave_barrier();

  // (3) scores: this lane's K row (or this token's K) against each q head in
  //     K layout, 8-lane sums
  const bool fresh = PREP && key == kslot;
  float kf[EPL][8];
#pragma unroll
  for (int m = 0; m < EPL; ++m)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kf[m][2 * e] = h2f((uint16_t)(ku[m][e] & 0xFFFFu));
      kf[m][2 * e + 1] = h2f((uint16_t)(ku[m][e] >> 16));
    }
  if (fresh) {
#pragma unroll
    for (int m = 0; m < EPL; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[m][e] = rw[ATT_HPW][8 * (c8 + 8 * m) + e];
  }
#pragma unroll
  for (int h = 0; h < ATT_HPW; ++h) {
    if (h >= hpw) break;
    float d = 0.0f;
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
      const float4 a = *reinterpret_cast<const float4*>(&rw[h][8 * (c8 + 8 * m)]);
      const float4 b = *reinterpret_cast<const float4*>(&rw[h][8 * (c8 + 8 * m) + 4]);
      const float qv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) d = fmaf(qv[e], kf[m][e], d);
    }
    d = reduce8<false>(d);
    if (c8 == 0) ps[h][key] = key < n ? d : -INFINITY;
  }
  __syncthreads();

  // (4) softmax of the split, two heads per wave pass (lanes 0-31, 32-63),
  //     in every wave: m and l, and the p of this wave's keys by broadcast.
  //     Lane l of a half holds keys l, l + 32, ..; this wave's keys
  //     KPW wave .. + KPW - 1 are all element (KPW wave) / 32 of lanes
  //     (KPW wave) % 32 ...
  float pw[ATT_HPW][KPW], mh[ATT_HPW], lh[ATT_HPW];
  const int we = (KPW * wave) / 32, wl = (KPW * wave) % 32;  // wave-uniform
#pragma unroll
  for (int hb = 0; hb < ATT_HPW; hb += 2) {
    if (hb >= hpw) break;
    const int h = hb + (lane >> 5);
    float sc[KPL];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      sc[i] = h < hpw ? ps[h][32 * i + (lane & 31)] : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    const float m = reduce32<true>(mx);
    float pj[KPL], ls = 0.0f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      pj[i] = sc[i] != -INFINITY ? expf(sc[i] - m) : 0.0f;
      ls += pj[i];
    }
    const float l = reduce32<false>(ls);
    float pm = pj[0];  // element we of this lane (a wave-uniform choice)
#pragma unroll
    for (int i = 1; i < KPL; ++i)
      if (we == i) pm = pj[i];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int k = 0; k < KPW; ++k)
        pw[hb + u][k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pm), 32 * u + wl + k));
      mh[hb + u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32 * u));
      lh[hb + u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), 32 * u));
    }
  }

  // (5) unnormalised p V of every head from the same V registers; the waves
  //     meet in LDS. Rows past the length are taken as zero (their p is
  //     zero, and a never-written cache row may hold a NaN).
  float vf[KPW][EPL];
#pragma unroll
  for (int k = 0; k < KPW; ++k)
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      vf[k][e] = KPW * wave + k >= n                    ? 0.0f
                 : (PREP && KPW * wave + k == kslot) ? vnew[e]
                                                     : h2f(vv[k].h[e]);
#pragma unroll
  for (int h = 0; h < ATT_HPW; ++h) {
    if (h >= hpw) break;
    float a[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) a[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < KPW; ++k)
#pragma unroll
      for (int e = 0; e < EPL; ++e) a[e] = fmaf(pw[h][k], vf[k][e], a[e]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) accp[wave][h][EPL * lane + e] = a[e];
  }
  __syncthreads();
  for (int i = t; i < hpw * HD; i += NT) {
    const int h = i / HD, c = i % HD;
    float* o = part + ((long)(h0 + h) * nsplit + sp) * (HD + 2);
    float v = accp[0][h][c];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += accp[w][h][c];  // waves in order
    o[2 + c] = v;
  }
  if (t == 0) {
#pragma unroll
    for (int h = 0; h < ATT_HPW; ++h) {
      if (h >= hpw) break;
      float* o = part + ((long)(h0 + h) * nsplit + sp) * (HD + 2);
      o[0] = mh[h];
      o[1] = lh[h];
    }
  }
}

// Head blockIdx.x, dims 64 blockIdx.y .. + 63, one wave (lane = dim):
// out = sum_c acc_c e^(m_c - M) / sum_c l_c e^(m_c - M), M = max_c m_c,
// over the live splits c. No barrier: the wave loads its dims of the first
// MB splits and the (m, l) of splits lane, lane + 64, .. before the position
// (which sets the live split count) arrives, takes M and L with cross-lane
// reductions (lane c holds split c, c + 64, ..), passes the weights through
// its own LDS and sums the splits in order. Per head and dim the arithmetic
// and its order are the same whichever wave does it. ml: nsplit floats of
// dynamic shared memory. out fp32 or fp16.
template <int YT, int EPL, int MB>
__global__ void __launch_bounds__(64) attn_merge_kernel(const float* __restrict__ part, void* __restrict__ out,
                                                        int nsplit, int kch, int stride, int window,
                                                        const uint32_t* __restrict__ dyn) {
  constexpr int HD = 64 * EPL;
  extern __shared__ float ml[];
  const int h = blockIdx.x, t = threadIdx.x, d = blockIdx.y * 64 + t;
  const float* w = part + (long)h * nsplit * (HD + 2);
  // indices clamped to the workspace until the live split count is known
  float x[MB];
  auto fetch = [&](int c0, int cmax) {
#pragma unroll
    for (int c = 0; c < MB; ++c) x[c] = w[(long)min(c0 + c, cmax) * (HD + 2) + 2 + d];
  };
  fetch(0, nsplit - 1);
  const int c_t = min(t, nsplit - 1);
  const float m_t = w[(long)c_t * (HD + 2)], l_t = w[(long)c_t * (HD + 2) + 1];
  const int T = att_len(load_pos(dyn), window, stride);
  const int ns = (T + kch - 1) / kch;
  float M = t < ns ? m_t : -INFINITY;
  for (int c = t + 64; c < ns; c += 64) M = fmaxf(M, w[(long)c * (HD + 2)]);
  M = reduce64<true>(M);
  float L = 0.0f;
  for (int c = t; c < ns; c += 64) {
    const float mc = c == t ? m_t : w[(long)c * (HD + 2)];
    const float lc = c == t ? l_t : w[(long)c * (HD + 2) + 1];
    const float wc = expf(mc - M);
    ml[c] = wc;
    L = fmaf(lc, wc, L);
  }
  L = reduce64<false>(L);
  float acc = 0.0f;
  for (int c0 = 0; c0 < ns; c0 += MB) {
    if (c0 > 0) fetch(c0, ns - 1);
#pragma unroll
    for (int c = 0; c < MB; ++c)
      if (c0 + c < ns) acc = fmaf(x[c], ml[c0 + c], acc);
  }
  const float v = acc / L;
  if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(out)[h * HD + d] = f2h(v);
  else reinterpret_cast<float*>(out)[h * HD + d] = v;
}

// Waves per attention split workgroup (8 keys each): 8 (64-key splits, 512
// threads) up to hd 256, 4 (32 keys) at hd 512, whose per-wave LDS rows are
// twice as long. Measured in the decode token's graph (hd 256, 1024 keys, 8
// KV heads of 2 query heads): 64-key splits 2.190 ms per token, 32-key 2.208
// ms, 128-key (16 waves, 64 workgroups) 2.316 ms.
static int attn_waves(int hd) { return hd <= 256 ? 8 : 4; }
static int attn_kch(int hd) { return ATT_KPW * attn_waves(hd); }
static int attn_splits(int stride, int hd) { return ceil_div(stride, attn_kch(hd)); }
// query heads per attention workgroup: the largest of ATT_HPW, .., 2, 1 dividing grp
static int attn_hpw(int grp) {
  int h = ATT_HPW;
  while (grp % h) h >>= 1;
  return h;
}

template <bool FUSE, int YT>
static void pre_normadd_launch(const void* x, int x_dtype, const float* w, float* h, int D, int M, float sc,
                               const float* w2, void* y, hipStream_t st) {
  if (x_dtype == Q4_DT_F16)
    hipLaunchKernelGGL((normadd_kernel<FUSE, YT, Q4_DT_F16>), dim3(M), dim3(NORM_THREADS), 0, st, x, w, h, D, sc, w2, y);
  else
    hipLaunchKernelGGL((normadd_kernel<FUSE, YT, Q4_DT_F32>), dim3(M), dim3(NORM_THREADS), 0, st, x, w, h, D, sc, w2, y);
}

// ---- per-token inputs at the head of a decode graph ------------------------
// The host writes of the reference's forward() (src/vk_engine.py:312-314:
// the embedding row into h, DYN = (pos, pos + 1), each layer type's RoPE
// cos/sin rows) done on the device from (tid, pos) in step[0..1], so a token
// is one graph launch: workgroup 0 gathers the embedding row and writes DYN,
// workgroup 1 + t gathers the rows of RoPE table t. step is read with
// system-scope loads (it may be pinned host memory the host rewrites before
// each launch). Out-of-range values are clamped (the host checks them
// before writing; nothing here reads outside the tables).
struct TokTabs {
  const float* cos_tab[Q4_TOKEN_MAX_TABLES];
  const float* sin_tab[Q4_TOKEN_MAX_TABLES];
  float* cos_out[Q4_TOKEN_MAX_TABLES];
  float* sin_out[Q4_TOKEN_MAX_TABLES];
  int hd[Q4_TOKEN_MAX_TABLES];
  int count;
};

__global__ void __launch_bounds__(256) token_inputs_kernel(const int32_t* __restrict__ step,
                                                           const float* __restrict__ emb, int vocab, int H,
                                                           float* __restrict__ h, uint32_t* __restrict__ dyn,
                                                           int max_pos, const TokTabs tabs) {
  const int tid_raw = __hip_atomic_load(step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const int pos_raw = __hip_atomic_load(step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const int tok = min(max(tid_raw, 0), vocab - 1), pos = min(max(pos_raw, 0), max_pos - 1);
  const int t = threadIdx.x;
  if (blockIdx.x == 0) {
    const float* src = emb + (long)tok * H;
    if ((H & 3) == 0) {
      for (int i = t; i < H / 4; i += 256)
        reinterpret_cast<float4*>(h)[i] = reinterpret_cast<const float4*>(src)[i];
    } else {
      for (int i = t; i < H; i += 256) h[i] = src[i];
    }
    if (t == 0) {
      dyn[0] = (uint32_t)pos;
      dyn[1] = (uint32_t)pos + 1u;
    }
    return;
  }
  // compile-time table index (the argument block stays in kernarg memory)
#pragma unroll
  for (int k = 0; k < Q4_TOKEN_MAX_TABLES; ++k) {
    if (k == (int)blockIdx.x - 1 && k < tabs.count) {
      const int hd = tabs.hd[k];
      const long o = (long)pos * hd;
      for (int i = t; i < hd; i += 256) {
        tabs.cos_out[k][i] = tabs.cos_tab[k][o + i];
        tabs.sin_out[k][i] = tabs.sin_tab[k][o + i];
      }
    }
  }
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int D, void* stream) {
  clear_error();
  Q4_ARG(x && w && y, "null pointer");
  Q4_ARG(D > 0, "bad D=%d", D);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y_dtype");
  if (y_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(rmsnorm_kernel<Q4_DT_F16>, dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, y, D);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<Q4_DT_F32>, dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, y, D);
  Q4_LAUNCHED("rmsnorm");
  return Q4_OK;
}

int q4_normadd(const float* x, const float* w, float* h, int D, float scale, void* stream) {
  clear_error();
  Q4_ARG(x && w && h, "null pointer");
  Q4_ARG(D > 0, "bad D=%d", D);
  hipLaunchKernelGGL((normadd_kernel<false, Q4_DT_F32>), dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, h, D,
                     scale == 0.0f ? 1.0f : scale, nullptr, nullptr);
  Q4_LAUNCHED("normadd");
  return Q4_OK;
}

int q4_normadd_rmsnorm(const float* x, const float* w, float* h, int D, float scale, const float* w2, void* y,
                       int y_dtype, void* stream) {
  clear_error();
  Q4_ARG(x && w && h && w2 && y, "null pointer");
  Q4_ARG(D > 0, "bad D=%d", D);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y_dtype");
  const float sc = scale == 0.0f ? 1.0f : scale;
  if (y_dtype == Q4_DT_F16)
    hipLaunchKernelGGL((normadd_kernel<true, Q4_DT_F16>), dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, h, D,
                       sc, w2, y);
  else
    hipLaunchKernelGGL((normadd_kernel<true, Q4_DT_F32>), dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, h, D,
                       sc, w2, y);
  Q4_LAUNCHED("normadd_rmsnorm");
  return Q4_OK;
}

int q4_gelumul(const float* gate, const float* up, void* out, int out_dtype, int n, void* stream) {
  clear_error();
  Q4_ARG(gate && up && out, "null pointer");
  Q4_ARG(n > 0, "bad n=%d", n);
  Q4_ARG(out_dtype == Q4_DT_F32 || out_dtype == Q4_DT_F16, "bad out_dtype");
  if (out_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(gelumul_kernel<Q4_DT_F16>, dim3(ceil_div(n, 256)), dim3(256), 0, as_stream(stream), gate, up, out, n);
  else
    hipLaunchKernelGGL(gelumul_kernel<Q4_DT_F32>, dim3(ceil_div(n, 256)), dim3(256), 0, as_stream(stream), gate, up, out, n);
  Q4_LAUNCHED("gelumul");
  return Q4_OK;
}

int q4_prepkv(const float* qkv, const float* knw, const float* cosb, const float* sinb, uint16_t* kc, uint16_t* vc,
              int nkv, int hd, int koff, int voff, int keqv, int stride, int window, const uint32_t* dyn,
              void* stream) {
  clear_error();
  Q4_ARG(qkv && knw && cosb && sinb && kc && vc && dyn, "null pointer");
  Q4_ARG(nkv > 0 && stride > 0 && window >= 0 && koff >= 0 && voff >= 0, "bad sizes");
  Q4_ARG(hd > 0 && hd % 2 == 0 && hd <= ATT_MAX_HD, "head dim must be even and <= %d (got %d)", ATT_MAX_HD, hd);
  Q4_ARG(window <= stride, "window %d exceeds the cache depth %d", window, stride);
  Q4_ARG(((uintptr_t)qkv & 15) == 0 && ((uintptr_t)knw & 15) == 0 && ((uintptr_t)cosb & 15) == 0 &&
             ((uintptr_t)sinb & 15) == 0 && koff % 4 == 0 && voff % 4 == 0,
         "qkv, knw, cos and sin must be 16-byte aligned and the k/v offsets multiples of 4 elements");
  const hipStream_t st = as_stream(stream);
  const int vo = keqv ? koff : voff;
  // head dims the attention takes: the attention's own layouts and sums, so
  // these rows equal those of q4_prepkv_attn bit for bit
  switch (hd) {
    case 64: hipLaunchKernelGGL(prepkv_row_kernel<1>, dim3(nkv), dim3(64), 0, st, qkv, knw, cosb, sinb, kc, vc, koff,
                                vo, stride, window, dyn); break;
    case 128: hipLaunchKernelGGL(prepkv_row_kernel<2>, dim3(nkv), dim3(64), 0, st, qkv, knw, cosb, sinb, kc, vc, koff,
                                 vo, stride, window, dyn); break;
    case 256: hipLaunchKernelGGL(prepkv_row_kernel<4>, dim3(nkv), dim3(64), 0, st, qkv, knw, cosb, sinb, kc, vc, koff,
                                 vo, stride, window, dyn); break;
    case 512: hipLaunchKernelGGL(prepkv_row_kernel<8>, dim3(nkv), dim3(64), 0, st, qkv, knw, cosb, sinb, kc, vc, koff,
                                 vo, stride, window, dyn); break;
    default: hipLaunchKernelGGL(prepkv_kernel, dim3(nkv), dim3(ATT_THREADS), 0, st, qkv, knw, cosb, sinb, kc, vc, hd,
                                koff, vo, stride, window, dyn); break;
  }
  Q4_LAUNCHED("prepkv");
  return Q4_OK;
}

size_t q4_attn_workspace_bytes(int nH, int hd, int stride) {
  if (nH <= 0 || hd <= 0 || stride <= 0) return 0;
  return (size_t)nH * attn_splits(stride, hd) * (hd + 2) * sizeof(float);
}

static int attn_launch(const float* qkv, const float* qnw, const float* cosb, const float* sinb, uint16_t* kc,
                       uint16_t* vc, void* out, int out_dtype, int nH, int nkv, int hd, int stride, int window,
                       int qoff, int grp, const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream,
                       const float* knw, int koff, int voff) {
  Q4_ARG(qkv && qnw && cosb && sinb && kc && vc && out && dyn && ws, "null pointer");
  Q4_ARG(out_dtype == Q4_DT_F32 || out_dtype == Q4_DT_F16, "bad out_dtype");
  Q4_ARG(nH > 0 && nkv > 0 && grp > 0 && nH == nkv * grp, "need nH == nkv * grp (got %d, %d, %d)", nH, nkv, grp);
  Q4_ARG(hd == 64 || hd == 128 || hd == 256 || hd == 512, "head dim must be 64, 128, 256 or 512 (got %d)", hd);
  Q4_ARG(stride > 0 && window >= 0 && window <= stride && qoff >= 0 && koff >= 0 && voff >= 0, "bad sizes");
  Q4_ARG(((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0, "kc and vc must be 16-byte aligned");
  Q4_ARG(((uintptr_t)qkv & 15) == 0 && ((uintptr_t)qnw & 15) == 0 && ((uintptr_t)cosb & 15) == 0 &&
             ((uintptr_t)sinb & 15) == 0 && ((uintptr_t)knw & 15) == 0 && qoff % 4 == 0 && koff % 4 == 0 &&
             voff % 4 == 0,
         "qkv, qnw, cos, sin and knw must be 16-byte aligned and the q/k/v offsets multiples of 4 elements");
  const size_t need = q4_attn_workspace_bytes(nH, hd, stride);
  Q4_ARG(ws_bytes >= need, "attention workspace too small: %zu < %zu bytes", ws_bytes, need);
  const int ns = attn_splits(stride, hd), hpw = attn_hpw(grp), kch = attn_kch(hd);
  const size_t msh = (size_t)ns * sizeof(float);
  Q4_ARG(msh <= 64 * 1024, "cache depth %d needs %d attention splits (more than the merge stages)", stride, ns);
  hipStream_t st = as_stream(stream);
  float* part = reinterpret_cast<float*>(ws);
  const dim3 grid(nH / hpw, ns), blk(64 * attn_waves(hd));
  const bool prep = knw != nullptr, h16 = out_dtype == Q4_DT_F16;
#define Q4_ATT(E, P, W)                                                                                               \
  hipLaunchKernelGGL((attn_split_kernel<E, P, W>), grid, blk, 0, st, qkv, qnw, cosb, sinb, kc, vc, stride, window, \
                     qoff, grp, hpw, dyn, part, ns, knw, koff, voff)
  // the merge fetches its splits MB at a time: the smallest of 8, 16, 32 that covers them all, or 32
#define Q4_MRG2(E, MB)                                                                                               \
  if (h16) hipLaunchKernelGGL((attn_merge_kernel<Q4_DT_F16, E, MB>), dim3(nH, E), dim3(64), msh, st, part, out, ns, \
                              kch, stride, window, dyn);                                                            \
  else hipLaunchKernelGGL((attn_merge_kernel<Q4_DT_F32, E, MB>), dim3(nH, E), dim3(64), msh, st, part, out, ns,     \
                          kch, stride, window, dyn)
#define Q4_MRG(E)                  \
  if (ns <= 8) { Q4_MRG2(E, 8); }  \
  else if (ns <= 16) { Q4_MRG2(E, 16); } \
  else { Q4_MRG2(E, 32); }
  switch (hd) {
    case 64: if (prep) { Q4_ATT(1, true, 8); } else { Q4_ATT(1, false, 8); } break;
    case 128: if (prep) { Q4_ATT(2, true, 8); } else { Q4_ATT(2, false, 8); } break;
    case 256: if (prep) { Q4_ATT(4, true, 8); } else { Q4_ATT(4, false, 8); } break;
    default: if (prep) { Q4_ATT(8, true, 4); } else { Q4_ATT(8, false, 4); } break;
  }
  Q4_LAUNCHED("attn_split");
  switch (hd) {
    case 64: Q4_MRG(1); break;
    case 128: Q4_MRG(2); break;
    case 256: Q4_MRG(4); break;
    default: Q4_MRG(8); break;
  }
#undef Q4_MRG2
#undef Q4_MRG
#undef Q4_ATT
  Q4_LAUNCHED("attn_merge");
  return Q4_OK;
}

int q4_attn(const float* qkv, const float* qnw, const float* cosb, const float* sinb, const uint16_t* kc,
            const uint16_t* vc, void* out, int out_dtype, int nH, int nkv, int hd, int stride, int window, int qoff,
            int grp, const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream) {
  clear_error();
  // the cache is only read without the folded prepkv
  return attn_launch(qkv, qnw, cosb, sinb, const_cast<uint16_t*>(kc), const_cast<uint16_t*>(vc), out, out_dtype, nH,
                     nkv, hd, stride, window, qoff, grp, dyn, ws, ws_bytes, stream, nullptr, 0, 0);
}

int q4_prepkv_attn(const float* qkv, const float* knw, const float* qnw, const float* cosb, const float* sinb,
                   uint16_t* kc, uint16_t* vc, void* out, int out_dtype, int nH, int nkv, int hd, int stride,
                   int window, int qoff, int koff, int voff, int keqv, int grp, const uint32_t* dyn, void* ws,
                   size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(knw, "null pointer");
  return attn_launch(qkv, qnw, cosb, sinb, kc, vc, out, out_dtype, nH, nkv, hd, stride, window, qoff, grp, dyn, ws,
                     ws_bytes, stream, knw, koff, keqv ? koff : voff);
}

// ---- batched prefill (one chunk of M tokens) --------------------------------

int q4_pre_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int D, int M, void* stream) {
  clear_error();
  Q4_ARG(x && w && y, "null pointer");
  Q4_ARG(D > 0 && M > 0, "bad sizes D=%d M=%d", D, M);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y_dtype");
  if (y_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(rmsnorm_kernel<Q4_DT_F16>, dim3(M), dim3(NORM_THREADS), 0, as_stream(stream), x, w, y, D);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<Q4_DT_F32>, dim3(M), dim3(NORM_THREADS), 0, as_stream(stream), x, w, y, D);
  Q4_LAUNCHED("pre_rmsnorm");
  return Q4_OK;
}

int q4_pre_normadd(const void* x, int x_dtype, const float* w, float* h, int D, int M, float scale, void* stream) {
  clear_error();
  Q4_ARG(x && w && h, "null pointer");
  Q4_ARG(D > 0 && M > 0, "bad sizes D=%d M=%d", D, M);
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x_dtype");
  pre_normadd_launch<false, Q4_DT_F32>(x, x_dtype, w, h, D, M, scale == 0.0f ? 1.0f : scale, nullptr, nullptr,
                                       as_stream(stream));
  Q4_LAUNCHED("pre_normadd");
  return Q4_OK;
}

int q4_pre_normadd_rmsnorm(const void* x, int x_dtype, const float* w, float* h, int D, int M, float scale,
                           const float* w2, void* y, int y_dtype, void* stream) {
  clear_error();
  Q4_ARG(x && w && h && w2 && y, "null pointer");
  Q4_ARG(D > 0 && M > 0, "bad sizes D=%d M=%d", D, M);
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x_dtype");
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y_dtype");
  const float sc = scale == 0.0f ? 1.0f : scale;
  if (y_dtype == Q4_DT_F16)
    pre_normadd_launch<true, Q4_DT_F16>(x, x_dtype, w, h, D, M, sc, w2, y, as_stream(stream));
  else
    pre_normadd_launch<true, Q4_DT_F32>(x, x_dtype, w, h, D, M, sc, w2, y, as_stream(stream));
  Q4_LAUNCHED("pre_normadd_rmsnorm");
  return Q4_OK;
}

size_t q4_gemm_w4a16_normadd_workspace_bytes(int M, int N, int K) { return w4a16_partials_bytes(M, N, K); }

int q4_gemm_w4a16_qkv_prepkv(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M, int N, int K,
                             uint16_t* q, int ldq, int nq, const float* knw, const float* cosM, const float* sinM,
                             uint16_t* kc, uint16_t* vc, int nkv, int hd, int keqv, int stride, int window,
                             const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(q && knw && cosM && sinM && kc && vc && dyn, "null pointer");
  Q4_ARG(nq > 0 && nq % 4 == 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && hd <= ATT_MAX_HD,
         "bad q/k/v sizes nq=%d nkv=%d hd=%d (nq a multiple of 4, hd even and <= %d)", nq, nkv, hd, ATT_MAX_HD);
  Q4_ARG(N == nq + nkv * hd * (keqv ? 1 : 2), "N=%d is not nq + nk%s = %d", N, keqv ? "" : " + nk",
         nq + nkv * hd * (keqv ? 1 : 2));
  Q4_ARG(N % 4 == 0, "N=%d must be a multiple of 4 (16-byte partial rows)", N);
  Q4_ARG(ldq >= nq && ldq % 4 == 0 && ((uintptr_t)q & 7) == 0, "q rows: ldq=%d must be >= nq and a multiple of 4, "
         "q 8-byte aligned", ldq);
  Q4_ARG(stride > 0 && window >= 0 && window <= stride, "bad cache sizes stride=%d window=%d", stride, window);
  int split = 0;
  if (int st = w4a16_partials(X, wq, sc16, M, N, K, ws, ws_bytes, as_stream(stream), &split)) return st;
  const int qb = (nq + QKV_QCOLS - 1) / QKV_QCOLS;
  const int nk = nkv * hd;
  hipLaunchKernelGGL(pre_qkv_prepkv_kernel, dim3(qb + nkv, M), dim3(ATT_THREADS), 0, as_stream(stream),
                     reinterpret_cast<const float*>(ws), split, (long)M * N, N, nq, nq, keqv ? nq : nq + nk, q, ldq,
                     knw, cosM, sinM, kc, vc, hd, stride, window, M, dyn);
  Q4_LAUNCHED("gemm_w4a16_qkv_prepkv reduce + prepkv");
  return Q4_OK;
}

int q4_gemm_w4a16_normadd(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M, int N, int K,
                          const float* w, float* h, float scale, const float* w2, void* y, int y_dtype, void* ws,
                          size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(w && h, "null pointer");
  Q4_ARG((w2 == nullptr) == (y == nullptr), "w2 and y come together (the rmsnorm after the normadd)");
  Q4_ARG(!y || y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y_dtype");
  int split = 0;
  if (int st = w4a16_partials(X, wq, sc16, M, N, K, ws, ws_bytes, as_stream(stream), &split)) return st;
  const float sc = scale == 0.0f ? 1.0f : scale;
  const float* P = reinterpret_cast<const float*>(ws);
  const long ps = (long)M * N;
  hipStream_t st = as_stream(stream);
  if (!y)
    hipLaunchKernelGGL((normadd_kernel<false, Q4_DT_F32, XT_SPLITK>), dim3(M), dim3(NORM_THREADS), 0, st, P, w, h, N,
                       sc, nullptr, nullptr, split, ps);
  else if (y_dtype == Q4_DT_F16)
    hipLaunchKernelGGL((normadd_kernel<true, Q4_DT_F16, XT_SPLITK>), dim3(M), dim3(NORM_THREADS), 0, st, P, w, h, N,
                       sc, w2, y, split, ps);
  else
    hipLaunchKernelGGL((normadd_kernel<true, Q4_DT_F32, XT_SPLITK>), dim3(M), dim3(NORM_THREADS), 0, st, P, w, h, N,
                       sc, w2, y, split, ps);
  Q4_LAUNCHED("gemm_w4a16_normadd normadd");
  return Q4_OK;
}

int q4_pre_gelumul(const void* gate, const void* up, int in_dtype, void* out, int out_dtype, long n, void* stream) {
  clear_error();
  Q4_ARG(gate && up && out, "null pointer");
  Q4_ARG(n > 0 && n <= (1L << 40), "bad n=%ld", n);
  Q4_ARG(in_dtype == Q4_DT_F32 || in_dtype == Q4_DT_F16, "bad in_dtype");
  Q4_ARG(out_dtype == Q4_DT_F32 || out_dtype == Q4_DT_F16, "bad out_dtype");
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = as_stream(stream);
  if (in_dtype == Q4_DT_F16) {
    if (out_dtype == Q4_DT_F16) hipLaunchKernelGGL((gelumul_kernel<Q4_DT_F16, Q4_DT_F16>), grid, dim3(256), 0, st, gate, up, out, n);
    else hipLaunchKernelGGL((gelumul_kernel<Q4_DT_F32, Q4_DT_F16>), grid, dim3(256), 0, st, gate, up, out, n);
  } else {
    if (out_dtype == Q4_DT_F16) hipLaunchKernelGGL((gelumul_kernel<Q4_DT_F16, Q4_DT_F32>), grid, dim3(256), 0, st, gate, up, out, n);
    else hipLaunchKernelGGL((gelumul_kernel<Q4_DT_F32, Q4_DT_F32>), grid, dim3(256), 0, st, gate, up, out, n);
  }
  Q4_LAUNCHED("pre_gelumul");
  return Q4_OK;
}

int q4_pre_prepkv(const void* k, const void* v, int kv_dtype, int ld, const float* knw, const float* cosM,
                  const float* sinM, uint16_t* kc, uint16_t* vc, int nkv, int hd, int stride, int window, int M,
                  const uint32_t* dyn, void* stream) {
  clear_error();
  Q4_ARG(k && v && knw && cosM && sinM && kc && vc && dyn, "null pointer");
  Q4_ARG(kv_dtype == Q4_DT_F32 || kv_dtype == Q4_DT_F16, "bad kv_dtype");
  Q4_ARG(nkv > 0 && M > 0 && stride > 0 && window >= 0, "bad sizes");
  Q4_ARG(hd > 0 && hd % 2 == 0 && hd <= ATT_MAX_HD, "head dim must be even and <= %d (got %d)", ATT_MAX_HD, hd);
  Q4_ARG(ld >= nkv * hd, "row stride %d is shorter than nkv * hd = %d", ld, nkv * hd);
  Q4_ARG(window <= stride, "window %d exceeds the cache depth %d", window, stride);
  if (kv_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(pre_prepkv_kernel<Q4_DT_F16>, dim3(nkv, M), dim3(ATT_THREADS), 0, as_stream(stream), k, v, ld,
                       knw, cosM, sinM, kc, vc, hd, stride, window, M, dyn);
  else
    hipLaunchKernelGGL(pre_prepkv_kernel<Q4_DT_F32>, dim3(nkv, M), dim3(ATT_THREADS), 0, as_stream(stream), k, v, ld,
                       knw, cosM, sinM, kc, vc, hd, stride, window, M, dyn);
  Q4_LAUNCHED("pre_prepkv");
  return Q4_OK;
}


int q4_token_inputs(const int32_t* step, const float* emb, int vocab, int H, float* h, uint32_t* dyn, int ntab,
                    const float* const* cos_tab, const float* const* sin_tab, const int* hd, int max_pos,
                    float* const* cos_out, float* const* sin_out, void* stream) {
  clear_error();
  Q4_ARG(step && emb && h && dyn, "null pointer");
  Q4_ARG(vocab > 0 && H > 0 && max_pos > 0, "bad sizes vocab=%d H=%d max_pos=%d", vocab, H, max_pos);
  Q4_ARG(ntab >= 0 && ntab <= Q4_TOKEN_MAX_TABLES, "at most %d RoPE tables (got %d)", Q4_TOKEN_MAX_TABLES, ntab);
  Q4_ARG((H & 3) != 0 || (((uintptr_t)emb | (uintptr_t)h) & 15) == 0, "emb and h must be 16-byte aligned");
  TokTabs tabs{};
  tabs.count = ntab;
  for (int k = 0; k < ntab; ++k) {
    Q4_ARG(cos_tab && sin_tab && hd && cos_out && sin_out, "null table arrays");
    Q4_ARG(cos_tab[k] && sin_tab[k] && cos_out[k] && sin_out[k], "null pointer in RoPE table %d", k);
    Q4_ARG(hd[k] > 0, "bad head dim %d of RoPE table %d", hd[k], k);
    tabs.cos_tab[k] = cos_tab[k];
    tabs.sin_tab[k] = sin_tab[k];
    tabs.cos_out[k] = cos_out[k];
    tabs.sin_out[k] = sin_out[k];
    tabs.hd[k] = hd[k];
  }
  hipLaunchKernelGGL(token_inputs_kernel, dim3(1 + ntab), dim3(256), 0, as_stream(stream), step, emb, vocab, H, h, dyn,
                     max_pos, tabs);
  Q4_LAUNCHED("token_inputs");
  return Q4_OK;
}

}  // extern "C"
