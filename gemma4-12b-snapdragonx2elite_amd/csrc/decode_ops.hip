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
//    (head, split) scores up to ATT_CH keys, one key per thread (the q row
//    broadcast from LDS, 16-byte fp16 key loads), forms its chunk's softmax
//    numerator and running max, and accumulates p V with coalesced V-row
//    reads; a second kernel merges the splits' (max, sum, accumulator)
//    triples. The grid covers the cache capacity and splits past the
//    current length exit at once, so the launch shape does not depend on
//    the position.
#include "q4mi_common.h"

namespace q4 {

constexpr int NORM_THREADS = 1024;
constexpr int ATT_THREADS = 256;
constexpr int ATT_CH = 256;       // keys per attention split (one per thread)
constexpr int ATT_MAX_HD = 512;   // head dims up to 512 (global layers)
constexpr float NORM_EPS = 1e-6f;

// Sum over the workgroup, identical in every thread. red: blockDim/64 floats.
__device__ inline float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}
__device__ inline float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
  return m;
}

__device__ inline float inv_rms(float sumsq, int D) { return 1.0f / sqrtf(sumsq / (float)D + NORM_EPS); }

// y = (x * inv) * w   (vk/rmsnorm.comp:8-12); y fp32 or fp16
template <int YT>
__global__ void __launch_bounds__(NORM_THREADS) rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               void* __restrict__ y, int D) {
  __shared__ float red[NORM_THREADS / 64];
  float s = 0.0f;
  for (int i = threadIdx.x; i < D; i += NORM_THREADS) s = fmaf(x[i], x[i], s);
  const float inv = inv_rms(block_sum(s, red), D);
  for (int i = threadIdx.x; i < D; i += NORM_THREADS) {
    const float v = __fmul_rn(__fmul_rn(x[i], inv), w[i]);
    if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(y)[i] = f2h(v);
    else reinterpret_cast<float*>(y)[i] = v;
  }
}

// h = (h + (x * inv) * w) * sc   (vk/normadd.comp:8-12)
__global__ void __launch_bounds__(NORM_THREADS) normadd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                               float* __restrict__ h, int D, float sc) {
  __shared__ float red[NORM_THREADS / 64];
  float s = 0.0f;
  for (int i = threadIdx.x; i < D; i += NORM_THREADS) s = fmaf(x[i], x[i], s);
  const float inv = inv_rms(block_sum(s, red), D);
  for (int i = threadIdx.x; i < D; i += NORM_THREADS)
    h[i] = __fmul_rn(__fadd_rn(h[i], __fmul_rn(__fmul_rn(x[i], inv), w[i])), sc);
}

// out = gelu_tanh(gate) * up   (vk/gelumul.comp:7-8); out fp32 or fp16
template <int YT>
__global__ void __launch_bounds__(256) gelumul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                      void* __restrict__ out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float x = gate[i];
  const float inner = __fmul_rn(0.7978845608028654f, __fadd_rn(x, __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x)));
  const float g = __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
  const float v = __fmul_rn(g, up[i]);
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

__device__ inline int kv_slot(uint32_t pos, int window) { return window > 0 ? (int)(pos % (uint32_t)window) : (int)pos; }

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

__device__ inline int att_len(uint32_t pos, int window, int stride) {
  const long T = window > 0 ? min((long)pos + 1, (long)window) : (long)pos + 1;
  return (int)min(T, (long)stride);
}

// Split blockIdx.y of head blockIdx.x: keys [ATT_CH y, ATT_CH (y+1)) of the
// current length. Writes (max, sum, unnormalised accumulator[hd]) to ws.
__global__ void __launch_bounds__(ATT_THREADS) attn_split_kernel(const float* __restrict__ qkv, const float* __restrict__ qnw,
                                                                 const float* __restrict__ cs, const float* __restrict__ sn,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc, int hd, int stride,
                                                                 int window, int qoff, int grp,
                                                                 const uint32_t* __restrict__ dyn,
                                                                 float* __restrict__ ws) {
  __shared__ float qv[ATT_MAX_HD], qr[ATT_MAX_HD], p[ATT_CH], red[ATT_THREADS / 64];
  __shared__ float accp[ATT_THREADS / 64][ATT_MAX_HD];
  const int h = blockIdx.x, sp = blockIdx.y, t = threadIdx.x;
  const int T = att_len(dyn[0], window, stride);
  const int j0 = sp * ATT_CH;
  if (j0 >= T) return;  // past the current length: the merge reads only the live splits
  const int n = min(ATT_CH, T - j0);
  const int kvh = h / grp;

  // q: norm with weight, RoPE (vk/attn.comp:23-30)
  for (int i = t; i < hd; i += ATT_THREADS) qv[i] = qkv[qoff + h * hd + i];
  __syncthreads();
  norm_rope_head(qv, qr, qnw, cs, sn, hd, red);

  // scores, one key per thread: q . k_j, 8 fp16 per 16-byte load
  float s = -INFINITY;
  if (t < n) {
    const v4u* kr = reinterpret_cast<const v4u*>(kc + ((long)kvh * stride + j0 + t) * hd);
    float d = 0.0f;
    for (int c = 0; c < hd / 8; ++c) {
      const v4u u = kr[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d = fmaf(qr[8 * c + 2 * e], h2f((uint16_t)(u[e] & 0xFFFFu)), d);
        d = fmaf(qr[8 * c + 2 * e + 1], h2f((uint16_t)(u[e] >> 16)), d);
      }
    }
    s = d;
  }
  const float m = block_max(s, red);
  const float pj = t < n ? expf(s - m) : 0.0f;
  p[t] = pj;
  const float l = block_sum(pj, red);  // (its barriers also publish p)

  // p V: wave w takes keys w, w+4, ...; lanes cover hd (coalesced V rows)
  const int wave = t >> 6, lane = t & 63;
  float a[ATT_MAX_HD / 64];
#pragma unroll
  for (int r = 0; r < ATT_MAX_HD / 64; ++r) a[r] = 0.0f;
  for (int j = wave; j < n; j += ATT_THREADS / 64) {
    const uint16_t* vr = vc + ((long)kvh * stride + j0 + j) * hd;
    const float pw = p[j];
#pragma unroll
    for (int r = 0; r < ATT_MAX_HD / 64; ++r)
      if (64 * r + lane < hd) a[r] = fmaf(pw, h2f(vr[64 * r + lane]), a[r]);
  }
#pragma unroll
  for (int r = 0; r < ATT_MAX_HD / 64; ++r)
    if (64 * r + lane < hd) accp[wave][64 * r + lane] = a[r];
  __syncthreads();
  float* out = ws + ((long)h * gridDim.y + sp) * (hd + 2);
  if (t == 0) {
    out[0] = m;
    out[1] = l;
  }
  for (int i = t; i < hd; i += ATT_THREADS) out[2 + i] = ((accp[0][i] + accp[1][i]) + accp[2][i]) + accp[3][i];
}

// out[h] = sum_c acc_c exp(m_c - M) / sum_c l_c exp(m_c - M) over the live splits
__global__ void __launch_bounds__(ATT_THREADS) attn_merge_kernel(const float* __restrict__ ws, float* __restrict__ out,
                                                                 int hd, int nsplit, int stride, int window,
                                                                 const uint32_t* __restrict__ dyn) {
  const int h = blockIdx.x, t = threadIdx.x;
  const int T = att_len(dyn[0], window, stride);
  const int ns = (T + ATT_CH - 1) / ATT_CH;
  const float* w = ws + (long)h * nsplit * (hd + 2);
  float M = -INFINITY;
  for (int c = 0; c < ns; ++c) M = fmaxf(M, w[(long)c * (hd + 2)]);
  float L = 0.0f;
  for (int c = 0; c < ns; ++c) L = fmaf(w[(long)c * (hd + 2) + 1], expf(w[(long)c * (hd + 2)] - M), L);
  for (int i = t; i < hd; i += ATT_THREADS) {
    float a = 0.0f;
    for (int c = 0; c < ns; ++c) a = fmaf(w[(long)c * (hd + 2) + 2 + i], expf(w[(long)c * (hd + 2)] - M), a);
    out[h * hd + i] = a / L;
  }
}

static int attn_splits(int stride) { return ceil_div(stride, ATT_CH); }

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
  hipLaunchKernelGGL(normadd_kernel, dim3(1), dim3(NORM_THREADS), 0, as_stream(stream), x, w, h, D,
                     scale == 0.0f ? 1.0f : scale);
  Q4_LAUNCHED("normadd");
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
  hipLaunchKernelGGL(prepkv_kernel, dim3(nkv), dim3(ATT_THREADS), 0, as_stream(stream), qkv, knw, cosb, sinb, kc, vc,
                     hd, koff, keqv ? koff : voff, stride, window, dyn);
  Q4_LAUNCHED("prepkv");
  return Q4_OK;
}

size_t q4_attn_workspace_bytes(int nH, int hd, int stride) {
  if (nH <= 0 || hd <= 0 || stride <= 0) return 0;
  return (size_t)nH * attn_splits(stride) * (hd + 2) * sizeof(float);
}

int q4_attn(const float* qkv, const float* qnw, const float* cosb, const float* sinb, const uint16_t* kc,
            const uint16_t* vc, float* out, int nH, int nkv, int hd, int stride, int window, int qoff, int grp,
            const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(qkv && qnw && cosb && sinb && kc && vc && out && dyn && ws, "null pointer");
  Q4_ARG(nH > 0 && nkv > 0 && grp > 0 && nH == nkv * grp, "need nH == nkv * grp (got %d, %d, %d)", nH, nkv, grp);
  Q4_ARG(hd > 0 && hd % 8 == 0 && hd <= ATT_MAX_HD, "head dim must be a multiple of 8 and <= %d (got %d)",
         ATT_MAX_HD, hd);
  Q4_ARG(stride > 0 && window >= 0 && window <= stride && qoff >= 0, "bad sizes");
  Q4_ARG(((uintptr_t)kc & 15) == 0, "kc must be 16-byte aligned");
  const size_t need = q4_attn_workspace_bytes(nH, hd, stride);
  Q4_ARG(ws_bytes >= need, "attention workspace too small: %zu < %zu bytes", ws_bytes, need);
  const int ns = attn_splits(stride);
  hipLaunchKernelGGL(attn_split_kernel, dim3(nH, ns), dim3(ATT_THREADS), 0, as_stream(stream), qkv, qnw, cosb, sinb,
                     kc, vc, hd, stride, window, qoff, grp, dyn, reinterpret_cast<float*>(ws));
  Q4_LAUNCHED("attn_split");
  hipLaunchKernelGGL(attn_merge_kernel, dim3(nH), dim3(ATT_THREADS), 0, as_stream(stream),
                     reinterpret_cast<const float*>(ws), out, hd, ns, stride, window, dyn);
  Q4_LAUNCHED("attn_merge");
  return Q4_OK;
}

}  // extern "C"
