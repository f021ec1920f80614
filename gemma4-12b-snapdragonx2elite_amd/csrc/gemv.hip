// int4 block-quantized decode GEMV for gfx950.
//
//   y[n] = inv * sum_b s[n,b] * sum_{k in b} (q[n,k] - 8) * x[k]      (fp32)
//
// Replaces vk/gemv.comp (fp16 scales), vk/gemv_fp8.comp (e4m3 scales) and
// vk/reduce.comp of the reference engine.
//
// Design (MI355X-first, not a translation of the shader):
//  * Weights live in the panel-64 layout: a wave64 owns a 64-row panel,
//    lane = row, and every 16-byte unit load of a wave covers 1 KB of
//    contiguous HBM (one 32-element block of 64 rows). Scales of the same
//    64 rows are 128 contiguous bytes.
//  * A workgroup (4 waves) owns one panel and a contiguous block range;
//    the x slice for that range is staged once in LDS (and summed per
//    block), the 4 waves split the range, and an LDS reduction combines
//    them. No cross-lane shuffles are needed in the inner loop.
//  * Register dequant without conversions: masking a word with 0x000F000F
//    yields two fp16 subnormals q*2^-24; with 0x00F000F0, 16q*2^-24.
//    v_dot2_f32_f16 multiplies them by an fp16 x pair with fp32
//    accumulation (products exact), and the offset-8 is removed once per
//    block with the staged block sum: sum (q-8) x = sum q x - 8 sum x.
//    The device nibble order puts elements (2m, 2m+1) of a word into the
//    two halves, so x pairs are used as stored. 9 VALU ops per 8 weights.
//  * fp32 x (the engine's residual-stream activations) takes an exact fp32
//    path: bytes of (w & 0x0F0F0F0F) and (w >> 4 & 0x0F0F0F0F) convert
//    with v_cvt_f32_ubyteN and accumulate with FMAs.
//  * K is split across workgroups when a matrix has too few panels to fill
//    256 CUs. The last workgroup of a panel (atomic ticket) sums the fp32
//    partials in split order and writes y, then re-arms the ticket, so one
//    launch does the whole GEMV deterministically and the workspace stays
//    ready for the next call (and for hipGraph replay) without a memset.
#include "q4mi_common.h"

namespace q4 {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / 64;
constexpr int GEMV_MAXB = 128;    // blocks of x a workgroup stages (LDS cap)
constexpr int GEMV_U = 8;         // units in flight per lane
constexpr int GEMV_TARGET_WGS = 1024;
// Split-K workspace layout: tickets for up to GEMV_MAX_TICKETS panels at a
// fixed offset 0 (so GEMVs of different shapes sharing one workspace never
// see each other's partials as tickets), then the fp32 partials.
constexpr int GEMV_MAX_TICKETS = 16384;
constexpr size_t GEMV_TICKET_BYTES = GEMV_MAX_TICKETS * sizeof(uint32_t);

__device__ inline v2h as_h2(uint32_t v) { return __builtin_bit_cast(v2h, v); }

// sum_{k in block} (q_k - 8) x_k for fp16 x. xp: 16 fp16 pairs of the block.
__device__ inline float block_dot_h(const uint4 u, const uint32_t* __restrict__ xp, float xsum) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w8 = w[i] >> 8;
    lo = __builtin_amdgcn_fdot2(as_h2(w[i] & 0x000F000Fu), as_h2(xp[4 * i + 0]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(w[i] & 0x00F000F0u), as_h2(xp[4 * i + 1]), hi, false);
    lo = __builtin_amdgcn_fdot2(as_h2(w8 & 0x000F000Fu), as_h2(xp[4 * i + 2]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(w8 & 0x00F000F0u), as_h2(xp[4 * i + 3]), hi, false);
  }
  // lo = 2^-24 * sum q x over low nibbles, hi = 2^-20 * sum q x over high nibbles
  return fmaf(hi, 1048576.0f, lo * 16777216.0f) - 8.0f * xsum;
}

// Same for fp32 x. xf: 32 floats of the block in natural order.
__device__ inline float block_dot_f(const uint4 u, const float* __restrict__ xf, float xsum) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = w[i] & 0x0F0F0F0Fu;          // bytes: e0 e4 e1 e5
    const uint32_t b = (w[i] >> 4) & 0x0F0F0F0Fu;   // bytes: e2 e6 e3 e7
    const float* x = xf + 8 * i;
    acc = fmaf((float)(a & 0xFFu), x[0], acc);
    acc = fmaf((float)((a >> 8) & 0xFFu), x[4], acc);
    acc = fmaf((float)((a >> 16) & 0xFFu), x[1], acc);
    acc = fmaf((float)(a >> 24), x[5], acc);
    acc = fmaf((float)(b & 0xFFu), x[2], acc);
    acc = fmaf((float)((b >> 8) & 0xFFu), x[6], acc);
    acc = fmaf((float)((b >> 16) & 0xFFu), x[3], acc);
    acc = fmaf((float)(b >> 24), x[7], acc);
  }
  return acc - 8.0f * xsum;
}

template <int ST>
__device__ inline float load_scale(const void* __restrict__ scv, long idx) {
  if constexpr (ST == Q4_SCALE_F16) {
    return h2f(reinterpret_cast<const uint16_t*>(scv)[idx]);
  } else {
    return h2f(e4m3_to_h_scaled(reinterpret_cast<const uint8_t*>(scv)[idx]));  // value * 2^-8
  }
}

template <int XT, int ST, int YT>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_kernel(const void* __restrict__ xv, const uint4* __restrict__ wq, const void* __restrict__ scv, float outscale,
            void* __restrict__ yv, int N, int nblk, int split, float* __restrict__ part, uint32_t* __restrict__ cnt) {
  constexpr bool XH = (XT == Q4_DT_F16);
  __shared__ __attribute__((aligned(16))) uint32_t xs_h[XH ? GEMV_MAXB * 16 : 1];
  __shared__ __attribute__((aligned(16))) float xs_f[XH ? 1 : GEMV_MAXB * BLK];
  __shared__ float xsum[GEMV_MAXB];
  __shared__ float red[GEMV_WAVES][64];
  __shared__ int is_last;

  const int p = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int b_lo = (int)((long)s * nblk / split);
  const int nb = (int)((long)(s + 1) * nblk / split) - b_lo;
  const long k0 = (long)b_lo * BLK;

  // ---- stage the x slice [k0, k0 + 32 nb) ----
  if constexpr (XH) {
    const uint32_t* x2 = reinterpret_cast<const uint32_t*>(xv) + k0 / 2;
    for (int i = tid; i < nb * 16; i += GEMV_THREADS) xs_h[i] = x2[i];
  } else {
    const float* xf = reinterpret_cast<const float*>(xv) + k0;
    for (int i = tid; i < nb * BLK; i += GEMV_THREADS) xs_f[i] = xf[i];
  }
  __syncthreads();
  for (int j = tid; j < nb; j += GEMV_THREADS) {
    float t = 0.0f;
    if constexpr (XH) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        v2h pr = as_h2(xs_h[j * 16 + i]);
        t += (float)pr.x + (float)pr.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < BLK; ++i) t += xs_f[j * BLK + i];
    }
    xsum[j] = t;
  }
  __syncthreads();

  // ---- this wave's share of the block range ----
  const int j_lo = wave * nb / GEMV_WAVES, j_hi = (wave + 1) * nb / GEMV_WAVES;
  const long ubase = ((long)p * nblk + b_lo) * PANEL + lane;  // unit (p, b_lo + j) = ubase + 64 j
  float acc = 0.0f;
  for (int j = j_lo; j < j_hi; j += GEMV_U) {
    uint4 u[GEMV_U];
    float sc[GEMV_U];
#pragma unroll
    for (int t = 0; t < GEMV_U; ++t) {
      const int jj = min(j + t, j_hi - 1);
      u[t] = wq[ubase + (long)jj * PANEL];
      sc[t] = load_scale<ST>(scv, ubase + (long)jj * PANEL);
    }
#pragma unroll
    for (int t = 0; t < GEMV_U; ++t) {
      if (j + t < j_hi) {
        float d;
        if constexpr (XH) d = block_dot_h(u[t], xs_h + (j + t) * 16, xsum[j + t]);
        else d = block_dot_f(u[t], xs_f + (j + t) * BLK, xsum[j + t]);
        acc = fmaf(sc[t], d, acc);
      }
    }
  }
  red[wave][lane] = acc;
  __syncthreads();

  const int n = p * PANEL + lane;
  if (split == 1) {
    if (wave == 0 && n < N) {
      float v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
      v *= outscale;
      if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(yv)[n] = f2h(v);
      else reinterpret_cast<float*>(yv)[n] = v;
    }
    return;
  }

  // ---- split-K: publish this workgroup's partial, last one reduces ----
  const long NP = (long)gridDim.x * PANEL;
  if (wave == 0) {
    float v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    part[(long)s * NP + n] = v * outscale;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&cnt[p], 1u);
    is_last = (prev == (uint32_t)(split - 1));
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (wave == 0) {
    float v = 0.0f;
    for (int c = 0; c < split; ++c)
      v += __hip_atomic_load(part + (long)c * NP + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n < N) {
      if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(yv)[n] = f2h(v);
      else reinterpret_cast<float*>(yv)[n] = v;
    }
  }
  if (tid == 0) __hip_atomic_store(&cnt[p], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*gemv_fn)(const void*, const uint4*, const void*, float, void*, int, int, int, float*, uint32_t*);

template <int XT, int ST>
static gemv_fn pick_y(int yt) {
  return yt == Q4_DT_F16 ? gemv_kernel<XT, ST, Q4_DT_F16> : gemv_kernel<XT, ST, Q4_DT_F32>;
}
template <int XT>
static gemv_fn pick_s(int st, int yt) {
  return st == Q4_SCALE_E4M3 ? pick_y<XT, Q4_SCALE_E4M3>(yt) : pick_y<XT, Q4_SCALE_F16>(yt);
}
static gemv_fn pick(int xt, int st, int yt) {
  return xt == Q4_DT_F16 ? pick_s<Q4_DT_F16>(st, yt) : pick_s<Q4_DT_F32>(st, yt);
}

static int auto_split(int N, int K) {
  const int nblk = K / BLK;
  const int panels = ceil_div(N, PANEL);
  int s = ceil_div(GEMV_TARGET_WGS, panels);
  const int cap = nblk / 8 > 0 ? nblk / 8 : 1;  // keep >= 8 blocks (2 per wave) per workgroup
  if (s > cap) s = cap;
  const int need = ceil_div(nblk, GEMV_MAXB);
  if (s < need) s = need;
  return s < 1 ? 1 : s;
}

static int effective_split(int N, int K, int split) {
  const int nblk = K / BLK;
  int s = split > 0 ? split : auto_split(N, K);
  const int need = ceil_div(nblk, GEMV_MAXB);
  if (s < need) s = need;
  if (s > nblk) s = nblk;
  return s;
}

static size_t ws_bytes(int N, int K, int split) {
  if (split <= 1) return 0;
  const size_t NP = (size_t)pad_rows(N);
  size_t b = GEMV_TICKET_BYTES + (size_t)split * NP * sizeof(float);
  return (b + 255) & ~(size_t)255;
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_gemv_auto_split(int N, int K) {
  if (N <= 0 || K <= 0 || K % BLK) return 1;
  return effective_split(N, K, 0);
}

size_t q4_workspace_bytes(int op, int N, int K, int split) {
  if (op != Q4_OP_GEMV || N <= 0 || K <= 0 || K % BLK) return 0;
  return ws_bytes(N, K, effective_split(N, K, split));
}

int q4_workspace_init(void* ws, size_t bytes, void* stream) {
  clear_error();
  if (!ws || bytes == 0) return Q4_OK;
  Q4_HIP(hipMemsetAsync(ws, 0, bytes, as_stream(stream)));
  return Q4_OK;
}

int q4_gemv(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv, void* y,
            int y_dtype, int N, int K, int split, void* ws, size_t ws_size, void* stream) {
  clear_error();
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad GEMV shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  Q4_ARG(x && wq && scales && y, "null pointer");
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x dtype %d", x_dtype);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
  Q4_ARG(scale_fmt == Q4_SCALE_F16 || scale_fmt == Q4_SCALE_E4M3, "bad scale format %d", scale_fmt);
  Q4_ARG(((uintptr_t)wq & 15) == 0, "wq must be 16-byte aligned");
  Q4_ARG(((uintptr_t)x & (x_dtype == Q4_DT_F16 ? 3 : 3)) == 0, "x must be 4-byte aligned");
  Q4_ARG(N <= (1 << 30) && (long)K <= (1L << 24), "GEMV too large");
  const int s = effective_split(N, K, split);
  const size_t need = ws_bytes(N, K, s);
  Q4_ARG(need == 0 || (ws && ws_size >= need), "GEMV N=%d K=%d split=%d needs a %zu-byte workspace (got %zu)", N, K,
         s, need, ws ? ws_size : (size_t)0);
  const int panels = ceil_div(N, PANEL);
  Q4_ARG(need == 0 || panels <= GEMV_MAX_TICKETS, "split-K GEMV supports at most %d rows", GEMV_MAX_TICKETS * PANEL);
  uint32_t* cnt = need ? reinterpret_cast<uint32_t*>(ws) : nullptr;
  float* part = need ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + GEMV_TICKET_BYTES) : nullptr;
  const float outscale = scale_fmt == Q4_SCALE_E4M3 ? inv * 256.0f : 1.0f;
  gemv_fn fn = pick(x_dtype, scale_fmt, y_dtype);
  hipLaunchKernelGGL(fn, dim3(panels, s), dim3(GEMV_THREADS), 0, as_stream(stream), x,
                     reinterpret_cast<const uint4*>(wq), scales, outscale, y, N, K / BLK, s, part, cnt);
  Q4_LAUNCHED("gemv");
  return Q4_OK;
}

int q4_gemv_f16s(const void* x, int x_dtype, const uint32_t* wq, const uint16_t* sc16, void* y, int y_dtype, int N,
                 int K, int split, void* ws, size_t ws_size, void* stream) {
  return q4_gemv(x, x_dtype, wq, sc16, Q4_SCALE_F16, 1.0f, y, y_dtype, N, K, split, ws, ws_size, stream);
}

int q4_gemv_e4m3s(const void* x, int x_dtype, const uint32_t* wq, const uint8_t* sc8, float inv, void* y, int y_dtype,
                  int N, int K, int split, void* ws, size_t ws_size, void* stream) {
  return q4_gemv(x, x_dtype, wq, sc8, Q4_SCALE_E4M3, inv, y, y_dtype, N, K, split, ws, ws_size, stream);
}

}  // extern "C"
