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
//  * A workgroup (4 waves) owns R consecutive rows of a panel (R = 8..64,
//    chosen per shape so the grid has enough workgroups to fill 256 CUs)
//    and the whole K range: lane = (row r, block slot), 64/R slots per wave,
//    so each wave load covers R*16 contiguous bytes (>= one 128 B line) per
//    block. The x vector is staged once per workgroup in LDS together with
//    per-block sums; slots reduce with xor-shuffles and then across waves
//    through LDS, in a fixed order (deterministic). No cross-workgroup
//    communication is needed for any decode shape.
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
//  * Matrices with fewer than 2048 rows also split K across workgroups; the
//    last workgroup of a row group (atomic ticket, agent-scope
//    release/acquire by one wave) sums the fp32 partials in split order and
//    re-arms the ticket, so the launch stays single and deterministic and
//    the workspace is ready for the next call (and hipGraph replay).
#include "q4mi_common.h"

namespace q4 {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / 64;
constexpr int GEMV_LDS_MAX = 64 * 1024;    // x staging cap per workgroup (bytes)
constexpr int GEMV_TARGET_WGS = 768;       // preferred workgroup count (see plan())
constexpr int GEMV_MIN_WGS = 256;          // one per CU; below this K is split across workgroups
// Split-K workspace layout: tickets for up to GEMV_MAX_TICKETS row groups at
// a fixed offset 0 (so GEMVs of different shapes sharing one workspace never
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

template <int R, int U, int XT, int ST, int YT>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_kernel(const void* __restrict__ xv, const uint4* __restrict__ wq, const void* __restrict__ scv, float outscale,
            void* __restrict__ yv, int N, int nblk, int split, float* __restrict__ part, uint32_t* __restrict__ cnt) {
  constexpr bool XH = (XT == Q4_DT_F16);
  constexpr int SW = 64 / R;               // block slots per wave
  constexpr int S = SW * GEMV_WAVES;       // block slots per workgroup
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[GEMV_WAVES][R];

  const int g = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane % R, slot = wave * SW + lane / R;
  const int b_lo = (int)((long)s * nblk / split);
  const int nb = (int)((long)(s + 1) * nblk / split) - b_lo;
  const long k0 = (long)b_lo * BLK;
  uint32_t* xs_h = smem;
  float* xs_f = reinterpret_cast<float*>(smem);
  float* xsum = reinterpret_cast<float*>(smem + (XH ? nb * 16 : nb * BLK));

  // ---- stage the x slice [k0, k0 + 32 nb). The first round of x loads is
  //      issued, then the first batch of weight units, then the x stores to
  //      LDS: every load is unconditional (indices clamped) so the in-order
  //      load counter lets the x stores wait for the x loads only, and the
  //      weight latency overlaps the staging (the barrier waits on LDS). ----
  constexpr int XU = 4;  // 16-byte x loads per thread per round
  const int n16 = XH ? nb * 4 : nb * 8;
  const uint4* x4 = XH ? reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(xv) + k0)
                       : reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(xv) + k0);
  uint4 t4[XU];
#pragma unroll
  for (int q = 0; q < XU; ++q) t4[q] = x4[min(tid + q * GEMV_THREADS, n16 - 1)];
  const int n0 = g * R;
  const long ubase = ((long)(n0 / PANEL) * nblk + b_lo) * PANEL + (n0 % PANEL) + r;  // unit of block j: ubase + 64 j
  uint4 u[U];
  float sc[U];
#pragma unroll
  for (int t = 0; t < U; ++t) {  // first batch (same as load_batch(slot) below)
    const int jj = min(slot + t * S, nb - 1);
    u[t] = wq[ubase + (long)jj * PANEL];
    sc[t] = load_scale<ST>(scv, ubase + (long)jj * PANEL);
  }
#pragma unroll
  for (int q = 0; q < XU; ++q) {
    const int i = tid + q * GEMV_THREADS;
    if (i < n16) reinterpret_cast<uint4*>(smem)[i] = t4[q];
  }
  for (int i0 = tid + XU * GEMV_THREADS; i0 < n16; i0 += GEMV_THREADS * XU) {  // long K only
#pragma unroll
    for (int q = 0; q < XU; ++q) t4[q] = x4[min(i0 + q * GEMV_THREADS, n16 - 1)];
#pragma unroll
    for (int q = 0; q < XU; ++q) {
      const int i = i0 + q * GEMV_THREADS;
      if (i < n16) reinterpret_cast<uint4*>(smem)[i] = t4[q];
    }
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

  // ---- this lane's blocks: slot, slot + S, slot + 2S, ... in batches of U;
  //      a batch is loaded (unconditionally, clamped) before it is used ----
  auto load_batch = [&](int j) {
#pragma unroll
    for (int t = 0; t < U; ++t) {
      const int jj = min(j + t * S, nb - 1);
      u[t] = wq[ubase + (long)jj * PANEL];
      sc[t] = load_scale<ST>(scv, ubase + (long)jj * PANEL);
    }
  };
  float acc = 0.0f;
  for (int j = slot;;) {
#pragma unroll
    for (int t = 0; t < U; ++t) {
      const int jj = j + t * S;
      if (jj < nb) {
        float d;
        if constexpr (XH) d = block_dot_h(u[t], xs_h + jj * 16, xsum[jj]);
        else d = block_dot_f(u[t], xs_f + jj * BLK, xsum[jj]);
        acc = fmaf(sc[t], d, acc);
      }
    }
    j += S * U;
    if (j >= nb) break;
    load_batch(j);
  }
  // slots of a row: lanes r, r + R, r + 2R, ... of each wave, then the 4 waves
#pragma unroll
  for (int off = R; off < 64; off <<= 1) acc += __shfl_xor(acc, off, 64);
  if (lane < R) red[wave][r] = acc;
  __syncthreads();
  if (wave != 0) return;

  const int n = n0 + r;
  float v = 0.0f;
  if (lane < R) v = (((red[0][r] + red[1][r]) + red[2][r]) + red[3][r]) * outscale;
  if (split == 1) {
    if (lane < R && n < N) {
      if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(yv)[n] = f2h(v);
      else reinterpret_cast<float*>(yv)[n] = v;
    }
    return;
  }

  // ---- split-K: publish this workgroup's partial; the last one reduces ----
  const long NP = (long)gridDim.x * R;
  if (lane < R) part[(long)s * NP + n] = v;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, 64);
  if (prev != (uint32_t)(split - 1)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (lane < R) {
    float t = 0.0f;
    for (int c = 0; c < split; ++c)
      t += __hip_atomic_load(part + (long)c * NP + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n < N) {
      if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(yv)[n] = f2h(t);
      else reinterpret_cast<float*>(yv)[n] = t;
    }
  }
  if (lane == 0) __hip_atomic_store(&cnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*gemv_fn)(const void*, const uint4*, const void*, float, void*, int, int, int, float*, uint32_t*);

template <int R, int U, int XT, int ST>
static gemv_fn pick_y(int yt) {
  return yt == Q4_DT_F16 ? gemv_kernel<R, U, XT, ST, Q4_DT_F16> : gemv_kernel<R, U, XT, ST, Q4_DT_F32>;
}
template <int R, int U, int XT>
static gemv_fn pick_s(int st, int yt) {
  return st == Q4_SCALE_E4M3 ? pick_y<R, U, XT, Q4_SCALE_E4M3>(yt) : pick_y<R, U, XT, Q4_SCALE_F16>(yt);
}
template <int R, int U>
static gemv_fn pick_x(int xt, int st, int yt) {
  return xt == Q4_DT_F16 ? pick_s<R, U, Q4_DT_F16>(st, yt) : pick_s<R, U, Q4_DT_F32>(st, yt);
}
template <int R>
static gemv_fn pick_u(int U, int xt, int st, int yt) {
  return U == 4 ? pick_x<R, 4>(xt, st, yt) : pick_x<R, 8>(xt, st, yt);
}
static gemv_fn pick(int R, int U, int xt, int st, int yt) {
  switch (R) {
    case 64: return pick_u<64>(U, xt, st, yt);
    case 32: return pick_u<32>(U, xt, st, yt);
    case 16: return pick_u<16>(U, xt, st, yt);
    default: return pick_u<8>(U, xt, st, yt);
  }
}

struct GemvPlan {
  int R, U, split, nb_max;
  size_t lds, ws;
};

// Rows per workgroup R, units in flight U and K split for an N x K GEMV
// (measured on MI355X over the decode shapes: the largest R that still gives
// GEMV_TARGET_WGS workgroups, else the largest that gives one per CU; U = 4
// when every lane's blocks fit one batch of 4). Q4MI_GEMV_ROWS (8/16/32/64)
// overrides R for tuning sweeps.
static GemvPlan plan(int N, int K, int split_req, int x_dtype) {
  const int NP = pad_rows(N), nblk = K / BLK;
  int R = 0;
  for (int c : {64, 32, 16, 8})
    if (NP / c >= GEMV_TARGET_WGS) { R = c; break; }
  if (R == 0)
    for (int c : {64, 32, 16, 8})
      if (NP / c >= GEMV_MIN_WGS) { R = c; break; }
  if (R == 0) R = 8;
  if (const char* e = getenv("Q4MI_GEMV_ROWS")) {
    int v = atoi(e);
    if (v == 8 || v == 16 || v == 32 || v == 64) R = v;
  }
  const int wgs = NP / R;
  int s = split_req;
  if (s <= 0) {
    s = 1;
    if (wgs < GEMV_MIN_WGS) {
      s = ceil_div(2 * GEMV_MIN_WGS, wgs);
      const int cap = nblk / 16 > 0 ? nblk / 16 : 1;   // keep >= 16 blocks per workgroup
      if (s > cap) s = cap;
    }
  }
  const int per_block = (x_dtype == Q4_DT_F16 ? 64 : 128) + 4;
  const int max_nb = GEMV_LDS_MAX / per_block;
  if (s < ceil_div(nblk, max_nb)) s = ceil_div(nblk, max_nb);
  if (s > nblk) s = nblk;
  GemvPlan p;
  p.R = R;
  p.split = s;
  p.nb_max = ceil_div(nblk, s);
  p.U = ceil_div(p.nb_max, (64 / R) * GEMV_WAVES) <= 4 ? 4 : 8;
  p.lds = (size_t)p.nb_max * per_block;
  p.ws = 0;
  if (s > 1) p.ws = (GEMV_TICKET_BYTES + (size_t)s * NP * sizeof(float) + 255) & ~(size_t)255;
  return p;
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_gemv_auto_split(int N, int K) {
  if (N <= 0 || K <= 0 || K % BLK) return 1;
  return plan(N, K, 0, Q4_DT_F16).split;
}

size_t q4_workspace_bytes(int op, int N, int K, int split) {
  if (op != Q4_OP_GEMV || N <= 0 || K <= 0 || K % BLK) return 0;
  // size for the larger (fp32-x) staging plan so one workspace serves both activation types
  GemvPlan a = plan(N, K, split, Q4_DT_F16), b = plan(N, K, split, Q4_DT_F32);
  return a.ws > b.ws ? a.ws : b.ws;
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
  Q4_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)x & 15) == 0, "wq and x must be 16-byte aligned");
  Q4_ARG(N <= (1 << 30) && (long)K <= (1L << 24), "GEMV too large");
  const GemvPlan pl = plan(N, K, split, x_dtype);
  Q4_ARG(pl.ws == 0 || (ws && ws_size >= pl.ws), "GEMV N=%d K=%d split=%d needs a %zu-byte workspace (got %zu)", N,
         K, pl.split, pl.ws, ws ? ws_size : (size_t)0);
  const int groups = pad_rows(N) / pl.R;
  Q4_ARG(pl.ws == 0 || groups <= GEMV_MAX_TICKETS, "split-K GEMV supports at most %d row groups", GEMV_MAX_TICKETS);
  uint32_t* cnt = pl.ws ? reinterpret_cast<uint32_t*>(ws) : nullptr;
  float* part = pl.ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + GEMV_TICKET_BYTES) : nullptr;
  const float outscale = scale_fmt == Q4_SCALE_E4M3 ? inv * 256.0f : 1.0f;
  gemv_fn fn = pick(pl.R, pl.U, x_dtype, scale_fmt, y_dtype);
  hipLaunchKernelGGL(fn, dim3(groups, pl.split), dim3(GEMV_THREADS), pl.lds, as_stream(stream), x,
                     reinterpret_cast<const uint4*>(wq), scales, outscale, y, N, K / BLK, pl.split, part, cnt);
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
