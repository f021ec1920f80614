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
//    chosen per shape so the grid fills 256 CUs) and the whole K range:
//    lane = (row r, block slot), 64/R slots per wave, so each wave load
//    covers R*16 contiguous bytes (>= one 128 B line) per block. Workgroups
//    are ordered XCD-major so the workgroups of one panel share its scale
//    lines in one L2.
//  * The x slice is copied to LDS with direct-to-LDS loads; every lane then
//    keeps U weight units and their scales in flight in a register ring
//    (streaming loads, explicit wait counts): a unit is used as soon as it
//    has landed and its registers are refilled with a unit U places on. U
//    is sized so the whole grid keeps about 8 MB in flight.
//  * Register dequant without conversions: masking a word with 0x000F000F
//    yields two fp16 subnormals q*2^-24; with 0x00F000F0, 16q*2^-24.
//    v_dot2_f32_f16 multiplies them by an fp16 x pair with fp32
//    accumulation (products exact), and the offset 8 is removed once per
//    block with the block sum staged next to x: sum (q-8) x = sum q x -
//    8 sum x. The block scale multiplies the block's sum.
//  * Slots reduce with xor-shuffles and then across waves through LDS, in a
//    fixed order (deterministic).
//  * fp32 x (the engine's residual-stream activations) takes an fp32 path:
//    bytes of (w & 0x0F0F0F0F) and (w >> 4 & 0x0F0F0F0F) convert with
//    v_cvt_f32_ubyteN and accumulate with FMAs.
//  * Matrices with fewer than 2048 rows also split K across workgroups; the
//    last workgroup of a row group (atomic ticket, agent-scope
//    release/acquire by one wave) sums the fp32 partials in split order and
//    re-arms the ticket, so the launch stays single and deterministic and
//    the workspace is ready for the next call (and hipGraph replay).
#include "q4mi_common.h"

#include <mutex>

namespace q4 {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = GEMV_THREADS / 64;
constexpr int GEMV_LDS_MAX = 64 * 1024;    // x staging cap per workgroup (bytes)
constexpr size_t GEMV_MV_LDS_MAX = 144 * 1024;  // x staging cap of the multi-vector GEMV (of 160 KB LDS)
constexpr int GEMV_MV_MAX = 8;              // vectors per multi-vector GEMV launch
constexpr int GEMV_TARGET_WGS = 480;       // preferred workgroup count (see rows_per_group())
constexpr int GEMV_MIN_WGS = 240;          // about one per CU; below this K is split across workgroups
constexpr long GEMV_INFLIGHT_UNITS = 8L << 16;  // 16-byte weight units in flight over a grid (8 MB)
// Split-K workspace layout: tickets for up to GEMV_MAX_TICKETS row groups at
// a fixed offset 0 (so GEMVs of different shapes sharing one workspace never
// see each other's partials as tickets), then the fp32 partials.
constexpr int GEMV_MAX_TICKETS = 16384;
constexpr size_t GEMV_TICKET_BYTES = GEMV_MAX_TICKETS * sizeof(uint32_t);

__device__ inline v2h as_h2(uint32_t v) { return __builtin_bit_cast(v2h, v); }

// sum_{k in block} (q_k - 8) x_k for fp16 x; xp: the block's 16 fp16 pairs,
// xsum: the block's sum of x. Conversion-free dequant: masking a word with
// 0x000F000F yields the fp16 pair q * 2^-24 (two subnormals), with
// 0x00F000F0 the pair 16q * 2^-24; v_dot2_f32_f16 multiplies them by the x
// pair exactly and accumulates in fp32, and the offset 8 is taken off once
// per block with the block sum: sum (q - 8) x = sum q x - 8 sum x. The
// device nibble order puts elements (2m, 2m+1) in the two halves, so the x
// pairs are used as stored. 9 VALU ops per 8 weights.
__device__ inline float block_dot_h(const v4u u, const uint32_t* __restrict__ xp, float xsum) {
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = u[i], w8 = w >> 8;
    lo = __builtin_amdgcn_fdot2(as_h2(w & 0x000F000Fu), as_h2(xp[4 * i + 0]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(w & 0x00F000F0u), as_h2(xp[4 * i + 1]), hi, false);
    lo = __builtin_amdgcn_fdot2(as_h2(w8 & 0x000F000Fu), as_h2(xp[4 * i + 2]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(w8 & 0x00F000F0u), as_h2(xp[4 * i + 3]), hi, false);
  }
  // lo = 2^-24 sum q x over the low nibbles, hi = 2^-20 sum q x over the high ones
  return fmaf(hi, 1048576.0f, lo * 16777216.0f) - 8.0f * xsum;
}

// Same for fp32 x; xf: the block's 32 floats in natural order. Bytes of
// (w & 0x0F0F0F0F) are elements e0 e4 e1 e5, of (w >> 4 & 0x0F0F0F0F)
// e2 e6 e3 e7; q - 8 is exact in fp32.
__device__ inline float block_dot_f(const v4u u, const float* __restrict__ xf) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = u[i] & 0x0F0F0F0Fu;
    const uint32_t b = (u[i] >> 4) & 0x0F0F0F0Fu;
    const float* x = xf + 8 * i;
    acc = fmaf((float)(a & 0xFFu) - 8.0f, x[0], acc);
    acc = fmaf((float)((a >> 8) & 0xFFu) - 8.0f, x[4], acc);
    acc = fmaf((float)((a >> 16) & 0xFFu) - 8.0f, x[1], acc);
    acc = fmaf((float)(a >> 24) - 8.0f, x[5], acc);
    acc = fmaf((float)(b & 0xFFu) - 8.0f, x[2], acc);
    acc = fmaf((float)((b >> 8) & 0xFFu) - 8.0f, x[6], acc);
    acc = fmaf((float)((b >> 16) & 0xFFu) - 8.0f, x[3], acc);
    acc = fmaf((float)(b >> 24) - 8.0f, x[7], acc);
  }
  return acc;
}

// Load of the block scale at index idx, as raw bits. Not a streaming load:
// a panel's 128-byte scale line is shared by the 64/R workgroups of that
// panel, which should find it in L2.
template <int ST>
__device__ inline uint32_t load_scale(const void* __restrict__ scv, long idx) {
  if constexpr (ST == Q4_SCALE_F16) return ld2(reinterpret_cast<const uint16_t*>(scv) + idx);
  else return ld1(reinterpret_cast<const uint8_t*>(scv) + idx);
}
template <int ST>
__device__ inline float scale_value(uint32_t bits) {
  if constexpr (ST == Q4_SCALE_F16) return h2f((uint16_t)bits);
  else return h2f(e4m3_to_h_scaled(bits));  // value * 2^-8
}

// Row group of workgroup b in a launch of G workgroups. Workgroups are
// dispatched round-robin over the 8 XCDs (b % 8), each with its own L2.
// XCD-major order gives every XCD one contiguous range of row groups, so
// the 64/R workgroups of a 64-row panel, which share the panel's 128-byte
// scale lines, run on one XCD (at most one panel per XCD boundary is split)
// and each line is fetched from HBM once instead of once per XCD.
__device__ inline int xcd_major(int b, int G) {
  const int x = b & 7, per = G >> 3, rem = G & 7;
  return x * per + min(x, rem) + (b >> 3);
}

// Output of wave 0 (all 64 lanes call this; lanes with live hold row n):
// y[n], or, for a gate/up matrix with interleaved rows (row 2i = gate row
// i, row 2i + 1 = up row i), act[i] = gelu_tanh(y[2i]) * y[2i + 1]: the
// pair sits in lanes r, r ^ 1 of the wave (R and the row group's first row
// are even). This is vk/gelumul.comp applied in the GEMV's epilogue.
template <int YT>
__device__ inline void store_rows(void* __restrict__ yv, int n, float v, int N, bool live, int gated) {
  int o = n;
  if (gated) {
    const float up = dpp_f<DPP_XOR1>(v);
    if (n & 1) return;
    v = __fmul_rn(gelu_tanh(v), up);
    o = n >> 1;
  }
  if (live && n < N) {
    if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(yv)[o] = f2h(v);
    else reinterpret_cast<float*>(yv)[o] = v;
  }
}

// 32-bit words of LDS one row group stages for nb blocks (the x blocks of
// its 4 waves in whole 1 KB direct-load rows, then their fp32 block sums for
// fp16 x); the host's x_stage_lds() is the same size in bytes.
template <int R, int XT>
__device__ inline int stage_words(int nb) {
  constexpr int SW = 64 / R, S = SW * GEMV_WAVES, XB = XT == Q4_DT_F16 ? 64 : 128, BPD = 1024 / XB;
  const int nbw = (nb + S - 1) / S * SW, nvw = (nbw + BPD - 1) / BPD;
  return GEMV_WAVES * nvw * 256 + (XT == Q4_DT_F16 ? GEMV_WAVES * nbw : 0);
}

// Fused input of a GEMV (the normadd and rmsnorm recorded before it,
// vk/normadd.comp:8-12 then vk/rmsnorm.comp:8-12 on the new residual):
//   h_out = (h + (a * inv_rms(a)) * w) * sc,   x = f16((h_out * inv_rms(h_out)) * w2)
// over K = D elements. Every workgroup computes x itself (the GEMV's x is
// never written to memory); workgroup 0 writes h_out, which must not alias
// h or a (other workgroups may still be reading them).
struct NormIn {
  const float* a;
  const float* w;
  const float* h;
  float* h_out;
  const float* w2;
  float sc;
};
constexpr int NX_PER = 4;                                    // 16-byte loads per thread per operand
constexpr int NX_MAX_K = NX_PER * 4 * GEMV_THREADS;          // 4096 elements

// Sum over the 4 waves of one 256-thread half, in a fixed order (slot: 4
// floats of the half's own LDS).
__device__ inline float half_sum(float v, float* slot) {
  v = reduce64<false>(v);
  if ((threadIdx.x & 63) == 0) slot[(threadIdx.x >> 6) & (GEMV_WAVES - 1)] = v;
  __syncthreads();
  return ((slot[0] + slot[1]) + slot[2]) + slot[3];
}

// The normadd + rmsnorm of a NormIn on the operands this thread loaded
// (elements 4 i4 .. 4 i4 + 3 for i4 = t + 256 r), the fp16 result written
// straight into the per-wave x staging areas of gemv_rows (block j belongs
// to wave (j mod S) / SW at local block (j / S) SW + j mod SW), then one
// barrier. Arithmetic per element as normadd_kernel's. (Elements are
// converted by value, __uint_as_float(v[c]): a bit cast of a vector element
// lvalue inside an unrolled loop is compiled to element 0 every time.)
template <int R>
__device__ inline void nx_stage(const NormIn& nx, const v4u* na, const v4u* nh, const v4u* nw, const v4u* nw2,
                                int nblk, int nvw, uint32_t* __restrict__ smem, float (*red)[R], bool writer) {
  static_assert(R >= GEMV_WAVES, "reduction slots");
  constexpr int SW = 64 / R, S = SW * GEMV_WAVES;
  const int ht = threadIdx.x & (GEMV_THREADS - 1), D = nblk * BLK, K4 = D / 4;
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < NX_PER; ++r) {
    const bool ok = ht + GEMV_THREADS * r < K4;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float a = ok ? __uint_as_float(na[r][c]) : 0.0f;
      s = fmaf(a, a, s);
    }
  }
  const float inv = inv_rms(half_sum(s, red[0]), D);
  float hv[NX_PER][4];
  float s2 = 0.0f;
#pragma unroll
  for (int r = 0; r < NX_PER; ++r) {
    const bool ok = ht + GEMV_THREADS * r < K4;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float a = __uint_as_float(na[r][c]), w = __uint_as_float(nw[r][c]);
      const float v = __fmul_rn(__fadd_rn(__uint_as_float(nh[r][c]), __fmul_rn(__fmul_rn(a, inv), w)), nx.sc);
      hv[r][c] = ok ? v : 0.0f;
      s2 = fmaf(hv[r][c], hv[r][c], s2);
    }
  }
  const float inv2 = inv_rms(half_sum(s2, red[1]), D);
#pragma unroll
  for (int r = 0; r < NX_PER; ++r) {
    const int i4 = ht + GEMV_THREADS * r;
    if (i4 < K4) {
      uint32_t e[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) e[c] = f2h(__fmul_rn(__fmul_rn(hv[r][c], inv2), __uint_as_float(nw2[r][c])));
      const int j = i4 / (BLK / 4), lb = j / S * SW + j % SW;
      uint32_t* dst = smem + ((j % S) / SW) * nvw * 256 + lb * 16 + (i4 % (BLK / 4)) * 2;
      *reinterpret_cast<uint2*>(dst) = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
      if (writer) *reinterpret_cast<float4*>(nx.h_out + 4 * i4) = make_float4(hv[r][0], hv[r][1], hv[r][2], hv[r][3]);
    }
  }
  __syncthreads();
}

// Rows [lo, lo + cnt) of row group g: a balanced partition of the rows into
// groups of gq units plus one more unit for the first gr groups (gq, gr =
// quotient and remainder of the units by the group count, from the host), a
// unit being a row, or a row pair for a gated matrix (row 2i = gate row i,
// 2i + 1 = up row i stay together). One 32-bit multiply: the first weight
// addresses wait for it.
__device__ inline void group_rows(int g, int gq, int gr, int gated, int& lo, int& cnt) {
  const int u = gated ? 2 : 1;
  lo = (g * gq + min(g, gr)) * u;
  cnt = (gq + (g < gr ? 1 : 0)) * u;
}
// (gq, gr) of Gm groups over N rows
__host__ inline void group_split(int N, int Gm, int gated, int& gq, int& gr) {
  const int Nu = gated ? N / 2 : N;
  gq = Nu / Gm;
  gr = Nu % Gm;
}

// Rows [lo, lo + cnt) (group_rows(g, gq, gr): cnt <= R) of one GEMV over the K
// slice s of split (the whole K when split == 1); lane row r >= cnt
// repeats row lo + cnt - 1 and stores nothing. The rows may span two
// panels. NP = split-K partial stride (>= N).
//
// Order of work per wave: (1) direct-to-LDS loads of the wave's share of the
// x slice (no registers), (2) the lane's first U weight units (streaming
// loads) and scales (clamped indices so the count is static), (3) wait for
// the x loads only (s_waitcnt vmcnt(2U): loads return in order) and one
// barrier, (4) each unit is used as soon as it has landed and its registers
// are refilled with the lane's unit U places further on, so every lane keeps
// U units in flight until its last round.
//
// NX (fp16 x, split 1): x is not read from memory but formed from the
// NormIn's operands, which are loaded in place of step (1) (before the
// weights, so the same wait covers them) and turned into x in LDS after it.
template <int R, int U, int XT, int ST, int YT, bool NX = false>
__device__ __forceinline__ void gemv_rows(const void* __restrict__ xv, const uint4* __restrict__ wq,
                                          const void* __restrict__ scv, float outscale, void* __restrict__ yv,
                                          int N, int nblk, int g, int gq, int gr, int s, int split, long NP,
                                          float* __restrict__ part, uint32_t* __restrict__ cnt,
                                          uint32_t* __restrict__ smem, float (*red)[R], int gated,
                                          NormIn nx = {}) {
  static_assert(!NX || XT == Q4_DT_F16, "fused norm input is staged as fp16");
  constexpr bool XH = (XT == Q4_DT_F16);
  constexpr int SW = 64 / R;               // block slots per wave
  constexpr int S = SW * GEMV_WAVES;       // block slots per workgroup
  const int tid = threadIdx.x, wave = (tid >> 6) & (GEMV_WAVES - 1), lane = tid & 63;  // wave within its half
  const int r = lane % R, slot = wave * SW + lane / R;
  int b_lo = 0, nb = nblk;
  if (split > 1) {  // (a 64-bit division: kept off the common path)
    b_lo = (int)((long)s * nblk / split);
    nb = (int)((long)(s + 1) * nblk / split) - b_lo;
  }
  const long k0 = (long)b_lo * BLK;

  // (1) the x blocks this wave uses -> LDS, 1 KB per direct-load
  //     instruction. Wave w uses blocks j with (j mod S) / SW == w, i.e. SW
  //     consecutive blocks every S; its local block lb = (j / S) SW + j mod SW
  //     is stored at lb * XB in the wave's own area (positions past the
  //     slice re-read its last block), so no other wave's data is needed.
  constexpr int XB = XH ? 64 : 128;         // x bytes per block
  constexpr int CPB = XB / 16;              // 16-byte chunks per block
  constexpr int BPD = 64 / CPB;             // blocks per direct load
  const int nbw = (nb + S - 1) / S * SW;    // local blocks per wave (wave-uniform)
  const int nvw = (nbw + BPD - 1) / BPD;    // direct loads per wave
  uint32_t* xw = smem + wave * nvw * 256;
  [[maybe_unused]] v4u na[NX ? NX_PER : 1], nh[NX ? NX_PER : 1], nw[NX ? NX_PER : 1], nw2[NX ? NX_PER : 1];
  if constexpr (NX) {
    // index clamped so every thread issues the same loads; elements past K are zeroed in nx_stage
    const int ht = threadIdx.x & (GEMV_THREADS - 1), K4 = nblk * (BLK / 4);
#pragma unroll
    for (int v = 0; v < NX_PER; ++v) {
      const long o = 4L * min(ht + GEMV_THREADS * v, K4 - 1);
      na[v] = ld16(nx.a + o);
      nh[v] = ld16(nx.h + o);
      nw[v] = ld16(nx.w + o);
      nw2[v] = ld16(nx.w2 + o);
    }
  } else {
    const uint8_t* xsrc = reinterpret_cast<const uint8_t*>(xv) + k0 * (XH ? 2 : 4);
    for (int v = 0; v < nvw; ++v) {
      const int lb = v * BPD + lane / CPB;
      const int j = min(lb / SW * S + wave * SW + lb % SW, nb - 1);
      dma16(xsrc + (long)j * XB + (lane % CPB) * 16, xw + v * 256);
    }
  }

  // (2) first U weight units and scales of the lane: blocks slot, slot + S, ...
  int n0, rows;
  group_rows(g, gq, gr, gated, n0, rows);
  const bool live = r < rows;
  const int nl = n0 + min(r, rows - 1);
  const long ubase = ((long)(nl / PANEL) * nblk + b_lo) * PANEL + (nl % PANEL);  // unit of block j: ubase + 64 j
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(wq);
  v4u u[U];
  uint32_t sb[U];
#pragma unroll
  for (int t = 0; t < U; ++t) {
    const long ix = ubase + (long)min(slot + t * S, nb - 1) * PANEL;
    u[t] = ld16_nt(wb + ix * 16);
    sb[t] = load_scale<ST>(scv, ix);
  }
  // (3) this wave's x blocks have landed (loads complete in order); for fp16
  //     x the wave sums each of its blocks into its own LDS area. A wave's
  //     LDS operations execute in order: no barrier is needed.
  vmwait<2 * U>();
  if constexpr (NX) {
#pragma unroll
    for (int v = 0; v < NX_PER; ++v) {
      pin(na[v]);
      pin(nh[v]);
      pin(nw[v]);
      pin(nw2[v]);
    }
    nx_stage<R>(nx, na, nh, nw, nw2, nblk, nvw, smem, red, blockIdx.x == 0 && threadIdx.x < GEMV_THREADS);
  }
  const uint32_t* xs_h = xw;
  const float* xs_f = reinterpret_cast<const float*>(xw);
  float* xsum = reinterpret_cast<float*>(smem + GEMV_WAVES * nvw * 256) + wave * nbw;
  if constexpr (XH) {
    const v2h one2 = {(_Float16)1.0f, (_Float16)1.0f};
    for (int lb = lane; lb < nbw; lb += 64) {
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) t = __builtin_amdgcn_fdot2(as_h2(xs_h[lb * 16 + i]), one2, t, false);
      xsum[lb] = t;
    }
  }

  // (4) dot products, unit by unit as they arrive. Unit c of the lane is
  //     block slot + c S, local block c SW + slot % SW. In every round but
  //     the last, unit t's registers are refilled with unit t + U right
  //     after use, so U units (2U loads) stay in flight and unit t is always
  //     2(U-1) loads behind the newest; the last round drains them.
  float acc = 0.0f;
  auto use = [&](int jj, int lb, const v4u& w, uint32_t sv) {
    if (jj < nb) {
      float d;
      if constexpr (XH) d = block_dot_h(w, xs_h + lb * 16, xsum[lb]);
      else d = block_dot_f(w, xs_f + lb * BLK);
      acc = fmaf(scale_value<ST>(sv), d, acc);
    }
  };
  const int rounds = ((nb + S - 1) / S + U - 1) / U;  // wave-uniform (slot 0 has the most units)
  int j = slot, lb = lane / R;
  for (int rd = 1; rd < rounds; ++rd) {
    static_for<0, U>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      vmwait<2 * (U - 1)>();
      pin(u[t]);
      pin(sb[t]);
      use(j + t * S, lb + t * SW, u[t], sb[t]);
      const long ix = ubase + (long)min(j + (t + U) * S, nb - 1) * PANEL;
      u[t] = ld16_nt(wb + ix * 16);
      sb[t] = load_scale<ST>(scv, ix);
    });
    j += S * U;
    lb += SW * U;
  }
  static_for<0, U>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    vmwait<2 * (U - 1 - t)>();
    pin(u[t]);
    pin(sb[t]);
    use(j + t * S, lb + t * SW, u[t], sb[t]);
  });
  // slots of a row: lanes r, r + R, r + 2R, ... of each wave, then the 4 waves
  acc = slot_sum<R>(acc);
  if (lane < R) red[wave][r] = acc;
  __syncthreads();
  if (wave != 0) return;

  const int n = n0 + r;
  const bool own = lane < R && live;
  float v = 0.0f;
  if (own) v = (((red[0][r] + red[1][r]) + red[2][r]) + red[3][r]) * outscale;
  if (split == 1) {
    store_rows<YT>(yv, n, v, N, own, gated);
    return;
  }

  // ---- split-K: publish this workgroup's partial; the last one reduces ----
  if (own) part[(long)s * NP + n] = v;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(&cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, 64);
  if (prev != (uint32_t)(split - 1)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  float t = 0.0f;
  if (own)
    for (int c = 0; c < split; ++c)
      t += __hip_atomic_load(part + (long)c * NP + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  store_rows<YT>(yv, n, t, N, own, gated);
  if (lane == 0) __hip_atomic_store(&cnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A workgroup of 256 threads runs one row group; one of 512 threads runs two
// adjacent row groups (halves of 4 waves, each with its own LDS area and
// reduction slots; split 1 only): both start together and share the CU from
// the first cycle, where two 256-thread workgroups on one CU would start one
// after the other and the second one's x copy would wait behind the first
// one's weight loads.
template <int R, int U, int XT, int ST, int YT>
__global__ void __launch_bounds__(2 * GEMV_THREADS)
gemv_kernel(const void* __restrict__ xv, const uint4* __restrict__ wq, const void* __restrict__ scv, float outscale,
            void* __restrict__ yv, int N, int nblk, int split, float* __restrict__ part, uint32_t* __restrict__ cnt,
            int gated, int gq, int gr) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[2][GEMV_WAVES][R];
  const int halves = blockDim.x / GEMV_THREADS, half = threadIdx.x / GEMV_THREADS;
  // split-K grids (small matrices only) keep the plain order: their row
  // groups are reduced through the workspace, not through L2 reuse
  const int g = (gridDim.y == 1 ? xcd_major(blockIdx.x, gridDim.x) : blockIdx.x) * halves + half;
  gemv_rows<R, U, XT, ST, YT>(xv, wq, scv, outscale, yv, N, nblk, g, gq, gr, blockIdx.y, split, N, part, cnt,
                              smem + half * stage_words<R, XT>(nblk), red[half], gated);
}

// Several activation vectors through one weight stream (speculative-decode
// verification: M <= MV tokens against the same matrix): rows [g*R, g*R+R)
// of Y[v][n] = GEMV(x_v) for v < M, fp16 x rows of X[M][K]. The structure
// is gemv_rows' (per-wave x staging, now MV vectors per wave, the load ring,
// split 1) and each vector's arithmetic is q4_gemv's exactly (same block
// dot product, same block order, same reduction order), so every output
// row is bit-identical to a single GEMV with the same plan; the weight
// words and scales are loaded once for all vectors.
template <int R, int U, int ST, int YT, int MV>
__device__ __forceinline__ void gemv_rows_mv(const uint16_t* __restrict__ X, int M, const uint4* __restrict__ wq,
                                             const void* __restrict__ scv, float outscale, void* __restrict__ Y,
                                             int ldy, int N, int nblk, int g, uint32_t* __restrict__ smem,
                                             float (*red)[MV][R]) {
  constexpr int SW = 64 / R, S = SW * GEMV_WAVES;
  constexpr int XB = 64, CPB = XB / 16, BPD = 64 / CPB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane % R, slot = wave * SW + lane / R;
  const int nb = nblk;
  const int nbw = (nb + S - 1) / S * SW, nvw = (nbw + BPD - 1) / BPD;
  // LDS: wave w's x areas (one per vector, nvw KB each), then every wave's
  // block sums (nbw floats per vector)
  uint32_t* xw = smem + wave * MV * nvw * 256;
#pragma unroll
  for (int v = 0; v < MV; ++v) {
    const uint8_t* xsrc = reinterpret_cast<const uint8_t*>(X + (long)min(v, M - 1) * nblk * BLK);
    for (int d = 0; d < nvw; ++d) {
      const int lb = d * BPD + lane / CPB;
      const int j = min(lb / SW * S + wave * SW + lb % SW, nb - 1);
      dma16(xsrc + (long)j * XB + (lane % CPB) * 16, xw + (v * nvw + d) * 256);
    }
  }
  const int n0 = g * R;
  const long ubase = ((long)(n0 / PANEL) * nblk) * PANEL + (n0 % PANEL) + r;
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(wq);
  v4u u[U];
  uint32_t sb[U];
#pragma unroll
  for (int t = 0; t < U; ++t) {
    const long ix = ubase + (long)min(slot + t * S, nb - 1) * PANEL;
    u[t] = ld16_nt(wb + ix * 16);
    sb[t] = load_scale<ST>(scv, ix);
  }
  vmwait<2 * U>();
  float* xsum = reinterpret_cast<float*>(smem + GEMV_WAVES * MV * nvw * 256) + wave * MV * nbw;
  {
    const v2h one2 = {(_Float16)1.0f, (_Float16)1.0f};
    for (int lb = lane; lb < nbw; lb += 64) {
#pragma unroll
      for (int v = 0; v < MV; ++v) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) t = __builtin_amdgcn_fdot2(as_h2(xw[(v * nvw) * 256 + lb * 16 + i]), one2, t, false);
        xsum[v * nbw + lb] = t;
      }
    }
  }
  float acc[MV];
#pragma unroll
  for (int v = 0; v < MV; ++v) acc[v] = 0.0f;
  auto use = [&](int jj, int lb, const v4u& w, uint32_t sv) {
    if (jj < nb) {
      const float sc = scale_value<ST>(sv);
#pragma unroll
      for (int v = 0; v < MV; ++v)
        acc[v] = fmaf(sc, block_dot_h(w, xw + (v * nvw) * 256 + lb * 16, xsum[v * nbw + lb]), acc[v]);
    }
  };
  const int rounds = ((nb + S - 1) / S + U - 1) / U;
  int j = slot, lb = lane / R;
  for (int rd = 1; rd < rounds; ++rd) {
    static_for<0, U>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      vmwait<2 * (U - 1)>();
      pin(u[t]);
      pin(sb[t]);
      use(j + t * S, lb + t * SW, u[t], sb[t]);
      const long ix = ubase + (long)min(j + (t + U) * S, nb - 1) * PANEL;
      u[t] = ld16_nt(wb + ix * 16);
      sb[t] = load_scale<ST>(scv, ix);
    });
    j += S * U;
    lb += SW * U;
  }
  static_for<0, U>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    vmwait<2 * (U - 1 - t)>();
    pin(u[t]);
    pin(sb[t]);
    use(j + t * S, lb + t * SW, u[t], sb[t]);
  });
#pragma unroll
  for (int v = 0; v < MV; ++v) {
    acc[v] = slot_sum<R>(acc[v]);
    if (lane < R) red[wave][v][r] = acc[v];
  }
  __syncthreads();
  if (wave != 0) return;
  const int n = n0 + r;
  for (int v = 0; v < M && v < MV; ++v) {
    if (lane < R && n < N) {
      const float y = (((red[0][v][r] + red[1][v][r]) + red[2][v][r]) + red[3][v][r]) * outscale;
      if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(Y)[(long)v * ldy + n] = f2h(y);
      else reinterpret_cast<float*>(Y)[(long)v * ldy + n] = y;
    }
  }
}

template <int R, int U, int ST, int YT, int MV>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_multi_kernel(const uint16_t* __restrict__ X, int M, const uint4* __restrict__ wq, const void* __restrict__ scv,
                  float outscale, void* __restrict__ Y, int ldy, int N, int nblk) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[GEMV_WAVES][MV][R];
  gemv_rows_mv<R, U, ST, YT, MV>(X, M, wq, scv, outscale, Y, ldy, N, nblk, xcd_major(blockIdx.x, gridDim.x), smem,
                                 red);
}

// ---- small-M GEMV on MFMA ------------------------------------------------------
// Y[m][n] = outscale * sum_b s[n,b] * sum_{k in b} (q[n,k] - 8) x_m[k] for up
// to 16 fp16 vectors x_m, the decode GEMV's arithmetic per block (exact
// (q - 8) times fp16 x summed in fp32, times the fp32 block scale, blocks
// accumulated in fp32) with the block sums of all vectors from one
// v_mfma_f32_16x16x32_f16 per 16 rows and block:
//   A (16 x 32) = the block's x slice of the 16 vector slots (slot m >= M
//                 repeats vector M - 1; its outputs are not stored),
//   B (32 x 16) = (q - 8) of 16 weight rows, exact in fp16,
//   D (16 x 16) = per-block sums; lane (c, g) = (lane % 16, lane / 16) holds
//                 vectors 4g .. 4g+3 of weight row c and adds them, times the
//                 block scale of row c, to its fp32 accumulators.
// Lane (c, g) supplies k = 8g .. 8g+7 of the block to both operands: x
// elements 8g .. 8g+7 (16 bytes) and word g of the row's 16-byte unit
// (elements 8g .. 8g+7 at nibbles (e & 1) * 4 + (e >> 1)). Dequant: the
// masked nibble pairs OR 0x6400 (low nibbles: 1024 + q) or 0x5400 (high
// nibbles, mantissa bits 4-7: 64 + q), minus 1032 or 72, give q - 8
// exactly; 9 VALU operations per 8 codes, whatever the number of vectors.
//
// A workgroup (4 waves) owns T tiles of 16 rows (16T rows of one 64-row
// panel). One step of a wave covers 4 (tile, block) pairs, 4/T blocks of
// all T tiles: each lane loads one whole 16-byte unit (lane (c, g): tile
// g % T, row c, block g / T of the step; 1 KB of contiguous weights per
// wave for T = 4), and a 4 x 4 transpose of the words across the four
// 16-lane rows (two v_permlane32_swap, two v_permlane16_swap) hands lane
// (c, g) word g of the 4 units of its column, one per MFMA. Steps go to
// the waves round-robin (the 4 waves read adjacent blocks together); U
// steps of loads stay in flight (x slices, the unit, 4 scales per step;
// explicit wait counts as in the GEMV), and the 4 waves' partial sums meet
// in LDS in wave order (deterministic).
__device__ inline v8h codes_to_h8(uint32_t w) {
  const uint32_t w8 = w >> 8;
  const v2h lo = {(_Float16)-1032.0f, (_Float16)-1032.0f}, hi = {(_Float16)-72.0f, (_Float16)-72.0f};
  const v2h p0 = as_h2(and_or(w, 0x000F000Fu, 0x64006400u)) + lo;   // e0 e1
  const v2h p1 = as_h2(and_or(w, 0x00F000F0u, 0x54005400u)) + hi;   // e2 e3
  const v2h p2 = as_h2(and_or(w8, 0x000F000Fu, 0x64006400u)) + lo;  // e4 e5
  const v2h p3 = as_h2(and_or(w8, 0x00F000F0u, 0x54005400u)) + hi;  // e6 e7
  return v8h{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// 4 x 4 transpose across the 16-lane rows: on entry word j of lane (c, g)
// is element (g, j); on return word t of lane (c, g) is element (t, g), the
// word g of the unit that lane (c, t) loaded.
__device__ inline v4u transpose_rows(v4u a) {
  const auto p02 = __builtin_amdgcn_permlane32_swap(a[0], a[2], false, false);
  const auto p13 = __builtin_amdgcn_permlane32_swap(a[1], a[3], false, false);
  const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
  const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
  return v4u{q01[0], q01[1], q23[0], q23[1]};
}

// Scale bits at a uniform base + the lane's offset + OFF bytes.
template <int ST, int OFF>
__device__ inline uint32_t mm_scale(const uint8_t* sbase, uint32_t voff) {
  if constexpr (ST == Q4_SCALE_F16) return ld2_so_off<OFF>(sbase, voff);
  else return ld1_so_off<OFF>(sbase, voff);
}

template <int T, int U, int ST, int YT>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_mm_kernel(const uint16_t* __restrict__ X, int M, const uint8_t* __restrict__ wq, const void* __restrict__ scv,
               float outscale, void* __restrict__ Y, int N, int nblk, int kspan, float* __restrict__ part) {
  constexpr int BPS = 4 / T;                      // blocks per step
  constexpr int L = BPS + 1 + 4;                  // loads per step: x slices, the unit, 4 scales
  constexpr int SB = ST == Q4_SCALE_F16 ? 2 : 1;  // scale bytes
  static_assert(U * L < 64, "vmcnt range");
  __shared__ v4f red[GEMV_WAVES][T][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: block indices and bases live in SGPRs
  const int c = lane & 15, g = lane >> 4;
  const int n0 = xcd_major(blockIdx.x, gridDim.x) * 16 * T;
  // K split ky (blockIdx.y) owns blocks [kb0, kb0 + nb); the host leaves no split empty
  const int ky = blockIdx.y, kb0 = ky * kspan, nb = min(kspan, nblk - kb0);
  // unit index of (row n0 + r, block b) = pu + r + 64 b (the 16T rows lie in one panel)
  const long pu = (long)(n0 / PANEL) * nblk * PANEL + (n0 % PANEL);
  const uint8_t* xbase = reinterpret_cast<const uint8_t*>(X) + (long)kb0 * (BLK * 2);
  const uint8_t* wbase = wq + pu * 16 + (long)kb0 * (PANEL * 16);
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>(scv) + (pu + (long)kb0 * PANEL) * SB;
  const uint32_t xo = (uint32_t)min(c, M - 1) * (uint32_t)(nblk * BLK * 2) + g * 16;
  const int lrow = 16 * (g % T) + c, lblk = g / T;  // the unit lane (c, g) loads: row, block within the step
  const uint32_t so = c * SB;
  const int nsteps = (nb + BPS - 1) / BPS;
  const int rounds = ((nsteps + GEMV_WAVES - 1) / GEMV_WAVES + U - 1) / U;
  v4u xr[U][BPS], wr[U];
  uint32_t sr[U][4];
  auto issue = [&](int u, int s) {
    const int b0 = (wave + GEMV_WAVES * s) * BPS;  // first block of the step
    static_for<0, BPS>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      xr[u][i] = ld16_so(xbase + (long)min(b0 + i, nb - 1) * (BLK * 2), xo);
    });
    wr[u] = ld16_so(wbase, (uint32_t)(lrow * 16) + ((uint32_t)min(b0 + lblk, nb - 1) << 10));
    static_for<0, 4>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      sr[u][j] = mm_scale<ST, 16 * (j % T) * SB>(sbase + (long)min(b0 + j / T, nb - 1) * (PANEL * SB), so);
    });
  };
  v4f acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto use = [&](int u, int s) {
    const int b0 = (wave + GEMV_WAVES * s) * BPS;
    if (b0 < nb) {
      const v4u w = transpose_rows(wr[u]);
      v4f d[4];
      static_for<0, 4>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (j / T == 0 || b0 + j / T < nb)
          d[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, xr[u][j / T]), codes_to_h8(w[j]),
                                                        v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      });
      static_for<0, 4>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (j / T == 0 || b0 + j / T < nb) {
          const float sc = scale_value<ST>(sr[u][j]);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j % T][r] = fmaf(sc, d[j][r], acc[j % T][r]);
        }
      });
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) issue(u, u);
  int s = 0;
  for (int rd = 1; rd < rounds; ++rd) {
    static_for<0, U>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      vmwait<(U - 1) * L>();
      pin(wr[u]);
#pragma unroll
      for (int i = 0; i < BPS; ++i) pin(xr[u][i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) pin(sr[u][j]);
      use(u, s + u);
      issue(u, s + u + U);
    });
    s += U;
  }
  static_for<0, U>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    vmwait<(U - 1 - u) * L>();
    pin(wr[u]);
#pragma unroll
    for (int i = 0; i < BPS; ++i) pin(xr[u][i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) pin(sr[u][j]);
    use(u, s + u);
  });
#pragma unroll
  for (int t = 0; t < T; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  for (int t = wave; t < T; t += GEMV_WAVES) {
    const v4f y = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
    const int n = n0 + 16 * t + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * g + r;
      if (m < M && n < N) {
        if (part) {  // split K: this split's fp32 sums, scaled after the split-order sum
          part[((long)ky * M + m) * N + n] = y[r];
          continue;
        }
        const float v = y[r] * outscale;
        if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(Y)[(long)m * N + n] = f2h(v);
        else reinterpret_cast<float*>(Y)[(long)m * N + n] = v;
      }
    }
  }
}

// Y[e] = (P[0][e] + P[1][e] + ... + P[split-1][e]) * outscale over the
// split partials P[split][mn] (mn = M * N, rows of Y contiguous), summed in
// split order. VEC: four outputs per thread (mn % 4 == 0, Y aligned to four
// outputs; the partials always are, at 16-byte split strides).
template <int YT, bool VEC>
__global__ void __launch_bounds__(256)
gemv_mm_reduce_kernel(const float* __restrict__ P, void* __restrict__ Y, long mn, int split, float outscale) {
  const long e = ((long)blockIdx.x * 256 + threadIdx.x) * (VEC ? 4 : 1);
  if (e >= mn) return;
  if constexpr (VEC) {
    v4f t = *reinterpret_cast<const v4f*>(P + e);
    for (int s = 1; s < split; ++s) t += *reinterpret_cast<const v4f*>(P + (long)s * mn + e);
    t *= outscale;
    if constexpr (YT == Q4_DT_F16)
      *reinterpret_cast<ushort4*>(reinterpret_cast<uint16_t*>(Y) + e) =
          make_ushort4(f2h(t[0]), f2h(t[1]), f2h(t[2]), f2h(t[3]));
    else
      *reinterpret_cast<v4f*>(reinterpret_cast<float*>(Y) + e) = t;
  } else {
    float t = P[e];
    for (int s = 1; s < split; ++s) t += P[(long)s * mn + e];
    t *= outscale;
    if constexpr (YT == Q4_DT_F16) reinterpret_cast<uint16_t*>(Y)[e] = f2h(t);
    else reinterpret_cast<float*>(Y)[e] = t;
  }
}

// Several GEMVs over one x (same K and types) in one launch: segment i owns
// row groups [g_end[i-1], g_end[i]) of the grid; every segment covers whole
// panels.
struct GemvSeg {
  const uint4* wq;
  const void* sc;
  void* y;
  float outscale;
  int N;
  int g_end;
  int gq, gr;  // row partition of the segment's groups (group_rows)
};
struct GemvSegs {
  GemvSeg s[Q4_GEMV_MAX_BATCH];
  int count;
};

// The segment of row group g: its matrix, scales, output, scale factor,
// rows, and its first row group g0. Compile-time indices only (the argument
// block stays in the kernarg segment; a dynamic index would copy it to
// scratch).
struct SegSel {
  const uint4* wq;
  const void* sc;
  void* y;
  float os;
  int N, g0, gq, gr;
};
__device__ inline SegSel select_seg(const GemvSegs& segs, int g) {
  SegSel r{segs.s[0].wq, segs.s[0].sc, segs.s[0].y, segs.s[0].outscale, segs.s[0].N, 0, segs.s[0].gq, segs.s[0].gr};
#pragma unroll
  for (int t = 1; t < Q4_GEMV_MAX_BATCH; ++t) {
    if (t < segs.count && g >= segs.s[t - 1].g_end)
      r = SegSel{segs.s[t].wq, segs.s[t].sc, segs.s[t].y, segs.s[t].outscale, segs.s[t].N, segs.s[t - 1].g_end,
                 segs.s[t].gq, segs.s[t].gr};
  }
  return r;
}

// Row group of this wave in a launch of 256-thread halves (halves = 1 or
// 2 per workgroup, passed by the host: reading blockDim.x here is a vector
// load from the dispatch's implicit arguments that the first weight loads
// would wait behind). A wave lies in one half, so g is wave-uniform and the
// segment selection stays in scalar registers.
__device__ inline int wave_group(int halves) {
  const int half = threadIdx.x / GEMV_THREADS;
  return __builtin_amdgcn_readfirstlane(xcd_major(blockIdx.x, gridDim.x) * halves + half);
}

template <int R, int U, int XT, int ST, int YT>
__global__ void __launch_bounds__(2 * GEMV_THREADS)
gemv_batch_kernel(const void* __restrict__ xv, int nblk, const GemvSegs segs, int halves) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[2][GEMV_WAVES][R];
  const int half = threadIdx.x / GEMV_THREADS;
  const int g = wave_group(halves);
  const SegSel q = select_seg(segs, g);
  gemv_rows<R, U, XT, ST, YT>(xv, q.wq, q.sc, q.os, q.y, q.N, nblk, g - q.g0, q.gq, q.gr, 0, 1, 0, nullptr, nullptr,
                              smem + half * stage_words<R, XT>(nblk), red[half], 0);
}

// gemv_kernel and gemv_batch_kernel (split 1) with x formed from a NormIn
// in every workgroup (see nx_stage).
template <int R, int U, int ST, int YT>
__global__ void __launch_bounds__(2 * GEMV_THREADS)
gemv_nx_kernel(const NormIn nx, const uint4* __restrict__ wq, const void* __restrict__ scv, float outscale,
               void* __restrict__ yv, int N, int nblk, int gated, int halves, int gq, int gr) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[2][GEMV_WAVES][R];
  const int half = threadIdx.x / GEMV_THREADS;
  const int g = wave_group(halves);
  gemv_rows<R, U, Q4_DT_F16, ST, YT, true>(nullptr, wq, scv, outscale, yv, N, nblk, g, gq, gr, 0, 1, 0, nullptr,
                                           nullptr, smem + half * stage_words<R, Q4_DT_F16>(nblk), red[half], gated,
                                           nx);
}
template <int R, int U, int ST, int YT>
__global__ void __launch_bounds__(2 * GEMV_THREADS)
gemv_batch_nx_kernel(const NormIn nx, int nblk, const GemvSegs segs, int halves) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  __shared__ float red[2][GEMV_WAVES][R];
  const int half = threadIdx.x / GEMV_THREADS;
  const int g = wave_group(halves);
  const SegSel q = select_seg(segs, g);
  gemv_rows<R, U, Q4_DT_F16, ST, YT, true>(nullptr, q.wq, q.sc, q.os, q.y, q.N, nblk, g - q.g0, q.gq, q.gr, 0, 1, 0,
                                           nullptr, nullptr, smem + half * stage_words<R, Q4_DT_F16>(nblk), red[half],
                                           0, nx);
}

typedef void (*gemv_fn)(const void*, const uint4*, const void*, float, void*, int, int, int, float*, uint32_t*, int, int,
                        int);
typedef void (*gemv_batch_fn)(const void*, int, const GemvSegs, int);
struct GemvFns {
  gemv_fn one;
  gemv_batch_fn many;
};

template <int R, int U, int XT, int ST>
static GemvFns pick_y(int yt) {
  if (yt == Q4_DT_F16) return {gemv_kernel<R, U, XT, ST, Q4_DT_F16>, gemv_batch_kernel<R, U, XT, ST, Q4_DT_F16>};
  return {gemv_kernel<R, U, XT, ST, Q4_DT_F32>, gemv_batch_kernel<R, U, XT, ST, Q4_DT_F32>};
}
template <int R, int U, int XT>
static GemvFns pick_s(int st, int yt) {
  return st == Q4_SCALE_E4M3 ? pick_y<R, U, XT, Q4_SCALE_E4M3>(yt) : pick_y<R, U, XT, Q4_SCALE_F16>(yt);
}
template <int R, int U>
static GemvFns pick_x(int xt, int st, int yt) {
  return xt == Q4_DT_F16 ? pick_s<R, U, Q4_DT_F16>(st, yt) : pick_s<R, U, Q4_DT_F32>(st, yt);
}
template <int R>
static GemvFns pick_u(int U, int xt, int st, int yt) {
  return U == 4 ? pick_x<R, 4>(xt, st, yt) : pick_x<R, 8>(xt, st, yt);
}
static GemvFns pick(int R, int U, int xt, int st, int yt) {
  switch (R) {
    case 64: return pick_u<64>(U, xt, st, yt);
    case 32: return pick_u<32>(U, xt, st, yt);
    case 16: return pick_u<16>(U, xt, st, yt);
    default: return pick_u<8>(U, xt, st, yt);
  }
}

typedef void (*gemv_nx_fn)(const NormIn, const uint4*, const void*, float, void*, int, int, int, int, int, int);
typedef void (*gemv_batch_nx_fn)(const NormIn, int, const GemvSegs, int);
struct GemvNxFns {
  gemv_nx_fn one;
  gemv_batch_nx_fn many;
};
template <int R, int U, int ST>
static GemvNxFns pick_nx_y(int yt) {
  if (yt == Q4_DT_F16) return {gemv_nx_kernel<R, U, ST, Q4_DT_F16>, gemv_batch_nx_kernel<R, U, ST, Q4_DT_F16>};
  return {gemv_nx_kernel<R, U, ST, Q4_DT_F32>, gemv_batch_nx_kernel<R, U, ST, Q4_DT_F32>};
}
template <int R, int U>
static GemvNxFns pick_nx_s(int st, int yt) {
  return st == Q4_SCALE_E4M3 ? pick_nx_y<R, U, Q4_SCALE_E4M3>(yt) : pick_nx_y<R, U, Q4_SCALE_F16>(yt);
}
template <int R>
static GemvNxFns pick_nx_u(int U, int st, int yt) {
  return U == 4 ? pick_nx_s<R, 4>(st, yt) : pick_nx_s<R, 8>(st, yt);
}
static GemvNxFns pick_nx(int R, int U, int st, int yt) {
  switch (R) {
    case 64: return pick_nx_u<64>(U, st, yt);
    case 32: return pick_nx_u<32>(U, st, yt);
    case 16: return pick_nx_u<16>(U, st, yt);
    default: return pick_nx_u<8>(U, st, yt);
  }
}

typedef void (*gemv_multi_fn)(const uint16_t*, int, const uint4*, const void*, float, void*, int, int, int);
template <int R, int U, int ST, int YT>
static gemv_multi_fn pick_mv_v(int mv) {
  return mv == 2 ? gemv_multi_kernel<R, U, ST, YT, 2>
                 : mv == 4 ? gemv_multi_kernel<R, U, ST, YT, 4> : gemv_multi_kernel<R, U, ST, YT, 8>;
}
template <int R, int U>
static gemv_multi_fn pick_mv_sy(int mv, int st, int yt) {
  if (st == Q4_SCALE_E4M3)
    return yt == Q4_DT_F16 ? pick_mv_v<R, U, Q4_SCALE_E4M3, Q4_DT_F16>(mv) : pick_mv_v<R, U, Q4_SCALE_E4M3, Q4_DT_F32>(mv);
  return yt == Q4_DT_F16 ? pick_mv_v<R, U, Q4_SCALE_F16, Q4_DT_F16>(mv) : pick_mv_v<R, U, Q4_SCALE_F16, Q4_DT_F32>(mv);
}
template <int R>
static gemv_multi_fn pick_mv_u(int U, int mv, int st, int yt) {
  return U == 4 ? pick_mv_sy<R, 4>(mv, st, yt) : pick_mv_sy<R, 8>(mv, st, yt);
}
static gemv_multi_fn pick_mv(int R, int U, int mv, int st, int yt) {
  switch (R) {
    case 64: return pick_mv_u<64>(U, mv, st, yt);
    case 32: return pick_mv_u<32>(U, mv, st, yt);
    case 16: return pick_mv_u<16>(U, mv, st, yt);
    default: return pick_mv_u<8>(U, mv, st, yt);
  }
}

typedef void (*gemv_mm_fn)(const uint16_t*, int, const uint8_t*, const void*, float, void*, int, int, int, float*);
template <int T, int U>
static gemv_mm_fn pick_mm_sy(int st, int yt) {
  if (st == Q4_SCALE_E4M3)
    return yt == Q4_DT_F16 ? gemv_mm_kernel<T, U, Q4_SCALE_E4M3, Q4_DT_F16> : gemv_mm_kernel<T, U, Q4_SCALE_E4M3, Q4_DT_F32>;
  return yt == Q4_DT_F16 ? gemv_mm_kernel<T, U, Q4_SCALE_F16, Q4_DT_F16> : gemv_mm_kernel<T, U, Q4_SCALE_F16, Q4_DT_F32>;
}
// (T, U) pairs built: U = 4 or the deepest ring whose U (4/T + 5) loads
// per step stay under the 63 the wait count can express (T = 1: 6,
// T = 2: 8, T = 4: 10); the deeper one is the default.
static gemv_mm_fn pick_mm(int T, bool deep, int st, int yt) {
  switch (T) {
    case 4: return deep ? pick_mm_sy<4, 10>(st, yt) : pick_mm_sy<4, 4>(st, yt);
    case 2: return deep ? pick_mm_sy<2, 8>(st, yt) : pick_mm_sy<2, 4>(st, yt);
    default: return deep ? pick_mm_sy<1, 6>(st, yt) : pick_mm_sy<1, 4>(st, yt);
  }
}
// Row tiles of 16 per workgroup for NP padded rows: the largest T of 4, 2, 1
// that still gives GEMV_MIN_WGS workgroups (about one per CU): the x slices
// each wave reads are shared by T tiles. The Q4_TUNE_GEMV_MM_TILES and
// Q4_TUNE_GEMV_MM_DEEP overrides (q4_tune_set) replace the plan in tests and sweeps.
static int mm_tiles(int NP) {
  int T = 1;
  for (int c : {4, 2})
    if (NP / (16 * c) >= GEMV_MIN_WGS) { T = c; break; }
  const int v = tune_value(Q4_TUNE_GEMV_MM_TILES);
  if (v == 1 || v == 2 || v == 4) T = v;
  return T;
}
// K splits for the small-M GEMV at T = 4 tiles: 1 where NP / 64 row groups
// already give GEMV_MIN_WGS workgroups, else enough splits to reach it, each
// split at least GEMV_MM_MIN_SPLIT_BLOCKS blocks (8 steps per wave).
// The Q4_TUNE_GEMV_MM_SPLIT override (q4_tune_set) replaces it in tests and sweeps.
constexpr int GEMV_MM_MIN_SPLIT_BLOCKS = 32;
static int mm_split(int NP, int nblk) {
  const int groups = NP / 64;
  int s = groups >= GEMV_MIN_WGS ? 1 : (GEMV_MIN_WGS + groups - 1) / groups;
  s = std::min(s, std::max(1, nblk / GEMV_MM_MIN_SPLIT_BLOCKS));
  const int v = tune_value(Q4_TUNE_GEMV_MM_SPLIT);
  if (v >= 1 && v <= 64) s = v;
  const int span = (nblk + s - 1) / s;
  return (nblk + span - 1) / span;  // no empty split
}
static bool mm_deep() { return tune_value(Q4_TUNE_GEMV_MM_DEEP) > 0; }

// Rows per workgroup R for NP padded rows: the largest R of 64, 32, 16 that
// gives GEMV_TARGET_WGS workgroups (about two per CU), else the largest R
// that gives GEMV_MIN_WGS (about one per CU), else 8. Measured on MI355X over
// the decode shapes: 64 rows for gate_up and lm_head, 32 for 15360 rows, 16
// for the batched q/k/v and for the 3840-row o and down (240 workgroups with
// 8 units in flight beat 480 with 4: each workgroup stages the whole x, 30 KB
// for down). The Q4_TUNE_GEMV_ROWS override (q4_tune_set) replaces R in tests and sweeps.
static int rows_per_group(int NP) {
  int R = 0;
  for (int c : {64, 32, 16})
    if (NP / c >= GEMV_TARGET_WGS) { R = c; break; }
  if (R == 0)
    for (int c : {64, 32, 16, 8})
      if (NP / c >= GEMV_MIN_WGS) { R = c; break; }
  if (R == 0) R = 8;
  const int v = tune_value(Q4_TUNE_GEMV_ROWS);
  if (v == 8 || v == 16 || v == 32 || v == 64) R = v;
  return R;
}

// Rows per workgroup of a fused-norm launch: every workgroup forms the whole
// x from the normadd operands (16 bytes per element, 61 KB at K = 3840, read
// from L2), so the launch takes the fewest workgroups that still give about
// one per CU: the largest R with NP / R >= GEMV_MIN_WGS. Measured in the
// decode token's graph (the q/k/v batch, 8192 rows: 256 groups of 32 rows
// instead of 512 of 16): token 2.253 -> 2.216 ms; gate/up (30720 rows)
// keeps 64 either way. The Q4_TUNE_GEMV_ROWS override replaces R here too.
static int rows_per_group_nx(int NP) {
  const int v = tune_value(Q4_TUNE_GEMV_ROWS);
  if (v == 8 || v == 16 || v == 32 || v == 64) return v;
  for (int c : {64, 32, 16})
    if (NP / c >= GEMV_MIN_WGS) return c;
  return 8;
}

// Units in flight per lane for a grid of wgs workgroups with nb blocks each:
// 8 while the whole grid keeps at most GEMV_INFLIGHT_UNITS in flight (8 MB
// of weights, what HBM needs at ~1.1 us of loaded latency), else 4; 4 when
// a lane has at most 4 blocks. Measured on MI355X: the best of 4/8/16 for
// every decode shape follows this rule (more in flight only queues).
// The Q4_TUNE_GEMV_UNITS override (q4_tune_set) replaces it in tests and sweeps.
static int units_in_flight(int nb, int R, long wgs) {
  const int v = tune_value(Q4_TUNE_GEMV_UNITS);
  if (v == 4 || v == 8) return v;
  const int per_lane = ceil_div(nb, (64 / R) * GEMV_WAVES);
  return per_lane > 4 && wgs * GEMV_THREADS * 8 <= GEMV_INFLIGHT_UNITS ? 8 : 4;
}

// Row groups per workgroup: 2 (a 512-thread workgroup, see gemv_kernel) for
// the batched launch without a fused norm (`paired`) when its grid is
// unsplit, has an even number of groups that still give one workgroup per
// CU after pairing (>= 2 GEMV_MIN_WGS groups) and its two staging areas fit
// 64 KB of LDS; else 1. Measured on MI355X in the graph of a decode token:
// pairing the q/k/v batch saves 0.14 us per launch (5.80 -> 5.66 us), while
// the single and fused-norm launches run faster unpaired between their
// neighbours (the 48-layer GEMV set 1.611 -> 1.595 ms, the fused token
// 2.362 -> 2.293 ms). The Q4_TUNE_GEMV_PAIR override forces 1 (0) or pairs
// every unsplit even grid (1), for tests and tuning sweeps.
static int pair_groups(int groups, int split, size_t lds, bool paired) {
  const bool can = split == 1 && groups % 2 == 0 && 2 * lds <= 64 * 1024;
  const int f = tune_value(Q4_TUNE_GEMV_PAIR);
  if (f >= 0) return f != 0 && can ? 2 : 1;
  return paired && can && groups >= 2 * GEMV_MIN_WGS ? 2 : 1;
}

// LDS bytes of x per block, and of the staging area for nb blocks and R
// rows per workgroup: each wave's local blocks in whole 1 KB direct-load
// rows, then (fp16 x) each wave's fp32 block sums.
static int x_block_bytes(int x_dtype) { return x_dtype == Q4_DT_F16 ? 64 : 128; }
static size_t x_stage_lds(int nb, int x_dtype, int R) {
  const int SW = 64 / R, S = SW * GEMV_WAVES;
  const long nbw = (long)ceil_div(nb, S) * SW;
  const size_t per_wave = (size_t)ceil_div(nbw * x_block_bytes(x_dtype), 1024) * 1024;
  return GEMV_WAVES * per_wave + (x_dtype == Q4_DT_F16 ? (size_t)GEMV_WAVES * nbw * sizeof(float) : 0);
}


struct GemvPlan {
  int R, U, split, nb_max;
  size_t lds, ws;
};

// Balanced unsplit grids (the Q4_TUNE_GEMV_BAL override m, tuning): 256 m row groups (or
// more, until a group fits 64 rows) spread the rows evenly over all CUs, in
// units of `unit` rows (2: gate/up pairs); R is the smallest of 8..64 that
// holds the largest group. Returns 0 when not selected.
static int balance_mult() {
  const int m = tune_value(Q4_TUNE_GEMV_BAL);
  return m > 0 && m <= 64 ? m : 0;
}
static int pow2_rows(int rows) {
  int R = 8;
  while (R < rows) R <<= 1;
  return R;
}
static bool balanced_groups(int N, int unit, int& R, int& groups) {
  const int m = balance_mult();
  if (!m) return false;
  const long Nu = N / unit;
  long G = 256L * m;
  while (G < Nu && unit * ceil_div(Nu, G) > 64) G += 256;
  if (G > Nu) G = Nu;
  groups = (int)G;
  R = pow2_rows(unit * ceil_div(Nu, G));
  return true;
}

static GemvPlan plan(int N, int K, int split_req, int x_dtype) {
  const int NP = pad_rows(N), nblk = K / BLK;
  const int R = rows_per_group(NP);
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
  const int max_nb = GEMV_LDS_MAX / x_block_bytes(x_dtype);
  if (s < ceil_div(nblk, max_nb)) s = ceil_div(nblk, max_nb);
  if (s > nblk) s = nblk;
  GemvPlan p;
  p.R = R;
  p.split = s;
  p.nb_max = ceil_div(nblk, s);
  p.U = units_in_flight(p.nb_max, R, (long)wgs * s);
  p.lds = x_stage_lds(p.nb_max, x_dtype, R);
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

// Checks of a NormIn over K elements: operands present and 16-byte aligned,
// K within what one thread's loads cover, h_out apart from every operand.
static int nx_check(const NormIn& nx, int K) {
  Q4_ARG(nx.a && nx.w && nx.h && nx.h_out && nx.w2, "null norm operand");
  Q4_ARG(K <= NX_MAX_K, "a GEMV with a fused norm input takes K <= %d (got %d)", NX_MAX_K, K);
  const void* ops[5] = {nx.a, nx.w, nx.h, nx.h_out, nx.w2};
  for (const void* p : ops) Q4_ARG(((uintptr_t)p & 15) == 0, "norm operands must be 16-byte aligned");
  const uintptr_t o = (uintptr_t)nx.h_out, n = (uintptr_t)K * sizeof(float);
  for (int i = 0; i < 5; ++i) {
    if (i == 3) continue;
    const uintptr_t p = (uintptr_t)ops[i];
    Q4_ARG(o + n <= p || p + n <= o, "h_out must not overlap h, a, w or w2");
  }
  return Q4_OK;
}

// An output y of y_bytes of a norm-fused GEMV apart from every norm operand
// and h_out: workgroups that finish early write y while others still read
// a and h, and workgroup 0 writes h_out.
static int nx_check_y(const NormIn& nx, int K, const void* y, size_t y_bytes) {
  const void* ops[5] = {nx.a, nx.w, nx.h, nx.h_out, nx.w2};
  const uintptr_t yo = (uintptr_t)y, n = (uintptr_t)K * sizeof(float);
  for (const void* q : ops) {
    const uintptr_t p = (uintptr_t)q;
    Q4_ARG(yo + y_bytes <= p || p + n <= yo, "y must not overlap a, w, h, h_out or w2 of a fused norm input");
  }
  return Q4_OK;
}

// x (x_dtype) or, with nx, x formed from the NormIn (split 1).
// Argument checks of a GEMV whose x comes from memory (no fused norm), in
// the order gemv_launch applies them: callers that queue work of their own
// before the launch (q4_gemv_noalloc's ticket fill) run them first, so a
// rejected call enqueues nothing.
static int gemv_plain_args(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt,
                           const void* y, int y_dtype, int N, int K) {
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad GEMV shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  Q4_ARG(x && wq && scales && y, "null pointer");
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x dtype %d", x_dtype);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
  Q4_ARG(scale_fmt == Q4_SCALE_F16 || scale_fmt == Q4_SCALE_E4M3, "bad scale format %d", scale_fmt);
  Q4_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)x & 15) == 0, "wq and x must be 16-byte aligned");
  Q4_ARG(N <= (1 << 30) && (long)K <= (1L << 24), "GEMV too large");
  return Q4_OK;
}

static int gemv_launch(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv,
                       void* y, int y_dtype, int N, int K, int split, void* ws, size_t ws_size, void* stream,
                       int gated, const NormIn* nx = nullptr) {
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad GEMV shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  Q4_ARG((x || nx) && wq && scales && y, "null pointer");
  if (nx) {
    x_dtype = Q4_DT_F16;
    split = 1;
    if (int e = nx_check(*nx, K)) return e;
    Q4_ARG(N > 0 && (y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16), "bad GEMV rows N=%d or y dtype %d", N, y_dtype);
    const size_t rows = gated ? (size_t)N / 2 : (size_t)N;
    if (int e = nx_check_y(*nx, K, y, rows * (y_dtype == Q4_DT_F16 ? 2 : 4))) return e;
  }
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x dtype %d", x_dtype);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
  Q4_ARG(scale_fmt == Q4_SCALE_F16 || scale_fmt == Q4_SCALE_E4M3, "bad scale format %d", scale_fmt);
  Q4_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)x & 15) == 0, "wq and x must be 16-byte aligned");
  Q4_ARG(N <= (1 << 30) && (long)K <= (1L << 24), "GEMV too large");
  GemvPlan pl = plan(N, K, split, x_dtype);
  if (nx && pl.split == 1) {
    pl.R = rows_per_group_nx(pad_rows(N));
    pl.U = units_in_flight(pl.nb_max, pl.R, pad_rows(N) / pl.R);
    pl.lds = x_stage_lds(pl.nb_max, x_dtype, pl.R);
  }
  Q4_ARG(pl.ws == 0 || (ws && ws_size >= pl.ws), "GEMV N=%d K=%d split=%d needs a %zu-byte workspace (got %zu)", N,
         K, pl.split, pl.ws, ws ? ws_size : (size_t)0);
  // row groups: NP / R of the plan, at most one per row (pair, when gated)
  const int unit = gated ? 2 : 1;
  int groups = pad_rows(N) / pl.R;
  if (groups > N / unit) groups = N / unit;
  if (pl.split == 1 && balanced_groups(N, unit, pl.R, groups)) {
    pl.U = units_in_flight(pl.nb_max, pl.R, groups);
    pl.lds = x_stage_lds(pl.nb_max, x_dtype, pl.R);
  }
  // A fused-norm launch forms x (normadd + norm) before its first dot
  // product; with 64-row groups its lanes keep 8 units in flight through
  // that prologue. Measured in the decode token's graph (gate/up, 480 groups
  // of 64 rows): token 2.298 -> 2.282 ms, where the plain gate/up GEMV of the
  // same shape is faster with 4 (GEMV set 1.600 against 1.630 ms with 8).
  if (nx && pl.R == 64 && tune_value(Q4_TUNE_GEMV_UNITS) < 0 && ceil_div(pl.nb_max, GEMV_WAVES) > 4) pl.U = 8;
  Q4_ARG(pl.ws == 0 || groups <= GEMV_MAX_TICKETS, "split-K GEMV supports at most %d row groups", GEMV_MAX_TICKETS);
  uint32_t* cnt = pl.ws ? reinterpret_cast<uint32_t*>(ws) : nullptr;
  float* part = pl.ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + GEMV_TICKET_BYTES) : nullptr;
  const float outscale = scale_fmt == Q4_SCALE_E4M3 ? inv * 256.0f : 1.0f;
  const int hv = pair_groups(groups, pl.split, pl.lds, false);
  int gq = 0, gr = 0;
  group_split(N, groups, gated, gq, gr);
  if (nx) {
    Q4_ARG(pl.split == 1, "internal: fused-norm GEMV planned with split %d", pl.split);
    hipLaunchKernelGGL(pick_nx(pl.R, pl.U, scale_fmt, y_dtype).one, dim3(groups / hv), dim3(GEMV_THREADS * hv),
                       pl.lds * hv, as_stream(stream), *nx, reinterpret_cast<const uint4*>(wq), scales, outscale, y, N,
                       K / BLK, gated, hv, gq, gr);
    Q4_LAUNCHED("gemv_normadd");
    return Q4_OK;
  }
  gemv_fn fn = pick(pl.R, pl.U, x_dtype, scale_fmt, y_dtype).one;
  hipLaunchKernelGGL(fn, dim3(groups / hv, pl.split), dim3(GEMV_THREADS * hv), pl.lds * hv, as_stream(stream), x,
                     reinterpret_cast<const uint4*>(wq), scales, outscale, y, N, K / BLK, pl.split, part, cnt, gated, gq,
                     gr);
  Q4_LAUNCHED("gemv");
  return Q4_OK;
}

int q4_gemv(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv, void* y,
            int y_dtype, int N, int K, int split, void* ws, size_t ws_size, void* stream) {
  clear_error();
  return gemv_launch(x, x_dtype, wq, scales, scale_fmt, inv, y, y_dtype, N, K, split, ws, ws_size, stream, 0);
}

int q4_gemv_gated(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv,
                  void* act, int act_dtype, int N, int K, int split, void* ws, size_t ws_size, void* stream) {
  clear_error();
  Q4_ARG(N > 0 && N % 2 == 0, "gated GEMV needs an even row count (interleaved gate/up rows), got N=%d", N);
  return gemv_launch(x, x_dtype, wq, scales, scale_fmt, inv, act, act_dtype, N, K, split, ws, ws_size, stream, 1);
}

int q4_gemv_f16s(const void* x, int x_dtype, const uint32_t* wq, const uint16_t* sc16, void* y, int y_dtype, int N,
                 int K, int split, void* ws, size_t ws_size, void* stream) {
  return q4_gemv(x, x_dtype, wq, sc16, Q4_SCALE_F16, 1.0f, y, y_dtype, N, K, split, ws, ws_size, stream);
}

int q4_gemv_e4m3s(const void* x, int x_dtype, const uint32_t* wq, const uint8_t* sc8, float inv, void* y, int y_dtype,
                  int N, int K, int split, void* ws, size_t ws_size, void* stream) {
  return q4_gemv(x, x_dtype, wq, sc8, Q4_SCALE_E4M3, inv, y, y_dtype, N, K, split, ws, ws_size, stream);
}

// The MFMA small-M GEMV: unsplit (ws == nullptr) as one launch of T tiles,
// else T = 4 and `split` K ranges into fp32 partials in ws, then the
// split-order reduce.
static int gemv_mm_launch(const void* x, int M, const uint32_t* wq, const void* scales, int scale_fmt,
                          float outscale, void* y, int y_dtype, int N, int nblk, int split, float* ws,
                          hipStream_t st) {
  const int NP = pad_rows(N);
  if (split <= 1) {
    const int T = mm_tiles(NP);
    hipLaunchKernelGGL(pick_mm(T, mm_deep(), scale_fmt, y_dtype), dim3(NP / (16 * T)), dim3(GEMV_THREADS), 0, st,
                       reinterpret_cast<const uint16_t*>(x), M, reinterpret_cast<const uint8_t*>(wq), scales,
                       outscale, y, N, nblk, nblk, nullptr);
    Q4_LAUNCHED("gemv_mm");
    return Q4_OK;
  }
  const int span = (nblk + split - 1) / split;
  hipLaunchKernelGGL(pick_mm(4, mm_deep(), scale_fmt, y_dtype), dim3(NP / 64, split), dim3(GEMV_THREADS), 0, st,
                     reinterpret_cast<const uint16_t*>(x), M, reinterpret_cast<const uint8_t*>(wq), scales, outscale,
                     y, N, nblk, span, ws);
  Q4_LAUNCHED("gemv_mm split");
  const long mn = (long)M * N;
  const size_t ysz = y_dtype == Q4_DT_F16 ? 2 : 4;
  const bool vec = mn % 4 == 0 && (uintptr_t)y % (4 * ysz) == 0;
  const long per = vec ? 4 : 1;
  const dim3 grid((unsigned)((mn + 256 * per - 1) / (256 * per)));
  typedef void (*reduce_fn)(const float*, void*, long, int, float);
  const reduce_fn f16v[2] = {gemv_mm_reduce_kernel<Q4_DT_F16, false>, gemv_mm_reduce_kernel<Q4_DT_F16, true>};
  const reduce_fn f32v[2] = {gemv_mm_reduce_kernel<Q4_DT_F32, false>, gemv_mm_reduce_kernel<Q4_DT_F32, true>};
  const reduce_fn fn = y_dtype == Q4_DT_F16 ? f16v[vec] : f32v[vec];
  hipLaunchKernelGGL(fn, grid, dim3(256), 0, st, ws, y, mn, split, outscale);
  Q4_LAUNCHED("gemv_mm reduce");
  return Q4_OK;
}

static int gemv_multi_check(const void* x, int M, const uint32_t* wq, const void* scales, int scale_fmt, void* y,
                            int y_dtype, int N, int K) {
  Q4_ARG(M >= 1 && M <= Q4_GEMV_MAX_VECTORS, "multi-vector GEMV takes 1..%d vectors (got M=%d)", Q4_GEMV_MAX_VECTORS,
         M);
  Q4_ARG(N > 0 && K > 0 && K % BLK == 0, "bad GEMV shape N=%d K=%d (K must be a positive multiple of 32)", N, K);
  Q4_ARG(x && wq && scales && y, "null pointer");
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
  Q4_ARG(scale_fmt == Q4_SCALE_F16 || scale_fmt == Q4_SCALE_E4M3, "bad scale format %d", scale_fmt);
  Q4_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)x & 15) == 0, "wq and x must be 16-byte aligned");
  Q4_ARG(N <= (1 << 30) && (long)K <= (1L << 24), "GEMV too large");
  return Q4_OK;
}

size_t q4_gemv_multi_workspace_bytes(int M, int N, int K) {
  if (M < 1 || M > Q4_GEMV_MAX_VECTORS || N <= 0 || K <= 0 || K % BLK || N > (1 << 30) || (long)K > (1L << 24))
    return 0;
  const int split = mm_split(pad_rows(N), K / BLK);
  return split > 1 ? (size_t)split * M * N * sizeof(float) : 0;
}

int q4_gemv_multi_ws(const void* x, int M, const uint32_t* wq, const void* scales, int scale_fmt, float inv, void* y,
                     int y_dtype, int N, int K, void* ws, size_t ws_size, void* stream) {
  clear_error();
  if (const int rc = gemv_multi_check(x, M, wq, scales, scale_fmt, y, y_dtype, N, K)) return rc;
  Q4_ARG(((uintptr_t)ws & 15) == 0, "workspace must be 16-byte aligned");
  const int nblk = K / BLK;
  const float outscale = scale_fmt == Q4_SCALE_E4M3 ? inv * 256.0f : 1.0f;
  const size_t need = q4_gemv_multi_workspace_bytes(M, N, K);
  const bool split = need && ws && ws_size >= need;
  return gemv_mm_launch(x, M, wq, scales, scale_fmt, outscale, y, y_dtype, N, nblk,
                        split ? mm_split(pad_rows(N), nblk) : 1, split ? reinterpret_cast<float*>(ws) : nullptr,
                        as_stream(stream));
}

int q4_gemv_multi(const void* x, int M, const uint32_t* wq, const void* scales, int scale_fmt, float inv, void* y,
                  int y_dtype, int N, int K, int exact, void* stream) {
  clear_error();
  if (const int rc = gemv_multi_check(x, M, wq, scales, scale_fmt, y, y_dtype, N, K)) return rc;
  const int NP = pad_rows(N), nblk = K / BLK;
  const float outscale = scale_fmt == Q4_SCALE_E4M3 ? inv * 256.0f : 1.0f;
  if (!exact)
    return gemv_mm_launch(x, M, wq, scales, scale_fmt, outscale, y, y_dtype, N, nblk, 1, nullptr, as_stream(stream));
  const int R = rows_per_group(NP), groups = NP / R;
  const int U = units_in_flight(nblk, R, groups);
  const size_t ysz = y_dtype == Q4_DT_F16 ? 2 : 4;
  // launches of up to 8 vectors, fewer where their x slices do not fit the LDS
  const size_t per_vec = x_stage_lds(nblk, Q4_DT_F16, R);
  int chunk = GEMV_MV_MAX;
  while (chunk > 2 && (size_t)chunk * per_vec > GEMV_MV_LDS_MAX) chunk >>= 1;
  Q4_ARG((size_t)2 * per_vec <= GEMV_MV_LDS_MAX, "multi-vector GEMV with K=%d needs %zu bytes of LDS (max %zu)", K,
         2 * per_vec, GEMV_MV_LDS_MAX);
  for (int m0 = 0; m0 < M; m0 += chunk) {
    const int m = M - m0 < chunk ? M - m0 : chunk;
    const int mv = m <= 2 ? 2 : m <= 4 ? 4 : 8;
    hipLaunchKernelGGL(pick_mv(R, U, mv, scale_fmt, y_dtype), dim3(groups), dim3(GEMV_THREADS), mv * per_vec,
                       as_stream(stream), reinterpret_cast<const uint16_t*>(x) + (long)m0 * K, m,
                       reinterpret_cast<const uint4*>(wq), scales, outscale,
                       reinterpret_cast<char*>(y) + (long)m0 * N * ysz, N, N, nblk);
    Q4_LAUNCHED("gemv_multi");
  }
  return Q4_OK;
}

}  // extern "C"

// x (x_dtype) or, with nx, x formed from the NormIn.
static int gemv_batch_launch(const void* x, int x_dtype, int K, int scale_fmt, int y_dtype, int count,
                             const uint32_t* const* wq, const void* const* scales, const float* inv, void* const* y,
                             const int* N, void* stream, const NormIn* nx) {
  Q4_ARG(count >= 1 && count <= Q4_GEMV_MAX_BATCH, "batch of %d GEMVs (1..%d)", count, Q4_GEMV_MAX_BATCH);
  Q4_ARG(wq && scales && y && N && (x || nx), "null pointer");
  if (nx) {
    x_dtype = Q4_DT_F16;
    Q4_ARG(K > 0 && K % BLK == 0, "bad GEMV K=%d (a positive multiple of 32)", K);
    if (int e = nx_check(*nx, K)) return e;
  }
  Q4_ARG(K > 0 && K % BLK == 0 && (long)K <= (1L << 24), "bad GEMV K=%d (a positive multiple of 32)", K);
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x dtype %d", x_dtype);
  Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
  Q4_ARG(scale_fmt == Q4_SCALE_F16 || scale_fmt == Q4_SCALE_E4M3, "bad scale format %d", scale_fmt);
  Q4_ARG(((uintptr_t)x & 15) == 0, "x must be 16-byte aligned");
  const int nblk = K / BLK;
  Q4_ARG((long)nblk * x_block_bytes(x_dtype) <= GEMV_LDS_MAX, "batched GEMV needs K <= %d for this x dtype (got %d)",
         GEMV_LDS_MAX / x_block_bytes(x_dtype) * BLK, K);
  long NP = 0;
  for (int i = 0; i < count; ++i) {
    Q4_ARG(wq[i] && scales[i] && y[i], "null pointer in batch entry %d", i);
    Q4_ARG(N[i] > 0 && N[i] <= (1 << 30), "bad N=%d in batch entry %d", N[i], i);
    Q4_ARG(((uintptr_t)wq[i] & 15) == 0, "wq of batch entry %d must be 16-byte aligned", i);
    NP += pad_rows(N[i]);
  }
  Q4_ARG(NP <= (1L << 30), "batched GEMV too large");
  if (nx) {
    Q4_ARG(y_dtype == Q4_DT_F32 || y_dtype == Q4_DT_F16, "bad y dtype %d", y_dtype);
    for (int i = 0; i < count; ++i)
      if (int e = nx_check_y(*nx, K, y[i], (size_t)N[i] * (y_dtype == Q4_DT_F16 ? 2 : 4))) return e;
  }
  int R = nx ? rows_per_group_nx((int)NP) : rows_per_group((int)NP);
  // row groups per matrix: NP_i / R, or with a balanced plan 256 m groups
  // shared out in proportion to the rows (same rows per group everywhere)
  int gm[Q4_GEMV_MAX_BATCH];
  int Rb = 0, Gb = 0;
  if (balanced_groups((int)NP, 1, Rb, Gb)) {
    R = 8;
    for (int i = 0; i < count; ++i) {
      gm[i] = (int)(((long)Gb * N[i] + NP / 2) / NP);
      if (gm[i] < 1) gm[i] = 1;
      if (gm[i] > N[i]) gm[i] = N[i];
      while (ceil_div(N[i], gm[i]) > 64) ++gm[i];
      R = max(R, pow2_rows(ceil_div(N[i], gm[i])));
    }
  } else {
    for (int i = 0; i < count; ++i) gm[i] = min(pad_rows(N[i]) / R, N[i]);
  }
  GemvSegs segs;
  memset(&segs, 0, sizeof(segs));
  segs.count = count;
  int groups = 0;
  for (int i = 0; i < count; ++i) {
    groups += gm[i];
    segs.s[i].wq = reinterpret_cast<const uint4*>(wq[i]);
    segs.s[i].sc = scales[i];
    segs.s[i].y = y[i];
    segs.s[i].outscale = scale_fmt == Q4_SCALE_E4M3 ? (inv ? inv[i] : 1.0f) * 256.0f : 1.0f;
    segs.s[i].N = N[i];
    segs.s[i].g_end = groups;
    group_split(N[i], gm[i], 0, segs.s[i].gq, segs.s[i].gr);
  }
  const int U = units_in_flight(nblk, R, groups);
  const size_t lds = x_stage_lds(nblk, x_dtype, R);
  const int hv = pair_groups(groups, 1, lds, nx == nullptr);
  if (nx) {
    hipLaunchKernelGGL(pick_nx(R, U, scale_fmt, y_dtype).many, dim3(groups / hv), dim3(GEMV_THREADS * hv), lds * hv,
                       as_stream(stream), *nx, nblk, segs, hv);
    Q4_LAUNCHED("gemv_batch_normadd");
    return Q4_OK;
  }
  gemv_batch_fn fn = pick(R, U, x_dtype, scale_fmt, y_dtype).many;
  hipLaunchKernelGGL(fn, dim3(groups / hv), dim3(GEMV_THREADS * hv), lds * hv,
                     as_stream(stream), x, nblk, segs, hv);
  Q4_LAUNCHED("gemv_batch");
  return Q4_OK;
}

extern "C" {

int q4_gemv_batch(const void* x, int x_dtype, int K, int scale_fmt, int y_dtype, int count,
                  const uint32_t* const* wq, const void* const* scales, const float* inv, void* const* y,
                  const int* N, void* stream) {
  clear_error();
  return gemv_batch_launch(x, x_dtype, K, scale_fmt, y_dtype, count, wq, scales, inv, y, N, stream, nullptr);
}

int q4_gemv_normadd(const float* a, const float* w, const float* h, float* h_out, float scale, const float* w2,
                    const uint32_t* wq, const void* scales, int scale_fmt, float inv, void* y, int y_dtype, int N,
                    int K, int gated, void* stream) {
  clear_error();
  Q4_ARG(!gated || (N > 0 && N % 2 == 0), "gated GEMV needs an even row count (interleaved gate/up rows), got N=%d",
         N);
  const NormIn nx{a, w, h, h_out, w2, scale == 0.0f ? 1.0f : scale};
  return gemv_launch(nullptr, Q4_DT_F16, wq, scales, scale_fmt, inv, y, y_dtype, N, K, 1, nullptr, 0, stream,
                     gated ? 1 : 0, &nx);
}

int q4_gemv_batch_normadd(const float* a, const float* w, const float* h, float* h_out, float scale, const float* w2,
                          int K, int scale_fmt, int y_dtype, int count, const uint32_t* const* wq,
                          const void* const* scales, const float* inv, void* const* y, const int* N, void* stream) {
  clear_error();
  const NormIn nx{a, w, h, h_out, w2, scale == 0.0f ? 1.0f : scale};
  return gemv_batch_launch(nullptr, Q4_DT_F16, K, scale_fmt, y_dtype, count, wq, scales, inv, y, N, stream, &nx);
}

}  // extern "C"

// ---- allocation-free split-K GEMV ------------------------------------------
// q4_gemv_noalloc runs q4_gemv's kernels with the split-K workspace (tickets,
// then fp32 partials) in this file-scope device array instead of a caller
// buffer: one copy per GPU, held until the process ends. Every call on a GPU
// shares it, so calls that overlap on one GPU (other streams, other threads)
// race; calls issued in order on one stream do not.
constexpr size_t GEMV_SCRATCH_BYTES = 2u << 20;
static __device__ __align__(256) uint8_t scratch[GEMV_SCRATCH_BYTES];

namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES];

// Device address of this GPU's scratch array (the current device's), resolved
// once per device with hipGetSymbolAddress: the host-side name of a
// __device__ array is a stand-in, not a device address.
int scratch_addr(void** out) {
  int dev = 0;
  Q4_HIP(hipGetDevice(&dev));
  Q4_ARG(dev >= 0 && dev < SCRATCH_MAX_DEVICES, "device %d out of range for the GEMV scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    Q4_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    Q4_ARG(p != nullptr, "hipGetSymbolAddress returned no address for the GEMV scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return Q4_OK;
}
}  // namespace

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

extern "C" {

size_t q4_gemv_scratch_bytes(void) { return GEMV_SCRATCH_BYTES; }

int q4_gemv_noalloc(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv,
                    void* y, int y_dtype, int N, int K, int split, void* stream) {
  clear_error();
  if (int e = gemv_plain_args(x, x_dtype, wq, scales, scale_fmt, y, y_dtype, N, K)) return e;
  const GemvPlan pl = plan(N, K, split, x_dtype);
  if (pl.ws == 0)   // unsplit plan: no workspace at all
    return gemv_launch(x, x_dtype, wq, scales, scale_fmt, inv, y, y_dtype, N, K, split, nullptr, 0, stream, 0);
  Q4_ARG(pl.ws <= GEMV_SCRATCH_BYTES,
         "q4_gemv_noalloc: GEMV N=%d K=%d split=%d needs %zu bytes of split-K scratch, more than its %zu", N, K,
         pl.split, pl.ws, GEMV_SCRATCH_BYTES);
  const int groups = pad_rows(N) / pl.R;
  Q4_ARG(groups <= GEMV_MAX_TICKETS, "split-K GEMV supports at most %d row groups", GEMV_MAX_TICKETS);
  void* ws = nullptr;
  if (int e = scratch_addr(&ws)) return e;
  // the tickets of this call's row groups start at zero (a fill kernel, not a
  // memset node, so the call can be captured in a graph)
  hipLaunchKernelGGL(zero_words_kernel, dim3(ceil_div(groups, 256)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<uint32_t*>(ws), groups);
  Q4_LAUNCHED("zero_words");
  return gemv_launch(x, x_dtype, wq, scales, scale_fmt, inv, y, y_dtype, N, K, split, ws, GEMV_SCRATCH_BYTES, stream,
                     0);
}

}  // extern "C"
