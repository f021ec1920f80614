// Prefill GEMMs on gfx950 MFMA, plus the per-row int8 activation quantizer.
//
//   W8A8 : C = A8 @ W8^T (int32, exact), Y = f16((f32(C) * sa[m]) * sw[n])
//          (vk/coopgemm_w8a8.comp)          v_mfma_i32_32x32x32_i8
//   W4A8 : as W8A8 with W8 = int8(clamp(rint((q-8) * ratio), +-127)) made
//          on the fly from the int4 codes (vk/coopgemm_w4a8.comp)
//   W4A16: Y = f16(X @ f16((q-8) * s)^T), fp32 accumulate
//          (vk/coopgemm_i4h.comp, which accumulates in f16; this one
//          accumulates in fp32)          v_mfma_f32_32x32x16_f16
//
// One kernel template serves all three: every k-step stages 64-byte rows of
// both operands in LDS (64 int8 or 32 f16 elements), so the LDS layout, the
// XOR swizzle and the MFMA fragment reads are shared; only the B-operand
// producer (byte copy, int4 -> f16 dequant, int4 -> int8 requant) and the
// MFMA/epilogue differ.
//
// Tiling: BM x BN macro tile per 256-thread workgroup (4 waves as 2 x 2),
// each wave a (BM/2) x (BN/2) block of 32x32 MFMA tiles
// (v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_f16: both take 16 operand
// bytes per lane, half the operand traffic per MAC of the 16x16 shapes);
// a 64-byte k-row is two MFMA k-slices. LDS double buffered with one
// barrier per k-step; the next k-step's global loads are in flight while
// the current one's MFMAs run. Workgroups are remapped so
// each XCD (8 per MI355X, own L2) works on a contiguous 1/8 of the grid
// ordered by weight panel, which keeps a weight panel's re-reads in one L2.
#include "q4mi_common.h"

namespace q4 {

enum { OP_W8A8 = 0, OP_W4A16 = 1, OP_W4A8 = 2 };
constexpr int GEMM_WAVES_EPI = 4;

struct GemmArgs {
  const void* A;        // int8 [M][K] or f16 [M][K]
  const void* B;        // int8 [N][K] (W8A8) or panel-64 int4 units
  const uint16_t* bsc;  // panel-64 fp16 scales (W4A16) or ratio (W4A8)
  const float* sa;      // [M]
  const void* sw;       // [N] f32 or f16
  int sw_f16;
  uint16_t* Y;          // f16 [M][N] (may be NULL for int paths if C given)
  int32_t* C;           // int32 [M][N] or NULL
  int M, N, K;
};

// LDS byte offset of 16-byte chunk c (0..3) of staged row r. The XOR keeps
// both the row-per-lane MFMA reads and the chunk-per-lane stores free of
// bank conflicts.
#ifndef Q4MI_GEMM_SWZ
#define Q4MI_GEMM_SWZ 1
#endif
__device__ inline int lds_off(int r, int c) {
#if Q4MI_GEMM_SWZ
  // distinct 16-byte bank groups for any 8 consecutive rows (same chunk) and
  // for rows {0, 4, 8, 12} (+1, +2, +3) of any 16: conflict-free whether the
  // LDS serves 8 or 16 lanes of a ds_read_b128 per cycle
  return r * 64 + ((c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1))) << 4);
#else
  return r * 64 + ((c ^ ((r >> 1) & 3)) << 4);
#endif
}

__device__ inline uint32_t pk_h2(v2h v) { return __builtin_bit_cast(uint32_t, v); }

// int4 unit -> 32 f16 values f16((q - 8) * s), 4 chunks of 8 (k order).
// Low nibbles: 0x6400 | q = 1024 + q; high nibbles: 0x6400 | 16q =
// 1024 + 16q. Both become q - 8 exactly, then one RNE multiply by s, which
// is the reference's float16_t((float(q) - 8.0) * scl).
__device__ inline void dequant_unit_f16(const v4u u, _Float16 s, v4u out[4]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  const v2h sv = {s, s};
  const v2h off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
  const v2h sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const v2h off_hi = {(_Float16)72.0f, (_Float16)72.0f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w8 = w[i] >> 8;
    v2h p0 = __builtin_bit_cast(v2h, (w[i] & 0x000F000Fu) | 0x64006400u);
    v2h p1 = __builtin_bit_cast(v2h, (w[i] & 0x00F000F0u) | 0x64006400u);
    v2h p2 = __builtin_bit_cast(v2h, (w8 & 0x000F000Fu) | 0x64006400u);
    v2h p3 = __builtin_bit_cast(v2h, (w8 & 0x00F000F0u) | 0x64006400u);
    p0 = (p0 - off_lo) * sv;
    p1 = (p1 * sixteenth - off_hi) * sv;
    p2 = (p2 - off_lo) * sv;
    p3 = (p3 * sixteenth - off_hi) * sv;
    out[i] = v4u{pk_h2(p0), pk_h2(p1), pk_h2(p2), pk_h2(p3)};
  }
}

// int4 unit -> 32 int8 values clamp(rint((q - 8) * r), -127, 127), k order.
__device__ inline void requant_unit_i8(const v4u u, float r, v4u out[2]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t word = 0;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int e = 4 * h + e4;
        const float q = (float)(int)((w[i] >> (4 * nib_pos(e))) & 15u) - 8.0f;
        float v = rintf(__fmul_rn(q, r));
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        word |= ((uint32_t)(int)v & 0xFFu) << (8 * e4);
      }
      o[2 * i + h] = word;
    }
  }
  out[0] = v4u{o[0], o[1], o[2], o[3]};
  out[1] = v4u{o[4], o[5], o[6], o[7]};
}

typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Copy one 32x32 accumulator tile (16 registers per lane) into an LDS strip
// with row stride `st` words: register v goes to row 8 (v / 4) + v % 4 (the
// lane's 4-row half is folded into p). Each element is moved to a VGPR
// first (the empty asm with a "v" operand): LDS stores taking the elements
// straight from the accumulator registers were compiled to 16 stores of the
// tile's first register.
template <class V>
__device__ inline void store_tile_strip(uint32_t* p, int st, const V t) {
  uint32_t e[16];
  __builtin_memcpy(e, &t, sizeof(e));
#pragma unroll
  for (int v = 0; v < 16; ++v) p[(8 * (v >> 2) + (v & 3)) * st] = e[v];
}

template <bool F16, class A>
__device__ inline A q4_mfma(v4i a, v4i b, A c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <int OP, int BM, int BN, int D>
__global__ void __launch_bounds__(256) gemm_kernel(const GemmArgs g) {
  constexpr int STAGE = (BM + BN) * 64;
  constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
  constexpr int A_CH = BM / 64;                                      // A chunks per thread per k-step
  constexpr int B_CH = (OP == OP_W8A8) ? BN / 64 : (OP == OP_W4A16 ? BN / 256 : BN / 128);
  constexpr bool F16 = (OP == OP_W4A16);
  static_assert(BN % 256 == 0 || OP == OP_W8A8, "int4 B producers need BN % 256 == 0");
  typedef typename std::conditional<F16, v16f, v16i>::type acc_t;

  constexpr int EST = 36;  // epilogue strip row stride in 32-bit words (16-byte aligned, staggers banks)
  constexpr int EPI = GEMM_WAVES_EPI * WM * EST * 4;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE > EPI ? 2 * STAGE : EPI];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = g.M, N = g.N, K = g.K;
  const int ntm = (M + BM - 1) / BM;
  const int G = gridDim.x, w = blockIdx.x;
  const int v = (G % 8 == 0) ? (w % 8) * (G / 8) + w / 8 : w;
  const int tm = v % ntm, tn = v / ntm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nblk = K / BLK;
  const int nk = F16 ? K / 32 : K / 64;                               // k-steps (64-byte rows)
  const long a_row_bytes = F16 ? 2L * K : (long)K;

  // ---- per-thread global sources: rows (tid / 4) + 64 i, 16-byte chunk tid % 4 ----
  const uint8_t* Ab = reinterpret_cast<const uint8_t*>(g.A);
  const int a_chunk = tid & 3;
  const uint8_t* a_src[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i)
    a_src[i] = Ab + (long)min(m0 + (tid >> 2) + 64 * i, M - 1) * a_row_bytes + a_chunk * 16;
  const uint8_t* b_src[(OP == OP_W8A8) ? B_CH : 1];
  if constexpr (OP == OP_W8A8) {
#pragma unroll
    for (int i = 0; i < B_CH; ++i)
      b_src[i] = reinterpret_cast<const uint8_t*>(g.B) + (long)min(n0 + (tid >> 2) + 64 * i, N - 1) * K + a_chunk * 16;
  }

  // D rotating register buffers of one k-step each (native vector registers:
  // HIP's uint4 is a union struct the compiler keeps in scratch here). A
  // k-step is loaded D iterations before it is staged into LDS, so D - 1
  // k-steps of MFMA work hide the global load latency.
  v4u ra[D][A_CH];
  v4u rb[D][(OP == OP_W8A8) ? B_CH : 1];
  v4u ru[D][(OP == OP_W8A8) ? 1 : B_CH];
  uint16_t rs[D][(OP == OP_W8A8) ? 1 : B_CH];

#define Q4_LOAD_REGS(buf_, kt_)                                                                        \
  do {                                                                                                 \
    const int kt_v = min((kt_), nk - 1); /* clamped: every load unconditional */                       \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) ra[buf_][i] =                                    \
        *reinterpret_cast<const v4u*>(a_src[i] + (long)kt_v * 64);                                   \
    if constexpr (OP == OP_W8A8) {                                                                     \
      _Pragma("unroll") for (int i = 0; i < B_CH; ++i) rb[buf_][i] =                                  \
          *reinterpret_cast<const v4u*>(b_src[i] + (long)kt_v * 64);                                 \
    } else {                                                                                           \
      const v4u* U = reinterpret_cast<const v4u*>(g.B);                                               \
      _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                              \
        /* W4A16: one block per k-step, row = tid + 256 i;                                          */ \
        /* W4A8: two blocks per k-step, i = 2 rr + h, row = tid + 256 rr                              */ \
        const int rr = (OP == OP_W4A16) ? i : i / 2;                                                   \
        const int blk = (OP == OP_W4A16) ? kt_v : 2 * kt_v + (i & 1);                                  \
        const int n = min(n0 + tid + 256 * rr, N - 1);                                                 \
        const long idx = panel_index(n, blk, nblk);                                                    \
        ru[buf_][i] = U[idx];                                                                          \
        rs[buf_][i] = g.bsc[idx];                                                                      \
      }                                                                                                \
    }                                                                                                  \
  } while (0)

#define Q4_STORE_LDS(buf_, stage_)                                                                     \
  do {                                                                                                 \
    uint8_t* base_ = lds + (stage_) * STAGE;                                                           \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                                                \
      const int r = (tid >> 2) + 64 * i;                                                               \
      *reinterpret_cast<v4u*>(base_ + lds_off(r, a_chunk)) = ra[buf_][i];                              \
    }                                                                                                  \
    if constexpr (OP == OP_W8A8) {                                                                     \
      _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                              \
        const int r = BM + (tid >> 2) + 64 * i;                                                        \
        *reinterpret_cast<v4u*>(base_ + lds_off(r, a_chunk)) = rb[buf_][i];                            \
      }                                                                                                \
    } else if constexpr (OP == OP_W4A16) {                                                             \
      _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                              \
        const int r = BM + tid + 256 * i;                                                              \
        v4u o[4];                                                                                      \
        dequant_unit_f16(ru[buf_][i], __builtin_bit_cast(_Float16, rs[buf_][i]), o);                   \
        _Pragma("unroll") for (int c = 0; c < 4; ++c)                                                  \
            *reinterpret_cast<v4u*>(base_ + lds_off(r, c)) = o[c];                                     \
      }                                                                                                \
    } else {                                                                                           \
      _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                              \
        const int r = BM + tid + 256 * (i / 2);                                                        \
        v4u o[2];                                                                                      \
        requant_unit_i8(ru[buf_][i], h2f(rs[buf_][i]), o);                                             \
        *reinterpret_cast<v4u*>(base_ + lds_off(r, 2 * (i & 1))) = o[0];                               \
        *reinterpret_cast<v4u*>(base_ + lds_off(r, 2 * (i & 1) + 1)) = o[1];                           \
      }                                                                                                \
    }                                                                                                  \
  } while (0)

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};

#pragma unroll
  for (int d = 0; d < D; ++d) Q4_LOAD_REGS(d, d);
  Q4_STORE_LDS(0, 0);
  __syncthreads();

  // MFMA operand: row lane % 32 of a 32-row tile, 16 bytes at byte 16 * (lane / 32) of the 32-byte k-slice
  const int frow = lane & 31, fhalf = lane >> 5;
  {
    // Explicit software pipeline per k-step, D rotating register buffers:
    // global loads of k-step kt + D first, both k-slices' fragments read from
    // LDS, then MFMAs of slice 0 interleaved with the slice-1 fragment reads
    // and MFMAs of slice 1 interleaved with the LDS stores of k-step kt + 1
    // (loaded D - 1 k-steps ago, into the other stage), one barrier. The
    // sched_group_barrier sequence pins that order so the MFMA pipe is fed
    // while LDS and memory requests are in flight.
#define Q4_KSTEP(dl_, ds_)                                                                               \
    do {                                                                                                \
      Q4_LOAD_REGS(dl_, kt + D);                                                                        \
      const uint8_t* base = lds + (kt & 1) * STAGE;                                                     \
      v4i fa0[FM], fb0[FN], fa1[FM], fb1[FN];                                                           \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                    \
          fa0[i] = *reinterpret_cast<const v4i*>(base + lds_off(wm * WM + 32 * i + frow, fhalf));       \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                    \
          fb0[j] = *reinterpret_cast<const v4i*>(base + lds_off(BM + wn * WN + 32 * j + frow, fhalf));  \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                    \
          fa1[i] = *reinterpret_cast<const v4i*>(base + lds_off(wm * WM + 32 * i + frow, 2 + fhalf));   \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                    \
          fb1[j] = *reinterpret_cast<const v4i*>(base + lds_off(BM + wn * WN + 32 * j + frow, 2 + fhalf)); \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                    \
        _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = q4_mfma<F16>(fa0[i], fb0[j], acc[i][j]); \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                    \
        _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = q4_mfma<F16>(fa1[i], fb1[j], acc[i][j]); \
      Q4_STORE_LDS(ds_, (kt + 1) & 1); /* past the last k-step: clamped data nobody reads */            \
      Q4_SCHED();                                                                                       \
      __syncthreads();                                                                                  \
    } while (0)
#if !defined(Q4MI_GEMM_SGB) || Q4MI_GEMM_SGB
    constexpr int NMF = FM * FN;                                          // MFMAs per k-slice
    constexpr int NRD = FM + FN;                                          // fragment reads per k-slice
    constexpr int NVM = (OP == OP_W8A8) ? A_CH + B_CH : A_CH + 2 * B_CH;  // global loads per k-step
    constexpr int NWR = (OP == OP_W8A8) ? A_CH + B_CH : (OP == OP_W4A16 ? A_CH + 4 * B_CH : A_CH + 2 * B_CH);
#define Q4_SCHED()                                                                                      \
    do {                                                                                                \
      __builtin_amdgcn_sched_group_barrier(0x020, NVM, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);                                              \
      _Pragma("unroll") for (int q = 0; q < NRD; ++q) {                                                 \
        __builtin_amdgcn_sched_group_barrier(0x008, NMF / NRD > 0 ? NMF / NRD : 1, 0);                  \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                              \
      }                                                                                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, NMF - (NMF / NRD) * NRD, 0);                          \
      _Pragma("unroll") for (int q = 0; q < NWR; ++q) {                                                 \
        __builtin_amdgcn_sched_group_barrier(0x008, NMF / NWR > 0 ? NMF / NWR : 1, 0);                  \
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                                              \
      }                                                                                                 \
    } while (0)
#else
#define Q4_SCHED() do {} while (0)
#endif
    for (int kt0 = 0; kt0 < nk; kt0 += D) {
      { const int kt = kt0;     Q4_KSTEP(0, 1 % D); }
      if constexpr (D > 1) { const int kt = kt0 + 1; Q4_KSTEP(1 % D, 2 % D); }
      if constexpr (D > 2) { const int kt = kt0 + 2; Q4_KSTEP(2 % D, 3 % D); }
      if constexpr (D > 3) { const int kt = kt0 + 3; Q4_KSTEP(3 % D, 4 % D); }
    }
#undef Q4_KSTEP
#undef Q4_SCHED
  }

  // ---- epilogue through LDS (free after the loop's last barrier). Register
  //      v of lane holds D[8 (v / 4) + 4 (lane / 32) + v % 4][lane % 32].
  //      Each wave copies one 32-column strip of its tile into its own LDS
  //      region with straight-line code (no branches next to the
  //      accumulator reads), then reads it back 4 columns per lane for
  //      bounds-checked, row-contiguous stores. ----
  uint32_t* strip = reinterpret_cast<uint32_t*>(lds) + wave * (WM * EST);
  const int col = lane & 31, rh = (lane >> 5) * 4;
  const int mw = m0 + wm * WM, nw = n0 + wn * WN;
  const int rrow = lane >> 3, rcol = (lane & 7) * 4;
  constexpr int NIT = WM / 8;  // strip rows handled per lane: 8 it + lane / 8
  // every per-row / per-column scale this lane needs, loaded up front (the
  // loads are independent; issuing them inside the store loop would put one
  // L2 round trip per row on the critical path)
  float sav[F16 ? 1 : NIT];
  float swv[F16 ? 1 : FN][4];
  if constexpr (!F16) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) sav[it] = g.sa ? g.sa[min(mw + 8 * it + rrow, M - 1)] : 0.0f;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ne = min(nw + 32 * j + rcol + e, N - 1);
        swv[j][e] = g.sw_f16 ? h2f(reinterpret_cast<const uint16_t*>(g.sw)[ne])
                             : (g.sw ? reinterpret_cast<const float*>(g.sw)[ne] : 0.0f);
      }
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int i = 0; i < FM; ++i) store_tile_strip(strip + (32 * i + rh) * EST + col, EST, acc[i][j]);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's strip is in LDS
    __builtin_amdgcn_wave_barrier();
    const int n = nw + 32 * j + rcol;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int row = 8 * it + rrow;
      const int m = mw + row;
      const uint4 q = *reinterpret_cast<const uint4*>(strip + row * EST + rcol);
      const uint32_t qv[4] = {q.x, q.y, q.z, q.w};
      if (m < M) {
        const long o = (long)m * N + n;
        const bool vec = n + 3 < N && (o & 3) == 0;
        if constexpr (F16) {
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = f2h(__builtin_bit_cast(float, qv[e]));
          if (vec) {
            *reinterpret_cast<ushort4*>(g.Y + o) = make_ushort4(h[0], h[1], h[2], h[3]);
          } else {
            for (int e = 0; e < 4; ++e)
              if (n + e < N) g.Y[o + e] = h[e];
          }
        } else {
          if (g.C) {
            if (vec) *reinterpret_cast<uint4*>(g.C + o) = q;
            else
              for (int e = 0; e < 4; ++e)
                if (n + e < N) g.C[o + e] = (int32_t)qv[e];
          }
          if (g.Y) {
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              h[e] = f2h_after_f32(__fmul_rn(__fmul_rn((float)(int)qv[e], sav[it]), swv[j][e]));
            if (vec) *reinterpret_cast<ushort4*>(g.Y + o) = make_ushort4(h[0], h[1], h[2], h[3]);
            else
              for (int e = 0; e < 4; ++e)
                if (n + e < N) g.Y[o + e] = h[e];
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // strip reads done before the next strip overwrites it
  }
}
#undef Q4_LOAD_REGS
#undef Q4_STORE_LDS

// ---- per-row int8 activation quantizer (vk/cast_i8.comp) -----------------
template <int XT>
__global__ void __launch_bounds__(256) quant_act_kernel(const void* __restrict__ X, int K, int8_t* __restrict__ A,
                                                        float* __restrict__ sa) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  auto ld4 = [&](int i, float v[4]) {  // elements 4i..4i+3 of row m
    if constexpr (XT == Q4_DT_F16) {
      ushort4 h = reinterpret_cast<const ushort4*>(reinterpret_cast<const uint16_t*>(X) + (long)m * K)[i];
      v[0] = h2f(h.x); v[1] = h2f(h.y); v[2] = h2f(h.z); v[3] = h2f(h.w);
    } else {
      float4 f = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(X) + (long)m * K)[i];
      v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    }
  };
  const int K4 = K / 4;
  float mx = 0.0f;
  for (int i = tid; i < K4; i += 256) {
    float v[4];
    ld4(i, v);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(__fdiv_rn(mx, 127.0f), 1e-12f);
  if (tid == 0) sa[m] = s;
  uint32_t* dst = reinterpret_cast<uint32_t*>(A + (long)m * K);
  for (int i = tid; i < K4; i += 256) {
    float v[4];
    ld4(i, v);
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float q = rintf(__fdiv_rn(v[e], s));
      q = fminf(fmaxf(q, -127.0f), 127.0f);
      word |= ((uint32_t)(int)q & 0xFFu) << (8 * e);
    }
    dst[i] = word;
  }
}

template <int OP, int BM, int BN>
static int launch_tiles(const GemmArgs& g, void* stream, const char* name) {
  const int ntm = ceil_div(g.M, BM), ntn = ceil_div(g.N, BN);
  const int nk = OP == OP_W4A16 ? g.K / 32 : g.K / 64;
#ifndef Q4MI_GEMM_DEEP
#define Q4MI_GEMM_DEEP 2
#endif
#ifndef Q4MI_GEMM_DEEP_SMALL
#define Q4MI_GEMM_DEEP_SMALL 4
#endif
  constexpr int DEEP = BM >= 256 ? Q4MI_GEMM_DEEP : Q4MI_GEMM_DEEP_SMALL;
  if (nk % DEEP == 0)
    hipLaunchKernelGGL((gemm_kernel<OP, BM, BN, DEEP>), dim3(ntm * ntn), dim3(256), 0, as_stream(stream), g);
  else
    hipLaunchKernelGGL((gemm_kernel<OP, BM, BN, 1>), dim3(ntm * ntn), dim3(256), 0, as_stream(stream), g);
  Q4_LAUNCHED(name);
  return Q4_OK;
}

// 128 x 256 tiles: with a 4-deep register prefetch they fit the register
// file without spills (256 x 256 tiles spill at any prefetch depth > 1).
template <int OP>
static int launch_gemm(const GemmArgs& g, void* stream, const char* name) {
#if !defined(Q4MI_GEMM_BIG) || Q4MI_GEMM_BIG
  if ((long)ceil_div(g.M, 256) * ceil_div(g.N, 256) >= 256) return launch_tiles<OP, 256, 256>(g, stream, name);
#endif
  return launch_tiles<OP, 128, 256>(g, stream, name);
}

}  // namespace q4

using namespace q4;

extern "C" {

int q4_quant_act_i8(const void* X, int x_dtype, int8_t* A, float* sa, int M, int K, void* stream) {
  clear_error();
  Q4_ARG(M > 0 && K > 0 && K % 4 == 0, "bad shape M=%d K=%d (K must be a multiple of 4)", M, K);
  Q4_ARG(X && A && sa, "null pointer");
  Q4_ARG(x_dtype == Q4_DT_F32 || x_dtype == Q4_DT_F16, "bad x dtype %d", x_dtype);
  Q4_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)A & 3) == 0, "misaligned X or A");
  if (x_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(quant_act_kernel<Q4_DT_F16>, dim3(M), dim3(256), 0, as_stream(stream), X, K, A, sa);
  else
    hipLaunchKernelGGL(quant_act_kernel<Q4_DT_F32>, dim3(M), dim3(256), 0, as_stream(stream), X, K, A, sa);
  Q4_LAUNCHED("quant_act_i8");
  return Q4_OK;
}

int q4_gemm_w8a8(const int8_t* A, const int8_t* W8, const float* sa, const void* sw, int sw_dtype, uint16_t* Y,
                 int32_t* C, int M, int N, int K, void* stream) {
  clear_error();
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 64 == 0, "bad W8A8 shape M=%d N=%d K=%d (K must be a multiple of 64)", M, N,
         K);
  Q4_ARG((long)127 * 127 * K < (1L << 31), "K=%d overflows the int32 accumulator", K);
  Q4_ARG(A && W8 && (Y || C), "null pointer");
  Q4_ARG(!Y || (sa && sw), "Y needs sa and sw");
  Q4_ARG(sw_dtype == Q4_DT_F32 || sw_dtype == Q4_DT_F16, "bad sw dtype %d", sw_dtype);
  Q4_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)W8 & 15) == 0, "A and W8 must be 16-byte aligned");
  GemmArgs g{A, W8, nullptr, sa, sw, sw_dtype == Q4_DT_F16, Y, C, M, N, K};
  return launch_gemm<OP_W8A8>(g, stream, "gemm_w8a8");
}

int q4_gemm_w4a8(const int8_t* A, const uint32_t* wq, const uint16_t* ratio, const float* sa, const void* sw,
                 int sw_dtype, uint16_t* Y, int32_t* C, int M, int N, int K, void* stream) {
  clear_error();
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 64 == 0, "bad W4A8 shape M=%d N=%d K=%d (K must be a multiple of 64)", M, N,
         K);
  Q4_ARG((long)127 * 127 * K < (1L << 31), "K=%d overflows the int32 accumulator", K);
  Q4_ARG(A && wq && ratio && (Y || C), "null pointer");
  Q4_ARG(!Y || (sa && sw), "Y needs sa and sw");
  Q4_ARG(sw_dtype == Q4_DT_F32 || sw_dtype == Q4_DT_F16, "bad sw dtype %d", sw_dtype);
  Q4_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)wq & 15) == 0, "A and wq must be 16-byte aligned");
  GemmArgs g{A, wq, ratio, sa, sw, sw_dtype == Q4_DT_F16, Y, C, M, N, K};
  return launch_gemm<OP_W4A8>(g, stream, "gemm_w4a8");
}

int q4_gemm_w4a16(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, uint16_t* Y, int M, int N, int K,
                  void* stream) {
  clear_error();
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 32 == 0, "bad W4A16 shape M=%d N=%d K=%d (K must be a multiple of 32)", M, N,
         K);
  Q4_ARG(X && wq && sc16 && Y, "null pointer");
  Q4_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)wq & 15) == 0, "X and wq must be 16-byte aligned");
  GemmArgs g{X, wq, sc16, nullptr, nullptr, 0, Y, nullptr, M, N, K};
  return launch_gemm<OP_W4A16>(g, stream, "gemm_w4a16");
}

}  // extern "C"
