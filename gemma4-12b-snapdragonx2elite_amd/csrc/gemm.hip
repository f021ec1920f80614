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
// Both kernels stage the activation tile A through an LDS ring filled by
// direct-to-LDS loads (global_load_lds_dwordx4: no VGPR round trip, no
// staging registers) and feed 4 waves (2 x 2, each a (BM/2) x 128 block of
// 32x32 MFMA tiles) from it. They differ in how the weight operand B
// arrives:
//  * W8A8 (w8a8_kernel): int8 rows are loaded into registers one and a half
//    k-steps ahead and written into a second LDS ring; fragments are read
//    from LDS like A's. Direct-to-LDS loads sustain only ~24 B/clk per CU on
//    MI355X, half of what the 256x256 tile needs, so the two operands take
//    the two load paths.
//  * W4A16 / W4A8 (w4_kernel): each lane loads the 8-byte half of a
//    32-element int4 unit that its MFMA fragment needs (the panel-64 layout
//    makes the 32 rows of a fragment 512 contiguous bytes) several k-steps
//    ahead, and dequantizes (f16) or requantizes (int8) it straight into
//    fragment registers. B never touches LDS, which leaves LDS bandwidth to
//    A: with the 128-row tiles that M = 512 needs, staging both operands in
//    LDS would need more than the ~128 B/clk LDS read bandwidth per CU.
//    The k order inside a fragment is permuted consistently for A and B
//    (a dot product does not care) so each lane's 16 k-values come from one
//    contiguous half-unit.
//
// All global loads are issued through inline asm and all waits are explicit
// s_waitcnt vmcnt(n) with the count fixed by the issue order: the compiler's
// own tracking of direct-to-LDS writes is conservative (it waits for every
// outstanding load before each LDS access), which would serialize the ring.
// Each wait also pins the registers it covers (an empty asm that reads and
// writes them), so no use of a loaded value can be scheduled above its wait.
//
// Packed W8A8 on large grids (w8q_kernel) is persistent instead: one
// workgroup per CU walks its share of 128 x 320 tiles through one load
// pipeline and stages each tile's fp16 Y in LDS, stored behind the next
// tile's MFMAs.
//
// Workgroups are remapped so each XCD (8 per MI355X, own L2) works on a
// contiguous 1/8 of the tile grid ordered by weight panel. W4A16 splits K
// across workgroups when the tile grid alone cannot fill the 256 CUs
// (tall-K shapes such as the down projection), writing fp32 partials that a
// second kernel sums in split order (deterministic).
#include "q4mi_common.h"

namespace q4 {

enum { OP_W8A8 = 0, OP_W4A16 = 1, OP_W4A8 = 2 };

typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const void* A;        // int8 [M][K] or f16 [M][K]
  const void* B;        // int8 [N][K] (W8A8) or panel-64 int4 units
  const uint16_t* bsc;  // panel-64 fp16 scales (W4A16) or ratio (W4A8)
  const float* sa;      // [M]
  const void* sw;       // [N] f32 or f16
  int sw_f16;
  uint16_t* Y;          // f16 [M][N] (may be NULL for int paths if C given)
  int32_t* C;           // int32 [M][N] or NULL
  float* P;             // W4A16 split-K: fp32 partials [split][M][N]
  int M, N, K;
  unsigned long long* stamps;  // stamped W8A8 only: 4 words per workgroup
};

// LDS byte offset of 16-byte chunk c (0..3) of staged 64-byte row r. The XOR
// keeps both the row-per-lane MFMA reads and the chunk-per-lane writes free
// of bank conflicts: distinct 16-byte bank groups for any 8 consecutive rows
// (same chunk) and for rows {0, 4, 8, 12} (+1, +2, +3) of any 16, whether
// the LDS serves 8 or 16 lanes of a ds_read_b128 per cycle.
__device__ inline int swz(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }
__device__ inline int lds_off(int r, int c) { return r * 64 + ((c ^ swz(r)) << 4); }

__device__ inline uint32_t pk_h2(v2h v) { return __builtin_bit_cast(uint32_t, v); }

// One device word (8 int4 codes, k order e = 0..7 at nibble (e&1)*4 + (e>>1))
// -> 8 f16 values f16((q - 8) * s) in k order. Low nibbles: 0x6400 | q =
// 1024 + q; high nibbles: 0x6400 | 16q = 1024 + 16q. Both become q - 8
// exactly, then one RNE multiply by s: the reference's
// float16_t((float(q) - 8.0) * scl) (vk/coopgemm_i4h.comp:24).
__device__ inline v4u dequant_word_f16(uint32_t w, v2h sv) {
  const v2h off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
  const v2h sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const v2h off_hi = {(_Float16)72.0f, (_Float16)72.0f};
  const uint32_t w8 = w >> 8;
  v2h p0 = __builtin_bit_cast(v2h, (w & 0x000F000Fu) | 0x64006400u);
  v2h p1 = __builtin_bit_cast(v2h, (w & 0x00F000F0u) | 0x64006400u);
  v2h p2 = __builtin_bit_cast(v2h, (w8 & 0x000F000Fu) | 0x64006400u);
  v2h p3 = __builtin_bit_cast(v2h, (w8 & 0x00F000F0u) | 0x64006400u);
  p0 = (p0 - off_lo) * sv;
  p1 = (p1 * sixteenth - off_hi) * sv;
  p2 = (p2 - off_lo) * sv;
  p3 = (p3 * sixteenth - off_hi) * sv;
  return v4u{pk_h2(p0), pk_h2(p1), pk_h2(p2), pk_h2(p3)};
}

// Pair P (codes e = 2P, 2P + 1 in k order) of dequant_word_f16, in three VALU
// operations: high nibbles use 0x5400 | 16q = 64 + q (ulp 1/16), so both
// halves become q - 8 with one exact add before the RNE multiply by s. mlo =
// 0x64006400 and mhi = 0x54005400 come in VGPRs: v_and_or_b32 takes no
// literal constants, and the masks go to SGPRs.
template <int P>
__device__ inline uint32_t dequant_pair_f16(uint32_t w, v2h sv, uint32_t mlo, uint32_t mhi) {
  const uint32_t x = P >= 2 ? w >> 8 : w;
  v2h p;
  if constexpr (P & 1) {
    const v2h off = {(_Float16)-72.0f, (_Float16)-72.0f};
    p = __builtin_bit_cast(v2h, (x & 0x00F000F0u) | mhi) + off;
  } else {
    const v2h off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    p = __builtin_bit_cast(v2h, (x & 0x000F000Fu) | mlo) + off;
  }
  return pk_h2(p * sv);
}

// Two device words (16 codes, k order) -> 16 int8 values
// clamp(rint((q - 8) * r), -127, 127) in k order (vk/coopgemm_w4a8.comp:28-34).
__device__ inline v4u requant_words_i8(uint32_t wa, uint32_t wb, float r) {
  const uint32_t w[2] = {wa, wb};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
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
  return v4u{o[0], o[1], o[2], o[3]};
}

// Copy one 32x32 accumulator tile (16 registers per lane) into an LDS strip
// with row stride `st` words: register v goes to row 8 (v / 4) + v % 4 (the
// lane's 4-row half is folded into p). The elements go through a memcpy to a
// plain array first: LDS stores taking the elements straight from the
// accumulator registers were compiled to 16 stores of the tile's first
// register.
template <class V>
__device__ inline void store_tile_strip(uint32_t* p, int st, const V t) {
  uint32_t e[16];
  __builtin_memcpy(e, &t, sizeof(e));
#pragma unroll
  for (int v = 0; v < 16; ++v) p[(8 * (v >> 2) + (v & 3)) * st] = e[v];
}

// Tile (tm, tn) of workgroup w: each XCD (workgroups w % 8, round-robin
// dispatch) gets a contiguous 1/8 of the grid, M fastest, so the tiles an XCD
// runs together share weight panels in its L2.
__device__ inline void tile_of(int w, int G, int ntm, int& tm, int& tn) {
  const int v = (G % 8 == 0) ? (w % 8) * (G / 8) + w / 8 : w;
  tm = v % ntm;
  tn = v / ntm;
}

constexpr int EST = 68;  // epilogue strip row stride (words): 64 columns + 4 to stagger banks

// Epilogue: the wave's WM x (32 FN) accumulator block goes through a
// 64-column LDS strip per 64 columns (so each stored row segment is a full 128-byte line of
// f16 Y) and is stored row-contiguously, 4 columns per lane. MODE 0: int32
// accumulators -> Y = f16((f32(C) * sa) * sw) and/or C; MODE 1: fp32 -> f16
// Y; MODE 2: fp32 -> fp32 partials P.
template <int MODE, int WM, int FN = 4, class acc_t>
__device__ inline void epilogue(const GemmArgs& g, uint32_t* strip, const acc_t (&acc)[WM / 32][FN], int mw, int nw,
                                float* P) {
  static_assert(FN == 2 || FN == 4, "64 or 128 columns per wave block");
  constexpr int FM = WM / 32, NIT = WM / 4;
  const int lane = threadIdx.x & 63;
  const int col = lane & 31, rh = (lane >> 5) * 4;
  const int rrow = lane >> 4, rcol = (lane & 15) * 4;
  const int M = g.M, N = g.N;
  // every per-row scale this lane needs, loaded up front (independent loads;
  // inside the store loop each would put an L2 round trip on the critical path)
  float sav[MODE == 0 ? NIT : 1];
  if constexpr (MODE == 0) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) sav[it] = g.Y ? g.sa[min(mw + 4 * it + rrow, M - 1)] : 0.0f;
  }
#pragma unroll
  for (int jp = 0; jp < FN / 2; ++jp) {
    const int n = nw + 64 * jp + rcol;
    float swv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (MODE == 0) {
      if (g.Y) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ne = min(n + e, N - 1);
          swv[e] = g.sw_f16 ? h2f(reinterpret_cast<const uint16_t*>(g.sw)[ne]) : reinterpret_cast<const float*>(g.sw)[ne];
        }
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < FM; ++i) store_tile_strip(strip + (32 * i + rh) * EST + 32 * h + col, EST, acc[i][2 * jp + h]);
    lgkm0();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int row = 4 * it + rrow;
      const int m = mw + row;
      const v4u q = *reinterpret_cast<const v4u*>(strip + row * EST + rcol);
      // elements through a plain array: bit-casting q[e] of the vector inside
      // the unrolled loop was compiled to four stores of element 0
      uint32_t qv[4];
      __builtin_memcpy(qv, &q, sizeof(qv));
      if (m < M) {
        const long o = (long)m * N + n;
        const bool vec = n + 3 < N && (o & 3) == 0;
        if constexpr (MODE == 2) {
          if (vec) {
            *reinterpret_cast<v4u*>(P + o) = q;
          } else {
            for (int e = 0; e < 4; ++e)
              if (n + e < N) P[o + e] = __builtin_bit_cast(float, qv[e]);
          }
        } else {
          uint16_t hv[4];
          if constexpr (MODE == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = f2h(__builtin_bit_cast(float, qv[e]));
          } else {
            if (g.C) {
              if (vec) {
                *reinterpret_cast<v4u*>(g.C + o) = q;
              } else {
                for (int e = 0; e < 4; ++e)
                  if (n + e < N) g.C[o + e] = (int32_t)qv[e];
              }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
              hv[e] = f2h_after_f32(__fmul_rn(__fmul_rn((float)(int)qv[e], sav[it]), swv[e]));
          }
          if (MODE == 1 || g.Y) {
            if (vec) {
              *reinterpret_cast<ushort4*>(g.Y + o) = make_ushort4(hv[0], hv[1], hv[2], hv[3]);
            } else {
              for (int e = 0; e < 4; ++e)
                if (n + e < N) g.Y[o + e] = hv[e];
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // strip reads done before the next half overwrites it
  }
}

// Epilogue of a wave's 256 x 64 int32 block that lies wholly inside Y, with
// no int32 output: Y = f16((f32(C) * sa) * sw), the same arithmetic as
// epilogue<0> without its bounds and output-kind branches. Four 64-row
// chunks go through the wave's LDS strip; a chunk's scales are loaded
// before its strip is filled. Each lane stores 8 columns (16 bytes) of a
// row, 8 rows per instruction, with nontemporal stores: Y is not read again
// by this kernel, and lines left out of L2 shorten the kernel's end (its
// release writes back less). Measured at M=2048, N=15360, K=3840 against
// 8-byte stores: the epilogue 7.1 -> 6.5 us per tile and the gap before the
// next launch 2.7 -> 1.1 us. Needs N % 8 == 0 (16-byte aligned rows).
template <class acc_t>
__device__ inline void epilogue_w8_full(const GemmArgs& g, uint32_t* strip, const acc_t (&acc)[8][2], int m0, int nw) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 31, rh = (lane >> 5) * 4;
  const int rrow = lane >> 3, rcol = (lane & 7) * 8;
  const int N = g.N;
  float swv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    swv[e] = g.sw_f16 ? h2f(reinterpret_cast<const uint16_t*>(g.sw)[nw + rcol + e])
                      : reinterpret_cast<const float*>(g.sw)[nw + rcol + e];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float sav[8];  // this chunk's row scales, loaded before the strip is filled
#pragma unroll
    for (int it = 0; it < 8; ++it) sav[it] = g.sa[m0 + 64 * c + 8 * it + rrow];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 2; ++i) store_tile_strip(strip + (32 * i + rh) * EST + 32 * h + col, EST, acc[2 * c + i][h]);
    lgkm0();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 8 * it + rrow;
      const v4u q0 = *reinterpret_cast<const v4u*>(strip + row * EST + rcol);
      const v4u q1 = *reinterpret_cast<const v4u*>(strip + row * EST + rcol + 4);
      // elements through a plain array (see epilogue<>)
      uint32_t qv[8];
      __builtin_memcpy(qv, &q0, 16);
      __builtin_memcpy(qv + 4, &q1, 16);
      uint32_t hv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hv[e] = f2h_after_f32(__fmul_rn(__fmul_rn((float)(int)qv[e], sav[it]), swv[e]));
      const v4u o = {hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16)};
      __builtin_nontemporal_store(o, reinterpret_cast<v4u*>(g.Y + (long)(m0 + 64 * c + row) * N + nw + rcol));
    }
    __builtin_amdgcn_wave_barrier();  // strip reads done before the next chunk overwrites it
  }
}

// ---- W8A8 ---------------------------------------------------------------------
// BM x 256 tile, K step 64 bytes. LDS: A ring (4 stages, direct loads) and B
// ring (4 stages, register loads + ds_write) in two arrays.
// Issue order per k-step j: B(j + 3) register loads, then A(j + 4) direct
// loads (into the stage k-step j used, whose fragments every wave read in
// the previous k-step); in the middle of k-step j, B(j + 2) is written to
// LDS; one barrier at the end makes k-step j + 2 visible. MFMAs of k-step j
// run from registers while k-step j + 1's fragments are read.
template <int BM>
__global__ void __launch_bounds__(256) w8a8_kernel(const GemmArgs g) {
  constexpr int BN = 256, S = 4, WM = BM / 2, WN = 128, FM = WM / 32, FN = 4;
  constexpr int NA = BM / 64;  // A direct loads per thread per k-step
  constexpr int NB = 4;        // B register loads per thread per k-step
  constexpr int AST = BM * 64, BST = BN * 64;
  constexpr int EPI = 2 * WM * EST * 4;  // two waves' epilogue strips per array
  constexpr int LA = S * AST > EPI ? S * AST : EPI;
  constexpr int LB = S * BST > EPI ? S * BST : EPI;
  // separate arrays: ldsA is written only by direct loads, ldsB only by ds_write
  __shared__ __attribute__((aligned(16))) uint8_t ldsA[LA];
  __shared__ __attribute__((aligned(16))) uint8_t ldsB[LB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = g.M, N = g.N, K = g.K;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K / 64;

  // A: wave instruction i stages rows (wave * NA + i) * 16 .. + 16, 4 lanes per row
  const int8_t* asrc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = (wave * NA + i) * 16 + (lane >> 2);
    asrc[i] = reinterpret_cast<const int8_t*>(g.A) + (long)min(m0 + r, M - 1) * K + (((lane & 3) ^ swz(r)) << 4);
  }
  // B: thread rows (tid / 4) + 64 i, chunk tid % 4
  const int8_t* bsrc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
    bsrc[i] = reinterpret_cast<const int8_t*>(g.B) + (long)min(n0 + (tid >> 2) + 64 * i, N - 1) * K + (tid & 3) * 16;
  const int bdst = lds_off(tid >> 2, tid & 3);  // + 4096 i (64 rows further, same swizzle)

  v4u rb[2][NB];
#define W8_LOAD_B(set_, kt_)                                                                    \
  do {                                                                                          \
    const long ko_ = (long)min((kt_), nk - 1) * 64;                                             \
    _Pragma("unroll") for (int i = 0; i < NB; ++i) rb[set_][i] = ld16(bsrc[i] + ko_);          \
  } while (0)
#define W8_LOAD_A(kt_)                                                                          \
  do {                                                                                          \
    const long ko_ = (long)min((kt_), nk - 1) * 64;                                             \
    uint8_t* st_ = ldsA + ((kt_) % S) * AST;                                                    \
    _Pragma("unroll") for (int i = 0; i < NA; ++i) dma16(asrc[i] + ko_, st_ + (wave * NA + i) * 1024); \
  } while (0)
#define W8_STORE_B(set_, kt_)                                                                   \
  do {                                                                                          \
    uint8_t* st_ = ldsB + ((kt_) % S) * BST + bdst;                                             \
    _Pragma("unroll") for (int i = 0; i < NB; ++i) {                                            \
      pin(rb[set_][i]);                                                                         \
      *reinterpret_cast<v4u*>(st_ + 4096 * i) = rb[set_][i];                                    \
    }                                                                                           \
  } while (0)

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

  const int frow = lane & 31, fh = lane >> 5;
  auto rdA = [&](int stage, int i, int c) {
    return *reinterpret_cast<const v4i*>(ldsA + stage * AST + lds_off(wm * WM + 32 * i + frow, c));
  };
  auto rdB = [&](int stage, int j, int c) {
    return *reinterpret_cast<const v4i*>(ldsB + stage * BST + lds_off(wn * WN + 32 * j + frow, c));
  };

  // prologue, in the steady-state issue order: A0, [B0 A1], [B1 A2], [B2 A3]
  W8_LOAD_A(0);
  W8_LOAD_B(0, 0);
  W8_LOAD_A(1);
  W8_LOAD_B(1, 1);
  W8_LOAD_A(2);
  vmwait<2 * NA + NB>();  // B0 (and A0) landed
  W8_STORE_B(0, 0);
  W8_LOAD_B(0, 2);
  W8_LOAD_A(3);
  vmwait<2 * NA + NB>();  // B1 (and A1) landed
  W8_STORE_B(1, 1);
  lgkm0();
  __builtin_amdgcn_s_barrier();  // stages 0 and 1 visible
  v4i fa[2][2][FM], fb[2][2][FN];  // [buffer][k-slice][tile]
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[0][sl][i] = rdA(0, i, 2 * sl + fh);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[0][sl][j] = rdB(0, j, 2 * sl + fh);
  }
  lgkm0();
  __builtin_amdgcn_s_barrier();  // stage 0 read by every wave: the first k-step may refill it

  constexpr int NRD = FM + FN;  // fragment reads per k-slice
  constexpr int NMF = FM * FN;  // MFMAs per k-slice
#define W8_KSTEP(cur, nxt)                                                                                  \
  do {                                                                                                      \
    W8_LOAD_B(nxt, kt + 3);                                                                                 \
    W8_LOAD_A(kt + 4);                                                                                      \
    const int st1 = (kt + 1) % S;                                                                           \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) fa[nxt][0][i] = rdA(st1, i, fh);                         \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) fb[nxt][0][j] = rdB(st1, j, fh);                         \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                          \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                        \
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][0][i], fb[cur][0][j], acc[i][j], 0, 0, 0);   \
    _Pragma("unroll") for (int q = 0; q < NRD; ++q) {                                                       \
      __builtin_amdgcn_sched_group_barrier(0x008, NMF / NRD > 0 ? NMF / NRD : 1, 0);                        \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                    \
    }                                                                                                       \
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - (NMF / NRD) * NRD, 0);                                \
    vmwait<2 * NA + NB>(); /* B(kt + 2) landed */                                                           \
    W8_STORE_B(cur, kt + 2);                                                                                \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) fa[nxt][1][i] = rdA(st1, i, 2 + fh);                     \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) fb[nxt][1][j] = rdB(st1, j, 2 + fh);                     \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                          \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                        \
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][1][i], fb[cur][1][j], acc[i][j], 0, 0, 0);   \
    _Pragma("unroll") for (int q = 0; q < NB; ++q) {                                                        \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                    \
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                                                    \
    }                                                                                                       \
    _Pragma("unroll") for (int q = 0; q < NRD; ++q) {                                                       \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                    \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                    \
    }                                                                                                       \
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - NB - NRD > 0 ? NMF - NB - NRD : 0, 0);                \
    lgkm0();                                                                                                \
    __builtin_amdgcn_s_barrier(); /* k-step kt + 2 visible */                                               \
  } while (0)
  // register sets alternate: B(kt + 2) sits in set kt & 1, B(kt + 3) goes to the other
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    W8_KSTEP(0, 1);
    ++kt;
    W8_KSTEP(1, 0);
    --kt;
  }
  if (kt < nk) W8_KSTEP(0, 1);
#undef W8_KSTEP
#undef W8_LOAD_A
#undef W8_LOAD_B
#undef W8_STORE_B
  vmwait<0>();
  // The last k-steps' B loads (clamped, never stored) are dead to the
  // compiler right after their asm: without this pin it may hand their
  // registers to epilogue address arithmetic that the in-flight data would
  // then overwrite.
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < NB; ++i) pin(rb[s][i]);
  __builtin_amdgcn_s_barrier();  // every direct load landed before the strips reuse LDS

  uint32_t* strip = reinterpret_cast<uint32_t*>(wave < 2 ? ldsA : ldsB) + (wave & 1) * (WM * EST);
  epilogue<0, WM>(g, strip, acc, m0 + wm * WM, n0 + wn * WN, nullptr);
}

// ---- W8A8 on packed weights ----------------------------------------------------
// Packed ("tile-32") int8 weights: rows padded to a multiple of 32 and K to
// a multiple of 128 (Kp), padding zero; the 32 x 32-byte block of n-tile t
// (rows 32t .. 32t+31) and k-slice s (bytes 32s .. 32s+31) is 1 KB at byte
// (t * (Kp/32) + s) * 1024, and lane l of a wave finds its
// v_mfma_i32_32x32x32_i8 B operand (row 32t + l % 32, bytes
// 32s + 16 (l / 32) .. +16) at byte 16 l of the block. A wave fetches one B
// fragment as 1 KB of contiguous HBM/L2 straight into registers.
__host__ __device__ inline int w8p_kpad(int K) { return (K + 127) / 128 * 128; }
// Position XOR of the 16-byte chunks of staged A row r (128-byte rows): rows
// r .. r+7 (r % 8 == 0) get distinct values, and so do the even and the odd
// rows of any 16 (r % 16 == 0), so a ds_read_b128 of one chunk index over
// 32 consecutive rows is bank-conflict-free whether the LDS serves 8 lanes
// (32 banks) or 16 lanes (64 banks) per cycle: with 128-byte rows, 64 banks
// see rows r and r + 2 at the same bank offset.
__device__ inline int w8p_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__host__ __device__ inline long w8p_block(int t, int s, int kslices) { return ((long)t * kslices + s) * 1024; }

// W8 [N][K] -> packed. One thread per 16-byte chunk; padding is zero.
__global__ void __launch_bounds__(256) w8_pack_kernel(const int8_t* __restrict__ W8, int N, int K,
                                                      int8_t* __restrict__ out, long chunks) {
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int ks = w8p_kpad(K) / 32;
  const long b = c >> 6;
  const int l = (int)(c & 63);
  const int t = (int)(b / ks), sl = (int)(b % ks);
  const int row = 32 * t + (l & 31);
  const long k0 = 32L * sl + 16 * (l >> 5);
  v4u v = {0u, 0u, 0u, 0u};
  if (row < N && k0 < K) v = *reinterpret_cast<const v4u*>(W8 + (long)row * K + k0);
  *reinterpret_cast<v4u*>(out + c * 16) = v;
}

// BM x 256 tile, K step 128 bytes (4 k-slices of 32). Wave w owns columns
// n0 + 64w .. +64 and all BM rows: (BM/32) x 2 MFMA tiles, BM/32 * 2 * 16
// accumulators. A: S = 4 stage LDS ring of direct loads (BM rows x 128 B,
// 16-byte chunks XOR-swizzled by w8p_swz(row)); B: each lane's fragments of the wave's
// two n-tiles for one k-step (8 x 16 B) are loaded two k-steps ahead into a
// 3-set register ring. Per k-step kt:
//   top:      B(kt+2) loads, A(kt+2) direct loads (into the stage k-step kt-2 used)
//   slice 0:  read A slice 1 | MFMAs of slice 0
//   slice 1:  read A slice 2 | MFMAs of slice 1
//   wait for B(kt+1), A(kt+1) (vmcnt: 16 loads of k-step kt+2 may be in flight); barrier
//   slice 2:  read A slice 3 | MFMAs of slice 2
//   slice 3:  read A slice 0 of k-step kt+1 | MFMAs of slice 3
// The stage written at the top of k-step kt was last read in k-step kt-2,
// before the barrier of k-step kt-1. When K % 128 == 64 the packed weights
// of the last k-step's two missing slices are zero, so the (clamped, stale)
// activation chunks there add nothing: every k-step runs all four slices.
// STAMP: thread 0 of workgroup b writes g.stamps[4b ..] = wall clock at the
// start, after the k-loop and at the end, and shader-clock cycles from start
// to end (measurement only: the product path is STAMP = false).
template <int BM, bool TAIL, bool STAMP = false>
__global__ void __launch_bounds__(256) w8p_kernel(const GemmArgs g) {
  constexpr int S = 4, FM = BM / 32, FN = 2;
  constexpr int AST = BM * 128;        // bytes per A stage
  constexpr int NA = BM / 32;          // A direct loads per wave per k-step (8 rows of 128 B each)
  constexpr int NB = FN * 4;           // B loads per lane per k-step
  constexpr int EPI = 4 * 64 * EST * 4;  // four waves' epilogue strips (64 rows each)
  __shared__ __attribute__((aligned(16))) uint8_t ldsA[S * AST > EPI ? S * AST : EPI];

  unsigned long long sw0 = 0, sc0 = 0, sw1 = 0;
  if constexpr (STAMP) {
    sw0 = wall_clock64();
    sc0 = clock64();
  }
  auto stamp_end = [&]() {
    if constexpr (STAMP) {
      const unsigned long long sw2 = wall_clock64(), sc2 = clock64();
      if (threadIdx.x == 0) {
        unsigned long long* o = g.stamps + 4 * (long)blockIdx.x;
        o[0] = sw0;
        o[1] = sw1;
        o[2] = sw2;
        o[3] = sc2 - sc0;
      }
    }
  };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = g.M, N = g.N, K = g.K;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, tm, tn);
  const int m0 = tm * BM, n0 = tn * 256;
  const int ks = w8p_kpad(K) / 32;     // k-slices of the packed weights
  const int nk = ks / 4;               // k-steps

  // A: wave instruction i stages rows (wave * NA + i) * 8 .. +8; lane -> row r = row0 + lane / 8,
  // LDS position lane % 8 of row r holds chunk (lane % 8) ^ w8p_swz(r). Byte offsets from A
  // are 32-bit (the entry point checks M * K < 2^31).
  int chunk[2];  // chunk byte offset for even / odd i (bit 3 of the row)
#pragma unroll
  for (int e = 0; e < 2; ++e) chunk[e] = ((lane & 7) ^ ((lane >> 3) & 7) ^ e) << 4;
  uint32_t aoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i)
    aoff[i] = (uint32_t)(min(m0 + (wave * NA + i) * 8 + (lane >> 3), M - 1) * K + chunk[(wave * NA + i) & 1]);
  // B: n-tiles (n0 + 64 wave) / 32 + j of the packed weights (32-bit offsets: the
  // entry point checks the packed size < 2^31)
  const int ntiles = (N + 31) / 32;
  uint32_t boff[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) boff[j] = (uint32_t)(w8p_block(min((n0 + 64 * wave) / 32 + j, ntiles - 1), 0, ks) + 16 * lane);
  const uint8_t* Ab = reinterpret_cast<const uint8_t*>(g.A);
  const uint8_t* Bb = reinterpret_cast<const uint8_t*>(g.B);

  v4i rb[3][FN][4];
  // VMEM operation o (0 .. NB + NA - 1) of a k-step: o < NB loads B fragment
  // (slice o / FN, n-tile o % FN) of k-step kl into register set SETL; the
  // next NA are the direct loads of k-step kl's A rows into stage kst % 4.
  auto vmem_op = [&](auto oc, auto setlc, int kl, int kst) {
    constexpr int o = decltype(oc)::value, setl = decltype(setlc)::value;
    if constexpr (o < NB) {
      constexpr int q = o / FN, j = o % FN;
      rb[setl][j][q] = __builtin_bit_cast(v4i, ld16_so(Bb + (long)min(kl * 4 + q, ks - 1) * 1024, boff[j]));
    } else if constexpr (o < NB + NA) {
      constexpr int i = o - NB;
      uint8_t* st = ldsA + (kst & 3) * AST + (wave * NA + i) * 1024;
      if constexpr (TAIL) {  // chunk offsets clamped inside the row (a two-slice last k-step)
        const int c = chunk[(wave * NA + i) & 1];
        dma16_so(Ab, aoff[i] + (min(kl * 128 + c, K - 16) - c), st);
      } else {
        dma16_so(Ab + (long)kl * 128, aoff[i], st);
      }
    }
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

  const int frow = lane & 31, fh = lane >> 5;
  // A fragment of m-tile i, k-slice q (0..3) from stage st: row 32 i + lane % 32,
  // chunk 2 q + lane / 32, found at position chunk ^ w8p_swz(row)
  auto rdA = [&](int st, int i, int q) {
    const int r = 32 * i + frow;
    return *reinterpret_cast<const v4i*>(ldsA + st * AST + r * 128 + (((2 * q + fh) ^ w8p_swz(r)) << 4));
  };
  v4i fa[2][FM];

  // prologue: A0, B0, A1, B1; wait for A0, B0; read slice 0 of stage 0
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  auto load_kstep = [&](auto setc, int kl, int kst) {  // A rows first, then the B fragments
    static_for<NB, NB + NA>([&](auto oc) { vmem_op(oc, setc, kl, kst); });
    static_for<0, NB>([&](auto oc) { vmem_op(oc, setc, kl, kst); });
  };
  load_kstep(I0{}, 0, 0);
  load_kstep(I1{}, min(1, nk - 1), 1);
  vmwait<NA + NB>();
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) pin(rb[0][j][q]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = rdA(0, i, 0);

  // One k-step: 4 slices of 4 groups; group g of slice q reads two fragments
  // of the next slice, runs the MFMAs of m-tiles 2g, 2g+1 and issues VMEM
  // operation 4q + g of k-step kt+2 (so the 16 loads of a k-step are spread
  // over its MFMAs instead of queueing at the texture unit together). B(kt+2)
  // goes out in slices 0-1 and A(kt+2) in slices 2-3, so at the start of
  // slice 2 exactly the NB loads of B(kt+2) may still be in flight after
  // A(kt+1): vmcnt(NB), then the barrier publishes A(kt+1) before slice 3
  // reads its first fragments.
  static_assert(NB == 8 && NB + NA <= 16 && FM % 4 == 0, "one VMEM operation per group");
  int kt = 0;
  auto kstep = [&](auto setc, auto setnc, auto setlc) {
    constexpr int set = decltype(setc)::value, setn = decltype(setnc)::value;
    const int st = kt & 3, stn = (kt + 1) & 3;
    const int kl = min(kt + 2, nk - 1);
    static_for<0, 4>([&](auto qc) {
      constexpr int q = decltype(qc)::value, cb = q & 1, nbuf = cb ^ 1;
      if constexpr (q == 2) {
        vmwait<NB>();  // B(kt+1), A(kt+1) landed in this wave
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) pin(rb[setn][j][qq]);
        __syncthreads();  // ... and in every wave
      }
      static_for<0, 4>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        constexpr int i0 = g * (FM / 4);
#pragma unroll
        for (int ii = i0; ii < i0 + FM / 4; ++ii) fa[nbuf][ii] = q < 3 ? rdA(st, ii, q + 1) : rdA(stn, ii, 0);
#pragma unroll
        for (int ii = i0; ii < i0 + FM / 4; ++ii)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[ii][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cb][ii], rb[set][j][q], acc[ii][j], 0, 0, 0);
#pragma unroll
        for (int r = 0; r < FM / 4; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);
        }
        vmem_op(std::integral_constant<int, 4 * q + g>{}, setlc, kl, kt + 2);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };
  // B register sets rotate with period 3: B(kt) lives in set kt % 3
  for (; kt + 2 < nk; kt += 3) {
    kstep(I0{}, I1{}, I2{});
    ++kt;
    kstep(I1{}, I2{}, I0{});
    ++kt;
    kstep(I2{}, I0{}, I1{});
    kt -= 2;
  }
  if (kt < nk) {
    kstep(I0{}, I1{}, I2{});
    ++kt;
    if (kt < nk) kstep(I1{}, I2{}, I0{});
  }
  vmwait<0>();
  // the last k-steps' B loads (clamped, never used) must land before their
  // registers can be reused by the epilogue
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) pin(rb[s][j][q]);
  __syncthreads();  // every direct load landed and every fragment read before the strips reuse LDS
  if constexpr (STAMP) sw1 = wall_clock64();

  uint32_t* strip = reinterpret_cast<uint32_t*>(ldsA) + wave * (64 * EST);
  if constexpr (BM == 256) {
    // a tile wholly inside Y (N % 8 == 0 keeps the 16-byte stores aligned), Y only
    if (m0 + BM <= M && n0 + 256 <= N && !g.C && g.Y && (N & 7) == 0) {
      epilogue_w8_full(g, strip, acc, m0, n0 + 64 * wave);
      stamp_end();
      return;
    }
  }
#pragma unroll
  for (int c = 0; c < FM / 2; ++c) {
    // by value: a reference into acc would take its address and put it in scratch
    const v16i sub[2][FN] = {{acc[2 * c][0], acc[2 * c][1]}, {acc[2 * c + 1][0], acc[2 * c + 1][1]}};
    epilogue<0, 64, FN>(g, strip, sub, m0 + 64 * c, n0 + 64 * wave, nullptr);
  }
  stamp_end();
}

// ---- W8A8 on packed weights, persistent 128 x 320 tiles --------------------------
// One workgroup per CU runs a list of 128 x 320 output tiles through one
// continuous load pipeline: at M = 2048, N = 15360 that is 768 tiles, three
// per CU, so no CU idles in a last partial round (the 256 x 256 grid has 480
// tiles: a second round on 224 CUs). Wave w owns columns 80 w .. 80 w + 79 of
// a tile and all 128 rows: 8 x 5 tiles of v_mfma_i32_16x16x64_i8 with the
// weights as the first operand, so a lane's 4 accumulators are 4
// consecutive columns of one output row (D row = weight row n, D column =
// activation row m). Per 128-byte k-step a wave reads 16 KB of A from LDS
// and 10 KB of B from L2 for 80 MFMAs.
//  * A: 3-stage LDS ring of direct loads, 128-byte rows with the 16-byte
//    chunks at wq_swz_i positions.
//  * B: from the tile-32 packing, lane l takes the 16 bytes of row l % 16 of
//    its 16-column group and k-bytes 16 (l / 16) .. of the 64-byte slice
//    (the same k-bytes as its A fragment, so the dot products pair the same
//    k), two k-steps ahead in a 3-set register ring.
//  * Per k-step: slice 0 (40 MFMAs, one A fragment read and one load per 5)
//    issues 7 of the 14 loads of k-step + 2; vmcnt(7) then leaves only those
//    in flight, so A and B of k-step + 1 have landed, and one barrier
//    publishes A; slice 1 issues the other 7.
//  * Epilogue: at the end of a tile each lane forms Y = f16((f32(C) sa) sw)
//    (the reference's order, vk/coopgemm_w8a8.comp:35) from its accumulators
//    and writes it to an 82 KB LDS stage of the tile; the next tile's first
//    20 k-steps drain the stage to Y, one 16-byte nontemporal store per
//    thread per k-step, behind the MFMAs. Only the last tile's stores are
//    exposed. The tile's 128 row scales and 320 column scales arrive by
//    direct loads at its first k-step (4 KB block, double-buffered by tile
//    parity). With C the int32 accumulators are stored directly.
// Measured at M = 2048, N = 15360, K = 3840 against w8p_kernel on the same
// boxes: 2-3% faster. Every CU works to the end and the exposed epilogues
// fall from two of ~8 us to one of ~4.5 us (the Y stores issued during the
// k-loops cost ~8 us there), but a 16x16x64 int8 MFMA issues every ~20.6
// cycles in this loop (a copy without loads or LDS reads), against 34 for a
// 32x32x32 with twice the products, and the layout needs 16-column groups.
// Needs M % 128 == 0, N % 320 == 0, K % 64 == 0 with ceil(K / 128) % 3 == 0
// (a last k-step of two slices clamps its A chunks inside the row; its
// weights are zero padding), Y, and 16-byte aligned Y, sa and sw.
constexpr int WQ_BM = 128, WQ_BN = 320;
#define Q4_INLINE __attribute__((always_inline))
constexpr int WQ_YP = 656;  // staged Y row pitch in bytes: 640 + 16, so 16 rows of one 8-byte column hit distinct banks

// Position XOR of the 16-byte chunks of staged A row r: wq_swz_i((r >> 1) & 7),
// bits 1 and 2 of (r >> 1) & 7 swapped. A 16x16x64 fragment read serves
// lanes l and l + 32 together (rows r .. r + 7 at chunks c and c + 2, c % 4
// == 0); these positions put those 16 reads, and those of chunks c + 1 and
// c + 3, in 16 distinct 16-byte bank groups (measured: 10x fewer bank
// conflicts than w8p_swz, whose positions repeat for rows r and r ^ 2).
__device__ inline int wq_swz_i(int i) { return (i & 1) | ((i & 2) << 1) | ((i & 4) >> 1); }
template <bool TAIL, bool STAMP = false>
__global__ void __launch_bounds__(256) w8q_kernel(const GemmArgs g) {
  constexpr int S = 3, FR = WQ_BM / 16, FG = 5, NA = WQ_BM / 32, NB = 2 * FG;
  constexpr int AST = WQ_BM * 128;       // bytes per A stage
  constexpr int YCH = WQ_BN / 8;         // 16-byte Y chunks per tile row
  constexpr int DR = WQ_BM * YCH / 256;  // Y chunks per thread per tile
  static_assert(NB + NA == 14 && WQ_BM * YCH % 256 == 0, "7 loads per slice, whole drain rounds");
  __shared__ __attribute__((aligned(16))) uint8_t ldsA[S * AST];
  __shared__ __attribute__((aligned(16))) uint8_t ys[WQ_BM * WQ_YP];
  __shared__ __attribute__((aligned(16))) uint8_t scl[2][4096];

  unsigned long long sw0 = 0, sc0 = 0, sw1 = 0;
  if constexpr (STAMP) {
    sw0 = wall_clock64();
    sc0 = clock64();
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = g.M, N = g.N, K = g.K;
  const int ntm = M / WQ_BM, T = ntm * (N / WQ_BN);
  const int G = gridDim.x, w = blockIdx.x;
  // This workgroup's tiles first, first + tstride, ..: with both counts
  // multiples of 8, XCD x (workgroups w % 8 == x) takes the contiguous
  // eighth x of the tile order, so the 32 tiles an XCD runs together share
  // weight panels and activation rows in its L2. The order runs M fastest
  // within groups of 4 n-tiles, 4 n-tiles fastest within 8 m-tiles, so 32
  // consecutive tiles are 8 m-tiles x 4 n-tiles: 3.9 MB of A and 4.9 MB of
  // weights per XCD round at N = 15360, K = 3840, against 7.9 + 2.5 MB for
  // 16 x 2 (measured: 1.5% faster, 7% fewer k-loop cycles). Shapes without
  // whole groups take M fastest.
  int first, tstride, count;
  if (T % 8 == 0 && G % 8 == 0) {
    const int per = T / 8, gx = G / 8, i = w / 8;
    first = (w % 8) * per + i;
    tstride = gx;
    count = i < per ? (per - i + gx - 1) / gx : 0;
  } else {
    first = w;
    tstride = G;
    count = w < T ? (T - w + G - 1) / G : 0;
  }
  // The host launches at most T workgroups, so count >= 1; a workgroup
  // without tiles would leave before issuing any load.
  if (count == 0) return;
  const int ks = w8p_kpad(K) / 32, nk = ks / 4;
  const bool grp = ntm % 8 == 0 && (N / WQ_BN) % 4 == 0;
  auto tile_mn = [&](int j, int& m0, int& n0) Q4_INLINE {
    const int v = first + j * tstride;
    if (grp) {
      const int grp4 = v / (4 * ntm), r = v - grp4 * 4 * ntm;  // group of 4 n-tiles, tile within it
      m0 = (8 * (r >> 5) + ((r & 31) >> 2)) * WQ_BM;
      n0 = (4 * grp4 + (r & 3)) * WQ_BN;
    } else {
      m0 = (v % ntm) * WQ_BM;
      n0 = (v / ntm) * WQ_BN;
    }
  };

  // per-lane offsets, the same for every tile
  // A: wave instruction i stages tile row r = (wave NA + i) 8 + lane / 8, the
  // 16-byte chunk that belongs at LDS position lane % 8 (chunk = position ^
  // wq_swz_i((r >> 1) & 7), and (r >> 1) & 7 = ((wave NA + i) & 1) 4 + lane / 16)
  auto a_chunk = [&](int i) Q4_INLINE { return ((lane & 7) ^ wq_swz_i((((wave * NA + i) & 1) << 2) | (lane >> 4))) << 4; };
  uint32_t aoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) aoff[i] = (uint32_t)(((wave * NA + i) * 8 + (lane >> 3)) * K + a_chunk(i));
  uint32_t boff[FG];  // B: 16-column group cg of the wave, lane's 16 bytes in k-slice 2 s2 + lane / 32
#pragma unroll
  for (int cg = 0; cg < FG; ++cg) {
    const int nb = 80 * wave + 16 * cg;
    boff[cg] = (uint32_t)((nb >> 5) * ks * 1024 + (lane >> 5) * 1024 +
                          ((nb & 31) + (lane & 15) + 32 * ((lane >> 4) & 1)) * 16);
  }
  const uint8_t* Ab = reinterpret_cast<const uint8_t*>(g.A);
  const uint8_t* Bb = reinterpret_cast<const uint8_t*>(g.B);

  // load cursor: tile lj, k-step lk; past the last k-step it stays there
  // (the pipeline's two extra k-steps reload it, unused)
  int lj = 0, lk = 0, lm0, ln0;
  tile_mn(0, lm0, ln0);
  auto advance = [&]() Q4_INLINE {
    if (lk + 1 < nk) {
      ++lk;
    } else if (lj + 1 < count) {
      ++lj;
      lk = 0;
      tile_mn(lj, lm0, ln0);
    }
  };

  v4i bw[3][FG][2];
  // VMEM operation o (0 .. 13) of the cursor's k-step: o < NB loads B
  // fragment (slice o / FG, group o % FG) into register set SETL; the next NA
  // are the direct loads of its A rows into stage SETL.
  auto vmem_op = [&](auto oc, auto setlc) Q4_INLINE {
    constexpr int o = decltype(oc)::value, setl = decltype(setlc)::value;
    if constexpr (o < NB) {
      constexpr int s2 = o / FG, cg = o % FG;
      const uint8_t* base = Bb + ((long)(ln0 >> 5) * ks + lk * 4 + 2 * s2) * 1024;
      bw[setl][cg][s2] = __builtin_bit_cast(v4i, ld16_so(base, boff[cg]));
    } else {
      constexpr int i = o - NB;
      uint8_t* st = ldsA + setl * AST + (wave * NA + i) * 1024;
      const uint8_t* base = Ab + (long)lm0 * K;
      if constexpr (TAIL) {  // chunks past K clamped inside the row (their weights are zero)
        const int c = a_chunk(i);
        dma16_so(base, aoff[i] - c + min(lk * 128 + c, K - 16), st);
      } else {
        dma16_so(base + lk * 128, aoff[i], st);
      }
    }
  };

  // the scale block of tile j (4 KB): wave 0 puts sa[m0 .. m0 + 127] at
  // byte 0 (lanes 32-63 reload it into bytes 512-1023, unused), waves 1-2
  // put sw[n0 .. n0 + 319] (fp32 or fp16) at byte 1024 (lanes past its end
  // reload its last 16 bytes); wave 3 loads nothing
  auto scale_dma = [&](int j) Q4_INLINE {
    int m0, n0;
    tile_mn(j, m0, n0);
    int l = lane;
    asm volatile("" : "+v"(l));  // offsets formed here, not kept live (spilled) across the k-loop
    if (wave == 0) {
      dma16_so(g.sa + m0, (uint32_t)((l & 31) * 16), scl[j & 1]);
    } else if (wave < 3) {
      const int esz = g.sw_f16 ? 2 : 4;
      const uint32_t o = (uint32_t)min((wave - 1) * 1024 + l * 16, WQ_BN * esz - 16);
      dma16_so(reinterpret_cast<const uint8_t*>(g.sw) + (long)n0 * esz, o, scl[j & 1] + wave * 1024);
    }
  };

  v4i acc[FR][FG];  // set by the first k-step of each tile (C = 0)

  const int frow = lane & 15, fq = lane >> 4;
  // A fragment of row block rb, 64-byte slice s2 from stage st: row
  // 16 rb + lane % 16, chunk 4 s2 + lane / 16 at its wq_swz_i position
  auto rdA = [&](int st, int rb, int s2) Q4_INLINE {
    const int r = 16 * rb + frow;
    return *reinterpret_cast<const v4i*>(ldsA + st * AST + r * 128 + (((4 * s2 + fq) ^ wq_swz_i((r >> 1) & 7)) << 4));
  };
  v4i fa[2][FR];

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  auto load_kstep = [&](auto setc) Q4_INLINE {
    static_for<NB, NB + NA>([&](auto oc) { vmem_op(oc, setc); });
    static_for<0, NB>([&](auto oc) { vmem_op(oc, setc); });
    advance();
  };
  load_kstep(I0{});
  load_kstep(I1{});
  vmwait<NA + NB>();
#pragma unroll
  for (int cg = 0; cg < FG; ++cg) {
    pin(bw[0][cg][0]);
    pin(bw[0][cg][1]);
  }
  __syncthreads();
#pragma unroll
  for (int rb = 0; rb < FR; ++rb) fa[0][rb] = rdA(0, rb, 0);

  // Y drain: chunk tid + 256 d of the staged tile (m0, n0)
  auto drain = [&](int m0, int n0, int d) Q4_INLINE {
    int t = tid;
    asm volatile("" : "+v"(t));  // the address math stays here, not hoisted out of the loop into spills
    const int c = t + 256 * d, row = c / YCH, cc = c - row * YCH;
    const v4u v = *reinterpret_cast<const v4u*>(ys + row * WQ_YP + 16 * cc);
    __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(g.Y + (long)(m0 + row) * N + n0 + 8 * cc));
  };
  // tile j's accumulators -> staged Y (and C)
  auto convert = [&](int j, int m0, int n0) Q4_INLINE {
    const float* sab = reinterpret_cast<const float*>(scl[j & 1]);
    const uint8_t* swb = scl[j & 1] + 1024;
    float swv[FG][4];
    if (g.sw_f16) {
#pragma unroll
      for (int cg = 0; cg < FG; ++cg) {
        const v2u h = *reinterpret_cast<const v2u*>(swb + 2 * (80 * wave + 16 * cg + 4 * fq));
        swv[cg][0] = h2f((uint16_t)(h[0] & 0xFFFFu));
        swv[cg][1] = h2f((uint16_t)(h[0] >> 16));
        swv[cg][2] = h2f((uint16_t)(h[1] & 0xFFFFu));
        swv[cg][3] = h2f((uint16_t)(h[1] >> 16));
      }
    } else {
#pragma unroll
      for (int cg = 0; cg < FG; ++cg) {
        const float4 f = *reinterpret_cast<const float4*>(swb + 4 * (80 * wave + 16 * cg + 4 * fq));
        swv[cg][0] = f.x;
        swv[cg][1] = f.y;
        swv[cg][2] = f.z;
        swv[cg][3] = f.w;
      }
    }
    if (g.C) {
#pragma unroll
      for (int rb = 0; rb < FR; ++rb)
#pragma unroll
        for (int cg = 0; cg < FG; ++cg)
          *reinterpret_cast<v4i*>(g.C + (long)(m0 + 16 * rb + frow) * N + n0 + 80 * wave + 16 * cg + 4 * fq) =
              acc[rb][cg];
    }
#pragma unroll
    for (int rb = 0; rb < FR; ++rb) {
      const int ml = 16 * rb + frow;
      const float sav = sab[ml];
#pragma unroll
      for (int cg = 0; cg < FG; ++cg) {
        const int nl = 80 * wave + 16 * cg + 4 * fq;
        int c[4];
        __builtin_memcpy(c, &acc[rb][cg], 16);
        uint32_t hv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) hv[r] = f2h_after_f32(__fmul_rn(__fmul_rn((float)c[r], sav), swv[cg][r]));
        *reinterpret_cast<v2u*>(ys + ml * WQ_YP + 2 * nl) = v2u{hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16)};
      }
    }
  };

  int kt = 0, pm0 = 0, pn0 = 0;
  // One k-step of register set / stage SET (= k-step % 3; nk % 3 == 0, so
  // the rotation is the same in every tile). j: this tile; (pm0, pn0): the
  // previous tile, whose staged Y this tile's first DR k-steps drain.
  // FIRST: the tile's k-step 0, whose MFMAs start from C = 0 (no separate
  // zeroing, so the finished tile's accumulators and the new ones can share
  // registers) and which fetches the tile's scale block.
  auto kstep = [&](auto setc, auto firstc, int j) Q4_INLINE {
    constexpr int set = decltype(setc)::value, setn = (set + 1) % 3, setl = (set + 2) % 3;
    constexpr bool FIRST = decltype(firstc)::value;
    using IL = std::integral_constant<int, setl>;
    if constexpr (FIRST) scale_dma(j);  // lands with this k-step's A
    static_for<0, FR>([&](auto rc) {
      constexpr int rb = decltype(rc)::value;
      fa[1][rb] = rdA(set, rb, 1);
#pragma unroll
      for (int cg = 0; cg < FG; ++cg)
        acc[rb][cg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[set][cg][0], fa[0][rb], FIRST ? v4i{} : acc[rb][cg],
                                                            0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, FG, 0);
      if constexpr (rb < 7) vmem_op(std::integral_constant<int, rb>{}, IL{});
      __builtin_amdgcn_sched_barrier(0);
    });
    vmwait<7>();  // only slice 0's loads of k-step + 2 in flight: k-step + 1 landed in this wave
#pragma unroll
    for (int cg = 0; cg < FG; ++cg) {
      pin(bw[setn][cg][0]);
      pin(bw[setn][cg][1]);
    }
    __syncthreads();  // ... and in every wave
    static_for<0, FR>([&](auto rc) {
      constexpr int rb = decltype(rc)::value;
      fa[0][rb] = rdA(setn, rb, 0);
#pragma unroll
      for (int cg = 0; cg < FG; ++cg)
        acc[rb][cg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[set][cg][1], fa[1][rb], acc[rb][cg], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, FG, 0);
      if constexpr (rb < 7) vmem_op(std::integral_constant<int, 7 + rb>{}, IL{});
      __builtin_amdgcn_sched_barrier(0);
    });
    advance();
    if (j > 0 && kt < DR) drain(pm0, pn0, kt);
    ++kt;
  };
  using F1 = std::true_type;
  using F0 = std::false_type;
  for (int j = 0; j < count; ++j) {
    kt = 0;
    kstep(I0{}, F1{}, j);
    kstep(I1{}, F0{}, j);
    kstep(I2{}, F0{}, j);
    while (kt < nk) {
      kstep(I0{}, F0{}, j);
      kstep(I1{}, F0{}, j);
      kstep(I2{}, F0{}, j);
    }
    int cm0, cn0;
    tile_mn(j, cm0, cn0);
    const bool last = j + 1 == count;
    if (last) {
      vmwait<0>();  // the unused reloads, before their registers are reused
#pragma unroll
      for (int s = 0; s < 3; ++s)
#pragma unroll
        for (int cg = 0; cg < FG; ++cg) {
          pin(bw[s][cg][0]);
          pin(bw[s][cg][1]);
        }
      if constexpr (STAMP) sw1 = wall_clock64();
    }
    if (j > 0 && nk <= DR) {
      // a short tile: the rest of the previous tile's stage, then a barrier
      // before the stage is overwritten
      for (int d = nk; d < DR; ++d) drain(pm0, pn0, d);
      __syncthreads();
    }
    convert(j, cm0, cn0);
    if (last) {
      __syncthreads();
#pragma unroll 4
      for (int d = 0; d < DR; ++d) drain(cm0, cn0, d);
    }
    pm0 = cm0;
    pn0 = cn0;
  }
  if constexpr (STAMP) {
    const unsigned long long sw2 = wall_clock64(), sc2 = clock64();
    if (threadIdx.x == 0) {
      unsigned long long* o = g.stamps + 4 * (long)blockIdx.x;
      o[0] = sw0;
      o[1] = sw1;
      o[2] = sw2;
      o[3] = sc2 - sc0;
    }
  }
}

// ---- W4A16, waves split along N -------------------------------------------------
// BM x 256 tile, K step 64 (128 bytes of f16 A = two int4 blocks). Wave w owns
// columns n0 + 64w .. +64 and all BM rows: (BM/32) x 2 tiles of
// v_mfma_f32_32x32x16_f16, fp32 accumulate. A: 4-stage LDS ring of direct
// loads (128-byte rows, chunks swizzled by w8p_swz). B: each lane's
// half-units (8 bytes: words 2h, 2h+1 of the unit of its row and block,
// h = lane / 32) and block scales for the wave's 2 n-tiles x 2 blocks are
// loaded two k-steps ahead into a 3-set register ring and dequantized to f16
// fragments slice by slice (f16((q - 8) * s), one RNE multiply, as
// vk/coopgemm_i4h.comp:24). In k-slice q = 2bb + s (block bb of the k-step)
// lane half h multiplies A chunk 4bb + 2h + s (k = 32bb + 16h + 8s .. +8 of
// the step) by word 2h + s of its unit, the same k: the k order inside an
// MFMA is permuted identically for A and B. The schedule is w8p_kernel's:
// one VMEM operation per group of MFMAs (B(kt+2) in slices 0-1, A(kt+2) in
// slices 2-3), vmcnt(NB) + barrier at the start of slice 2. An odd block
// count leaves a last k-step with one block: the other block's scales read
// as zero, and its (clamped, stale) A chunks add nothing. With split > 1,
// blockIdx.y selects a contiguous range of k-steps and fp32 partials go to P.
// KG = 2 runs two groups of 4 waves (512 threads, two waves per SIMD, each
// with its own A ring) over the two halves of the workgroup's k-steps: one
// wave per SIMD is bound by its own instruction issue (dequant, A reads,
// addresses between the MFMAs), and a second wave issues while the first
// one's MFMAs run. Both groups run the same number of k-steps (barriers stay
// paired): for an odd count the second group runs one k-step fewer and
// then joins the first group's last barrier without any MFMA, so no
// operand is multiplied that a one-group launch would not multiply (a
// surplus step on zero scales would turn an Inf in X into NaN). Group 1
// then hands its accumulators to group 0 through LDS, and group 0 adds them
// (acc0 + acc1) and runs the epilogue.
template <int BM, bool TAIL, int KG = 1>
__global__ void __launch_bounds__(256 * KG) w4p_kernel(const GemmArgs g, int split) {
  constexpr int S = 4, FM = BM / 32, FN = 2;
  constexpr int AST = BM * 128;      // bytes per A stage
  constexpr int NA = BM / 32;        // A direct loads per wave per k-step
  constexpr int NB = FN * 2 * 2;     // B loads per lane per k-step: n-tile x block x (half-unit, scale)
  constexpr int EPI = 4 * 64 * EST * 4;
  constexpr int RING = KG * S * AST;
  constexpr int XCH = KG > 1 ? 4 * FM * FN * 16 * 64 * 4 : 0;  // group 1's accumulators
  constexpr int LDSB = RING > EPI ? (RING > XCH ? RING : XCH) : (EPI > XCH ? EPI : XCH);
  static_assert(KG == 1 || (KG == 2 && BM == 128), "two k-groups at 128-row tiles");
  __shared__ __attribute__((aligned(16))) uint8_t ldsA[LDSB];

  // grp through readfirstlane: wave-uniform, so the group's k range stays in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3,
            grp = KG > 1 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;
  const int M = g.M, N = g.N, K = g.K;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, tm, tn);
  const int m0 = tm * BM, n0 = tn * 256;
  const int nblk = K / BLK;
  const int nk_all = (nblk + 1) / 2;
  const int kz = blockIdx.y;
  const int k_wg = (int)((long)kz * nk_all / split), nk_wg = (int)((long)(kz + 1) * nk_all / split) - k_wg;
  // this group's k-steps: [k_lo, k_lo + nk); group 0 runs nit = nk steps,
  // group 1 nk = nit or nit - 1 (the entry point gives KG = 2 workgroups at
  // least 2 k-steps, so nk >= 1)
  const int nit = KG > 1 ? (nk_wg + 1) / 2 : nk_wg;
  const int k_lo = k_wg + grp * nit, nk = grp ? nk_wg - nit : nit;
  const int h = lane >> 5;
  uint8_t* const ring = ldsA + grp * (S * AST);

  // A: as w8p_kernel, rows of 2K bytes (32-bit offsets: the entry point checks 2MK < 2^31)
  int chunk[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) chunk[e] = ((lane & 7) ^ ((lane >> 3) & 7) ^ e) << 4;
  uint32_t aoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i)
    aoff[i] = (uint32_t)((long)min(m0 + (wave * NA + i) * 8 + (lane >> 3), M - 1) * 2 * K + (long)k_lo * 128 +
                         chunk[(wave * NA + i) & 1]);
  // B: unit index of (row, block 0) for the lane's row of each n-tile
  uint32_t ubase[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int row = min(n0 + 64 * wave + 32 * j + (lane & 31), N - 1);
    ubase[j] = (uint32_t)panel_index(row, 0, nblk);
  }
  const uint8_t* Ab = reinterpret_cast<const uint8_t*>(g.A);
  const uint8_t* Bb = reinterpret_cast<const uint8_t*>(g.B);
  const uint8_t* Sb = reinterpret_cast<const uint8_t*>(g.bsc);
  uint32_t mlo = 0x64006400u, mhi = 0x54005400u;  // dequant_pair_f16's VGPR operands
  asm volatile("" : "+v"(mlo), "+v"(mhi));

  v2u ru[3][FN][2];        // [set][n-tile][block] half-units
  uint32_t rs[3][FN][2];   // [set][n-tile][block] scale bits
  // VMEM operation o of a k-step: o < NB loads (n-tile, block, half-unit or
  // scale) of k-step kl (relative to k_lo) into set SETL; then NA direct loads
  // of A into stage kst % 4.
  auto vmem_op = [&](auto oc, auto setlc, int kl, int kst) {
    constexpr int o = decltype(oc)::value, setl = decltype(setlc)::value;
    if constexpr (o < NB) {
      constexpr int j = o / 4, bb = (o / 2) % 2, kind = o % 2;
      const int blk = min(2 * (k_lo + kl) + bb, nblk - 1);
      if constexpr (kind == 0) ru[setl][j][bb] = ld8_so(Bb + (long)blk * PANEL * 16, ubase[j] * 16 + 8 * h);
      else rs[setl][j][bb] = ld2_so(Sb + (long)blk * PANEL * 2, ubase[j] * 2);
    } else if constexpr (o < NB + NA) {
      constexpr int i = o - NB;
      uint8_t* st = ring + (kst & 3) * AST + (wave * NA + i) * 1024;
      if constexpr (TAIL) {  // chunks past the row's end (a one-block last k-step) clamped inside the row
        const int c = chunk[(wave * NA + i) & 1];
        const int lim = 2 * K - 16 - k_lo * 128;  // last 16-byte chunk of the row, relative to k_lo
        dma16_so(Ab, aoff[i] + (min(kl * 128 + c, lim) - c), st);
      } else {
        dma16_so(Ab + (long)kl * 128, aoff[i], st);
      }
    }
  };

  v16f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

  const int frow = lane & 31;
  // A fragment of m-tile i, k-slice q = 2bb + s from stage st: chunk 4bb + 2h + s of row 32i + lane % 32
  auto rdA = [&](int st, int i, int q) {
    const int r = 32 * i + frow;
    const int c = 4 * (q >> 1) + 2 * h + (q & 1);
    return *reinterpret_cast<const v4i*>(ring + st * AST + r * 128 + ((c ^ w8p_swz(r)) << 4));
  };
  v4i fa[2][FM];

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  auto load_kstep = [&](auto setc, int kl, int kst) {  // A rows first, then B
    static_for<NB, NB + NA>([&](auto oc) { vmem_op(oc, setc, kl, kst); });
    static_for<0, NB>([&](auto oc) { vmem_op(oc, setc, kl, kst); });
  };
  load_kstep(I0{}, 0, 0);
  load_kstep(I1{}, min(1, nk - 1), 1);
  vmwait<NA + NB>();
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      pin(ru[0][j][bb]);
      pin(rs[0][j][bb]);
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = rdA(0, i, 0);

  // Word P of the B fragment of n-tile j for k-slice q = 2bb + s of the
  // k-step whose half-units sit in register set SET; zero scale for the
  // absent second block of an odd block count (half)
  auto bpair = [&](auto setc, int j, int q, bool half, auto pc) -> int {
    constexpr int set = decltype(setc)::value, P = decltype(pc)::value;
    const int bb = q >> 1;
    const uint16_t sbits = (bb == 1 && half) ? (uint16_t)0 : (uint16_t)rs[set][j][bb];
    const _Float16 sc = __builtin_bit_cast(_Float16, sbits);
    const v2h sv = {sc, sc};
    return (int)dequant_pair_f16<P>((q & 1) ? ru[set][j][bb].y : ru[set][j][bb].x, sv, mlo, mhi);
  };
  v4i fb[2][FN];  // [slice parity][n-tile]: slice q's fragments, built during slice q - 1
#pragma unroll
  for (int j = 0; j < FN; ++j)
    static_for<0, 4>([&](auto pc) { fb[0][j][decltype(pc)::value] = bpair(I0{}, j, 0, 2 * k_lo + 1 >= nblk, pc); });

  static_assert(NB == 8 && NB + NA <= 16 && FM % 4 == 0, "one VMEM operation per group");
  int kt = 0;
  auto kstep = [&](auto setc, auto setnc, auto setlc) {
    constexpr int set = decltype(setc)::value, setn = decltype(setnc)::value;
    const int st = kt & 3, stn = (kt + 1) & 3;
    const int kl = min(kt + 2, nk - 1);
    const bool half = 2 * (k_lo + kt) + 1 >= nblk, half_n = 2 * (k_lo + kt + 1) + 1 >= nblk;
    static_for<0, 4>([&](auto qc) {
      constexpr int q = decltype(qc)::value, cb = q & 1, nbuf = cb ^ 1;
      if constexpr (q == 2) {
        vmwait<NB>();  // B(kt+1), A(kt+1) landed in this wave
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int b2 = 0; b2 < 2; ++b2) {
            pin(ru[setn][j][b2]);
            pin(rs[setn][j][b2]);
          }
        __syncthreads();  // ... and in every wave
      }
      static_for<0, 4>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        constexpr int i0 = g * (FM / 4);
#pragma unroll
        for (int ii = i0; ii < i0 + FM / 4; ++ii) fa[nbuf][ii] = q < 3 ? rdA(st, ii, q + 1) : rdA(stn, ii, 0);
        // word g of the next slice's B fragments, while this slice's MFMAs
        // run: the dequant spreads evenly over the slice's MFMAs
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if constexpr (q < 3) fb[nbuf][j][g] = bpair(setc, j, q + 1, half, gc);
          else fb[nbuf][j][g] = bpair(setnc, j, 0, half_n, gc);
        }
#pragma unroll
        for (int ii = i0; ii < i0 + FM / 4; ++ii)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[ii][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, fa[cb][ii]),
                                                                __builtin_bit_cast(v8h, fb[cb][j]), acc[ii][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, FM / 4, 0);
#pragma unroll
        for (int r = 0; r < FM / 4 * FN; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 16 / FM, 0);
        }
        vmem_op(std::integral_constant<int, 4 * q + g>{}, setlc, kl, kt + 2);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };
  for (; kt + 2 < nk; kt += 3) {
    kstep(I0{}, I1{}, I2{});
    ++kt;
    kstep(I1{}, I2{}, I0{});
    ++kt;
    kstep(I2{}, I0{}, I1{});
    kt -= 2;
  }
  if (kt < nk) {
    kstep(I0{}, I1{}, I2{});
    ++kt;
    if (kt < nk) kstep(I1{}, I2{}, I0{});
  }
  if constexpr (KG > 1) {
    if (nk < nit) __syncthreads();  // group 1 of an odd count: group 0's last k-step barrier
  }
  vmwait<0>();
#pragma unroll
  for (int s3 = 0; s3 < 3; ++s3)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        pin(ru[s3][j][bb]);
        pin(rs[s3][j][bb]);
      }
  __syncthreads();  // every direct load landed and every fragment read before the strips reuse LDS

  if constexpr (KG > 1) {
    // group 1's accumulators to group 0: tile (i, j) of wave w, 16-byte piece
    // c, lane l at float ((((w * FM + i) * FN + j) * 4 + c) * 64 + l) * 4
    float* xch = reinterpret_cast<float*>(ldsA);
    if (grp) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const v4f t = {acc[i][j][4 * c], acc[i][j][4 * c + 1], acc[i][j][4 * c + 2], acc[i][j][4 * c + 3]};
            *reinterpret_cast<v4f*>(xch + ((((wave * FM + i) * FN + j) * 4 + c) * 64 + lane) * 4) = t;
          }
    }
    __syncthreads();
    if (!grp) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const v4f t = *reinterpret_cast<const v4f*>(xch + ((((wave * FM + i) * FN + j) * 4 + c) * 64 + lane) * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * c + e] += t[e];
          }
    }
    __syncthreads();  // the exchange is read before the strips reuse LDS
    if (grp) return;
  }

  uint32_t* strip = reinterpret_cast<uint32_t*>(ldsA) + wave * (64 * EST);
#pragma unroll
  for (int c = 0; c < FM / 2; ++c) {
    const v16f sub[2][FN] = {{acc[2 * c][0], acc[2 * c][1]}, {acc[2 * c + 1][0], acc[2 * c + 1][1]}};
    if (g.P)  // split-K partials (also at split 1 for the gated entry point)
      epilogue<2, 64, FN>(g, strip, sub, m0 + 64 * c, n0 + 64 * wave, g.P + (long)kz * M * N);
    else
      epilogue<1, 64, FN>(g, strip, sub, m0 + 64 * c, n0 + 64 * wave, nullptr);
  }
}

// ---- W4A16 / W4A8 ---------------------------------------------------------------
// BM x 256 tile, K step one 64-byte A row (32 f16 for W4A16, 64 int8 for
// W4A8). A: S-stage LDS ring of direct loads (k-step j + S goes into the
// stage k-step j used). B: each lane's half-units for its FN tiles, loaded
// three k-steps ahead into a 4-deep register ring, converted to fragments
// one k-step ahead.
//   W4A16, slice s (16 k), lane half h: B = dequant(word 2h + s of the unit
//     of block kt) = k 16h + 8s .. + 8; A = chunk 2h + s of the row.
//   W4A8, slice s (32 k = block 2kt + s), half h: B = requant(words 2h,
//     2h + 1 of that block's unit) = k 32s + 16h .. + 16; A = chunk 2s + h.
template <int OP, int BM>
__global__ void __launch_bounds__(256) w4_kernel(const GemmArgs g, int split) {
  constexpr bool F16 = (OP == OP_W4A16);
  constexpr int BN = 256, WM = BM / 2, WN = 128, FM = WM / 32, FN = 4;
  constexpr int S = BM == 128 ? 8 : 6;        // A ring stages
  constexpr int NA = BM / 64;                 // A direct loads per thread per k-step
  constexpr int NBLK = F16 ? 1 : 2;           // int4 blocks per k-step
  constexpr int NBR = 2 * NBLK * FN;          // B loads per thread per k-step (half-unit + scale per block per tile)
  constexpr int AST = BM * 64;
  constexpr int EPI = 4 * WM * EST * 4;
  constexpr int LA = S * AST > EPI ? S * AST : EPI;
  static_assert(S >= 5, "the wait counts assume A(j + 2) is issued before B(j + 1)");
  __shared__ __attribute__((aligned(16))) uint8_t ldsA[LA];
  typedef typename std::conditional<F16, v16f, v16i>::type acc_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = g.M, N = g.N, K = g.K;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nblk = K / BLK;
  const int nk_all = F16 ? nblk : nblk / 2;
  const int kz = blockIdx.y;
  const int k_lo = (int)((long)kz * nk_all / split), nk = (int)((long)(kz + 1) * nk_all / split) - k_lo;
  const long a_row_bytes = F16 ? 2L * K : (long)K;

  const uint8_t* asrc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = (wave * NA + i) * 16 + (lane >> 2);
    asrc[i] = reinterpret_cast<const uint8_t*>(g.A) + (long)min(m0 + r, M - 1) * a_row_bytes + (long)k_lo * 64 +
              (((lane & 3) ^ swz(r)) << 4);
  }
  // B: tile j covers rows n0 + wn * 128 + 32 j + lane % 32; lane half h = lane / 32
  const int h = lane >> 5;
  const uint8_t* Bu = reinterpret_cast<const uint8_t*>(g.B);
  long bidx[FN];  // panel index of (row, block k_lo * NBLK)
#pragma unroll
  for (int j = 0; j < FN; ++j) bidx[j] = panel_index(min(n0 + wn * WN + 32 * j + (lane & 31), N - 1), k_lo * NBLK, nblk);

  v2u ru[4][FN][NBLK];
  uint32_t rs[4][FN][NBLK];
#define W4_LOAD_B(set_, kt_)                                                                         \
  do {                                                                                               \
    const long bo_ = (long)min((kt_), nk - 1) * NBLK * PANEL;                                        \
    _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                   \
      _Pragma("unroll") for (int b = 0; b < NBLK; ++b) {                                             \
        const long ix_ = bidx[j] + bo_ + b * PANEL;                                                  \
        ru[set_][j][b] = ld8(Bu + ix_ * 16 + 8 * h);                                                 \
        rs[set_][j][b] = ld2(g.bsc + ix_);                                                           \
      }                                                                                              \
  } while (0)
#define W4_LOAD_A(kt_)                                                                               \
  do {                                                                                               \
    const long ko_ = (long)min((kt_), nk - 1) * 64;                                                  \
    uint8_t* st_ = ldsA + ((kt_) % S) * AST;                                                         \
    _Pragma("unroll") for (int i = 0; i < NA; ++i) dma16(asrc[i] + ko_, st_ + (wave * NA + i) * 1024); \
  } while (0)

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};

  const int frow = lane & 31;
  auto rdA = [&](int stage, int i, int s) {
    const int c = F16 ? 2 * h + s : 2 * s + h;
    return *reinterpret_cast<const v4i*>(ldsA + stage * AST + lds_off(wm * WM + 32 * i + frow, c));
  };
  v4i fa[2][2][FM], fb[2][2][FN];  // [buffer][k-slice][tile]
#define W4_MAKE_B(buf_, set_)                                                                        \
  do {                                                                                               \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                                 \
      pin(ru[set_][j][0]);                                                                           \
      pin(rs[set_][j][0]);                                                                           \
      if constexpr (F16) {                                                                           \
        const _Float16 s_ = __builtin_bit_cast(_Float16, (uint16_t)rs[set_][j][0]);                   \
        const v2h sv_ = {s_, s_};                                                                    \
        fb[buf_][0][j] = __builtin_bit_cast(v4i, dequant_word_f16(ru[set_][j][0].x, sv_));           \
        fb[buf_][1][j] = __builtin_bit_cast(v4i, dequant_word_f16(ru[set_][j][0].y, sv_));           \
      } else {                                                                                       \
        pin(ru[set_][j][NBLK - 1]);                                                                  \
        pin(rs[set_][j][NBLK - 1]);                                                                  \
        _Pragma("unroll") for (int b = 0; b < NBLK; ++b) fb[buf_][b][j] = __builtin_bit_cast(v4i,   \
            requant_words_i8(ru[set_][j][b].x, ru[set_][j][b].y, h2f((uint16_t)rs[set_][j][b])));      \
      }                                                                                              \
    }                                                                                                \
  } while (0)

  // prologue in the steady-state issue order: A0 .. A(S-4), [B0 A(S-3)], [B1 A(S-2)], [B2 A(S-1)]
#pragma unroll
  for (int s = 0; s < S - 3; ++s) W4_LOAD_A(s);
  W4_LOAD_B(0, 0);
  W4_LOAD_A(S - 3);
  W4_LOAD_B(1, 1);
  W4_LOAD_A(S - 2);
  W4_LOAD_B(2, 2);
  W4_LOAD_A(S - 1);
  vmwait<3 * NA + 2 * NBR>();  // B0 and A0 .. A(S-4) landed
  W4_MAKE_B(0, 0);
  __builtin_amdgcn_s_barrier();  // stages 0 and 1 visible
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[0][sl][i] = rdA(0, i, sl);
  lgkm0();
  __builtin_amdgcn_s_barrier();  // stage 0 read by every wave: the first k-step may refill it

  constexpr int NMF = 2 * FM * FN;
#define W4_KSTEP(cur, nxt, bset_load, bset_make)                                                     \
  do {                                                                                               \
    W4_LOAD_B(bset_load, kt + 3);                                                                    \
    W4_LOAD_A(kt + S);                                                                               \
    vmwait<3 * NA + 2 * NBR>(); /* B(kt + 1) landed, and A(kt + 2) before it */                      \
    const int st1 = (kt + 1) % S;                                                                    \
    _Pragma("unroll") for (int sl = 0; sl < 2; ++sl)                                                 \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) fa[nxt][sl][i] = rdA(st1, i, sl);               \
    W4_MAKE_B(nxt, bset_make);                                                                       \
    _Pragma("unroll") for (int sl = 0; sl < 2; ++sl)                                                 \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                 \
        _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                             \
          if constexpr (F16)                                                                         \
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, fa[cur][sl][i]), \
                          __builtin_bit_cast(v8h, fb[cur][sl][j]), acc[i][j], 0, 0, 0);              \
          else                                                                                       \
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][sl][i], fb[cur][sl][j], acc[i][j], 0, 0, 0); \
        }                                                                                            \
    if constexpr (F16) { /* W4A8 (not a throughput path) is left to the default scheduler */       \
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * FM, 0);                                        \
      _Pragma("unroll") for (int q = 0; q < NMF; ++q) {                                              \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);                                           \
      }                                                                                              \
    }                                                                                                \
    lgkm0();                                                                                         \
    __builtin_amdgcn_s_barrier(); /* k-step kt + 2 visible; stage kt free */                         \
  } while (0)
  // register ring: B(kt) in set kt % 4; fragment buffers alternate with kt % 2
  int kt = 0;
  for (; kt + 3 < nk; kt += 4) {
    W4_KSTEP(0, 1, 3, 1);
    ++kt;
    W4_KSTEP(1, 0, 0, 2);
    ++kt;
    W4_KSTEP(0, 1, 1, 3);
    ++kt;
    W4_KSTEP(1, 0, 2, 0);
    kt -= 3;
  }
  if (kt < nk) {
    W4_KSTEP(0, 1, 3, 1);
    ++kt;
    if (kt < nk) {
      W4_KSTEP(1, 0, 0, 2);
      ++kt;
      if (kt < nk) W4_KSTEP(0, 1, 1, 3);
    }
  }
#undef W4_KSTEP
#undef W4_LOAD_A
#undef W4_LOAD_B
#undef W4_MAKE_B
  vmwait<0>();
  // keep the last k-steps' (unused) B registers live until their loads landed:
  // otherwise the compiler may reuse them for epilogue addresses
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        pin(ru[s][j][b]);
        pin(rs[s][j][b]);
      }
  __builtin_amdgcn_s_barrier();  // every direct load landed before the strips reuse LDS

  uint32_t* strip = reinterpret_cast<uint32_t*>(ldsA) + wave * (WM * EST);
  if constexpr (F16) {
    if (split > 1)
      epilogue<2, WM>(g, strip, acc, m0 + wm * WM, n0 + wn * WN, g.P + (long)kz * M * N);
    else
      epilogue<1, WM>(g, strip, acc, m0 + wm * WM, n0 + wn * WN, nullptr);
  } else {
    epilogue<0, WM>(g, strip, acc, m0 + wm * WM, n0 + wn * WN, nullptr);
  }
}

// Y[i] = f16(sum over splits of P[s][i]) in split order (4 elements per thread).
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ P, uint16_t* __restrict__ Y,
                                                            long n, int split) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 3 < n && (n & 3) == 0) {  // 16-byte loads need 16-byte split strides
    v4f t = *reinterpret_cast<const v4f*>(P + i);
    for (int s = 1; s < split; ++s) t += *reinterpret_cast<const v4f*>(P + (long)s * n + i);
    *reinterpret_cast<ushort4*>(Y + i) = make_ushort4(f2h(t.x), f2h(t.y), f2h(t.z), f2h(t.w));
  } else {
    for (long e = i; e < min(i + 4, n); ++e) {
      float t = P[e];
      for (int s = 1; s < split; ++s) t += P[(long)s * n + e];
      Y[e] = f2h(t);
    }
  }
}

// Gate/up rows interleaved (row 2i gate i, 2i + 1 up i): Y[o] = f16(gelu(g)
// u) with g = f16(sum over splits of P[s][2o]), u = f16(... P[s][2o + 1]),
// split order: the separate gate and up GEMMs' fp16 outputs through
// gelumul_kernel (vk/gelumul.comp:7-8), bit for bit at the same split. An
// output row m holds P columns m N .. + N, so output o reads partial 2o. 4
// outputs per thread.
__global__ void __launch_bounds__(256) splitk_reduce_gated_kernel(const float* __restrict__ P,
                                                                  uint16_t* __restrict__ Y, long n, int split) {
  const long o = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (o >= n) return;
  const long np = 2 * n;  // partials per split
  auto act = [](float g, float u) {
    return f2h(__fmul_rn(gelu_tanh(h2f(f2h(g))), h2f(f2h(u))));
  };
  if (o + 3 < n && (np & 3) == 0) {  // 16-byte loads need 16-byte split strides
    v4f a = *reinterpret_cast<const v4f*>(P + 2 * o), b = *reinterpret_cast<const v4f*>(P + 2 * o + 4);
    for (int s = 1; s < split; ++s) {
      a += *reinterpret_cast<const v4f*>(P + (long)s * np + 2 * o);
      b += *reinterpret_cast<const v4f*>(P + (long)s * np + 2 * o + 4);
    }
    *reinterpret_cast<ushort4*>(Y + o) = make_ushort4(act(a.x, a.y), act(a.z, a.w), act(b.x, b.y), act(b.z, b.w));
  } else {
    for (long e = o; e < min(o + 4, n); ++e) {
      float gs = P[2 * e], us = P[2 * e + 1];
      for (int s = 1; s < split; ++s) {
        gs += P[(long)s * np + 2 * e];
        us += P[(long)s * np + 2 * e + 1];
      }
      Y[e] = act(gs, us);
    }
  }
}

// ---- per-row int8 activation quantizer (vk/cast_i8.comp) -----------------
template <int XT>
__global__ void __launch_bounds__(256) quant_act_kernel(const void* __restrict__ X, int K, int8_t* __restrict__ A,
                                                        float* __restrict__ sa) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  auto ld4 = [&](int i, float v[4]) {  // elements 4i..4i+3 of row m
    if constexpr (XT == Q4_DT_F16) {
      ushort4 hh = reinterpret_cast<const ushort4*>(reinterpret_cast<const uint16_t*>(X) + (long)m * K)[i];
      v[0] = h2f(hh.x); v[1] = h2f(hh.y); v[2] = h2f(hh.z); v[3] = h2f(hh.w);
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
  mx = reduce64<true>(mx);
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

// W4A8's int8 weights computed once: unit u (row n, block b) of the
// panel-64 words -> W8[n][32 b .. 32 b + 31] = the bytes requant_words_i8
// gives for that unit (the values w4_kernel forms on the fly, per M-tile).
__global__ void __launch_bounds__(256) w4a8_weights_kernel(const uint4* __restrict__ wq,
                                                           const uint16_t* __restrict__ ratio, int N, int K,
                                                           int8_t* __restrict__ W8) {
  const int nblk = K / BLK;
  const long u = (long)blockIdx.x * 256 + threadIdx.x;  // unit index over the rows' (row, block) pairs
  if (u >= (long)N * nblk) return;
  const int n = (int)(u / nblk), b = (int)(u % nblk);
  const long ix = panel_index(n, b, nblk);
  const uint4 w = wq[ix];
  const float r = h2f(ratio[ix]);
  const v4u lo = requant_words_i8(w.x, w.y, r), hi = requant_words_i8(w.z, w.w, r);
  uint4* dst = reinterpret_cast<uint4*>(W8 + (long)n * K + (long)b * BLK);
  dst[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  dst[1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
}

// ---- host-side launch policy ----------------------------------------------------
// 256 x 256 tiles when they give >= 256 workgroups (one per CU), else
// 128 x 256. W4A16 splits K until the grid has >= 240 workgroups, keeping
// >= 8 k-steps of 64 per split, when a workspace for the partials is
// available. Measured on MI355X at M = 128 and 512 over the prefill shapes:
// the per-launch time falls with the split until the grid is about one
// workgroup per CU (k/v at M = 128: 25 -> 20 us; 512 rows: 23 -> 16 us)
// and then rises with the partials' traffic; the o projection (K 4096) at
// 8 splits instead of 16 (half the partials) took the 128-token prefill
// chunk from 8.20 to 7.97 ms.
static int tiles(int M, int N, int BM) { return ceil_div(M, BM) * ceil_div(N, 256); }
static int pick_bm(int M, int N) { return tiles(M, N, 256) >= 256 ? 256 : 128; }

static int w4a16_split(int M, int N, int K) {
  const int t = tiles(M, N, pick_bm(M, N));
  const int nk = (K / 32 + 1) / 2;  // k-steps of 64
  int s = min(ceil_div(240, t), max(1, nk / 8));
  const int v = tune_value(Q4_TUNE_W4A16_SPLIT);  // tests and tuning sweeps
  if (v >= 1 && v <= nk) s = v;
  return s;
}

// k-groups per W4A16 workgroup: two at 128-row tiles when every split has
// at least 32 k-steps. Measured at M = 512: 62 against 65 us (N 15360, K
// 3840) and 69 against 73 us (N 3840, K 15360); at 15 k-steps per group the
// two are even, and below that the hand-over and the shorter loops lose.
static int w4a16_kgroups(int M, int N, int K, int split) {
  if (pick_bm(M, N) != 128) return 1;
  const int nk = (K / 32 + 1) / 2;
  int kg = nk / split >= 32 ? 2 : 1;
  const int v = tune_value(Q4_TUNE_W4A16_KG);  // tests and tuning sweeps: force one or two groups
  if (v == 1 || (v == 2 && nk / split >= 2)) kg = v;
  return kg;
}

template <int BM, int KG = 1>
static void launch_w4p(const GemmArgs& g, int split, hipStream_t st) {
  const dim3 grid(tiles(g.M, g.N, BM), split);
  if (g.K % 64) hipLaunchKernelGGL((w4p_kernel<BM, true, KG>), grid, dim3(256 * KG), 0, st, g, split);
  else hipLaunchKernelGGL((w4p_kernel<BM, false, KG>), grid, dim3(256 * KG), 0, st, g, split);
}

template <int OP, int BM>
static void launch_w4(const GemmArgs& g, int split, hipStream_t st) {
  hipLaunchKernelGGL((w4_kernel<OP, BM>), dim3(tiles(g.M, g.N, BM), split), dim3(256), 0, st, g, split);
}

size_t w4a16_partials_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32) return 0;
  return (size_t)w4a16_split(M, N, K) * M * N * sizeof(float);
}

int w4a16_partials(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M, int N, int K, void* ws,
                   size_t ws_bytes, hipStream_t st, int* split_out) {
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 32 == 0, "bad W4A16 shape M=%d N=%d K=%d (K must be a multiple of 32)", M,
         N, K);
  Q4_ARG(X && wq && sc16 && ws, "null pointer");
  Q4_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)wq & 15) == 0 && ((uintptr_t)ws & 15) == 0,
         "X, wq and the workspace must be 16-byte aligned");
  const int split = w4a16_split(M, N, K);
  Q4_ARG(ws_bytes >= w4a16_partials_bytes(M, N, K), "W4A16 partials workspace too small: %zu < %zu bytes", ws_bytes,
         w4a16_partials_bytes(M, N, K));
  Q4_ARG(2L * M * K < (1L << 31) && (long)pad_rows(N) * (K / BLK) * 16 < (1L << 31),
         "W4A16 needs X and the int4 weights under 2 GiB (32-bit offsets)");
  GemmArgs g{X, wq, sc16, nullptr, nullptr, 0, nullptr, nullptr, reinterpret_cast<float*>(ws), M, N, K};
  if (pick_bm(M, N) == 256)
    launch_w4p<256>(g, split, st);
  else if (w4a16_kgroups(M, N, K, split) == 2)
    launch_w4p<128, 2>(g, split, st);
  else
    launch_w4p<128>(g, split, st);
  Q4_LAUNCHED("gemm_w4a16 (partials)");
  *split_out = split;
  return Q4_OK;
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
  Q4_ARG((((uintptr_t)Y | (uintptr_t)C) & 15) == 0, "Y and C must be 16-byte aligned (vector stores)");
  GemmArgs g{A, W8, nullptr, sa, sw, sw_dtype == Q4_DT_F16, Y, C, nullptr, M, N, K};
  if (pick_bm(M, N) == 256)
    hipLaunchKernelGGL(w8a8_kernel<256>, dim3(tiles(M, N, 256)), dim3(256), 0, as_stream(stream), g);
  else
    hipLaunchKernelGGL(w8a8_kernel<128>, dim3(tiles(M, N, 128)), dim3(256), 0, as_stream(stream), g);
  Q4_LAUNCHED("gemm_w8a8");
  return Q4_OK;
}

size_t q4_w8_packed_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) return 0;
  return (size_t)ceil_div(N, 32) * 32 * w8p_kpad(K);
}

int q4_w4a8_weights(const uint32_t* wq, const uint16_t* ratio, int N, int K, int8_t* W8, void* stream) {
  clear_error();
  Q4_ARG(N > 0 && K > 0 && K % 32 == 0, "bad W4A8 weight shape N=%d K=%d (K must be a multiple of 32)", N, K);
  Q4_ARG(wq && ratio && W8, "null pointer");
  Q4_ARG(((uintptr_t)wq & 15) == 0 && ((uintptr_t)W8 & 15) == 0, "wq and W8 must be 16-byte aligned");
  const long units = (long)N * (K / BLK);
  hipLaunchKernelGGL(w4a8_weights_kernel, dim3((unsigned)ceil_div(units, 256)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4*>(wq), ratio, N, K, W8);
  Q4_LAUNCHED("w4a8_weights");
  return Q4_OK;
}

int q4_w8_pack(const int8_t* W8, int N, int K, int8_t* W8p, void* stream) {
  clear_error();
  Q4_ARG(N > 0 && K > 0 && K % 32 == 0, "bad W8 shape N=%d K=%d (K must be a multiple of 32)", N, K);
  Q4_ARG(W8 && W8p, "null pointer");
  Q4_ARG(((uintptr_t)W8 & 15) == 0 && ((uintptr_t)W8p & 15) == 0, "W8 and W8p must be 16-byte aligned");
  const long chunks = (long)q4_w8_packed_bytes(N, K) / 16;
  hipLaunchKernelGGL(w8_pack_kernel, dim3(ceil_div(chunks, 256)), dim3(256), 0, as_stream(stream), W8, N, K, W8p,
                     chunks);
  Q4_LAUNCHED("w8_pack");
  return Q4_OK;
}

// Persistent 128 x 320 tiles (w8q_kernel) when the shape tiles exactly into
// more tiles than there are CUs, with k-steps (K / 128, rounded up) a
// multiple of 3: 0 when the 256-row kernel runs, else the grid (at most one
// workgroup per CU). Measured against the 256-row kernel (K = 3840, HIP
// events, rotating weights): 384 tiles 66.5 against 74.9 us, 512 tiles 71.3
// against 99.9, 768 tiles 109.9 against 112.8, 1536 tiles 201.1 against
// 220.7; with 192 tiles (2048 x 3840 x 15360) 118.5 against 113.2, so fewer
// tiles than CUs keep the 256-row kernel. Plan override Q4_TUNE_W8A8_TILES.
// The caller also needs Y and 16-byte aligned Y, sa and sw.
static int w8q_grid(int M, int N, int K) {
  if (M % WQ_BM || N % WQ_BN || K <= 0 || K % 64 || (w8p_kpad(K) / 128) % 3) return 0;
  const int t = (M / WQ_BM) * (N / WQ_BN);
  const int v = tune_value(Q4_TUNE_W8A8_TILES);
  if (v == 0 || (v != 1 && t <= 256)) return 0;
  return min(t, 256);
}

static int gemm_w8a8_packed(const int8_t* A, const int8_t* W8p, const float* sa, const void* sw, int sw_dtype,
                            uint16_t* Y, int32_t* C, int M, int N, int K, unsigned long long* stamps,
                            size_t stamps_bytes, void* stream) {
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 64 == 0, "bad W8A8 shape M=%d N=%d K=%d (K must be a multiple of 64)", M, N,
         K);
  Q4_ARG((long)127 * 127 * K < (1L << 31), "K=%d overflows the int32 accumulator", K);
  Q4_ARG(A && W8p && (Y || C), "null pointer");
  Q4_ARG(!Y || (sa && sw), "Y needs sa and sw");
  Q4_ARG(sw_dtype == Q4_DT_F32 || sw_dtype == Q4_DT_F16, "bad sw dtype %d", sw_dtype);
  Q4_ARG(((uintptr_t)A & 15) == 0 && ((uintptr_t)W8p & 15) == 0, "A and W8p must be 16-byte aligned");
  Q4_ARG((((uintptr_t)Y | (uintptr_t)C) & 15) == 0, "Y and C must be 16-byte aligned (vector stores)");
  Q4_ARG((long)M * K < (1L << 31) && (long)q4_w8_packed_bytes(N, K) < (1L << 31),
         "packed W8A8 needs M*K and the packed weights under 2 GiB (32-bit offsets)");
  const int bm = pick_bm(M, N);
  const bool aligned16 = Y && (((uintptr_t)Y | (uintptr_t)sa | (uintptr_t)sw) & 15) == 0;
  const int wq = aligned16 ? w8q_grid(M, N, K) : 0;
  const int wgs = wq ? wq : tiles(M, N, bm);
  if (stamps) Q4_ARG(stamps_bytes >= (size_t)wgs * 32 && ((uintptr_t)stamps & 7) == 0,
                     "stamps need 4 aligned 8-byte words per workgroup (%d workgroups)", wgs);
  GemmArgs g{A, W8p, nullptr, sa, sw, sw_dtype == Q4_DT_F16, Y, C, nullptr, M, N, K, stamps};
  const bool tail = K % 128 != 0;
  const hipStream_t st = as_stream(stream);
  void (*fn)(const GemmArgs);
  if (wq) {
    fn = stamps ? (tail ? w8q_kernel<true, true> : w8q_kernel<false, true>)
                : (tail ? w8q_kernel<true> : w8q_kernel<false>);
  } else if (bm == 256) {
    fn = stamps ? (tail ? w8p_kernel<256, true, true> : w8p_kernel<256, false, true>)
                : (tail ? w8p_kernel<256, true> : w8p_kernel<256, false>);
  } else {
    fn = stamps ? (tail ? w8p_kernel<128, true, true> : w8p_kernel<128, false, true>)
                : (tail ? w8p_kernel<128, true> : w8p_kernel<128, false>);
  }
  hipLaunchKernelGGL(fn, dim3(wgs), dim3(256), 0, st, g);
  Q4_LAUNCHED("gemm_w8a8_packed");
  return Q4_OK;
}

int q4_gemm_w8a8_packed(const int8_t* A, const int8_t* W8p, const float* sa, const void* sw, int sw_dtype,
                        uint16_t* Y, int32_t* C, int M, int N, int K, void* stream) {
  clear_error();
  return gemm_w8a8_packed(A, W8p, sa, sw, sw_dtype, Y, C, M, N, K, nullptr, 0, stream);
}

int q4_gemm_w8a8_packed_stamped(const int8_t* A, const int8_t* W8p, const float* sa, const void* sw, int sw_dtype,
                                uint16_t* Y, int32_t* C, int M, int N, int K, unsigned long long* stamps,
                                size_t stamps_bytes, void* stream) {
  clear_error();
  Q4_ARG(stamps, "null stamps");
  return gemm_w8a8_packed(A, W8p, sa, sw, sw_dtype, Y, C, M, N, K, stamps, stamps_bytes, stream);
}

size_t q4_gemm_w8a8_packed_workgroups(int M, int N, int K) {
  if (M <= 0 || N <= 0) return 0;
  const int wq = w8q_grid(M, N, K);
  return (size_t)(wq ? wq : tiles(M, N, pick_bm(M, N)));
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
  Q4_ARG((((uintptr_t)Y | (uintptr_t)C) & 15) == 0, "Y and C must be 16-byte aligned (vector stores)");
  GemmArgs g{A, wq, ratio, sa, sw, sw_dtype == Q4_DT_F16, Y, C, nullptr, M, N, K};
  // 128-row tiles only: with 256 rows the requant register ring does not fit
  // without spills, and a spill of a register whose load is still in flight
  // would store it before the data arrives
  launch_w4<OP_W4A8, 128>(g, 1, as_stream(stream));
  Q4_LAUNCHED("gemm_w4a8");
  return Q4_OK;
}

size_t q4_gemm_workspace_bytes(int op, int M, int N, int K) {
  if (op != Q4_OP_W4A16 || M <= 0 || N <= 0 || K <= 0 || K % 32) return 0;
  const int s = w4a16_split(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

int q4_gemm_w4a16_ws(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, uint16_t* Y, int M, int N, int K,
                     void* ws, size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(M > 0 && N > 0 && K > 0 && K % 32 == 0, "bad W4A16 shape M=%d N=%d K=%d (K must be a multiple of 32)", M, N,
         K);
  Q4_ARG(X && wq && sc16 && Y, "null pointer");
  Q4_ARG(((uintptr_t)X & 15) == 0 && ((uintptr_t)wq & 15) == 0, "X and wq must be 16-byte aligned");
  Q4_ARG(((uintptr_t)Y & 7) == 0, "Y must be 8-byte aligned");
  Q4_ARG(!ws || ((uintptr_t)ws & 15) == 0, "workspace must be 16-byte aligned");
  int split = w4a16_split(M, N, K);
  if (split > 1 && (!ws || ws_bytes < (size_t)split * M * N * sizeof(float))) split = 1;  // no room: one pass
  GemmArgs g{X, wq, sc16, nullptr, nullptr, 0, Y, nullptr, split > 1 ? reinterpret_cast<float*>(ws) : nullptr,
             M, N, K};
  Q4_ARG(2L * M * K < (1L << 31) && (long)pad_rows(N) * (K / BLK) * 16 < (1L << 31),
         "W4A16 needs X and the int4 weights under 2 GiB (32-bit offsets)");
  if (pick_bm(M, N) == 256)
    launch_w4p<256>(g, split, as_stream(stream));
  else if (w4a16_kgroups(M, N, K, split) == 2)
    launch_w4p<128, 2>(g, split, as_stream(stream));
  else
    launch_w4p<128>(g, split, as_stream(stream));
  Q4_LAUNCHED("gemm_w4a16");
  if (split > 1) {
    const long n = (long)M * N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(ceil_div(n, 1024)), dim3(256), 0, as_stream(stream), g.P, Y, n,
                       split);
    Q4_LAUNCHED("gemm_w4a16 split-K reduce");
  }
  return Q4_OK;
}

size_t q4_gemm_w4a16_gated_workspace_bytes(int M, int N, int K) {
  if (N % 2) return 0;
  return w4a16_partials_bytes(M, N, K);
}

int q4_gemm_w4a16_gated(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, uint16_t* Y, int M, int N,
                        int K, void* ws, size_t ws_bytes, void* stream) {
  clear_error();
  Q4_ARG(M > 0 && N > 0 && N % 2 == 0 && K > 0 && K % 32 == 0,
         "bad gated W4A16 shape M=%d N=%d K=%d (N even: interleaved gate/up rows; K a multiple of 32)", M, N, K);
  Q4_ARG(Y, "null pointer");
  Q4_ARG(((uintptr_t)Y & 7) == 0, "Y must be 8-byte aligned");
  int split = 0;
  if (int st = w4a16_partials(X, wq, sc16, M, N, K, ws, ws_bytes, as_stream(stream), &split)) return st;
  const long n = (long)M * (N / 2);
  hipLaunchKernelGGL(splitk_reduce_gated_kernel, dim3(ceil_div(n, 1024)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const float*>(ws), Y, n, split);
  Q4_LAUNCHED("gemm_w4a16_gated reduce");
  return Q4_OK;
}

int q4_gemm_w4a16(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, uint16_t* Y, int M, int N, int K,
                  void* stream) {
  return q4_gemm_w4a16_ws(X, wq, sc16, Y, M, N, K, nullptr, 0, stream);
}

}  // extern "C"
