// Batched-prefill attention for gfx950: every token of a chunk of M tokens
// (positions p0 .. p0+M-1, p0 read from device memory) attends the fp16 KV
// cache causally, after the chunk's own K/V were written.
//
// Replaces vk/pre_attn.comp (recorded per layer at src/vk_engine.py:417),
// which runs one workgroup per (head, token) and walks the keys one scalar
// dot product at a time; here the query rows of a KV head are tiled onto
// MFMAs:
//  * A workgroup owns 64 query rows of one KV head (row = token * grp +
//    query head within the group, so the rows share their K and V), in 4
//    row groups of 16, and one split of the cache slots (a multiple of 32
//    keys, long enough that the grid has about 256 workgroups: 128 keys for
//    a 1024-slot ring of 8 KV heads, 512 for 4096 keys of one KV head); the
//    grid covers the keys the caller bounds and splits past a workgroup's
//    last token exit at once, so the launch shape does not depend on p0
//    (graph replay). Head dims up to 256 take one wave per row group
//    (pre_attn_kernel); head dim 512 takes two, each holding half of the
//    head dims (pre_attn512_kernel).
//  * q prologue, in registers: lane (c, g) of a row group holds row c,
//    elements 32j + 8g .. 32j + 8g + 7 of every 32-element chunk j; the
//    RoPE partner of element e (e +- hd/2) is in the same lane, and the
//    row's sum of squares needs two xor-shuffles. q is split into fp16
//    hi + lo parts (q = hi + lo to ~22 bits), so q . k is exact to fp32
//    rounding with fp16 MFMAs (two per k-step; k is fp16 in the cache).
//  * Per 32-key tile the workgroup stages K row-major ([key][hd], rows
//    padded by 16 bytes) and V transposed ([hd][key], pairs of keys per
//    32-bit word) in LDS. Scores S^T = K q^T: one v_mfma_f32_16x16x32_f16
//    pair per 16 keys x 16 rows x 32 elements; lane (c, g) gets keys
//    4g .. 4g+3 of row c in each 16-key subtile. Masked keys (past the
//    row's length, or in a ring slot a later token of the chunk now holds:
//    slot s holds position last - ((last - s) mod window) once the chunk's
//    last position is written, vk/pre_attn.comp:40) are -inf. Online
//    softmax per row over the tile (xor-shuffles across the 4 lanes of a
//    row), then O^T += V^T P^T with one v_mfma_f32_16x16x32_f16 per 16
//    output dims: the B operand is the score layout of both subtiles (P
//    rounded to fp16), the A operand 16 bytes of the transposed V, whose
//    rows keep their keys in that order (pv_slot).
//  * Each workgroup writes its rows' (max, sum, unnormalised accumulator)
//    for its split; q4_pre_attn's second kernel merges the splits.
#include "q4mi_common.h"

namespace q4 {

constexpr int PA_WAVES = 4;             // row groups of 16 rows per workgroup
constexpr int PA_THREADS = 64 * PA_WAVES;
constexpr int PA_ROWS = 16 * PA_WAVES;  // query rows per workgroup
constexpr int PA_KT = 32;               // keys per LDS tile
constexpr int PA_TARGET_WGS = 256;      // workgroups the split length aims for (one per CU)
constexpr float PA_EPS = 1e-6f;

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// 8 consecutive elements at element index i (a multiple of 8) of fp32 or
// fp16 data, as fp32, in 16-byte loads.
template <int QT>
__device__ inline void ld8f(const void* q, long i, float* out) {
  if constexpr (QT == Q4_DT_F16) {
    const v4u u = *reinterpret_cast<const v4u*>(reinterpret_cast<const uint16_t*>(q) + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      out[2 * k] = h2f((uint16_t)(u[k] & 0xFFFFu));
      out[2 * k + 1] = h2f((uint16_t)(u[k] >> 16));
    }
  } else {
    const v4f a = *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(q) + i);
    const v4f b = *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(q) + i + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      out[k] = a[k];
      out[4 + k] = b[k];
    }
  }
}

// Workspace row of (token m, head h), split ks: [max, sum, -, -, acc[HD]].
__device__ inline long pa_ws_index(int m, int h, int nH, int ks, int nsplit, int hd) {
  return (((long)m * nH + h) * nsplit + ks) * (hd + 4);
}

// Position of key k of a 32-key tile in its V^T row: k = 16 st + 4 g + e
// sits at 8 g + 4 st + e, so lane (c, g)'s weights of both 16-key subtiles
// are the 8 consecutive k of one 16x16x32 MFMA.
__device__ inline int pv_slot(int k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }

// Lane (c, g)'s part of its query row (q element offset qb; cs, sn: the
// row's cos and sin): elements 32 j + 8 g .. + 7 of every chunk j after the
// rms norm with qnw and RoPE, in fp32.
template <int HD, int QT>
__device__ __forceinline__ void pa_q_row(const void* __restrict__ qin, long qb, const float* __restrict__ qnw,
                                         const float* __restrict__ cs, const float* __restrict__ sn, int g,
                                         float (&qf)[HD / 32][8]) {
  constexpr int NCH = HD / 32;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    ld8f<QT>(qin, qb + 32 * j + 8 * g, qf[j]);
#pragma unroll
    for (int u = 0; u < 8; ++u) ss = fmaf(qf[j][u], qf[j][u], ss);
  }
  ss = slot_reduce<16>(ss);
  const float inv = 1.0f / sqrtf(ss / (float)HD + PA_EPS);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    float w[8];
    ld8f<Q4_DT_F32>(qnw, 32 * j + 8 * g, w);
#pragma unroll
    for (int u = 0; u < 8; ++u) qf[j][u] = __fmul_rn(__fmul_rn(qf[j][u], inv), w[u]);
  }
#pragma unroll
  for (int j = 0; j < NCH / 2; ++j) {
    const int e = 32 * j + 8 * g, e2 = e + HD / 2;
    float c1[8], s1[8], c2[8], s2[8];
    ld8f<Q4_DT_F32>(cs, e, c1);
    ld8f<Q4_DT_F32>(sn, e, s1);
    ld8f<Q4_DT_F32>(cs, e2, c2);
    ld8f<Q4_DT_F32>(sn, e2, s2);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float a = qf[j][u], b = qf[j + NCH / 2][u];
      const float ra = __fadd_rn(__fmul_rn(a, c1[u]), __fmul_rn(-b, s1[u]));
      const float rb = __fadd_rn(__fmul_rn(b, c2[u]), __fmul_rn(a, s2[u]));
      qf[j][u] = ra;
      qf[j + NCH / 2][u] = rb;
    }
  }
}

// fp16 hi + lo parts of chunks j0 .. j0 + N - 1 of a lane's row.
template <int N, int NCH>
__device__ __forceinline__ void pa_q_split(const float (&qf)[NCH][8], int j0, v8h* qh, v8h* ql) {
#pragma unroll
  for (int j = 0; j < N; ++j)
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const _Float16 hi = (_Float16)qf[j0 + j][u];
      qh[j][u] = hi;
      ql[j][u] = (_Float16)(qf[j0 + j][u] - (float)hi);
    }
}

// The keys of slots t0 .. t0 + 31 for row (T: its length, pos: its
// position): -inf where masked (past the split's end kend, past the row's
// length, or a ring slot a later token holds; rt = (last - t0) mod window).
__device__ __forceinline__ void pa_mask(const v4f* sp, float (*sc)[4], int t0, int g, int kend, int T, int window,
                                        int rt, uint32_t last, uint32_t pos) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const v4f s = sp[st];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * st + 4 * g + e, slot = t0 + i;
      bool ok = slot < kend && slot < T;
      if (window > 0) {
        const int r = rt - i;  // (last - slot) mod window, for i < window
        ok = ok && (long)last - (r >= 0 ? r : r + window) <= (long)pos;
      }
      sc[st][e] = ok ? s[e] : -INFINITY;
    }
  }
}

// Keys below the returned slot are live for every row of a workgroup
// (rows r0 ..): without a ring a row's keys are the slots below its length,
// and the workgroup's first token has the shortest; with a ring, none is
// taken as known.
__device__ inline int pa_full_keys(int k0, int kend, int r0, int grp, uint32_t p0, int window, int stride) {
  return window > 0 ? k0 : min(kend, att_len(p0 + (uint32_t)(r0 / grp), window, stride));
}

// Online softmax of a lane's 8 masked scores of the tile (row maximum and
// sum across the row's 4 lanes) and the rescale of its accumulators: P in
// fp16 for the V product, the running (mrun, lrun) updated.
template <int NDT>
__device__ __forceinline__ v8h pa_softmax(const float (*sc)[4], float& mrun, float& lrun, v4f* oacc) {
  float tmax = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, sc[st][e]);
  tmax = slot_reduce<16, true>(tmax);
  const float mnew = fmaxf(mrun, tmax);
  const bool any = mnew != -INFINITY;
  // v_exp_f32-based exponentials (relative error ~1e-6): the weights are
  // rounded to fp16 (2^-11) before use, and the reference's GLSL exp() is
  // itself approximate; 8 fewer VALU operations per score
  const float corr = any ? __expf(mrun - mnew) : 1.0f;
  float psum = 0.0f;
  v8h pb;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the weights the V product uses are the fp16-rounded ones: the sum
      // is taken over the same values, so the output stays a weighted mean
      // of V rows (the row maximum's weight, 1, is exact)
      const _Float16 p = (_Float16)(any ? __expf(sc[st][e] - mnew) : 0.0f);
      psum += (float)p;
      pb[4 * st + e] = p;
    }
  psum = slot_reduce<16>(psum);
  lrun = fmaf(lrun, corr, psum);
  mrun = mnew;
#pragma unroll
  for (int d = 0; d < NDT; ++d)
#pragma unroll
    for (int e = 0; e < 4; ++e) oacc[d][e] *= corr;
  return pb;
}

// The 8 key-pair words of one 16-byte V chunk pair into the V^T tile:
// elements 8 ch + 2w, 8 ch + 2w + 1 of keys 2 pr (low half) and 2 pr + 1
// (high half), at the pair's pv_slot position of each row.
template <int VP>
__device__ __forceinline__ void pa_store_vpair(uint8_t* vsh, v4u a, v4u b, int ch, int pr) {
  const int wo = 2 * pv_slot(2 * pr);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    // (a & 0xFFFF) | (b << 16) and (a >> 16) | (b & 0xFFFF0000), one byte permute each
    *reinterpret_cast<uint32_t*>(vsh + (8 * ch + 2 * w) * VP + wo) = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);
    *reinterpret_cast<uint32_t*>(vsh + (8 * ch + 2 * w + 1) * VP + wo) = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);
  }
}

// Head dims 64 .. 256: one wave per row group (4 waves), K and V of the next
// tile loaded into registers one tile ahead and stored to LDS after the
// tile's first barrier.
template <int HD, int QT>
__global__ void __launch_bounds__(PA_THREADS)
pre_attn_kernel(const void* __restrict__ qin, int ldq, const float* __restrict__ qnw, const float* __restrict__ cosM,
                const float* __restrict__ sinM, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                int stride, int window, int grp, int nH, int M, const uint32_t* __restrict__ dyn,
                float* __restrict__ ws, int nsplit, int ksl) {
  constexpr int KT = PA_KT, NT = PA_THREADS;
  constexpr int NCH = HD / 32;        // 32-element chunks
  constexpr int NDT = HD / 16;        // 16-element output tiles
  constexpr int CPR = HD / 8;         // 16-byte chunks per K/V row
  constexpr int KP = HD * 2 + 16;     // K tile row pitch (bytes)
  constexpr int VP = KT * 2 + 8;      // V^T tile row pitch (bytes)
  constexpr int KITEMS = KT * CPR, VITEMS = (KT / 2) * CPR;  // 16-byte K chunks, V key-pair chunks per tile
  constexpr int KLD = (KITEMS + NT - 1) / NT, VLD = (VITEMS + NT - 1) / NT;
  static_assert(HD <= 256 && NCH % 2 == 0, "head dim");
  __shared__ __attribute__((aligned(16))) uint8_t ksh[KT * KP];
  __shared__ __attribute__((aligned(16))) uint8_t vsh[HD * VP];

  const int kvh = blockIdx.x, ks = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
  const uint32_t p0 = dyn[0];
  const int nrows = M * grp, r0 = blockIdx.y * PA_ROWS;
  const int mlast = (min(r0 + PA_ROWS, nrows) - 1) / grp;
  const int Tlast = att_len(p0 + (uint32_t)mlast, window, stride);
  const int k0 = ks * ksl;
  if (k0 >= Tlast) return;  // no row of this workgroup has keys in this split (uniform)
  const int kend = min(k0 + ksl, Tlast);
  const uint32_t last = p0 + (uint32_t)M - 1;  // the chunk's last position (all of its K/V are written)

  // ---- the next tile's K and V rows, loaded into registers one tile ahead.
  //      K chunks go to LDS row-major (lanes take consecutive chunks of a
  //      row); V chunks of key pairs (2 pr, 2 pr + 1) are interleaved into
  //      32-bit words of the transposed tile, lanes taking consecutive pairs
  //      so their LDS words are consecutive (no bank conflicts) ----
  v4u kr[KLD], va[VLD], vb[VLD];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int q = min(tid + NT * i, KITEMS - 1), key = q / CPR, ch = q % CPR;
      const int slot = min(t0 + key, stride - 1);
      kr[i] = *reinterpret_cast<const v4u*>(kc + ((long)kvh * stride + slot) * HD + ch * 8);
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int q = min(tid + NT * i, VITEMS - 1), pr = q % (KT / 2), ch = q / (KT / 2);
      const int s0 = min(t0 + 2 * pr, stride - 1), s1 = min(t0 + 2 * pr + 1, stride - 1);
      va[i] = *reinterpret_cast<const v4u*>(vc + ((long)kvh * stride + s0) * HD + ch * 8);
      vb[i] = *reinterpret_cast<const v4u*>(vc + ((long)kvh * stride + s1) * HD + ch * 8);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int q = tid + NT * i, key = q / CPR, ch = q % CPR;
      if (q < KITEMS) *reinterpret_cast<v4u*>(ksh + key * KP + ch * 16) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int q = tid + NT * i;
      if (q < VITEMS) pa_store_vpair<VP>(vsh, va[i], vb[i], q / (KT / 2), q % (KT / 2));
    }
  };
  load_tile(k0);  // in flight while q is prepared

  // ---- this lane's query row: q-norm, RoPE, hi/lo split ----
  const int R = r0 + 16 * wave + c;
  const bool live = R < nrows;
  const int m = live ? R / grp : 0;
  const int h = kvh * grp + (live ? R % grp : 0);
  const uint32_t pos = p0 + (uint32_t)m;
  const int T = att_len(pos, window, stride);
  v8h qh[NCH], ql[NCH];
  {
    float qf[NCH][8];
    pa_q_row<HD, QT>(qin, (long)m * ldq + (long)h * HD, qnw, cosM + (long)m * HD, sinM + (long)m * HD, g, qf);
    pa_q_split<NCH>(qf, 0, qh, ql);
  }

  v4f oacc[NDT];
#pragma unroll
  for (int d = 0; d < NDT; ++d) oacc[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = -INFINITY, lrun = 0.0f;
  const int kfull = pa_full_keys(k0, kend, r0, grp, p0, window, stride);

  for (int t0 = k0; t0 < kend; t0 += KT) {
    __syncthreads();  // every wave is done with the previous tile
    store_tile();
    __syncthreads();
    if (t0 + KT < kend) load_tile(t0 + KT);  // the next tile's loads run under this tile's math

    // ---- scores of the tile's keys for this lane's row: four independent
    //      MFMA chains (hi/lo x even/odd chunks) so consecutive MFMAs do not
    //      wait on each other's results ----
    // ring slots t0 + i hold position last - ((last - t0 - i) mod window):
    // one (uniform) division per tile
    const int rt = window > 0 ? (int)(((long)last - t0) % window) : 0;
    v4f sp[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      v4f s0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, s2 = s0, s3 = s0;
      const uint8_t* kr0 = ksh + (16 * st + c) * KP + g * 16;
#pragma unroll
      for (int j = 0; j < NCH; j += 2) {
        const v8h a0 = *reinterpret_cast<const v8h*>(kr0 + 4 * j * 16);
        const v8h a1 = *reinterpret_cast<const v8h*>(kr0 + (4 * j + 4) * 16);
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[j], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[j + 1], s1, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[j], s2, 0, 0, 0);
        s3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[j + 1], s3, 0, 0, 0);
      }
      sp[st] = (s0 + s1) + (s2 + s3);
    }
    float sc[2][4];
    if (t0 + KT <= kfull) {  // every key of the tile is live for every row of the workgroup (uniform)
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[st][e] = sp[st][e];
    } else {
      pa_mask(sp, sc, t0, g, kend, T, window, rt, last, pos);
    }
    const v8h pb = pa_softmax<NDT>(sc, mrun, lrun, oacc);
    // ---- O^T += V^T P^T, both subtiles in one K = 32 MFMA per output tile ----
#pragma unroll
    for (int d = 0; d < NDT; ++d) {
      const uint8_t* va8 = vsh + (16 * d + c) * VP + 16 * g;
      const v4h lo = *reinterpret_cast<const v4h*>(va8), hi = *reinterpret_cast<const v4h*>(va8 + 8);
      const v8h a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, pb, oacc[d], 0, 0, 0);
    }
  }

  // ---- this split's partial for the row ----
  if (!live) return;
  float* o = ws + pa_ws_index(m, h, nH, ks, nsplit, HD);
  if (g == 0) {
    o[0] = mrun;
    o[1] = lrun;
  }
#pragma unroll
  for (int d = 0; d < NDT; ++d) *reinterpret_cast<v4f*>(o + 4 + 16 * d + 4 * g) = oacc[d];
}

// Head dim 512 (Gemma's global layers: one KV head shared by all 16 query
// heads): two waves per row group, each holding q (hi + lo) for half of the
// head dims. Each computes the partial scores over its half and the pair adds
// the two halves through LDS (half 0 + half 1, the same bits in both
// waves); each then accumulates its half of the output dims. So q, the
// accumulators and the loads in flight fit two waves per SIMD (8 waves, 512
// threads) without spills, and no score is computed twice (a pair that
// computed the full scores in both waves took 137 us against 102 us for
// one wave per row group, 128 tokens x 16 heads over 4096 keys). Per 32-key
// tile:
//  * K rows go from global memory straight into LDS (a 1 KB direct load
//    per key row, no registers), into one of two buffers: tile i + 1's rows
//    are loaded after tile i's score exchange and land while tile i's
//    softmax and V product run. V rows come through registers, loaded one
//    tile ahead right after the V^T store.
//  * Two barriers: (A) every wave's K rows and V registers of the tile have
//    landed and every wave is done with the previous tile; (B) the pair's
//    partial scores are exchanged (this also publishes the V^T tile).
//  * Row addresses advance by one tile away from the end of the cache, and
//    tiles whose keys are live for every row of the workgroup skip the mask.
// Measured on the workload above (kernel-only, same box): 77 us with one
// 16-key tile per three barriers and registers staging K; 68.5 us with
// 32-key tiles, K direct loads and the K = 32 V product; 63.7 us with the
// row address and mask changes; 58.5 us with the K rows loaded after the
// exchange instead of with the V rows (the tile's loads all at once held
// the score MFMAs back: 1.6k of ~7k cycles per tile). Not kept: the q
// prologue (~10 us of the span) done once per row by a separate launch
// (25 us for that launch), or reading qnw, cos and sin from LDS (67 us:
// one more barrier, spills); the V rows loaded after the exchange too
// (67 us: they no longer land before the next tile's store).
constexpr int PA512_THREADS = 512;
template <int QT>
__global__ void __launch_bounds__(PA512_THREADS)
pre_attn512_kernel(const void* __restrict__ qin, int ldq, const float* __restrict__ qnw,
                   const float* __restrict__ cosM, const float* __restrict__ sinM, const uint16_t* __restrict__ kc,
                   const uint16_t* __restrict__ vc, int stride, int window, int grp, int nH, int M,
                   const uint32_t* __restrict__ dyn, float* __restrict__ ws, int nsplit, int ksl) {
  constexpr int HD = 512, KT = PA_KT, DS = 2, WAVES = 8, NT = PA512_THREADS;
  constexpr int NCH = HD / 32;        // 32-element chunks
  constexpr int NQC = NCH / DS;       // chunks of this wave's QK
  constexpr int NDT = HD / 16 / DS;   // 16-element output tiles of this wave
  constexpr int CPR = HD / 8;         // 16-byte chunks per V row
  constexpr int KP = HD * 2 + 16;     // K tile row pitch (bytes)
  constexpr int VP = KT * 2 + 8;      // V^T tile row pitch (bytes)
  constexpr int VITEMS = (KT / 2) * CPR, VLD = VITEMS / NT;  // V key-pair chunks per tile, per thread
  constexpr int KPW = KT / WAVES;     // K rows each wave loads per tile
  static_assert(VITEMS % NT == 0 && KT % WAVES == 0 && NQC % 2 == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) uint8_t ksh[2][KT * KP];
  __shared__ __attribute__((aligned(16))) uint8_t vsh[HD * VP];
  __shared__ v4f xs[WAVES][2][64];  // each wave's partial scores of the tile

  const int kvh = blockIdx.x, ks = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
  const int rg = wave / DS, dp = wave % DS;  // row group, half of the head dims
  const uint32_t p0 = dyn[0];
  const int nrows = M * grp, r0 = blockIdx.y * PA_ROWS;
  const int mlast = (min(r0 + PA_ROWS, nrows) - 1) / grp;
  const int Tlast = att_len(p0 + (uint32_t)mlast, window, stride);
  const int k0 = ks * ksl;
  if (k0 >= Tlast) return;  // uniform
  const int kend = min(k0 + ksl, Tlast);
  const uint32_t last = p0 + (uint32_t)M - 1;

  // K rows of tile t0 -> ksh[b] (wave w loads rows w KPW .. + KPW - 1) and
  // the V rows of its key pairs -> registers. Away from the end of the cache
  // the addresses advance by one tile of rows (kp, vp: at the next tile to
  // load); a tile that reaches past row stride - 1 clamps every row to it.
  const uint16_t* kp = kc + ((long)kvh * stride + k0 + KPW * wave) * HD + lane * 8;
  const uint16_t* vp[VLD];
#pragma unroll
  for (int i = 0; i < VLD; ++i) {
    const int q = tid + NT * i, pr = q % (KT / 2), ch = q / (KT / 2);
    vp[i] = vc + ((long)kvh * stride + k0 + 2 * pr) * HD + ch * 8;
  }
  v4u va[VLD], vb[VLD];
  auto load_v = [&](int t0) {
    if (t0 + KT <= stride) {
#pragma unroll
      for (int i = 0; i < VLD; ++i) {
        va[i] = *reinterpret_cast<const v4u*>(vp[i]);
        vb[i] = *reinterpret_cast<const v4u*>(vp[i] + HD);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VLD; ++i) {
        const int q = tid + NT * i, pr = q % (KT / 2), ch = q / (KT / 2);
        const int s0 = min(t0 + 2 * pr, stride - 1), s1 = min(t0 + 2 * pr + 1, stride - 1);
        va[i] = *reinterpret_cast<const v4u*>(vc + ((long)kvh * stride + s0) * HD + ch * 8);
        vb[i] = *reinterpret_cast<const v4u*>(vc + ((long)kvh * stride + s1) * HD + ch * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) vp[i] += KT * HD;
  };
  auto load_k = [&](int t0, int b) {
    if (t0 + KT <= stride) {
#pragma unroll
      for (int i = 0; i < KPW; ++i) dma16(kp + i * HD, ksh[b] + (KPW * wave + i) * KP);
    } else {
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int key = KPW * wave + i, slot = min(t0 + key, stride - 1);
        dma16(kc + ((long)kvh * stride + slot) * HD + lane * 8, ksh[b] + key * KP);
      }
    }
    kp += KT * HD;
  };
  load_v(k0);
  load_k(k0, 0);

  // ---- this lane's query row: q-norm, RoPE, the hi/lo split of the wave's half ----
  const int R = r0 + 16 * rg + c;
  const bool live = R < nrows;
  const int m = live ? R / grp : 0;
  const int h = kvh * grp + (live ? R % grp : 0);
  const uint32_t pos = p0 + (uint32_t)m;
  const int T = att_len(pos, window, stride);
  v8h qh[NQC], ql[NQC];
  {
    float qf[NCH][8];
    pa_q_row<HD, QT>(qin, (long)m * ldq + (long)h * HD, qnw, cosM + (long)m * HD, sinM + (long)m * HD, g, qf);
    // a wave-uniform branch keeps the register indices static
    if (dp == 0) pa_q_split<NQC>(qf, 0, qh, ql);
    else pa_q_split<NQC>(qf, NQC, qh, ql);
  }

  v4f oacc[NDT];
#pragma unroll
  for (int d = 0; d < NDT; ++d) oacc[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = -INFINITY, lrun = 0.0f;
  const int kfull = pa_full_keys(k0, kend, r0, grp, p0, window, stride);

  int b = 0;
  for (int t0 = k0; t0 < kend; t0 += KT, b ^= 1) {
    vmwait<0>();      // this wave's K rows (direct loads) and V registers of the tile
    __syncthreads();  // (A)
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int q = tid + NT * i;
      pa_store_vpair<VP>(vsh, va[i], vb[i], q / (KT / 2), q % (KT / 2));
    }
    const bool more = t0 + KT < kend;
    if (more) load_v(t0 + KT);  // the next tile's V rows run under this tile's math
    const int rt = window > 0 ? (int)(((long)last - t0) % window) : 0;
    v4f sp[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      v4f s0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, s2 = s0, s3 = s0;
      const uint8_t* kr0 = ksh[b] + (16 * st + c) * KP + (4 * dp * NQC + g) * 16;
#pragma unroll
      for (int j = 0; j < NQC; j += 2) {
        const v8h a0 = *reinterpret_cast<const v8h*>(kr0 + 4 * j * 16);
        const v8h a1 = *reinterpret_cast<const v8h*>(kr0 + (4 * j + 4) * 16);
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[j], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[j + 1], s1, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[j], s2, 0, 0, 0);
        s3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[j + 1], s3, 0, 0, 0);
      }
      sp[st] = (s0 + s1) + (s2 + s3);
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) xs[wave][st][lane] = sp[st];
    __syncthreads();  // (B)
    // the next tile's K rows, into the buffer tile t0 - KT used (free since (A))
    if (more) load_k(t0 + KT, b ^ 1);
#pragma unroll
    for (int st = 0; st < 2; ++st) sp[st] = xs[rg * DS][st][lane] + xs[rg * DS + 1][st][lane];
    float sc[2][4];
    if (t0 + KT <= kfull) {  // uniform
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[st][e] = sp[st][e];
    } else {
      pa_mask(sp, sc, t0, g, kend, T, window, rt, last, pos);
    }
    const v8h pb = pa_softmax<NDT>(sc, mrun, lrun, oacc);
#pragma unroll
    for (int d = 0; d < NDT; ++d) {
      const uint8_t* va8 = vsh + (16 * (dp * NDT + d) + c) * VP + 16 * g;
      const v4h lo = *reinterpret_cast<const v4h*>(va8), hi = *reinterpret_cast<const v4h*>(va8 + 8);
      const v8h a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, pb, oacc[d], 0, 0, 0);
    }
  }

  if (!live) return;
  float* o = ws + pa_ws_index(m, h, nH, ks, nsplit, HD);
  if (g == 0 && dp == 0) {
    o[0] = mrun;
    o[1] = lrun;
  }
#pragma unroll
  for (int d = 0; d < NDT; ++d) *reinterpret_cast<v4f*>(o + 4 + 16 * (dp * NDT + d) + 4 * g) = oacc[d];
}

// out[m][h hd + i] = sum_c acc_c w_c / sum_c l_c w_c over the splits that
// hold keys of token m, w_c = exp(max_c - max); fp32 or fp16 out. A
// workgroup of 256 threads merges 1024 / hd rows; each thread takes 4
// consecutive elements of its row (16-byte loads of every split's
// accumulator).
template <int OT>
__global__ void __launch_bounds__(256)
pre_attn_merge_kernel(const float* __restrict__ ws, void* __restrict__ out, int ldo, int hd, int nH, int nsplit,
                      int ksl, int stride, int window, int rows, const uint32_t* __restrict__ dyn) {
  const int tpr = hd / 4;  // threads per row
  const int row = blockIdx.x * (256 / tpr) + threadIdx.x / tpr, i = 4 * (threadIdx.x % tpr);
  if (row >= rows) return;
  const int m = row / nH, h = row % nH;
  const int T = att_len(dyn[0] + (uint32_t)m, window, stride);
  const int ns = min((T + ksl - 1) / ksl, nsplit);
  const float* w = ws + (long)row * nsplit * (hd + 4);
  // each batch of PM_CB splits is loaded with all of its loads in flight
  // (one round trip per batch, not one per split); the arithmetic and its
  // order are those of a split-by-split walk
  constexpr int PM_CB = 8;
  float mx = -INFINITY, L = 0.0f;
  v4f a = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float mv[PM_CB], lv[PM_CB];
  v4f vv[PM_CB];
  auto fetch = [&](int c0, bool all) {
#pragma unroll
    for (int j = 0; j < PM_CB; ++j) {
      const float* wc = w + (long)min(c0 + j, ns - 1) * (hd + 4);
      mv[j] = wc[0];
      if (all) {
        lv[j] = wc[1];
        vv[j] = *reinterpret_cast<const v4f*>(wc + 4 + i);
      }
    }
  };
  auto accumulate = [&](int c0) {
#pragma unroll
    for (int j = 0; j < PM_CB; ++j) {
      if (c0 + j >= ns || mv[j] == -INFINITY) continue;
      const float e = expf(mv[j] - mx);
      L = fmaf(lv[j], e, L);
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = fmaf(vv[j][k], e, a[k]);
    }
  };
  if (ns <= PM_CB) {  // every split in one batch (the chunk layouts: 4 or 8 splits)
    fetch(0, true);
#pragma unroll
    for (int j = 0; j < PM_CB; ++j)
      if (j < ns) mx = fmaxf(mx, mv[j]);
    accumulate(0);
  } else {
    for (int c0 = 0; c0 < ns; c0 += PM_CB) {
      fetch(c0, false);
#pragma unroll
      for (int j = 0; j < PM_CB; ++j)
        if (c0 + j < ns) mx = fmaxf(mx, mv[j]);
    }
    for (int c0 = 0; c0 < ns; c0 += PM_CB) {
      fetch(c0, true);
      accumulate(c0);
    }
  }
  const long oi = (long)m * ldo + (long)h * hd + i;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float v = a[k] / L;
    if constexpr (OT == Q4_DT_F16) reinterpret_cast<uint16_t*>(out)[oi + k] = f2h(v);
    else reinterpret_cast<float*>(out)[oi + k] = v;
  }
}

// Keys per split for a launch: a multiple of the tile, long enough that the
// (KV head, row block, split) grid has about PA_TARGET_WGS workgroups.
static int pa_split_len(int M, int nH, int nkv, int max_keys) {
  const int blocks = nkv * ceil_div(M * (nH / nkv), PA_ROWS);
  const int want = max(1, ceil_div(PA_TARGET_WGS, blocks));
  return PA_KT * ceil_div(max_keys, PA_KT * want);
}

}  // namespace q4

using namespace q4;

extern "C" {

size_t q4_pre_attn_workspace_bytes(int M, int nH, int nkv, int hd, int max_keys) {
  if (M <= 0 || nH <= 0 || nkv <= 0 || nH % nkv || hd <= 0 || max_keys <= 0) return 0;
  const int ns = ceil_div(max_keys, pa_split_len(M, nH, nkv, max_keys));
  return (size_t)M * nH * ns * (hd + 4) * sizeof(float);
}

int q4_pre_attn(const void* q, int q_dtype, int ldq, const float* qnw, const float* cosM, const float* sinM,
                const uint16_t* kc, const uint16_t* vc, void* out, int out_dtype, int ldo, int nH, int nkv, int hd,
                int stride, int window, int M, int max_keys, const uint32_t* dyn, void* ws, size_t ws_bytes,
                void* stream) {
  clear_error();
  Q4_ARG(q && qnw && cosM && sinM && kc && vc && out && dyn && ws, "null pointer");
  Q4_ARG(((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0 && ((uintptr_t)ws & 15) == 0,
         "kc, vc and ws must be 16-byte aligned");
  Q4_ARG(q_dtype == Q4_DT_F32 || q_dtype == Q4_DT_F16, "bad q_dtype");
  Q4_ARG(out_dtype == Q4_DT_F32 || out_dtype == Q4_DT_F16, "bad out_dtype");
  Q4_ARG(hd == 64 || hd == 128 || hd == 256 || hd == 512, "prefill attention takes head dims 64/128/256/512 (got %d)",
         hd);
  Q4_ARG(nH > 0 && nkv > 0 && nH % nkv == 0, "nH=%d must be a multiple of nkv=%d", nH, nkv);
  Q4_ARG(M > 0 && stride > 0 && window >= 0 && window <= stride, "bad sizes M=%d stride=%d window=%d", M, stride,
         window);
  Q4_ARG(window == 0 || M <= window, "a chunk of %d tokens is longer than the %d-slot ring", M, window);
  Q4_ARG(ldq >= nH * hd && ldo >= nH * hd, "row strides ldq=%d ldo=%d are shorter than nH * hd = %d", ldq, ldo,
         nH * hd);
  Q4_ARG(ldq % 8 == 0 && ((uintptr_t)q & 15) == 0 && ((uintptr_t)qnw & 15) == 0 && ((uintptr_t)cosM & 15) == 0 &&
             ((uintptr_t)sinM & 15) == 0,
         "q, qnw, cosM and sinM must be 16-byte aligned and ldq a multiple of 8");
  Q4_ARG(max_keys > 0 && max_keys <= stride, "max_keys=%d must be in 1..stride=%d", max_keys, stride);
  Q4_ARG(window == 0 || max_keys >= window, "a ring layer needs max_keys >= window (%d)", window);
  const size_t need = q4_pre_attn_workspace_bytes(M, nH, nkv, hd, max_keys);
  Q4_ARG(ws_bytes >= need, "prefill attention needs a %zu-byte workspace (got %zu)", need, ws_bytes);
  const int grp = nH / nkv, ksl = pa_split_len(M, nH, nkv, max_keys), ns = ceil_div(max_keys, ksl);
  const dim3 grid(nkv, ceil_div(M * grp, PA_ROWS), ns);
  hipStream_t st = as_stream(stream);
  float* w = reinterpret_cast<float*>(ws);
#define PA_LAUNCH(K16, K32, NTH)                                                                           \
  if (q_dtype == Q4_DT_F16)                                                                                \
    hipLaunchKernelGGL(K16, grid, dim3(NTH), 0, st, q, ldq, qnw, cosM, sinM, kc, vc, stride, window, grp, nH, M, \
                       dyn, w, ns, ksl);                                                                       \
  else                                                                                                     \
    hipLaunchKernelGGL(K32, grid, dim3(NTH), 0, st, q, ldq, qnw, cosM, sinM, kc, vc, stride, window, grp, nH, M, \
                       dyn, w, ns, ksl);
  switch (hd) {
    case 64: PA_LAUNCH((pre_attn_kernel<64, Q4_DT_F16>), (pre_attn_kernel<64, Q4_DT_F32>), PA_THREADS) break;
    case 128: PA_LAUNCH((pre_attn_kernel<128, Q4_DT_F16>), (pre_attn_kernel<128, Q4_DT_F32>), PA_THREADS) break;
    case 256: PA_LAUNCH((pre_attn_kernel<256, Q4_DT_F16>), (pre_attn_kernel<256, Q4_DT_F32>), PA_THREADS) break;
    default: PA_LAUNCH(pre_attn512_kernel<Q4_DT_F16>, pre_attn512_kernel<Q4_DT_F32>, PA512_THREADS) break;
  }
#undef PA_LAUNCH
  Q4_LAUNCHED("pre_attn");
  const int rows = M * nH, mgrid = ceil_div(rows, 256 / (hd / 4));
  if (out_dtype == Q4_DT_F16)
    hipLaunchKernelGGL(pre_attn_merge_kernel<Q4_DT_F16>, dim3(mgrid), dim3(256), 0, st, w, out, ldo, hd, nH, ns, ksl,
                       stride, window, rows, dyn);
  else
    hipLaunchKernelGGL(pre_attn_merge_kernel<Q4_DT_F32>, dim3(mgrid), dim3(256), 0, st, w, out, ldo, hd, nH, ns, ksl,
                       stride, window, rows, dyn);
  Q4_LAUNCHED("pre_attn_merge");
  return Q4_OK;
}

}  // extern "C"
