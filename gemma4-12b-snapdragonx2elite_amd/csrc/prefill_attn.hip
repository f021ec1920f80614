// Batched-prefill attention for gfx950: every token of a chunk of M tokens
// (positions p0 .. p0+M-1, p0 read from device memory) attends the fp16 KV
// cache causally, after the chunk's own K/V were written.
//
// Replaces vk/pre_attn.comp (recorded per layer at src/vk_engine.py:417),
// which runs one workgroup per (head, token) and walks the keys one scalar
// dot product at a time; here the query rows of a KV head are tiled onto
// MFMAs:
//  * A workgroup (4 waves; 8 at hd 512, two per row group splitting the head
//    dims, see PaGeom) owns 64 query rows of one KV head (row = token *
//    grp + query head within the group, so the rows share their K and V)
//    and one split of the cache slots (a multiple of 32 keys, long enough
//    that the grid has about 256 workgroups: 128 keys for a 1024-slot ring
//    of 8 KV heads, 512 for 4096 keys of one KV head); the grid covers the
//    keys the caller bounds and splits past a workgroup's last token exit
//    at once, so the launch shape does not depend on p0 (graph replay).
//  * q prologue, in registers: lane (c, g) of wave w holds row 16w + c,
//    elements 32j + 8g .. 32j + 8g + 7 of every 32-element chunk j; the
//    RoPE partner of element e (e +- hd/2) is in the same lane, and the
//    row's sum of squares needs two xor-shuffles. q is split into fp16
//    hi + lo parts (q = hi + lo to ~22 bits), so q . k is exact to fp32
//    rounding with fp16 MFMAs (two per k-step; k is fp16 in the cache).
//  * Per 32-key tile the workgroup stages K row-major ([key][hd], rows
//    padded by 16 bytes) and V transposed ([hd][key], pairs of keys per
//    32-bit word) in LDS from registers. Scores S^T = K q^T: one
//    v_mfma_f32_16x16x32_f16 pair per 16 keys x 16 rows x 32 elements; lane
//    (c, g) gets keys 4g .. 4g+3 of row c. Masked keys (past the row's
//    length, or in a ring slot a later token of the chunk now holds: slot s
//    holds position last - ((last - s) mod window) once the chunk's last
//    position is written, vk/pre_attn.comp:40) are -inf. Online softmax per row over the tile (xor-shuffles across the 4
//    lanes of a row), then O^T += V^T P^T with v_mfma_f32_16x16x16_f16: the
//    B operand is exactly the score layout (P rounded to fp16), the A
//    operand one 8-byte LDS read of the transposed V.
//  * Each workgroup writes its rows' (max, sum, unnormalised accumulator)
//    for its split; q4_pre_attn's second kernel merges the splits.
#include "q4mi_common.h"

namespace q4 {

constexpr int PA_WAVES = 4;
constexpr int PA_THREADS = 64 * PA_WAVES;
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

// Tile geometry per head dim: KT keys per LDS tile and DS waves per row
// group, 4 row groups of 16 rows per workgroup. With DS = 2 (hd 512) the two
// waves of a row group split the head dims: each holds q (hi + lo) for half
// of them, computes the partial scores over that half, and the pair adds
// the two halves through LDS (half 0 + half 1, the same bits in both
// waves); each then accumulates its half of the output dims. So q, the
// accumulators and the prefetch registers of a wave fit two waves per SIMD
// without spills, and no score is computed twice (a pair that computed the
// full scores in both waves took 137 us against 102 us for one wave per
// row group, 128 tokens x 16 heads over 4096 keys, MQA). Measured in the
// prefill chunk (the 8 global layers, kernel-only): 85.6 us with one wave
// per row group, 77.8 us with the split pair; 32-key tiles with the pair
// spill registers (87.6 us). Without the next tile's loads (timing only) the
// pair takes 67 us: the rest is issue and the three barriers per tile.
template <int HD>
struct PaGeom {
  static constexpr int KT = HD >= 512 ? 16 : 32;
  static constexpr int DS = HD >= 512 ? 2 : 1;
  static constexpr int WAVES = PA_WAVES * DS;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS = 16 * PA_WAVES;  // query rows per workgroup
};

template <int HD, int QT>
__global__ void __launch_bounds__(PaGeom<HD>::THREADS)
pre_attn_kernel(const void* __restrict__ qin, int ldq, const float* __restrict__ qnw, const float* __restrict__ cosM,
                const float* __restrict__ sinM, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                int stride, int window, int grp, int nH, int M, const uint32_t* __restrict__ dyn,
                float* __restrict__ ws, int nsplit, int ksl) {
  constexpr int KT = PaGeom<HD>::KT, DS = PaGeom<HD>::DS, ROWS = PaGeom<HD>::ROWS, NT = PaGeom<HD>::THREADS;
  constexpr int NST = KT / 16;        // 16-key subtiles per tile
  constexpr int NCH = HD / 32;        // 32-element chunks
  constexpr int NQC = NCH / DS;       // chunks of this wave's QK (its part of the head dims)
  constexpr int NDT = HD / 16 / DS;   // 16-element output tiles of this wave
  constexpr int CPR = HD / 8;         // 16-byte chunks per K/V row
  constexpr int KP = HD * 2 + 16;     // K tile row pitch (bytes)
  constexpr int VP = KT * 2 + 8;      // V^T tile row pitch (bytes)
  constexpr int KITEMS = KT * CPR, VITEMS = (KT / 2) * CPR;  // 16-byte K chunks, V key-pair chunks per tile
  constexpr int KLD = (KITEMS + NT - 1) / NT, VLD = (VITEMS + NT - 1) / NT;
  static_assert(NQC % 2 == 0, "head dim");
  __shared__ __attribute__((aligned(16))) uint8_t ksh[KT * KP];
  __shared__ __attribute__((aligned(16))) uint8_t vsh[HD * VP];
  __shared__ v4f xs[DS > 1 ? PaGeom<HD>::WAVES : 1][NST][64];  // partial scores of each wave (DS > 1)

  const int kvh = blockIdx.x, ks = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
  const int rg = wave / DS, dp = wave % DS;  // row group, output part
  const uint32_t p0 = dyn[0];
  const int nrows = M * grp, r0 = blockIdx.y * ROWS;
  const int mlast = (min(r0 + ROWS, nrows) - 1) / grp;
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
      const int q = tid + NT * i, pr = q % (KT / 2), ch = q / (KT / 2);
      if (q >= VITEMS) continue;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // elements 8 ch + 2w, 8 ch + 2w + 1 of keys 2 pr (low half) and 2 pr + 1 (high half)
        const uint32_t a = va[i][w], b = vb[i][w];
        *reinterpret_cast<uint32_t*>(vsh + (8 * ch + 2 * w) * VP + 4 * pr) = (a & 0xFFFFu) | (b << 16);
        *reinterpret_cast<uint32_t*>(vsh + (8 * ch + 2 * w + 1) * VP + 4 * pr) = (a >> 16) | (b & 0xFFFF0000u);
      }
    }
  };
  load_tile(k0);  // in flight while q is prepared

  // ---- this lane's query row: q-norm, RoPE, hi/lo split ----
  const int R = r0 + 16 * rg + c;
  const bool live = R < nrows;
  const int m = live ? R / grp : 0;
  const int h = kvh * grp + (live ? R % grp : 0);
  const uint32_t pos = p0 + (uint32_t)m;
  const int T = att_len(pos, window, stride);
  v8h qh[NQC], ql[NQC];  // chunks dp NQC .. of the row
  {
    // the lane's 8 consecutive elements of each chunk come in 16-byte loads
    float qf[NCH][8];
    const long qb = (long)m * ldq + (long)h * HD;
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
    const float* cs = cosM + (long)m * HD;
    const float* sn = sinM + (long)m * HD;
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
    // this wave's part of the head dims (a wave-uniform branch keeps the
    // register indices static)
    auto split = [&](int j0) {
#pragma unroll
      for (int j = 0; j < NQC; ++j)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const _Float16 hi = (_Float16)qf[j0 + j][u];
          qh[j][u] = hi;
          ql[j][u] = (_Float16)(qf[j0 + j][u] - (float)hi);
        }
    };
    if (DS == 1 || dp == 0) split(0);
    else split(NQC);
  }

  v4f oacc[NDT];
#pragma unroll
  for (int d = 0; d < NDT; ++d) oacc[d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = -INFINITY, lrun = 0.0f;

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
    float sc[NST][4];
    v4f sp[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      v4f s0 = v4f{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, s2 = s0, s3 = s0;
      const uint8_t* kr0 = ksh + (16 * st + c) * KP + (4 * dp * NQC + g) * 16;
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
    if constexpr (DS > 1) {  // the pair's partial scores: half 0 + half 1, in both waves
#pragma unroll
      for (int st = 0; st < NST; ++st) xs[wave][st][lane] = sp[st];
      __syncthreads();
#pragma unroll
      for (int st = 0; st < NST; ++st) sp[st] = xs[rg * DS][st][lane] + xs[rg * DS + 1][st][lane];
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) {
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
    // ---- online softmax over the tile ----
    float tmax = -INFINITY;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, sc[st][e]);
    tmax = slot_reduce<16, true>(tmax);
    const float mnew = fmaxf(mrun, tmax);
    const bool any = mnew != -INFINITY;
    // v_exp_f32-based exponentials (relative error ~1e-6): the weights are
    // rounded to fp16 (2^-11) before use, and the reference's GLSL exp()
    // is itself approximate; 8 fewer VALU operations per score
    const float corr = any ? __expf(mrun - mnew) : 1.0f;
    float psum = 0.0f;
    v4h pb[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the weights the V product uses are the fp16-rounded ones: the sum
        // is taken over the same values, so the output stays a weighted mean
        // of V rows (the row maximum's weight, 1, is exact)
        const _Float16 p = (_Float16)(any ? __expf(sc[st][e] - mnew) : 0.0f);
        psum += (float)p;
        pb[st][e] = p;
      }
    psum = slot_reduce<16>(psum);
    lrun = fmaf(lrun, corr, psum);
    mrun = mnew;
#pragma unroll
    for (int d = 0; d < NDT; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) oacc[d][e] *= corr;
    // ---- O^T += V^T P^T over this wave's output dims ----
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int d = 0; d < NDT; ++d) {
        const v4h a = *reinterpret_cast<const v4h*>(vsh + (16 * (dp * NDT + d) + c) * VP + (16 * st + 4 * g) * 2);
        oacc[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb[st], oacc[d], 0, 0, 0);
      }
  }

  // ---- this split's partial for the row ----
  if (!live) return;
  float* o = ws + pa_ws_index(m, h, nH, ks, nsplit, HD);
  if (g == 0 && dp == 0) {
    o[0] = mrun;
    o[1] = lrun;
  }
#pragma unroll
  for (int d = 0; d < NDT; ++d) *reinterpret_cast<v4f*>(o + 4 + 16 * (dp * NDT + d) + 4 * g) = oacc[d];
}

// rows per workgroup for head dim hd (PaGeom<hd>::ROWS)
static int pa_rows(int hd) { return hd >= 512 ? PaGeom<512>::ROWS : PaGeom<256>::ROWS; }

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
static int pa_split_len(int M, int nH, int nkv, int hd, int max_keys) {
  const int blocks = nkv * ceil_div(M * (nH / nkv), pa_rows(hd));
  const int want = max(1, ceil_div(PA_TARGET_WGS, blocks));
  return PA_KT * ceil_div(max_keys, PA_KT * want);
}

}  // namespace q4

using namespace q4;

extern "C" {

size_t q4_pre_attn_workspace_bytes(int M, int nH, int nkv, int hd, int max_keys) {
  if (M <= 0 || nH <= 0 || nkv <= 0 || nH % nkv || hd <= 0 || max_keys <= 0) return 0;
  const int ns = ceil_div(max_keys, pa_split_len(M, nH, nkv, hd, max_keys));
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
  const int grp = nH / nkv, ksl = pa_split_len(M, nH, nkv, hd, max_keys), ns = ceil_div(max_keys, ksl);
  const dim3 grid(nkv, ceil_div(M * grp, pa_rows(hd)), ns);
  hipStream_t st = as_stream(stream);
  float* w = reinterpret_cast<float*>(ws);
#define PA_LAUNCH(HD_)                                                                                           \
  if (q_dtype == Q4_DT_F16)                                                                                      \
    hipLaunchKernelGGL((pre_attn_kernel<HD_, Q4_DT_F16>), grid, dim3(PaGeom<HD_>::THREADS), 0, st, q, ldq, qnw,  \
                       cosM, sinM, kc, vc, stride, window, grp, nH, M, dyn, w, ns, ksl);                             \
  else                                                                                                           \
    hipLaunchKernelGGL((pre_attn_kernel<HD_, Q4_DT_F32>), grid, dim3(PaGeom<HD_>::THREADS), 0, st, q, ldq, qnw,  \
                       cosM, sinM, kc, vc, stride, window, grp, nH, M, dyn, w, ns, ksl);
  switch (hd) {
    case 64: PA_LAUNCH(64) break;
    case 128: PA_LAUNCH(128) break;
    case 256: PA_LAUNCH(256) break;
    default: PA_LAUNCH(512) break;
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
