/*
 * q4mi.h - C ABI of the MI355X (gfx950) int4/int8 quantized matrix-product
 * library (libq4mi.so).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream), enqueues work on
 * that stream and returns an int status (Q4_OK on success). On failure
 * q4_last_error() returns a message for the calling thread. The library
 * never allocates or frees caller memory; the split-K workspace is
 * caller-owned and sized by q4_workspace_bytes().
 *
 * Citations are relative to the reference repository
 * (monstercameron/Gemma4-12B-SnapdragonX2Elite) root.
 *
 * Weight formats
 *   reference ("ref"): wp[K][N/8] uint32, nibble j of wp[k][i] = code of row
 *     8i+j at k (src/vk_engine.py:129-130); fp16 scales [K/32][N]
 *     (src/vk_engine.py:131); e4m3 scales [K/32][N] bytes
 *     (src/vk_engine.py:133-137); int8 weights [K][N] (src/vk_engine.py:155).
 *   device ("panel-64", this library): rows padded to a multiple of 64; one
 *     16-byte unit per (row n, block b) at unit index
 *     ((n/64)*(K/32) + b)*64 + n%64; word i of a unit holds k = 32b+8i+e,
 *     e = 0..7, at nibble position (e&1)*4 + (e>>1). Scales (fp16, e4m3, or
 *     the fp16 W4A8 ratio) use the same ((n/64)*(K/32) + b)*64 + n%64 index.
 *     int8 weights for W8A8 are [N][K] (K contiguous).
 *   Codes are stored offset-8: nibble value = signed code + 8.
 */
#ifndef Q4MI_H
#define Q4MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define Q4_OK 0
#define Q4_ERR_ARG 1         /* bad shape, pointer, dtype or size */
#define Q4_ERR_HIP 2         /* a HIP runtime call failed */
#define Q4_ERR_TIMEOUT 3     /* bounded wait expired (q4_stream_wait) */

/* element types for activations / outputs / per-row weight scales */
#define Q4_DT_F32 0
#define Q4_DT_F16 1

/* block-scale formats of the int4 GEMV */
#define Q4_SCALE_F16 0
#define Q4_SCALE_E4M3 1

/* op ids for q4_workspace_bytes / q4_gemm_workspace_bytes */
#define Q4_OP_GEMV 0
#define Q4_OP_W4A16 1

/* ---- library info / errors --------------------------------------------- */
const char* q4_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* q4_last_error(void);
/* Bytes of the panel-64 weight words and of one per-(row,block) fp16 array
 * for an N x K matrix (K multiple of 32). */
int q4_dev_bytes(int N, int K, size_t* wq_bytes, size_t* scale_elems);

/* ---- plan overrides (tests and tuning sweeps) ---------------------------
 * No counterpart in the reference (its split heuristic is fixed,
 * src/vk_engine.py:143-148). Every launch plan (rows per GEMV workgroup,
 * units in flight, pairing, K splits, W4A16 k-groups) is chosen from the
 * shape alone unless an override is set here; environment variables are
 * never read. An override applies to every later call in the process, may
 * change the fp32 summation order of split or grouped plans (results stay
 * within the stated tolerances; integer outputs do not change), and is not
 * synchronized with calls running on other threads. Values outside a
 * knob's accepted set are ignored by the planner (the default plan runs). */
#define Q4_TUNE_GEMV_ROWS 0      /* rows per GEMV workgroup: 8, 16, 32, 64 */
#define Q4_TUNE_GEMV_UNITS 1     /* weight units in flight per lane: 4, 8 */
#define Q4_TUNE_GEMV_PAIR 2      /* 0: one row group per workgroup; 1: pair every unsplit even grid */
#define Q4_TUNE_GEMV_BAL 3       /* balanced grids of 256*m row groups, m 1..64 (0: off) */
#define Q4_TUNE_GEMV_MM_TILES 4  /* small-M GEMV 16-row tiles per workgroup: 1, 2, 4 */
#define Q4_TUNE_GEMV_MM_SPLIT 5  /* small-M GEMV K splits: 1..64 */
#define Q4_TUNE_GEMV_MM_DEEP 6   /* small-M GEMV deeper load ring: 0, 1 */
#define Q4_TUNE_W4A16_SPLIT 7    /* W4A16 K splits: 1..k-steps */
#define Q4_TUNE_W4A16_KG 8       /* W4A16 k-groups per workgroup: 1, 2 */
#define Q4_TUNE_W8A8_TILES 9     /* packed W8A8: 0: 256-row tiles; 1: persistent 128x320 tiles wherever they apply */
#define Q4_TUNE_COUNT 10
/* Set knob to value (value < 0 clears it). Q4_ERR_ARG for an unknown knob. */
int q4_tune_set(int knob, int value);
/* Current override of knob, -1 when none (or an unknown knob). */
int q4_tune_get(int knob);
/* Clear every override. */
void q4_tune_reset(void);

/* ---- weight preparation (load time) -------------------------------------
 * Replaces the numpy quantizer quant() (src/vk_engine.py:125-159).        */

/* W f32 [N][K] -> codes (panel-64 words), fp16 scales (panel-64) and the
 * unrounded fp32 scales sc32 [N][K/32] (row-major; may be NULL).
 * src/vk_engine.py:126-131. */
int q4_quantize(const float* W, int N, int K, uint32_t* wq, uint16_t* sc16,
                float* sc32, void* stream);

/* fp32 scales sc32 [N][K/32] -> e4m3 scales (panel-64 bytes) with the
 * per-tensor power-of-two lift; writes inv = 2^-shift to *inv_dev (device
 * float) and the max scale bits to *work (device uint32, caller-owned,
 * zeroed by this call). src/vk_engine.py:133-137. */
int q4_scales_e4m3(const float* sc32, int N, int K, uint8_t* sc8,
                   float* inv_dev, uint32_t* work, void* stream);

/* W8A8 weight fold from codes + unrounded fp32 scales:
 * W8 [N][K] int8, s_w [N] as fp32 (sw32, may be NULL) and fp16 (sw16, may
 * be NULL). src/vk_engine.py:152-157. */
int q4_w8_fold(const uint32_t* wq, const float* sc32, int N, int K,
               int8_t* W8, float* sw32, uint16_t* sw16, void* stream);

/* W4A8 requant ratio f16(sc32 / s_w) in panel-64 order.
 * benchmarks/coopgemm_w4a8.py:84. */
int q4_w4a8_ratio(const float* sc32, const float* sw32, int N, int K,
                  uint16_t* ratio, void* stream);

/* Reference layouts -> device layouts (drop-in for buffers produced by the
 * reference quantizer). wp [K][N/8] -> panel-64 words; fp16 scales
 * [K/32][N] -> panel-64 (sc_ref/sc_dev may be NULL to skip).
 * src/vk_engine.py:129-131. */
int q4_repack_ref(const uint32_t* wp, const uint16_t* sc_ref, int N, int K,
                  uint32_t* wq, uint16_t* sc_dev, void* stream);
/* Gate and up matrices (panel-64, N rows each, N % 32 == 0) -> one panel-64
 * matrix of 2N rows with row 2i = gate row i and row 2i+1 = up row i, words
 * and scales (scale_bytes 2 for fp16, 1 for e4m3) as they are: the layout
 * q4_gemv_gated reads. Load time; the reference keeps gate_proj and
 * up_proj as two matrices (src/vk_engine.py:198) and runs gelumul on their
 * outputs (:246). */
int q4_interleave_rows(const uint32_t* wa, const void* sa, const uint32_t* wb, const void* sb,
                       int N, int K, int scale_bytes, uint32_t* wout, void* sout, void* stream);
/* e4m3 scales [K/32][N] bytes -> panel-64 bytes. src/vk_engine.py:137. */
int q4_repack_e4m3_ref(const uint8_t* sc_ref, int N, int K, uint8_t* sc_dev,
                       void* stream);
/* int8 weights [K][N] -> [N][K]. src/vk_engine.py:155. */
int q4_repack_w8_ref(const int8_t* w8_kn, int N, int K, int8_t* w8_nk,
                     void* stream);

/* ---- decode GEMV ---------------------------------------------------------
 * y[N] = sum_k ((q[n,k]-8) * s[n,k/32]) * x[k]   (fp32 accumulate), times
 * inv for e4m3 scales. Replaces gemv.comp + reduce.comp
 * (vk/gemv.comp:11-33, vk/reduce.comp:8-12) / gemv_fp8.comp
 * (vk/gemv_fp8.comp:20-40) as recorded by gemv_ds()/gemv()
 * (src/vk_engine.py:214-226, 270-272).
 * x: x_dtype [K]; y: y_dtype [N]. split = number of workgroups sharing one
 * 64-row panel along K (0 = choose automatically). When the effective split
 * is > 1 a workspace of q4_workspace_bytes(Q4_OP_GEMV, N, K, split) bytes is
 * required; it must be zero-filled once before first use (q4_workspace_init)
 * and is left ready for the next call. One workspace per stream. */
size_t q4_workspace_bytes(int op, int N, int K, int split);
int q4_workspace_init(void* ws, size_t bytes, void* stream);
/* The split the library uses for an N x K GEMV when asked for split = 0
 * (the MI355X counterpart of src/vk_engine.py:143-148). */
int q4_gemv_auto_split(int N, int K);

int q4_gemv(const void* x, int x_dtype, const uint32_t* wq,
            const void* scales, int scale_fmt, float inv, void* y,
            int y_dtype, int N, int K, int split, void* ws, size_t ws_bytes,
            void* stream);
/* q4_gemv without a workspace argument, for callers that cannot allocate
 * (code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The split-K workspace is a
 * file-scope device array of q4_gemv_scratch_bytes() (2 MiB) per GPU, held
 * until the process ends; a GEMV whose split-K plan needs more is rejected
 * (Q4_ERR_ARG). Nothing is allocated or freed. The array is shared by every
 * call on that GPU: calls that overlap on one GPU (other streams or
 * threads) race; calls in order on one stream do not. Its address is
 * resolved on the first call per device (make that call outside a stream
 * capture). Results are bit-identical to q4_gemv's. */
size_t q4_gemv_scratch_bytes(void);
int q4_gemv_noalloc(const void* x, int x_dtype, const uint32_t* wq, const void* scales, int scale_fmt, float inv,
                    void* y, int y_dtype, int N, int K, int split, void* stream);
/* fp16-scale GEMV (vk/gemv.comp). */
int q4_gemv_f16s(const void* x, int x_dtype, const uint32_t* wq,
                 const uint16_t* sc16, void* y, int y_dtype, int N, int K,
                 int split, void* ws, size_t ws_bytes, void* stream);
/* e4m3-scale GEMV (vk/gemv_fp8.comp); inv as in the shader's uniform e.x. */
int q4_gemv_e4m3s(const void* x, int x_dtype, const uint32_t* wq,
                  const uint8_t* sc8, float inv, void* y, int y_dtype, int N,
                  int K, int split, void* ws, size_t ws_bytes, void* stream);

/* GEMV over an interleaved gate/up matrix (q4_interleave_rows; N = 2 I
 * rows) with the gelumul of the reference (vk/gelumul.comp:7-8, d_gm at
 * src/vk_engine.py:246) in its epilogue: act[i] = gelu_tanh(y[2i]) * y[2i+1]
 * for i < N/2, act in act_dtype. Same arguments and plan as q4_gemv; the
 * gate/up GEMVs (:242-243) and the gelumul dispatch become one launch. */
int q4_gemv_gated(const void* x, int x_dtype, const uint32_t* wq, const void* scales,
                  int scale_fmt, float inv, void* act, int act_dtype, int N, int K, int split,
                  void* ws, size_t ws_bytes, void* stream);

/* Several decode GEMVs that read the same activation x, in one launch:
 * y_i[N_i] = (GEMV of matrix i) x for i < count, with the arithmetic of
 * q4_gemv (split 1, no workspace). All matrices share K, the x dtype, the
 * scale format and the y dtype; each has its own words wq[i], scales[i],
 * output y[i] (may be offsets into one buffer) and, for e4m3 scales,
 * inv[i] (inv may be NULL for fp16 scales). The reference records these
 * as consecutive gemv_ds() dispatches on one input buffer, each followed by
 * a global barrier: q/k/v into the qkv buffer (src/vk_engine.py:232-234,
 * recorded at :278-279) and gate/up (:242-243, recorded at :284). The x
 * slice must fit the workgroup staging area: K <= 32768 for fp16 x,
 * K <= 16384 for fp32 x. */
#define Q4_GEMV_MAX_BATCH 8
int q4_gemv_batch(const void* x, int x_dtype, int K, int scale_fmt,
                  int y_dtype, int count, const uint32_t* const* wq,
                  const void* const* scales, const float* inv,
                  void* const* y, const int* N, void* stream);

/* The normadd and rmsnorm recorded before a decode GEMV, fused into its
 * launch: h_out = (h + rmsnorm(a) * w) * scale (scale 0: unscaled) as
 * q4_normadd, then x = fp16(rmsnorm(h_out) * w2) as q4_rmsnorm, and y = the
 * GEMV of x (q4_gemv's arithmetic with fp16 x, split 1; gated as
 * q4_gemv_gated). Replaces the d_na / d_nas normadd followed by the norm
 * and the GEMV(s) that read it (src/vk_engine.py:242-243 -> :284,
 * :248-249 -> the next layer's :231-234). Every workgroup forms x itself;
 * x is never written to memory. h_out is a separate buffer (it may not
 * overlap h, a, w or w2): callers alternate two residual buffers. a, w, h,
 * h_out and w2 are fp32 [K], 16-byte aligned; K <= 4096. The norm sums
 * are reduced in another order than q4_normadd_rmsnorm's, so h_out and x
 * may differ from the two-launch sequence in the last bits. */
int q4_gemv_normadd(const float* a, const float* w, const float* h, float* h_out, float scale,
                    const float* w2, const uint32_t* wq, const void* scales, int scale_fmt,
                    float inv, void* y, int y_dtype, int N, int K, int gated, void* stream);

/* q4_gemv_batch with x formed as in q4_gemv_normadd (q/k/v after the
 * previous layer's closing normadd and this layer's input norm). */
int q4_gemv_batch_normadd(const float* a, const float* w, const float* h, float* h_out,
                          float scale, const float* w2, int K, int scale_fmt, int y_dtype,
                          int count, const uint32_t* const* wq, const void* const* scales,
                          const float* inv, void* const* y, const int* N, void* stream);

/* Several activation vectors through one matrix: Y[m][n] = (GEMV of x_m)
 * for m < M, x fp16 [M][K] (row-major), Y y_dtype [M][N], with the decode
 * GEMV's arithmetic (exact (q - 8) x products summed per block in fp32,
 * times the block scale, blocks accumulated in fp32, times inv for e4m3
 * scales). This is the small-M (M ~ 8) batched GEMV that speculative
 * decode verification needs and the reference lacks: its coopmat GEMM pads
 * M to 64 and its GEMV reads the weights once per token (JOURNEY.md:666).
 *   exact = 0: one launch for all M <= 16 vectors, the block sums from int4
 *              x fp16 MFMAs; rows agree with q4_gemv to fp32 rounding.
 *   exact = 1: each row bit-identical to q4_gemv of that x row when
 *              q4_gemv runs unsplit (N >= 1920), so verification scores
 *              exactly what token-by-token decode would. The x rows of one
 *              launch are staged in LDS (144 KB): a launch takes 8 vectors
 *              for K <= 8192, 4 for K <= 16384, 2 for K <= 32768 (larger K
 *              is an error), and M is covered by as many launches as
 *              needed, each reading the weights once. */
#define Q4_GEMV_MAX_VECTORS 16
int q4_gemv_multi(const void* x, int M, const uint32_t* wq,
                  const void* scales, int scale_fmt, float inv, void* y,
                  int y_dtype, int N, int K, int exact, void* stream);
/* The MFMA path (exact = 0) with a caller-owned workspace for matrices
 * with fewer than 15360 rows and K >= 2048 (tall-K shapes such as the down
 * projection): K is split across workgroups into ceil(240 / (rows / 64))
 * ranges (fewer where a range would hold under 32 blocks), so each
 * workgroup reads 64 rows' x slices once for four 16-row tiles; fp32
 * partials [split][M][N] go to ws (16-byte aligned) and a second kernel
 * sums them in split order, times the scale
 * factor. Rows agree with q4_gemv to fp32 rounding, as the unsplit path's
 * do. ws may be NULL or smaller than q4_gemv_multi_workspace_bytes(M, N,
 * K) (0 where no split is planned): the call then runs unsplit, exactly
 * like q4_gemv_multi(..., exact = 0, ...). Same row as q4_gemv_multi:
 * JOURNEY.md:666. */
size_t q4_gemv_multi_workspace_bytes(int M, int N, int K);
int q4_gemv_multi_ws(const void* x, int M, const uint32_t* wq,
                     const void* scales, int scale_fmt, float inv, void* y,
                     int y_dtype, int N, int K, void* ws, size_t ws_size,
                     void* stream);

/* ---- prefill GEMMs -------------------------------------------------------
 * W4A16: Y f16 [M][N] = X f16 [M][K] @ f16((q-8)*s)^T, fp32 accumulate; X
 * and wq 16-byte aligned, Y 8-byte aligned.
 * Replaces coopgemm_i4h.comp (vk/coopgemm_i4h.comp:13-35) as wired by
 * gemm_ds()/gmm() (src/vk_engine.py:351-365, 391-400). */
int q4_gemm_w4a16(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16,
                  uint16_t* Y, int M, int N, int K, void* stream);
/* The same product with a caller-owned workspace: when the M x N tile grid
 * is too small to fill the GPU (tall-K shapes such as the down projection,
 * src/vk_engine.py:423), K is split across workgroups and fp32 partials
 * [split][M][N] are summed in split order by a second kernel
 * (deterministic). ws may be NULL or smaller than
 * q4_gemm_workspace_bytes(Q4_OP_W4A16, M, N, K); the call then runs
 * without splitting, exactly like q4_gemm_w4a16. */
size_t q4_gemm_workspace_bytes(int op, int M, int N, int K);
int q4_gemm_w4a16_ws(const uint16_t* X, const uint32_t* wq,
                     const uint16_t* sc16, uint16_t* Y, int M, int N, int K,
                     void* ws, size_t ws_bytes, void* stream);
/* The prefill gate and up GEMMs and the gelumul after them (p_g, p_u and
 * p_gm: src/vk_engine.py:381-382, 421-422; vk/gelumul.comp:7-8) as one
 * W4A16 product over an interleaved gate/up matrix (q4_interleave_rows; N
 * = 2 I rows): Y f16 [M][N/2], Y[m][i] = f16(gelu_tanh(g) * u) with g and u
 * the fp16-rounded products of rows 2i and 2i + 1, as the reference's fp16
 * GEMM outputs reach its gelumul. fp32 partials go to ws
 * (q4_gemm_w4a16_gated_workspace_bytes, required, 16-byte aligned) and
 * the split-K reduce applies the gelumul. */
size_t q4_gemm_w4a16_gated_workspace_bytes(int M, int N, int K);
/* A prefill GEMM whose output goes straight into the residual normadd (and
 * the rmsnorm after it): the o projection with p_na (+ p_pfn) and the down
 * projection with p_nas (+ the next layer's p_in), src/vk_engine.py:418-420,
 * 423-424 and :413. W4A16 into fp32 partials in ws
 * (q4_gemm_w4a16_normadd_workspace_bytes, required, 16-byte aligned), then
 * one launch per row: x = f16 of the partials' sum in split order (the
 * GEMM's fp16 output, as q4_gemm_w4a16_ws rounds it), h = (h + rmsnorm(x)
 * w) * scale (scale 0 = 1) as q4_pre_normadd, and with w2 and y the
 * rmsnorm of the new h into y (y_dtype) as q4_pre_normadd_rmsnorm. D = N. */
size_t q4_gemm_w4a16_normadd_workspace_bytes(int M, int N, int K);
/* The stacked q/k/v prefill GEMM (p_q, p_k, p_v over rows stacked q, k, v;
 * k == v layers stack q, k) and the prepkv after it (p_prep:
 * src/vk_engine.py:370-374, 414-416): W4A16 into fp32 partials in ws
 * (q4_gemm_w4a16_normadd_workspace_bytes(M, N, K), required), then one
 * launch that writes the q columns as fp16 (the GEMM's output, summed in
 * split order) to q [M][ldq] and, per (KV head, token), the k and v columns
 * rounded the same way through q4_pre_prepkv's arithmetic into kc and vc
 * (the k and v outputs themselves are not stored). N = nq + nk (+ nk). */
int q4_gemm_w4a16_qkv_prepkv(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M,
                             int N, int K, uint16_t* q, int ldq, int nq, const float* knw,
                             const float* cosM, const float* sinM, uint16_t* kc, uint16_t* vc,
                             int nkv, int hd, int keqv, int stride, int window,
                             const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream);
int q4_gemm_w4a16_normadd(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16, int M,
                          int N, int K, const float* w, float* h, float scale, const float* w2,
                          void* y, int y_dtype, void* ws, size_t ws_bytes, void* stream);
int q4_gemm_w4a16_gated(const uint16_t* X, const uint32_t* wq, const uint16_t* sc16,
                        uint16_t* Y, int M, int N, int K, void* ws, size_t ws_bytes,
                        void* stream);

/* Per-row int8 activation quantizer: sa[m] = max(absmax/127, 1e-12),
 * A = clamp(rint(x / sa), -127, 127) (IEEE fp32 divide).
 * vk/cast_i8.comp:11-19, rounding per benchmarks/coopgemm_w4a8.py:87-88. */
int q4_quant_act_i8(const void* X, int x_dtype, int8_t* A, float* sa, int M,
                    int K, void* stream);

/* W8A8: C int32 = A int8 [M][K] @ W8 int8 [N][K]^T (exact),
 * Y f16 [M][N] = f16((f32(C) * sa[m]) * sw[n]); sw is sw_dtype [N].
 * C (int32 [M][N]) is written only if non-NULL. Y may be NULL when C is not.
 * A, the weights, Y and C must be 16-byte aligned (Q4_ERR_ARG otherwise).
 * K must be a multiple of 64 (Q4_ERR_ARG otherwise), narrower than the
 * reference shader, which steps K by 32 (vk/coopgemm_w8a8.comp:23): every
 * engine shape (K = 3840, 4096, 15360) satisfies it. The same rule holds for
 * q4_gemm_w8a8_packed and q4_gemm_w4a8. 127^2 * K must stay below 2^31.
 * vk/coopgemm_w8a8.comp:18-37. */
int q4_gemm_w8a8(const int8_t* A, const int8_t* W8, const float* sa,
                 const void* sw, int sw_dtype, uint16_t* Y, int32_t* C, int M,
                 int N, int K, void* stream);

/* The same W8A8 product on packed weights: the layout the int8 MFMA reads
 * one 1 KB fragment at a time (rows padded to a multiple of 32 and K to a
 * multiple of 128, Kp; the block of rows 32t..32t+31 and K bytes
 * 32s..32s+31 is 1 KB at (t*(Kp/32) + s)*1024, lane l's 16 bytes at 16*l:
 * row 32t + l%32, bytes 32s + 16*(l/32)). q4_w8_pack converts W8 [N][K]
 * once at load time (q4_w8_packed_bytes bytes, padding zero).
 * Bit-identical results to q4_gemm_w8a8.
 * vk/coopgemm_w8a8.comp:18-37 (weights as folded at src/vk_engine.py:152-157). */
size_t q4_w8_packed_bytes(int N, int K);
int q4_w8_pack(const int8_t* W8, int N, int K, int8_t* W8p, void* stream);
int q4_gemm_w8a8_packed(const int8_t* A, const int8_t* W8p, const float* sa,
                        const void* sw, int sw_dtype, uint16_t* Y,
                        int32_t* C, int M, int N, int K, void* stream);

/* q4_gemm_w8a8_packed with per-workgroup timestamps (measurement; no
 * counterpart in the reference, which times its GEMMs only from the host,
 * benchmarks/coopgemm_i8.py:85): stamps[4b .. 4b+3] of workgroup b = wall
 * clock (q4_probe_wall_clock_khz ticks) at its start, after its k-loop and at
 * its end, and shader-clock cycles from start to end, so the clock the chip
 * ran the GEMM at and the main-loop / epilogue split are read from the run
 * itself (for the persistent plan, "after its k-loop" is after its last
 * tile's k-loop). stamps_bytes >= 32 * q4_gemm_w8a8_packed_workgroups(M, N, K).
 * Results are those of q4_gemm_w8a8_packed. */
int q4_gemm_w8a8_packed_stamped(const int8_t* A, const int8_t* W8p, const float* sa,
                                const void* sw, int sw_dtype, uint16_t* Y,
                                int32_t* C, int M, int N, int K,
                                unsigned long long* stamps, size_t stamps_bytes,
                                void* stream);
/* Workgroups of a q4_gemm_w8a8_packed launch that passes Y, with Y, sa and
 * sw 16-byte aligned: at most 256 (one per CU) when M % 128 == 0,
 * N % 320 == 0, the 128-byte k-steps (K / 128, rounded up) are a multiple
 * of 3 and there are more than 256 tiles of 128 x 320 (each workgroup then
 * runs its share of those tiles), else one per 256 x 256 (or 128 x 256)
 * tile. */
size_t q4_gemm_w8a8_packed_workgroups(int M, int N, int K);

/* W4A8: as W8A8 with B = int8(clamp(rint((q-8) * ratio[n,b]), -127, 127))
 * formed on the fly from the int4 codes and the panel-64 fp16 ratio.
 * vk/coopgemm_w4a8.comp:21-50. */
int q4_gemm_w4a8(const int8_t* A, const uint32_t* wq, const uint16_t* ratio,
                 const float* sa, const void* sw, int sw_dtype, uint16_t* Y,
                 int32_t* C, int M, int N, int K, void* stream);

/* W4A8's int8 weights formed once instead of per M-tile: W8 [N][K] =
 * int8(clamp(rint((q-8) * ratio[n,b]), -127, 127)), exactly the values
 * q4_gemm_w4a8 forms on the fly (vk/coopgemm_w4a8.comp:28-34). With
 * q4_w8_pack and q4_gemm_w8a8_packed this gives q4_gemm_w4a8's results bit
 * for bit at the W8A8 speed, for callers that can hold the int8 weights
 * (twice the int4 bytes; the reference's PREFILL_I8 path holds int8 weights
 * too, src/vk_engine.py:152-157). */
int q4_w4a8_weights(const uint32_t* wq, const uint16_t* ratio, int N, int K,
                    int8_t* W8, void* stream);

/* f32 <-> f16 staging casts around a prefill GEMM.
 * vk/cast_dn.comp:7, vk/cast_up.comp:7 (wired at src/vk_engine.py:398-400). */
int q4_cast_f32_f16(const float* src, uint16_t* dst, size_t n, void* stream);
int q4_cast_f16_f32(const uint16_t* src, float* dst, size_t n, void* stream);

/* ---- decode-token ops between the GEMVs ------------------------------------
 * fp32 activations as in the reference; the KV cache is fp16
 * [nkv][stride][hd] per layer (src/vk_engine.py:204). The token position is
 * read from device memory (dyn[0], the reference's DYN buffer,
 * src/vk_engine.py:306-310) so a captured graph replays every token. */

/* y = x * inv * w, inv = 1/sqrt(mean(x^2) + 1e-6); y fp32 or fp16
 * (y_dtype). vk/rmsnorm.comp:8-12 (normbg, src/vk_engine.py:227-228). */
int q4_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int D, void* stream);

/* h = (h + x * inv * w) * scale (scale 0 = unscaled).
 * vk/normadd.comp:8-12 (d_na / d_nas, src/vk_engine.py:242,248-249). */
int q4_normadd(const float* x, const float* w, float* h, int D, float scale, void* stream);

/* q4_normadd followed by q4_rmsnorm of the new h with weight w2 into y (fp32
 * or fp16), in one launch: the normadd the reference records at the end of
 * an attention or MLP block and the rmsnorm it records next on h
 * (src/vk_engine.py:242-243, and :248-249 followed by the next layer's :231
 * or the final norm :250). */
int q4_normadd_rmsnorm(const float* x, const float* w, float* h, int D, float scale,
                       const float* w2, void* y, int y_dtype, void* stream);

/* out = 0.5 g (1 + tanh(0.79788456 (g + 0.044715 g^3))) * up; out fp32 or
 * fp16. vk/gelumul.comp:7-8 (d_gm, src/vk_engine.py:246). */
int q4_gelumul(const float* gate, const float* up, void* out, int out_dtype, int n, void* stream);

/* This token's K (k-norm with weight knw, RoPE with cosb/sinb) and V
 * (v-norm; read at koff when keqv) of every KV head into cache slot
 * dyn[0] % window (window > 0) or dyn[0]; nothing is written when the slot
 * is past stride. qkv, knw, cosb and sinb 16-byte aligned, koff and voff
 * multiples of 4. vk/prepkv.comp:16-30 (d_prep, src/vk_engine.py:236-237). */
int q4_prepkv(const float* qkv, const float* knw, const float* cosb, const float* sinb,
              uint16_t* kc, uint16_t* vc, int nkv, int hd, int koff, int voff, int keqv,
              int stride, int window, const uint32_t* dyn, void* stream);

/* Decode attention of nH query heads (q at qoff in qkv; q-norm with qnw,
 * RoPE) over the first T = dyn[0]+1 (or min(dyn[0]+1, window)) cached keys
 * of KV head h/grp: softmax(q.k) weighted sum of V into out[nH*hd] (fp32
 * or fp16, out_dtype). Split along the keys (two launches: the splits of
 * each group of query heads sharing a KV head, then their merge); ws:
 * q4_attn_workspace_bytes(nH, hd, stride) bytes, no initialisation needed.
 * hd 64, 128, 256 or 512; qkv, qnw, cosb, sinb (and knw), kc and vc 16-byte
 * aligned, qoff (koff, voff) multiples of 4.
 * vk/attn.comp:18-53 (d_attn, src/vk_engine.py:238-239). */
size_t q4_attn_workspace_bytes(int nH, int hd, int stride);
int q4_attn(const float* qkv, const float* qnw, const float* cosb, const float* sinb,
            const uint16_t* kc, const uint16_t* vc, void* out, int out_dtype, int nH, int nkv,
            int hd, int stride, int window, int qoff, int grp, const uint32_t* dyn, void* ws,
            size_t ws_bytes, void* stream);

/* Per-token inputs at the head of a recorded decode graph, from (tid, pos) =
 * step[0..1] read on the device when the graph runs (step: pinned host memory
 * the host rewrites before each launch, read with system-scope loads, or
 * device memory): h[0..H) = emb[tid*H ..] (the pre-scaled fp32 embedding
 * rows [vocab][H]), dyn[0] = pos, dyn[1] = pos + 1, and for each of ntab
 * RoPE tables cos_out[t][0..hd[t]) = cos_tab[t][pos*hd[t] ..] (rows
 * [max_pos][hd[t]]), sin likewise. Replaces the host writes of the
 * reference's forward() (src/vk_engine.py:312-314: EMB row, DYN, set_rope),
 * so a token is one graph launch and one bounded wait. Values out of range
 * are clamped on the device (callers check tid < vocab, pos < max_pos). */
#define Q4_TOKEN_MAX_TABLES 4
int q4_token_inputs(const int32_t* step, const float* emb, int vocab, int H, float* h, uint32_t* dyn, int ntab,
                    const float* const* cos_tab, const float* const* sin_tab, const int* hd, int max_pos,
                    float* const* cos_out, float* const* sin_out, void* stream);

/* q4_prepkv and q4_attn of one layer as one pass (two launches instead of
 * three): the workgroups of the key split that holds this token's slot form
 * its K (k-norm with knw, RoPE) and V (v-norm; read at koff when keqv),
 * rounded to fp16 as the cache holds them, use them for that key, and write
 * them to the cache; outputs and cache contents are those of q4_prepkv
 * followed by q4_attn. d_prep + d_attn (src/vk_engine.py:235-239,281). */
int q4_prepkv_attn(const float* qkv, const float* knw, const float* qnw, const float* cosb,
                   const float* sinb, uint16_t* kc, uint16_t* vc, void* out, int out_dtype, int nH,
                   int nkv, int hd, int stride, int window, int qoff, int koff, int voff, int keqv,
                   int grp, const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream);

/* ---- batched prefill layer ops --------------------------------------------
 * One chunk of M tokens at positions p0 .. p0+M-1 (p0 = dyn[0], read on the
 * device so a recorded graph replays every chunk), the reference's prefill
 * layer graph (src/vk_engine.py:410-424, buffers :339-383). Rows are
 * [M][D] row-major; x inputs may be fp16 where the reference up-casts an
 * fp16 GEMM output to fp32 first (that value is exact), outputs that feed a
 * GEMM may be fp16 where the reference down-casts them (the same rounding).
 * Row-wise rmsnorm: vk/pre_norm.comp:9-13. */
int q4_pre_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int D,
                   int M, void* stream);
/* Row-wise h = (h + rmsnorm(x) * w) * sc (sc = scale, or 1 for 0):
 * vk/pre_na.comp:9-14; x fp32 or fp16. */
int q4_pre_normadd(const void* x, int x_dtype, const float* w, float* h, int D,
                   int M, float scale, void* stream);
/* The same followed by the rmsnorm the reference records next on the new h
 * (p_na then p_pfn, p_nas then the next layer's p_in: :419-420, :424, :413),
 * one launch per row set. */
int q4_pre_normadd_rmsnorm(const void* x, int x_dtype, const float* w, float* h,
                           int D, int M, float scale, const float* w2, void* y,
                           int y_dtype, void* stream);
/* gelumul over n = M * I elements with fp32 or fp16 gate/up (the prefill
 * dispatch of vk/gelumul.comp at :422). */
int q4_pre_gelumul(const void* gate, const void* up, int in_dtype, void* out,
                   int out_dtype, long n, void* stream);
/* Every token's K (k-norm with weight, RoPE with the token's cos/sin row)
 * and V (v-norm) of every KV head into the fp16 caches at the token's slot:
 * vk/pre_prepkv.comp:18-32. k, v [M][ld] (v may equal k for k == v layers),
 * cosM/sinM [M][hd]. When the chunk wraps a ring, the later token of a
 * shared slot is the one written. */
int q4_pre_prepkv(const void* k, const void* v, int kv_dtype, int ld,
                  const float* knw, const float* cosM, const float* sinM,
                  uint16_t* kc, uint16_t* vc, int nkv, int hd, int stride,
                  int window, int M, const uint32_t* dyn, void* stream);
/* Causal attention of every token of the chunk (vk/pre_attn.comp:18-53):
 * q [M][ldq] (head h at h*hd; fp32 or fp16) with q-norm and RoPE per token,
 * scores over the first min(pos+1, window or stride) slots of KV head
 * h / (nH / nkv) (no score scaling), ring slots holding a later token of
 * the chunk skipped, softmax, fp16 V; out [M][ldo]. Head dims 64, 128,
 * 256, 512; M <= window for ring layers. max_keys bounds the keys any token
 * of any chunk the call (or a graph of it) will see (window for ring
 * layers, the prompt length for global ones); ws: workspace of
 * q4_pre_attn_workspace_bytes(M, nH, nkv, hd, max_keys) bytes. Two launches
 * (split-key MFMA attention, then the split merge). */
size_t q4_pre_attn_workspace_bytes(int M, int nH, int nkv, int hd, int max_keys);
int q4_pre_attn(const void* q, int q_dtype, int ldq, const float* qnw,
                const float* cosM, const float* sinM, const uint16_t* kc,
                const uint16_t* vc, void* out, int out_dtype, int ldo, int nH,
                int nkv, int hd, int stride, int window, int M, int max_keys,
                const uint32_t* dyn, void* ws, size_t ws_bytes, void* stream);

/* ---- measurement probes ----------------------------------------------------
 * Ceilings measured on the part itself; they compute nothing of the model.
 * Streaming read of `bytes` (16-byte nontemporal loads, `units` (4/8/16) per
 * lane in flight, `wgs` workgroups of 256 threads over contiguous chunks
 * (chunked) or grid-strided 4 KB rows): the counterpart of the reference's
 * streaming-read microbenchmark (benchmarks/microbench_bw.py:26-35). With
 * next/prefetch_bytes, each workgroup then reads its successor's first
 * prefetch_bytes/wgs bytes of `next` (laid out like buf, reads clamped to
 * next_bytes) with L2-allocating loads. With comp (>= bytes / 8), every
 * 16-byte load has a 2-byte companion load from comp at the unit's index
 * (the access pattern of the GEMV's fp16 block scales). sink: one uint32
 * per workgroup, written only when a data hash hits a magic value. */
int q4_probe_stream_read(const void* buf, size_t bytes, int wgs, int units, int chunked, const void* next,
                         size_t next_bytes, size_t prefetch_bytes, const void* comp, size_t comp_bytes,
                         uint32_t* sink, size_t sink_bytes, void* stream);
/* `iters` (a multiple of 8) rounds of four independent MFMAs per wave, wgs
 * workgroups of four waves: kind 0 = v_mfma_i32_32x32x32_i8 (65536 int ops
 * each), 1 = v_mfma_f32_32x32x16_f16 (32768 flops each). operands: 64 KB of
 * (random) bytes, 8 A and 8 B fragments per lane taken in turn, or NULL for
 * the same fragments every time (less bit toggling, less power). clocks[2b]
 * = shader-clock cycles and clocks[2b+1] = wall-clock ticks
 * (q4_probe_wall_clock_khz) of workgroup b's loop: the matrix-core ceiling
 * and the clock under that load (the counterpart of vk/coopgemm_i8.comp,
 * benchmarks/coopgemm_i8.py:85). */
int q4_probe_mfma(int kind, int wgs, int iters, const void* operands, size_t operand_bytes,
                  unsigned long long* clocks, size_t clocks_bytes, int* sink, size_t sink_bytes, void* stream);
int q4_probe_wall_clock_khz(int* khz);

/* ---- record-once submit --------------------------------------------------
 * The per-token command buffer recorded once and resubmitted
 * (src/vk_engine.py:254-290, forward() :312-319) becomes a hipGraph captured
 * from a (non-null) stream. */
int q4_graph_begin(void* stream);
int q4_graph_end(void* stream, void** graph_exec);
int q4_graph_launch(void* graph_exec, void* stream);
int q4_graph_destroy(void* graph_exec);
/* Bounded wait for all work on the stream: Q4_ERR_TIMEOUT after timeout_ms
 * (<= 0 waits forever). The counterpart of the fence wait with
 * GEMMA4_FENCE_TIMEOUT_MS (src/vk_engine.py:293-302). */
int q4_stream_wait(void* stream, int timeout_ms);

/* GPU timestamps for a per-op profile of a recorded graph (PROFILE=1 /
 * PREPROF=1: vkCmdWriteTimestamp after each op into a query pool, read back
 * after the fence, src/vk_engine.py:37-46,263-265,321-335,491-504). n >= 2
 * slots of device memory (allocated here, freed by q4_timestamps_destroy).
 * q4_timestamp_record enqueues a one-wave launch that writes the constant-
 * rate wall clock into slot i when it runs, stream-ordered after the work
 * before it (inside a q4_graph_begin/end capture it becomes a node of the
 * graph and stamps again at every replay; each stamp adds one small
 * dependent launch). q4_timestamps_read, after the stream's work is done,
 * gives ms[i] = milliseconds from slot 0 to slot i (ms: n doubles). */
int q4_timestamps_create(int n, void** ts);
int q4_timestamp_record(void* ts, int i, void* stream);
int q4_timestamps_read(void* ts, double* ms);
int q4_timestamps_destroy(void* ts);

#ifdef __cplusplus
}
#endif
#endif /* Q4MI_H */
