"""numpy restatement of the reference's int4/int8 quantized matrix-product path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the shipped package
never imports this file; tests, ``smoke()`` and the CPU-baseline leg of
``bench.py`` use it as the checker.

Conventions (all follow the reference; citations are relative to the
reference repository root):

* ``BLK = 32`` K-elements per scale block (``src/vk_engine.py:12``).
* Weights ``W[N, K]`` (N output rows, K reduction), codes ``q = code + 8`` in
  ``[0, 15]`` stored as ``uint8`` (``src/vk_engine.py:128``).
* Block scales ``sc[N, nblk]`` float32, unrounded (``src/vk_engine.py:127``).
* Reference storage formats: ``wp[K, N/8]`` uint32, nibble ``j`` of
  ``wp[k, i]`` holding ``q[8i + j, k]`` (``src/vk_engine.py:129-130``); fp16
  scales ``[nblk, N]`` (``src/vk_engine.py:131``); e4m3 scales ``[nblk, N]``
  bytes + ``inv`` (``src/vk_engine.py:133-137``); int8 weights ``[K, N]`` +
  fp16 ``s_w[N]`` (``src/vk_engine.py:152-157``).
* Device format of this build ("panel-64", defined here so tests can check
  the GPU repack/quantize kernels bit for bit): rows padded to a multiple of
  64; one 16-byte unit per (row n, block b) at unit index
  ``((n // 64) * nblk + b) * 64 + n % 64``; word ``i`` of the unit holds
  ``k = 32 b + 8 i + e`` (e = 0..7) at nibble position
  ``NIB_POS[e] = (e & 1) * 4 + (e >> 1)``. Scales use the same
  ``((n // 64) * nblk + b) * 64 + n % 64`` index. Padded rows hold code 8 and
  scale 0.

Parity status of each function is recorded in its docstring; every function
here is pinned by a check in ``tests/test_oracle.py`` that does not retype
the formula.
"""
from __future__ import annotations

import numpy as np

BLK = 32
PANEL = 64
# nibble position of element e (0..7) inside a device word
NIB_POS = np.array([(e & 1) * 4 + (e >> 1) for e in range(8)], dtype=np.uint32)


def _check_wk(N: int, K: int) -> int:
    if K % BLK:
        raise ValueError(f"K={K} is not a multiple of {BLK}")
    return K // BLK


# --------------------------------------------------------------------------
# quantizer: src/vk_engine.py:125-159
# --------------------------------------------------------------------------
def quant_codes(W: np.ndarray):
    """int4 codes + fp32 block scales (``src/vk_engine.py:126-128``).

    ``sc[n, b] = max(max_k |W[n, 32b + k]| / 7, 1e-8)`` in float32, then
    ``q = clip(rint(W / sc) + 8, 0, 15)`` with an IEEE fp32 divide and numpy's
    round-half-to-even. Returns ``(q uint8 [N, K], sc float32 [N, nblk])``.
    Pinned by hand-computed known answers incl. half-way ties.
    """
    W = np.ascontiguousarray(W, dtype=np.float32)
    N, K = W.shape
    nblk = _check_wk(N, K)
    blocks = W.reshape(N, nblk, BLK)
    amax = np.abs(blocks).max(axis=2)                       # float32
    sc = np.maximum(amax / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    ratio = blocks / sc[:, :, None]                          # float32 divide
    codes = np.clip(np.rint(ratio) + np.float32(8.0), 0, 15)
    return codes.astype(np.uint8).reshape(N, K), sc


def pack_ref(q: np.ndarray) -> np.ndarray:
    """Reference N-packed nibble layout ``wp[K, N/8]`` (``src/vk_engine.py:129-130``).

    Nibble ``j`` (bits ``4j..4j+3``) of ``wp[k, i]`` is ``q[8i + j, k]``.
    Pinned by a per-bit brute-force loop and an exhaustive round trip.
    """
    N, K = q.shape
    if N % 8:
        raise ValueError("N must be a multiple of 8 for the reference layout")
    qT = np.ascontiguousarray(q.T).astype(np.uint32) & 15    # [K, N]
    grouped = qT.reshape(K, N // 8, 8)
    shifts = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    return np.bitwise_or.reduce(grouped << shifts, axis=2).astype(np.uint32)


def unpack_ref(wp: np.ndarray, N: int) -> np.ndarray:
    """Inverse of :func:`pack_ref` (the shaders' ``(wp[...] >> 4j) & 15``,
    ``vk/coopgemm_i4h.comp:21``). Returns ``q[N, K]`` uint8."""
    K = wp.shape[0]
    shifts = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    nib = (wp[:, :, None] >> shifts) & 15                    # [K, N/8, 8]
    return np.ascontiguousarray(nib.reshape(K, N).T).astype(np.uint8)


def scales_f16_ref(sc: np.ndarray) -> np.ndarray:
    """fp16 scale layout ``[nblk, N]`` (``src/vk_engine.py:131``): RNE to fp16."""
    return np.ascontiguousarray(sc.T).astype(np.float16)


def split_ref(N: int, nblk: int) -> int:
    """The reference's Adreno K-split heuristic (``src/vk_engine.py:143-148``).

    Informational only: the MI355X kernels choose their own split. Pinned by
    the values the reference's comments quote (lm_head -> 1, down -> 48,
    gate -> 12).
    """
    rows = (N // 8 + 63) // 64
    want = max(1, -(-384 // max(rows, 1)))
    divs = [s for s in range(1, nblk + 1) if nblk % s == 0]
    return min(divs, key=lambda s: (abs(s - want), s))


# --------------------------------------------------------------------------
# e4m3 (OCP E4M3FN: bias 7, no infinities, max 448)
# --------------------------------------------------------------------------
def e4m3_decode(b: np.ndarray) -> np.ndarray:
    """e4m3fn byte -> float32 (``vk/gemv_fp8.comp:14-18``).

    exp field 0: ``m * 2^-9``; else ``(1 + m/8) * 2^(e-7)``; sign bit 7.
    Pinned exhaustively (all 256 codes) against torch's float8_e4m3fn.
    Codes 0x7F/0xFF (NaN in e4m3fn) decode to 480 here exactly as the shader
    formula does; the encoder never produces them.
    """
    b = np.asarray(b, dtype=np.uint32)
    s = (b >> 7) & 1
    e = (b >> 3) & 15
    m = (b & 7).astype(np.float64)
    mag = np.where(e == 0, m / 512.0, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    return np.where(s == 1, -mag, mag).astype(np.float32)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn byte, round-half-to-even, for finite ``|v| <= 448``.

    This is the arithmetic of torch's ``.to(torch.float8_e4m3fn)`` that
    ``src/vk_engine.py:136`` calls, restated from the format definition
    (torch is a third-party dependency; pinned exhaustively against torch in
    ``tests/test_oracle.py``). Magnitudes above 448 are outside the domain the
    reference feeds it (it clips to ``[0, 448]`` first) and raise here.
    """
    v = np.asarray(v, dtype=np.float32).astype(np.float64)
    if np.any(~np.isfinite(v)) or np.any(np.abs(v) > 448.0):
        raise ValueError("e4m3_encode domain is finite |v| <= 448")
    sign = (v < 0) | ((v == 0) & np.signbit(v))
    a = np.abs(v)
    out = np.zeros(a.shape, dtype=np.uint32)
    sub = a < 2.0 ** -6
    # subnormal band: spacing 2^-9, codes 0..8 (8 == smallest normal)
    out[sub] = np.rint(a[sub] * 512.0).astype(np.uint32)
    nrm = ~sub
    mant, ex = np.frexp(a[nrm])              # a = mant * 2^ex, mant in [0.5, 1)
    e = ex - 1                               # a = (2 mant) * 2^e, 2 mant in [1, 2)
    m8 = np.rint(mant * 16.0).astype(np.int64)   # (1 + m/8) * 8, in [8, 16]
    carry = m8 == 16
    e = np.where(carry, e + 1, e)
    m8 = np.where(carry, 8, m8)
    out[nrm] = (((e + 7) << 3) | (m8 - 8)).astype(np.uint32)
    out = np.where(sign, out | 0x80, out)
    return out.astype(np.uint8)


def e4m3_lift(sc: np.ndarray):
    """Per-tensor power-of-two lift of the block scales into e4m3
    (``src/vk_engine.py:133-137``).

    ``shift = floor(log2(256 / max sc))`` (0 if the max is 0), scales times
    ``2^shift`` clipped to ``[0, 448]`` and rounded to e4m3, ``inv = 2^-shift``.
    Returns ``(e8 uint8 [N, nblk], inv float, shift int)``; the reference
    stores ``e8.T`` (``[nblk, N]``).
    """
    sc = np.asarray(sc, dtype=np.float32)
    mx = float(sc.max())
    shift = int(np.floor(np.log2(256.0 / mx))) if mx > 0 else 0
    lifted = np.clip(sc * np.float32(2.0 ** shift), np.float32(0.0), np.float32(448.0))
    return e4m3_encode(lifted), float(2.0 ** -shift), shift


# --------------------------------------------------------------------------
# device format of this build (panel-64)
# --------------------------------------------------------------------------
def _pad_rows(a: np.ndarray, fill) -> np.ndarray:
    N = a.shape[0]
    NP = -(-N // PANEL) * PANEL
    if NP == N:
        return a
    out = np.full((NP,) + a.shape[1:], fill, dtype=a.dtype)
    out[:N] = a
    return out


def pack_dev(q: np.ndarray) -> np.ndarray:
    """Codes ``q[N, K]`` -> panel-64 device words (uint32, flat)."""
    N, K = q.shape
    nblk = _check_wk(N, K)
    qp = _pad_rows(np.asarray(q, dtype=np.uint8), 8).astype(np.uint32) & 15
    NP = qp.shape[0]
    t = qp.reshape(NP // PANEL, PANEL, nblk, 4, 8).transpose(0, 2, 1, 3, 4)  # p,b,r,i,e
    words = np.bitwise_or.reduce(t << (4 * NIB_POS), axis=4)
    return np.ascontiguousarray(words).reshape(-1).astype(np.uint32)


def unpack_dev(words: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of :func:`pack_dev` (drops padded rows)."""
    nblk = _check_wk(N, K)
    NP = -(-N // PANEL) * PANEL
    w = np.asarray(words, dtype=np.uint32).reshape(NP // PANEL, nblk, PANEL, 4)
    nib = (w[..., None] >> (4 * NIB_POS)) & 15                      # p,b,r,i,e
    q = nib.transpose(0, 2, 1, 3, 4).reshape(NP, K)
    return q[:N].astype(np.uint8)


def scales_dev(s: np.ndarray) -> np.ndarray:
    """Per-(row, block) array ``s[N, nblk]`` -> panel-64 order (flat).

    Works for fp16 scales, e4m3 bytes and the fp16 W4A8 ratio alike; padded
    rows are zero.
    """
    N, nblk = s.shape
    sp = _pad_rows(np.asarray(s), 0)
    NP = sp.shape[0]
    return np.ascontiguousarray(sp.reshape(NP // PANEL, PANEL, nblk).transpose(0, 2, 1)).reshape(-1)


def unscales_dev(flat: np.ndarray, N: int, nblk: int) -> np.ndarray:
    NP = -(-N // PANEL) * PANEL
    return np.ascontiguousarray(np.asarray(flat).reshape(NP // PANEL, nblk, PANEL).transpose(0, 2, 1)).reshape(NP, nblk)[:N]


def pack_w8_dev(W8: np.ndarray) -> np.ndarray:
    """int8 ``W8[N, K]`` -> the packed W8A8 layout of this build (flat int8).

    Rows padded to a multiple of 32 and K to a multiple of 128 (``Kp``), the
    padding zero. The 32 x 32-byte block of n-tile ``t`` (rows ``32t ..
    32t+31``) and k-slice ``s`` (bytes ``32s .. 32s+31``) is 1 KB at byte
    ``(t * Kp/32 + s) * 1024``; its 16-byte chunk ``l`` (0..63) holds row
    ``32t + l % 32``, bytes ``32s + 16 (l // 32) .. +16``.
    """
    W8 = np.asarray(W8, dtype=np.int8)
    N, K = W8.shape
    if K % 32:
        raise ValueError(f"K={K} is not a multiple of 32")
    NP, Kp = -(-N // 32) * 32, -(-K // 128) * 128
    Wp = np.zeros((NP, Kp), np.int8)
    Wp[:N, :K] = W8
    t = Wp.reshape(NP // 32, 32, Kp // 32, 2, 16)          # t, r, s, h, byte
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(-1)   # t, s, h, r, byte


def unpack_w8_dev(flat: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of :func:`pack_w8_dev` (drops the padding)."""
    NP, Kp = -(-N // 32) * 32, -(-K // 128) * 128
    t = np.asarray(flat, dtype=np.int8).reshape(NP // 32, Kp // 32, 2, 32, 16)   # t, s, h, r, byte
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(NP, Kp)[:N, :K]


# --------------------------------------------------------------------------
# dequant + matmul references (the reference's own numpy checks)
# --------------------------------------------------------------------------
def dequant(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Exact fp32 dequant ``Wdq = (q - 8) * scale`` per block
    (``benchmarks/coopgemm_i4.py:51``). ``scale[N, nblk]`` float32."""
    N, K = q.shape
    nblk = _check_wk(N, K)
    codes = (q.astype(np.float32) - np.float32(8.0)).reshape(N, nblk, BLK)
    return (codes * np.asarray(scale, np.float32)[:, :, None]).reshape(N, K)


def gemv_ref(q: np.ndarray, scale: np.ndarray, x: np.ndarray, inv: float = 1.0) -> np.ndarray:
    """Decode GEMV ``y = Wdq @ x`` in fp32 (``vk/gemv.comp:16-32`` computes
    ``sum_k ((q-8) * s) * x``; ``vk/gemv_fp8.comp:39`` multiplies by ``inv``;
    the numpy form is ``benchmarks/coopgemm_i4.py:51-52``).

    ``scale`` is the scale the kernel reads, as float32 (fp16 scales
    upcast, or decoded e4m3). Pinned by a float64 brute-force loop.
    """
    y = dequant(q, scale) @ np.asarray(x, dtype=np.float32)
    return (y * np.float32(inv)).astype(np.float32)


def gemm_w4a16_ref(X: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """W4A16 prefill ``Y = X.f32 @ Wdq.T`` with exact fp32 Wdq
    (``benchmarks/coopgemm_i4.py:51-52``)."""
    return np.asarray(X, np.float32) @ dequant(q, scale).T


def quant_act_i8(X: np.ndarray):
    """Per-row symmetric int8 activation quantizer.

    Semantics of ``vk/cast_i8.comp:13-18`` with the numpy rounding of
    ``benchmarks/coopgemm_w4a8.py:87-88``: ``s = max(absmax / 127, 1e-12)``
    (fp32), ``a = clip(rint(x / s), -127, 127)`` with an IEEE fp32 divide.
    fp16 inputs are upcast to fp32 first (exact). Returns
    ``(A int8 [M, K], sa float32 [M])``. Pinned by tie and edge cases.
    """
    Xf = np.asarray(X).astype(np.float32)
    sa = np.maximum(np.abs(Xf).max(axis=1) / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    A = np.clip(np.rint(Xf / sa[:, None]), -127, 127).astype(np.int8)
    return A, sa


def w8_fold(q: np.ndarray, sc: np.ndarray):
    """Precomputed int8 weights for W8A8 (``src/vk_engine.py:152-157``).

    ``deqW = (q - 8) * sc`` (fp32, the UNROUNDED fp32 block scale),
    ``s_w[n] = max(max_k |deqW| / 127, 1e-12)``,
    ``W8 = clip(rint(deqW / s_w), -127, 127)``. Returns
    ``(W8 int8 [N, K], s_w float32 [N])``; the reference stores ``W8.T``
    (``[K, N]``) and ``s_w`` as fp16.
    """
    deqW = dequant(q, sc)
    s_w = np.maximum(np.abs(deqW).max(axis=1) / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    W8 = np.clip(np.rint(deqW / s_w[:, None]), -127, 127).astype(np.int8)
    return W8, s_w


def w4a8_ratio(sc: np.ndarray, s_w: np.ndarray) -> np.ndarray:
    """W4A8 requant ratio ``f16(sc / s_w)`` as ``[N, nblk]``
    (``benchmarks/coopgemm_w4a8.py:84``; the harness stores the transpose)."""
    return (np.asarray(sc, np.float32) / np.asarray(s_w, np.float32)[:, None]).astype(np.float16)


def w4a8_weights(q: np.ndarray, ratio: np.ndarray) -> np.ndarray:
    """On-the-fly int8 requant of the int4 codes (``vk/coopgemm_w4a8.comp:28-34``):
    ``int8(clamp(round((q - 8) * ratio[n, b]), -127, 127))`` in fp32. GLSL
    ``round`` leaves the .5 direction open; this build uses half-to-even.
    Returns ``B int8 [N, K]``."""
    N, K = q.shape
    nblk = _check_wk(N, K)
    r = np.asarray(ratio).astype(np.float32)[:, :, None]
    v = (q.astype(np.float32) - np.float32(8.0)).reshape(N, nblk, BLK) * r
    return np.clip(np.rint(v), -127, 127).astype(np.int8).reshape(N, K)


def int_matmul_exact(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """``C = A @ B.T`` for int8 ``A[M, K]``, ``B[N, K]``, exactly, as int32.

    Uses float64 BLAS: every product and partial sum is an integer of
    magnitude below ``127 * 127 * K < 2^53``, so float64 is exact in any
    summation order. Pinned against an int64 matmul on small shapes.
    """
    K = A.shape[1]
    if 127 * 127 * K >= 2 ** 31:
        raise ValueError("K too large for an int32 accumulator")
    C = A.astype(np.float64) @ B.astype(np.float64).T
    return C.astype(np.int64).astype(np.int32)


def w8a8_epilogue(C: np.ndarray, sa: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """``Y = f16((f32(C) * sa[m]) * sw[n])`` (``vk/coopgemm_w8a8.comp:32-35``),
    left-to-right fp32 products, RNE to fp16."""
    t = C.astype(np.float32) * np.asarray(sa, np.float32)[:, None]
    t = t * np.asarray(sw, np.float32)[None, :]
    return t.astype(np.float16)


def gemm_w8a8_ref(A, W8, sa, sw):
    """W8A8 GEMM reference: exact int32 ``C`` and fp16 ``Y``."""
    C = int_matmul_exact(A, W8)
    return C, w8a8_epilogue(C, sa, sw)


# --------------------------------------------------------------------------
# error metrics
# --------------------------------------------------------------------------
def normwise_rel_err(y, ref) -> float:
    """``max|y - ref| / max|ref|`` (per-element relative error is unbounded
    near zero outputs)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(y - ref).max() / den) if den > 0 else float(np.abs(y).max())


def cosine(a, b) -> float:
    """Cosine similarity, the reference's own quality metric
    (``benchmarks/vk_gemv.py:143``)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))
