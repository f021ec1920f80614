"""Writes ``tests/golden/q4_small.npz``: seeded inputs and expected outputs of
every step of the quantized matrix-product path at a small shape.

The reference ships no golden vectors for this path (its harnesses check
cosine thresholds only), so these fixtures are written here, once, from the
oracle, with two outputs computed independently of it:

* the e4m3 scale bytes come from ``torch``'s ``float8_e4m3fn`` conversion,
  the call the reference's quantizer makes (``src/vk_engine.py:136``);
* the W8A8 / W4A8 int32 accumulators come from an int64 numpy matmul.

Inputs follow the reference harnesses' seed convention
(``np.random.default_rng(0)``, ``benchmarks/vk_gemv.py:56``) and add rows
that hit the rounding edges: an all-zero weight block and activation row
(the 1e-8 / 1e-12 scale floors) and rows whose quotients are exact
half-way ties (numpy's round-half-to-even).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import q4_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "q4_small.npz"
M, N, K = 64, 96, 256


def inputs():
    rng = np.random.default_rng(0)
    W = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
    W[0, :32] = 0.0                                   # zero block: scale floor 1e-8
    c = np.float32(2.0 ** -6)                          # amax 7c -> scale exactly c
    W[1, :8] = c * np.array([7.0, 3.5, -2.5, 0.5, -0.5, 1.5, -7.0, 2.5], np.float32)
    W[2, 32:64] = c * (np.arange(32, dtype=np.float32) % 15 - 7.0)
    x = rng.standard_normal(K).astype(np.float16)
    X = rng.standard_normal((M, K)).astype(np.float16)
    X[0] = 0.0                                        # zero row: scale floor 1e-12
    X[1] = ((np.arange(K) % 254) - 127 + 0.5).astype(np.float16) / np.float16(16.0)
    X[1, 0] = np.float16(127.0 / 16.0)                 # absmax 127/16 -> s = 1/16 exactly
    return W, x, X


def torch_e4m3(v: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def build() -> dict:
    W, x, X = inputs()
    q, sc = O.quant_codes(W)
    wp = O.pack_ref(q)                                 # [K, N/8] reference words
    scb16 = O.scales_f16_ref(sc)                       # [nblk, N] fp16
    s16 = scb16.T.astype(np.float32)                   # the scale the f16 kernels read
    _, inv, shift = O.e4m3_lift(sc)
    lifted = np.clip(sc * np.float32(2.0 ** shift), np.float32(0.0), np.float32(448.0))
    e8 = torch_e4m3(lifted)                            # [N, nblk], torch's encoder
    W8, sw32 = O.w8_fold(q, sc)
    sw16 = sw32.astype(np.float16)
    ratio = O.w4a8_ratio(sc, sw32)
    B48 = O.w4a8_weights(q, ratio)
    A, sa = O.quant_act_i8(X)
    C = (A.astype(np.int64) @ W8.astype(np.int64).T).astype(np.int32)
    C48 = (A.astype(np.int64) @ B48.astype(np.int64).T).astype(np.int32)
    return dict(
        M=np.int32(M), N=np.int32(N), K=np.int32(K),
        W=W, x=x, X=X,
        q=q, sc=sc, wp_ref=wp, scb16_ref=scb16,
        e8=e8, e4m3_inv=np.float32(inv), e4m3_shift=np.int32(shift),
        W8=W8, sw32=sw32, sw16=sw16, ratio=ratio, W8_w4a8=B48,
        y_f16s=O.gemv_ref(q, s16, x),
        y_e4m3=O.gemv_ref(q, O.e4m3_decode(e8), x, inv=inv),
        A=A, sa=sa,
        C_w8a8=C, Y_w8a8_sw32=O.w8a8_epilogue(C, sa, sw32), Y_w8a8_sw16=O.w8a8_epilogue(C, sa, sw16),
        C_w4a8=C48, Y_w4a8=O.w8a8_epilogue(C48, sa, sw32),
        Y_w4a16=O.gemm_w4a16_ref(X, q, s16),
    )


def main() -> None:
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
