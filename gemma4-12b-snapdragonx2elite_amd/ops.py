"""Functional API over libq4mi: torch tensors in, torch tensors out.

PyTorch is only plumbing here (device memory, streams); every byte of
arithmetic runs in the HIP kernels of libq4mi.so. All tensors must be CUDA
(ROCm) tensors on the current device; work is enqueued on torch's current
stream. Storage dtypes: panel-64 weight words as int32, fp16 values as
float16, e4m3 bytes as uint8, int8 as int8.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import DT_F16, DT_F32, GEMV_MAX_BATCH, OP_GEMV, SCALE_E4M3, SCALE_F16, call, lib

BLK = 32
PANEL = 64


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _p(t) -> C.c_void_p:
    if t is None:
        return C.c_void_p(0)
    if isinstance(t, int):
        return C.c_void_p(t)
    if not t.is_cuda:
        raise ValueError("libq4mi takes device tensors only")
    if not t.is_contiguous():
        raise ValueError("libq4mi takes contiguous tensors only")
    return C.c_void_p(t.data_ptr())


def _dt(t) -> int:
    if t.dtype == torch.float32:
        return DT_F32
    if t.dtype == torch.float16:
        return DT_F16
    raise ValueError(f"unsupported dtype {t.dtype} (float32 or float16)")


def dev_sizes(N: int, K: int):
    """(bytes of the panel-64 words, number of per-(row, block) scale entries)."""
    wb, se = C.c_size_t(), C.c_size_t()
    call("q4_dev_bytes", N, K, C.byref(wb), C.byref(se))
    return wb.value, se.value


def tune_set(knob: str, value: int | None) -> None:
    """Plan override for tests and tuning sweeps (q4_tune_set): ``knob`` is a
    name of ``_lib.TUNE_KNOBS``; None clears it. Applies to every later call
    in the process."""
    call("q4_tune_set", _lib.TUNE_KNOBS[knob], -1 if value is None else int(value))


def tune_reset() -> None:
    """Clear every plan override (q4_tune_reset)."""
    lib().q4_tune_reset()


def _nbytes(t) -> int:
    return t.numel() * t.element_size()


def _need(t, nbytes: int, what: str) -> None:
    """Host-side bound check: the kernels trust these sizes."""
    if t is None or _nbytes(t) < nbytes:
        got = None if t is None else _nbytes(t)
        raise ValueError(f"{what}: need {nbytes} bytes, got {got}")


def _check_int4(wq, scales, N, K, scale_bytes=2):
    wb, se = dev_sizes(N, K)
    _need(wq, wb, "panel-64 weight words")
    _need(scales, se * scale_bytes, "panel-64 scales")


def _empty_weights(N, K, device):
    wb, se = dev_sizes(N, K)
    return torch.empty(wb // 4, dtype=torch.int32, device=device), se


# ---------------------------------------------------------------- weights
def quantize(W: torch.Tensor):
    """W float32 [N, K] (device) -> (wq int32 words, sc16 float16 panel, sc32 float32 [N, K/32])."""
    if W.dtype != torch.float32 or W.dim() != 2:
        raise ValueError("quantize expects a 2-D float32 tensor")
    W = W.contiguous()
    N, K = W.shape
    wq, se = _empty_weights(N, K, W.device)
    sc16 = torch.empty(se, dtype=torch.float16, device=W.device)
    sc32 = torch.empty((N, K // BLK), dtype=torch.float32, device=W.device)
    call("q4_quantize", _p(W), N, K, _p(wq), _p(sc16), _p(sc32), _stream())
    return wq, sc16, sc32


def scales_e4m3(sc32: torch.Tensor, N: int, K: int):
    """fp32 scales [N, K/32] -> (e4m3 panel bytes uint8, inv float). Synchronizes once to read inv."""
    _, se = dev_sizes(N, K)
    sc8 = torch.empty(se, dtype=torch.uint8, device=sc32.device)
    inv = torch.empty(1, dtype=torch.float32, device=sc32.device)
    work = torch.empty(1, dtype=torch.int32, device=sc32.device)
    call("q4_scales_e4m3", _p(sc32.contiguous()), N, K, _p(sc8), _p(inv), _p(work), _stream())
    return sc8, float(inv.item())


def w8_fold(wq: torch.Tensor, sc32: torch.Tensor, N: int, K: int):
    """-> (W8 int8 [N, K], s_w float32 [N], s_w float16 [N])."""
    W8 = torch.empty((N, K), dtype=torch.int8, device=wq.device)
    sw32 = torch.empty(N, dtype=torch.float32, device=wq.device)
    sw16 = torch.empty(N, dtype=torch.float16, device=wq.device)
    call("q4_w8_fold", _p(wq), _p(sc32.contiguous()), N, K, _p(W8), _p(sw32), _p(sw16), _stream())
    return W8, sw32, sw16


def w4a8_ratio(sc32: torch.Tensor, sw32: torch.Tensor, N: int, K: int) -> torch.Tensor:
    _, se = dev_sizes(N, K)
    ratio = torch.empty(se, dtype=torch.float16, device=sc32.device)
    call("q4_w4a8_ratio", _p(sc32.contiguous()), _p(sw32), N, K, _p(ratio), _stream())
    return ratio


def repack_ref(wp: torch.Tensor | None, sc_ref: torch.Tensor | None, N: int, K: int):
    """Reference layouts (wp [K, N/8] words, fp16 scales [K/32, N]) -> (wq, sc16 panel)."""
    dev = (wp if wp is not None else sc_ref).device
    wq, se = _empty_weights(N, K, dev) if wp is not None else (None, dev_sizes(N, K)[1])
    sc = torch.empty(se, dtype=torch.float16, device=dev) if sc_ref is not None else None
    call("q4_repack_ref", _p(wp), _p(sc_ref), N, K, _p(wq), _p(sc), _stream())
    return wq, sc


def repack_e4m3_ref(sc_ref: torch.Tensor, N: int, K: int) -> torch.Tensor:
    _, se = dev_sizes(N, K)
    out = torch.empty(se, dtype=torch.uint8, device=sc_ref.device)
    call("q4_repack_e4m3_ref", _p(sc_ref), N, K, _p(out), _stream())
    return out


def repack_w8_ref(w8_kn: torch.Tensor, N: int, K: int) -> torch.Tensor:
    out = torch.empty((N, K), dtype=torch.int8, device=w8_kn.device)
    call("q4_repack_w8_ref", _p(w8_kn), N, K, _p(out), _stream())
    return out


# ------------------------------------------------------------------ GEMV
class Workspace:
    """Caller-owned split-K workspace (fp32 partials + per-panel tickets).

    Zero-filled once at creation; every GEMV leaves it ready for the next
    one, so it can be shared by all GEMVs issued in order on one stream
    (including inside a captured hipGraph). Do not share across streams.
    """

    def __init__(self, nbytes: int, device="cuda"):
        self.nbytes = int(nbytes)
        self.t = torch.empty(max(self.nbytes, 256), dtype=torch.uint8, device=device)
        call("q4_workspace_init", _p(self.t), self.t.numel(), _stream())

    @staticmethod
    def bytes_for(N: int, K: int, split: int = 0) -> int:
        return int(lib().q4_workspace_bytes(OP_GEMV, N, K, split))

    @property
    def ptr(self):
        return self.t.data_ptr()


def auto_split(N: int, K: int) -> int:
    return int(lib().q4_gemv_auto_split(N, K))


_WS = {}
_CAPTURING = [0]   # > 0 while a Graph capture is open on this thread


def default_workspace(N: int, K: int, split: int = 0, device="cuda") -> Workspace | None:
    """A per-device workspace big enough for this GEMV (grown, never shrunk)."""
    need = Workspace.bytes_for(N, K, split)
    if need == 0:
        return None
    if _CAPTURING[0]:
        raise RuntimeError("a split-K GEMV inside a graph capture needs a workspace allocated before "
                           "the capture (pass ws=...); allocating and zero-filling one cannot be captured")
    key = torch.device(device).index if torch.device(device).index is not None else torch.cuda.current_device()
    ws = _WS.get(key)
    if ws is None or ws.nbytes < need:
        if ws is not None:  # keep the old one alive: descriptors/graphs may still point at it
            _WS.setdefault(("old", key), []).append(ws)
        ws = Workspace(max(need, 1 << 20), device=device)
        _WS[key] = ws
    return ws


def gemv(x: torch.Tensor, wq: torch.Tensor, scales: torch.Tensor, N: int, K: int, *, scale_fmt: int = SCALE_F16,
         inv: float = 1.0, y: torch.Tensor | None = None, y_dtype=None, split: int = 0,
         ws: Workspace | None = None) -> torch.Tensor:
    """y[N] = sum_k ((q-8) * s) * x[k] (fp32 accumulate; times inv for e4m3 scales)."""
    if x.numel() != K:
        raise ValueError(f"x has {x.numel()} elements, expected K={K}")
    if y is None:
        y = torch.empty(N, dtype=y_dtype or x.dtype, device=x.device)
    elif y.numel() < N:
        raise ValueError("y too small")
    _check_int4(wq, scales, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
    _need(y, N * y.element_size(), "y")
    if ws is None:
        ws = default_workspace(N, K, split, x.device)
    call("q4_gemv", _p(x), _dt(x), _p(wq), _p(scales), scale_fmt, C.c_float(inv), _p(y), _dt(y), N, K, split,
         _p(ws.t) if ws else C.c_void_p(0), ws.t.numel() if ws else 0, _stream())
    return y


GEMV_MAX_VECTORS = 16


def gemv_multi_workspace_bytes(M: int, N: int, K: int) -> int:
    """Bytes of the K-split workspace of the MFMA small-M GEMV (0: unsplit)."""
    return int(lib().q4_gemv_multi_workspace_bytes(M, N, K))


def gemv_multi(x: torch.Tensor, wq: torch.Tensor, scales: torch.Tensor, N: int, K: int, *,
               scale_fmt: int = SCALE_F16, inv: float = 1.0, y: torch.Tensor | None = None,
               y_dtype=None, exact: bool = False, ws: torch.Tensor | None = None,
               ksplit: bool = True) -> torch.Tensor:
    """Y[m] = GEMV of x[m] for the M fp16 rows of ``x`` [M][K] (M <= 16),
    reading the weights once. ``exact``: every row bit-identical to
    :func:`gemv` of that row when :func:`gemv` runs unsplit (VALU path, one
    weight stream per 2-8 vectors); otherwise the MFMA path, equal to
    :func:`gemv` to fp32 rounding: one launch, or for matrices of fewer than
    15360 rows and K >= 2048 a K-split launch into fp32 partials plus their
    reduce — pass
    ``ws`` (at least :func:`gemv_multi_workspace_bytes` bytes) or one is
    allocated here; capture code must pass its own. ``ksplit=False`` runs
    the MFMA path unsplit whatever the shape. Returns Y [M][N]."""
    if x.dtype != torch.float16:
        raise ValueError("multi-vector GEMV takes fp16 activations")
    if x.dim() != 2 or x.shape[1] != K or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous [M][K={K}] tensor")
    M = x.shape[0]
    if not 1 <= M <= GEMV_MAX_VECTORS:
        raise ValueError(f"multi-vector GEMV takes 1..{GEMV_MAX_VECTORS} vectors (got {M})")
    if y is None:
        y = torch.empty(M, N, dtype=y_dtype or torch.float16, device=x.device)
    elif y.dim() != 2 or tuple(y.shape) != (M, N) or not y.is_contiguous():
        raise ValueError(f"y must be a contiguous [{M}][{N}] tensor")
    _check_int4(wq, scales, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
    if exact:
        call("q4_gemv_multi", _p(x), M, _p(wq), _p(scales), scale_fmt, C.c_float(inv), _p(y), _dt(y), N, K, 1,
             _stream())
        return y
    need = gemv_multi_workspace_bytes(M, N, K) if ksplit else 0
    if not ksplit:
        ws = None
    if need and ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("a K-split small-M GEMV inside a graph capture needs a workspace allocated before "
                               "the capture (pass ws=...)")
        ws = torch.empty(need, dtype=torch.uint8, device=x.device)
    if ws is not None:
        _need(ws, need, "small-M GEMV split-K workspace")
    call("q4_gemv_multi_ws", _p(x), M, _p(wq), _p(scales), scale_fmt, C.c_float(inv), _p(y), _dt(y), N, K,
         _p(ws), _nbytes(ws) if ws is not None else 0, _stream())
    return y


def interleave_rows(wa: torch.Tensor, sa: torch.Tensor, wb: torch.Tensor, sb: torch.Tensor, N: int, K: int):
    """Gate/up matrices (panel-64, N rows each) -> one of 2N rows, row 2i from
    ``wa``/``sa`` and row 2i + 1 from ``wb``/``sb`` (the layout of :func:`gemv_gated`)."""
    sbytes = sa.element_size()
    if sb.element_size() != sbytes:
        raise ValueError("both scale arrays must have the same element size")
    _check_int4(wa, sa, N, K, sbytes)
    _check_int4(wb, sb, N, K, sbytes)
    wo, se = _empty_weights(2 * N, K, wa.device)
    so = torch.empty(se, dtype=sa.dtype, device=wa.device)
    call("q4_interleave_rows", _p(wa), _p(sa), _p(wb), _p(sb), N, K, sbytes, _p(wo), _p(so), _stream())
    return wo, so


def gemv_gated(x: torch.Tensor, wq: torch.Tensor, scales: torch.Tensor, N: int, K: int, *,
               scale_fmt: int = SCALE_F16, inv: float = 1.0, act: torch.Tensor | None = None, act_dtype=None,
               split: int = 0, ws: Workspace | None = None) -> torch.Tensor:
    """act[i] = gelu_tanh(y[2i]) * y[2i+1] of the GEMV y over an interleaved
    gate/up matrix of N rows (:func:`interleave_rows`); act has N/2 elements."""
    if x.numel() != K:
        raise ValueError(f"x has {x.numel()} elements, expected K={K}")
    if N % 2:
        raise ValueError("gated GEMV needs an even row count")
    if act is None:
        act = torch.empty(N // 2, dtype=act_dtype or x.dtype, device=x.device)
    _check_int4(wq, scales, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
    _need(act, (N // 2) * act.element_size(), "act")
    if ws is None:
        ws = default_workspace(N, K, split, x.device)
    call("q4_gemv_gated", _p(x), _dt(x), _p(wq), _p(scales), scale_fmt, C.c_float(inv), _p(act), _dt(act), N, K,
         split, _p(ws.t) if ws else C.c_void_p(0), ws.t.numel() if ws else 0, _stream())
    return act


def gemv_batch_max_k(x_dtype) -> int:
    """Largest K a batched GEMV stages for this activation dtype."""
    return 32768 if x_dtype == torch.float16 else 16384


def gemv_batch(x: torch.Tensor, mats, K: int, *, scale_fmt: int = SCALE_F16, y_dtype=None):
    """Several GEMVs over one activation ``x`` in one launch.

    ``mats``: sequence of ``(wq, scales, N, y, inv)`` (``y`` may be None: a new
    tensor; ``inv`` only matters for e4m3 scales). Returns the list of outputs.
    Every output gets the arithmetic of :func:`gemv` with split 1."""
    n = len(mats)
    if not 1 <= n <= GEMV_MAX_BATCH:
        raise ValueError(f"gemv_batch takes 1..{GEMV_MAX_BATCH} matrices, got {n}")
    if x.numel() != K:
        raise ValueError(f"x has {x.numel()} elements, expected K={K}")
    ys, keep = [], []
    wqs, scs, yps = (C.c_void_p * n)(), (C.c_void_p * n)(), (C.c_void_p * n)()
    Ns, invs = (C.c_int * n)(), (C.c_float * n)()
    ydt = None
    for i, (wq, sc, N, y, inv) in enumerate(mats):
        if y is None:
            y = torch.empty(N, dtype=y_dtype or x.dtype, device=x.device)
        _check_int4(wq, sc, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
        _need(y, N * y.element_size(), f"y of batch entry {i}")
        if ydt is None:
            ydt = _dt(y)
        elif _dt(y) != ydt:
            raise ValueError("all outputs of a GEMV batch must share one dtype")
        wqs[i], scs[i], yps[i] = _p(wq), _p(sc), _p(y)
        Ns[i], invs[i] = int(N), float(inv if inv is not None else 1.0)
        ys.append(y)
        keep.append((wq, sc))
    call("q4_gemv_batch", _p(x), _dt(x), K, scale_fmt, ydt, n, wqs, scs, invs, yps, Ns, _stream())
    return ys


GEMV_NORMADD_MAX_K = 4096


def _norm_in(a, w, h, h_out, w2, K: int):
    """Checks of the fused normadd + rmsnorm operands of a GEMV."""
    for t, nm in ((a, "a"), (w, "w"), (h, "h"), (h_out, "h_out"), (w2, "w2")):
        _f32(t, K, nm)
    if K > GEMV_NORMADD_MAX_K:
        raise ValueError(f"a GEMV with a fused norm input takes K <= {GEMV_NORMADD_MAX_K}, got {K}")
    lo, hi = h_out.data_ptr(), h_out.data_ptr() + 4 * K
    for t, nm in ((a, "a"), (w, "w"), (h, "h"), (w2, "w2")):
        if t.data_ptr() < hi and lo < t.data_ptr() + 4 * K:
            raise ValueError(f"h_out must not overlap {nm}")


def _norm_out(y, nbytes: int, a, w, h, h_out, w2, K: int) -> None:
    """A fused-norm GEMV's output must not overlap its norm operands or h_out:
    early workgroups write y while later ones still read a and h."""
    lo, hi = y.data_ptr(), y.data_ptr() + nbytes
    for t, nm in ((a, "a"), (w, "w"), (h, "h"), (h_out, "h_out"), (w2, "w2")):
        if t.data_ptr() < hi and lo < t.data_ptr() + 4 * K:
            raise ValueError(f"y must not overlap {nm}")


def gemv_normadd(a: torch.Tensor, w: torch.Tensor, h: torch.Tensor, h_out: torch.Tensor, w2: torch.Tensor,
                 wq: torch.Tensor, scales: torch.Tensor, N: int, K: int, *, scale: float = 0.0,
                 scale_fmt: int = SCALE_F16, inv: float = 1.0, y: torch.Tensor | None = None,
                 y_dtype=torch.float32, gated: bool = False) -> torch.Tensor:
    """:func:`normadd_rmsnorm` (fp16 norm output, into ``h_out`` instead of
    ``h`` in place) and the GEMV (or, with ``gated``, :func:`gemv_gated`)
    that reads its output, in one launch; returns ``y`` (``act`` when gated)."""
    _norm_in(a, w, h, h_out, w2, K)
    if gated and N % 2:
        raise ValueError("gated GEMV needs an even row count")
    rows = N // 2 if gated else N
    if y is None:
        y = torch.empty(rows, dtype=y_dtype, device=a.device)
    _check_int4(wq, scales, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
    _need(y, rows * y.element_size(), "y")
    _norm_out(y, rows * y.element_size(), a, w, h, h_out, w2, K)
    call("q4_gemv_normadd", _p(a), _p(w), _p(h), _p(h_out), C.c_float(scale), _p(w2), _p(wq), _p(scales),
         scale_fmt, C.c_float(inv), _p(y), _dt(y), N, K, int(gated), _stream())
    return y


def gemv_batch_normadd(a: torch.Tensor, w: torch.Tensor, h: torch.Tensor, h_out: torch.Tensor, w2: torch.Tensor,
                       mats, K: int, *, scale: float = 0.0, scale_fmt: int = SCALE_F16, y_dtype=torch.float32):
    """:func:`gemv_batch` whose x is formed as in :func:`gemv_normadd`.
    ``mats``: sequence of ``(wq, scales, N, y, inv)``; returns the outputs."""
    _norm_in(a, w, h, h_out, w2, K)
    n = len(mats)
    if not 1 <= n <= GEMV_MAX_BATCH:
        raise ValueError(f"gemv_batch_normadd takes 1..{GEMV_MAX_BATCH} matrices, got {n}")
    ys = []
    wqs, scs, yps = (C.c_void_p * n)(), (C.c_void_p * n)(), (C.c_void_p * n)()
    Ns, invs = (C.c_int * n)(), (C.c_float * n)()
    ydt = None
    for i, (wq, sc, N, y, inv) in enumerate(mats):
        if y is None:
            y = torch.empty(N, dtype=y_dtype, device=a.device)
        _check_int4(wq, sc, N, K, 1 if scale_fmt == SCALE_E4M3 else 2)
        _need(y, N * y.element_size(), f"y of batch entry {i}")
        _norm_out(y, N * y.element_size(), a, w, h, h_out, w2, K)
        if ydt is None:
            ydt = _dt(y)
        elif _dt(y) != ydt:
            raise ValueError("all outputs of a GEMV batch must share one dtype")
        wqs[i], scs[i], yps[i] = _p(wq), _p(sc), _p(y)
        Ns[i], invs[i] = int(N), float(inv if inv is not None else 1.0)
        ys.append(y)
    call("q4_gemv_batch_normadd", _p(a), _p(w), _p(h), _p(h_out), C.c_float(scale), _p(w2), K, scale_fmt, ydt, n,
         wqs, scs, invs, yps, Ns, _stream())
    return ys


# ------------------------------------------------------------------ GEMMs
def gemm_w4a16(X: torch.Tensor, wq: torch.Tensor, sc16: torch.Tensor, N: int, Y: torch.Tensor | None = None,
               ws: torch.Tensor | None = None):
    """Y f16 [M, N] = X f16 [M, K] @ f16((q-8) * s)^T (fp32 accumulate).

    Tall-K shapes split K across workgroups into fp32 partials: pass ``ws``
    (a device tensor of at least ``gemm_workspace_bytes(M, N, K)`` bytes) or
    one is allocated here; capture code must pass its own."""
    if X.dtype != torch.float16 or X.dim() != 2:
        raise ValueError("X must be a 2-D float16 tensor")
    M, K = X.shape
    _check_int4(wq, sc16, N, K)
    Y = torch.empty((M, N), dtype=torch.float16, device=X.device) if Y is None else Y
    _need(Y, M * N * 2, "Y")
    need = gemm_workspace_bytes(M, N, K)
    if need and ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("a split-K W4A16 GEMM inside a graph capture needs a workspace allocated before "
                               "the capture (pass ws=...)")
        ws = torch.empty(need, dtype=torch.uint8, device=X.device)
    if ws is not None:
        _need(ws, need, "W4A16 split-K workspace")
    call("q4_gemm_w4a16_ws", _p(X), _p(wq), _p(sc16), _p(Y), M, N, K, _p(ws), _nbytes(ws) if ws is not None else 0,
         _stream())
    return Y


def gemm_w4a16_gated(X: torch.Tensor, wq: torch.Tensor, sc16: torch.Tensor, N: int, Y: torch.Tensor | None = None,
                     ws: torch.Tensor | None = None):
    """Y f16 [M, N/2] = gelu_tanh(G) * U of the W4A16 product over an
    interleaved gate/up matrix of N rows (:func:`interleave_rows`), G and U
    rounded to fp16 first (the reference's p_g, p_u then p_gm). ``ws``: at
    least ``gemm_gated_workspace_bytes(M, N, K)`` bytes (allocated here when
    omitted; capture code must pass its own)."""
    if X.dtype != torch.float16 or X.dim() != 2:
        raise ValueError("X must be a 2-D float16 tensor")
    if N % 2:
        raise ValueError("gated W4A16 needs an even row count (interleaved gate/up rows)")
    M, K = X.shape
    _check_int4(wq, sc16, N, K)
    Y = torch.empty((M, N // 2), dtype=torch.float16, device=X.device) if Y is None else Y
    _need(Y, M * (N // 2) * 2, "Y")
    need = gemm_gated_workspace_bytes(M, N, K)
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("a gated W4A16 GEMM inside a graph capture needs a workspace allocated before the "
                               "capture (pass ws=...)")
        ws = torch.empty(need, dtype=torch.uint8, device=X.device)
    _need(ws, need, "gated W4A16 workspace")
    call("q4_gemm_w4a16_gated", _p(X), _p(wq), _p(sc16), _p(Y), M, N, K, _p(ws), _nbytes(ws), _stream())
    return Y


def gemm_gated_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes of :func:`gemm_w4a16_gated` (fp32 partials, at least one split)."""
    return int(lib().q4_gemm_w4a16_gated_workspace_bytes(M, N, K))


def gemm_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes of a W4A16 GEMM (0 when it runs without splitting K)."""
    return int(lib().q4_gemm_workspace_bytes(_lib.OP_W4A16, M, N, K))


def quant_act_i8(X: torch.Tensor, A: torch.Tensor | None = None, sa: torch.Tensor | None = None):
    M, K = X.shape
    A = torch.empty((M, K), dtype=torch.int8, device=X.device) if A is None else A
    sa = torch.empty(M, dtype=torch.float32, device=X.device) if sa is None else sa
    _need(A, M * K, "A")
    _need(sa, M * 4, "sa")
    call("q4_quant_act_i8", _p(X), _dt(X), _p(A), _p(sa), M, K, _stream())
    return A, sa


def gemm_w8a8(A: torch.Tensor, W8: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, *, want_c: bool = False,
              Y: torch.Tensor | None = None):
    M, K = A.shape
    N = W8.shape[0]
    if A.dtype != torch.int8 or W8.dtype != torch.int8 or W8.dim() != 2 or W8.shape[1] != K:
        raise ValueError("gemm_w8a8 expects int8 A [M, K] and int8 W8 [N, K]")
    _need(sa, M * 4, "sa")
    _need(sw, N * sw.element_size(), "sw")
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device) if Y is None else Y
    _need(Y, M * N * 2, "Y")
    Cm = torch.empty((M, N), dtype=torch.int32, device=A.device) if want_c else None
    call("q4_gemm_w8a8", _p(A), _p(W8), _p(sa), _p(sw), _dt(sw), _p(Y), _p(Cm), M, N, K, _stream())
    return (Y, Cm) if want_c else Y


def w8_pack(W8: torch.Tensor) -> torch.Tensor:
    """int8 W8 [N, K] -> the packed layout of :func:`gemm_w8a8_packed` (flat int8)."""
    if W8.dtype != torch.int8 or W8.dim() != 2:
        raise ValueError("w8_pack expects int8 W8 [N, K]")
    N, K = W8.shape
    out = torch.empty(int(lib().q4_w8_packed_bytes(N, K)), dtype=torch.int8, device=W8.device)
    call("q4_w8_pack", _p(W8.contiguous()), N, K, _p(out), _stream())
    return out


def gemm_w8a8_packed(A: torch.Tensor, W8p: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, N: int, *,
                     want_c: bool = False, Y: torch.Tensor | None = None, stamps: torch.Tensor | None = None):
    """W8A8 on packed weights (:func:`w8_pack`); same results as :func:`gemm_w8a8`.
    ``stamps`` (int64 [w8a8_workgroups(M, N, K), 4]) takes the stamped launch:
    per workgroup the wall clock at start / after the k-loop / at the end and
    the shader cycles from start to end."""
    M, K = A.shape
    if A.dtype != torch.int8 or W8p.dtype != torch.int8:
        raise ValueError("gemm_w8a8_packed expects int8 A [M, K] and packed int8 weights")
    _need(W8p, int(lib().q4_w8_packed_bytes(N, K)), "packed W8")
    _need(sa, M * 4, "sa")
    _need(sw, N * sw.element_size(), "sw")
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device) if Y is None else Y
    _need(Y, M * N * 2, "Y")
    Cm = torch.empty((M, N), dtype=torch.int32, device=A.device) if want_c else None
    if stamps is None:
        call("q4_gemm_w8a8_packed", _p(A), _p(W8p), _p(sa), _p(sw), _dt(sw), _p(Y), _p(Cm), M, N, K, _stream())
    else:
        call("q4_gemm_w8a8_packed_stamped", _p(A), _p(W8p), _p(sa), _p(sw), _dt(sw), _p(Y), _p(Cm), M, N, K,
             _p(stamps), _nbytes(stamps), _stream())
    return (Y, Cm) if want_c else Y


def w8a8_workgroups(M: int, N: int, K: int) -> int:
    """Workgroups of one :func:`gemm_w8a8_packed` launch (rows of its stamps)."""
    return int(lib().q4_gemm_w8a8_packed_workgroups(M, N, K))


def w4a8_weights(wq: torch.Tensor, ratio: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """The int8 weights W4A8 forms on the fly, once: W8 [N][K] (pack with
    :func:`w8_pack` and run :func:`gemm_w8a8_packed` for W4A8's results at
    the W8A8 speed)."""
    _check_int4(wq, ratio, N, K)
    W8 = torch.empty((N, K), dtype=torch.int8, device=wq.device)
    call("q4_w4a8_weights", _p(wq), _p(ratio), N, K, _p(W8), _stream())
    return W8


def gemm_w4a8(A: torch.Tensor, wq: torch.Tensor, ratio: torch.Tensor, sa: torch.Tensor, sw: torch.Tensor, N: int, *,
              want_c: bool = False, Y: torch.Tensor | None = None):
    M, K = A.shape
    if A.dtype != torch.int8:
        raise ValueError("gemm_w4a8 expects int8 A [M, K]")
    _check_int4(wq, ratio, N, K)
    _need(sa, M * 4, "sa")
    _need(sw, N * sw.element_size(), "sw")
    Y = torch.empty((M, N), dtype=torch.float16, device=A.device) if Y is None else Y
    _need(Y, M * N * 2, "Y")
    Cm = torch.empty((M, N), dtype=torch.int32, device=A.device) if want_c else None
    call("q4_gemm_w4a8", _p(A), _p(wq), _p(ratio), _p(sa), _p(sw), _dt(sw), _p(Y), _p(Cm), M, N, K, _stream())
    return (Y, Cm) if want_c else Y


def cast_f32_f16(src: torch.Tensor, dst: torch.Tensor | None = None) -> torch.Tensor:
    dst = torch.empty(src.shape, dtype=torch.float16, device=src.device) if dst is None else dst
    _need(dst, src.numel() * 2, "dst")
    call("q4_cast_f32_f16", _p(src), _p(dst), src.numel(), _stream())
    return dst


def cast_f16_f32(src: torch.Tensor, dst: torch.Tensor | None = None) -> torch.Tensor:
    dst = torch.empty(src.shape, dtype=torch.float32, device=src.device) if dst is None else dst
    _need(dst, src.numel() * 4, "dst")
    call("q4_cast_f16_f32", _p(src), _p(dst), src.numel(), _stream())
    return dst


# ------------------------------------------------------ decode-token ops
def _f32(t, n: int, what: str) -> None:
    if t.dtype != torch.float32:
        raise ValueError(f"{what} must be float32")
    _need(t, 4 * n, what)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor | None = None, y_dtype=torch.float32) -> torch.Tensor:
    """y = x / sqrt(mean(x^2) + 1e-6) * w over the whole of ``x`` (fp32)."""
    D = x.numel()
    _f32(x, D, "x")
    _f32(w, D, "w")
    y = torch.empty(D, dtype=y_dtype, device=x.device) if y is None else y
    _need(y, D * y.element_size(), "y")
    call("q4_rmsnorm", _p(x), _p(w), _p(y), _dt(y), D, _stream())
    return y


def normadd(x: torch.Tensor, w: torch.Tensor, h: torch.Tensor, scale: float = 0.0) -> torch.Tensor:
    """h = (h + rmsnorm(x) * w) * scale in place (scale 0: unscaled)."""
    D = x.numel()
    for t, nm in ((x, "x"), (w, "w"), (h, "h")):
        _f32(t, D, nm)
    call("q4_normadd", _p(x), _p(w), _p(h), D, C.c_float(scale), _stream())
    return h


def normadd_rmsnorm(x: torch.Tensor, w: torch.Tensor, h: torch.Tensor, w2: torch.Tensor, scale: float = 0.0,
                    y: torch.Tensor | None = None, y_dtype=torch.float32) -> torch.Tensor:
    """:func:`normadd` then :func:`rmsnorm` of the new ``h`` with ``w2``, one launch; returns ``y``."""
    D = x.numel()
    for t, nm in ((x, "x"), (w, "w"), (h, "h"), (w2, "w2")):
        _f32(t, D, nm)
    y = torch.empty(D, dtype=y_dtype, device=x.device) if y is None else y
    _need(y, D * y.element_size(), "y")
    call("q4_normadd_rmsnorm", _p(x), _p(w), _p(h), D, C.c_float(scale), _p(w2), _p(y), _dt(y), _stream())
    return y


def gelumul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None, out_dtype=torch.float32):
    """out = gelu_tanh(gate) * up (fp32 in)."""
    n = gate.numel()
    _f32(gate, n, "gate")
    _f32(up, n, "up")
    out = torch.empty(n, dtype=out_dtype, device=gate.device) if out is None else out
    _need(out, n * out.element_size(), "out")
    call("q4_gelumul", _p(gate), _p(up), _p(out), _dt(out), n, _stream())
    return out


def _kv_checks(kc, vc, nkv, stride, hd, dyn):
    for t, nm in ((kc, "kc"), (vc, "vc")):
        if t.dtype != torch.float16:
            raise ValueError(f"{nm} must be float16")
        _need(t, 2 * nkv * stride * hd, nm)
    if dyn.dtype != torch.int32 or dyn.numel() < 1 or not dyn.is_cuda:
        raise ValueError("dyn must be a device int32 tensor holding the position")


def prepkv(qkv, knw, cosb, sinb, kc, vc, *, nkv: int, hd: int, koff: int, voff: int, keqv: bool, stride: int,
           window: int, dyn: torch.Tensor) -> None:
    """Write this token's normed+roped K and normed V of every KV head into
    the fp16 caches at slot dyn[0] (mod window for a ring)."""
    _f32(qkv, max(koff, koff if keqv else voff) + nkv * hd, "qkv")
    _f32(knw, hd, "knw")
    _f32(cosb, hd, "cosb")
    _f32(sinb, hd, "sinb")
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    call("q4_prepkv", _p(qkv), _p(knw), _p(cosb), _p(sinb), _p(kc), _p(vc), nkv, hd, koff, voff, int(bool(keqv)),
         stride, window, _p(dyn), _stream())


def attn_workspace(nH: int, hd: int, stride: int, device="cuda") -> torch.Tensor:
    """Scratch of q4_attn for this shape (no initialisation needed)."""
    n = int(lib().q4_attn_workspace_bytes(nH, hd, stride))
    return torch.empty(max(n, 4) // 4, dtype=torch.float32, device=device)


def attn(qkv, qnw, cosb, sinb, kc, vc, out=None, *, nH: int, nkv: int, hd: int, stride: int, window: int,
         qoff: int, grp: int, dyn: torch.Tensor, ws: torch.Tensor | None = None, out_dtype=torch.float32):
    """Decode attention of nH query heads over the cached keys (softmax of
    q.k, no score scaling); out[nH * hd] fp32 or fp16."""
    _f32(qkv, qoff + nH * hd, "qkv")
    _f32(qnw, hd, "qnw")
    _f32(cosb, hd, "cosb")
    _f32(sinb, hd, "sinb")
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    out = torch.empty(nH * hd, dtype=out_dtype, device=qkv.device) if out is None else out
    _need(out, nH * hd * out.element_size(), "out")
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("attention inside a graph capture needs a workspace allocated before the capture")
        ws = attn_workspace(nH, hd, stride, qkv.device)
    call("q4_attn", _p(qkv), _p(qnw), _p(cosb), _p(sinb), _p(kc), _p(vc), _p(out), _dt(out), nH, nkv, hd, stride,
         window, qoff, grp, _p(dyn), _p(ws), _nbytes(ws), _stream())
    return out


def prepkv_attn(qkv, knw, qnw, cosb, sinb, kc, vc, out=None, *, nH: int, nkv: int, hd: int, stride: int,
                window: int, qoff: int, koff: int, voff: int, keqv: bool, grp: int, dyn: torch.Tensor,
                ws: torch.Tensor | None = None, out_dtype=torch.float32) -> torch.Tensor:
    """:func:`prepkv` then :func:`attn` of one layer in one pass (same results)."""
    _f32(qkv, max(qoff + nH * hd, max(koff, koff if keqv else voff) + nkv * hd), "qkv")
    for t, nm in ((knw, "knw"), (qnw, "qnw"), (cosb, "cosb"), (sinb, "sinb")):
        _f32(t, hd, nm)
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    out = torch.empty(nH * hd, dtype=out_dtype, device=qkv.device) if out is None else out
    _need(out, nH * hd * out.element_size(), "out")
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("attention inside a graph capture needs a workspace allocated before the capture")
        ws = attn_workspace(nH, hd, stride, qkv.device)
    call("q4_prepkv_attn", _p(qkv), _p(knw), _p(qnw), _p(cosb), _p(sinb), _p(kc), _p(vc), _p(out), _dt(out), nH, nkv,
         hd, stride, window, qoff, koff, voff, int(bool(keqv)), grp, _p(dyn), _p(ws), _nbytes(ws), _stream())
    return out


# ----------------------------------------------------------- graphs/waits
class Graph:
    """A hipGraph captured from a stream: ``with g.capture(): ...`` then ``g.launch()``."""

    def __init__(self, stream: torch.cuda.Stream | None = None):
        self.stream = stream or torch.cuda.Stream()
        self.exec = None

    def capture(self):
        g = self

        class _Cap:
            def __enter__(self_):
                g.stream.wait_stream(torch.cuda.current_stream())
                self_.ctx = torch.cuda.stream(g.stream)
                self_.ctx.__enter__()
                call("q4_graph_begin", _stream(g.stream))
                _CAPTURING[0] += 1
                return g

            def __exit__(self_, et, ev, tb):
                h = C.c_void_p()
                _CAPTURING[0] -= 1
                try:
                    call("q4_graph_end", _stream(g.stream), C.byref(h))
                finally:
                    self_.ctx.__exit__(et, ev, tb)
                g.exec = h
                return False

        return _Cap()

    def launch(self, stream=None):
        if self.exec is None:
            raise RuntimeError("graph not captured")
        call("q4_graph_launch", self.exec, _stream(stream or self.stream))

    def destroy(self):
        if self.exec is not None:
            call("q4_graph_destroy", self.exec)
            self.exec = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# ---- batched prefill (one chunk of M tokens, positions dyn[0] .. dyn[0]+M-1) ----

def _rows(t, M: int, D: int, what: str, dtypes=(torch.float32,)):
    if t.dtype not in dtypes:
        raise ValueError(f"{what} must be {' or '.join(str(d) for d in dtypes)}")
    _need(t, M * D * t.element_size(), what)


def _rows_ld(t, M: int, ld: int, width: int, what: str, dtypes=(torch.float32,)):
    """M rows of ``width`` elements ``ld`` apart (the last row needs only its width)."""
    if t.dtype not in dtypes:
        raise ValueError(f"{what} must be {' or '.join(str(d) for d in dtypes)}")
    if ld < width:
        raise ValueError(f"{what}: row stride {ld} is shorter than the row width {width}")
    _need(t, ((M - 1) * ld + width) * t.element_size(), what)


def pre_rmsnorm(x, w, y=None, *, M: int, D: int, y_dtype=torch.float32):
    """rmsnorm of each of the M rows of x [M][D] (fp32)."""
    _rows(x, M, D, "x")
    _f32(w, D, "w")
    y = torch.empty(M, D, dtype=y_dtype, device=x.device) if y is None else y
    _rows(y, M, D, "y", (torch.float32, torch.float16))
    call("q4_pre_rmsnorm", _p(x), _p(w), _p(y), _dt(y), D, M, _stream())
    return y


def pre_normadd(x, w, h, *, M: int, D: int, scale: float = 0.0, w2=None, y=None, y_dtype=torch.float32):
    """h[m] = (h[m] + rmsnorm(x[m]) * w) * scale per row (x fp32 or fp16);
    with ``w2``, also y = rmsnorm(h) * w2 in the same launch (returns y)."""
    _rows(x, M, D, "x", (torch.float32, torch.float16))
    _f32(w, D, "w")
    _rows(h, M, D, "h")
    if w2 is None:
        call("q4_pre_normadd", _p(x), _dt(x), _p(w), _p(h), D, M, C.c_float(scale), _stream())
        return h
    _f32(w2, D, "w2")
    y = torch.empty(M, D, dtype=y_dtype, device=x.device) if y is None else y
    _rows(y, M, D, "y", (torch.float32, torch.float16))
    call("q4_pre_normadd_rmsnorm", _p(x), _dt(x), _p(w), _p(h), D, M, C.c_float(scale), _p(w2), _p(y), _dt(y),
         _stream())
    return y


def gemm_w4a16_normadd(X: torch.Tensor, wq: torch.Tensor, sc16: torch.Tensor, N: int, w, h, *, scale: float = 0.0,
                       w2=None, y=None, y_dtype=torch.float32, ws: torch.Tensor | None = None):
    """The W4A16 GEMM ``X @ W^T`` (N outputs per row, rounded to fp16 as
    :func:`gemm_w4a16` rounds them) straight into :func:`pre_normadd` on h
    [M][N] (and, with ``w2``, the rmsnorm of the new h into y), without the
    GEMM's output in memory. ``ws``: at least
    ``gemm_normadd_workspace_bytes(M, N, K)`` bytes."""
    if X.dtype != torch.float16 or X.dim() != 2:
        raise ValueError("X must be a 2-D float16 tensor")
    M, K = X.shape
    _check_int4(wq, sc16, N, K)
    _f32(w, N, "w")
    _rows(h, M, N, "h")
    need = gemm_normadd_workspace_bytes(M, N, K)
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("a GEMM + normadd inside a graph capture needs a workspace allocated before the "
                               "capture (pass ws=...)")
        ws = torch.empty(need, dtype=torch.uint8, device=X.device)
    _need(ws, need, "GEMM + normadd workspace")
    if w2 is None:
        call("q4_gemm_w4a16_normadd", _p(X), _p(wq), _p(sc16), M, N, K, _p(w), _p(h), C.c_float(scale),
             C.c_void_p(0), C.c_void_p(0), 0, _p(ws), _nbytes(ws), _stream())
        return h
    _f32(w2, N, "w2")
    y = torch.empty(M, N, dtype=y_dtype, device=X.device) if y is None else y
    _rows(y, M, N, "y", (torch.float32, torch.float16))
    call("q4_gemm_w4a16_normadd", _p(X), _p(wq), _p(sc16), M, N, K, _p(w), _p(h), C.c_float(scale), _p(w2), _p(y),
         _dt(y), _p(ws), _nbytes(ws), _stream())
    return y


def gemm_w4a16_qkv_prepkv(X: torch.Tensor, wq: torch.Tensor, sc16: torch.Tensor, N: int, q, knw, cosM, sinM, kc, vc,
                          *, nq: int, ldq: int, nkv: int, hd: int, keqv: bool, stride: int, window: int,
                          dyn: torch.Tensor, ws: torch.Tensor | None = None):
    """The stacked q/k/v W4A16 GEMM (rows q, k (, v); N = nq + nk (+ nk))
    with its q columns written as fp16 to ``q`` [M][ldq] and its k/v columns
    going straight through :func:`pre_prepkv`'s arithmetic into the caches
    (the k/v outputs are not stored). ``ws``: at least
    ``gemm_normadd_workspace_bytes(M, N, K)`` bytes."""
    if X.dtype != torch.float16 or X.dim() != 2:
        raise ValueError("X must be a 2-D float16 tensor")
    M, K = X.shape
    if N != nq + nkv * hd * (1 if keqv else 2):
        raise ValueError(f"N={N} is not nq + nk{'' if keqv else ' + nk'}")
    _check_int4(wq, sc16, N, K)
    _rows_ld(q, M, ldq, nq, "q", (torch.float16,))
    _f32(knw, hd, "knw")
    _f32(cosM, M * hd, "cosM")
    _f32(sinM, M * hd, "sinM")
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    need = gemm_normadd_workspace_bytes(M, N, K)
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("a q/k/v GEMM + prepkv inside a graph capture needs a workspace allocated before the "
                               "capture (pass ws=...)")
        ws = torch.empty(need, dtype=torch.uint8, device=X.device)
    _need(ws, need, "q/k/v GEMM + prepkv workspace")
    call("q4_gemm_w4a16_qkv_prepkv", _p(X), _p(wq), _p(sc16), M, N, K, _p(q), ldq, nq, _p(knw), _p(cosM), _p(sinM),
         _p(kc), _p(vc), nkv, hd, int(bool(keqv)), stride, window, _p(dyn), _p(ws), _nbytes(ws), _stream())
    return q


def gemm_normadd_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes of :func:`gemm_w4a16_normadd` (fp32 partials, at least one split)."""
    return int(lib().q4_gemm_w4a16_normadd_workspace_bytes(M, N, K))


def pre_gelumul(gate, up, out=None, out_dtype=torch.float32):
    """out = gelu_tanh(gate) * up elementwise (gate/up fp32 or fp16, same dtype)."""
    n = gate.numel()
    if up.dtype != gate.dtype or up.numel() < n:
        raise ValueError("gate and up must share dtype and size")
    _rows(gate, 1, n, "gate", (torch.float32, torch.float16))
    out = torch.empty(n, dtype=out_dtype, device=gate.device) if out is None else out
    _need(out, n * out.element_size(), "out")
    call("q4_pre_gelumul", _p(gate), _p(up), _dt(gate), _p(out), _dt(out), C.c_long(n), _stream())
    return out


def pre_prepkv(k, v, knw, cosM, sinM, kc, vc, *, M: int, ld: int, nkv: int, hd: int, stride: int, window: int,
               dyn: torch.Tensor) -> None:
    """K (normed, roped with each token's cos/sin row) and V (normed) of the
    M tokens into the fp16 caches; k, v [M][ld] fp32 or fp16 (v may be k)."""
    v = k if v is None else v
    if v.dtype != k.dtype:
        raise ValueError("k and v must share a dtype")
    _rows_ld(k, M, ld, nkv * hd, "k", (torch.float32, torch.float16))
    _rows_ld(v, M, ld, nkv * hd, "v", (torch.float32, torch.float16))
    _f32(knw, hd, "knw")
    _f32(cosM, M * hd, "cosM")
    _f32(sinM, M * hd, "sinM")
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    call("q4_pre_prepkv", _p(k), _p(v), _dt(k), ld, _p(knw), _p(cosM), _p(sinM), _p(kc), _p(vc), nkv, hd, stride,
         window, M, _p(dyn), _stream())


def pre_attn_workspace(M: int, nH: int, nkv: int, hd: int, max_keys: int, device="cuda") -> torch.Tensor:
    """Scratch of :func:`pre_attn` for this shape (no initialisation needed)."""
    n = int(lib().q4_pre_attn_workspace_bytes(M, nH, nkv, hd, max_keys))
    return torch.empty(max(n, 16) // 4, dtype=torch.float32, device=device)


def pre_attn(q, qnw, cosM, sinM, kc, vc, out=None, *, M: int, ldq: int, nH: int, nkv: int, hd: int, stride: int,
             window: int, max_keys: int, dyn: torch.Tensor, ws: torch.Tensor | None = None,
             out_dtype=torch.float32) -> torch.Tensor:
    """Causal attention of the chunk's M tokens over the cache (after the
    chunk's K/V were written); q [M][ldq] fp32 or fp16; out [M][nH * hd]."""
    _rows_ld(q, M, ldq, nH * hd, "q", (torch.float32, torch.float16))
    _f32(qnw, hd, "qnw")
    _f32(cosM, M * hd, "cosM")
    _f32(sinM, M * hd, "sinM")
    _kv_checks(kc, vc, nkv, stride, hd, dyn)
    out = torch.empty(M, nH * hd, dtype=out_dtype, device=q.device) if out is None else out
    _rows(out, M, nH * hd, "out", (torch.float32, torch.float16))
    if ws is None:
        if _CAPTURING[0]:
            raise RuntimeError("prefill attention inside a graph capture needs a workspace allocated before it")
        ws = pre_attn_workspace(M, nH, nkv, hd, max_keys, q.device)
    call("q4_pre_attn", _p(q), _dt(q), ldq, _p(qnw), _p(cosM), _p(sinM), _p(kc), _p(vc), _p(out), _dt(out), nH * hd,
         nH, nkv, hd, stride, window, M, max_keys, _p(dyn), _p(ws), _nbytes(ws), _stream())
    return out


TOKEN_MAX_TABLES = 4


def token_inputs(step: torch.Tensor, emb: torch.Tensor, h: torch.Tensor, dyn: torch.Tensor, tables=(), *,
                 vocab: int, H: int, max_pos: int, stream=None) -> None:
    """The per-token inputs of a decode graph from (tid, pos) = ``step[0:2]``
    (int32; pinned host memory rewritten by the host before each launch, or
    device memory), read when the launch runs (q4_token_inputs): ``h`` =
    the fp32 embedding row ``emb[tid]`` (``emb`` [vocab, H]), ``dyn[0:2]`` =
    (pos, pos + 1), and for each ``(cos_tab, sin_tab, hd, cos_out, sin_out)``
    of ``tables`` the fp32 rows ``cos_tab[pos]``, ``sin_tab[pos]`` (tables
    [max_pos, hd]) into the outputs."""
    if step.dtype != torch.int32 or step.numel() < 2:
        raise ValueError("step must hold two int32 values (tid, pos)")
    if not (step.is_cuda or step.is_pinned()) or not step.is_contiguous():
        raise ValueError("step must be contiguous device memory or pinned host memory")
    if emb.dtype != torch.float32 or h.dtype != torch.float32:
        raise ValueError("emb and h are fp32")
    _need(emb, vocab * H * 4, "emb")
    _need(h, H * 4, "h")
    _need(dyn, 8, "dyn")
    n = len(tables)
    if n > TOKEN_MAX_TABLES:
        raise ValueError(f"at most {TOKEN_MAX_TABLES} RoPE tables")
    ptrs = {k: (C.c_void_p * max(1, n))() for k in ("ct", "st", "co", "so")}
    hds = (C.c_int * max(1, n))()
    for i, (ct, st, hd, co, so) in enumerate(tables):
        for t in (ct, st, co, so):
            if t.dtype != torch.float32:
                raise ValueError("RoPE tables and rows are fp32")
        _need(ct, max_pos * hd * 4, "cos table")
        _need(st, max_pos * hd * 4, "sin table")
        _need(co, hd * 4, "cos row")
        _need(so, hd * 4, "sin row")
        ptrs["ct"][i], ptrs["st"][i] = _p(ct).value, _p(st).value
        ptrs["co"][i], ptrs["so"][i] = _p(co).value, _p(so).value
        hds[i] = int(hd)
    vp = lambda a: C.cast(a, C.c_void_p)  # noqa: E731
    call("q4_token_inputs", C.c_void_p(step.data_ptr()), _p(emb), vocab, H, _p(h), _p(dyn), n, vp(ptrs["ct"]),
         vp(ptrs["st"]), vp(hds), max_pos, vp(ptrs["co"]), vp(ptrs["so"]), _stream(stream))


class Timestamps:
    """``n`` GPU timestamps (q4_timestamps_*): ``record(i)`` enqueues a stamp
    on the current stream, inside a graph capture too (then every replay
    stamps again); ``read_ms()`` (after the work is done) gives the
    milliseconds from stamp 0 to each stamp."""

    def __init__(self, n: int):
        h = C.c_void_p()
        call("q4_timestamps_create", int(n), C.byref(h))
        self.h, self.n = h, int(n)

    def record(self, i: int, stream=None) -> None:
        call("q4_timestamp_record", self.h, int(i), _stream(stream))

    def read_ms(self) -> list:
        ms = (C.c_double * self.n)()
        call("q4_timestamps_read", self.h, ms)
        return list(ms)

    def destroy(self) -> None:
        if self.h:
            call("q4_timestamps_destroy", self.h)
            self.h = None


def stream_wait(stream=None, timeout_ms: int = 0, label: str = "") -> None:
    """Bounded wait; raises RuntimeError('GPU fence TIMEOUT after <ms>ms at [label]') on expiry,
    the message the reference's fence wait raises (src/vk_engine.py:299-302)."""
    st = lib().q4_stream_wait(_stream(stream), int(timeout_ms))
    if st == _lib.Q4_ERR_TIMEOUT:
        raise RuntimeError(f"GPU fence TIMEOUT after {timeout_ms}ms at [{label}]")
    _lib.check("q4_stream_wait", st)


# ------------------------------------------------------------------ probes
def probe_stream_read(buf: torch.Tensor, wgs: int, *, units: int = 8, chunked: bool = True,
                      next: torch.Tensor | None = None, prefetch_bytes: int = 0,
                      comp: torch.Tensor | None = None, sink: torch.Tensor | None = None) -> torch.Tensor:
    """Streaming read of all of ``buf`` (a measurement probe; computes nothing).
    With ``next``, each workgroup then reads its successor's first
    ``prefetch_bytes / wgs`` bytes of ``next`` into L2; with ``comp`` (>= 1/8
    of ``buf``), every 16-byte load has a 2-byte companion load (the GEMV's
    scale pattern). Returns the sink."""
    if sink is None:
        sink = torch.empty(wgs, dtype=torch.int32, device=buf.device)
    _need(sink, 4 * wgs, "sink")
    nb = _nbytes(next) if next is not None else 0
    call("q4_probe_stream_read", _p(buf), _nbytes(buf) // 16 * 16, wgs, units, int(chunked),
         _p(next) if next is not None else None, nb, prefetch_bytes if next is not None else 0,
         _p(comp) if comp is not None else None, _nbytes(comp) if comp is not None else 0, _p(sink),
         _nbytes(sink), _stream())
    return sink


def probe_mfma(kind: int, wgs: int, iters: int, clocks: torch.Tensor, sink: torch.Tensor,
               operands: torch.Tensor | None = None) -> None:
    """MFMA-only loop (kind 0 int8 32x32x32, 1 f16 32x32x16); ``clocks`` int64
    [wgs, 2] receives (shader cycles, wall-clock ticks) per workgroup;
    ``operands`` (64 KB of random bytes) makes every MFMA take other operand
    bits, None repeats the same fragments."""
    call("q4_probe_mfma", kind, wgs, iters, _p(operands), _nbytes(operands) if operands is not None else 0,
         _p(clocks), _nbytes(clocks), _p(sink), _nbytes(sink), _stream())


def probe_wall_clock_khz() -> int:
    k = C.c_int()
    call("q4_probe_wall_clock_khz", C.byref(k))
    return k.value
