"""ctypes binding of libq4mi.so (the C ABI declared in include/q4mi.h).

Loading fails loudly: there is no CPU fallback anywhere in this package. If
the shared library is missing, build it with ``build.py`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("Q4MI_LIB", Path(__file__).resolve().parent / "libq4mi.so"))

Q4_OK, Q4_ERR_ARG, Q4_ERR_HIP, Q4_ERR_TIMEOUT = 0, 1, 2, 3
DT_F32, DT_F16 = 0, 1
SCALE_F16, SCALE_E4M3 = 0, 1
OP_GEMV = 0
OP_W4A16 = 1
GEMV_MAX_BATCH = 8
# plan overrides of q4_tune_set (include/q4mi.h Q4_TUNE_*), by name
TUNE_KNOBS = {"gemv_rows": 0, "gemv_units": 1, "gemv_pair": 2, "gemv_bal": 3, "gemv_mm_tiles": 4,
              "gemv_mm_split": 5, "gemv_mm_deep": 6, "w4a16_split": 7, "w4a16_kg": 8, "w8a8_tiles": 9}

_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t

# name -> (restype, argtypes); mirrors include/q4mi.h one for one.
SIGNATURES = {
    "q4_version": (C.c_char_p, []),
    "q4_last_error": (C.c_char_p, []),
    "q4_dev_bytes": (_i, [_i, _i, C.POINTER(_sz), C.POINTER(_sz)]),
    "q4_tune_set": (_i, [_i, _i]),
    "q4_tune_get": (_i, [_i]),
    "q4_tune_reset": (None, []),
    "q4_quantize": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "q4_scales_e4m3": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "q4_w8_fold": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp]),
    "q4_w4a8_ratio": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "q4_repack_ref": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "q4_repack_e4m3_ref": (_i, [_vp, _i, _i, _vp, _vp]),
    "q4_repack_w8_ref": (_i, [_vp, _i, _i, _vp, _vp]),
    "q4_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "q4_workspace_init": (_i, [_vp, _sz, _vp]),
    "q4_gemv_auto_split": (_i, [_i, _i]),
    "q4_gemv": (_i, [_vp, _i, _vp, _vp, _i, _f, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemv_scratch_bytes": (_sz, []),
    "q4_gemv_noalloc": (_i, [_vp, _i, _vp, _vp, _i, _f, _vp, _i, _i, _i, _i, _vp]),
    "q4_gemv_f16s": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemv_e4m3s": (_i, [_vp, _i, _vp, _vp, _f, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemv_batch": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "q4_gemv_gated": (_i, [_vp, _i, _vp, _vp, _i, _f, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemv_normadd": (_i, [_vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _f, _vp, _i, _i, _i, _i, _vp]),
    "q4_gemv_batch_normadd": (_i, [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "q4_pre_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "q4_pre_normadd": (_i, [_vp, _i, _vp, _vp, _i, _i, _f, _vp]),
    "q4_pre_normadd_rmsnorm": (_i, [_vp, _i, _vp, _vp, _i, _i, _f, _vp, _vp, _i, _vp]),
    "q4_pre_gelumul": (_i, [_vp, _vp, _i, _vp, _i, C.c_long, _vp]),
    "q4_pre_prepkv": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "q4_pre_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "q4_pre_attn": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp,
                         _sz, _vp]),
    "q4_gemv_multi": (_i, [_vp, _i, _vp, _vp, _i, _f, _vp, _i, _i, _i, _i, _vp]),
    "q4_gemv_multi_workspace_bytes": (_sz, [_i, _i, _i]),
    "q4_gemv_multi_ws": (_i, [_vp, _i, _vp, _vp, _i, _f, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "q4_interleave_rows": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "q4_gemm_w4a16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "q4_gemm_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "q4_gemm_w4a16_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemm_w4a16_gated_workspace_bytes": (_sz, [_i, _i, _i]),
    "q4_gemm_w4a16_gated": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemm_w4a16_normadd_workspace_bytes": (_sz, [_i, _i, _i]),
    "q4_gemm_w4a16_qkv_prepkv": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                                      _i, _i, _vp, _vp, _sz, _vp]),
    "q4_gemm_w4a16_normadd": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _f, _vp, _vp, _i, _vp, _sz, _vp]),
    "q4_quant_act_i8": (_i, [_vp, _i, _vp, _vp, _i, _i, _vp]),
    "q4_gemm_w8a8": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "q4_w4a8_weights": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "q4_gemm_w4a8": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "q4_w8_packed_bytes": (_sz, [_i, _i]),
    "q4_w8_pack": (_i, [_vp, _i, _i, _vp, _vp]),
    "q4_gemm_w8a8_packed": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "q4_gemm_w8a8_packed_stamped": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "q4_gemm_w8a8_packed_workgroups": (_sz, [_i, _i, _i]),
    "q4_cast_f32_f16": (_i, [_vp, _vp, _sz, _vp]),
    "q4_cast_f16_f32": (_i, [_vp, _vp, _sz, _vp]),
    "q4_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "q4_normadd": (_i, [_vp, _vp, _vp, _i, _f, _vp]),
    "q4_normadd_rmsnorm": (_i, [_vp, _vp, _vp, _i, _f, _vp, _vp, _i, _vp]),
    "q4_gelumul": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "q4_prepkv": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "q4_attn_workspace_bytes": (_sz, [_i, _i, _i]),
    "q4_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "q4_token_inputs": (_i, [_vp, _vp, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "q4_prepkv_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp,
                            _vp, _sz, _vp]),
    "q4_probe_stream_read": (_i, [_vp, _sz, _i, _i, _i, _vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp]),
    "q4_probe_mfma": (_i, [_i, _i, _i, _vp, _sz, _vp, _sz, _vp, _sz, _vp]),
    "q4_probe_wall_clock_khz": (_i, [C.POINTER(_i)]),
    "q4_graph_begin": (_i, [_vp]),
    "q4_graph_end": (_i, [_vp, C.POINTER(_vp)]),
    "q4_graph_launch": (_i, [_vp, _vp]),
    "q4_graph_destroy": (_i, [_vp]),
    "q4_stream_wait": (_i, [_vp, _i]),
    "q4_timestamps_create": (_i, [_i, _vp]),
    "q4_timestamp_record": (_i, [_vp, _i, _vp]),
    "q4_timestamps_read": (_i, [_vp, _vp]),
    "q4_timestamps_destroy": (_i, [_vp]),
}


class Q4Error(RuntimeError):
    """A libq4mi call returned a non-zero status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn}: {msg} (status {status})")
        self.fn, self.status, self.msg = fn, status, msg


class Q4Timeout(Q4Error):
    pass


_LIB = None


def lib(path: Path | None = None):
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path or LIB_PATH)
    if not p.exists():
        raise FileNotFoundError(
            f"libq4mi.so not found at {p}: build it first (python build.py in the package, "
            "or __graft_entry__.build()). There is no CPU fallback.")
    h = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(h, name)
        fn.restype, fn.argtypes = res, args
    if path is None:
        _LIB = h
    return h


def check(fn_name: str, status: int) -> None:
    if status != Q4_OK:
        msg = (lib().q4_last_error() or b"").decode(errors="replace")
        if status == Q4_ERR_TIMEOUT:
            raise Q4Timeout(fn_name, status, msg)
        raise Q4Error(fn_name, status, msg)


def call(name: str, *args) -> None:
    """Call an int-status entry point and raise on failure."""
    check(name, getattr(lib(), name)(*args))
