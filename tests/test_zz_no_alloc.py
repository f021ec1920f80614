"""q4_gemv_noalloc (the GEMV with its split-K workspace in a file-scope
device array instead of a caller buffer) against q4_gemv with a caller
workspace: bit-identical outputs, through the C ABI, for two calls in a
row (the second smaller, reusing the array's previous contents), split-K
and unsplit plans, fp16 and e4m3 scales; and against the oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import synth_int4, to_np, upload_int4

pytestmark = pytest.mark.gpu


def _call_noalloc(lib, x, wq, sc, fmt, inv, y, N, K, split=0):
    return lib.q4_gemv_noalloc(x.data_ptr(), 1, wq.data_ptr(), sc.data_ptr(), fmt, C.c_float(inv), y.data_ptr(), 0,
                               N, K, split, None)


def _call_ws(lib, x, wq, sc, fmt, inv, y, N, K, ws, split=0):
    return lib.q4_gemv(x.data_ptr(), 1, wq.data_ptr(), sc.data_ptr(), fmt, C.c_float(inv), y.data_ptr(), 0, N, K,
                       split, ws.data_ptr(), ws.numel(), None)


@pytest.mark.parametrize("e4m3", [False, True])
def test_noalloc_matches_workspace_gemv(g4, gpu, e4m3):
    from g4mi import _lib
    lib = _lib.lib()
    assert lib.q4_gemv_scratch_bytes() == 2 << 20
    rng = np.random.default_rng(31 + int(e4m3))
    fmt = gpu.SCALE_E4M3 if e4m3 else gpu.SCALE_F16
    # first a split-K plan with many row groups, then a smaller one (fewer groups, other split):
    # the second call must not see the first call's partials or tickets; then two unsplit shapes
    for N, K in [(1792, 3840), (320, 2048), (64, 256), (2048, 4096), (4096, 3840)]:
        print(f"noalloc N={N} K={K} e4m3={e4m3} split={gpu.auto_split(N, K)}", flush=True)
        q, s = synth_int4(rng, N, K)
        wq, sc = upload_int4(q, s)
        inv = 1.0
        s_used = s
        if e4m3:
            sc, inv = gpu.scales_e4m3(torch.from_numpy(s).cuda(), N, K)
            e8, inv_o, _ = O.e4m3_lift(s)
            assert inv == inv_o
            s_used = O.e4m3_decode(e8).astype(np.float32)
        xh = rng.standard_normal(K).astype(np.float16)
        x = torch.from_numpy(xh).cuda()
        ws = torch.zeros(max(256, gpu.Workspace.bytes_for(N, K)), dtype=torch.uint8, device="cuda")
        y_ref = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
        y_na = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
        assert _call_ws(lib, x, wq, sc, fmt, inv, y_ref, N, K, ws) == 0, lib.q4_last_error()
        for rep in range(2):
            assert _call_noalloc(lib, x, wq, sc, fmt, inv, y_na, N, K) == 0, lib.q4_last_error()
            torch.cuda.synchronize()
            assert (to_np(y_na).view(np.uint32) == to_np(y_ref).view(np.uint32)).all(), (N, K, rep)
        ref = O.gemv_ref(q, s_used, xh, inv)
        assert O.normwise_rel_err(to_np(y_na), ref) <= 2e-5      # fp32 output, fp32 accumulate


def test_noalloc_rejects_oversized_scratch(g4, gpu):
    from g4mi import _lib
    lib = _lib.lib()
    # K large enough that the x staging forces a split (fp16 x stages at most 1024 blocks), N large
    # enough that the partials exceed 2 MiB: rejected on the host, nothing is launched
    N, K = 262144, 65536
    split = gpu.auto_split(N, K)
    need = gpu.Workspace.bytes_for(N, K)
    assert split > 1 and need > lib.q4_gemv_scratch_bytes()
    dummy = torch.zeros(16, dtype=torch.uint8, device="cuda")
    # x, x_dtype (1: fp16), wq, scales, scale_fmt (0: fp16), inv, y, y_dtype (0: fp32), N, K, split, stream
    rc = lib.q4_gemv_noalloc(dummy.data_ptr(), 1, dummy.data_ptr(), dummy.data_ptr(), 0, C.c_float(1.0),
                             dummy.data_ptr(), 0, N, K, 0, None)
    assert rc == _lib.Q4_ERR_ARG and b"scratch" in lib.q4_last_error()
    torch.cuda.synchronize()
