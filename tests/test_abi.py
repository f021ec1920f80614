"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/q4mi.h declares, the ctypes table matches the header, and argument
validation fails with a status + message before any device work."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "q4mi.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(q4_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_parse_sane():
    names = header_functions()
    assert "q4_gemv" in names and "q4_gemm_w8a8" in names and "q4_last_error" in names
    assert len(names) >= 25


def test_library_exports_every_header_symbol(g4):
    lib = g4._lib.lib()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_ctypes_table_matches_header(g4):
    assert sorted(g4._lib.SIGNATURES) == header_functions()


def test_version_and_error_strings(g4):
    lib = g4._lib.lib()
    assert lib.q4_version().decode().startswith("q4mi")
    assert lib.q4_last_error() is not None


def _err(g4):
    return g4._lib.lib().q4_last_error().decode()


def test_argument_errors_without_gpu(g4):
    lib = g4._lib.lib()
    null = C.c_void_p(0)
    # K not a multiple of 32
    st = lib.q4_gemv(null, 0, null, null, 0, C.c_float(1.0), null, 0, 128, 100, 0, null, 0, null)
    assert st == g4._lib.Q4_ERR_ARG and "multiple of 32" in _err(g4)
    # null pointers
    st = lib.q4_gemv(null, 0, null, null, 0, C.c_float(1.0), null, 0, 128, 128, 0, null, 0, null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)
    # W8A8: K must be a multiple of 64
    st = lib.q4_gemm_w8a8(null, null, null, null, 0, null, null, 64, 64, 96, null)
    assert st == g4._lib.Q4_ERR_ARG and "multiple of 64" in _err(g4)
    # int32 accumulator bound
    st = lib.q4_gemm_w8a8(null, null, null, null, 0, null, null, 64, 64, 64 * 2100, null)
    assert st == g4._lib.Q4_ERR_ARG and "overflow" in _err(g4)
    # graph capture needs a real stream
    assert lib.q4_graph_begin(null) == g4._lib.Q4_ERR_ARG
    # reference layout needs N % 8 == 0
    st = lib.q4_repack_ref(null, null, 12, 32, null, null, null)
    assert st == g4._lib.Q4_ERR_ARG and "N % 8" in _err(g4)
    # batched GEMV: count outside 1..8, K beyond the x staging area, bad entry
    P = C.c_void_p * 9
    ptrs, Ns = P(*([1 << 20] * 9)), (C.c_int * 9)(*([64] * 9))
    st = lib.q4_gemv_batch(C.c_void_p(1 << 20), 1, 256, 0, 1, 0, ptrs, ptrs, None, ptrs, Ns, null)
    assert st == g4._lib.Q4_ERR_ARG and "batch of 0" in _err(g4)
    st = lib.q4_gemv_batch(C.c_void_p(1 << 20), 1, 256, 0, 1, 9, ptrs, ptrs, None, ptrs, Ns, null)
    assert st == g4._lib.Q4_ERR_ARG and "batch of 9" in _err(g4)
    st = lib.q4_gemv_batch(C.c_void_p(1 << 20), 0, 16416, 0, 1, 2, ptrs, ptrs, None, ptrs, Ns, null)
    assert st == g4._lib.Q4_ERR_ARG and "K <= 16384" in _err(g4)
    Ns[1] = 0
    st = lib.q4_gemv_batch(C.c_void_p(1 << 20), 1, 256, 0, 1, 2, ptrs, ptrs, None, ptrs, Ns, null)
    assert st == g4._lib.Q4_ERR_ARG and "entry 1" in _err(g4)
    # multi-vector GEMV: M outside 1..16, K beyond two vectors' staging, null pointers
    p = C.c_void_p(1 << 20)
    for M in (0, 17):
        st = lib.q4_gemv_multi(p, M, p, p, 0, C.c_float(1.0), p, 1, 256, 256, 1, null)
        assert st == g4._lib.Q4_ERR_ARG and f"M={M}" in _err(g4)
    st = lib.q4_gemv_multi(p, 2, p, p, 0, C.c_float(1.0), p, 1, 256, 65536, 1, null)
    assert st == g4._lib.Q4_ERR_ARG and "LDS" in _err(g4)
    st = lib.q4_gemv_multi(p, 2, null, p, 0, C.c_float(1.0), p, 1, 256, 256, 0, null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)
    # its K-split variant: the same checks, a misaligned workspace, and the plan's workspace size
    for M in (0, 17):
        st = lib.q4_gemv_multi_ws(p, M, p, p, 0, C.c_float(1.0), p, 1, 256, 256, p, 1 << 20, null)
        assert st == g4._lib.Q4_ERR_ARG and f"M={M}" in _err(g4)
    st = lib.q4_gemv_multi_ws(p, 2, p, p, 0, C.c_float(1.0), p, 1, 3840, 15360, C.c_void_p((1 << 20) + 8), 1 << 24,
                              null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte" in _err(g4)
    # 3840 rows: 60 groups of 64 rows, split 4 (240 workgroups); 15360 rows fill the grid unsplit
    assert lib.q4_gemv_multi_workspace_bytes(16, 3840, 15360) == 4 * 16 * 3840 * 4
    assert lib.q4_gemv_multi_workspace_bytes(16, 15360, 3840) == 0
    assert lib.q4_gemv_multi_workspace_bytes(17, 3840, 15360) == 0


def test_prefill_op_argument_errors_without_gpu(g4):
    lib = g4._lib.lib()
    p = C.c_void_p(1 << 20)
    null = C.c_void_p(0)
    # head dims outside 64/128/256/512
    st = lib.q4_pre_attn(p, 0, 96 * 4, p, p, p, p, p, p, 0, 96 * 4, 4, 2, 96, 64, 0, 8, 64, p, p, 1 << 30, null)
    assert st == g4._lib.Q4_ERR_ARG and "head dims" in _err(g4)
    # a chunk longer than the ring
    st = lib.q4_pre_attn(p, 0, 1024, p, p, p, p, p, p, 0, 1024, 4, 2, 256, 64, 32, 33, 64, p, p, 1 << 30, null)
    assert st == g4._lib.Q4_ERR_ARG and "longer than" in _err(g4)
    # workspace too small
    need = lib.q4_pre_attn_workspace_bytes(8, 4, 2, 256, 64)
    assert need == 8 * 4 * 2 * (256 + 4) * 4  # 2 KV-head blocks -> 128 splits wanted -> 2 splits of 32 keys
    st = lib.q4_pre_attn(p, 0, 1024, p, p, p, p, p, p, 0, 1024, 4, 2, 256, 64, 0, 8, 64, p, p, need - 1, null)
    assert st == g4._lib.Q4_ERR_ARG and "workspace" in _err(g4)
    # prepkv row stride shorter than nkv * hd
    st = lib.q4_pre_prepkv(p, p, 0, 100, p, p, p, p, p, 2, 64, 16, 16, 4, p, null)
    assert st == g4._lib.Q4_ERR_ARG and "row stride" in _err(g4)
    st = lib.q4_pre_normadd(p, 2, p, p, 64, 4, C.c_float(0.0), null)
    assert st == g4._lib.Q4_ERR_ARG and "x_dtype" in _err(g4)


def test_sizes_and_split_queries(g4):
    lib = g4._lib.lib()
    wb, se = C.c_size_t(), C.c_size_t()
    assert lib.q4_dev_bytes(15360, 3840, C.byref(wb), C.byref(se)) == 0
    assert wb.value == 15360 * 3840 // 2 and se.value == 15360 * 120
    assert lib.q4_dev_bytes(70, 64, C.byref(wb), C.byref(se)) == 0
    assert se.value == 128 * 2  # rows padded to whole 64-row panels
    # every decode shape runs without split-K (no workspace) ...
    for N, K in [(262144, 3840), (30720, 3840), (15360, 3840), (2048, 3840), (3840, 15360), (3840, 4096)]:
        assert lib.q4_gemv_auto_split(N, K) == 1
        assert lib.q4_workspace_bytes(0, N, K, 0) == 0
    # ... small matrices split K across workgroups and need the workspace
    for N, K in [(512, 3840), (256, 15360), (64, 4096)]:
        s = lib.q4_gemv_auto_split(N, K)
        assert 1 < s <= K // 32
        ws = lib.q4_workspace_bytes(0, N, K, 0)
        assert ws >= 65536 + s * N * 4 and ws % 256 == 0
    # an explicit split too small for the LDS staging cap is raised
    assert lib.q4_workspace_bytes(0, 64, 32768, 1) > 0  # fp32 x of K=32768 exceeds one LDS staging


def test_missing_library_fails_loudly(g4, tmp_path):
    with pytest.raises(FileNotFoundError, match="no CPU fallback"):
        g4._lib.lib(tmp_path / "nope.so")


def test_decode_op_argument_errors_without_gpu(g4):
    lib = g4._lib.lib()
    fake = C.c_void_p(256)  # never dereferenced: every call below fails its checks before any launch
    null = C.c_void_p(0)
    # per head and 32-key split: (max, sum, accumulator[hd])
    assert lib.q4_attn_workspace_bytes(16, 256, 8192) == 16 * 128 * 258 * 4   # 64-key splits up to hd 256
    assert lib.q4_attn_workspace_bytes(16, 512, 1000) == 16 * 32 * 514 * 4    # 32-key splits at hd 512
    assert lib.q4_attn_workspace_bytes(0, 256, 8) == 0
    st = lib.q4_attn(*[fake] * 7, 0, 16, 8, 100, 64, 0, 0, 2, fake, fake, 1 << 20, null)
    assert st == g4._lib.Q4_ERR_ARG and "64, 128, 256 or 512" in _err(g4)
    st = lib.q4_attn(*[fake] * 7, 0, 16, 8, 256, 64, 0, 0, 3, fake, fake, 1 << 20, null)
    assert st == g4._lib.Q4_ERR_ARG and "nkv * grp" in _err(g4)
    st = lib.q4_attn(*[fake] * 7, 0, 16, 8, 256, 64, 128, 0, 2, fake, fake, 1 << 20, null)
    assert st == g4._lib.Q4_ERR_ARG and "bad sizes" in _err(g4)  # window past the cache depth
    st = lib.q4_attn(*[fake] * 7, 0, 16, 8, 256, 8192, 0, 0, 2, fake, fake, 1000, null)
    assert st == g4._lib.Q4_ERR_ARG and "workspace too small" in _err(g4)
    st = lib.q4_prepkv(*[fake] * 6, 8, 255, 0, 0, 0, 64, 0, fake, null)
    assert st == g4._lib.Q4_ERR_ARG and "even" in _err(g4)
    st = lib.q4_prepkv(*[fake] * 6, 8, 256, 0, 0, 0, 64, 128, fake, null)
    assert st == g4._lib.Q4_ERR_ARG and "exceeds the cache depth" in _err(g4)
    st = lib.q4_rmsnorm(fake, fake, fake, 7, 3840, null)
    assert st == g4._lib.Q4_ERR_ARG and "y_dtype" in _err(g4)
    st = lib.q4_gelumul(fake, null, fake, 0, 10, null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)
    st = lib.q4_normadd(fake, fake, fake, 0, C.c_float(1.0), null)
    assert st == g4._lib.Q4_ERR_ARG and "bad D" in _err(g4)


def test_prepkv_attn_argument_errors_without_gpu(g4):
    lib = g4._lib.lib()
    fake, null = C.c_void_p(256), C.c_void_p(0)
    st = lib.q4_prepkv_attn(fake, null, *[fake] * 6, 0, 16, 8, 256, 64, 0, 0, 4096, 6144, 0, 2, fake, fake, 1 << 20,
                            null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)
    st = lib.q4_prepkv_attn(*[fake] * 8, 0, 16, 8, 96, 64, 0, 0, 4096, 6144, 0, 2, fake, fake, 1 << 20, null)
    assert st == g4._lib.Q4_ERR_ARG and "64, 128, 256 or 512" in _err(g4)


def test_probe_and_stamped_gemm_argument_errors_without_gpu(g4):
    """Entry points added for measurement reject bad arguments before any
    device work: the streaming-read probe (units, companion size), the MFMA
    probe (round count, operand buffer), the stamped W8A8 (stamp buffer)."""
    lib = g4._lib.lib()
    p, null = C.c_void_p(1 << 20), C.c_void_p(0)
    st = lib.q4_probe_stream_read(p, 1 << 20, 64, 3, 1, null, 0, 0, null, 0, p, 4096, null)
    assert st == g4._lib.Q4_ERR_ARG and "units" in _err(g4)
    st = lib.q4_probe_stream_read(p, 1 << 20, 64, 4, 1, null, 0, 0, p, (1 << 17) - 2, p, 4096, null)
    assert st == g4._lib.Q4_ERR_ARG and "companion" in _err(g4)
    st = lib.q4_probe_stream_read(p, 1 << 20, 64, 4, 1, p, 1 << 20, 1 << 20, p, 1 << 17, p, 4096, null)
    assert st == g4._lib.Q4_ERR_ARG and "separate probes" in _err(g4)
    st = lib.q4_probe_mfma(0, 4, 12, null, 0, p, 64, p, 16, null)
    assert st == g4._lib.Q4_ERR_ARG and "multiple of 8" in _err(g4)
    st = lib.q4_probe_mfma(0, 4, 16, p, 1024, p, 64, p, 16, null)
    assert st == g4._lib.Q4_ERR_ARG and "operands" in _err(g4)
    st = lib.q4_probe_mfma(2, 4, 16, null, 0, p, 64, p, 16, null)
    assert st == g4._lib.Q4_ERR_ARG and "kind" in _err(g4)
    # stamped W8A8: 256 persistent workgroups at M=2048, N=15360, K=3840 (768 tiles of
    # 128 x 320); 480 with 256-row tiles when the k-steps are not a multiple of 3; one stamp row short
    assert lib.q4_gemm_w8a8_packed_workgroups(2048, 15360, 3840) == 256
    assert lib.q4_gemm_w8a8_packed_workgroups(2048, 15360, 4096) == 480
    assert lib.q4_gemm_w8a8_packed_workgroups(2048, 15360, 320) == 256   # 3 k-steps, the last of two slices
    assert lib.q4_gemm_w8a8_packed_workgroups(1024, 15360, 3840) == 256  # 384 tiles of 128 x 320
    assert lib.q4_gemm_w8a8_packed_workgroups(2048, 3840, 15360) == 240  # 192 tiles: fewer than the CUs
    assert lib.q4_gemm_w8a8_packed_workgroups(128, 512, 3840) == 2       # 128-row tiles below 256 workgroups
    assert lib.q4_gemm_w8a8_packed_workgroups(0, 512, 64) == 0
    st = lib.q4_gemm_w8a8_packed_stamped(p, p, p, p, 0, p, null, 2048, 15360, 3840, p, 256 * 32 - 8, null)
    assert st == g4._lib.Q4_ERR_ARG and "stamps" in _err(g4)
    st = lib.q4_gemm_w8a8_packed(p, p, p, p, 0, C.c_void_p((1 << 20) + 8), null, 2048, 15360, 3840, null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte aligned" in _err(g4)
    st = lib.q4_gemm_w8a8_packed_stamped(p, p, p, p, 0, p, null, 2048, 15360, 3840, null, 0, null)
    assert st == g4._lib.Q4_ERR_ARG and "stamps" in _err(g4)


def test_attention_alignment_errors_without_gpu(g4):
    """The decode attention and prepkv read q, k, v, the norm weights and the
    RoPE row in 16-byte pieces: misaligned buffers or offsets are refused."""
    lib = g4._lib.lib()
    a, m, null = C.c_void_p(1 << 20), C.c_void_p((1 << 20) + 4), C.c_void_p(0)
    ws = lib.q4_attn_workspace_bytes(16, 256, 1024)
    st = lib.q4_attn(m, a, a, a, a, a, a, 0, 16, 8, 256, 1024, 1024, 0, 2, a, a, ws, null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte aligned" in _err(g4)
    st = lib.q4_attn(a, a, a, a, a, a, a, 0, 16, 8, 256, 1024, 1024, 2, 2, a, a, ws, null)
    assert st == g4._lib.Q4_ERR_ARG and "offsets" in _err(g4)
    st = lib.q4_prepkv_attn(a, m, a, a, a, a, a, a, 0, 16, 8, 256, 1024, 1024, 0, 4096, 6144, 0, 2, a, a, ws, null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte aligned" in _err(g4)
    st = lib.q4_prepkv(a, a, a, m, a, a, 8, 256, 4096, 6144, 0, 1024, 1024, a, null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte aligned" in _err(g4)


def test_gated_w4a16_argument_errors_without_gpu(g4):
    """The gated W4A16 GEMM (interleaved gate/up rows) takes an even row
    count, a workspace of at least one split of fp32 partials, and 16-byte
    aligned operands; every refusal comes before a launch."""
    lib = g4._lib.lib()
    a, m, null = C.c_void_p(1 << 20), C.c_void_p((1 << 20) + 8), C.c_void_p(0)
    need = lib.q4_gemm_w4a16_gated_workspace_bytes(128, 30720, 3840)
    assert need == 2 * 128 * 30720 * 4   # split 2 at the prefill chunk's gate/up
    assert lib.q4_gemm_w4a16_gated_workspace_bytes(128, 30721, 3840) == 0
    assert lib.q4_gemm_w4a16_gated_workspace_bytes(2048, 1024, 256) == 2048 * 1024 * 4  # split 1: still partials
    st = lib.q4_gemm_w4a16_gated(a, a, a, a, 128, 30721, 3840, a, need, null)
    assert st == g4._lib.Q4_ERR_ARG and "N even" in _err(g4)
    st = lib.q4_gemm_w4a16_gated(a, a, a, a, 128, 30720, 3840, null, need, null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)
    st = lib.q4_gemm_w4a16_gated(a, a, a, a, 128, 30720, 3840, a, need - 4, null)
    assert st == g4._lib.Q4_ERR_ARG and "workspace too small" in _err(g4)
    st = lib.q4_gemm_w4a16_gated(m, a, a, a, 128, 30720, 3840, a, need, null)
    assert st == g4._lib.Q4_ERR_ARG and "16-byte aligned" in _err(g4)


def test_gemm_normadd_argument_errors_without_gpu(g4):
    """The GEMM + normadd entry point: w2 and y come together, a workspace of
    fp32 partials is required, and the W4A16 checks apply."""
    lib = g4._lib.lib()
    a, null = C.c_void_p(1 << 20), C.c_void_p(0)
    need = lib.q4_gemm_w4a16_normadd_workspace_bytes(128, 3840, 15360)
    assert need == 16 * 128 * 3840 * 4   # the down projection at M = 128 splits K 16 ways
    assert lib.q4_gemm_w4a16_normadd_workspace_bytes(128, 3840, 100) == 0
    st = lib.q4_gemm_w4a16_normadd(a, a, a, 128, 3840, 15360, a, a, C.c_float(0.5), a, null, 1, a, need, null)
    assert st == g4._lib.Q4_ERR_ARG and "come together" in _err(g4)
    st = lib.q4_gemm_w4a16_normadd(a, a, a, 128, 3840, 15360, a, a, C.c_float(0.5), null, null, 1, a, need - 4, null)
    assert st == g4._lib.Q4_ERR_ARG and "workspace too small" in _err(g4)
    st = lib.q4_gemm_w4a16_normadd(a, a, a, 128, 3840, 15360, null, a, C.c_float(0.5), null, null, 1, a, need, null)
    assert st == g4._lib.Q4_ERR_ARG and "null" in _err(g4)


def test_qkv_prepkv_argument_errors_without_gpu(g4):
    """The stacked q/k/v GEMM + prepkv: N must be nq + nk (+ nk), the q rows
    wide and aligned enough, the workspace large enough; refusals come before
    any launch."""
    lib = g4._lib.lib()
    a, m, null = C.c_void_p(1 << 20), C.c_void_p((1 << 20) + 2), C.c_void_p(0)
    need = lib.q4_gemm_w4a16_normadd_workspace_bytes(128, 8192, 3840)
    args = lambda N=8192, q=a, ldq=8192, keqv=0, ws_bytes=need: (a, a, a, 128, N, 3840, q, ldq, 4096, a, a, a, a, a,
                                                                 8, 256, keqv, 1024, 1024, a, a, ws_bytes, null)
    st = lib.q4_gemm_w4a16_qkv_prepkv(*args(N=8190))
    assert st == g4._lib.Q4_ERR_ARG and "nq + nk" in _err(g4)
    st = lib.q4_gemm_w4a16_qkv_prepkv(*args(keqv=1))   # k == v: N would be 4096 + 2048
    assert st == g4._lib.Q4_ERR_ARG and "nq + nk" in _err(g4)
    st = lib.q4_gemm_w4a16_qkv_prepkv(*args(ldq=4094))
    assert st == g4._lib.Q4_ERR_ARG and "ldq" in _err(g4)
    st = lib.q4_gemm_w4a16_qkv_prepkv(*args(q=m))
    assert st == g4._lib.Q4_ERR_ARG and "aligned" in _err(g4)
    st = lib.q4_gemm_w4a16_qkv_prepkv(*args(ws_bytes=need - 4))
    assert st == g4._lib.Q4_ERR_ARG and "workspace too small" in _err(g4)


def test_plan_overrides_are_explicit(g4, tune, monkeypatch):
    """Launch plans change only through q4_tune_set (environment variables are
    never read); overrides clear individually and all at once, and an unknown
    knob is an argument error."""
    lib = g4._lib.lib()
    knobs = g4._lib.TUNE_KNOBS
    monkeypatch.setenv("Q4MI_GEMV_ROWS", "8")
    assert all(lib.q4_tune_get(k) == -1 for k in knobs.values())
    split = lib.q4_gemv_auto_split(1024, 3840)
    tune("gemv_rows", 16)
    tune("w4a16_kg", 2)
    assert lib.q4_tune_get(knobs["gemv_rows"]) == 16 and lib.q4_tune_get(knobs["w4a16_kg"]) == 2
    tune("gemv_rows", None)
    assert lib.q4_tune_get(knobs["gemv_rows"]) == -1 and lib.q4_tune_get(knobs["w4a16_kg"]) == 2
    lib.q4_tune_reset()
    assert all(lib.q4_tune_get(k) == -1 for k in knobs.values())
    assert lib.q4_gemv_auto_split(1024, 3840) == split
    assert lib.q4_tune_set(len(knobs), 1) == g4._lib.Q4_ERR_ARG and "unknown tuning knob" in _err(g4)
    assert lib.q4_tune_get(len(knobs)) == -1 and lib.q4_tune_get(-1) == -1


def test_noalloc_rejects_bad_arguments_before_any_device_work(g4):
    """q4_gemv_noalloc checks every argument before it looks up its scratch
    array or queues the ticket fill of a split-K plan (N=1024 plans a split):
    with no GPU at all, bad calls still return Q4_ERR_ARG with a message."""
    lib = g4._lib.lib()
    p, null = C.c_void_p(4096), C.c_void_p(0)
    assert lib.q4_gemv_auto_split(1024, 3840) > 1
    cases = [((null, 1, p, p, 0, C.c_float(1.0), p, 0, 1024, 3840, 0, null), "null"),
             ((p, 1, p, p, 7, C.c_float(1.0), p, 0, 1024, 3840, 0, null), "scale format"),
             ((p, 1, p, p, 0, C.c_float(1.0), p, 5, 1024, 3840, 0, null), "y dtype"),
             ((C.c_void_p(4100), 1, p, p, 0, C.c_float(1.0), p, 0, 1024, 3840, 0, null), "aligned")]
    for args, msg in cases:
        assert lib.q4_gemv_noalloc(*args) == g4._lib.Q4_ERR_ARG
        assert msg in _err(g4), (msg, _err(g4))
