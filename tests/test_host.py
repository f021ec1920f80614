"""Host-side logic on the CPU: error mapping, the labelled fence-timeout
message the reference's callers match on (src/vk_engine.py:299-302,
src/serve.py:49), split/workspace bookkeeping, and loud failure without a
GPU. The timeout is forced from the host (the wait entry point reports
expiry), so no GPU work is involved."""
import ctypes as C
import importlib

import pytest


class _FakeLib:
    def __init__(self, status, msg=b""):
        self.status, self.msg = status, msg

    def q4_stream_wait(self, stream, ms):
        return self.status

    def q4_last_error(self):
        return self.msg


@pytest.fixture
def ops(g4, monkeypatch):
    ops = importlib.import_module("g4mi.ops")
    monkeypatch.setattr(ops, "_stream", lambda s=None: C.c_void_p(0))
    return ops


def test_fence_timeout_message(ops, g4, monkeypatch):
    fake = _FakeLib(g4._lib.Q4_ERR_TIMEOUT, b"stream wait timed out after 5 ms")
    monkeypatch.setattr(ops, "lib", lambda: fake)
    monkeypatch.setattr(g4._lib, "lib", lambda path=None: fake)
    with pytest.raises(RuntimeError, match=r"GPU fence TIMEOUT after 5ms at \[decode pos=7\]"):
        ops.stream_wait(None, 5, "decode pos=7")


def test_wait_other_error_is_q4error(ops, g4, monkeypatch):
    fake = _FakeLib(g4._lib.Q4_ERR_HIP, b"hipStreamQuery failed: boom")
    monkeypatch.setattr(ops, "lib", lambda: fake)
    monkeypatch.setattr(g4._lib, "lib", lambda path=None: fake)
    with pytest.raises(g4._lib.Q4Error, match="boom"):
        ops.stream_wait(None, 5, "x")


def test_wait_ok(ops, g4, monkeypatch):
    fake = _FakeLib(0)
    monkeypatch.setattr(ops, "lib", lambda: fake)
    ops.stream_wait(None, 0, "x")


def test_engine_wait_uses_env_bound(g4, monkeypatch):
    E = importlib.import_module("g4mi.vk_engine")
    seen = {}
    monkeypatch.setattr(E.ops, "stream_wait", lambda s, ms, label: seen.update(ms=ms, label=label))
    monkeypatch.setattr(E, "_FENCE_MS", 1234)
    E.wait(None, "decode pos=3")
    assert seen == {"ms": 1234, "label": "decode pos=3"}


def test_call_raises_with_library_message(g4):
    with pytest.raises(g4._lib.Q4Error, match="multiple of 32"):
        g4._lib.call("q4_dev_bytes", 64, 33, None, None)


def test_ops_reject_host_tensors(ops):
    torch = pytest.importorskip("torch")
    with pytest.raises(ValueError, match="device tensors"):
        ops._p(torch.zeros(4))


def test_graph_capture_refuses_workspace_allocation(ops, g4, monkeypatch):
    monkeypatch.setattr(ops, "_CAPTURING", [1])
    with pytest.raises(RuntimeError, match="before the capture"):
        ops.default_workspace(512, 3840)  # a small matrix: split-K, needs a workspace


def test_split_matches_library(ops, g4):
    for N, K in [(15360, 3840), (262144, 3840), (3840, 15360), (2048, 3840), (30720, 3840)]:
        s = ops.auto_split(N, K)
        assert 1 <= s <= K // 32
        ws = ops.Workspace.bytes_for(N, K)
        assert (ws == 0) == (s == 1)


def test_norm_gemv_fusion_alternates_the_residual(g4):
    """The recorder's norm-into-GEMV pass on CPU tensors (no launch): each
    fused launch reads the buffer that holds the residual and writes the
    other one, later descriptors that use the residual follow it, an fp32
    norm output or an lm_head-sized GEMV stays unfused, and a final copy
    puts the residual back in its own buffer when the count is odd."""
    import torch

    E = importlib.import_module("g4mi.vk_engine")
    ops = importlib.import_module("g4mi.ops")
    D = 256
    f32 = lambda: torch.zeros(D, dtype=torch.float32)  # noqa: E731
    h, x, w, w2 = f32(), f32(), f32(), f32()
    y16 = torch.zeros(D, dtype=torch.float16)
    y32 = f32()

    def gemv_desc(xin, N):
        dp = (xin, None, None, ops.SCALE_F16, 1.0, torch.zeros(N), N, D, 1, None)
        return E.GemvDesc(dp, None, N, 1, (N + 63) // 64)

    na = lambda y: E.OpDesc(ops.normadd_rmsnorm, (x, w, h, w2, 0.0, y), {})  # noqa: E731
    seq = [na(y16), ("gemvs", [gemv_desc(y16, 512), gemv_desc(y16, 256)]),
           E.OpDesc(ops.normadd, (x, w, h, 0.5), {}),
           na(y32), ("gemvs", [gemv_desc(y32, 512)]),
           na(y16), ("gemvs", [gemv_desc(y16, 262144)])]
    out = E._fuse_norm_gemvs(seq)
    assert out[0][0] == "gemvs_nx"
    a, ww, h_in, h_out, ww2, sc = out[0][1]
    assert h_in.data_ptr() == h.data_ptr() and h_out.data_ptr() != h.data_ptr() and h_out.numel() == D
    twin = h_out
    # the unfused normadd and the fp32-output norm now act on the twin
    assert out[1].fn is ops.normadd and out[1].args[2].data_ptr() == twin.data_ptr()
    assert out[2].fn is ops.normadd_rmsnorm and out[2].args[2].data_ptr() == twin.data_ptr()
    assert out[3][0] == "gemvs"
    # lm_head-sized GEMV: its norm stays a launch of its own, on the twin
    assert out[4].fn is ops.normadd_rmsnorm and out[4].args[2].data_ptr() == twin.data_ptr()
    assert out[5][0] == "gemvs"
    # one fused launch: the residual is copied back into h at the end
    assert out[6].fn is E._copy_into and out[6].args[0].data_ptr() == h.data_ptr()
    assert out[6].args[1].data_ptr() == twin.data_ptr() and len(out) == 7
    # two fused launches: back in h, no copy
    seq2 = [na(y16), ("gemvs", [gemv_desc(y16, 512)]), na(y16), ("gemvs", [gemv_desc(y16, 512)])]
    out2 = E._fuse_norm_gemvs(seq2)
    assert [op[0] for op in out2] == ["gemvs_nx", "gemvs_nx"]
    assert out2[1][1][2].data_ptr() == out2[0][1][3].data_ptr()      # second reads what the first wrote
    assert out2[1][1][3].data_ptr() == h.data_ptr()


def test_prefill_gemm_fusions_pair_gemms_with_their_consumers(g4, monkeypatch):
    """The prefill recorder's GEMM passes on CPU tensors (no launch): a W4A16
    GEMM with fp16 in and out followed by the pre_na(+norm) that reads its
    output becomes one gemm_w4a16_normadd; the stacked q/k/v GEMM followed by
    the pre_prepkv that reads its k/v columns becomes one
    gemm_w4a16_qkv_prepkv (q stored at the GEMM's own output with ldq = N);
    a consumer of some other buffer, or a GEMM with a cast, stays as it is."""
    import torch

    E = importlib.import_module("g4mi.vk_engine")
    ops = importlib.import_module("g4mi.ops")
    monkeypatch.setattr(E, "_stage", lambda name, nbytes: E.Buf(tensor=torch.empty(nbytes, dtype=torch.uint8)))
    MC, K = E.MC, 256
    x16 = torch.zeros(MC, K, dtype=torch.float16)
    f32 = lambda n: torch.zeros(n, dtype=torch.float32)  # noqa: E731

    def gmm(N, y16, cin=None):
        return ("gmm", (cin, ("w4a16", x16, torch.zeros(N * K // 8, dtype=torch.int32),
                              torch.zeros(N * K // 32, dtype=torch.float16), N, y16.view(MC, N), None), None, N, K))

    # o projection + pre_na + pre_norm (already merged by _fuse_pre_norms)
    N = 512
    T = torch.zeros(MC * N, dtype=torch.float16)
    h, w, w2, y = f32(MC * N), f32(N), f32(N), torch.zeros(MC * N, dtype=torch.float16)
    na = E.OpDesc(ops.pre_normadd, (T, w, h), dict(M=MC, D=N, scale=0.5, w2=w2, y=y))
    out = E._fuse_gemm_normadd([gmm(N, T), na])
    assert len(out) == 1 and out[0].fn is ops.gemm_w4a16_normadd
    assert out[0].args[3] == N and out[0].args[5].data_ptr() == h.data_ptr()
    assert out[0].kw["scale"] == 0.5 and out[0].kw["y"] is y and out[0].kw["w2"] is w2
    other = torch.zeros(MC * N, dtype=torch.float16)
    na_other = E.OpDesc(ops.pre_normadd, (other, w, h), dict(M=MC, D=N, scale=0.5))
    assert [type(o) for o in E._fuse_gemm_normadd([gmm(N, T), na_other])] == [tuple, E.OpDesc]
    assert len(E._fuse_gemm_normadd([gmm(N, T, cin=("cast_dn", None, None)), na])) == 2
    # the fused launch never writes T: no fusion while a later op reads T, unless a GEMM rewrote it first
    reader = E.OpDesc(ops.pre_rmsnorm, (T, w, y), dict(M=MC, D=N))
    assert len(E._fuse_gemm_normadd([gmm(N, T), na, reader])) == 3
    assert len(E._fuse_gemm_normadd([gmm(N, T), na, gmm(N, T), reader])) == 3   # first pair fused
    assert E._fuse_gemm_normadd([gmm(N, T), na, gmm(N, T), reader])[0].fn is ops.gemm_w4a16_normadd
    x_reads_T = ("gmm", (None, ("w4a16", T.view(MC, N), torch.zeros(N * N // 8, dtype=torch.int32),
                                torch.zeros(N * N // 32, dtype=torch.float16), N, other.view(MC, N), None), None, N, N))
    assert len(E._fuse_gemm_normadd([gmm(N, T), na, x_reads_T])) == 3

    # stacked q/k/v + pre_prepkv, with and without k == v
    nkv, hd, nq = 2, 64, 256
    dyn = torch.zeros(4, dtype=torch.int32)
    tabs = (f32(hd), f32(MC * hd), f32(MC * hd), torch.zeros(8, dtype=torch.float16), torch.zeros(8, dtype=torch.float16))
    for keqv in (False, True):
        nk = nkv * hd
        N = nq + nk * (1 if keqv else 2)
        QKV = torch.zeros(MC * N, dtype=torch.float16)
        kv = QKV[nq:], QKV[nq if keqv else nq + nk:]
        prep = E.OpDesc(ops.pre_prepkv, kv + tabs, dict(M=MC, ld=N, nkv=nkv, hd=hd, stride=64, window=32, dyn=dyn))
        out = E._fuse_gemm_prepkv([gmm(N, QKV), prep])
        assert len(out) == 1 and out[0].fn is ops.gemm_w4a16_qkv_prepkv
        assert out[0].kw["nq"] == nq and out[0].kw["ldq"] == N and out[0].kw["keqv"] is keqv
        assert out[0].args[4].data_ptr() == QKV.data_ptr() and out[0].kw["window"] == 32
        # k/v rows of another buffer: no fusion
        Kp = torch.zeros(MC * N, dtype=torch.float16)
        prep2 = E.OpDesc(ops.pre_prepkv, (Kp[nq:], Kp[nq:]) + tabs,
                         dict(M=MC, ld=N, nkv=nkv, hd=hd, stride=64, window=32, dyn=dyn))
        assert len(E._fuse_gemm_prepkv([gmm(N, QKV), prep2])) == 2


def test_forward_checks_token_and_position_before_any_launch(g4):
    """forward() refuses a token id or position outside the tables it was
    recorded with before touching the step buffer or the GPU."""
    import torch

    E = importlib.import_module("g4mi.vk_engine")
    step = torch.zeros(2, dtype=torch.int32)
    for tid, pos in [(10, 0), (-1, 0), (0, 10), (0, -1)]:
        with pytest.raises(ValueError, match="out of range"):
            E.forward(None, step, tid, pos, vocab=10, max_pos=10)
    assert step.tolist() == [0, 0]
