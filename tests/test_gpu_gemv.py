"""Decode GEMV (fp16 and e4m3 block scales) vs the oracle.

Tolerance: normwise max|y - ref| / max|ref| <= 1e-3 with the oracle's fp32
dequant+matmul (the reference's own numpy formulation) on the same inputs;
fp32 outputs are held to 2e-5. Full-size shapes are checked entirely against
the oracle plus size-independent properties (linearity, split invariance,
determinism, graph replay == eager).
"""
import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import synth_int4, to_np, upload_int4

pytestmark = pytest.mark.gpu
TOL_F16 = 1e-3
TOL_F32 = 2e-5


def _case(rng, N, K):
    q, s = synth_int4(rng, N, K)
    x = rng.standard_normal(K).astype(np.float16)
    return q, s, x


@pytest.mark.parametrize("N,K", [(64, 32), (100, 96), (256, 256), (520, 3840), (4096, 3840), (3840, 4096),
                                 (2048, 3840), (1000, 15360)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float16, torch.float32),
                                     (torch.float32, torch.float32)])
def test_gemv_f16_scales(gpu, N, K, xdt, ydt):
    rng = np.random.default_rng(N * 7 + K)
    q, s, x = _case(rng, N, K)
    xin = x.astype(np.float32) if xdt == torch.float32 else x
    ref = O.gemv_ref(q, s, xin)
    wq, sc = upload_int4(q, s)
    y = gpu.gemv(torch.from_numpy(xin).cuda(), wq, sc, N, K, y_dtype=ydt)
    err = O.normwise_rel_err(to_np(y).astype(np.float32), ref)
    assert err <= (TOL_F16 if ydt == torch.float16 else TOL_F32), err


@pytest.mark.parametrize("split", [1, 2, 3, 5, 8, 120])
@pytest.mark.parametrize("rows", [None, "8", "64"])
def test_gemv_split_invariance(gpu, split, rows, tune):
    if rows:
        tune("gemv_rows", rows)
    rng = np.random.default_rng(21)
    N, K = 512, 3840
    q, s, x = _case(rng, N, K)
    ref = O.gemv_ref(q, s, x)
    wq, sc = upload_int4(q, s)
    y = gpu.gemv(torch.from_numpy(x).cuda(), wq, sc, N, K, y_dtype=torch.float32, split=split)
    assert O.normwise_rel_err(to_np(y), ref) <= TOL_F32


@pytest.mark.parametrize("rows", ["8", "16", "32", "64"])
@pytest.mark.parametrize("N,nblk", [(64, 3), (256, 37), (192, 200), (320, 481)])
def test_gemv_units_in_flight(gpu, rows, N, nblk, tune):
    """Every rows-per-workgroup x units-in-flight variant against the oracle,
    with block counts that leave the lanes' last round of the load ring
    partly empty (3, 37, 200, 481 blocks), fp16 and fp32 x. The units are
    consumed in the same order whatever the ring size, so U = 4 and U = 8
    give bit-identical outputs."""
    tune("gemv_rows", rows)
    K = 32 * nblk
    rng = np.random.default_rng(N + nblk)
    q, s, x = _case(rng, N, K)
    wq, sc = upload_int4(q, s)
    for xin, ydt, tol in [(x, torch.float16, TOL_F16), (x.astype(np.float32), torch.float32, TOL_F32)]:
        ref = O.gemv_ref(q, s, xin)
        outs = []
        for units in ["4", "8"]:
            tune("gemv_units", units)
            y = gpu.gemv(torch.from_numpy(xin).cuda(), wq, sc, N, K, y_dtype=ydt, split=1)
            assert O.normwise_rel_err(to_np(y).astype(np.float32), ref) <= tol, (units, ydt)
            outs.append(y)
        assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("K,xdt,rows", [(32768, torch.float16, "64"), (32768, torch.float16, "8"),
                                        (16384, torch.float32, "16")])
def test_gemv_largest_x_staging(gpu, K, xdt, rows, tune):
    """The longest x one workgroup stages without a K split (64 KB of x, plus
    the block sums for fp16 x), through q4_gemv and q4_gemv_batch: the same
    rows per workgroup give bit-identical outputs."""
    tune("gemv_rows", rows)
    N = 128
    rng = np.random.default_rng(K + int(rows))
    q, s, x = _case(rng, N, K)
    xin = x if xdt == torch.float16 else x.astype(np.float32)
    ref = O.gemv_ref(q, s, xin)
    wq, sc = upload_int4(q, s)
    xt = torch.from_numpy(xin).cuda()
    y = gpu.gemv(xt, wq, sc, N, K, y_dtype=torch.float32, split=1)
    assert O.normwise_rel_err(to_np(y), ref) <= TOL_F32
    (yb,) = gpu.gemv_batch(xt, [(wq, sc, N, None, None)], K, y_dtype=torch.float32)
    assert torch.equal(y, yb)


def test_gemv_c1_full_size(gpu):
    """Down-projection-sized GEMV N=15360, K=3840, fp16 x and y, seed 0."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal(3840).astype(np.float16)
    codes = rng.integers(-8, 8, (15360, 3840))
    s = np.abs(rng.normal(0, 0.02, (15360, 120))).astype(np.float16).astype(np.float32)
    q = (codes + 8).astype(np.uint8)
    ref = O.gemv_ref(q, s, x)
    wq, sc = upload_int4(q, s)
    y = gpu.gemv(torch.from_numpy(x).cuda(), wq, sc, 15360, 3840)
    yh = to_np(y)
    assert yh.dtype == np.float16
    assert O.normwise_rel_err(yh.astype(np.float32), ref) <= TOL_F16
    assert O.cosine(yh, ref) > 0.99999
    # deterministic: same bits on a second launch (fixed split-K reduction order)
    y2 = gpu.gemv(torch.from_numpy(x).cuda(), wq, sc, 15360, 3840)
    assert torch.equal(y, y2)


def test_gemv_e4m3_scales(gpu):
    """e4m3 block scales; the oracle uses identically rounded scales."""
    rng = np.random.default_rng(2)
    for N, K in [(256, 256), (15360, 3840), (3840, 15360)]:
        q, s, x = _case(rng, N, K)
        e8, inv, _ = O.e4m3_lift(s)
        s_used = O.e4m3_decode(e8)
        ref = O.gemv_ref(q, s_used, x, inv=inv)
        wq, _ = upload_int4(q, s)
        sc8 = torch.from_numpy(O.scales_dev(e8)).cuda()
        y = gpu.gemv(torch.from_numpy(x).cuda(), wq, sc8, N, K, scale_fmt=gpu.SCALE_E4M3, inv=inv,
                     y_dtype=torch.float32)
        assert O.normwise_rel_err(to_np(y), ref) <= TOL_F32


def test_gemv_e4m3_from_gpu_quantizer(gpu):
    rng = np.random.default_rng(3)
    N, K = 1024, 3840
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    q, sc = O.quant_codes(W)
    e8, inv, _ = O.e4m3_lift(sc)
    ref = O.gemv_ref(q, O.e4m3_decode(e8), x, inv=inv)
    wq, _sc16, sc32 = gpu.quantize(torch.from_numpy(W).cuda())
    sc8, ginv = gpu.scales_e4m3(sc32, N, K)
    y = gpu.gemv(torch.from_numpy(x).cuda(), wq, sc8, N, K, scale_fmt=gpu.SCALE_E4M3, inv=ginv)
    assert O.normwise_rel_err(to_np(y), ref) <= TOL_F32


def test_gemv_lm_head_rows(gpu):
    """lm_head shape N=262144, K=3840 (no split-K): every row checked in row slices."""
    N, K = 262144, 3840
    g = torch.Generator(device="cuda").manual_seed(5)
    nblk = K // 32
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * nblk * 4,), dtype=torch.int64, device="cuda",
                          generator=g).to(torch.int32)
    sc = (torch.randn(N * nblk, device="cuda", generator=g) * 0.02).abs().to(torch.float16)
    x = torch.randn(K, device="cuda", generator=g).to(torch.float16)
    y = to_np(gpu.gemv(x, words, sc, N, K, y_dtype=torch.float32))
    wh, sh, xh = to_np(words).view(np.uint32), to_np(sc), to_np(x)
    npan = 256                                              # 16384-row slices, all 16 of them
    for p0 in range(0, N // 64, npan):
        sl = slice(p0 * nblk * 64 * 4, (p0 + npan) * nblk * 64 * 4)
        rows = npan * 64
        q = O.unpack_dev(wh[sl], rows, K)
        s = O.unscales_dev(sh[p0 * nblk * 64:(p0 + npan) * nblk * 64], rows, nblk).astype(np.float32)
        ref = O.gemv_ref(q, s, xh)
        assert O.normwise_rel_err(y[p0 * 64:p0 * 64 + rows], ref) <= TOL_F32


def test_gemv_linearity_full_size(gpu):
    """y(a x1 + b x2) == a y(x1) + b y(x2) at the gate_up shape (size-independent property)."""
    N, K = 30720, 3840
    g = torch.Generator(device="cuda").manual_seed(9)
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * (K // 32) * 4,), dtype=torch.int64, device="cuda",
                          generator=g).to(torch.int32)
    sc = (torch.randn(N * (K // 32), device="cuda", generator=g) * 0.02).abs().to(torch.float16)
    x1 = torch.randn(K, device="cuda", generator=g)
    x2 = torch.randn(K, device="cuda", generator=g)
    y1 = gpu.gemv(x1, words, sc, N, K)
    y2 = gpu.gemv(x2, words, sc, N, K)
    y3 = gpu.gemv(0.5 * x1 + 2.0 * x2, words, sc, N, K)
    comb = 0.5 * y1 + 2.0 * y2
    rel = (y3 - comb).abs().max() / comb.abs().max()
    assert rel.item() < 1e-5


def test_gemv_output_offset_and_untouched_neighbours(gpu):
    rng = np.random.default_rng(6)
    N, K = 200, 128
    q, s, x = _case(rng, N, K)
    wq, sc = upload_int4(q, s)
    out = torch.full((N + 64,), 7.0, device="cuda")
    gpu.gemv(torch.from_numpy(x.astype(np.float32)).cuda(), wq, sc, N, K, y=out[32:32 + N])
    o = to_np(out)
    assert (o[:32] == 7.0).all() and (o[32 + N:] == 7.0).all()
    assert O.normwise_rel_err(o[32:32 + N], O.gemv_ref(q, s, x)) <= TOL_F32


def test_gemv_graph_replay_matches_eager(gpu):
    """A captured sequence of split-K GEMVs sharing one workspace replays
    bit-identically to eager execution, replay after replay."""
    rng = np.random.default_rng(7)
    shapes = [(4096, 3840), (512, 3840), (2048, 3840), (256, 15360), (3840, 4096), (3840, 15360), (15360, 3840)]
    mats = []
    for N, K in shapes:
        q, s = synth_int4(rng, N, K)
        wq, sc = upload_int4(q, s)
        x = torch.from_numpy(rng.standard_normal(K).astype(np.float16)).cuda()
        mats.append((N, K, wq, sc, x, torch.empty(N, device="cuda")))
    ws = gpu.Workspace(max(gpu.Workspace.bytes_for(N, K) for N, K in shapes))

    def body():
        for N, K, wq, sc, x, y in mats:
            gpu.gemv(x, wq, sc, N, K, y=y, ws=ws)

    body()
    torch.cuda.synchronize()
    eager = [m[5].clone() for m in mats]
    for m in mats:
        m[5].zero_()
    graph = gpu.Graph()
    with graph.capture():
        body()
    for _ in range(3):
        for m in mats:
            m[5].zero_()
        torch.cuda.synchronize()
        graph.launch()
        gpu.stream_wait(graph.stream)
        for m, e in zip(mats, eager):
            assert torch.equal(m[5], e)
        torch.cuda.synchronize()
    graph.destroy()


def test_gemv_rejects_small_workspace(gpu):
    N, K = 2048, 3840
    wq = torch.zeros(N * K // 8, dtype=torch.int32, device="cuda")
    sc = torch.zeros(N * K // 32, dtype=torch.float16, device="cuda")
    x = torch.zeros(K, dtype=torch.float16, device="cuda")
    small = gpu.Workspace(256)
    with pytest.raises(gpu._lib.Q4Error, match="workspace"):
        gpu.gemv(x, wq, sc, N, K, ws=small, split=8)


# ---------------------------------------------------------------- batched launch
@pytest.mark.parametrize("shapes,K", [([4096, 2048, 2048], 3840),      # q, k, v of one layer
                                      ([15360, 15360], 3840),         # gate, up
                                      ([64, 100, 520, 8, 64], 256),   # ragged, padded panels
                                      ([3840], 15360)])               # one entry, long K
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float32, torch.float32)])
def test_gemv_batch_vs_oracle(gpu, shapes, K, xdt, ydt):
    rng = np.random.default_rng(sum(shapes) + K)
    x = rng.standard_normal(K).astype(np.float16)
    xin = x.astype(np.float32) if xdt == torch.float32 else x
    mats, refs = [], []
    for N in shapes:
        q, s = synth_int4(rng, N, K)
        wq, sc = upload_int4(q, s)
        mats.append((wq, sc, N, None, None))
        refs.append(O.gemv_ref(q, s, xin))
    ys = gpu.gemv_batch(torch.from_numpy(xin).cuda(), mats, K, y_dtype=ydt)
    tol = TOL_F16 if ydt == torch.float16 else TOL_F32
    for y, ref in zip(ys, refs):
        assert O.normwise_rel_err(to_np(y).astype(np.float32), ref) <= tol


@pytest.mark.parametrize("rows", ["8", "16", "32", "64"])
def test_gemv_batch_bit_identical_to_single_launches(gpu, rows, tune):
    """Same rows-per-workgroup => the batched launch sums in the same order as
    one q4_gemv per matrix (split 1): bit-identical outputs, written into one
    buffer at the q/k/v offsets without touching the gaps."""
    tune("gemv_rows", rows)
    rng = np.random.default_rng(int(rows))
    K = 3840
    shapes = [512, 256, 256]
    x = torch.from_numpy(rng.standard_normal(K).astype(np.float16)).cuda()
    out = torch.full((sum(shapes) + 64,), 7.0, dtype=torch.float16, device="cuda")
    mats, singles, off = [], [], 0
    for N in shapes:
        q, s = synth_int4(rng, N, K)
        wq, sc = upload_int4(q, s)
        mats.append((wq, sc, N, out[off + 16: off + 16 + N], None))
        singles.append(gpu.gemv(x, wq, sc, N, K, split=1))
        off += N
    gpu.gemv_batch(x, mats, K)
    o = to_np(out).view(np.uint16)
    off = 0
    for N, y1 in zip(shapes, singles):
        assert (o[off + 16: off + 16 + N] == to_np(y1).view(np.uint16)).all()
        off += N
    assert (to_np(out)[:16] == 7.0).all() and (to_np(out)[16 + sum(shapes):] == 7.0).all()


def test_gemv_batch_e4m3(gpu):
    rng = np.random.default_rng(5)
    K = 3840
    x = rng.standard_normal(K).astype(np.float16)
    mats, refs = [], []
    for N in (1024, 512):
        q, s32 = synth_int4(rng, N, K)
        e8, inv, _ = O.e4m3_lift(s32)
        sc8 = torch.from_numpy(O.scales_dev(e8)).cuda()
        wq = torch.from_numpy(O.pack_dev(q).view(np.int32)).cuda()
        mats.append((wq, sc8, N, None, inv))
        refs.append(O.gemv_ref(q, O.e4m3_decode(e8), x, inv=inv))
    ys = gpu.gemv_batch(torch.from_numpy(x).cuda(), mats, K, scale_fmt=gpu.SCALE_E4M3, y_dtype=torch.float32)
    for y, ref in zip(ys, refs):
        assert O.normwise_rel_err(to_np(y), ref) <= TOL_F32


# ------------------------------------------------------------ gated gate/up
@pytest.mark.parametrize("I,K", [(15360, 3840), (64, 256), (96, 3840)])
@pytest.mark.parametrize("xdt,adt", [(torch.float16, torch.float16), (torch.float32, torch.float32)])
def test_gemv_gated_vs_oracle(gpu, I, K, xdt, adt):
    """Interleaved gate/up rows and the gelumul epilogue: act = gelu_tanh(W_g x)
    * (W_u x) against the oracle's GEMVs and gelumul (normwise <= 5e-5 fp32,
    the product doubles the GEMVs' relative error; <= 1e-3 fp16). I = 64 and
    96 take the split-K path."""
    from oracle import decode_ops_oracle as D
    rng = np.random.default_rng(I + K)
    qg, sg = synth_int4(rng, I, K)
    qu, su = synth_int4(rng, I, K)
    x = rng.standard_normal(K).astype(np.float16)
    xin = x if xdt == torch.float16 else x.astype(np.float32)
    ref = D.gelumul_ref(O.gemv_ref(qg, sg, xin), O.gemv_ref(qu, su, xin))
    wg, scg = upload_int4(qg, sg)
    wu, scu = upload_int4(qu, su)
    wo, so = gpu.interleave_rows(wg, scg, wu, scu, I, K)
    # layout: row 2i of the interleaved matrix is gate row i, row 2i+1 up row i, bit for bit
    codes = O.unpack_dev(to_np(wo).view(np.uint32), 2 * I, K)
    assert np.array_equal(codes[0::2], qg) and np.array_equal(codes[1::2], qu)
    sc = O.unscales_dev(to_np(so), 2 * I, K // 32)
    assert np.array_equal(sc[0::2], sg.astype(np.float16)) and np.array_equal(sc[1::2], su.astype(np.float16))
    act = gpu.gemv_gated(torch.from_numpy(xin).cuda(), wo, so, 2 * I, K, act_dtype=adt)
    assert act.numel() == I and act.dtype == adt
    tol = 1e-3 if adt == torch.float16 else 5e-5
    assert O.normwise_rel_err(to_np(act).astype(np.float64), ref) <= tol


@pytest.mark.parametrize("N,K,rows", [(15360, 3840, None), (30720, 3840, None), (1024, 4096, "16"), (4096, 15360, "32"),
                                      (128, 256, None)])
def test_gemv_paired_row_groups_bit_identical(gpu, N, K, rows, tune):
    """Two row groups per 512-thread workgroup compute exactly what two
    256-thread workgroups do: q4_gemv, q4_gemv_batch and q4_gemv_gated give
    the same bits with pairing forced on and off (128 rows: split-K, never
    paired), and match the oracle."""
    from oracle import decode_ops_oracle as D
    if rows:
        tune("gemv_rows", rows)
    rng = np.random.default_rng(N + K)
    q, s, x = _case(rng, N, K)
    q2, s2 = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    wq2, sc2 = upload_int4(q2, s2)
    xt = torch.from_numpy(x).cuda()
    wo, so = gpu.interleave_rows(wq, sc, wq2, sc2, N, K) if N % 32 == 0 else (None, None)
    outs = {}
    for pair in ("0", "1"):
        tune("gemv_pair", pair)
        y = gpu.gemv(xt, wq, sc, N, K, y_dtype=torch.float32)
        yb = gpu.gemv_batch(xt, [(wq, sc, N, None, None), (wq2, sc2, N, None, None)], K, y_dtype=torch.float32)
        act = gpu.gemv_gated(xt, wo, so, 2 * N, K, act_dtype=torch.float32)
        torch.cuda.synchronize()
        outs[pair] = (y, yb[0], yb[1], act)
    for a, b in zip(outs["0"], outs["1"]):
        assert torch.equal(a, b)
    assert O.normwise_rel_err(to_np(outs["1"][0]), O.gemv_ref(q, s, x)) <= TOL_F32
    assert O.normwise_rel_err(to_np(outs["1"][2]), O.gemv_ref(q2, s2, x)) <= TOL_F32
    ref_act = D.gelumul_ref(O.gemv_ref(q, s, x), O.gemv_ref(q2, s2, x))
    assert O.normwise_rel_err(to_np(outs["1"][3]).astype(np.float64), ref_act) <= 5e-5
