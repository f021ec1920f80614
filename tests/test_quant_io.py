"""On-disk quantized weights (vk_engine.save_quant / load_quant): a round
trip is bit-exact for every stored array and keeps shape, split, e4m3 lift
and the optional int8 weights; files of another format or with missing or
mis-sized arrays are refused. CPU tensors here; the GPU tests check that
GEMVs on loaded weights give the same bits as on the originals and that the
loaded arrays and GEMV match the oracle."""
import importlib

import numpy as np
import pytest
import torch


def _qw(E, ops, N, K, e4m3=False, w8=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    wb, se = ops.dev_sizes(N, K)
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (wb // 4,), dtype=torch.int64, generator=g).to(torch.int32)
    sc16 = torch.rand(se, generator=g).to(torch.float16)
    bs16 = E.Buf(tensor=sc16)
    bs = E.Buf(tensor=torch.randint(0, 255, (se,), dtype=torch.int32, generator=g).to(torch.uint8)) if e4m3 else bs16
    w8b = E.Buf(tensor=torch.randint(-127, 128, (N * K,), dtype=torch.int32, generator=g).to(torch.int8)) if w8 else None
    sw8 = E.Buf(tensor=torch.rand(N, generator=g).to(torch.float16)) if w8 else None
    return (E.QW(E.Buf(tensor=words), bs, 3, K // 32, 0.125 if e4m3 else 1.0, bs16, w8b, sw8), (N, K))


def test_round_trip_bit_exact(g4, tmp_path):
    E = importlib.import_module("g4mi.vk_engine")
    ops = importlib.import_module("g4mi.ops")
    mats = {"q_proj": _qw(E, ops, 4096, 256), "down": _qw(E, ops, 100, 96, e4m3=True, seed=1),
            "gate": _qw(E, ops, 64, 128, w8=True, seed=2)}
    p = tmp_path / "model.q4mi.safetensors"
    E.save_quant(p, mats)
    back = E.load_quant(p, device="cpu")
    assert sorted(back) == sorted(mats)
    for name, ((bw, bs, split, nblk, inv, bs16, w8, sw8), shape) in mats.items():
        (bw2, bs2, split2, nblk2, inv2, bs162, w82, sw82), shape2 = back[name]
        assert shape2 == shape and (split2, nblk2, inv2) == (split, nblk, inv)
        assert torch.equal(bw2.t, bw.t) and torch.equal(bs162.t, bs16.t) and torch.equal(bs2.t, bs.t)
        assert bs2.t.dtype == bs.t.dtype
        assert (w82 is None) == (w8 is None)
        if w8 is not None:
            assert torch.equal(w82.t, w8.t) and torch.equal(sw82.t, sw8.t)


def test_refuses_foreign_or_broken_files(g4, tmp_path):
    E = importlib.import_module("g4mi.vk_engine")
    ops = importlib.import_module("g4mi.ops")
    from safetensors.torch import save_file
    p = tmp_path / "other.safetensors"
    save_file({"x": torch.zeros(4)}, str(p), metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a q4mi"):
        E.load_quant(p, device="cpu")
    (qw, (N, K)) = _qw(E, ops, 64, 64)
    good = tmp_path / "good.safetensors"
    E.save_quant(good, {"m": (qw, (N, K))})
    # the same arrays declared as a different shape
    from safetensors import safe_open
    with safe_open(str(good), framework="pt") as f:
        meta = dict(f.metadata())
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    meta["m"] = meta["m"].replace('"N": 64', '"N": 128')
    bad = tmp_path / "bad.safetensors"
    save_file(tensors, str(bad), metadata=meta)
    with pytest.raises(ValueError, match="wrong size"):
        E.load_quant(bad, device="cpu")
    del tensors["m.sc16"]
    save_file(tensors, str(bad), metadata=dict(meta, m=meta["m"].replace('"N": 128', '"N": 64')))
    with pytest.raises(ValueError, match="lacks"):
        E.load_quant(bad, device="cpu")
    with pytest.raises(ValueError, match="may not contain"):
        E.save_quant(tmp_path / "x.safetensors", {"a.b": (qw, (N, K))})


def test_refuses_bad_metadata_and_side_arrays(g4, tmp_path):
    E = importlib.import_module("g4mi.vk_engine")
    ops = importlib.import_module("g4mi.ops")
    from safetensors import safe_open
    from safetensors.torch import save_file
    good = tmp_path / "good.safetensors"
    E.save_quant(good, {"m": _qw(E, ops, 64, 128, e4m3=True, w8=True)})
    with safe_open(str(good), framework="pt") as f:
        meta = dict(f.metadata())
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    bad = tmp_path / "bad.safetensors"

    def refused(t, m, match):
        save_file(t, str(bad), metadata=m)
        with pytest.raises(ValueError, match=match):
            E.load_quant(bad, device="cpu")

    refused(tensors, dict(meta, m=meta["m"].replace('"nblk": 4', '"nblk": 3')), "bad shape")
    refused(dict(tensors, **{"m.sc8": tensors["m.sc8"][:-64]}), meta, "e4m3 scales of the wrong size")
    refused(dict(tensors, **{"m.w8": tensors["m.w8"][:-128]}), meta, "int8 weights of the wrong size")
    refused(dict(tensors, **{"m.sw8": tensors["m.sw8"][:-1]}), meta, "int8 weights of the wrong size")
    t2 = dict(tensors)
    del t2["m.sw8"]
    refused(t2, meta, "only one of")
    E.load_quant(good, device="cpu")          # the untouched file still loads


@pytest.mark.gpu
def test_gemv_on_loaded_weights_same_bits(g4, gpu, tmp_path):
    E = importlib.import_module("g4mi.vk_engine")
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((2048, 3840)) * 0.05).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal(3840).astype(np.float16)).cuda()
    for fp8 in (False, True):
        qw = E.quant(W, pf=True, fp8=fp8, prefill_i8=True)
        p = tmp_path / f"w{int(fp8)}.safetensors"
        E.save_quant(p, {"w": (qw, (2048, 3840))})
        (qw2, shape) = E.load_quant(p)["w"]
        fmt = gpu.SCALE_E4M3 if fp8 else gpu.SCALE_F16
        y1 = gpu.gemv(x, qw.bw.t, qw.bs.t, 2048, 3840, scale_fmt=fmt, inv=qw.inv)
        y2 = gpu.gemv(x, qw2.bw.t, qw2.bs.t, 2048, 3840, scale_fmt=fmt, inv=qw2.inv)
        assert torch.equal(y1, y2)
        assert torch.equal(qw.w8.t, qw2.w8.t) and torch.equal(qw.sw8.t, qw2.sw8.t)
@pytest.mark.gpu
def test_loaded_weights_match_oracle(g4, gpu, tmp_path):
    """quant -> save_quant -> load_quant gives the oracle's device arrays
    (src/vk_engine.py:125-159 restated in oracle/q4_oracle.py), and the GEMV
    on the loaded weights matches the oracle's dequant+matmul."""
    from oracle import q4_oracle as O

    E = importlib.import_module("g4mi.vk_engine")
    rng = np.random.default_rng(0)
    N, K = 2048, 3840
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    W[5, :32] = 0.0                                     # a zero block (scale floor)
    xh = rng.standard_normal(K).astype(np.float16)
    x = torch.from_numpy(xh).cuda()
    q, sc = O.quant_codes(W)
    W8, sw = O.w8_fold(q, sc)
    e8, inv, _ = O.e4m3_lift(sc)
    for fp8 in (False, True):
        qw = E.quant(W, pf=True, fp8=fp8, prefill_i8=True)
        p = tmp_path / f"w{int(fp8)}.safetensors"
        E.save_quant(p, {"w": (qw, (N, K))})
        (qw2, shape) = E.load_quant(p)["w"]
        assert shape == (N, K) and qw2.nblk == K // 32
        assert (qw2.bw.t.cpu().numpy().view(np.uint32) == O.pack_dev(q)).all()
        assert (qw2.bs16.t.cpu().numpy().view(np.uint16) == O.scales_dev(sc.astype(np.float16)).view(np.uint16)).all()
        assert (qw2.w8.t.cpu().numpy() == O.pack_w8_dev(W8)).all()
        assert (qw2.sw8.t.cpu().numpy().view(np.uint16) == sw.astype(np.float16).view(np.uint16)).all()
        if fp8:
            assert qw2.inv == inv
            assert (qw2.bs.t.cpu().numpy() == O.scales_dev(e8)).all()
            s_used = O.e4m3_decode(e8).astype(np.float32)
        else:
            s_used = sc.astype(np.float16).astype(np.float32)
        fmt = gpu.SCALE_E4M3 if fp8 else gpu.SCALE_F16
        y = gpu.gemv(x, qw2.bw.t, qw2.bs.t, N, K, scale_fmt=fmt, inv=qw2.inv)
        ref = O.gemv_ref(q, s_used, xh, inv if fp8 else 1.0)
        assert O.normwise_rel_err(y.float().cpu().numpy(), ref) <= 1e-3   # fp16 output, fp32 accumulate
