"""The measurement probes run at small sizes (they compute nothing of the
model: the checks are that they launch, finish and report sane clocks)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("units", [4, 8, 16])
@pytest.mark.parametrize("chunked", [True, False])
def test_stream_read_probe(gpu, units, chunked):
    g = torch.Generator(device="cuda").manual_seed(units)
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, ((3 << 20) // 4 + 4,), dtype=torch.int32, device="cuda", generator=g)
    comp = torch.randint(-2 ** 31, 2 ** 31 - 1, (buf.numel() // 8 + 1,), dtype=torch.int32, device="cuda",
                         generator=g)
    nxt = torch.zeros_like(buf)
    sink = torch.zeros(512, dtype=torch.int32, device="cuda")
    gpu.probe_stream_read(buf, 96, units=units, chunked=chunked, sink=sink)
    gpu.probe_stream_read(buf, 96, units=units, chunked=chunked, comp=comp, sink=sink)
    gpu.probe_stream_read(buf, 96, units=units, chunked=chunked, next=nxt, prefetch_bytes=1 << 20, sink=sink)
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", [0, 1])
def test_mfma_probe_clocks(gpu, kind):
    wgs, iters = 8, 64
    clocks = torch.zeros((wgs, 2), dtype=torch.int64, device="cuda")
    sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
    ops = torch.randint(-2 ** 31, 2 ** 31 - 1, (16384,), dtype=torch.int32, device="cuda")
    for operands in (None, ops if kind == 0 else ops & (0xBBFFBBFF - 2 ** 32)):
        clocks.zero_()
        gpu.probe_mfma(kind, wgs, iters, clocks, sink, operands)
        torch.cuda.synchronize()
        c = clocks.cpu()
        assert (c[:, 0] > 0).all() and (c[:, 1] > 0).all()
        khz = gpu.probe_wall_clock_khz()
        ghz = (c[:, 0].double() / (c[:, 1].double() / (khz * 1e3))) / 1e9
        assert ((ghz > 0.1) & (ghz < 5.0)).all(), ghz
