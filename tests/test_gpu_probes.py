"""GPU tier of the ceiling probes (fp64emu_probe_mfma, fp64emu_probe_stream),
through the C ABI.  The benchmark reports the rates they measure beside the
modular GEMM's, so their arithmetic is checked here: the MFMA loop's
accumulators element by element against the host's products of the same
fragments (every mode: registers only, LDS reads, LDS reads plus copies),
its clock counters for sanity, and the streaming kernels' outputs."""
import numpy as np
import pytest
import torch

from fp64_emu import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_probe_mfma_accumulators(dev, mode):
    print(f"case probe_mfma mode {mode}", flush=True)
    src = capi.probe_source(7)
    exp = capi.probe_expected(src)
    assert np.count_nonzero(exp) > exp.size // 2
    src_dev = torch.from_numpy(src).to(dev)
    for steps in (1, 3, 41):
        acc, clk = capi.probe_mfma(src_dev, 8, steps, mode)
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), exp), f"mode {mode}, {steps} steps"
    # An even step count: stage 1's negated A cancels stage 0.
    acc, clk = capi.probe_mfma(src_dev, 8, 2000, mode)
    torch.cuda.synchronize()
    assert not acc.cpu().numpy().any()
    c = clk.cpu().numpy()
    assert (c[:, 1] > c[:, 0]).all() and (c[:, 3] > c[:, 2]).all()
    ghz = (c[:, 1] - c[:, 0]) / (c[:, 3] - c[:, 2]) * 0.1
    print(f"mode {mode}: shader clock {np.median(ghz):.2f} GHz over 8 groups", flush=True)
    assert (ghz > 0.3).all() and (ghz < 3.0).all()


def test_probe_mfma_rejects_bad_arguments(dev):
    src_dev = torch.from_numpy(capi.probe_source(0)).to(dev)
    with pytest.raises(capi.CapiError, match="mode"):
        capi.probe_mfma(src_dev, 1, 1, 3)
    with pytest.raises(capi.CapiError, match="steps"):
        capi.probe_mfma(src_dev, 1, 0, 0)
    with pytest.raises(ValueError, match="source"):
        capi.probe_mfma(src_dev[:100], 1, 1, 0)


def test_probe_stream(dev):
    print("case probe_stream", flush=True)
    n = 1 << 20
    src = (torch.arange(n, dtype=torch.float64, device=dev) % 1000)   # sums stay exact
    dst = torch.zeros(n, dtype=torch.float64, device=dev)
    capi.probe_stream(dst, src, 2)
    torch.cuda.synchronize()
    assert torch.equal(dst, -src)
    capi.probe_stream(dst, None, 1)
    torch.cuda.synchronize()
    assert torch.equal(dst, torch.ones_like(dst))
    dst.zero_()
    capi.probe_stream(dst, src, 0)
    torch.cuda.synchronize()
    groups = min(max(n // 2 // 1024, 1), 4096)
    assert dst[:groups].sum().item() == src.sum().item()
    assert not dst[groups:].any().item()
