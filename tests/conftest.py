import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import esimd_learning_amd  # noqa: E402,F401  (puts the drop-in package on sys.path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")


@pytest.fixture(scope="session")
def ops():
    """The drop-in package; importing it loads the HIP build or fails."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return esimd_learning_amd.ops()


@pytest.fixture(scope="session")
def dev():
    return "cuda:0"


def assert_close_fp(out, ref, what="", atol_frac=1e-2, rtol=2e-2):
    """Tolerance of the op pack for floating-point outputs (the bar BASELINE
    states: max-abs error <= 1e-2 * max|ref| and rtol 2e-2).

    Two conditions, both asserted:
      * max |out - ref| <= atol_frac * max|ref|   (the max-abs bound, alone);
      * every element |out - ref| <= atol + rtol * |ref|, atol = atol_frac * max|ref|.
    """
    import torch
    out = torch.as_tensor(out).detach().cpu().double()
    ref = torch.as_tensor(ref).detach().cpu().double()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    refmax = ref.abs().max().item()
    atol = atol_frac * refmax
    err = (out - ref).abs()
    bad = err > atol + rtol * ref.abs()
    maxerr = err.max().item() if err.numel() else 0.0
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements out of tolerance; max err {maxerr:.4g}, "
                           f"max|ref| {refmax:.4g}")
    assert maxerr <= atol, f"{what}: max-abs error {maxerr:.4g} > {atol_frac:g} * max|ref| = {atol:.4g}"
    return maxerr, refmax
