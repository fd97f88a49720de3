"""Shared test setup: the `gpu` marker, import paths, device fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flashengine.cpp_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def dev():
    """The HIP device; GPU tests fail (not skip) when the library is missing."""
    import torch

    import feattn

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    feattn.lib()  # raises if libfeattn.so is not built: no silent fallback
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)


# (name, max |out err|, max |out err| / (atol + rtol |want|), max |lse err|)
# of the full-size sampled parity checks, printed in the session summary.
_ERRORS = []


@pytest.fixture
def err_report():
    def record(name, out, lse, want_out, want_lse, atol=1e-2, rtol=1e-2):
        """lse / want_lse may be None (the reference's own attention has no
        LSE output)."""
        d = (out.float() - want_out.float()).abs()
        ratio = (d / (atol + rtol * want_out.float().abs())).max().item()
        le = None if lse is None else (lse - want_lse).abs().max().item()
        _ERRORS.append((name, d.max().item(), ratio, le))

    return record


def pytest_terminal_summary(terminalreporter):
    if not _ERRORS:
        return
    terminalreporter.write_sep("-", "attention parity headroom (full-size sampled rows; vs oracle, "
                                    "and vs the reference's own ATen attention on the device: *_ref)")
    for name, e, ratio, le in _ERRORS:
        tail = "no LSE output" if le is None else f"max|lse err| {le:.3e}"
        terminalreporter.write_line(
            f"{name:18s} max|out err| {e:.3e}  (fraction of the 1e-2+1e-2|b| bound: {ratio:.3f})  {tail}")
