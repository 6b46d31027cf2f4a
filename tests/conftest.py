"""Shared test set-up: import paths, the `gpu` marker, GPU fixtures.

GPU tests (marked `gpu`) run on an MI355X box; they fail, never skip, when
the HIP library cannot reach a gfx950 device, so a silent CPU path can
never make them pass. CPU tests cover the oracle, the host logic and the
library's exports.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("aegean-tge_amd", "oracle", ""):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line per full-size parity check that ran: its outputs, worst
    absolute error and worst ratio of error to the bound (2e-3 + 1e-3|ref|),
    so the margins appear in the tail of a quiet run."""
    from _util import MARGINS
    if MARGINS:
        terminalreporter.write_line(
            "parity margins (outputs, max abs err, max err/bound): " +
            "; ".join(f"{k} {n} {e:.2e} {r:.3f}" for k, (n, e, r) in MARGINS.items()))


@pytest.fixture(scope="session")
def tk():
    import tge_kv
    tge_kv.lib()
    return tge_kv


@pytest.fixture(scope="session")
def gpu(tk):
    """The product library with a ready gfx950 backend (fails otherwise)."""
    status = tk.lib().tge_backend_init()
    assert status == tk.OK, (
        f"gfx950 backend unavailable: {tk.lib().tge_last_error().decode()} "
        f"(arch '{tk.lib().tge_backend_arch().decode()}')")
    return tk


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.orc()
    return oracle
