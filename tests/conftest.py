"""Test configuration: markers, import paths and the in-tree native build."""

from __future__ import annotations

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "minifield-training_amd"
for path in (ROOT, PKG_DIR):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def _ensure_library() -> None:
    lib = PKG_DIR / "mfattn" / "libmfattn.so"
    if not lib.exists():
        # load build.py by path: importing the package would need the library
        import importlib.util

        spec = importlib.util.spec_from_file_location("_mfattn_build", PKG_DIR / "mfattn" / "build.py")
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        module.build(verbose=False)


_ensure_library()


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """One line per full-shape bf16 parity case (C2-C5 outputs and gradients): the raw
    max-abs error against the fp32 reference and the error beyond one bf16 rounding,
    which the tests hold below 2e-2."""
    helpers = sys.modules.get("_helpers")
    rows = getattr(helpers, "PARITY_SUMMARY", None) if helpers else None
    if not rows:
        return
    terminalreporter.write_sep("-", "bf16 parity at the BASELINE shapes")
    for label, raw, excess in rows:
        terminalreporter.write_line(f"{label:<10} max-abs {raw:.4f}  beyond-rounding {excess:.4f}")
