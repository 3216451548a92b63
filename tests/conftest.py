import os
import sys

import pytest

REPO_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO_ROOT, "fused-attention_amd")
for p in (REPO_ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running case sweep")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def lib():
    from attention import _lib
    return _lib.load()


def pytest_sessionfinish(session, exitstatus):
    """Write the per-case records of the reference suites (tests/gpu_util.RECORDS) as CSVs in
    the reference's layout under $FA_RECORDS_DIR (default out/correctness/ at the repository root)."""
    mod = sys.modules.get("tests.gpu_util") or sys.modules.get("gpu_util")
    if mod is None or not getattr(mod, "RECORDS", None):
        return
    root = os.environ.get("FA_RECORDS_DIR", os.path.join(REPO_ROOT, "out", "correctness"))
    for path in mod.write_records(root):
        print(f"\nper-case record: {os.path.relpath(path, REPO_ROOT)}")
