"""pytest configuration: markers, import paths and shared GPU fixtures.

`-m "not gpu"` runs everywhere (oracle, host logic, ABI exports, algebra);
`-m gpu` needs an MI355X (gfx950) and fails loudly, never skips, when the
device is present but libhelix.so is not built.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU oracle work")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The HIP device and a HELIX context on it (libhelix.so must load)."""
    if not _has_gpu():
        pytest.skip("no GPU visible")
    import torch
    from helix_amd.abi import Context, LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"GPU present but {LIB_PATH} is not built")
    dev = torch.cuda.current_device()
    name = torch.cuda.get_device_properties(dev).gcnArchName
    print(f"[gpu] device {dev}: {name}", flush=True)
    ctx = Context(dev)
    yield ctx
    ctx.close()
