import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
# The host-side package lives in llama.zig_amd/ (a directory name Python
# cannot import directly because of the dot), so its parent goes on the path.
for p in (ROOT / "llama.zig_amd", ROOT / "tests", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# The backend's device-side fusion (GLU / ADD / ADD_ID on the device, fused
# gate / up / GLU runs in graph_compute) is opt-in; the tests in this process
# exercise it.  The default answer (MUL_MAT / MUL_MAT_ID only) is checked in
# fresh processes by test_backend_abi.py.
os.environ.setdefault("GGML_HIP_FUSION", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
