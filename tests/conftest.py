import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "mini-llm-inference-server_amd"
for p in (str(ROOT), str(PKG), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP library.  GPU tests fail loudly (not skip) when it is missing on a machine with a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from minillm import _native
    from minillm.attention.hip_backend import HipBackend

    HipBackend.check_plan = True  # every plan a GPU test builds through the backend must fit its capacities
    return _native.lib()


@pytest.fixture(params=[256, 128], ids=["rows256", "rows128"])
def prefill_rows(request, monkeypatch):
    """Forces the prefill items to 256 (token, head) rows (8-wavefront workgroups) or 128 (4-wavefront
    workgroups, two per CU), whatever the host's choice for the step."""
    monkeypatch.setenv("MLLM_PREFILL_ROWS", str(request.param))
    return request.param
