import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "iree-adreno-genai-tuner_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libq4llm.so")
    config.addinivalue_line("markers", "slow: long-running (large model) test")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name each GPU test on stdout before it runs, so a run that ends abruptly still says where.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield


@pytest.fixture
def kernel_override():
    """Sets library kernel-choice overrides (q4llm.ops.debug_override) for one test and clears every
    override afterwards, pass or fail: kernel_override("attn_generic", 1), kernel_override("x", None)."""
    from q4llm import ops
    try:
        yield ops.debug_override
    finally:
        ops.debug_clear()
