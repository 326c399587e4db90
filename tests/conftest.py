import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _ensure_built():
    lib = os.path.join(ROOT, "hachiue_amd", "lib", "libhachiue_sampler.so")
    orc = os.path.join(ROOT, "oracle", "liborc_sampler.so")
    if not os.path.exists(orc):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not os.path.exists(lib):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "hachiue_amd", "csrc")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def sampler():
    from hachiue_amd import Sampler
    s = Sampler(0)
    yield s
    s.close()


@pytest.fixture(scope="session")
def sampler_chunk():
    """A context that routes every row to the chunk + finalize kernels (the
    row kernel is used only for calls with at least HS_ROW_KERNEL_MIN_ROWS
    rows, read at context creation)."""
    from hachiue_amd import Sampler
    old = os.environ.get("HS_ROW_KERNEL_MIN_ROWS")
    os.environ["HS_ROW_KERNEL_MIN_ROWS"] = str(1 << 30)
    try:
        s = Sampler(0)
    finally:
        if old is None:
            del os.environ["HS_ROW_KERNEL_MIN_ROWS"]
        else:
            os.environ["HS_ROW_KERNEL_MIN_ROWS"] = old
    yield s
    s.close()


@pytest.fixture(params=["row", "chunk"])
def any_sampler(request, sampler, sampler_chunk):
    return sampler if request.param == "row" else sampler_chunk
