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


def _context(env):
    """A context created with the given environment overrides (each is read
    at context creation)."""
    from hachiue_amd import Sampler
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return Sampler(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="session")
def sampler_chunk():
    """A context that routes every row to the chunk + finalize kernels (the
    row kernel is used only for calls with at least HS_ROW_KERNEL_MIN_ROWS
    rows)."""
    s = _context({"HS_ROW_KERNEL_MIN_ROWS": str(1 << 30)})
    yield s
    s.close()


@pytest.fixture(scope="session")
def sampler_whole():
    """A context whose row kernel always takes whole rows (no split rows)."""
    s = _context({"HS_ROW_SPLIT": "1"})
    yield s
    s.close()


@pytest.fixture(scope="session")
def sampler_split():
    """A context whose row kernel splits every row over four workgroups, at
    any batch size."""
    s = _context({"HS_ROW_SPLIT": "4"})
    yield s
    s.close()


@pytest.fixture(params=["row", "whole", "split4", "chunk"])
def any_sampler(request, sampler, sampler_whole, sampler_split, sampler_chunk):
    return {"row": sampler, "whole": sampler_whole, "split4": sampler_split,
            "chunk": sampler_chunk}[request.param]
