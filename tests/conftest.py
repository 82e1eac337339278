import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")

# the library's measurement and probe kernels (probe_fast_math, probe_mfma_f16,
# copy16, ...) are registered only with this set
os.environ.setdefault("PFHIP_TOOLING", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


class Fixture:
    """One reference conformance fixture (tests/native/conformance/fixtures/<name>)."""

    def __init__(self, name):
        import json
        self.name = name
        self.dir = os.path.join(GOLDEN, "wgsl", name)
        with open(os.path.join(self.dir, "meta.json")) as f:
            self.meta = json.load(f)

    def raw(self, fname, dtype=np.uint8):
        return np.fromfile(os.path.join(self.dir, fname), dtype=dtype)

    def input(self, name, dtype=np.uint8):
        return self.raw(f"{name}.bin", dtype)

    @property
    def uniform_u32(self):
        return self.raw("uniform.bin", np.uint32)

    @property
    def uniform_f32(self):
        return self.raw("uniform.bin", np.float32)

    def expected(self, dtype):
        return self.raw("expected.bin", dtype)


@pytest.fixture
def fixture():
    return Fixture
