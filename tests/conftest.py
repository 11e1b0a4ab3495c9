import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "oracle", REPO / "cgcl-coraanns_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name):
    """Read a ref_dump directory (manifest.txt + raw little-endian arrays)."""
    d = GOLDEN / name
    out = {}
    dt = {"u8": np.uint8, "u32": np.uint32, "u64": np.uint64, "i32": np.int32, "f32": np.float32}
    for line in (d / "manifest.txt").read_text().split("\n"):
        if not line.strip():
            continue
        key, dtype, shape = line.split()
        shp = tuple(int(s) for s in shape.split(","))
        out[key] = np.fromfile(d / f"{key}.bin", dtype=dt[dtype]).reshape(shp)
    return out


def read_fbin(path, dtype=np.float32):
    raw = np.fromfile(path, dtype=np.uint8)
    rows, cols = np.frombuffer(raw[:8], dtype=np.uint32)
    return np.frombuffer(raw[8:], dtype=dtype).reshape(int(rows), int(cols)).copy()


@pytest.fixture(scope="session")
def golden():
    return load_golden
