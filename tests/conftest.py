import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def tsp():
    import tilespmm_amd
    tilespmm_amd.load()
    return tilespmm_amd


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def dc2_path(tmp_path_factory):
    """The reference's only shipped input (data/dc2.mtx), kept gzipped in
    tests/golden; decompressed once per session."""
    import gzip
    import shutil
    src = os.path.join(GOLDEN, "dc2.mtx.gz")
    if not os.path.exists(src):
        pytest.skip("dc2.mtx.gz fixture missing")
    dst = tmp_path_factory.mktemp("mtx") / "dc2.mtx"
    with gzip.open(src, "rb") as fi, open(dst, "wb") as fo:
        shutil.copyfileobj(fi, fo)
    return str(dst)
