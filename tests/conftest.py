import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lastro-rust_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs on the GPU box")
    # Build what is missing (the round's build step normally leaves both libraries in place).
    if not os.path.exists(os.path.join(ORACLE, "liboracle.so")):
        subprocess.run(["make", "-s", "-C", ORACLE], check=True)
    if not os.path.exists(os.path.join(PKG, "libmoert.so")):
        subprocess.run(["make", "-s", "-j4", "-C", PKG], check=True)


@pytest.fixture(scope="session")
def gpu():
    """The device; GPU tests are skipped without one unless MOERT_REQUIRE_GPU=1 (then they fail)."""
    import moert
    n, name = moert.device_info()
    if n == 0:
        if os.environ.get("MOERT_REQUIRE_GPU") == "1":
            pytest.fail("MOERT_REQUIRE_GPU=1 and no GPU visible")
        pytest.skip("no GPU visible")
    print(f"\n[gpu] {name}", flush=True)
    return name


@pytest.fixture(scope="session")
def granite_3b_q4():
    """The expert-cache workload's model: 3B-A800M shape, Q4_0 weights and head, Zipf(1.1) router bias."""
    import moert
    cfg = moert.Config(**moert.GRANITE_3B)
    print("[case] 3b q4_0 build", flush=True)
    m = moert.SynthModel(cfg, seed=4242, wdtype=moert.Q4_0, embed_dtype=moert.Q4_0, zipf_s=1.1)
    return cfg, m
