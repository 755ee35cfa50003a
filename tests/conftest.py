import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (TESTS, os.path.join(ROOT, "ltx-rust_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_sessionfinish(session, exitstatus):
    """Write the per-call statistics of the LoRA tolerance check (max ulp
    distance, elements beyond 1 ulp, ill-conditioned elements, Frobenius
    errors) of a GPU session to the JSON file named by LTXW_PARITY_STATS,
    when that variable is set."""
    gu = sys.modules.get("gpu_util")
    path = os.environ.get("LTXW_PARITY_STATS")
    if gu is None or not getattr(gu, "STATS", None) or not path:
        return
    import json

    with open(path, "w") as f:
        json.dump(gu.STATS, f, indent=0)
