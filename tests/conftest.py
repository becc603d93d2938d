import pytest

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "neutron-star_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through the C ABI on cuda:0)")


# Defaults of ns_ctx_set_tuning's keys (include/ns_ffn.h).
TUNING_DEFAULTS = {"gemv_pf": -1, "gemv_waves": 0, "gemv_whole": 1, "gemv_qslab": 1, "gemm_kparts": 0,
                   "gemm_q4_reg": 1, "mt_mfma": 1, "mt_parts": 0, "mt_slabs": 0, "mt_spw": 0, "block_fused": 1,
                   "block_spin": 0, "gemm_rs": 1, "stack_fused": 1}


@pytest.fixture
def tune(ctx):
    """tune(key, value) overrides one kernel choice of the module's context for
    this test; every key it touched is back at its default afterwards."""
    touched = set()

    def set_(key, value):
        ctx.set_tuning(key, int(value))
        touched.add(key)

    yield set_
    for key in touched:
        ctx.set_tuning(key, TUNING_DEFAULTS[key])
