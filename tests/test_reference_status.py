"""The reference's status expectations that need no device, through the C ABI
on the CPU: context options refused before any device call, and plan
validation (rns8_create_plan's checks, backend routing and schedule, run by
rns8_mi355x_plan_schedule without a context). Every other case of
tests/golden/reference_status_kats.json runs in test_gpu_reference_status.py.
"""
import pytest

import status_kats as sk

CASES = [c for c in sk.KATS["cases"] if sk.device_free(c)]


def test_fixture_covers_every_reference_check():
    """66 single-call cases (47 from test_semantics_validation_cases.inc, 19
    from test_api_validation_cases.inc, the wrap64 ones as context refusals)
    plus the two persistent finite sequences."""
    refs = [c["ref"] for c in sk.KATS["cases"]]
    assert len(refs) == len(set(refs)) == 66
    assert sum(r.startswith("test_semantics") for r in refs) == 47
    assert len(sk.KATS["sequences"]) == 2
    assert len(CASES) == 19


@pytest.mark.parametrize("case", CASES, ids=[c["ref"] for c in CASES])
def test_device_free_status(case):
    assert sk.run_device_free(case) == sk.STATUS[case["expect"]], case["ref"]
