"""The rate probes bench.py reports beside its rooflines (rns8_amd/probe).

They are measurement infrastructure, not product: these checks only pin their
contracts (status codes, positive rates below physical limits) so a broken
probe cannot silently report nonsense as `roofline.attainable` or
`stage_streams.*.attainable`.
"""
import ctypes as C
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent.parent / "rns8_amd" / "probe" / "librns8_probe.so"
HIP_INVALID_VALUE = 1


@pytest.fixture(scope="module")
def probe(gpu_ctx):
    lib = C.CDLL(str(LIB))
    lib.rns8_probe_mfma_rate.restype = C.c_int
    lib.rns8_probe_mfma_rate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double),
                                         C.POINTER(C.c_double)]
    lib.rns8_probe_hbm_stream.restype = C.c_int
    lib.rns8_probe_hbm_stream.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.POINTER(C.c_double)]
    return lib


def test_mfma_rate(probe):
    tops, ghz = C.c_double(), C.c_double()
    assert probe.rns8_probe_mfma_rate(1, 200, 1, 3, C.byref(tops), C.byref(ghz)) == 0
    # dense int8 peak is 5.0 POP/s at 2.4 GHz
    assert 100.0 < tops.value < 5000.0 * 1.02
    assert 0.5 < ghz.value < 2.6
    assert probe.rns8_probe_mfma_rate(1, 0, 1, 3, C.byref(tops), C.byref(ghz)) == HIP_INVALID_VALUE


@pytest.mark.parametrize("read,write", [(16 << 20, 0), (0, 16 << 20), (16 << 20, 16 << 20), (48, 16),
                                        (1 << 20, 9 << 20)])
def test_hbm_stream(probe, read, write):
    gbps = C.c_double()
    assert probe.rns8_probe_hbm_stream(read, write, 1, 3, C.byref(gbps)) == 0
    # small streams may sit in the 256 MB Infinity Cache, so allow more than
    # the 8 TB/s of HBM, but not an impossible rate
    assert 0.0 < gbps.value < 30000.0


@pytest.mark.parametrize("read,write", [(0, 0), (17, 0), (0, 8), (16, 16 << 20 | 4)])
def test_hbm_stream_rejects(probe, read, write):
    gbps = C.c_double(-1.0)
    assert probe.rns8_probe_hbm_stream(read, write, 1, 3, C.byref(gbps)) == HIP_INVALID_VALUE
    assert gbps.value == -1.0
