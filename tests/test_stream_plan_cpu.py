"""CPU checks of the weight-streaming decode kernel's launch plans
(``w8_stream_plan`` and ``gu16_stream_plan`` in csrc/w8a16_stream.h, reached
through the probe library's plan exports; no GPU call): every plan the
launchers can produce for 1 - 16 rows must be one the launcher accepts --
at most 16 waves and no more waves than 256-byte chunks, rows per workgroup
within its 4-row sets, and for more than 8 rows of x at most two weight sets
and one chunk in flight (the instantiations the launcher has) -- and fit
the kernel's LDS."""
import ctypes
import itertools
from pathlib import Path

import pytest

PROBE = Path(__file__).resolve().parents[1] / "llm-inference-optimizer_amd" / "libmi355_probe.so"


@pytest.fixture(scope="module")
def probe():
    if not PROBE.exists():
        pytest.skip("probe library not built")
    lib = ctypes.CDLL(str(PROBE))
    i32 = ctypes.c_int
    lib.mi355_probe_w8a16_stream_plan.argtypes = [i32, i32, i32, i32, i32, ctypes.POINTER(i32)]
    lib.mi355_probe_gate_up16_stream_plan.argtypes = [i32, i32, ctypes.POINTER(i32)]
    return lib


def _check(plan, rows, kbytes, nq):
    rpw, r4, waves, u = plan
    nchunk = -(-kbytes // 256)
    assert r4 in (1, 2, 4) and 1 <= rpw <= 4 * r4, plan
    assert 1 <= waves <= 16 and waves <= max(1, nchunk), (plan, nchunk)
    assert u in (1, 2), plan
    mt4 = -(-rows // 4)
    if mt4 > 2:  # 16-row workgroups only with three x sets against one int8 matrix
        assert (r4 <= 2 or (mt4 == 3 and nq == 1)) and u == 1, (rows, plan)
    assert waves * nq * r4 * mt4 * 16 * 4 <= 64 * 1024


KS = (16, 48, 256, 272, 896, 1536, 2048, 2056, 3584, 4864, 8960, 18944, 29568)
NS = (1, 7, 37, 256, 896, 1000, 1536, 2048, 3584, 4864, 8960, 18944, 29568, 65536)


@pytest.mark.parametrize("cus", [80, 256, 304])
def test_w8a16_plan_is_launchable(probe, cus):
    out = (ctypes.c_int * 4)()
    for rows, k, n, dual in itertools.product(range(1, 17), KS, NS, (0, 1)):
        probe.mi355_probe_w8a16_stream_plan(rows, k, n, dual, cus, out)
        _check(tuple(out), rows, k, 2 if dual else 1)


def test_gate_up16_plan_is_launchable(probe):
    out = (ctypes.c_int * 4)()
    for rows, k in itertools.product(range(1, 17), (8, 24, 136, 896, 1536, 2048, 2056, 3584, 8192)):
        probe.mi355_probe_gate_up16_stream_plan(rows, k, out)
        _check(tuple(out), rows, 2 * k, 2)
