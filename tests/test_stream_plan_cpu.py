"""CPU checks of the weight-streaming decode kernel's launch plans
(``w8_stream_plan``, ``l16_stream_plan`` and ``gu16_stream_plan`` in
csrc/w8a16_stream.h, reached
through the probe library's plan exports; no GPU call): every plan the
launchers can produce (1 - 64 rows; 48 for the dual kernel) must be one
the launcher accepts -- at most the kernel's thread limit (16 waves, 8 where its registers need
more room) and no more waves than 256-byte chunks, rows per workgroup
within its 4-row sets, and for more than 8 rows of x one chunk in flight
(the instantiations the launcher has) -- and fit the kernel's LDS."""
import ctypes
import importlib.util
import itertools
from pathlib import Path

import pytest

PROBE = Path(__file__).resolve().parents[1] / "llm-inference-optimizer_amd" / "libmi355_probe.so"


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_for_plans", PROBE.parents[1] / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def probe():
    if not PROBE.exists():
        pytest.skip("probe library not built")
    lib = ctypes.CDLL(str(PROBE))
    i32 = ctypes.c_int
    lib.mi355_probe_w8a16_stream_plan.argtypes = [i32, i32, i32, i32, i32, ctypes.POINTER(i32)]
    lib.mi355_probe_gate_up16_stream_plan.argtypes = [i32, i32, i32, i32, ctypes.POINTER(i32)]
    lib.mi355_probe_stream_max_threads.argtypes = [i32] * 5
    lib.mi355_probe_linear16_stream_plan.argtypes = [i32, i32, i32, i32, ctypes.POINTER(i32)]
    return lib


def _check(plan, rows, kbytes, nq, lib, wb=1):
    rpw, r4, waves, u = plan
    nchunk = -(-kbytes // 256)
    assert r4 in (1, 2, 4) and 1 <= rpw <= 4 * r4, plan
    assert 1 <= waves <= 16 and waves <= max(1, nchunk), (plan, nchunk)
    assert u in (1, 2), plan
    mt4 = -(-rows // 4) if rows <= 16 else (6 if rows <= 24 else (8 if rows <= 32 else (12 if rows <= 48 else 16)))
    if mt4 > 2:  # one chunk in flight with three or more x sets
        assert u == 1, (rows, plan)
    assert 64 * waves <= lib.mi355_probe_stream_max_threads(r4, mt4, u, nq - 1, wb), (rows, plan)
    assert waves * nq * r4 * mt4 * 16 * 4 <= 64 * 1024


KS = (16, 48, 256, 272, 896, 1536, 2048, 2056, 3584, 4864, 8960, 18944, 29568)
NS = (1, 7, 37, 256, 896, 1000, 1536, 2048, 3584, 4864, 8960, 18944, 29568, 65536)


@pytest.mark.parametrize("cus", [80, 256, 304])
def test_w8a16_plan_is_launchable(probe, cus):
    out = (ctypes.c_int * 4)()
    for rows, k, n, dual in itertools.product(range(1, 49), KS, NS, (0, 1)):
        if dual and rows > 48:  # the dual kernel serves up to 48 rows
            continue
        probe.mi355_probe_w8a16_stream_plan(rows, k, n, dual, cus, out)
        _check(tuple(out), rows, k, 2 if dual else 1, probe)


@pytest.mark.parametrize("cus", [80, 256, 304])
def test_linear16_plan_is_launchable(probe, cus):
    out = (ctypes.c_int * 4)()
    for rows, k, n in itertools.product(range(1, 65), (8, 24, 136, 896, 1536, 2056, 3584, 8960, 18944), NS):
        probe.mi355_probe_linear16_stream_plan(rows, k, n, cus, out)
        _check(tuple(out), rows, 2 * k, 1, probe, wb=2)


@pytest.mark.parametrize("cus", [80, 256, 304])
def test_gate_up16_plan_is_launchable(probe, cus):
    out = (ctypes.c_int * 4)()
    for rows, k, n in itertools.product(range(1, 33), (8, 24, 136, 896, 1536, 2048, 2056, 3584, 8192), NS):
        probe.mi355_probe_gate_up16_stream_plan(rows, k, n, cus, out)
        _check(tuple(out), rows, 2 * k, 2, probe, wb=2)


def test_thread_limit_matches_the_bench_sweep(probe, bench):
    """bench.py's sweep samples only launch shapes the kernel takes: its
    stream_max_waves is the kernel's own thread limit / 64, and the limit
    drops to 512 exactly where the register estimate reaches 112."""
    for r4, mt4, u, dual, wb in itertools.product((1, 2, 4), (1, 2, 3, 4, 6, 8, 12, 16), (1, 2), (0, 1), (1, 2)):
        lim = probe.mi355_probe_stream_max_threads(r4, mt4, u, dual, wb)
        assert lim in (0, 512, 1024)
        if mt4 <= 4 and u == 1:  # every shape up to 16 rows with one chunk in flight has a kernel
            assert lim > 0, (r4, mt4, dual, wb)
        assert bench.stream_max_waves(r4, mt4, u, bool(dual), wb) == lim // 64, (r4, mt4, u, dual, wb)
    # the shapes that spilled under 128 VGPRs take 512 threads; those in use
    # without spills keep 1024
    assert probe.mi355_probe_stream_max_threads(4, 4, 1, 0, 1) == 512
    assert probe.mi355_probe_stream_max_threads(2, 4, 1, 1, 1) == 512
    assert probe.mi355_probe_stream_max_threads(4, 2, 1, 1, 1) == 512
    assert probe.mi355_probe_stream_max_threads(4, 3, 1, 0, 1) == 1024
    assert probe.mi355_probe_stream_max_threads(4, 2, 1, 1, 2) == 1024
    assert probe.mi355_probe_stream_max_threads(2, 4, 1, 1, 2) == 1024
    # 33 - 64 rows of one matrix: two weight sets with 16-bit weights at 16 x
    # sets, with int8 weights at 12 (not 16), one at 16
    assert probe.mi355_probe_stream_max_threads(2, 16, 1, 0, 2) == 512
    assert probe.mi355_probe_stream_max_threads(2, 12, 1, 0, 1) == 512
    assert probe.mi355_probe_stream_max_threads(2, 16, 1, 0, 1) == 0
    assert probe.mi355_probe_stream_max_threads(1, 16, 1, 0, 1) == 512


def _plan(probe, fn, *args):
    out = (ctypes.c_int * 4)()
    fn(*args, out)
    return tuple(out)


def test_plans_picked_by_the_deep_row_sweep(probe):
    """The launch plans the 1 - 4 row sweep over the Qwen2.5-7B projections
    picked (256 CUs): 16-row workgroups from 2 rows of x on the deep rows
    (k >= 3072 bytes) of outputs that are not narrow -- from 4 rows with
    16-bit weights, and at k < 8192 only where every CU gets a 16-row
    workgroup --, the dual kernel on 8-row workgroups of 8 waves at 2 - 4
    rows; with one row of x the earlier 8-row (dual: 4-row) plans but where
    every CU gets a 16-row workgroup of one int8 matrix."""
    w8 = probe.mi355_probe_w8a16_stream_plan
    l16 = probe.mi355_probe_linear16_stream_plan
    for rows in (2, 3, 4):
        assert _plan(probe, w8, rows, 3584, 18944, 0, 256) == (15, 4, 2, 1), rows   # 7B gate/up
        assert _plan(probe, w8, rows, 18944, 3584, 0, 256) == (14, 4, 8, 1), rows   # 7B down
        assert _plan(probe, w8, rows, 3584, 18944, 1, 256) == (8, 2, 8, 1), rows    # 7B dual gate/up
        assert _plan(probe, w8, rows, 1536, 8960, 0, 256)[0] == 8, rows             # 1.5B gate/up: k < 3072
        assert _plan(probe, w8, rows, 8960, 1536, 0, 256)[0] <= 8, rows             # narrow: every CU a workgroup
        assert _plan(probe, w8, rows, 3584, 3584, 0, 256) == (8, 2, 8, 1), rows     # 7B q/o: 224 16-row groups
    assert _plan(probe, w8, 1, 3584, 18944, 0, 256) == (15, 4, 2, 1)   # every CU a 16-row workgroup
    assert _plan(probe, w8, 1, 3584, 3584, 0, 256)[0] == 8
    assert _plan(probe, w8, 1, 18944, 3584, 0, 256) == (8, 2, 8, 1)
    assert _plan(probe, w8, 1, 3584, 18944, 1, 256)[:3] == (4, 1, 8)   # one row, k >= 2048: 8 waves
    assert _plan(probe, w8, 1, 1536, 8960, 1, 256)[:3] == (4, 1, 3)
    assert _plan(probe, w8, 4, 13824, 5120, 0, 256) == (10, 4, 6, 1)  # 14B down: 12 waves per CU
    assert _plan(probe, w8, 1, 13824, 5120, 0, 256)[0] == 8           # one row: under 4 per CU
    assert _plan(probe, w8, 8, 3584, 18944, 1, 256) == (15, 4, 1, 1)
    assert _plan(probe, l16, 4, 18944, 3584, 256)[:3] == (14, 4, 8)
    assert _plan(probe, l16, 3, 18944, 3584, 256)[0] == 8


def test_dual_plans_by_workgroups_per_cu(probe):
    """The gate/up + SiLU-and-mul plans the sweep by workgroups per CU
    picked (256 CUs): with more than 4 (int8) or 8 (16-bit) rows of x, 4-row
    workgroups of 2 waves where 8-row ones would number under 4 per CU (the
    0.5B MLP, k 896 x n 4864), 8-row ones of 2 waves where they do not (1.5B,
    k 1536 x n 8960; int8 3B, k 2048 x n 11008), of one wave beyond 16 rows
    of x; 16-bit weights from k = 2048 on workgroups of the 16-row class
    (balanced over the CUs: 15 rows) of about 5 waves per CU (3B: 2, 7B: 1)."""
    w8 = probe.mi355_probe_w8a16_stream_plan
    gu = probe.mi355_probe_gate_up16_stream_plan
    for rows in (6, 8, 12, 16, 24, 32):
        assert _plan(probe, w8, rows, 896, 4864, 1, 256)[:3] == (4, 1, 2), rows
        assert _plan(probe, w8, rows, 1536, 8960, 1, 256)[:3] == (8, 2, 2 if rows <= 16 else 1), rows
    assert _plan(probe, w8, 16, 2048, 11008, 1, 256)[:3] == (8, 2, 2)
    assert _plan(probe, w8, 24, 2048, 11008, 1, 256)[:3] == (8, 2, 1)  # 6 or 8 x sets: one wave
    for rows in (10, 12, 16):
        assert _plan(probe, gu, rows, 896, 4864, 256) == (4, 1, 2, 1), rows
        assert _plan(probe, gu, rows, 1536, 8960, 256) == (8, 2, 2, 1), rows
        assert _plan(probe, gu, rows, 2048, 11008, 256) == (15, 4, 2, 1), rows   # balanced_rows16
        assert _plan(probe, gu, rows, 3584, 18944, 256) == (15, 4, 1, 1), rows
    assert _plan(probe, gu, 24, 896, 4864, 256) == (8, 2, 2, 1)
    # the int8 dual kernel's 16-row class: one wave with at least 4 workgroups
    # per CU (7B MLP), two with fewer (14B MLP)
    assert _plan(probe, w8, 8, 3584, 18944, 1, 256) == (15, 4, 1, 1)
    assert _plan(probe, w8, 12, 5120, 13824, 1, 256) == (14, 4, 2, 1)
    # 2 - 4 rows below k = 3072: half the chunks as waves, two in flight each
    assert _plan(probe, w8, 4, 896, 4864, 1, 256) == (4, 1, 2, 2)
    assert _plan(probe, w8, 2, 2048, 11008, 1, 256) == (4, 1, 4, 2)
    assert _plan(probe, w8, 1, 1536, 8960, 1, 256) == (4, 1, 3, 1)
    # the 16-bit kernel's 16-row class: about 6 waves per CU
    assert _plan(probe, gu, 12, 5120, 13824, 256) == (14, 4, 2, 1)


def test_wide_rows_from_k_2048_beyond_16_rows(probe):
    """Beyond 16 rows of x one int8 matrix takes the 16-row class from k =
    2048 (3B gate/up: 15 rows per workgroup, 2 waves), the 16-bit linear
    still from k = 3072 bytes."""
    w8 = probe.mi355_probe_w8a16_stream_plan
    for rows in (17, 24, 32):
        assert _plan(probe, w8, rows, 2048, 11008, 0, 256) == (15, 4, 2, 1), rows
    assert _plan(probe, w8, 16, 2048, 11008, 0, 256)[0] == 8
    assert _plan(probe, w8, 24, 896, 4864, 0, 256)[0] == 8
    assert _plan(probe, w8, 8, 3584, 3584, 0, 256)[0] == 14
