"""CPU tests of the promotion timing's C launch loops (radeon-kernels_amd/promotion/launch_loop.c).

Each loop must call its entry point exactly n times, walk the cache copies round-robin from ``first``,
pass every other argument through unchanged, and stop at the first non-zero status.  A ctypes callback
stands in for the GPU entry point, so nothing here touches a device.
"""

from __future__ import annotations

import ctypes
import importlib.util
from pathlib import Path

import pytest

PACKAGE = Path(__file__).resolve().parents[1] / "radeon-kernels_amd"


@pytest.fixture(scope="module")
def loops():
    spec = importlib.util.spec_from_file_location("rk_evaluate_under_test", PACKAGE / "promotion" / "evaluate.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    if not module.LaunchLoops.PATH.is_file():
        pytest.fail(f"{module.LaunchLoops.PATH} is not built; run __graft_entry__.build()")
    return module.LaunchLoops()


def test_append_loop_rotates_copies_and_passes_arguments(loops):
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    seen = []
    proto = ctypes.CFUNCTYPE(ctypes.c_int, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int, vp)

    def fake(key, value, kc, vc, slots, tokens, hkv, d, nb, bs, dtype, index, stream):
        seen.append((key, value, kc, vc, slots, tokens, hkv, d, nb, bs, dtype, index, stream))
        return 0

    callback = proto(fake)
    kc = (vp * 3)(0x1000, 0x2000, 0x3000)
    vc = (vp * 3)(0x1100, 0x2100, 0x3100)
    status = loops.lib.loop_append(ctypes.cast(callback, vp).value, 5, 2, 3, 0x10, 0x20, kc, vc, 0x30, 7, 8, 128,
                                   256, 16, 1, 0, 0x40)
    assert status == 0 and len(seen) == 5
    assert [s[2] for s in seen] == [0x3000, 0x1000, 0x2000, 0x3000, 0x1000]
    assert [s[3] for s in seen] == [0x3100, 0x1100, 0x2100, 0x3100, 0x1100]
    assert all(s[:2] == (0x10, 0x20) and s[4:] == (0x30, 7, 8, 128, 256, 16, 1, 0, 0x40) for s in seen)


def test_decode_loop_picks_the_form_by_counters_and_stops_at_an_error(loops):
    vp, i64, sz, ci, cf = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
    calls = []
    two = ctypes.CFUNCTYPE(ci, vp, vp, vp, vp, vp, vp, vp, sz, i64, i64, i64, i64, i64, i64, i64, cf, ci, ci, i64, ci,
                           vp)
    fused = ctypes.CFUNCTYPE(ci, vp, vp, vp, vp, vp, vp, vp, sz, vp, sz, i64, i64, i64, i64, i64, i64, i64, cf, ci, ci,
                             i64, ci, vp)

    def fake_two(q, k, v, bt, cl, out, ws, wsb, b, hq, hkv, d, nb, bs, mb, scale, dt, it, p, var, stream):
        calls.append(("two", k, v, wsb, b, hq, hkv, d, nb, bs, mb, round(scale, 6), dt, it, p, var, stream))
        return 0 if len(calls) < 3 else 3

    def fake_fused(q, k, v, bt, cl, out, ws, wsb, counters, words, b, hq, hkv, d, nb, bs, mb, scale, dt, it, p, var,
                   stream):
        calls.append(("fused", k, counters, words, b, p))
        return 0

    cb_two, cb_fused = two(fake_two), fused(fake_fused)
    kc = (vp * 2)(0xA000, 0xB000)
    vc = (vp * 2)(0xA100, 0xB100)
    args = (0x1, kc, vc, 0x2, 0x3, 0x4, 0x5, 4096)
    shape = (8, 32, 8, 128, 1024, 16, 64, 0.125, 1, 0, 256, 0, 0x9)
    status = loops.lib.loop_decode(ctypes.cast(cb_two, vp).value, 10, 1, 2, *args, None, 0, *shape)
    assert status == 3 and len(calls) == 3  # stopped at the first failing call
    assert [c[1] for c in calls] == [0xB000, 0xA000, 0xB000]
    assert calls[0][3:] == (4096, 8, 32, 8, 128, 1024, 16, 64, 0.125, 1, 0, 256, 0, 0x9)
    calls.clear()
    status = loops.lib.loop_decode(ctypes.cast(cb_fused, vp).value, 2, 0, 2, *args, 0x77, 64, *shape)
    assert status == 0 and calls == [("fused", 0xA000, 0x77, 64, 8, 256), ("fused", 0xB000, 0x77, 64, 8, 256)]
