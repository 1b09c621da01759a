"""GPU: the one-pass scan's bounded wait giving up, forced from the host so every kernel exits
normally (opworks_amd/csrc/tests/probe_scan_timeout.hip). The only workgroup takes unit 1 of a
two-unit scan whose unit 0 never runs, so the wait for unit 0's total gives up after a few polls:
the unit's outputs must all be NaN, for the prefix maximum as well as the sum (fmaxf would drop
a NaN carry and leave a finite, too-small prefix), the timeout must be counted in workspace
word 1, and unit 0's outputs must stay untouched."""
import ctypes
from ctypes import c_int, c_void_p
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent
UNIT = 16384


@pytest.fixture(scope="module")
def probe(ow):
    lib = ctypes.CDLL(str(ROOT / "opworks_amd" / "lib" / "tests" / "libprobe_scan_timeout.so"))
    lib.probe_scan_unit_timeout.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]
    lib.probe_scan_unit_timeout.restype = c_int
    lib.probe_scan_workspace_words.argtypes = [c_int]
    lib.probe_scan_workspace_words.restype = c_int
    return lib


@pytest.mark.parametrize("maximum", [0, 1])
@pytest.mark.parametrize("n", [UNIT + 5, 2 * UNIT])
def test_scan_wait_timeout_poisons_the_unit(ow, orc, probe, maximum, n):
    x = orc.fill_normal(n, 4242, 3, 0.0, 1.0)
    d_in = ow.DeviceBuffer.from_host(x)
    sentinel = np.float32(123.5)
    d_out = ow.DeviceBuffer.from_host(np.full(n, sentinel, np.float32))
    words = probe.probe_scan_workspace_words(n)
    ws = ow.DeviceBuffer.empty(words, np.uint32)
    print(f"[scan timeout] n={n} maximum={maximum}", flush=True)
    assert probe.probe_scan_unit_timeout(d_in.ptr, d_out.ptr, ws.ptr, n, maximum, 64, None) == 0
    out = d_out.to_host()
    assert np.all(out[:UNIT] == sentinel), "unit 0 never ran, so its outputs stay untouched"
    assert np.all(np.isnan(out[UNIT:])), f"{int(np.sum(~np.isnan(out[UNIT:])))} finite outputs after a timeout"
    header = ws.to_host()[:2]
    assert header[0] == 2 and header[1] >= 1, header


def test_scan_probe_rejects_other_sizes(probe):
    assert probe.probe_scan_unit_timeout(None, None, None, UNIT, 0, 64, None) == -1
    assert probe.probe_scan_unit_timeout(None, None, None, 2 * UNIT + 1, 0, 64, None) == -1
