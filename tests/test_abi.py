"""The C-ABI libraries load and export every symbol include/*.h declares, and
contract violations come back as errors before any device work (no GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(opw_\w+|solve)\s*\(", re.M)


def declared(header: Path):
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(DECL.findall(text)))


def test_headers_declare_symbols():
    assert HEADERS, "no C headers under include/"
    for h in HEADERS:
        assert declared(h), h


def test_main_library_exports_every_declared_symbol(ow):
    lib = ow.lib()
    missing = []
    for h in HEADERS:
        if h.name.startswith("opworks_solve"):
            continue
        for name in declared(h):
            if not hasattr(lib, name):
                missing.append(f"{h.name}:{name}")
    assert not missing, missing


def test_adapters_export_solve():
    adapters = sorted((ROOT / "opworks_amd" / "lib" / "adapters").glob("libopw_solve_*.so"))
    hdr = ROOT / "include" / "opworks_solve.h"
    if not hdr.exists():
        pytest.skip("no adapters declared yet")
    names = re.findall(r"libopw_solve_(\w+)\.so", hdr.read_text())
    assert names
    built = {p.name for p in adapters}
    for n in names:
        assert f"libopw_solve_{n}.so" in built, n
        lib = ctypes.CDLL(str(ROOT / "opworks_amd" / "lib" / "adapters" / f"libopw_solve_{n}.so"))
        for sym in declared(hdr) + ["solve"]:
            assert hasattr(lib, sym), (n, sym)


# Contract checks mirror tests/unit/framework.cu:91-106; none reaches the device.
def test_contracts_reject_before_launch(ow):
    E = ow.OpworksError
    ops = ow.ops
    ops.map_scale_add(None, None, None, 0, 2.5)  # n == 0 is a no-op
    ops.softmax(None, None, 0, 3)
    ops.layer_norm(None, None, None, None, 0, 3)
    with pytest.raises(E, match="nonnegative"):
        ops.map_scale(None, None, -1, 2.0)
    with pytest.raises(E, match="non-null"):
        ops.map_scale(None, None, 1, 2.0)
    with pytest.raises(E, match="valid input/output"):
        ops.reduce(None, None, 0)
    with pytest.raises(E, match="positive columns"):
        ops.softmax(None, None, 1, 0)
    with pytest.raises(E, match="nonnegative"):
        ops.softmax(None, None, -1, 2)
    with pytest.raises(E, match="positive columns"):
        ops.layer_norm(None, None, None, None, 1, 0)
    with pytest.raises(E, match="epsilon"):
        ops.layer_norm(None, None, None, None, 0, 3, 0.0)
    with pytest.raises(E, match="epsilon"):
        ops.layer_norm(None, None, None, None, 0, 3, float("inf"))
    with pytest.raises(E, match="INT_MAX"):
        ops.softmax(None, None, 65536, 65536)
    with pytest.raises(E, match="epsilon"):
        ops.rms_norm(1, 1, 1, 1, 4, 0.0)
    with pytest.raises(E, match="unknown reduction"):
        ow.check(ow.lib().opw_reduce_f32(1, 1, 0, 9, None, 0, None))
    with pytest.raises(E, match="workspace is too small"):
        ow.check(ow.lib().opw_reduce_f32(1, 1, 1 << 20, 0, 1, 0, None))


def test_workspace_sizes(ow):
    assert ow.ops.reduction_workspace_size(0) == 0
    assert ow.ops.reduction_workspace_size(8192) == 0  # one chunk: single launch
    assert ow.ops.reduction_workspace_size(8193) == 2
    assert ow.ops.reduction_workspace_size(1 << 28) == (1 << 28) // 8192


def test_scan_transform_gather_contracts(ow):
    E = ow.OpworksError
    ops = ow.ops
    assert ops.scan_workspace_size(0) == 0
    assert ops.scan_workspace_size(16384) == 0  # one unit (a pair of 8192-element tiles): no workspace
    # a 64-word header, then 2 words per unit, per group of 64 units and per super group of 4096 units
    assert ops.scan_workspace_size(16385) == 64 + 2 * (2 + 1 + 1)
    assert ops.scan_workspace_size(1 << 28) == 64 + 2 * (16384 + 256 + 4)
    assert ops.scan_workspace_size(2**31 - 1) == 64 + 2 * (131072 + 2048 + 32)
    ops.scan(None, None, 0)  # n == 0 is a no-op
    ops.transpose(None, None, 0, 5)
    ops.gather(None, 0, None, None, 0)
    ops.scatter(None, None, None, 0, 0)
    with pytest.raises(E, match="unknown scan op"):
        ow.check(ow.lib().opw_scan_f32(1, 1, 4, 7, 1, None, 0, None))
    with pytest.raises(E, match="non-null"):
        ops.scan(None, None, 4)
    with pytest.raises(E, match="workspace is too small"):
        ops.scan(1, 1, 20000, workspace=1, workspace_size=1)
    with pytest.raises(E, match="16-byte aligned"):
        ops.scan(1, 1, 20000, workspace=4, workspace_size=ops.scan_workspace_size(20000))
    with pytest.raises(E, match="nonnegative"):
        ops.scan(None, None, -1)
    with pytest.raises(E, match="in place"):
        ops.transpose(16, 16, 4, 4)
    with pytest.raises(E, match="nonnegative"):
        ops.transpose(None, None, -1, 4)
    with pytest.raises(E, match="non-null"):
        ops.gather(None, 10, 16, 32, 4)
    with pytest.raises(E, match="nonnegative"):
        ops.scatter(16, 32, 48, -1, 4)
