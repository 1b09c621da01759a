"""GPU parity of the kernels behind ScanBuilder, TransformBuilder and
GatherScatterBuilder (opw_scan_f32, opw_transpose_f32, opw_copy_f32,
opw_gather_f32, opw_scatter_f32) against the CPU oracle on seeded inputs.

The reference's builders carry only the operation metadata
(include/builders/scan.cuh:7-43, transform.cuh:7-38, gather_scatter.cuh:7-36);
the meaning checked here is the one oracle/oracle.h states.

Bars: prefix maximum, transpose, copy, gather and scatter bit-exact; prefix
sum |gpu - exact| <= 1e-5 * (running sum of |x|), the reduce bar applied to
every prefix, and bit-exact where every partial sum is an integer below 2^24
(ones, small integers)."""
import numpy as np
import pytest

from tests.conftest import bits

pytestmark = pytest.mark.gpu

SEED = 77


def upload(ow, arr, dtype=np.float32):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(arr, dtype), dtype=dtype)


def run_scan(ow, x, op, inclusive, offset=0, workspace=False):
    n = x.size
    dx = upload(ow, np.concatenate([np.zeros(offset, np.float32), x]))
    out = ow.DeviceBuffer.empty(n + offset)
    ws, ws_n = None, 0
    if workspace:
        ws_n = ow.ops.scan_workspace_size(n)
        ws = ow.DeviceBuffer.empty(max(ws_n, 1))
    ow.ops.scan(dx.offset(offset), out.offset(offset), n, op, inclusive, ws, ws_n)
    return out.to_host()[offset:]


SIZES = [1, 3, 4, 5, 63, 64, 255, 1023, 1024, 1025, 2049, 8191, 8192, 8193, 16_385, 100_003, 1 << 20,
         (1 << 22) + 5]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("inclusive", [True, False])
def test_scan_sum_matches_oracle(ow, orc, n, inclusive):
    x = orc.fill_normal(n, SEED, n % 97, 0.0, 1.0)
    got = run_scan(ow, x, "sum", inclusive)
    want, absp = orc.scan(x, maximum=False, inclusive=inclusive)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-5 * absp + 1e-30), float(np.max(err / (absp + 1e-30)))


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("inclusive", [True, False])
def test_scan_max_bit_exact(ow, orc, n, inclusive):
    x = orc.fill_normal(n, SEED + 1, n % 89, 0.0, 1.0)
    got = run_scan(ow, x, "maximum", inclusive)
    want, _ = orc.scan(x, maximum=True, inclusive=inclusive)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [7, 8193, 70_001])
@pytest.mark.parametrize("offset", [1, 2, 3])
def test_scan_unaligned_and_workspace_paths(ow, orc, n, offset):
    x = orc.fill_uniform(n, SEED + 2, offset, -1.0, 1.0)
    got = run_scan(ow, x, "sum", True, offset=offset)
    aligned = run_scan(ow, x, "sum", True)
    with_ws = run_scan(ow, x, "sum", True, workspace=True)
    want, absp = orc.scan(x)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * absp + 1e-30)
    # one geometry per n: the 16-byte and scalar paths, and both workspace forms, agree bit for bit
    assert np.array_equal(bits(got), bits(aligned)) and np.array_equal(bits(with_ws), bits(aligned))


def test_scan_known_answers_exact(ow):
    n = 5792  # every partial sum of 0..n-1 stays below 2^24, so any order is exact
    ints = np.arange(n, dtype=np.float32)
    tri = (np.arange(n, dtype=np.int64) * (np.arange(n) + 1) // 2).astype(np.float32)
    assert np.array_equal(run_scan(ow, ints, "sum", True), tri)
    assert np.array_equal(run_scan(ow, ints, "sum", False), np.concatenate([[0], tri[:-1]]).astype(np.float32))
    ones = np.ones(1 << 20, np.float32)
    assert np.array_equal(run_scan(ow, ones, "sum", True), np.arange(1, (1 << 20) + 1, dtype=np.float32))
    desc = np.arange(10_000, dtype=np.float32)[::-1].copy()
    assert np.array_equal(run_scan(ow, desc, "maximum", True), np.full(10_000, 9999, np.float32))
    mx_ex = run_scan(ow, desc, "maximum", False)
    assert mx_ex[0] == -np.inf and np.all(mx_ex[1:] == 9999)
    nan_first = np.array([np.nan, np.nan, 2.0, np.nan, 1.0], np.float32)
    assert np.array_equal(run_scan(ow, nan_first, "maximum", True), np.array([-np.inf, -np.inf, 2, 2, 2], np.float32))


def test_scan_in_place_and_deterministic(ow, orc):
    n = 300_007
    x = orc.fill_normal(n, SEED + 3, 0, 0.0, 1.0)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(n)
    ow.ops.scan(d, out, n)
    first = out.to_host()
    ow.ops.scan(d, out, n)
    assert np.array_equal(bits(out.to_host()), bits(first))
    ow.ops.scan(d, d, n)  # in place
    assert np.array_equal(bits(d.to_host()), bits(first))


TILE = 8192       # elements per scan tile
UNIT = 2 * TILE  # a unit of the one-pass protocol: a pair of tiles; 64 units make a group, 64 groups a super group


@pytest.mark.parametrize("n", [UNIT + TILE + 5, 2 * UNIT + TILE, 3 * UNIT - 1, 64 * UNIT, 64 * UNIT + 1,
                               65 * UNIT - 3, 4096 * UNIT, 4096 * UNIT + 1, (1 << 26) + 3 * 64 * UNIT + 100])
def test_scan_levels_and_stale_workspace_exact(ow, n):
    """The one-pass protocol at each level's edges (exactly one group or super group of units and
    one element past it), units whose second tile is partial or empty, and a second super group
    ending in a partial group and a partial unit, on a workspace whose every flag starts set:
    x[i] = (i mod 3) - 1 has prefix sums of -1 or 0 in any order, so every output is checked bit
    for bit, and a unit given a wrong or stale prefix shows up. Later calls reuse the earlier
    calls' workspace contents."""
    i = np.arange(n, dtype=np.int64)
    x = (i % 3 - 1).astype(np.float32)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(n)
    ws_n = ow.ops.scan_workspace_size(n)
    ws = upload(ow, np.full(ws_n, -1, np.int32), dtype=np.int32)
    for inclusive in (True, False, True):
        ow.ops.scan(d, out, n, "sum", inclusive, ws, ws_n)
        want = np.where((i + (1 if inclusive else 0)) % 3 == 0, 0.0, -1.0).astype(np.float32)
        assert np.array_equal(out.to_host(), want), inclusive
        assert ws.to_host()[1] == 0  # no wait timed out
    ow.ops.scan(d, out, n, "maximum", True, ws, ws_n)
    got = out.to_host()
    assert np.array_equal(got[:3], np.array([-1, 0, 1], np.float32)) and np.all(got[2:] == 1.0)


def test_scan_full_size_bound(ow, orc):
    """2^26 elements (4096 units, the multi-level path at scale) within the bar."""
    n = 1 << 26
    d = ow.DeviceBuffer.empty(n)
    ow.fill_normal(d, SEED, 9, 0.0, 1.0)
    out = ow.DeviceBuffer.empty(n)
    ow.ops.scan(d, out, n)
    x = orc.fill_normal(n, SEED, 9, 0.0, 1.0, mt=True)
    want, absp = orc.scan(x)
    got = out.to_host()
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * absp + 1e-30)


# ------------------------------------------------------------------ transform
@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (4, 4), (64, 64), (65, 129), (1000, 3), (128, 4096),
                                       (2048, 3000), (5, 70_000)])
@pytest.mark.parametrize("offset", [0, 1])
def test_transpose_bit_exact(ow, orc, rows, cols, offset):
    x = orc.fill_uniform(rows * cols + offset, SEED + 4, rows, -1.0, 1.0)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(rows * cols + offset)
    ow.ops.transpose(d.offset(offset), out.offset(offset), rows, cols)
    got = out.to_host()[offset:]
    assert np.array_equal(bits(got), bits(orc.transpose(x[offset:], rows, cols)))


def test_transpose_more_than_65535_tile_rows(ow):
    rows, cols = 8_388_736, 4  # 65537 tile rows of 128: the blockIdx.y loop
    x = np.arange(rows * cols, dtype=np.float32)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(rows * cols)
    ow.ops.transpose(d, out, rows, cols)
    assert np.array_equal(out.to_host().reshape(cols, rows), x.reshape(rows, cols).T)


@pytest.mark.parametrize("n", [1, 5, 4096, 100_003])
@pytest.mark.parametrize("offset", [0, 3])
def test_copy_bit_exact(ow, orc, n, offset):
    x = orc.fill_normal(n + offset, SEED + 5, n % 13, 0.0, 1.0)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(n + offset)
    ow.ops.copy(d.offset(offset), out.offset(offset), n)
    assert np.array_equal(bits(out.to_host()[offset:]), bits(x[offset:]))


# -------------------------------------------------------------- gather/scatter
@pytest.mark.parametrize("n,count", [(1, 1), (1000, 1000), (4097, 10_001), (1 << 20, 1 << 20)])
@pytest.mark.parametrize("offset", [0, 1])
def test_gather_bit_exact(ow, orc, n, count, offset):
    x = orc.fill_uniform(n, SEED + 6, n % 11, -1.0, 1.0)
    idx = np.random.default_rng(n + offset).integers(0, n, count).astype(np.int32)
    dx = upload(ow, x)
    di = upload(ow, np.concatenate([np.zeros(offset, np.int32), idx]), np.int32)
    out = ow.DeviceBuffer.empty(count + offset)
    ow.ops.gather(dx, n, di.offset(offset), out.offset(offset), count)
    assert np.array_equal(bits(out.to_host()[offset:]), bits(orc.gather(x, idx)))


def test_gather_out_of_range_is_nan(ow, orc):
    x = np.arange(10, dtype=np.float32)
    idx = np.array([0, -1, 9, 10, 2**31 - 1, -(2**31), 5, 3], np.int32)
    out = ow.DeviceBuffer.empty(idx.size)
    ow.ops.gather(upload(ow, x), 10, upload(ow, idx, np.int32), out, idx.size)
    got = out.to_host()
    want = orc.gather(x, idx)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(got[~np.isnan(want)],
                                                                               want[~np.isnan(want)])


@pytest.mark.parametrize("n", [1, 7, 4096, 100_003, 1 << 20])
@pytest.mark.parametrize("offset", [0, 1])
def test_scatter_permutation_bit_exact(ow, orc, n, offset):
    x = orc.fill_normal(n + offset, SEED + 7, n % 7, 0.0, 1.0)
    perm = np.random.default_rng(n).permutation(n).astype(np.int32)
    dx = upload(ow, x)
    di = upload(ow, np.concatenate([np.zeros(offset, np.int32), perm]), np.int32)
    out = upload(ow, np.full(n, -5.0, np.float32))
    ow.ops.scatter(dx.offset(offset), di.offset(offset), out, n, n)
    got = out.to_host()
    assert np.array_equal(bits(got), bits(orc.scatter(x[offset:], perm, np.full(n, -5.0, np.float32))))
    # gather through the same permutation undoes the scatter
    back = ow.DeviceBuffer.empty(n)
    ow.ops.gather(out, n, di.offset(offset), back, n)
    assert np.array_equal(bits(back.to_host()), bits(x[offset:]))


def test_scatter_skips_out_of_range(ow):
    x = np.array([1, 2, 3, 4, 5], np.float32)
    idx = np.array([4, -1, 7, 0, 2**31 - 1], np.int32)
    out = upload(ow, np.zeros(6, np.float32))
    ow.ops.scatter(upload(ow, x), upload(ow, idx, np.int32), out, 6, 5)
    assert np.array_equal(out.to_host(), np.array([4, 0, 0, 0, 1, 0], np.float32))


# ------------------------------------------------------------- maximum sizes
INT_MAX = 2**31 - 1
CHUNK = 1 << 27


@pytest.mark.slow
def test_scan_at_int_max_exact(ow):
    """n = INT_MAX (262144 tiles, 8 GiB each way): x[i] = (i mod 3) - 1, whose prefix sums are -1 or 0
    in any summation order, so every output is checked bit for bit; 8192 mod 3 != 0, so a tile
    given a neighbour's prefix shows up."""
    n = INT_MAX
    d = ow.DeviceBuffer.empty(n)
    for s in range(0, n, CHUNK):
        m = min(CHUNK, n - s)
        d.offset(s, m).copy_from_host((np.arange(s, s + m, dtype=np.int64) % 3 - 1).astype(np.float32))
    out = ow.DeviceBuffer.empty(n)
    for inclusive in (True, False):
        ow.ops.scan(d, out, n, "sum", inclusive)
        for s in range(0, n, CHUNK):
            m = min(CHUNK, n - s)
            i = np.arange(s, s + m, dtype=np.int64) + (1 if inclusive else 0)  # elements covered
            want = np.where(i % 3 == 0, 0.0, -1.0).astype(np.float32)
            got = out.offset(s, m).to_host()
            assert np.array_equal(got, want), (inclusive, s)
    ow.ops.scan(d, out, n, "maximum", True)
    got = out.offset(0, 4).to_host()
    assert np.array_equal(got, np.array([-1, 0, 1, 1], np.float32))
    assert np.all(out.offset(n - CHUNK, CHUNK).to_host() == 1.0)


@pytest.mark.slow
def test_transpose_at_int_max_elements(ow):
    """46341 x 46340 (2,147,441,940 elements, 8 GiB each way, ragged tiles on both sides); element
    values are their own index bits, so every output element names its source."""
    rows, cols = 46341, 46340
    n = rows * cols
    d = ow.DeviceBuffer.empty(n)
    for s in range(0, n, CHUNK):
        m = min(CHUNK, n - s)
        d.offset(s, m).copy_from_host(np.arange(s, s + m, dtype=np.uint32).view(np.float32))
    out = ow.DeviceBuffer.empty(n)
    ow.ops.transpose(d, out, rows, cols)
    # output row c holds in[:, c]; check whole output rows in chunks
    per = CHUNK // rows
    for c0 in range(0, cols, per):
        c1 = min(cols, c0 + per)
        got = out.offset(c0 * rows, (c1 - c0) * rows).to_host().view(np.uint32).reshape(c1 - c0, rows)
        want = (np.arange(rows, dtype=np.uint64)[None, :] * cols + np.arange(c0, c1, dtype=np.uint64)[:, None])
        assert np.array_equal(got, want.astype(np.uint32)), c0
