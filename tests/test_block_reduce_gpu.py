"""GPU parity of the public workgroup reductions block_reduce<Op> and
block_reduce_all<Op>, called from a user kernel (opworks_amd/csrc/tests/
probe_block_reduce.hip) at workgroup sizes that are multiples of 32 — the
reference's contract (include/core/block_reduce.cuh:9-41, README.md:228-229) —
including odd multiples (32, 96, 160, 992), whose last wave has 32 lanes.

Each workgroup reduces its own slice; the oracle is orc_block_reduce, the
reference's 32-lane shuffle tree restated. Bars: Max bit-exact on any data;
Product bit-exact on values that are powers of two (every partial product is
exact, so any order gives the same bits); Sum within 1e-5 * sum|x| on random
data, and bit-exact on small integers (exact in any order)."""
import ctypes

import numpy as np
import pytest

from tests.conftest import ROOT

pytestmark = pytest.mark.gpu

SEED = 2468
OPS = {"sum": 0, "max": 1, "product": 2}
SIZES = [32, 64, 96, 160, 256, 992, 1024]
BLOCKS = 7


@pytest.fixture(scope="module")
def probe(ow):
    path = ROOT / "opworks_amd" / "lib" / "tests" / "libprobe_block_reduce.so"
    assert path.exists(), "build the test libraries first (python -m opworks_amd.build tests)"
    lib = ctypes.CDLL(str(path))
    fn = lib.probe_block_reduce
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    fn.restype = ctypes.c_int
    return fn


def run(ow, probe, values, nthreads, op, mode):
    d_in = ow.DeviceBuffer.from_host(np.ascontiguousarray(values, np.float32))
    out = ow.DeviceBuffer.empty(values.size)
    print(f"[block_reduce] nthreads={nthreads} op={op} mode={mode}", flush=True)
    assert probe(d_in.ptr, out.ptr, nthreads, values.size // nthreads, OPS[op], mode) == 0
    got = out.to_host()
    if mode == 0:
        return got[: values.size // nthreads]
    return got.reshape(-1, nthreads)


def inputs(orc, op, n, kind):
    if op == "product":
        # powers of two with random signs: exact products of at most 2^+-16 per workgroup
        rng = np.random.default_rng(SEED + n)
        exps = rng.integers(-1, 2, n)
        exps[rng.random(n) < 0.9] = 0  # mostly +-1 so the product stays in range
        return (np.ldexp(1.0, exps) * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    if kind == "integers":
        return np.random.default_rng(SEED + n).integers(-50, 51, n).astype(np.float32)
    return orc.fill_normal(n, SEED, n, 0.0, 1.0)


@pytest.mark.parametrize("nthreads", SIZES)
@pytest.mark.parametrize("op", ["sum", "max", "product"])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_block_reduce_user_kernel(ow, orc, probe, nthreads, op, mode):
    kinds = ["random", "integers"] if op == "sum" else ["random"]
    for kind in kinds:
        vals = inputs(orc, op, nthreads * BLOCKS, kind)
        got = run(ow, probe, vals, nthreads, op, mode)
        for b in range(BLOCKS):
            sl = vals[b * nthreads:(b + 1) * nthreads]
            ref = np.float32(orc.block_reduce(sl, op))
            row = np.atleast_1d(got[b])  # mode 0: the workgroup's result; else every thread's copy
            if mode != 0:  # every thread of the workgroup sees the same value
                assert np.all(row.view(np.uint32) == row[0].view(np.uint32)), (b, row[:4])
            v = np.float32(row[0])
            if op == "sum" and kind == "random":
                assert abs(float(v) - float(ref)) <= 1e-5 * float(np.abs(sl.astype(np.float64)).sum()), (b, v, ref)
                assert abs(float(v) - float(sl.astype(np.float64).sum())) <= 1e-5 * float(np.abs(sl).sum())
            else:
                assert v.view(np.uint32) == ref.view(np.uint32), (op, kind, b, v, ref)


def test_block_reduce_identities_and_infinities(ow, orc, probe):
    """-inf everywhere gives Max's identity; a single +inf wins Max; NaN-free Product of all ones is 1."""
    n = 160
    vals = np.full(n, -np.inf, np.float32)
    assert run(ow, probe, vals, n, "max", 0)[0] == -np.inf
    vals[77] = np.inf
    assert run(ow, probe, vals, n, "max", 1)[0][0] == np.inf
    assert run(ow, probe, np.ones(n, np.float32), n, "product", 1)[0][0] == 1.0
    assert run(ow, probe, np.zeros(n, np.float32), n, "sum", 0)[0] == 0.0


def test_block_reduce_rejects_sizes_outside_the_contract(ow, probe):
    d = ow.DeviceBuffer.empty(64)
    for nthreads in (0, 16, 48, 1056):
        assert probe(d.ptr, d.ptr, nthreads, 1, 0, 0) == -1
