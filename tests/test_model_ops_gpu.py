"""GPU parity of the decoder-block steps exposed as public ops (add, swiglu,
causal_scale, embedding, split_heads / merge_heads, rope, argmax) through the
C ABI. Bars: permutations, gathers, add, causal_scale and argmax bit-exact;
swiglu within 4 ulp relative of the oracle (expf of the device library vs
the host libm); rope within 1e-6 * (|a| + |b|) per pair (cosf/sinf ulps)."""
import numpy as np
import pytest

from tests.conftest import bits

pytestmark = pytest.mark.gpu
SEED = 99


def up(ow, a, dtype=np.float32):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(a, dtype))


@pytest.mark.parametrize("n", [1, 3, 4, 1027, 1 << 20])
def test_add_bit_exact_and_in_place(ow, orc, n):
    a = orc.fill_normal(n, SEED, 0, 0, 1)
    b = orc.fill_normal(n, SEED, 1, 0, 1)
    da, db, out = up(ow, a), up(ow, b), ow.DeviceBuffer.empty(n)
    ow.ops.add(da, db, out, n)
    assert np.array_equal(bits(out.to_host()), bits(a + b))
    ow.ops.add(da, db, da, n)  # residual update in place
    assert np.array_equal(bits(da.to_host()), bits(a + b))


@pytest.mark.parametrize("n", [1, 5, 8192, 3 * 8192 + 3])
@pytest.mark.parametrize("offset", [0, 1])
def test_swiglu_matches_oracle(ow, orc, n, offset):
    g = orc.fill_normal(n + offset, SEED, 2, 0, 4)
    u = orc.fill_normal(n + offset, SEED, 3, 0, 1)
    dg, du, out = up(ow, g), up(ow, u), ow.DeviceBuffer.empty(n + offset)
    ow.ops.swiglu(dg.offset(offset), du.offset(offset), out.offset(offset), n)
    got = out.to_host()[offset:].astype(np.float64)
    want = orc.swiglu(g[offset:], u[offset:]).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-37)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 3), (5, 9), (7, 16), (32, 32), (64, 600), (512, 767)])
def test_causal_scale_bit_exact(ow, orc, rows, cols):
    x = orc.fill_normal(rows * cols, SEED, 4, 0, 3)
    d = up(ow, x)
    ow.ops.causal_scale(d, rows, cols, 0.125)
    assert np.array_equal(bits(d.to_host()), bits(orc.causal_scale(x, rows, cols, 0.125)))


@pytest.mark.parametrize("hidden", [4, 6, 2048])
@pytest.mark.parametrize("as_bf16", [False, True])
def test_embedding_gather_exact(ow, orc, hidden, as_bf16):
    vocab, n = 97, 33
    table = orc.fill_normal(vocab * hidden, SEED, 5, 0, 1)
    ids = np.random.default_rng(1).integers(0, vocab, n).astype(np.int32)
    ids[5] = vocab - 1
    ids[6] = 0
    if as_bf16:
        tb, tbits = orc.round_bf16(table)
        dt = up(ow, tbits, np.uint16)
        want = tb.reshape(vocab, hidden)[ids]
    else:
        dt = up(ow, table)
        want = table.reshape(vocab, hidden)[ids]
    di = up(ow, ids, np.int32)
    out = ow.DeviceBuffer.empty(n * hidden)
    ow.ops.embedding(dt, vocab, di, out, n, hidden, bf16=as_bf16)
    assert np.array_equal(bits(out.to_host().reshape(n, hidden)), bits(want))


def test_embedding_out_of_range_id_is_nan_row(ow, orc):
    vocab, hidden = 10, 8
    table = orc.fill_normal(vocab * hidden, SEED, 6, 0, 1)
    ids = np.array([3, 10, -1, 9], np.int32)
    dt, di, out = up(ow, table), up(ow, ids, np.int32), ow.DeviceBuffer.empty(4 * hidden)
    ow.ops.embedding(dt, vocab, di, out, 4, hidden)
    got = out.to_host().reshape(4, hidden)
    t = table.reshape(vocab, hidden)
    assert np.array_equal(got[0], t[3]) and np.array_equal(got[3], t[9])
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))


@pytest.mark.parametrize("rows,heads,D,stride,off", [(1, 1, 4, 1, 0), (7, 8, 64, 20, 5), (512, 32, 64, 512, 0),
                                                     (3, 2, 6, 9, 6), (1, 8, 64, 2048, 2047)])
def test_split_merge_heads_exact(ow, orc, rows, heads, D, stride, off):
    x = orc.fill_normal(rows * heads * D, SEED, 7, 0, 1)
    slab = np.full(heads * stride * D, 7.0, np.float32)
    dx, ds = up(ow, x), up(ow, slab)
    ow.ops.split_heads(dx, ds, rows, heads, D, stride, off)
    want = slab.reshape(heads, stride, D).copy()
    want[:, off:off + rows, :] = x.reshape(rows, heads, D).transpose(1, 0, 2)
    assert np.array_equal(bits(ds.to_host().reshape(heads, stride, D)), bits(want))
    back = ow.DeviceBuffer.empty(rows * heads * D)
    ow.ops.merge_heads(ds, back, rows, heads, D, stride, off)
    assert np.array_equal(bits(back.to_host()), bits(x))


@pytest.mark.parametrize("rows,heads,D,pos", [(1, 1, 2, 0), (5, 4, 64, 0), (3, 8, 64, 767), (512, 32, 64, 0),
                                              (2, 2, 32, 8190)])
def test_rope_matches_oracle(ow, orc, rows, heads, D, pos):
    inv = orc.rope_inv_freq(D, 500000.0, True, 32.0, 1.0, 4.0, 8192)
    x = orc.fill_normal(rows * heads * D, SEED, 8, 0, 1)
    dx, di = up(ow, x), up(ow, inv)
    ow.ops.rope(dx, di, rows, heads, D, pos)
    got = dx.to_host().reshape(rows, heads, 2, D // 2).astype(np.float64)
    want = orc.rope(x, inv, rows, heads, D, pos).reshape(rows, heads, 2, D // 2).astype(np.float64)
    src = x.reshape(rows, heads, 2, D // 2).astype(np.float64)
    scale = np.abs(src[:, :, 0]) + np.abs(src[:, :, 1])
    assert np.all(np.abs(got[:, :, 0] - want[:, :, 0]) <= 1e-6 * scale + 1e-30)
    assert np.all(np.abs(got[:, :, 1] - want[:, :, 1]) <= 1e-6 * scale + 1e-30)
    if pos == 0:  # position 0 is the identity on row 0
        assert np.array_equal(got[0], src[0])


ARGMAX_CASES = {
    "random": lambda n, r: r.normal(size=n),
    "ties": lambda n, r: np.where(np.arange(n) % 7 == 3, 5.0, 1.0),
    "neg_inf": lambda n, r: np.full(n, -np.inf),
    "nan_mix": lambda n, r: np.where(np.arange(n) % 3 == 0, np.nan, r.normal(size=n)),
    "all_nan": lambda n, r: np.full(n, np.nan),
}


@pytest.mark.parametrize("case", sorted(ARGMAX_CASES))
@pytest.mark.parametrize("n", [1, 5, 4099, 128256])
@pytest.mark.parametrize("offset", [0, 1])
def test_argmax_rules(ow, orc, case, n, offset):
    x = ARGMAX_CASES[case](n + offset, np.random.default_rng(n)).astype(np.float32)
    if case == "random" and n > 10:
        x[offset + n // 2] = x.max() + 1  # one clear winner in the middle
    d, out = up(ow, x), ow.DeviceBuffer.empty(1, np.int32)
    ow.ops.argmax(d.offset(offset), n, out)
    assert int(out.to_host()[0]) == orc.argmax(x[offset:])
