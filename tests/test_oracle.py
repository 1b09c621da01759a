"""Pins the CPU oracle (no GPU): golden values and known-answer tests from the
reference's own unit tests, closed forms, invariants and independent numpy
restatements chosen so that a dropped term, a wrong index or a wrong order
fails. The oracle is the checker for every GPU parity test."""
import math

import numpy as np
import pytest

from tests.conftest import framework_close

# SplitMix64 published output for state 0 (Vigna's reference implementation):
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def py_mix64(z):
    m = (1 << 64) - 1
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_splitmix_known_answers():
    golden = 0x9E3779B97F4A7C15
    got = [py_mix64(((i + 1) * golden) & ((1 << 64) - 1)) for i in range(3)]
    assert got == SPLITMIX64_SEED0


def test_uniform_matches_independent_restatement(orc):
    n = 1000
    x = orc.fill_uniform(n, 1234, 7, -1.0, 1.0)
    key = orc.lib().orc_stream_key(1234, 7)
    golden = 0x9E3779B97F4A7C15
    m = (1 << 64) - 1
    want = np.empty(n, np.float32)
    for i in range(n):
        k = py_mix64((key + (i + 1) * golden) & m) >> 40
        # u * 2 + (-1) is exact in float32 for a 24-bit u, so fmaf == plain arithmetic here
        want[i] = np.float32(k * 2.0 ** -24 * 2.0 - 1.0)
    assert np.array_equal(x, want)
    assert x.min() >= -1.0 and x.max() < 1.0


def test_uniform_and_normal_moments(orc):
    n = 1 << 20
    u = orc.fill_uniform(n, 99, 0, -1.0, 1.0, mt=True)
    assert abs(u.mean()) < 3e-3 and abs(u.var() - 1 / 3) < 3e-3
    z = orc.fill_normal(n, 99, 1, 0.0, 1.0, mt=True)
    assert abs(z.mean()) < 3e-3 and abs(z.var() - 1.0) < 5e-3
    assert np.abs(z).max() <= 2 * math.sqrt(3) + 1e-6  # Irwin-Hall(4) support
    z2 = orc.fill_normal(n, 99, 1, 0.5, 0.02, mt=True)
    assert abs(z2.mean() - 0.5) < 1e-4 and abs(z2.std() - 0.02) < 1e-4
    # single- and multi-threaded fills agree, streams differ
    assert np.array_equal(orc.fill_normal(4096, 99, 1, 0.0, 1.0), z[:4096])
    assert not np.array_equal(orc.fill_normal(64, 99, 2, 0.0, 1.0), z[:64])


def test_map_scale_add_is_one_fma(orc):
    # framework.cu:73-78 style KATs with exactly representable results
    a = np.array([1, 2, 3, -4, 0.5], np.float32)
    b = np.array([4, 5, 6, 1, -1.25], np.float32)
    assert np.array_equal(orc.map_scale_add(a, b, 2.5), (2.5 * a.astype(np.float64) + b).astype(np.float32))
    # A case where the fused and unfused results differ: the exact value
    # 2.5*a + b fits in float64, so rounding it once to float32 is fmaf.
    a = np.array([1 + 2.0 ** -23, 3 + 2.0 ** -22], np.float32)
    b = np.array([-2.5, -7.5], np.float32)
    exact = 2.5 * a.astype(np.float64) + b.astype(np.float64)
    fused = exact.astype(np.float32)
    unfused = (np.float32(2.5) * a).astype(np.float32) + b
    assert not np.array_equal(fused, unfused)
    assert np.array_equal(orc.map_scale_add(a, b, 2.5), fused)


def _np_reference_reduce(x: np.ndarray, op: str) -> np.float32:
    """Independent numpy restatement of ops::reduce's launch geometry:
    strided per-thread partials, 32-lane shuffle trees, cross-warp tree."""
    comb = {"sum": np.add, "max": np.fmax, "product": np.multiply}[op]
    ident = {"sum": 0.0, "max": -np.inf, "product": 1.0}[op]

    def tree(lanes):  # lanes: (..., 32) float32
        cur = lanes.copy()
        for off in (16, 8, 4, 2, 1):
            shifted = np.concatenate([cur[..., off:], cur[..., 32 - off:]], axis=-1)  # out-of-range lanes read themselves
            cur = comb(cur, shifted).astype(np.float32)
        return cur[..., 0]

    def block(vals):  # vals: (256,)
        w = tree(vals.reshape(8, 32))
        lanes = np.full(32, ident, np.float32)
        lanes[:8] = w
        return tree(lanes)

    def partial(data, b, grid):
        stride = grid * 256
        acc = np.full(256, ident, np.float32)
        for start in range(b * 256, data.size, stride):
            chunk = data[start:start + 256]
            acc[:chunk.size] = comb(acc[:chunk.size], chunk).astype(np.float32)
        return block(acc)

    n = x.size
    blocks = -(-n // 256)
    if blocks <= 1:
        return partial(x, 0, 1)
    blocks = min(blocks, 1024)
    parts = np.array([partial(x, b, blocks) for b in range(blocks)], np.float32)
    return partial(parts, 0, 1)


def test_reduce_known_answers(orc):
    ones = np.ones(4099, np.float32)
    for n in (0, 1, 31, 32, 33, 255, 256, 257, 4099):  # framework.cu:144-149
        assert orc.reduce(ones[:n], "sum") == n
    assert orc.reduce(np.zeros(0, np.float32), "product") == 1.0  # framework.cu:80
    assert orc.reduce(np.arange(1, 4, dtype=np.float32), "sum") == 6.0  # framework.cu:79
    assert orc.reduce(np.array([-3, 7, 2], np.float32), "max") == 7.0


@pytest.mark.parametrize("n", [7, 256, 300, 5000, 70000, 262144 + 1000])
def test_reduce_matches_independent_order(orc, n):
    x = orc.fill_normal(n, 5, n, 0.0, 1.0) * np.float32(1e3)
    x[::7] *= np.float32(1e4)  # wide dynamic range makes the summation order visible
    got = orc.reduce(x, "sum")
    want = _np_reference_reduce(x, "sum")
    assert np.float32(got) == want
    exact = orc.sum_f64(x)
    assert abs(got - exact) <= 1e-5 * orc.sum_abs_f64(x)
    # a wrong order (plain sequential float32 sum) is distinguishable on this data
    if n >= 5000:
        seq = np.float32(0)
        for v in x:
            seq = np.float32(seq + v)
        assert seq != np.float32(got)


def test_block_reduce_tree_by_hand(orc):
    # 64 threads, only thread 33 nonzero: result is exactly its value (no double counting)
    v = np.zeros(64, np.float32)
    v[33] = 5.0
    assert orc.block_reduce(v, "sum") == 5.0
    # lanes past the warp must not be re-added: one warp of 1..32
    v = np.arange(1, 33, dtype=np.float32)
    assert orc.block_reduce(v, "sum") == 528.0
    # max with a missing-warp identity
    v = -np.arange(96, dtype=np.float32)
    assert orc.block_reduce(v, "max") == 0.0


def test_softmax_known_answer(orc):
    # framework.cu:185-195: rows [-2..2] and [3..7] -> exp(j-4)/sum_j exp(j-4)
    x = np.arange(-2, 8, dtype=np.float32)
    out = orc.softmax_rows(x, 2, 5)
    den = sum(math.exp(j - 4) for j in range(5))
    want = [math.exp(i % 5 - 4) / den for i in range(10)]
    assert framework_close(out, want)
    # invariants: rows sum to one, shift invariance, argmax preserved
    z = orc.fill_normal(16 * 333, 3, 0, 0.0, 4.0)
    y = orc.softmax_rows(z, 16, 333).reshape(16, 333)
    assert np.allclose(y.sum(1), 1.0, atol=2e-6)
    y2 = orc.softmax_rows(z + np.float32(8.0), 16, 333).reshape(16, 333)
    assert np.allclose(y, y2, rtol=2e-5, atol=1e-12)
    assert np.array_equal(y.argmax(1), z.reshape(16, 333).argmax(1))


def test_layer_norm_known_answer(orc):
    # framework.cu:196-199: gamma 2, beta 1 -> (i%5-2)*2/sqrt(2+1e-5)+1
    x = np.arange(-2, 8, dtype=np.float32)
    out = orc.layer_norm_rows(x, np.full(5, 2, np.float32), np.ones(5, np.float32), 2, 5, 1e-5)
    want = [(i % 5 - 2) * 2 / math.sqrt(2 + 1e-5) + 1 for i in range(10)]
    assert framework_close(out, want)
    z = orc.fill_normal(8 * 1000, 4, 0, 3.0, 2.0)
    y = orc.layer_norm_rows(z, np.ones(1000, np.float32), np.zeros(1000, np.float32), 8, 1000, 1e-5)
    y = y.reshape(8, 1000).astype(np.float64)
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y.var(1), 1, atol=1e-4)


def test_rms_norm_closed_form(orc):
    cols, eps = 2048, 1e-5
    z = orc.fill_normal(4 * cols, 6, 0, 0.0, 1.0)
    y = orc.rms_norm_rows(z, np.ones(cols, np.float32), 4, cols, eps).reshape(4, cols).astype(np.float64)
    ms = (z.reshape(4, cols).astype(np.float64) ** 2).mean(1)
    assert np.allclose((y ** 2).mean(1), ms / (ms + eps), rtol=1e-5)
    # constant row c: out = c / sqrt(c^2 + eps) * w
    w = np.linspace(0.5, 1.5, 8).astype(np.float32)
    y = orc.rms_norm_rows(np.full(8, 0.25, np.float32), w, 1, 8, eps)
    assert framework_close(y, 0.25 / math.sqrt(0.0625 + eps) * w.astype(np.float64))


def test_round_bf16_known_bits(orc):
    # hand-computed: 1.0 -> 0x3F80; 1 + 2^-8 is a tie between 0x3F80 and 0x3F81 -> even 0x3F80;
    # 1 + 3*2^-8 ties between 0x3F81 and 0x3F82 -> even 0x3F82; 1 + 2^-8 + 2^-20 rounds up -> 0x3F81
    x = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 + 2 ** -8 + 2 ** -20, -2.0, 0.0, 3.0e38], np.float32)
    r, b = orc.round_bf16(x)
    assert list(b[:6]) == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC000, 0x0000]
    assert np.array_equal(r.view(np.uint32), b.astype(np.uint32) << 16)
    # 8 significant bits: relative rounding error at most 2^-8, and it is attained closely
    z = orc.fill_normal(10000, 8, 0, 0.0, 1.0)
    rz, _ = orc.round_bf16(z)
    rel = np.abs(rz - z) / np.abs(z)
    assert rel.max() <= 2 ** -8 and rel.max() > 2 ** -9


def test_mat_mul_oracle_vs_float64(orc):
    M, N, K = 37, 300, 29
    A = orc.fill_normal(M * N, 9, 0, 0.0, 1.0)
    B = orc.fill_normal(N * K, 9, 1, 0.0, 1.0)
    out, absdot = orc.mat_mul_rows(A, B, M, N, K)
    ref = A.reshape(M, N).astype(np.float64) @ B.reshape(N, K).astype(np.float64)
    assert np.max(np.abs(out - ref) / absdot) < 1e-6
    # transposed storage of B gives the same values; bias + relu applied after the sum
    bias = orc.fill_uniform(K, 9, 2, -0.1, 0.1)
    out_t, _ = orc.mat_mul_rows(A, np.ascontiguousarray(B.reshape(N, K).T), M, N, K, bias=bias, b_transposed=True,
                                act="relu")
    assert np.array_equal(out_t, np.maximum(out + bias, 0))
    # the reference GEMV order agrees within the same bound
    y = orc.gemv(A[:N], np.ascontiguousarray(B.reshape(N, K).T), N, K)
    assert np.max(np.abs(y - ref[0]) / absdot[0]) < 1e-6


def _np_attention(q, k, v, T, S, qh, kv_rep, D, cap):
    """float64 textbook causal attention (scripts/llama/export_reference.py:71-84 maths)."""
    q = q.reshape(qh, T, D).astype(np.float64)
    k = k.reshape(qh // kv_rep, cap, D)[:, :S].astype(np.float64)
    v = v.reshape(qh // kv_rep, cap, D)[:, :S].astype(np.float64)
    out = np.zeros((qh, T, D))
    for h in range(qh):
        s = q[h] @ k[h // kv_rep].T / np.sqrt(D)
        mask = np.arange(S)[None, :] <= (S - T + np.arange(T))[:, None]
        s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[h] = p @ v[h // kv_rep]
    return out


@pytest.mark.parametrize("T,S,qh,kv_rep,D,cap", [(5, 5, 4, 2, 16, 5), (17, 40, 8, 4, 64, 48), (64, 64, 2, 1, 32, 64)])
def test_attention_explicit_vs_float64(orc, T, S, qh, kv_rep, D, cap):
    q = orc.fill_normal(qh * T * D, 11, 0, 0.0, 1.0)
    k = orc.fill_normal(qh // kv_rep * cap * D, 11, 1, 0.0, 1.0)
    v = orc.fill_normal(qh // kv_rep * cap * D, 11, 2, 0.0, 1.0)
    out, bound = orc.attention_explicit(q, k, v, T, S, qh, kv_rep, D, cap)
    ref = _np_attention(q, k, v, T, S, qh, kv_rep, D, cap)
    assert np.max(np.abs(out - ref) / (bound + 1e-12)) < 1e-5
    # sampled rows equal the full run
    rows = [0, T - 1]
    out2, _ = orc.attention_explicit(q, k, v, T, S, qh, kv_rep, D, cap, rows=rows)
    assert np.array_equal(out2, out[:, rows])


def test_attention_special_cases(orc):
    # a query that sees one key returns that key's value row exactly
    T = S = 3
    D = 16
    q = orc.fill_normal(T * D, 12, 0, 0.0, 1.0)
    k = orc.fill_normal(S * D, 12, 1, 0.0, 1.0)
    v = orc.fill_normal(S * D, 12, 2, 0.0, 1.0)
    out, _ = orc.attention_explicit(q, k, v, T, S, 1, 1, D, S)
    assert np.array_equal(out[0, 0], v[:D])
    # identical keys: softmax is uniform and the output is the mean of the visible values
    k_same = np.tile(k[:D], S)
    out, _ = orc.attention_explicit(q, k_same, v, T, S, 1, 1, D, S)
    assert np.allclose(out[0, 2], v.reshape(S, D).mean(0), atol=1e-6)


@pytest.mark.parametrize("length", [1, 7, 256, 300])
def test_attention_decode_equals_last_row(orc, length):
    qh, kv_rep, D, cap = 8, 4, 64, 320
    q = orc.fill_normal(qh * D, 13, 0, 0.0, 1.0)
    k = orc.fill_normal(qh // kv_rep * cap * D, 13, 1, 0.0, 1.0)
    v = orc.fill_normal(qh // kv_rep * cap * D, 13, 2, 0.0, 1.0)
    dec = orc.attention_decode(q, k, v, qh, kv_rep, D, length, cap)
    # the decode query is the prefill row at position length - 1 (T = 1, S = length)
    exp_, bound = orc.attention_explicit(q, k, v, 1, length, qh, kv_rep, D, cap)
    assert np.max(np.abs(dec - exp_[:, 0]) / (bound[:, 0] + 1e-12)) < 1e-5


# ---- Scan / Transform / GatherScatter oracle (semantics defined in oracle.h) ----

def test_scan_closed_forms(orc):
    n = 5000
    ones = np.ones(n, np.float32)
    out, absp = orc.scan(ones)
    assert np.array_equal(out, np.arange(1, n + 1, dtype=np.float32)) and np.array_equal(absp, np.arange(1, n + 1))
    excl, _ = orc.scan(ones, inclusive=False)
    assert np.array_equal(excl, np.arange(0, n, dtype=np.float32))
    ints = np.arange(n, dtype=np.float32)  # triangular numbers stay below 2^24: exact in fp32
    out, _ = orc.scan(ints)
    assert np.array_equal(out, (np.arange(n, dtype=np.int64) * (np.arange(n) + 1) // 2).astype(np.float32))
    assert np.array_equal(orc.scan(np.zeros(0, np.float32))[0], np.zeros(0, np.float32))


def test_scan_matches_float64_cumsum_and_running_max(orc):
    x = orc.fill_normal(10007, 21, 0, 0.0, 1.0)
    out, absp = orc.scan(x)
    assert np.array_equal(out, np.cumsum(x.astype(np.float64)).astype(np.float32))
    assert np.allclose(absp, np.cumsum(np.abs(x.astype(np.float64))))
    excl, _ = orc.scan(x, inclusive=False)
    assert excl[0] == 0.0 and np.array_equal(excl[1:], out[:-1])
    mx, _ = orc.scan(x, maximum=True)
    assert np.array_equal(mx, np.maximum.accumulate(x))
    mex, _ = orc.scan(x, maximum=True, inclusive=False)
    assert mex[0] == -np.inf and np.array_equal(mex[1:], mx[:-1])
    mono = np.arange(100, dtype=np.float32)
    assert np.array_equal(orc.scan(mono, maximum=True)[0], mono)
    assert np.array_equal(orc.scan(mono[::-1].copy(), maximum=True)[0], np.full(100, 99, np.float32))
    # fmaxf drops NaN: a NaN-only prefix scans to -inf, later values take over
    nan_first = np.array([np.nan, np.nan, 2.0, np.nan, 1.0], np.float32)
    assert np.array_equal(orc.scan(nan_first, maximum=True)[0], np.array([-np.inf, -np.inf, 2, 2, 2], np.float32))


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 64), (65, 129), (1000, 3)])
def test_transpose_oracle(orc, rows, cols):
    x = orc.fill_uniform(rows * cols, 22, rows, -1.0, 1.0)
    t = orc.transpose(x, rows, cols)
    assert np.array_equal(t.reshape(cols, rows), x.reshape(rows, cols).T)
    assert np.array_equal(orc.transpose(t, cols, rows), x)


def test_gather_scatter_oracle(orc):
    x = orc.fill_uniform(1000, 23, 0, -1.0, 1.0)
    perm = np.random.default_rng(5).permutation(1000).astype(np.int32)
    g = orc.gather(x, perm)
    assert np.array_equal(g, x[perm])
    # scattering the gathered values back through the same permutation restores x
    assert np.array_equal(orc.scatter(g, perm, np.zeros(1000, np.float32)), x)
    bad = np.array([0, -1, 999, 1000, 2**31 - 1], np.int32)
    gb = orc.gather(x, bad)
    assert gb[0] == x[0] and gb[2] == x[999] and np.isnan(gb[[1, 3, 4]]).all()
    sb = orc.scatter(np.array([5, 6, 7], np.float32), np.array([1, -3, 1], np.int32), np.zeros(4, np.float32))
    assert np.array_equal(sb, np.array([0, 7, 0, 0], np.float32))  # in-order: the last duplicate wins


def test_threaded_oracle_functions_match_single_thread(orc):
    """reduce (independent partial blocks), decode attention (independent heads), transpose and gather
    split their work across threads for the CPU baseline; the results must not depend on the count."""
    x = orc.fill_normal(300_001, 91, 0, 0.0, 1.0)
    q = orc.fill_normal(8 * 64, 91, 1, 0.0, 1.0)
    k = orc.fill_normal(2 * 700 * 64, 91, 2, 0.0, 1.0)
    v = orc.fill_normal(2 * 700 * 64, 91, 3, 0.0, 1.0)
    idx = np.random.default_rng(91).permutation(x.size).astype(np.int32)
    results = []
    for threads in (1, 5):
        orc.set_threads(threads)
        results.append((np.float32(orc.reduce(x, "sum")).view(np.uint32),
                        orc.attention_decode(q, k, v, 8, 4, 64, 650, 700).view(np.uint32),
                        orc.transpose(x[:299 * 1003], 299, 1003).view(np.uint32),
                        orc.gather(x, idx).view(np.uint32)))
    orc.set_threads(1)
    for a, b in zip(*results):
        assert np.array_equal(a, b)
