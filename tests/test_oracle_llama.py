"""Pins the oracle's Llama pieces (no GPU): RoPE frequencies, rotation, argmax
rules, the tiled/GEMV linear orders, and a whole tiny model against an
independent float64 numpy forward (textbook maths of
scripts/llama/export_reference.py:32-88)."""
import math
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
TINY = dict(num_hidden_layers=2, hidden_size=256, intermediate_size=1024, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, vocab_size=512, rms_norm_eps=1e-5, rope_theta=500000.0,
            rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                          "original_max_position_embeddings": 64})


def test_inv_freq_plain_closed_form(orc):
    got = orc.rope_inv_freq(64, 500000.0)
    want = np.array([1.0 / 500000.0 ** (2 * i / 64) for i in range(32)]).astype(np.float32)
    assert np.array_equal(got, want)


def test_inv_freq_llama3_bands(orc):
    base = orc.rope_inv_freq(64, 500000.0).astype(np.float64)
    got = orc.rope_inv_freq(64, 500000.0, True, 32.0, 1.0, 4.0, 8192).astype(np.float64)
    wl = 2 * math.pi / base
    hi_band = wl < 8192 / 4.0
    lo_band = wl > 8192 / 1.0
    assert np.array_equal(got[hi_band], base[hi_band].astype(np.float32))     # short wavelengths unchanged
    assert np.allclose(got[lo_band], base[lo_band] / 32.0, rtol=1e-7)         # long wavelengths / factor
    mid = ~hi_band & ~lo_band
    assert mid.any() and np.all(got[mid] <= base[mid] * (1 + 1e-7)) and np.all(got[mid] >= base[mid] / 32 * (1 - 1e-7))
    # the interpolation weight rises towards the short-wavelength end
    frac = (got[mid] - base[mid] / 32) / (base[mid] - base[mid] / 32)
    assert np.all(np.diff(frac) < 0)


def test_inv_freq_matches_reference_build(orc):
    lib = ROOT / "oracle" / "_ref" / "libref_host.so"
    if not lib.exists():
        pytest.skip("oracle/_ref not built (the reference sources are absent here)")
    import ctypes
    h = ctypes.CDLL(str(lib))
    h.ref_rope_inv_freq.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int]
    h.ref_rope_inv_freq.restype = ctypes.c_int
    import json
    for cfg in (TINY, dict(TINY, rope_theta=10000.0, rope_scaling=None),
                dict(TINY, rope_scaling=dict(TINY["rope_scaling"], factor=8.0, original_max_position_embeddings=8192))):
        out = np.empty(32, np.float32)
        manifest = json.dumps({"config": cfg, "eos_token_ids": [1]})
        assert h.ref_rope_inv_freq(manifest.encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 32) == 0
        rs = cfg.get("rope_scaling") or {}
        mine = orc.rope_inv_freq(64, cfg["rope_theta"], bool(rs), rs.get("factor", 0.0), rs.get("low_freq_factor", 0.0),
                                 rs.get("high_freq_factor", 0.0), rs.get("original_max_position_embeddings", 0))
        assert np.array_equal(out, mine)


def test_rope_invariants(orc):
    inv = orc.rope_inv_freq(64, 500000.0)
    x = orc.fill_normal(3 * 2 * 64, 21, 0, 0.0, 1.0)
    y0 = orc.rope(x, inv, 3, 2, 64, 0)
    # position 0 rotates by angle 0 in every pair
    assert np.array_equal(y0.reshape(3, 2, 64)[0], x.reshape(3, 2, 64)[0])
    y = orc.rope(x, inv, 3, 2, 64, 100).reshape(3, 2, 64).astype(np.float64)
    xr = x.reshape(3, 2, 64).astype(np.float64)
    norm_x = xr[..., :32] ** 2 + xr[..., 32:] ** 2
    norm_y = y[..., :32] ** 2 + y[..., 32:] ** 2
    assert np.allclose(norm_x, norm_y, rtol=1e-5)
    # closed form of one pair: rotation by (pos * inv_freq) (HF rotate_half convention)
    r, h, i = 1, 1, 3
    ang = np.float32(101) * inv[i]
    a, b = xr[r, h, i], xr[r, h, i + 32]
    assert abs(y[r, h, i] - (a * math.cos(ang) - b * math.sin(ang))) < 1e-5
    assert abs(y[r, h, i + 32] - (b * math.cos(ang) + a * math.sin(ang))) < 1e-5


def test_argmax_rules(orc):
    assert orc.argmax([1, 5, 5, 2]) == 1                       # ties -> lowest index
    assert orc.argmax([np.nan, 1, np.nan, 3]) == 3             # NaN never wins
    assert orc.argmax([np.nan, np.nan]) == 0x7FFFFFFF          # all NaN
    assert orc.argmax([-np.inf, -np.inf]) == 0                 # all -inf: lowest index
    x = orc.fill_normal(10000, 22, 0, 0.0, 1.0)
    assert orc.argmax(x) == int(np.argmax(x))


def test_linear_orders(orc):
    X = orc.fill_normal(5 * 300, 23, 0, 0.0, 1.0)
    W = orc.fill_normal(70 * 300, 23, 1, 0.0, 1.0)
    Y = orc.linear(X, W, 5, 300, 70)
    ref, _ = orc.mat_mul_rows(X, W, 5, 300, 70, b_transposed=True)
    assert np.array_equal(Y, ref)  # the same k-ascending chain
    y1 = orc.linear(X[:300], W, 1, 300, 70)
    assert np.array_equal(y1[0], orc.gemv(X[:300], W, 300, 70))


def _bf16_np(a):
    """Round to bf16, nearest-even, returned as float64 (textbook bit recipe)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32).astype(np.float64)


def _np_forward(model, cfg, ids, round_x=False):
    """float64 textbook Llama forward (HF semantics) from the oracle's weights.
    round_x: projection inputs rounded to bf16 (the tensor-core path)."""
    rx = _bf16_np if round_x else (lambda a: a)
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    qh, kvh = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg["head_dim"]
    eps = cfg["rms_norm_eps"]
    rs = cfg.get("rope_scaling") or {}

    from tests import oracle as orc
    inv = orc.rope_inv_freq(D, cfg["rope_theta"], bool(rs), rs.get("factor", 0.0), rs.get("low_freq_factor", 0.0),
                            rs.get("high_freq_factor", 0.0), rs.get("original_max_position_embeddings", 0))
    w = lambda k, l, n: model.weight(k, l, n).astype(np.float64)
    T = len(ids)
    x = w(0, 0, V * H).reshape(V, H)[ids]

    def rms(v, g):
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + eps) * g

    pos = np.arange(T)[:, None] * inv.astype(np.float64)[None, :]
    cos, sin = np.cos(pos), np.sin(pos)

    def rope(t):  # t [T, heads, D]
        a, b = t[..., :D // 2], t[..., D // 2:]
        return np.concatenate([a * cos[:, None] - b * sin[:, None], b * cos[:, None] + a * sin[:, None]], -1)

    for l in range(L):
        h = rms(x, w(9, l, H))
        h = rx(h)
        q = rope((h @ w(2, l, qh * D * H).reshape(qh * D, H).T).reshape(T, qh, D))
        k = rope((h @ w(3, l, kvh * D * H).reshape(kvh * D, H).T).reshape(T, kvh, D))
        v = (h @ w(4, l, kvh * D * H).reshape(kvh * D, H).T).reshape(T, kvh, D)
        out = np.zeros((T, qh, D))
        for hh in range(qh):
            s = q[:, hh] @ k[:, hh // (qh // kvh)].T / math.sqrt(D)
            s = np.where(np.tri(T, dtype=bool), s, -np.inf)
            p = np.exp(s - s.max(1, keepdims=True))
            out[:, hh] = (p / p.sum(1, keepdims=True)) @ v[:, hh // (qh // kvh)]
        x = x + rx(out.reshape(T, qh * D)) @ w(5, l, H * qh * D).reshape(H, qh * D).T
        h = rx(rms(x, w(10, l, H)))
        g = h @ w(6, l, I * H).reshape(I, H).T
        u = h @ w(7, l, I * H).reshape(I, H).T
        x = x + rx(g / (1 + np.exp(-g)) * u) @ w(8, l, H * I).reshape(H, I).T
    return rms(x[-1], w(1, 0, H)) @ w(0, 0, V * H).reshape(V, H).T


def test_tiny_model_vs_float64(orc):
    m = orc.Llama(TINY, 31, norm_init="uniform")
    m.reset(32)
    ids = [5, 17, 300, 2, 99, 511, 0]
    tok, logits = m.prefill(ids)
    ref = _np_forward(m, TINY, ids)
    nrmse = np.sqrt(np.mean((logits - ref) ** 2)) / np.sqrt(np.mean(ref ** 2))
    assert nrmse < 1e-5 and tok == int(np.argmax(ref))
    # KV-cache decode equals the full recompute of the longer prompt
    tok2, logits2 = m.decode(tok)
    ref2 = _np_forward(m, TINY, ids + [tok])
    assert np.sqrt(np.mean((logits2 - ref2) ** 2)) / np.sqrt(np.mean(ref2 ** 2)) < 1e-5


def test_bf16_model_weights_are_rounded(orc):
    """LlamaModelBF16: every stored weight (norms too, as a bf16 pack holds them)
    equals the nearest-even bf16 rounding of the same seeded fp32 draw."""
    f = orc.Llama(TINY, 31, norm_init="uniform")
    b = orc.Llama(TINY, 31, norm_init="uniform", bf16=True)
    H, I, V = TINY["hidden_size"], TINY["intermediate_size"], TINY["vocab_size"]
    D, qh, kvh = TINY["head_dim"], TINY["num_attention_heads"], TINY["num_key_value_heads"]
    sizes = {0: V * H, 1: H, 2: qh * D * H, 3: kvh * D * H, 4: kvh * D * H, 5: H * qh * D, 6: I * H, 7: I * H,
             8: H * I, 9: H, 10: H}
    for kind, n in sizes.items():
        wf, wb = f.weight(kind, 1, n), b.weight(kind, 1, n)
        assert np.all(wb.view(np.uint32) & 0xFFFF == 0), kind
        assert np.array_equal(wb, _bf16_np(wf).astype(np.float32)), kind


@pytest.mark.parametrize("n,round_x", [(7, False), (20, True)])
def test_bf16_model_vs_float64(orc, n, round_x):
    """Projections of fewer than 16 rows keep fp32 inputs; from 16 rows they are
    rounded to bf16 (linear_dispatch, models/llama.cuh:190-199)."""
    m = orc.Llama(TINY, 32, norm_init="uniform", bf16=True)
    m.reset(32)
    ids = [(37 * i + 5) % TINY["vocab_size"] for i in range(n)]
    tok, logits = m.prefill(ids)
    ref = _np_forward(m, TINY, ids, round_x=round_x)
    nrmse = np.sqrt(np.mean((logits - ref) ** 2)) / np.sqrt(np.mean(ref ** 2))
    if not round_x:
        assert nrmse < 1e-5
    else:
        # fp32 and float64 activations straddle a bf16 rounding boundary now and
        # then, so the match is looser; the unrounded forward must be far away
        plain = _np_forward(m, TINY, ids, round_x=False)
        far = np.sqrt(np.mean((logits - plain) ** 2)) / np.sqrt(np.mean(plain ** 2))
        assert nrmse < 5e-4 and far > 5 * nrmse, (nrmse, far)


# ---- swiglu / causal_scale restatements (include/ops/swiglu.cuh:7-12,
#      include/ops/causal_scale.cuh:9-16), pinned by closed forms
def test_oracle_swiglu_closed_forms(orc):
    g = np.array([0.0, 0.0, 30.0, -100.0, 1.5, -1.5, 4.0, -4.0], np.float32)
    u = np.array([3.0, 0.0, 2.0, 5.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    out = orc.swiglu(g, u)
    assert out[0] == 0.0 and out[1] == 0.0          # silu(0) = 0
    assert out[2] == np.float32(60.0)               # sigmoid(30) rounds to 1 in fp32
    assert out[3] == 0.0                            # exp(100) overflows: g / inf = -0
    # silu(g) - silu(-g) = g
    assert abs(float(out[4]) - float(out[5]) - 1.5) <= 4e-7 * 1.5
    assert abs(float(out[6]) - float(out[7]) - 4.0) <= 4e-7 * 4.0
    rng = np.random.default_rng(3)
    gg = rng.normal(0, 4, 4096).astype(np.float32)
    uu = rng.normal(0, 1, 4096).astype(np.float32)
    want = gg.astype(np.float64) / (1 + np.exp(-gg.astype(np.float64))) * uu
    got = orc.swiglu(gg, uu).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-37)


def test_oracle_causal_scale_mask_shape(orc):
    rows, cols, scale = 5, 9, 0.125
    x = np.random.default_rng(4).normal(size=rows * cols).astype(np.float32)
    out = orc.causal_scale(x, rows, cols, scale).reshape(rows, cols)
    for r in range(rows):
        visible = np.isfinite(out[r])
        assert visible.sum() == cols - rows + r + 1
        assert np.all(visible[: cols - rows + r + 1])  # a prefix of the keys
        assert np.array_equal(out[r][visible], (x.reshape(rows, cols)[r][visible] * np.float32(scale)))
        assert np.all(out[r][~visible] == -np.inf)
    sq = orc.causal_scale(np.ones(16, np.float32), 4, 4, 1.0).reshape(4, 4)
    assert np.array_equal(np.isfinite(sq), np.tril(np.ones((4, 4), bool)))


def test_oracle_linear_exact_is_the_rounded_exact_sum(orc):
    """orc_linear_exact, the bf16 tensor-core projection's restatement (include/ops/linear_mma.cuh:19-115):
    on bf16-valued inputs every product is exact, and each output must be their exact sum (math.fsum)
    rounded once to fp32: never more than 1 ulp away and bit-equal for nearly all outputs. A dropped
    term, a transposed weight or an fp32 accumulation chain (orc_linear) fails it."""
    import math
    rng = np.random.default_rng(11)
    rows, K, N = 3, 2048, 70  # N past one 64-column block
    X = _bf16_np(rng.normal(0, 1, (rows, K))).astype(np.float32)
    W = _bf16_np(rng.normal(0, 0.02, (N, K))).astype(np.float32)
    got = orc.linear_exact(X, W, rows, K, N)
    exact = np.array([[math.fsum((X[r].astype(np.float64) * W[j].astype(np.float64)).tolist()) for j in range(N)]
                      for r in range(rows)], np.float32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps == 0).mean() >= 0.99, (ulps.max(), (ulps == 0).mean())
    chain = orc.linear(X, W, rows, K, N)
    assert (chain != got).mean() > 0.2  # the fp32 chain is a different function
