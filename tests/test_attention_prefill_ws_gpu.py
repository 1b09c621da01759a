"""GPU: the workspace form of flash prefill (opw_attention_prefill_ws_f32). The query-tile groups
with the longest K/V ranges run as two workgroups over the halves of the range, and the one that
finishes last merges them. Same bar as the plain kernel against the oracle's restatement of the
reference's explicit attention (per output |gpu - ref| <= 1e-4 * sum_key p|v| + 1e-6), and
within rounding of the plain kernel. The arrival counters must be zero again after every call."""
import numpy as np
import pytest

from tests.test_attention_gpu import SEED, attention_f64, check, upload

pytestmark = pytest.mark.gpu


def inputs(orc, T, cap, qh, kv_rep, D, stream0=0):
    kvh = qh // kv_rep
    q = orc.fill_normal(qh * T * D, SEED, stream0, 0.0, 1.0)
    k = orc.fill_normal(kvh * cap * D, SEED, stream0 + 1, 0.0, 1.0)
    v = orc.fill_normal(kvh * cap * D, SEED, stream0 + 2, 0.0, 1.0)
    return q, k, v


class Workspace:
    def __init__(self, ow, rec_floats, counter_ints):
        self.rec_floats, self.counter_ints = max(rec_floats, 1), max(counter_ints, 1)
        self.rec = ow.DeviceBuffer.empty(self.rec_floats)
        self.counters = ow.DeviceBuffer.from_host(np.zeros(self.counter_ints, np.int32))

    def counters_zero(self):
        return not np.any(self.counters.to_host().view(np.int32))


def run_ws(ow, data, T, S, qh, kv_rep, D, cap, thr, ws=None, shrink=1):
    q, k, v = data
    need_rec, need_ctr = ow.ops.attention_prefill_workspace_size(T, S, S - T, qh, kv_rep, D, thr)
    if ws is None:
        ws = Workspace(ow, need_rec // shrink, need_ctr)
    dq, dk, dv = upload(ow, q), upload(ow, k), upload(ow, v)
    out = ow.DeviceBuffer.empty(qh * T * D)
    print(f"[prefill ws] T={T} S={S} qh={qh} kv_rep={kv_rep} D={D} thr={thr} need={need_rec},{need_ctr}", flush=True)
    ow.ops.attention_prefill_ws(dq, dk, dv, out, T, S, S - T, qh, kv_rep, D, cap, ws.rec, ws.rec_floats,
                                ws.counters, ws.counter_ints, thr)
    plain = ow.DeviceBuffer.empty(qh * T * D)
    ow.ops.attention_prefill(dq, dk, dv, plain, T, S, S - T, qh, kv_rep, D, cap)
    return out.to_host().reshape(qh, T, D), plain.to_host().reshape(qh, T, D), ws, need_rec


SHAPES = [(40, 40, 4, 4, 64, 40), (100, 100, 8, 4, 64, 128), (257, 257, 32, 4, 64, 300), (64, 200, 8, 4, 64, 256),
          (96, 96, 4, 1, 64, 96), (96, 96, 4, 2, 32, 96), (80, 80, 8, 8, 64, 80), (70, 70, 16, 16, 64, 70),
          (65, 65, 6, 3, 48, 65), (65, 65, 2, 2, 16, 65), (512, 512, 32, 4, 64, 512), (33, 33, 4, 4, 64, 40)]


@pytest.mark.parametrize("thr", [-1, 0, 3])
@pytest.mark.parametrize("T,S,qh,kv_rep,D,cap", SHAPES)
def test_prefill_ws_matches_oracle(ow, orc, T, S, qh, kv_rep, D, cap, thr):
    data = inputs(orc, T, cap, qh, kv_rep, D)
    got, plain, ws, need = run_ws(ow, data, T, S, qh, kv_rep, D, cap, thr)
    ref, bound = orc.attention_explicit(*data, T, S, qh, kv_rep, D, cap)
    check(got, ref, bound)
    check(got, plain, bound, tol=1e-6)  # the halves' merge moves results by rounding only
    assert ws.counters_zero()
    if thr == 0 and T > 32:
        assert need > 0, "threshold 0 splits every group whose split point is at least one tile"


@pytest.mark.parametrize("qh,kv_rep,D,T,S", [(32, 4, 64, 2048, 2048), (8, 1, 64, 2048, 2048), (16, 2, 64, 2048, 2048),
                                             (64, 8, 64, 2048, 2048), (32, 16, 64, 4096, 4096),
                                             (32, 4, 64, 2064, 2064), (32, 4, 64, 2048, 3000),
                                             (32, 4, 32, 1024, 1024)])
@pytest.mark.parametrize("thr", [-1, 8])
def test_prefill_ws_two_tile_workgroups(ow, orc, qh, kv_rep, D, T, S, thr):
    """The two-query-tile grids (>= 4 workgroups per CU), every wave count, a chunk of a longer
    prompt (S > T) and an idle second tile (T = 2064); sampled rows of every head."""
    data = inputs(orc, T, S, qh, kv_rep, D, stream0=10)
    got, plain, ws, _ = run_ws(ow, data, T, S, qh, kv_rep, D, S, thr)
    rows = np.unique(np.concatenate([np.arange(0, 24), np.arange(T - 24, T),
                                     np.linspace(24, T - 25, 16).astype(np.int64)])).astype(np.int32)
    ref, bound = orc.attention_explicit(*data, T, S, qh, kv_rep, D, S, rows=rows)
    check(got[:, rows], ref, bound)
    check(got, plain, np.abs(plain) + 1.0, tol=1e-6)
    assert ws.counters_zero()


def test_prefill_ws_reuse_and_small_memory(ow, orc):
    """One workspace over consecutive calls of different shapes (counters back at zero each time),
    then memory for half the records: fewer groups split, same results."""
    need = [ow.ops.attention_prefill_workspace_size(T, T, 0, 32, 4, 64, 0) for T in (512, 300)]
    ws = Workspace(ow, max(n[0] for n in need), max(n[1] for n in need))
    for T in (512, 300, 512):
        data = inputs(orc, T, T, 32, 4, 64, stream0=20 + T % 7)
        got, plain, _, _ = run_ws(ow, data, T, T, 32, 4, 64, T, 0, ws=ws)
        ref, bound = orc.attention_explicit(*data, T, T, 32, 4, 64, T)
        check(got, ref, bound)
        assert ws.counters_zero()
    data = inputs(orc, 512, 512, 32, 4, 64, stream0=30)
    got, plain, small, _ = run_ws(ow, data, 512, 512, 32, 4, 64, 512, 0, shrink=2)
    ref, bound = orc.attention_explicit(*data, 512, 512, 32, 4, 64, 512)
    check(got, ref, bound)
    assert small.counters_zero()


def test_prefill_ws_rejects(ow):
    need = ow.ops.attention_prefill_workspace_size(256, 256, 0, 8, 4, 64, 0)
    assert need[0] > 0 and need[1] > 0
    with pytest.raises(ValueError):
        ow.ops.attention_prefill_workspace_size(256, 200, 0, 8, 4, 64, -1)  # S < T
    buf = ow.DeviceBuffer.empty(16)
    with pytest.raises(ValueError):  # records claimed but no memory
        ow.ops.attention_prefill_ws(buf, buf, buf, buf, 1, 1, 0, 4, 4, 64, 1, None, 1024, None, 0)


@pytest.mark.slow
def test_config4_prefill_ws_full_size_sampled(ow, orc):
    """Config 4 (32 q heads, 8 kv heads, D = 64, T = S = 2048, N(0,1), scale 1/8) with its groups
    past 8 K/V tiles split (the automatic threshold leaves this one-round grid unsplit): against
    float64 attention within 2e-6 of sum_key p|v| and NRMSE <= 2e-6, the fp32-arithmetic bar of
    the plain kernel's test."""
    T, qh, kvh, D = 2048, 32, 8, 64
    orc.set_threads(16)
    q = orc.fill_normal(qh * T * D, SEED, 400, 0.0, 1.0, mt=True)
    k = orc.fill_normal(kvh * T * D, SEED, 401, 0.0, 1.0, mt=True)
    v = orc.fill_normal(kvh * T * D, SEED, 402, 0.0, 1.0, mt=True)
    got, plain, ws, need = run_ws(ow, (q, k, v), T, T, qh, qh // kvh, D, T, 8)
    assert need > 0, "config 4 splits its heaviest groups"
    rows = np.concatenate([np.arange(0, 40), np.arange(T - 40, T), np.arange(40, T - 40, 97)]).astype(np.int32)
    ref, bound = orc.attention_explicit(q, k, v, T, T, qh, qh // kvh, D, T, rows=rows)
    got = got[:, rows]
    check(got, ref, bound)
    exact = attention_f64(q, k, v, T, qh, qh // kvh, D, rows)
    check(got, exact, bound, tol=2e-6)
    err = got.astype(np.float64) - exact
    assert float(np.sqrt(np.mean(err ** 2)) / np.sqrt(np.mean(exact ** 2))) <= 2e-6
    assert ws.counters_zero()
