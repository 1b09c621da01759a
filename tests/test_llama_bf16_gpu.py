"""GPU parity of the bf16-weight Llama path (LlamaModelBF16; reference:
include/models/llama.cuh:190-199, 290-291; runtime/weights.cuh:16-94) against
the oracle's bf16 model on the same seeded weights.

Bar (north_star, bf16 path): final logits within NRMSE 1e-2 of the oracle at
every step; in practice they agree to ~1e-4 (prefill projection inputs are
rounded to bf16 from 16 rows, as in the reference; shorter prompts keep fp32
inputs against the widened weights). Greedy ids are
compared like the fp32 path, with a near-tie margin of 1e-2 (the bf16 bar)."""
import numpy as np
import pytest

from tests.test_llama_gpu import MID, SMALL, margin, nrmse, prompt

pytestmark = pytest.mark.gpu
SEED = 4242
SMALL_BF = dict(SMALL, torch_dtype="bfloat16")
MID_BF = dict(MID, torch_dtype="bfloat16")
BAR = 1e-2


@pytest.fixture(scope="module")
def small_bf(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    return (LlamaModel.load_random(SMALL_BF, SEED, 0.02, "uniform"), orc.Llama(SMALL_BF, SEED, 0.02, "uniform"))


@pytest.fixture(scope="module")
def mid_bf(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    return (LlamaModel.load_random(MID_BF, SEED + 1, 0.02, "uniform"), orc.Llama(MID_BF, SEED + 1, 0.02, "uniform"))


def greedy_bf16(gpu, cpu, ids, steps, cap=256):
    s = gpu.session(cap)
    cpu.reset(cap)
    tok = s.prefill(ids)
    ctok, clog = cpu.prefill(ids)
    worst = nrmse(s.last_logits(), clog)
    n_same = 1 if tok == ctok else 0
    for _ in range(steps - 1):
        if tok != ctok:
            assert margin(clog) < BAR, f"divergence with margin {margin(clog)}"
            break
        tok = s.decode_step(tok)
        ctok, clog = cpu.decode(ctok)
        worst = max(worst, nrmse(s.last_logits(), clog))
        n_same += tok == ctok
    return worst, n_same


@pytest.mark.parametrize("fixture,n,steps", [("small_bf", 1, 16), ("small_bf", 5, 24), ("small_bf", 40, 24),
                                             ("mid_bf", 3, 16), ("mid_bf", 37, 24)])
def test_bf16_greedy_matches_oracle(request, fixture, n, steps):
    gpu, cpu = request.getfixturevalue(fixture)
    cfg = SMALL_BF if fixture == "small_bf" else MID_BF
    worst, n_same = greedy_bf16(gpu, cpu, prompt(n, cfg["vocab_size"], 7 + n), steps)
    print(f"{fixture} n={n}: worst logits nrmse {worst:.2e}, {n_same} identical tokens")
    assert worst <= BAR


@pytest.mark.parametrize("n", [1, 9, 33])
def test_bf16_debug_prefill_layers(small_bf, n):
    gpu, cpu = small_bf
    ids = prompt(n, SMALL_BF["vocab_size"], n)
    s = gpu.session(64)
    tok, caps = s.debug_prefill(ids)
    cpu.reset(64)
    _, clog, ccaps = cpu.prefill(ids, capture=True)
    for layer in range(SMALL_BF["num_hidden_layers"] + 1):
        assert nrmse(caps[layer], ccaps[layer]) <= BAR, layer
    assert nrmse(s.last_logits(), clog) <= BAR


@pytest.mark.parametrize("n", [2, 9, 15])
def test_bf16_short_prefill_uses_fp32_inputs(small_bf, n):
    """2..15 rows: projections take fp32 inputs against the widened bf16 weights, as the
    reference's linear_dispatch does below 16 rows, so the GPU agrees with the oracle to fp32
    summation-order noise, not to the bf16 bar."""
    gpu, cpu = small_bf
    ids = prompt(n, SMALL_BF["vocab_size"], 100 + n)
    s = gpu.session(64)
    tok, caps = s.debug_prefill(ids)
    cpu.reset(64)
    ctok, clog, ccaps = cpu.prefill(ids, capture=True)
    for layer in range(SMALL_BF["num_hidden_layers"] + 1):
        assert nrmse(caps[layer], ccaps[layer]) <= 1e-5, layer
    assert nrmse(s.last_logits(), clog) <= 1e-5
    assert tok == ctok or margin(clog) < 1e-3


def test_bf16_kv_decode_vs_recompute(mid_bf):
    """Decoding token by token equals prefilling the whole sequence (within the bar)."""
    gpu, _ = mid_bf
    ids = prompt(24, MID_BF["vocab_size"], 3)
    a = gpu.session(64)
    a.prefill(ids[:1])
    for t in ids[1:]:
        a.decode_step(t)
    b = gpu.session(64)
    b.prefill(ids)
    assert nrmse(a.last_logits(), b.last_logits()) <= BAR


def test_bf16_pack_load_matches_random_init(small_bf, tmp_path, ow):
    from opworks_amd.llama import LlamaModel
    from tests.packs import pack_from_oracle
    gpu, cpu = small_bf
    path = tmp_path / "small_bf16.pack"
    pack_from_oracle(path, cpu, SMALL_BF, dtype="bfloat16")
    packed = LlamaModel.load(str(path))
    ids = prompt(11, SMALL_BF["vocab_size"], 5)
    a, b = gpu.session(32), packed.session(32)
    assert a.prefill(ids) == b.prefill(ids)
    assert np.array_equal(a.last_logits(), b.last_logits())
    for _ in range(5):
        t = a.decode_step(int(np.argmax(a.last_logits())))
        assert t == b.decode_step(int(np.argmax(b.last_logits())))
    assert np.array_equal(a.last_logits(), b.last_logits())


def test_bf16_rejects_narrow_widths(ow):
    from opworks_amd.llama import LlamaModel
    from tests.test_llama_gpu import TINY
    with pytest.raises(ow.OpworksError, match="bf16"):
        LlamaModel.load_random(dict(TINY, torch_dtype="bfloat16"), 1, 0.02, "ones")


@pytest.mark.slow
def test_config5_bf16_llama_3_2_1b(ow):
    """Config 5's architecture with bf16 weights (the reference's LlamaModelBF16 path at full size):
    N(0, 0.02) weights rounded to bf16, gamma = 1, 128 prompt ids, 24 greedy tokens; logits within
    the bf16 bar at every step, ids identical up to a near tie (margin < 1e-2)."""
    from opworks_amd.llama import LLAMA_3_2_1B, LlamaModel
    from tests import oracle as orc
    orc.set_threads(16)
    cfg = dict(LLAMA_3_2_1B, torch_dtype="bfloat16")
    gpu = LlamaModel.load_random(cfg, 1234, 0.02, "ones")
    cpu = orc.Llama(cfg, 1234, 0.02, "ones")
    worst, n_same = greedy_bf16(gpu, cpu, prompt(128, cfg["vocab_size"], 1234), 24, cap=256)
    print(f"config5 bf16: {n_same} identical tokens, worst logits nrmse {worst:.2e}")
    assert worst <= BAR
