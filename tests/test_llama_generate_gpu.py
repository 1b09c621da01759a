"""GPU: long-context prefill/decode (SURVEY next row: prompts beyond the
reference's 2048-row explicit-attention limit, up to the 8192 session cap)
against the oracle, and the host generation loop (greedy / nucleus sampling
with EOS and capacity stops, examples/llama/generate.py:111-135)."""
import numpy as np
import pytest

from tests.test_llama_gpu import SMALL, TINY, margin, nrmse, prompt

pytestmark = pytest.mark.gpu
SEED = 515


@pytest.fixture(scope="module")
def small_pair(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    orc.set_threads(16)
    return LlamaModel.load_random(SMALL, SEED, 0.02, "uniform"), orc.Llama(SMALL, SEED, 0.02, "uniform")


@pytest.fixture(scope="module")
def tiny_pair(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    orc.set_threads(16)
    return LlamaModel.load_random(TINY, SEED + 1, 0.02, "uniform"), orc.Llama(TINY, SEED + 1, 0.02, "uniform")


def run_long(gpu, cpu, n, cap, steps):
    ids = prompt(n, gpu.vocab_size if hasattr(gpu, "vocab_size") else cpu.V, n)
    s = gpu.session(cap)
    cpu.reset(cap)
    tok, ctok = s.prefill(ids), None
    ctok, clog = cpu.prefill(ids)
    worst = nrmse(s.last_logits(), clog)
    done = 0
    for _ in range(steps):
        if tok != ctok:
            assert margin(clog) < 1e-3, margin(clog)
            break
        tok = s.decode_step(tok)
        ctok, clog = cpu.decode(ctok)
        worst = max(worst, nrmse(s.last_logits(), clog))
        done += 1
    assert worst <= 1e-5, worst
    return s, tok, n + done  # session, its last token, cache length


def test_prefill_beyond_2048_rows(small_pair):
    """2500-row prompt: the reference switches to its chunked kernel above 2048 rows."""
    gpu, cpu = small_pair
    run_long(gpu, cpu, 2500, 4096, 6)


def test_decode_to_the_session_cap(tiny_pair, ow):
    """8000-row prompt in an 8192 session, decode up to the cap, then the cap is enforced."""
    gpu, cpu = tiny_pair
    s, tok, length = run_long(gpu, cpu, 8000, 8192, 4)
    while length < 8192:  # every position up to the cap is usable
        tok = s.decode_step(tok)
        length += 1
    assert np.all(np.isfinite(s.last_logits()))
    with pytest.raises(ow.OpworksError, match="capacity"):
        s.decode_step(tok)


def test_generate_greedy_matches_decode_loop(small_pair):
    gpu, _ = small_pair
    ids = prompt(20, SMALL["vocab_size"], 8)
    s = gpu.session(128)
    toks, _, _ = s.generate_greedy(ids, 12)
    assert s.generate(ids, 12) == [int(t) for t in toks]


def test_generate_stops_at_eos_and_capacity(ow):
    from opworks_amd.llama import LlamaModel
    gpu = LlamaModel.load_random(TINY, SEED + 2, 0.02, "uniform")
    ids = prompt(5, TINY["vocab_size"], 9)
    s = gpu.session(64)
    free_run = s.generate(ids, 40)
    assert len(free_run) == 40
    # declare the 4th generated token an end-of-sequence id: generation stops right after it
    eos_cfg = dict(TINY, eos_token_id=[int(free_run[3])])
    m2 = LlamaModel.load_random(eos_cfg, SEED + 2, 0.02, "uniform")
    out = m2.session(64).generate(ids, 40)
    first = free_run.index(free_run[3])
    assert out == free_run[:first + 1]
    # capacity: prompt 5 + 59 new tokens fills a 64-entry session; the loop stops without overflowing
    assert len(s.generate(ids, 59)) == 59
    with pytest.raises(ValueError):
        s.generate(ids, 60)


def test_sampled_generation_is_seeded(small_pair):
    gpu, _ = small_pair
    ids = prompt(10, SMALL["vocab_size"], 10)
    s = gpu.session(64)
    a = s.generate(ids, 16, temperature=0.8, top_p=0.9, seed=3)
    b = s.generate(ids, 16, temperature=0.8, top_p=0.9, seed=3)
    c = s.generate(ids, 16, temperature=0.8, top_p=0.9, seed=4)
    assert a == b and len(a) == 16
    assert a != c or len(set(a)) == 1


def test_greedy_chain_stops_at_a_step_without_a_winner(ow, tmp_path):
    """Regression: chained greedy generation must not feed an argmax without a winner back in as a token.
    Token Z's embedding row is +inf in column 0 and zero elsewhere: its tied LM-head logit is +inf whenever
    the normalised final hidden state is positive there, so Z wins a step; fed back in, Z's row normalises
    to NaN, so the next step's logits are all NaN and its argmax is 0x7fffffff (the reference's all-NaN
    result, include/ops/argmax.cuh:8-14). The host loop of decode_step calls returns that index as the
    reference's decode_step does; a chained generation that reaches that step stops there and raises
    instead of reading embedding row 0x7fffffff, and a generation that ends at Z matches the host loop."""
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    from tests.packs import pack_from_oracle
    cfg = TINY
    V, H = cfg["vocab_size"], cfg["hidden_size"]
    cpu = orc.Llama(cfg, SEED + 7, 0.02, "uniform")
    Z = 300
    embed = cpu.weight(0, 0, V * H).reshape(V, H)
    embed[Z] = 0.0
    embed[Z, 0] = np.inf
    path = tmp_path / "inf_row.pack"
    pack_from_oracle(str(path), cpu, cfg, overrides={"model.embed_tokens.weight": embed})
    gpu = LlamaModel.load(str(path))
    ids = prompt(12, V, 99)
    s = gpu.session(128)
    toks = [s.prefill(ids)]
    while toks[-1] != Z and len(toks) < 40:
        toks.append(s.decode_step(toks[-1]))
    assert toks[-1] == Z, toks
    k = len(toks) - 1  # index of Z among the generated tokens
    assert s.decode_step(Z) == 0x7FFFFFFF
    with pytest.raises(ow.OpworksError, match="outside the vocabulary"):
        s.decode_step(0x7FFFFFFF)
    print(f"[greedy guard] Z generated at step {k}", flush=True)
    g = gpu.session(128)
    got, _, _ = g.generate_greedy(ids, k + 1)
    assert [int(t) for t in got] == toks
    g2 = gpu.session(128)
    with pytest.raises(ow.OpworksError, match="produced no token id"):
        g2.generate_greedy(ids, k + 6)
    g2.reset()
    again, _, _ = g2.generate_greedy(ids, k + 1)
    assert [int(t) for t in again] == toks
