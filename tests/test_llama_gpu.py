"""GPU parity of the Llama runtime (opw_llama_* C ABI) against the oracle's
restatement of the reference forward on the same seeded weights.

Bars: per-layer hidden states and logits NRMSE <= 1e-5 (the reference's fp32
model tests use 1e-3 against HF, tests/model/model_test_body.cuh:60-80);
greedy token ids identical, except that a divergence is accepted only at a
step whose oracle top-1/top-2 margin is below 1e-3 (the reference's near-tie
rule of model_test_body.cuh:246-264 with a 50x tighter margin); KV-cache
decode vs recompute NRMSE <= 1e-5 (model_test_body.cuh:106-169)."""
import numpy as np
import pytest

from tests.packs import pack_from_oracle

pytestmark = pytest.mark.gpu

TINY = dict(num_hidden_layers=2, hidden_size=256, intermediate_size=1024, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, vocab_size=512, rms_norm_eps=1e-5, rope_theta=500000.0,
            rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                          "original_max_position_embeddings": 64}, eos_token_id=[7, 9])
SMALL = dict(num_hidden_layers=4, hidden_size=512, intermediate_size=2048, num_attention_heads=8,
             num_key_value_heads=2, head_dim=64, vocab_size=1000, rms_norm_eps=1e-5, rope_theta=500000.0,
             rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                           "original_max_position_embeddings": 8192}, eos_token_id=[1])
# hidden >= 1024 selects the column-split qkv / o_proj GEMV kernels
MID = dict(num_hidden_layers=3, hidden_size=1024, intermediate_size=2048, num_attention_heads=16,
           num_key_value_heads=4, head_dim=64, vocab_size=3000, rms_norm_eps=1e-5, rope_theta=500000.0,
           rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                         "original_max_position_embeddings": 8192}, eos_token_id=[1])
SEED = 2024


def nrmse(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(np.sqrt(np.mean(b ** 2)), 1e-12))


def margin(logits):
    top = np.sort(np.asarray(logits, np.float64))[-2:]
    return float(top[1] - top[0])


@pytest.fixture(scope="module")
def tiny(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    return LlamaModel.load_random(TINY, SEED, 0.02, "uniform"), orc.Llama(TINY, SEED, 0.02, "uniform")


@pytest.fixture(scope="module")
def small(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    return LlamaModel.load_random(SMALL, SEED + 1, 0.02, "uniform"), orc.Llama(SMALL, SEED + 1, 0.02, "uniform")


@pytest.fixture(scope="module")
def mid(ow):
    from opworks_amd.llama import LlamaModel
    from tests import oracle as orc
    return LlamaModel.load_random(MID, SEED + 2, 0.02, "uniform"), orc.Llama(MID, SEED + 2, 0.02, "uniform")


def prompt(n, vocab, seed):
    return [int(v) for v in np.random.default_rng(seed).integers(0, vocab, n)]


@pytest.mark.parametrize("n", [1, 2, 7, 33, 100])
def test_debug_prefill_layers_match(tiny, n):
    gpu, cpu = tiny
    ids = prompt(n, TINY["vocab_size"], n)
    s = gpu.session(128)
    tok, caps = s.debug_prefill(ids)
    cpu.reset(128)
    ctok, clog, ccaps = cpu.prefill(ids, capture=True)
    for layer in range(TINY["num_hidden_layers"] + 1):
        assert nrmse(caps[layer], ccaps[layer]) <= 1e-5, layer
    logits = s.last_logits()
    assert nrmse(logits, clog) <= 1e-5
    assert tok == ctok or margin(clog) < 1e-3


def greedy_compare(gpu, cpu, ids, steps, cap):
    s = gpu.session(cap)
    cpu.reset(cap)
    tok = s.prefill(ids)
    ctok, clog = cpu.prefill(ids)
    got, want = [tok], [ctok]
    worst = nrmse(s.last_logits(), clog)
    for i in range(steps - 1):
        if tok != ctok:
            assert margin(clog) < 1e-3, f"divergence at step {i} with margin {margin(clog)}"
            return got, want, worst
        tok = s.decode_step(tok)
        ctok, clog = cpu.decode(ctok)
        worst = max(worst, nrmse(s.last_logits(), clog))
        got.append(tok)
        want.append(ctok)
    assert worst <= 1e-5, worst
    return got, want, worst


@pytest.mark.parametrize("fixture,n,steps", [("tiny", 5, 40), ("tiny", 1, 20), ("small", 64, 48), ("mid", 1, 24),
                                             ("mid", 37, 40)])
def test_greedy_matches_oracle(request, fixture, n, steps):
    gpu, cpu = request.getfixturevalue(fixture)
    cfg = {"tiny": TINY, "small": SMALL, "mid": MID}[fixture]
    got, want, _ = greedy_compare(gpu, cpu, prompt(n, cfg["vocab_size"], 99 + n), steps, 256)
    # identical ids; a divergence is accepted only at a near tie (< 1e-3, asserted
    # inside greedy_compare), after which the sequences are not compared further
    assert got[:-1] == want[:-1] and (got[-1] == want[-1] or len(got) < steps)


@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 64, 65, 127, 128, 129])
def test_kv_cache_decode_vs_recompute(small, L):
    gpu, _ = small
    ids = prompt(L + 1, SMALL["vocab_size"], 7)
    a = gpu.session(256)
    a.prefill(ids[:L])
    a.decode_step(ids[L])
    la = a.last_logits()
    b = gpu.session(256)
    b.prefill(ids[:L + 1])
    lb = b.last_logits()
    assert nrmse(la, lb) <= 1e-5


def test_reset_repeat_is_deterministic(tiny):
    gpu, _ = tiny
    s = gpu.session(64)
    ids = prompt(9, TINY["vocab_size"], 3)
    outs = []
    for _ in range(2):
        s.reset()
        tok = s.prefill(ids)
        seq = [tok]
        for _ in range(15):
            tok = s.decode_step(tok)
            seq.append(tok)
        outs.append((seq, s.last_logits()))
    assert outs[0][0] == outs[1][0] and np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("fixture,n,steps", [("tiny", 1, 30), ("tiny", 9, 2), ("small", 33, 20)])
def test_generate_greedy_chains_like_decode_steps(request, fixture, n, steps):
    """opw_llama_generate_greedy chains the steps on the device (the argmax kernel feeds the next step);
    its tokens, the last logits and the state it leaves (a further decode_step) must be bit-identical to a
    prefill + decode_step loop on another session."""
    gpu, _ = request.getfixturevalue(fixture)
    cfg = {"tiny": TINY, "small": SMALL}[fixture]
    ids = prompt(n, cfg["vocab_size"], 17 + n)
    a, b = gpu.session(128), gpu.session(128)
    toks, _, _ = a.generate_greedy(ids, steps)
    tok = b.prefill(ids)
    want = [tok]
    for _ in range(steps - 1):
        tok = b.decode_step(tok)
        want.append(tok)
    assert [int(t) for t in toks] == want
    assert np.array_equal(a.last_logits(), b.last_logits())
    assert a.decode_step(want[-1]) == b.decode_step(want[-1])
    assert np.array_equal(a.last_logits(), b.last_logits())
    with pytest.raises(Exception):
        gpu.session(8).generate_greedy(prompt(4, cfg["vocab_size"], 5), 6)  # 4 + 5 positions > 8


def test_stage_timing_leaves_the_sequence_unchanged(tiny, ow):
    """time_decode_stage runs stages out of order against the live session; the
    tokens and logits that follow must equal an untimed run's."""
    gpu, _ = tiny
    ids = prompt(6, TINY["vocab_size"], 4)
    runs = []
    for timed in (False, True):
        s = gpu.session(64)
        tok = s.prefill(ids)
        seq = [tok]
        for i in range(10):
            if timed and i == 3:
                for stage in s.STAGES:
                    assert s.time_decode_stage(stage, reps=2) > 0
            tok = s.decode_step(tok)
            seq.append(tok)
        runs.append((seq, s.last_logits()))
    assert runs[0][0] == runs[1][0] and np.array_equal(runs[0][1], runs[1][1])
    fresh = gpu.session(8)
    with pytest.raises(ow.OpworksError, match="prefilled"):
        fresh.time_decode_stage("gate_up")


def test_interleaved_sessions(tiny):
    gpu, _ = tiny
    ids_a, ids_b = prompt(6, TINY["vocab_size"], 4), prompt(11, TINY["vocab_size"], 5)
    solo = []
    for ids in (ids_a, ids_b):
        s = gpu.session(64)
        tok = s.prefill(ids)
        seq = [tok]
        for _ in range(10):
            tok = s.decode_step(tok)
            seq.append(tok)
        solo.append(seq)
    sa, sb = gpu.session(64), gpu.session(64)
    ta, tb = sa.prefill(ids_a), sb.prefill(ids_b)
    seq_a, seq_b = [ta], [tb]
    for _ in range(10):
        ta = sa.decode_step(ta)
        tb = sb.decode_step(tb)
        seq_a.append(ta)
        seq_b.append(tb)
    assert [seq_a, seq_b] == solo


def test_ffi_edge_cases(tiny, ow):
    """tests/model/test_edges.py:46-82 semantics through the C ABI."""
    gpu, _ = tiny
    s = gpu.session(8)
    with pytest.raises(ow.OpworksError, match="vocabulary"):
        s.prefill([TINY["vocab_size"]])
    with pytest.raises(ow.OpworksError, match="vocabulary"):
        s.prefill([-1])
    with pytest.raises(ow.OpworksError, match="at least one token"):
        s.prefill([])
    with pytest.raises(ow.OpworksError, match="capacity"):
        s.prefill(list(range(9)))
    tok = s.prefill([1, 2, 3])  # the session is still usable after errors
    with pytest.raises(ow.OpworksError, match="fresh session"):
        s.prefill([1])
    with pytest.raises(ow.OpworksError, match="vocabulary"):
        s.decode_step(10 ** 6)
    for _ in range(5):
        tok = s.decode_step(tok)
    with pytest.raises(ow.OpworksError, match="capacity exhausted"):
        s.decode_step(tok)
    assert s.is_eos(7) and s.is_eos(9) and not s.is_eos(8)
    with pytest.raises(ow.OpworksError):
        gpu.session(0)
    with pytest.raises(ow.OpworksError):
        gpu.session(8193)
    from opworks_amd import lib
    assert lib().opw_llama_prefill(None, None, 0, None, 0) == -1
    assert "null session" in lib().opw_llama_last_error().decode()


def test_rejected_calls_leave_the_session_untouched(tiny, ow):
    """Capacity and buffer checks of the added entry points run before any work: a rejected
    generate_greedy leaves the session fresh, a rejected profile_decode_step leaves its length."""
    import ctypes
    from ctypes import POINTER, c_float, c_int32
    from opworks_amd import lib
    gpu, cpu = tiny
    s = gpu.session(8)
    with pytest.raises(ow.OpworksError, match="capacity"):
        s.generate_greedy([1, 2, 3], 7)  # 3 + 7 - 1 > 8
    ids = [1, 2, 3]
    tok = s.prefill(ids)  # still fresh: prefill is accepted
    cpu.reset(8)
    assert tok == cpu.prefill(ids)[0]
    small = np.zeros(3, np.float32)
    err = ctypes.create_string_buffer(256)
    rc = lib().opw_llama_profile_decode_step(s.handle, tok, small.ctypes.data_as(POINTER(c_float)), small.size,
                                             err, 256)
    assert rc == -1 and b"entries" in err.value
    nxt = s.decode_step(tok)  # the rejected call did not advance the session
    assert nxt == cpu.decode(tok)[0]


def test_pack_load_matches_random_init(tiny, tmp_path, ow):
    from opworks_amd.llama import LlamaModel
    gpu, cpu = tiny
    path = tmp_path / "tiny.opwpack"
    pack_from_oracle(str(path), cpu, TINY)
    packed = LlamaModel.load(str(path))
    ids = prompt(12, TINY["vocab_size"], 8)
    a, b = gpu.session(32), packed.session(32)
    assert a.prefill(ids) == b.prefill(ids)
    assert np.array_equal(a.last_logits(), b.last_logits())
    assert b.is_eos(7) and b.is_eos(9)
    with pytest.raises(ow.OpworksError, match="not an OPWPACK1 file"):
        bad = tmp_path / "bad.pack"
        bad.write_bytes(b"NOTAPACK" + b"\0" * 64)
        LlamaModel.load(str(bad))
    with pytest.raises(ow.OpworksError, match="cannot be opened"):
        LlamaModel.load(str(tmp_path / "missing.pack"))


def test_pack_reader_agrees_with_reference_build(tiny, tmp_path):
    """The reference's own PackReader (oracle/_ref) reads the pack this suite writes."""
    import ctypes
    from pathlib import Path
    lib = Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "libref_host.so"
    if not lib.exists():
        pytest.skip("oracle/_ref not built")
    h = ctypes.CDLL(str(lib))
    h.ref_pack_read_f32.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64]
    h.ref_pack_read_f32.restype = ctypes.c_int64
    _, cpu = tiny
    path = tmp_path / "t.opwpack"
    pack_from_oracle(str(path), cpu, TINY)
    H, V = TINY["hidden_size"], TINY["vocab_size"]
    out = np.empty(V * H, np.float32)
    n = h.ref_pack_read_f32(str(path).encode(), b"lm_head.weight", out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                            out.size)
    assert n == V * H and np.array_equal(out, cpu.weight(0, 0, V * H))


@pytest.mark.slow
def test_config5_llama_3_2_1b_greedy(ow):
    """Config 5: Llama-3.2-1B architecture, fp32, N(0, 0.02) weights, gamma = 1, 512 random prompt ids,
    greedy 256 tokens; token ids against the oracle (near-tie rule) and logits NRMSE per step."""
    from opworks_amd.llama import LLAMA_3_2_1B, LlamaModel
    from tests import oracle as orc
    orc.set_threads(16)
    cfg = dict(LLAMA_3_2_1B)
    gpu = LlamaModel.load_random(cfg, 1234, 0.02, "ones")
    cpu = orc.Llama(cfg, 1234, 0.02, "ones")
    ids = prompt(512, cfg["vocab_size"], 1234)
    got, want, worst = greedy_compare(gpu, cpu, ids, 256, 1024)
    print(f"config5: {len(got)} tokens compared, worst logits nrmse {worst:.2e}")
    assert got == want


def test_lm_head_argmax_ties_and_nan(tiny, tmp_path, ow):
    """The LM head's argmax rules at model level (reference: include/ops/argmax.cuh:8-14), through its
    per-workgroup records and their merge. Embedding rows 38, 39 and 301 are set to the same vector, which
    gives the largest logit of the last prompt position: 38 and 39 share an LM-head workgroup, 301 lies in
    another. Equal maxima must go to the lowest index (38). Rows 2 and 300 (300 in 301's workgroup) are
    NaN, whose logits must never win. A table of NaN rows only yields 0x7fffffff."""
    from opworks_amd.llama import LlamaModel
    from tests.packs import pack_from_oracle, write_pack
    import json
    import struct
    _, cpu = tiny
    H, V = TINY["hidden_size"], TINY["vocab_size"]
    crafted = {2, 38, 39, 300, 301}
    ids = [t for t in prompt(40, V, 4242) if t not in crafted][:12]
    cpu.reset(64)
    _, _, caps = cpu.prefill(ids, capture=True)
    h = caps[-1][-1].astype(np.float64)  # last position's hidden state after the last layer
    gamma = cpu.weight(1, 0, H).astype(np.float64)
    nh = h / np.sqrt(np.mean(h * h) + TINY["rms_norm_eps"]) * gamma
    row = (nh * (10.0 / np.dot(nh, nh))).astype(np.float32)  # logit ~10, far above the N(0, 0.02) rows

    base = tmp_path / "base.opwpack"
    pack_from_oracle(str(base), cpu, TINY)
    raw = base.read_bytes()
    mlen = struct.unpack("<Q", raw[8:16])[0]
    manifest = json.loads(raw[16:16 + mlen])
    blob = raw[16 + mlen:]
    tensors = {}
    for name, meta in manifest["tensors"].items():
        n = int(np.prod(meta["shape"]))
        tensors[name] = np.frombuffer(blob, np.float32, n, meta["offset"]).reshape(meta["shape"]).copy()
    extra = {k: v for k, v in manifest.items() if k not in ("format_version", "dtype", "tensors", "aliases")}

    emb = tensors["model.embed_tokens.weight"]
    for r in (38, 39, 301):
        emb[r] = row
    emb[2] = np.nan
    emb[300] = np.nan
    path = tmp_path / "ties.opwpack"
    write_pack(str(path), tensors, aliases=manifest.get("aliases"), extra=extra)
    s = LlamaModel.load(str(path)).session(64)
    tok = s.prefill(ids)
    logits = s.last_logits()
    assert logits[38] == logits[39] == logits[301] and logits[38] > 5.0
    assert np.isnan(logits[2]) and np.isnan(logits[300])
    assert tok == 38
    assert 0 <= s.decode_step(tok) < V
    emb[:] = np.nan
    write_pack(str(path), tensors, aliases=manifest.get("aliases"), extra=extra)
    s = LlamaModel.load(str(path)).session(64)
    assert s.prefill(ids) == 0x7FFFFFFF
