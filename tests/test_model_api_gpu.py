"""The Llama runtime through its C++ API, called the way the reference's own
model tests call theirs (tests/model/model_test_body.cuh:52-306,
test_common.cuh:75-83): the hipcc-built executable opworks_amd/lib/tests/
model_api loads a weight pack by value, creates sessions by value, and checks
debug_prefill captures, greedy ids, the KV cache, session.cache.reset() and
interleaved sessions against a fixtures pack. The fixtures are written here from
the CPU oracle on the same weights, in the layout the reference's exporter
uses: ids stored as int32 bits in float32 tensors (read_int32), hidden.embed,
hidden.layer<i>, logits.last, generated_ids.

Bars (in the executable): fp32 NRMSE <= 1e-5 and cosine >= 0.99999; bf16
NRMSE <= 1e-2 and cosine >= 0.999 (the reference's bf16 tolerances); greedy ids
identical over the oracle's continuation, which is cut before the first step
whose top-1/top-2 margin is below 1e-4 (fp32) or 1e-2 (bf16)."""
import subprocess

import numpy as np
import pytest

from tests.conftest import ROOT
from tests.packs import pack_from_oracle, write_pack
from tests.test_llama_gpu import SMALL, TINY, prompt

pytestmark = pytest.mark.gpu
SEED = 5151
EXE = ROOT / "opworks_amd" / "lib" / "tests" / "model_api"


def write_fixtures(path, cpu, ids, steps, tie_margin):
    cpu.reset(2048)
    tok, logits, caps = cpu.prefill(ids, capture=True)
    tensors = {"input_ids": np.asarray(ids, np.int32).view(np.float32), "hidden.embed": caps[0].ravel(),
               "logits.last": logits}
    for i in range(1, caps.shape[0]):
        tensors[f"hidden.layer{i - 1}"] = caps[i].ravel()
    generated, step_logits = [], logits
    for _ in range(steps):
        top = np.sort(step_logits.astype(np.float64))[-2:]
        if top[1] - top[0] < tie_margin:
            break
        generated.append(tok)
        tok, step_logits = cpu.decode(tok)
    assert len(generated) >= 4, "too many near-ties for a meaningful generation check"
    tensors["generated_ids"] = np.asarray(generated, np.int32).view(np.float32)
    write_pack(path, tensors)
    return len(generated)


def run_exe(weights, fixtures):
    assert EXE.exists(), "build the C++ tests first (python -m opworks_amd.build tests)"
    print("[model_api] running", EXE, weights, fixtures, flush=True)
    proc = subprocess.run([str(EXE), str(weights), str(fixtures)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout
    assert "PASS: model API" in proc.stdout


@pytest.mark.parametrize("n", [40, 3])  # 3: one-row prefills (the decode kernels) in the sweep and split
def test_model_api_fp32(ow, tmp_path, n):
    from tests import oracle as orc
    cpu = orc.Llama(TINY, SEED, 0.02, "uniform")
    weights, fixtures = tmp_path / "w.opwpack", tmp_path / "fx.opwpack"
    pack_from_oracle(str(weights), cpu, TINY)
    ids = prompt(n, TINY["vocab_size"], SEED + n)
    write_fixtures(str(fixtures), cpu, ids, 16, 1e-4)
    run_exe(weights, fixtures)


def test_model_api_bf16(ow, tmp_path):
    from tests import oracle as orc
    cfg = dict(SMALL, num_hidden_layers=2, torch_dtype="bfloat16")
    cpu = orc.Llama(cfg, SEED + 1, 0.02, "uniform")
    weights, fixtures = tmp_path / "w.opwpack", tmp_path / "fx.opwpack"
    pack_from_oracle(str(weights), cpu, cfg, dtype="bfloat16")
    write_fixtures(str(fixtures), cpu, prompt(40, cfg["vocab_size"], SEED), 12, 1e-2)
    run_exe(weights, fixtures)
