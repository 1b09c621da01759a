"""CPU: the oracle and the product's host config code against the committed
golden fixtures (tests/golden/, written by make_golden.py from the reference's
own host code and unit-test known answers)."""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def rope_cases():
    return json.loads((GOLDEN / "rope_inv_freq.json").read_text())["cases"]


def kats():
    return json.loads((GOLDEN / "framework_kats.json").read_text())


@pytest.mark.parametrize("case", rope_cases(), ids=lambda c: c["name"])
def test_oracle_inv_freq_bitwise_equal_to_reference(orc, case):
    cfg = case["config"]
    want = np.array([int(b, 16) for b in case["inv_freq_bits"]], np.uint32).view(np.float32)
    rs = cfg.get("rope_scaling") or {}
    got = orc.rope_inv_freq(cfg["head_dim"], cfg["rope_theta"], bool(rs), rs.get("factor", 0.0),
                            rs.get("low_freq_factor", 0.0), rs.get("high_freq_factor", 0.0),
                            rs.get("original_max_position_embeddings", 0))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", rope_cases(), ids=lambda c: c["name"])
def test_runtime_inv_freq_bitwise_equal_to_reference(ow, case):
    """The product's host ModelConfig (no device work) derives the same floats."""
    lib = ow.lib()
    fn = lib.opw_llama_config_inv_freq
    fn.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
    fn.restype = ctypes.c_int
    want = np.array([int(b, 16) for b in case["inv_freq_bits"]], np.uint32)
    out = np.empty(want.size, np.float32)
    err = ctypes.create_string_buffer(256)
    assert fn(json.dumps(case["config"]).encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out.size,
              err, 256) == 0, err.value
    assert np.array_equal(out.view(np.uint32), want)


def test_oracle_framework_kats(orc):
    k = kats()
    close = lambda a, e: np.all(np.abs(np.asarray(a, np.float64) - np.asarray(e)) <= 1e-5 * (1 + np.abs(e)))
    a, b = np.array(k["add"]["a"], np.float32), np.array(k["add"]["b"], np.float32)
    assert np.array_equal(orc.map_scale_add(a, b, 1.0), np.array(k["add"]["out"], np.float32))
    x = np.array(k["scale3"]["x"], np.float32)
    assert np.array_equal(orc.map_scale_add(x, np.zeros(3, np.float32), 3.0), np.array(k["scale3"]["out"]))
    for n in k["sum_of_ones"]["n"]:
        assert orc.reduce(np.ones(n, np.float32), "sum") == n
    assert orc.reduce(np.zeros(0, np.float32), "product") == k["empty_product"]["out"]
    sm = k["softmax_2x5"]
    assert close(orc.softmax_rows(np.array(sm["x"], np.float32), 2, 5), sm["out"])
    ln = k["layer_norm_2x5"]
    g = np.full(5, ln["gamma"], np.float32)
    bt = np.full(5, ln["beta"], np.float32)
    assert close(orc.layer_norm_rows(np.array(ln["x"], np.float32), g, bt, 2, 5, ln["eps"]), ln["out"])
    mm = k["mat_mul_3x5x7_scale2"]
    out, _ = orc.mat_mul_rows(np.array(mm["a"], np.float32), np.array(mm["b"], np.float32), mm["M"], mm["N"], mm["K"])
    assert np.array_equal(2 * out.ravel(), np.array(mm["out"], np.float32))
