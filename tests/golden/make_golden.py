"""Writes the golden fixtures of this directory (run in the build container,
where /root/reference exists; the fixtures then travel without it).

rope_inv_freq.json
    RoPE inverse frequencies produced by the reference's own host code
    (include/runtime/model_config.cuh:68-89, compiled from its sources into
    oracle/_ref/libref_host.so by oracle/ref_host.mk) for several configs.
    Values are stored as float32 bit patterns.

framework_kats.json
    The known answers of the reference's unit test tests/unit/framework.cu
    (inputs and expected outputs as the test states them), as data.

    python tests/golden/make_golden.py
"""
import ctypes
import json
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent

ROPE_CASES = [
    # name, head_dim, theta, rope_scaling (None = plain RoPE)
    ("llama3.2-1b", 64, 500000.0, {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                   "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}),
    ("llama3.1-8b", 128, 500000.0, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                    "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}),
    ("plain-theta1e4-d64", 64, 10000.0, None),
    ("plain-theta5e5-d32", 32, 500000.0, None),
]


def rope_config(head_dim, theta, scaling):
    heads = 4
    cfg = {"num_hidden_layers": 1, "hidden_size": heads * head_dim, "intermediate_size": 4 * heads * head_dim,
           "num_attention_heads": heads, "num_key_value_heads": 2, "head_dim": head_dim, "vocab_size": 256,
           "rms_norm_eps": 1e-5, "rope_theta": theta, "tie_word_embeddings": True}
    if scaling:
        cfg["rope_scaling"] = scaling
    return cfg


def make_rope():
    lib = ctypes.CDLL(str(ROOT / "oracle" / "_ref" / "libref_host.so"))
    lib.ref_rope_inv_freq.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int]
    lib.ref_rope_inv_freq.restype = ctypes.c_int
    cases = []
    for name, d, theta, scaling in ROPE_CASES:
        cfg = rope_config(d, theta, scaling)
        out = np.empty(d // 2, np.float32)
        manifest = json.dumps({"config": cfg, "eos_token_ids": [1]}).encode()
        assert lib.ref_rope_inv_freq(manifest, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), d // 2) == 0, name
        cases.append({"name": name, "config": cfg, "inv_freq_bits": [f"{b:08x}" for b in out.view(np.uint32)]})
    return {"source": "reference include/runtime/model_config.cuh:68-89 via oracle/_ref/libref_host.so",
            "cases": cases}


def make_kats():
    ha = [float(i % 7 - 3) for i in range(15)]
    hb = [float(i % 5 - 2) for i in range(35)]
    mm = [[2 * sum(ha[r * 5 + k] * hb[k * 7 + c] for k in range(5)) for c in range(7)] for r in range(3)]
    den = sum(math.exp(j - 4) for j in range(5))
    bias = [-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0]
    return {
        "source": "reference tests/unit/framework.cu",
        "add": {"a": [1, 2, 3], "b": [4, 5, 6], "out": [5, 7, 9], "line": "framework.cu:73-75"},
        "scale3": {"x": [1, 2, 3], "out": [3, 6, 9], "line": "framework.cu:76-78"},
        "sum_of_ones": {"n": [0, 1, 31, 32, 33, 255, 256, 257, 4099], "line": "framework.cu:144-149"},
        "empty_product": {"out": 1.0, "line": "framework.cu:80"},
        "graph_replays": {"n": 4099, "after_first": 8198, "after_second": 16396, "line": "framework.cu:154-169"},
        "softmax_2x5": {"x": [-2, -1, 0, 1, 2, 3, 4, 5, 6, 7],
                        "out": [math.exp(i % 5 - 4) / den for i in range(10)], "line": "framework.cu:189-195"},
        "layer_norm_2x5": {"x": [-2, -1, 0, 1, 2, 3, 4, 5, 6, 7], "gamma": 2.0, "beta": 1.0, "eps": 1e-5,
                           "out": [(i % 5 - 2) * 2.0 / math.sqrt(2.0 + 1e-5) + 1 for i in range(10)],
                           "line": "framework.cu:196-199"},
        "mat_mul_3x5x7_scale2": {"a": ha, "b": hb, "M": 3, "N": 5, "K": 7, "out": [v for row in mm for v in row],
                                 "line": "framework.cu:201-218"},
        "mat_mul_zero_inner": {"M": 3, "N": 0, "K": 7, "out": 0.0, "line": "framework.cu:219-221"},
        "elementwise_boundaries": {"n": [1, 2, 3, 4, 5, 31, 32, 33, 255, 256, 257, 1025], "offsets": [0, 1],
                                   "value": "i - 10", "add_same": 2.0, "scale_in_place": 3.0,
                                   "line": "framework.cu:109-129"},
        "builder_relu_bias": {"a": ha, "b": hb, "M": 3, "N": 5, "K": 7, "bias": bias,
                              "out": [max(mm[r][c] / 2 + bias[c], 0.0) for r in range(3) for c in range(7)],
                              "line": "addition: MatmulBuilder.run() on the framework.cu:201-218 operands"},
        "tolerance": {"rule": "|a - e| <= 1e-5 * (1 + |e|)", "line": "framework.cu:45-48"},
    }


def main():
    (HERE / "rope_inv_freq.json").write_text(json.dumps(make_rope(), indent=1) + "\n")
    (HERE / "framework_kats.json").write_text(json.dumps(make_kats(), indent=1) + "\n")
    print("wrote", HERE / "rope_inv_freq.json", HERE / "framework_kats.json")


if __name__ == "__main__":
    main()
