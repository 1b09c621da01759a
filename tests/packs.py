"""Writer of OPWPACK1 weight packs for tests, following the format the
reference documents in scripts/llama/pack_format.py:1-17:
[8 B "OPWPACK1"][u64 LE manifest length][JSON manifest][blob, 64-B aligned tensors]."""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = b"OPWPACK1"


def write_pack(path, tensors: dict, aliases: dict | None = None, extra: dict | None = None, dtype="float32"):
    manifest = {"format_version": 1, "dtype": dtype, "tensors": {}}
    if aliases:
        manifest["aliases"] = aliases
    if extra:
        manifest.update(extra)
    blobs, offset = [], 0
    for name, arr in tensors.items():
        raw = np.ascontiguousarray(arr, np.float32 if dtype == "float32" else np.uint16).tobytes()
        manifest["tensors"][name] = {"offset": offset, "shape": list(np.shape(arr))}
        pad = (-len(raw)) % 64
        blobs.append(raw + b"\0" * pad)
        offset += len(raw) + pad
    js = json.dumps(manifest, sort_keys=True).encode()
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        for b in blobs:
            f.write(b)


def pack_from_oracle(path, model, cfg: dict, dtype: str = "float32", overrides: dict | None = None):
    """Writes the oracle model's seeded weights as an HF-named pack (tied LM head alias);
    dtype "bfloat16" stores every tensor as bf16 bits (the oracle's weights must
    already be bf16 values, e.g. a bf16 oracle model). `overrides` replaces tensors
    by HF name before they are written."""
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    qh, kvh = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg.get("head_dim", H // qh)
    t = {"model.embed_tokens.weight": model.weight(0, 0, V * H).reshape(V, H),
         "model.norm.weight": model.weight(1, 0, H)}
    for l in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{l}."
        t[p + "self_attn.q_proj.weight"] = model.weight(2, l, qh * D * H).reshape(qh * D, H)
        t[p + "self_attn.k_proj.weight"] = model.weight(3, l, kvh * D * H).reshape(kvh * D, H)
        t[p + "self_attn.v_proj.weight"] = model.weight(4, l, kvh * D * H).reshape(kvh * D, H)
        t[p + "self_attn.o_proj.weight"] = model.weight(5, l, H * qh * D).reshape(H, qh * D)
        t[p + "mlp.gate_proj.weight"] = model.weight(6, l, I * H).reshape(I, H)
        t[p + "mlp.up_proj.weight"] = model.weight(7, l, I * H).reshape(I, H)
        t[p + "mlp.down_proj.weight"] = model.weight(8, l, H * I).reshape(H, I)
        t[p + "input_layernorm.weight"] = model.weight(9, l, H)
        t[p + "post_attention_layernorm.weight"] = model.weight(10, l, H)
    for k, v in (overrides or {}).items():
        assert k in t and np.shape(v) == np.shape(t[k]), k
        t[k] = v
    if dtype == "bfloat16":
        for k, v in t.items():
            bits = np.ascontiguousarray(v, np.float32).view(np.uint32)
            assert np.all(bits & 0xFFFF == 0), k  # exact bf16 values
            t[k] = (bits >> 16).astype(np.uint16)
    hf = {k: v for k, v in cfg.items() if k != "eos_token_id"}
    write_pack(path, t, aliases={"lm_head.weight": "model.embed_tokens.weight"},
               extra={"config": hf, "eos_token_ids": cfg.get("eos_token_id", [])}, dtype=dtype)
