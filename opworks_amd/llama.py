"""ctypes binding of the opw_llama_* C ABI (include/opworks_llama.h).

Mirrors the reference's Python driver (examples/llama/generate.py:23-61): a
model handle, sessions, prefill / decode_step / last_logits, errors raised
from the ABI's message."""
from __future__ import annotations

import ctypes
import json
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint64, c_void_p
from typing import Optional, Sequence

import numpy as np

from . import OpworksError, declare, lib

_ERR_LEN = 1024

for _name, _res, _args in [
    ("opw_llama_load", c_void_p, [c_char_p, c_char_p, c_int]),
    ("opw_llama_free", None, [c_void_p]),
    ("opw_llama_create_session", c_void_p, [c_void_p, c_int, c_char_p, c_int]),
    ("opw_llama_destroy_session", None, [c_void_p]),
    ("opw_llama_reset_session", c_int, [c_void_p, c_char_p, c_int]),
    ("opw_llama_prefill", c_int, [c_void_p, POINTER(c_int32), c_int, c_char_p, c_int]),
    ("opw_llama_decode_step", c_int, [c_void_p, c_int32, c_char_p, c_int]),
    ("opw_llama_is_eos", c_int, [c_void_p, c_int32, c_char_p, c_int]),
    ("opw_llama_last_logits", c_int, [c_void_p, POINTER(c_float), c_int, c_char_p, c_int]),
    ("opw_llama_vocab_size", c_int, [c_void_p]),
    ("opw_llama_last_error", c_char_p, []),
    ("opw_llama_load_random", c_void_p, [c_char_p, c_uint64, c_float, c_int, c_char_p, c_int]),
    ("opw_llama_model_config", c_int, [c_void_p, POINTER(c_int), c_char_p, c_int]),
    ("opw_llama_debug_prefill", c_int, [c_void_p, POINTER(c_int32), c_int, POINTER(c_float), c_int64, c_char_p,
                                        c_int]),
    ("opw_llama_profile_decode_step", c_int, [c_void_p, c_int32, POINTER(c_float), c_int, c_char_p, c_int]),
    ("opw_llama_time_decode_stage", c_float, [c_void_p, c_int, c_int, c_char_p, c_int]),
    ("opw_llama_generate_greedy", c_int, [c_void_p, POINTER(c_int32), c_int, c_int, POINTER(c_int32),
                                          POINTER(c_double), POINTER(c_double), c_char_p, c_int]),
]:
    declare(_name, _res, _args)

LLAMA_3_2_1B = {
    "num_hidden_layers": 16, "hidden_size": 2048, "intermediate_size": 8192, "num_attention_heads": 32,
    "num_key_value_heads": 8, "head_dim": 64, "vocab_size": 128256, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
    "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                     "original_max_position_embeddings": 8192},
    "eos_token_id": [128001, 128008, 128009],
}


def _ids(tokens: Sequence[int]):
    arr = np.ascontiguousarray(tokens, dtype=np.int32)
    return arr, arr.ctypes.data_as(POINTER(c_int32))


class LlamaModel:
    def __init__(self, handle: int) -> None:
        self.handle = handle
        cfg = (c_int * 7)()
        err = ctypes.create_string_buffer(_ERR_LEN)
        if lib().opw_llama_model_config(handle, cfg, err, _ERR_LEN) != 0:
            raise OpworksError(err.value.decode())
        (self.num_layers, self.hidden_size, self.intermediate_size, self.num_q_heads, self.num_kv_heads,
         self.head_dim, self.vocab_size) = list(cfg)

    @classmethod
    def load(cls, pack_path: str) -> "LlamaModel":
        err = ctypes.create_string_buffer(_ERR_LEN)
        h = lib().opw_llama_load(pack_path.encode(), err, _ERR_LEN)
        if not h:
            raise OpworksError(err.value.decode())
        return cls(h)

    @classmethod
    def load_random(cls, config: dict, seed: int, init_std: float = 0.02, norm_init: str = "ones") -> "LlamaModel":
        err = ctypes.create_string_buffer(_ERR_LEN)
        h = lib().opw_llama_load_random(json.dumps(config).encode(), seed, init_std,
                                        {"ones": 0, "uniform": 1}[norm_init], err, _ERR_LEN)
        if not h:
            raise OpworksError(err.value.decode())
        return cls(h)

    def session(self, max_seq_len: int) -> "LlamaSession":
        return LlamaSession(self, max_seq_len)

    def free(self) -> None:
        if self.handle:
            lib().opw_llama_free(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


class LlamaSession:
    def __init__(self, model: LlamaModel, max_seq_len: int) -> None:
        err = ctypes.create_string_buffer(_ERR_LEN)
        h = lib().opw_llama_create_session(model.handle, max_seq_len, err, _ERR_LEN)
        if not h:
            raise OpworksError(err.value.decode())
        self.model = model  # sessions keep their model alive
        self.handle = h
        self.max_seq_len = max_seq_len
        self._err = err

    def _check(self, rc: int) -> int:
        if rc < 0:
            raise OpworksError(self._err.value.decode())
        return rc

    def reset(self) -> None:
        self._check(lib().opw_llama_reset_session(self.handle, self._err, _ERR_LEN))

    def prefill(self, tokens: Sequence[int]) -> int:
        arr, p = _ids(tokens)
        return self._check(lib().opw_llama_prefill(self.handle, p, arr.size, self._err, _ERR_LEN))

    def decode_step(self, prev_token: int) -> int:
        return self._check(lib().opw_llama_decode_step(self.handle, prev_token, self._err, _ERR_LEN))

    def is_eos(self, token: int) -> bool:
        return bool(self._check(lib().opw_llama_is_eos(self.handle, token, self._err, _ERR_LEN)))

    def last_logits(self) -> np.ndarray:
        out = np.empty(self.model.vocab_size, np.float32)
        self._check(lib().opw_llama_last_logits(self.handle, out.ctypes.data_as(POINTER(c_float)), out.size,
                                                self._err, _ERR_LEN))
        return out

    def debug_prefill(self, tokens: Sequence[int]):
        arr, p = _ids(tokens)
        m = self.model
        caps = np.empty((m.num_layers + 1) * arr.size * m.hidden_size, np.float32)
        tok = self._check(lib().opw_llama_debug_prefill(self.handle, p, arr.size,
                                                        caps.ctypes.data_as(POINTER(c_float)), caps.size, self._err,
                                                        _ERR_LEN))
        return tok, caps.reshape(m.num_layers + 1, arr.size, m.hidden_size)

    def generate_greedy(self, prompt: Sequence[int], max_new: int):
        """Returns (tokens, prefill_ms, decode_ms)."""
        arr, p = _ids(prompt)
        out = np.empty(max_new, np.int32)
        pre, dec = c_double(0), c_double(0)
        self._check(lib().opw_llama_generate_greedy(self.handle, p, arr.size, max_new,
                                                    out.ctypes.data_as(POINTER(c_int32)), ctypes.byref(pre),
                                                    ctypes.byref(dec), self._err, _ERR_LEN))
        return out, pre.value, dec.value

    def generate(self, prompt: Sequence[int], max_new_tokens: int, temperature: float = 0.0, top_p: float = 1.0,
                 seed: Optional[int] = None) -> list:
        """Host generation loop with the reference generator's contract
        (examples/llama/generate.py:111-135): greedy when temperature == 0,
        else temperature / nucleus sampling of the last logits on the host;
        stops after an end-of-sequence token or when the next input position
        would exceed the session capacity."""
        if len(prompt) + max_new_tokens > self.max_seq_len:
            raise ValueError(f"prompt ({len(prompt)}) + max_new_tokens ({max_new_tokens}) exceeds capacity "
                             f"{self.max_seq_len}")
        rng = np.random.default_rng(seed) if temperature > 0.0 else None
        self.reset()
        greedy = self.prefill(prompt)
        out = []
        for _ in range(max_new_tokens):
            tok = sample_top_p(self.last_logits(), rng, temperature, top_p) if rng is not None else greedy
            out.append(tok)
            if self.is_eos(tok):
                break
            if len(prompt) + len(out) >= self.max_seq_len and len(out) < max_new_tokens:
                break
            greedy = self.decode_step(tok)
        return out

    KERNELS_PER_LAYER = ("qkv_rope", "attention", "o_proj", "gate_up", "down")

    def profile_decode_step(self, prev_token: int):
        """Returns ({kernel name: [ms per layer]} + {"lm_head": [ms]}) for one eager decode step."""
        m = self.model
        n = 5 * m.num_layers + 1
        ms = np.empty(n, np.float32)
        self._check(lib().opw_llama_profile_decode_step(self.handle, prev_token, ms.ctypes.data_as(POINTER(c_float)),
                                                        n, self._err, _ERR_LEN))
        out = {k: [float(ms[5 * l + i]) for l in range(m.num_layers)] for i, k in enumerate(self.KERNELS_PER_LAYER)}
        out["lm_head"] = [float(ms[-1])]
        return out

    STAGES = ("qkv_rope", "attention", "o_proj", "gate_up", "down", "lm_head")

    def time_decode_stage(self, stage: str, reps: int = 10) -> float:
        """Average microseconds per launch of one decode stage, launched back to back over all layers."""
        us = lib().opw_llama_time_decode_stage(self.handle, self.STAGES.index(stage), reps, self._err, _ERR_LEN)
        if us < 0:
            raise OpworksError(self._err.value.decode(errors="replace"))
        return float(us)

    def close(self) -> None:
        if self.handle:
            lib().opw_llama_destroy_session(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def sample_top_p(logits: np.ndarray, rng: np.random.Generator, temperature: float = 1.0, top_p: float = 1.0) -> int:
    """One token from softmax(logits / temperature) restricted to the nucleus:
    tokens in descending probability while the running sum stays <= top_p,
    plus the token whose probability crosses top_p and always the most likely
    token, renormalised (the reference's host sampler, examples/llama/generate.py:83-109)."""
    z = np.asarray(logits, np.float64) / max(temperature, 1e-6)
    p = np.exp(z - z.max())
    p /= p.sum()
    if top_p < 1.0:
        order = np.argsort(p)[::-1]
        csum = np.cumsum(p[order])
        kept = csum <= top_p
        kept[0] = True
        first_over = int(np.searchsorted(csum, top_p))
        if first_over < kept.size:
            kept[first_over] = True
        q = np.zeros_like(p)
        q[order[kept]] = p[order[kept]]
        p = q / q.sum()
    return int(rng.choice(p.size, p=p))
