/* C ABI of the Llama-3.x runtime in libopworks_amd.so.
 *
 * The first eleven entry points are the reference's exports with identical
 * signatures and semantics (src/llama_c_api.cu:54-159): no C++ exception crosses
 * the ABI; failures return NULL / -1 and copy the message (truncated to
 * err_len - 1, NUL-terminated) into `err` when it is non-NULL; the message of
 * the calling thread's last failure is also available from
 * opw_llama_last_error(). A session refers to its model: destroy sessions
 * before freeing the model. One host thread per session at a time.
 *
 * Packs of dtype float32 load the fp32 model, bfloat16 packs the bf16-weight
 * model (projections and embedding bf16, norms and activations fp32), as the
 * reference's loader dispatches (src/llama_c_api.cu:56-73).
 */
#ifndef OPWORKS_LLAMA_H
#define OPWORKS_LLAMA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Loads an OPWPACK1 weight pack (scripts/llama/pack_format.py layout). NULL on error. */
void *opw_llama_load(const char *pack_path, char *err, int err_len);
void opw_llama_free(void *model);
/* max_seq_len in (0, 8192] */
void *opw_llama_create_session(void *model, int max_seq_len, char *err, int err_len);
void opw_llama_destroy_session(void *session);
/* 0 / -1; only invalidates the cache length */
int opw_llama_reset_session(void *session, char *err, int err_len);
/* Runs the prompt on a fresh session; returns the first generated token id, -1 on error. */
int opw_llama_prefill(void *session, const int32_t *tokens, int n, char *err, int err_len);
/* Appends prev_token at position length; returns the next token id (greedy), -1 on error. */
int opw_llama_decode_step(void *session, int32_t prev_token, char *err, int err_len);
/* 1 if token is an end-of-sequence id of the model, 0 if not, -1 on error */
int opw_llama_is_eos(void *session, int32_t token, char *err, int err_len);
/* Copies the last position's logits; n must equal the vocabulary size. 0 / -1. */
int opw_llama_last_logits(void *session, float *out, int n, char *err, int err_len);
int opw_llama_vocab_size(void *session);
const char *opw_llama_last_error(void);

/* ---- additions (no counterpart in the reference's C ABI) ---- */

/* Builds a model from an HF-style config JSON object with seeded random
 * weights: every projection and the (tied) embedding ~ N(0, init_std) from the
 * counter-based generator of include/opworks_ops.h (per-tensor streams fixed
 * by the runtime), RMSNorm weights = 1 (norm_init 0) or U[0.5, 1.5]
 * (norm_init 1). "torch_dtype": "bfloat16" in the config selects bf16 weights
 * (each value rounded to nearest-even, norms included, as a bf16 pack stores
 * them). Replaces writing a multi-GB synthetic pack. NULL on error. */
void *opw_llama_load_random(const char *config_json, uint64_t seed, float init_std, int norm_init, char *err,
                            int err_len);
/* RoPE inverse frequencies (head_dim / 2 floats) the runtime derives from an
 * HF-style config JSON object, llama3 scaling included (ModelConfig::rope_inv_freq,
 * include/runtime/model_config.cuh:68-89). Host only, no device work. 0 / -1. */
int opw_llama_config_inv_freq(const char *config_json, float *out, int n, char *err, int err_len);
/* Model shape: out[0..6] = layers, hidden, intermediate, q heads, kv heads, head_dim, vocab. 0 / -1. */
int opw_llama_model_config(void *model, int *out7, char *err, int err_len);
/* Prefill that also returns the residual stream after the embedding and after
 * every layer (LlamaModelT::debug_prefill, include/models/llama.cuh:159-181):
 * captures receives (layers + 1) * n * hidden floats. Returns the first token, -1 on error. */
int opw_llama_debug_prefill(void *session, const int32_t *tokens, int n, float *captures, int64_t capacity,
                            char *err, int err_len);
/* Greedy generation on a fresh session, as examples/llama/generate.py:111-135
 * runs it with no EOS stop: out_tokens[0] is the prefill's token, then
 * max_new - 1 decode steps. The decode steps are chained on the device (each
 * step's argmax is the next step's input; the host waits once), with the same
 * tokens as max_new - 1 opw_llama_decode_step calls; the prompt plus max_new - 1
 * positions must fit the session. Wall times of the prefill and of the decode
 * steps are returned in milliseconds. Returns the number of tokens written, -1 on error. */
int opw_llama_generate_greedy(void *session, const int32_t *prompt, int n, int max_new, int32_t *out_tokens,
                              double *prefill_ms, double *decode_ms, char *err, int err_len);

/* One decode step (appends prev_token like opw_llama_decode_step) launched
 * eagerly with a HIP event before every kernel on the session stream;
 * kernel_ms receives each kernel's duration in launch order (per layer:
 * qkv+rope, attention, o_proj, gate/up, down; then the LM head). Returns the
 * number of kernels (5 * layers + 1), -1 on error. */
int opw_llama_profile_decode_step(void *session, int32_t prev_token, float *kernel_ms, int capacity, char *err,
                                  int err_len);
/* Average duration (microseconds) of one launch of a decode stage: 0 qkv_rope, 1 attention (partial +
 * combine), 2 o_proj, 3 gate_up, 4 down, 5 lm_head + argmax. The stage alone runs for every layer in
 * order, `reps` times, between two events on the session stream (consecutive launches stream different
 * layers' weights). Needs a prefilled session with free capacity; -1 on error. Timing aid, no
 * counterpart in the reference. */
float opw_llama_time_decode_stage(void *session, int stage, int reps, char *err, int err_len);

#ifdef __cplusplus
}
#endif

#endif /* OPWORKS_LLAMA_H */
