/* OpWorks CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's algorithms for the operator hot
 * path (Xavier-86/OpWorks, include/ops/ *.cuh and include/core/block_reduce.cuh),
 * in the reference's own evaluation order where that order is fixed by the
 * code. It is the checker for the HIP kernels: only tests/, the smoke() entry
 * point and bench.py's cpu_baseline leg may load it, and the product path
 * never calls it.
 *
 * Floating-point contraction: the reference is compiled by nvcc with
 * -fmad=true, which fuses a*b+c into an FMA. This file is compiled with
 * -ffp-contract=off and writes fmaf() exactly where that fusion is
 * unambiguous (noted per function); elsewhere results are compared within
 * the tolerances the tests state.
 *
 * Pinning (what checks each function; details in tests/test_oracle.py):
 *  orc_fill_*            bit-equality with the GPU generator + moments
 *  orc_map_scale_add     fmaf closed form; framework.cu KATs (Add, Scale)
 *  orc_reduce            brute-force double sum; framework.cu KATs (ones, empty
 *                        product); exact tree reproduced by hand on tiny inputs
 *  orc_softmax_rows      framework.cu:189-195 closed form; sum-to-one, shift
 *                        invariance
 *  orc_layer_norm_rows   framework.cu:196-199 closed form; zero mean / unit var
 *  orc_rms_norm_rows     closed form mean(out^2)=ms/(ms+eps) at gamma=1
 *  orc_mat_mul_rows      framework.cu:201-221 integer KAT (exact), zero-K case,
 *                        float64 matmul bound, numpy reference on small shapes
 *  orc_gemv              float64 dot bound; agrees with orc_mat_mul_rows
 *  orc_round_bf16        hand-computed bit patterns incl. ties to even
 *  orc_attention_explicit  float64 softmax-attention on small shapes; one-key
 *                        rows return v_0 exactly; uniform keys average V
 *  orc_attention_decode  equals the explicit path's last row (same maths,
 *                        other order) and the float64 reference
 *  orc_linear            agrees with orc_mat_mul_rows (same chain) / orc_gemv
 *  orc_linear_exact      within 1 ulp of the exact sum (math.fsum of the float64
 *                        products, rounded once) on bf16-valued inputs, and
 *                        bit-equal to it for all but a rare near-halfway few
 *  orc_rope_inv_freq     closed form without scaling; llama3 bands by hand;
 *                        the reference's own model_config.cuh via oracle/_ref
 *  orc_rope              position 0 is the identity; pair norms preserved
 *  orc_argmax            brute force incl. ties, -inf and NaN
 *  orc_swiglu            zeros at g = 0 and u = 0; silu(g) - silu(-g) = g;
 *                        silu(g) -> g for large g and -> 0 for very negative g;
 *                        float64 formula within 4 ulp
 *  orc_causal_scale      visible count of row r is cols - rows + r + 1; each
 *                        visible value equals the fp32 product x * scale
 *  orc_llama_*           float64 numpy forward of a tiny model; KV-cache
 *                        decode equals full recompute
 *  orc_scan              closed forms (ones -> i + 1, integers -> triangular
 *                        numbers, both exact in fp32), exclusive = inclusive
 *                        shifted, float64 numpy cumsum, running max of
 *                        monotone and random inputs vs numpy maximum.accumulate
 *  orc_transpose         numpy .T on ragged shapes; transposing twice is the
 *                        identity
 *  orc_gather/scatter    numpy fancy indexing; scatter of a permutation is its
 *                        inverse gather; out-of-range indices by hand
 *  orc_llama_set_bf16    weights equal their bf16 rounding (bit patterns);
 *                        the >= 16-row projection equals orc_linear_exact on
 *                        bf16-rounded inputs; float64 forward of a tiny model
 */
#ifndef OPWORKS_ORACLE_H
#define OPWORKS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* worker threads used by the *_mt entry points (default 1) */
void orc_set_threads(int n);
int orc_get_threads(void);

/* seeded synthetic data, restating opworks_amd/include/core/random.hpp */
uint64_t orc_stream_key(uint64_t seed, uint64_t stream);
void orc_fill_uniform(float *dst, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi);
void orc_fill_normal(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd);
void orc_fill_uniform_mt(float *dst, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi);
void orc_fill_normal_mt(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd);

/* map */
void orc_map_scale_add(const float *a, const float *b, float *out, int64_t n, float alpha);
void orc_map_scale_add_mt(const float *a, const float *b, float *out, int64_t n, float alpha);

/* block_reduce<Op> of `nthreads` per-thread values (thread 0's result). op: 0 sum, 1 max, 2 product */
float orc_block_reduce(const float *vals, int nthreads, int op);
/* ops::reduce<Op> in the reference's launch geometry and order */
float orc_reduce(const float *in, int n, int op);
double orc_sum_f64(const float *in, int64_t n);
double orc_sum_abs_f64(const float *in, int64_t n);

/* row kernels, one reference "block" of 256 threads per row */
void orc_softmax_rows(const float *in, float *out, int rows, int cols);
void orc_layer_norm_rows(const float *in, float *out, const float *gamma, const float *beta, int rows, int cols,
                         float eps);
void orc_rms_norm_rows(const float *x, const float *w, float *out, int rows, int cols, float eps);

/* GEMM in reference names (A: M x N, B: N x K or K x N when b_transposed); see oracle.c */
void orc_mat_mul_rows(const float *A, const float *B, const float *bias, float *out, double *absdot, int M, int N,
                      int K, const int *rows, int nrows, int b_transposed, int act);
/* reference GEMV (rows == 1 path of ops::linear): y[out] = W[out][in] . x */
void orc_gemv(const float *x, const float *W, float *y, int in, int out);

/* fp32 -> bf16 round-to-nearest-even (bits and/or the rounded float) */
void orc_round_bf16(const float *in, float *out, uint16_t *bits, int64_t n);

/* attention (layouts of include/ops/attention_prefill.cuh:21-24) */
void orc_attention_explicit(const float *q, const float *k, const float *v, float *out, double *bound, int T, int S,
                            int qh, int kv_rep, int D, int cap, const int *rows, int nrows);
void orc_attention_decode(const float *q, const float *k, const float *v, float *out, int qh, int kv_rep, int D,
                          int len, int max_seq);

/* Llama forward (include/models/llama.cuh:216-285) on seeded random weights */
void orc_linear(const float *X, const float *W, float *Y, int rows, int in, int out);
/* the bf16 tensor-core projection: products summed in double, rounded once to fp32 */
void orc_linear_exact(const float *X, const float *W, float *Y, int rows, int in, int out);
void orc_rope_inv_freq(int head_dim, float theta, int llama3, float factor, float low, float high, int orig,
                       float *out);
void orc_rope(float *x, const float *inv_freq, int rows, int heads, int head_dim, int pos_start);
int orc_argmax(const float *x, int n);
void orc_swiglu(const float *gate, const float *up, float *out, int64_t n);
void orc_causal_scale(float *scores, int rows, int cols, float scale);
void *orc_llama_create(int L, int H, int I, int qh, int kvh, int D, int V, float eps, float theta, int llama3,
                       float factor, float low, float high, int orig, uint64_t seed, float sd, int norm_uniform);
void orc_llama_destroy(void *m);
const float *orc_llama_weight(void *m, int kind, int layer);
void orc_llama_reset(void *m, int cap);
int orc_llama_prefill(void *m, const int *ids, int n, float *logits, float *captures);
int orc_llama_decode(void *m, int token, float *logits);
void orc_llama_set_bf16(void *p);

/* Kernels behind the Scan / Transform / GatherScatter builders. The reference defines
 * only their metadata (include/builders/scan.cuh:7-17, transform.cuh:7-18,
 * gather_scatter.cuh:7-19); these state the meaning this build gives it. */
/* op 0: prefix sum, the exact float64 running sum rounded to float per element;
 * op 1: fmaxf fold from -inf. inclusive 0 shifts by one (out[0] = identity).
 * abs_prefix (may be NULL) receives the float64 running sum of |x| over the same
 * range, the scale of the tests' error bound. */
void orc_scan(const float *in, float *out, double *abs_prefix, int64_t n, int op, int inclusive);
/* out [cols][rows] = in [rows][cols] transposed */
void orc_transpose(const float *in, float *out, int rows, int cols);
/* out[i] = in[idx[i]], NaN for an index outside [0, in_size) */
void orc_gather(const float *in, int64_t in_size, const int *idx, float *out, int64_t count);
/* out[idx[i]] = in[i] for indices inside [0, out_size), in increasing i */
void orc_scatter(const float *in, const int *idx, float *out, int64_t out_size, int64_t count);

#ifdef __cplusplus
}
#endif

#endif
