/* OpWorks CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define REF_THREADS 256   /* kThreads, include/core/config.cuh:15-17,56 */
#define REF_WARP 32       /* kWarpSize, include/core/config.cuh:46 */
#define REF_MAX_PARTIALS 1024 /* kMaxThreadsPerBlock, include/core/config.cuh:47 */

/* ------------------------------------------------------------------ threads */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }

typedef void (*range_fn)(void *ctx, int64_t begin, int64_t end);
struct range_job {
    range_fn fn;
    void *ctx;
    int64_t begin, end;
};
static void *range_worker(void *p) {
    struct range_job *j = (struct range_job *)p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}
/* Splits [0, n) into g_threads contiguous chunks. */
static void parallel_for(int64_t n, range_fn fn, void *ctx) {
    int t = g_threads;
    if (t <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (t > n)
        t = (int)n;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * t);
    struct range_job *jobs = (struct range_job *)malloc(sizeof(struct range_job) * t);
    for (int i = 0; i < t; ++i) {
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].begin = n * i / t;
        jobs[i].end = n * (i + 1) / t;
        pthread_create(&th[i], NULL, range_worker, &jobs[i]);
    }
    for (int i = 0; i < t; ++i)
        pthread_join(th[i], NULL);
    free(th);
    free(jobs);
}

/* ---------------------------------------------------------------------- rng */
static const uint64_t kGolden = 0x9E3779B97F4A7C15ull;
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t orc_stream_key(uint64_t seed, uint64_t stream) { return mix64(seed ^ mix64(stream + kGolden)); }
static uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

void orc_fill_uniform(float *dst, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi) {
    const uint64_t key = orc_stream_key(seed, stream);
    for (int64_t i = 0; i < n; ++i) {
        const float u = (float)(uint32_t)(draw(key, (uint64_t)i) >> 40) * 0x1p-24f;
        dst[i] = fmaf(u, hi - lo, lo);
    }
}

void orc_fill_normal(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd) {
    const uint64_t key = orc_stream_key(seed, stream);
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t a = draw(key, 2 * (uint64_t)i), b = draw(key, 2 * (uint64_t)i + 1);
        const int32_t s = (int32_t)(a >> 40) + (int32_t)((a >> 16) & 0xFFFFFFu) + (int32_t)(b >> 40) +
                          (int32_t)((b >> 16) & 0xFFFFFFu) - (1 << 25);
        const float z = (float)s * 0x1.bb67aep-24f;
        dst[i] = fmaf(z, sd, mean);
    }
}

struct fill_ctx {
    float *dst;
    uint64_t seed, stream;
    float p0, p1;
    int normal;
};
/* The generators are counter-based, so a chunk [lo, hi) is filled independently. */
static void fill_range(void *p, int64_t lo, int64_t hi) {
    struct fill_ctx *c = (struct fill_ctx *)p;
    const uint64_t key = orc_stream_key(c->seed, c->stream);
    for (int64_t i = lo; i < hi; ++i) {
        if (c->normal) {
            const uint64_t a = draw(key, 2 * (uint64_t)i), b = draw(key, 2 * (uint64_t)i + 1);
            const int32_t s = (int32_t)(a >> 40) + (int32_t)((a >> 16) & 0xFFFFFFu) + (int32_t)(b >> 40) +
                              (int32_t)((b >> 16) & 0xFFFFFFu) - (1 << 25);
            c->dst[i] = fmaf((float)s * 0x1.bb67aep-24f, c->p1, c->p0);
        } else {
            const float u = (float)(uint32_t)(draw(key, (uint64_t)i) >> 40) * 0x1p-24f;
            c->dst[i] = fmaf(u, c->p1 - c->p0, c->p0);
        }
    }
}
void orc_fill_uniform_mt(float *dst, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi) {
    struct fill_ctx c = {dst, seed, stream, lo, hi, 0};
    parallel_for(n, fill_range, &c);
}
void orc_fill_normal_mt(float *dst, int64_t n, uint64_t seed, uint64_t stream, float mean, float sd) {
    struct fill_ctx c = {dst, seed, stream, mean, sd, 1};
    parallel_for(n, fill_range, &c);
}

/* ---------------------------------------------------------------------- map */
/* README.md:78-83 ScaleAdd `alpha * a + b`; nvcc contracts it to one FMA, and
 * ops::map applies the functor per element (include/ops/elementwise.cuh:20-35). */
void orc_map_scale_add(const float *a, const float *b, float *out, int64_t n, float alpha) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = fmaf(alpha, a[i], b[i]);
}
struct map_ctx {
    const float *a, *b;
    float *out;
    float alpha;
};
static void map_range(void *p, int64_t lo, int64_t hi) {
    struct map_ctx *c = (struct map_ctx *)p;
    orc_map_scale_add(c->a + lo, c->b + lo, c->out + lo, hi - lo, c->alpha);
}
void orc_map_scale_add_mt(const float *a, const float *b, float *out, int64_t n, float alpha) {
    struct map_ctx c = {a, b, out, alpha};
    parallel_for(n, map_range, &c);
}

/* ------------------------------------------------------------------- reduce */
static float combine(int op, float a, float b) {
    switch (op) {
    case 0: return a + b;
    case 1: return fmaxf(a, b);
    default: return a * b;
    }
}
static float identity(int op) { return op == 0 ? 0.f : (op == 1 ? -INFINITY : 1.f); }

/* One 32-lane __shfl_down_sync tree (offsets 16..1); lanes whose source is
 * past the warp keep their own value (include/core/block_reduce.cuh:17-18). */
static float warp_tree(const float *lanes, int op) {
    float cur[REF_WARP], nxt[REF_WARP];
    memcpy(cur, lanes, sizeof(cur));
    for (int off = REF_WARP / 2; off > 0; off >>= 1) {
        for (int l = 0; l < REF_WARP; ++l)
            nxt[l] = combine(op, cur[l], l + off < REF_WARP ? cur[l + off] : cur[l]);
        memcpy(cur, nxt, sizeof(cur));
    }
    return cur[0];
}

/* block_reduce<Op> (include/core/block_reduce.cuh:11-31): warp trees, lane 0
 * of each warp to shared[warp], warp 0 re-reduces with missing warps = identity. */
float orc_block_reduce(const float *vals, int nthreads, int op) {
    const int nwarps = (nthreads + REF_WARP - 1) / REF_WARP;
    float shared[REF_MAX_PARTIALS / REF_WARP];
    for (int w = 0; w < nwarps; ++w)
        shared[w] = warp_tree(vals + w * REF_WARP, op);
    float lanes[REF_WARP];
    for (int l = 0; l < REF_WARP; ++l)
        lanes[l] = l < nwarps ? shared[l] : identity(op);
    return warp_tree(lanes, op);
}

/* reduce_partial_kernel (include/ops/reduction.cuh:9-17) for one block: each
 * thread combines in[g], in[g+stride], ... in ascending order, then block_reduce. */
static float partial_block(const float *in, int64_t n, int block, int grid, int op) {
    float acc[REF_THREADS];
    const int64_t stride = (int64_t)grid * REF_THREADS;
    for (int t = 0; t < REF_THREADS; ++t) {
        float a = identity(op);
        for (int64_t i = (int64_t)block * REF_THREADS + t; i < n; i += stride)
            a = combine(op, a, in[i]);
        acc[t] = a;
    }
    return orc_block_reduce(acc, REF_THREADS, op);
}

struct reduce_ctx {
    const float *in;
    float *partial;
    int n, blocks, op;
};
static void reduce_blocks_range(void *p, int64_t b0, int64_t b1) {
    struct reduce_ctx *c = (struct reduce_ctx *)p;
    for (int64_t b = b0; b < b1; ++b)
        c->partial[b] = partial_block(c->in, c->n, (int)b, c->blocks, c->op);
}

/* ops::reduce (include/ops/reduction.cuh:34-54): blocks = min(ceil(n/256), 1024);
 * one block writes the result directly; otherwise partials, then
 * reduce_final_kernel (:19-27) with one block of 256 threads. */
float orc_reduce(const float *in, int n, int op) {
    int blocks = n / REF_THREADS + (n % REF_THREADS != 0);
    if (blocks <= 1)
        return partial_block(in, n, 0, 1, op);
    if (blocks > REF_MAX_PARTIALS)
        blocks = REF_MAX_PARTIALS;
    float *partial = (float *)malloc(sizeof(float) * blocks);
    struct reduce_ctx c = {in, partial, n, blocks, op};
    parallel_for(blocks, reduce_blocks_range, &c); /* blocks are independent: any thread count, same partials */
    const float r = partial_block(partial, blocks, 0, 1, op);
    free(partial);
    return r;
}

double orc_sum_f64(const float *in, int64_t n) {
    double s = 0;
    for (int64_t i = 0; i < n; ++i)
        s += in[i];
    return s;
}
double orc_sum_abs_f64(const float *in, int64_t n) {
    double s = 0;
    for (int64_t i = 0; i < n; ++i)
        s += fabs((double)in[i]);
    return s;
}

/* --------------------------------------------------------------------- rows */
/* Per-thread strided partials of one row (OPWORKS_BLOCK_LOOP with 256 threads). */
#define ROW_THREADS REF_THREADS

/* softmax_rows_kernel (include/ops/softmax.cuh:10-29). */
static void softmax_row(const float *x, float *y, int cols) {
    float part[ROW_THREADS];
    for (int t = 0; t < ROW_THREADS; ++t) {
        float m = -INFINITY;
        for (int j = t; j < cols; j += ROW_THREADS)
            m = fmaxf(m, x[j]);
        part[t] = m;
    }
    const float mx = orc_block_reduce(part, ROW_THREADS, 1);
    for (int t = 0; t < ROW_THREADS; ++t) {
        float s = 0.f;
        for (int j = t; j < cols; j += ROW_THREADS)
            s += expf(x[j] - mx);
        part[t] = s;
    }
    const float sum = orc_block_reduce(part, ROW_THREADS, 0);
    for (int j = 0; j < cols; ++j)
        y[j] = expf(x[j] - mx) / sum;
}

/* layer_norm_kernel (include/ops/layer_norm.cuh:10-31); `d*d` accumulation and
 * the final `(x-mean)*rstd*gamma + beta` are FMA-contracted by nvcc. rsqrtf is
 * restated as 1/sqrtf (CUDA's rsqrtf is not reproduced). */
static void layer_norm_row(const float *x, float *y, const float *g, const float *b, int cols, float eps) {
    float part[ROW_THREADS];
    for (int t = 0; t < ROW_THREADS; ++t) {
        float s = 0.f;
        for (int j = t; j < cols; j += ROW_THREADS)
            s += x[j];
        part[t] = s;
    }
    const float mean = orc_block_reduce(part, ROW_THREADS, 0) / cols;
    for (int t = 0; t < ROW_THREADS; ++t) {
        float s = 0.f;
        for (int j = t; j < cols; j += ROW_THREADS) {
            const float d = x[j] - mean;
            s = fmaf(d, d, s);
        }
        part[t] = s;
    }
    const float rstd = 1.0f / sqrtf(orc_block_reduce(part, ROW_THREADS, 0) / cols + eps);
    for (int j = 0; j < cols; ++j)
        y[j] = fmaf((x[j] - mean) * rstd, g[j], b[j]);
}

/* rms_norm_kernel (include/ops/rms_norm.cuh:9-24); `v*v` accumulation is an FMA. */
static void rms_norm_row(const float *x, const float *w, float *y, int cols, float eps) {
    float part[ROW_THREADS];
    for (int t = 0; t < ROW_THREADS; ++t) {
        float s = 0.f;
        for (int j = t; j < cols; j += ROW_THREADS)
            s = fmaf(x[j], x[j], s);
        part[t] = s;
    }
    const float inv = 1.0f / sqrtf(orc_block_reduce(part, ROW_THREADS, 0) / cols + eps);
    for (int j = 0; j < cols; ++j)
        y[j] = x[j] * inv * w[j];
}

struct row_ctx {
    const float *in, *p0, *p1;
    float *out;
    int cols;
    float eps;
    int kind;
};
static void rows_range(void *p, int64_t lo, int64_t hi) {
    struct row_ctx *c = (struct row_ctx *)p;
    for (int64_t r = lo; r < hi; ++r) {
        const float *x = c->in + r * c->cols;
        float *y = c->out + r * c->cols;
        if (c->kind == 0)
            softmax_row(x, y, c->cols);
        else if (c->kind == 1)
            layer_norm_row(x, y, c->p0, c->p1, c->cols, c->eps);
        else
            rms_norm_row(x, c->p0, y, c->cols, c->eps);
    }
}

void orc_softmax_rows(const float *in, float *out, int rows, int cols) {
    struct row_ctx c = {in, NULL, NULL, out, cols, 0.f, 0};
    parallel_for(rows, rows_range, &c);
}
void orc_layer_norm_rows(const float *in, float *out, const float *gamma, const float *beta, int rows, int cols,
                         float eps) {
    struct row_ctx c = {in, gamma, beta, out, cols, eps, 1};
    parallel_for(rows, rows_range, &c);
}
void orc_rms_norm_rows(const float *x, const float *w, float *out, int rows, int cols, float eps) {
    struct row_ctx c = {x, w, NULL, out, cols, eps, 2};
    parallel_for(rows, rows_range, &c);
}

/* --------------------------------------------------------------------- gemm */
struct mm_ctx {
    const float *A, *B, *bias;
    float *out;
    double *absdot;
    int M, N, K, act;
    const int *rows;
};

static float apply_act(float v, int act) {
    if (act == 1)
        return fmaxf(v, 0.f);
    if (act == 2)
        return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    return v;
}

static void mm_range(void *p, int64_t lo, int64_t hi) {
    struct mm_ctx *c = (struct mm_ctx *)p;
    float *acc = (float *)malloc(sizeof(float) * (size_t)c->K);
    double *ab = (double *)malloc(sizeof(double) * (size_t)c->K);
    for (int64_t r = lo; r < hi; ++r) {
        const int i = c->rows ? c->rows[r] : (int)r;
        for (int j = 0; j < c->K; ++j) {
            acc[j] = 0.f;
            ab[j] = 0.0;
        }
        const float *arow = c->A + (int64_t)i * c->N;
        for (int n = 0; n < c->N; ++n) {
            const float a = arow[n];
            const float *brow = c->B + (int64_t)n * c->K;
            for (int j = 0; j < c->K; ++j) {
                acc[j] = fmaf(a, brow[j], acc[j]);
                ab[j] += fabs((double)a * (double)brow[j]);
            }
        }
        for (int j = 0; j < c->K; ++j) {
            const float v = c->bias ? acc[j] + c->bias[j] : acc[j];
            c->out[r * c->K + j] = apply_act(v, c->act);
            if (c->absdot)
                c->absdot[r * c->K + j] = ab[j] + (c->bias ? fabs((double)c->bias[j]) : 0.0);
        }
    }
    free(acc);
    free(ab);
}

/* ops::mat_mul (include/ops/matmul.cuh:11-66) in reference names: A is M x N,
 * B is N x K (or, with b_transposed, stored K x N), out rows are `rows[0..nrows)`
 * (all M rows when rows == NULL). Each output is the k-ascending chain
 * acc = fmaf(a, b, acc) over n = 0..N-1 (nvcc contracts `acc += a*b`), then
 * v = acc + bias[j] and the activation (0 none, 1 relu, 2 gelu-erf) — the
 * reference's PassThrough result followed by the host-side bias/ReLU that
 * MatmulBuilder describes. absdot (optional) receives sum_n |a*b| + |bias|. */
void orc_mat_mul_rows(const float *A, const float *B, const float *bias, float *out, double *absdot, int M, int N,
                      int K, const int *rows, int nrows, int b_transposed, int act) {
    float *bt = NULL;
    if (b_transposed) {
        bt = (float *)malloc(sizeof(float) * (size_t)N * (size_t)K);
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < K; ++j)
                bt[(int64_t)n * K + j] = B[(int64_t)j * N + n];
    }
    struct mm_ctx c = {A, bt ? bt : B, bias, out, absdot, M, N, K, act, rows};
    parallel_for(rows ? nrows : M, mm_range, &c);
    free(bt);
}

/* gemv_kernel (include/ops/linear.cuh:77-96): y[o] = block_reduce over 256
 * threads of per-thread partials; with in % 4 == 0 thread t accumulates
 * local += w.x*x.x + w.y*x.y + w.z*x.z + w.w*x.w over packs t, t+256, ...
 * The four products are restated as the FMA chain
 * fmaf(w.w,x.w, fmaf(w.z,x.z, fmaf(w.y,x.y, w.x*x.x))) followed by a plain add
 * into `local` (one admissible nvcc contraction; results are compared within
 * tolerance). Otherwise local = fmaf(x[i], w[i], local). */
struct gemv_ctx {
    const float *x, *W;
    float *y;
    int in;
};
static void gemv_range(void *p, int64_t lo, int64_t hi) {
    struct gemv_ctx *c = (struct gemv_ctx *)p;
    float part[REF_THREADS];
    for (int64_t o = lo; o < hi; ++o) {
        const float *w = c->W + o * c->in;
        for (int t = 0; t < REF_THREADS; ++t) {
            float local = 0.f;
            if (c->in % 4 == 0) {
                for (int i4 = t; i4 < c->in / 4; i4 += REF_THREADS) {
                    const float *wv = w + 4 * i4, *xv = c->x + 4 * i4;
                    const float dot = fmaf(wv[3], xv[3], fmaf(wv[2], xv[2], fmaf(wv[1], xv[1], wv[0] * xv[0])));
                    local = local + dot;
                }
            } else {
                for (int i = t; i < c->in; i += REF_THREADS)
                    local = fmaf(c->x[i], w[i], local);
            }
            part[t] = local;
        }
        c->y[o] = orc_block_reduce(part, REF_THREADS, 0);
    }
}
void orc_gemv(const float *x, const float *W, float *y, int in, int out) {
    struct gemv_ctx c = {x, W, y, in};
    parallel_for(out, gemv_range, &c);
}

/* ---------------------------------------------------------------------- bf16 */
/* Round-to-nearest-even fp32 -> bf16 bits (tests/model/ops_test.cu:77-82
 * f2bf16_bits) and back: out[i] = float(bf16(in[i])). */
void orc_round_bf16(const float *in, float *out, uint16_t *bits, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        u += 0x7FFFu + ((u >> 16) & 1u);
        const uint16_t b = (uint16_t)(u >> 16);
        if (bits)
            bits[i] = b;
        if (out) {
            const uint32_t f = (uint32_t)b << 16;
            memcpy(&out[i], &f, 4);
        }
    }
}

/* ---------------------------------------------------------------- attention */
struct attn_ctx {
    const float *q, *k, *v;
    float *out;
    double *bound;
    int T, S, qh, kv_rep, D, cap;
    const int *rows;
    int nrows;
    float scale;
};

/* One (head, row) of the explicit path. */
static void attn_explicit_row(const struct attn_ctx *c, int h, int row, float *scores, float *o, double *b) {
    const int kvh = h / c->kv_rep;
    const float *qrow = c->q + ((int64_t)h * c->T + row) * c->D;
    const float *kh = c->k + (int64_t)kvh * c->cap * c->D;
    const float *vh = c->v + (int64_t)kvh * c->cap * c->D;
    /* linear(q_h, k_h): k-ascending fmaf chain over d (linear_kernel, include/ops/linear.cuh:18-73) */
    for (int j = 0; j < c->S; ++j) {
        float acc = 0.f;
        for (int d = 0; d < c->D; ++d)
            acc = fmaf(qrow[d], kh[(int64_t)j * c->D + d], acc);
        scores[j] = acc;
    }
    /* causal_scale (include/ops/causal_scale.cuh:9-16): col <= S - T + row ? s * scale : -inf */
    const int qpos = c->S - c->T + row;
    for (int j = 0; j < c->S; ++j)
        scores[j] = j <= qpos ? scores[j] * c->scale : -INFINITY;
    /* softmax over the row (include/ops/softmax.cuh:10-29) */
    softmax_row(scores, scores, c->S);
    /* mat_mul(P, v_h): fmaf chain over keys (include/ops/matmul.cuh:11-66) */
    for (int d = 0; d < c->D; ++d) {
        float acc = 0.f;
        double ab = 0.0;
        for (int j = 0; j < c->S; ++j) {
            acc = fmaf(scores[j], vh[(int64_t)j * c->D + d], acc);
            ab += fabs((double)scores[j] * vh[(int64_t)j * c->D + d]);
        }
        o[d] = acc;
        if (b)
            b[d] = ab;
    }
}

static void attn_range(void *p, int64_t lo, int64_t hi) {
    struct attn_ctx *c = (struct attn_ctx *)p;
    float *scores = (float *)malloc(sizeof(float) * (size_t)c->S);
    const int nr = c->rows ? c->nrows : c->T;
    for (int64_t w = lo; w < hi; ++w) {
        const int h = (int)(w / nr), ri = (int)(w % nr);
        const int row = c->rows ? c->rows[ri] : ri;
        float *o = c->out + ((int64_t)h * nr + ri) * c->D;
        double *b = c->bound ? c->bound + ((int64_t)h * nr + ri) * c->D : NULL;
        attn_explicit_row(c, h, row, scores, o, b);
    }
    free(scores);
}

/* Explicit prefill attention, as LlamaModelT::forward runs it for 2 <= rows <=
 * 2048 (include/models/llama.cuh:246-263): per q head, QK^T by ops::linear,
 * causal_scale with scale 1/sqrt(D) (llama.cuh:222), row softmax, then P V by
 * ops::mat_mul. Only rows listed in `rows` (all T when NULL) are produced:
 * out/bound are [qh][nrows][D]; bound receives sum_key p*|v| per output. */
void orc_attention_explicit(const float *q, const float *k, const float *v, float *out, double *bound, int T, int S,
                            int qh, int kv_rep, int D, int cap, const int *rows, int nrows) {
    struct attn_ctx c = {q, k, v, out, bound, T, S, qh, kv_rep, D, cap, rows, nrows, 1.0f / sqrtf((float)D)};
    parallel_for((int64_t)qh * (rows ? nrows : T), attn_range, &c);
}

/* attention_decode_kernel (include/ops/attention_decode.cuh:14-90), one block
 * of 256 threads per q head: scores[j] = (fmaf chain over d) * scale, block max,
 * e_j = expf(s_j - max), block sum, inv = 1/sum, per-thread acc[d] =
 * fmaf(e_j * inv, v_j[d], acc[d]) over keys j = t, t+256, ..., then a 32-lane
 * shuffle tree per d and a serial sum over the 8 warps. scale = rsqrtf(D),
 * restated as 1/sqrtf(D) (exact for D = 64). */
struct decode_ctx {
    const float *q, *k, *v;
    float *out;
    int kv_rep, D, len, max_seq;
};
/* Heads are independent: q heads [h0, h1) with their own scratch. */
static void decode_heads_range(void *p, int64_t h0, int64_t h1) {
    const struct decode_ctx *c = (const struct decode_ctx *)p;
    const int D = c->D, len = c->len, max_seq = c->max_seq;
    float *scores = (float *)malloc(sizeof(float) * (size_t)len);
    float *acc = (float *)malloc(sizeof(float) * REF_THREADS * (size_t)D);
    float part[REF_THREADS];
    const float scale = 1.0f / sqrtf((float)D);
    for (int h = (int)h0; h < (int)h1; ++h) {
        const int kvh = h / c->kv_rep;
        const float *kh = c->k + (int64_t)kvh * max_seq * D;
        const float *vh = c->v + (int64_t)kvh * max_seq * D;
        const float *qv = c->q + (int64_t)h * D;
        for (int j = 0; j < len; ++j) {
            float dot = 0.f;
            for (int d = 0; d < D; ++d)
                dot = fmaf(qv[d], kh[(int64_t)j * D + d], dot);
            scores[j] = dot * scale;
        }
        for (int t = 0; t < REF_THREADS; ++t) {
            float m = -INFINITY;
            for (int j = t; j < len; j += REF_THREADS)
                m = fmaxf(m, scores[j]);
            part[t] = m;
        }
        const float mx = orc_block_reduce(part, REF_THREADS, 1);
        for (int t = 0; t < REF_THREADS; ++t) {
            float s = 0.f;
            for (int j = t; j < len; j += REF_THREADS) {
                const float e = expf(scores[j] - mx);
                scores[j] = e;
                s += e;
            }
            part[t] = s;
        }
        const float inv = 1.f / orc_block_reduce(part, REF_THREADS, 0);
        for (int t = 0; t < REF_THREADS; ++t) {
            float *a = acc + (int64_t)t * D;
            for (int d = 0; d < D; ++d)
                a[d] = 0.f;
            for (int j = t; j < len; j += REF_THREADS) {
                const float p = scores[j] * inv;
                for (int d = 0; d < D; ++d)
                    a[d] = fmaf(p, vh[(int64_t)j * D + d], a[d]);
            }
        }
        for (int d = 0; d < D; ++d) {
            float total = 0.f;
            for (int w = 0; w < REF_THREADS / REF_WARP; ++w) {
                float lanes[REF_WARP];
                for (int l = 0; l < REF_WARP; ++l)
                    lanes[l] = acc[(int64_t)(w * REF_WARP + l) * D + d];
                total += warp_tree(lanes, 0);
            }
            c->out[(int64_t)h * D + d] = total;
        }
    }
    free(scores);
    free(acc);
}

void orc_attention_decode(const float *q, const float *k, const float *v, float *out, int qh, int kv_rep, int D,
                          int len, int max_seq) {
    struct decode_ctx c = {q, k, v, out, kv_rep, D, len, max_seq};
    parallel_for(qh, decode_heads_range, &c);
}

/* ------------------------------------------------------------ llama forward */
/* linear_kernel (include/ops/linear.cuh:18-73) order for rows >= 2: every
 * output is the k-ascending chain acc = fmaf(x, w, acc). Columns are processed
 * in blocks of 64 with the weight block transposed into a private buffer. */
struct lin_ctx {
    const float *X, *W;
    float *Y;
    int rows, in, out;
};
#define LIN_BLOCK 64
static void lin_range(void *p, int64_t lo, int64_t hi) {
    struct lin_ctx *c = (struct lin_ctx *)p;
    float *buf = (float *)malloc(sizeof(float) * (size_t)c->in * LIN_BLOCK);
    float acc[LIN_BLOCK];
    for (int64_t blk = lo; blk < hi; ++blk) {
        const int o0 = (int)blk * LIN_BLOCK;
        const int nb = c->out - o0 < LIN_BLOCK ? c->out - o0 : LIN_BLOCK;
        for (int j = 0; j < LIN_BLOCK; ++j)
            for (int n = 0; n < c->in; ++n)
                buf[(int64_t)n * LIN_BLOCK + j] = j < nb ? c->W[(int64_t)(o0 + j) * c->in + n] : 0.f;
        for (int r = 0; r < c->rows; ++r) {
            const float *x = c->X + (int64_t)r * c->in;
            for (int j = 0; j < LIN_BLOCK; ++j)
                acc[j] = 0.f;
            for (int n = 0; n < c->in; ++n) {
                const float a = x[n];
                const float *b = buf + (int64_t)n * LIN_BLOCK;
                for (int j = 0; j < LIN_BLOCK; ++j)
                    acc[j] = fmaf(a, b[j], acc[j]);
            }
            for (int j = 0; j < nb; ++j)
                c->Y[(int64_t)r * c->out + o0 + j] = acc[j];
        }
    }
    free(buf);
}

/* The bf16 tensor-core projection (ops::linear_mma_bf16, include/ops/linear_mma.cuh:19-115) on
 * inputs already rounded to bf16: every product of two bf16 values is exact in fp32, and the
 * WMMA fragments accumulate them inside the tensor core in an order the code does not fix. This
 * restatement sums the exact products in double (its error far below an fp32 ulp) and rounds once
 * to fp32: the correctly rounded dot product but for rare near-halfway cases, the value any
 * accumulation order approximates. A k-ascending fp32 chain would add its own ~sqrt(K)-ulp
 * rounding walk to the difference from the GPU. */
static void lin_exact_range(void *p, int64_t lo, int64_t hi) {
    struct lin_ctx *c = (struct lin_ctx *)p;
    double *buf = (double *)malloc(sizeof(double) * (size_t)c->in * LIN_BLOCK);
    double acc[LIN_BLOCK];
    for (int64_t blk = lo; blk < hi; ++blk) {
        const int o0 = (int)blk * LIN_BLOCK;
        const int nb = c->out - o0 < LIN_BLOCK ? c->out - o0 : LIN_BLOCK;
        for (int j = 0; j < LIN_BLOCK; ++j)
            for (int n = 0; n < c->in; ++n)
                buf[(int64_t)n * LIN_BLOCK + j] = j < nb ? (double)c->W[(int64_t)(o0 + j) * c->in + n] : 0.0;
        for (int r = 0; r < c->rows; ++r) {
            const float *x = c->X + (int64_t)r * c->in;
            for (int j = 0; j < LIN_BLOCK; ++j)
                acc[j] = 0.0;
            for (int n = 0; n < c->in; ++n) {
                const double a = x[n];
                const double *b = buf + (int64_t)n * LIN_BLOCK;
                for (int j = 0; j < LIN_BLOCK; ++j)
                    acc[j] += a * b[j];
            }
            for (int j = 0; j < nb; ++j)
                c->Y[(int64_t)r * c->out + o0 + j] = (float)acc[j];
        }
    }
    free(buf);
}

void orc_linear_exact(const float *X, const float *W, float *Y, int rows, int in, int out) {
    struct lin_ctx c = {X, W, Y, rows, in, out};
    parallel_for((out + LIN_BLOCK - 1) / LIN_BLOCK, lin_exact_range, &c);
}

/* ops::linear (include/ops/linear.cuh:130-153): the GEMV order for one row,
 * the tiled order otherwise. */
void orc_linear(const float *X, const float *W, float *Y, int rows, int in, int out) {
    if (rows == 1) {
        orc_gemv(X, W, Y, in, out);
        return;
    }
    struct lin_ctx c = {X, W, Y, rows, in, out};
    parallel_for((out + LIN_BLOCK - 1) / LIN_BLOCK, lin_range, &c);
}

/* ModelConfig::rope_inv_freq (include/runtime/model_config.cuh:68-89): double
 * arithmetic, with int/float and float-float subexpressions in float as there. */
void orc_rope_inv_freq(int head_dim, float theta, int llama3, float factor, float low, float high, int orig,
                       float *out) {
    const double pi = 3.14159265358979323846;
    for (int i = 0; i < head_dim / 2; ++i) {
        double f = 1.0 / pow((double)theta, (2.0 * i) / head_dim);
        if (llama3) {
            const double wavelen = 2.0 * pi / f;
            const double low_wl = (float)orig / low;
            const double high_wl = (float)orig / high;
            if (wavelen > low_wl) {
                f /= factor;
            } else if (wavelen >= high_wl) {
                const double smooth = (orig / wavelen - low) / (double)(high - low);
                f = (1.0 - smooth) * f / factor + smooth * f;
            }
        }
        out[i] = (float)f;
    }
}

/* rope_kernel (include/ops/rope.cuh:10-25): pair (i, i + D/2) at position p,
 * freq = p * inv_freq[i] in float, c = cosf(freq), s = sinf(freq),
 * lo = a*c - b*s, hi = b*c + a*s. The products are restated with the
 * contraction lo = fmaf(a, c, -(b*s)), hi = fmaf(b, c, a*s). */
void orc_rope(float *x, const float *inv_freq, int rows, int heads, int head_dim, int pos_start) {
    const int half = head_dim / 2;
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < heads; ++h)
            for (int i = 0; i < half; ++i) {
                const float freq = (float)(pos_start + r) * inv_freq[i];
                const float c = cosf(freq), s = sinf(freq);
                float *p = x + (int64_t)r * heads * head_dim + h * head_dim + i;
                const float a = p[0], b = p[half];
                p[0] = fmaf(a, c, -(b * s));
                p[half] = fmaf(b, c, a * s);
            }
}

/* swiglu_kernel (include/ops/swiglu.cuh:7-12): out = g / (1 + expf(-g)) * u,
 * evaluated left to right in float. */
void orc_swiglu(const float *gate, const float *up, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = gate[i];
        out[i] = g / (1.f + expf(-g)) * up[i];
    }
}

/* causal_scale_kernel (include/ops/causal_scale.cuh:9-16): query row r sits at
 * position cols - rows + r; keys up to it are scaled, later ones become -inf. */
void orc_causal_scale(float *scores, int rows, int cols, float scale) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            float *p = scores + (int64_t)r * cols + c;
            *p = c <= cols - rows + r ? *p * scale : -INFINITY;
        }
}

typedef struct {
    int L, H, I, qh, kvh, D, V;
    float eps;
    float *embed, *final_norm, *inv_freq;
    float **in_norm, **post_norm, **wq, **wk, **wv, **wo, **wg, **wu, **wd;
    int bf16; /* weights hold bf16 values; projections of >= 16 rows round X to bf16 */
    /* session */
    int cap, length;
    float *kc, *vc; /* [L][kvh][cap][D] */
} orc_llama;

static float *alloc_f(int64_t n) { return (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1)); }

static void fill_norm(float *dst, int64_t n, uint64_t seed, uint64_t stream, int uniform) {
    if (uniform)
        orc_fill_uniform(dst, n, seed, stream, 0.5f, 1.5f);
    else
        for (int64_t i = 0; i < n; ++i)
            dst[i] = 1.f;
}

/* Seeded weights as the runtime's random init creates them (logical HF
 * tensors; streams: embed 1, final norm 2, layer l base 64 + 16 l: q 0, k 1,
 * v 2, o 3, gate 4, up 5, down 6, input norm 7, post norm 8). */
void *orc_llama_create(int L, int H, int I, int qh, int kvh, int D, int V, float eps, float theta, int llama3,
                       float factor, float low, float high, int orig, uint64_t seed, float sd, int norm_uniform) {
    orc_llama *m = (orc_llama *)calloc(1, sizeof(orc_llama));
    m->L = L, m->H = H, m->I = I, m->qh = qh, m->kvh = kvh, m->D = D, m->V = V, m->eps = eps;
    m->embed = alloc_f((int64_t)V * H);
    orc_fill_normal_mt(m->embed, (int64_t)V * H, seed, 1, 0.f, sd);
    m->final_norm = alloc_f(H);
    fill_norm(m->final_norm, H, seed, 2, norm_uniform);
    m->inv_freq = alloc_f(D / 2);
    orc_rope_inv_freq(D, theta, llama3, factor, low, high, orig, m->inv_freq);
    float ***lists[] = {&m->in_norm, &m->post_norm, &m->wq, &m->wk, &m->wv, &m->wo, &m->wg, &m->wu, &m->wd};
    for (int k = 0; k < 9; ++k)
        *lists[k] = (float **)calloc((size_t)L, sizeof(float *));
    const int64_t qw = (int64_t)qh * D, kw = (int64_t)kvh * D;
    for (int l = 0; l < L; ++l) {
        const uint64_t b = 64 + 16 * (uint64_t)l;
        m->wq[l] = alloc_f(qw * H), orc_fill_normal_mt(m->wq[l], qw * H, seed, b + 0, 0.f, sd);
        m->wk[l] = alloc_f(kw * H), orc_fill_normal_mt(m->wk[l], kw * H, seed, b + 1, 0.f, sd);
        m->wv[l] = alloc_f(kw * H), orc_fill_normal_mt(m->wv[l], kw * H, seed, b + 2, 0.f, sd);
        m->wo[l] = alloc_f((int64_t)H * qw), orc_fill_normal_mt(m->wo[l], (int64_t)H * qw, seed, b + 3, 0.f, sd);
        m->wg[l] = alloc_f((int64_t)I * H), orc_fill_normal_mt(m->wg[l], (int64_t)I * H, seed, b + 4, 0.f, sd);
        m->wu[l] = alloc_f((int64_t)I * H), orc_fill_normal_mt(m->wu[l], (int64_t)I * H, seed, b + 5, 0.f, sd);
        m->wd[l] = alloc_f((int64_t)H * I), orc_fill_normal_mt(m->wd[l], (int64_t)H * I, seed, b + 6, 0.f, sd);
        m->in_norm[l] = alloc_f(H), fill_norm(m->in_norm[l], H, seed, b + 7, norm_uniform);
        m->post_norm[l] = alloc_f(H), fill_norm(m->post_norm[l], H, seed, b + 8, norm_uniform);
    }
    return m;
}

void orc_llama_destroy(void *p) {
    orc_llama *m = (orc_llama *)p;
    if (!m)
        return;
    for (int l = 0; l < m->L; ++l) {
        free(m->wq[l]), free(m->wk[l]), free(m->wv[l]), free(m->wo[l]), free(m->wg[l]), free(m->wu[l]);
        free(m->wd[l]), free(m->in_norm[l]), free(m->post_norm[l]);
    }
    free(m->wq), free(m->wk), free(m->wv), free(m->wo), free(m->wg), free(m->wu), free(m->wd);
    free(m->in_norm), free(m->post_norm), free(m->embed), free(m->final_norm), free(m->inv_freq);
    free(m->kc), free(m->vc);
    free(m);
}

/* Raw weight access for tests that write packs: kind 0 embed, 1 final norm,
 * per layer 2 q, 3 k, 4 v, 5 o, 6 gate, 7 up, 8 down, 9 input norm, 10 post norm. */
const float *orc_llama_weight(void *p, int kind, int layer) {
    orc_llama *m = (orc_llama *)p;
    switch (kind) {
    case 0: return m->embed;
    case 1: return m->final_norm;
    case 2: return m->wq[layer];
    case 3: return m->wk[layer];
    case 4: return m->wv[layer];
    case 5: return m->wo[layer];
    case 6: return m->wg[layer];
    case 7: return m->wu[layer];
    case 8: return m->wd[layer];
    case 9: return m->in_norm[layer];
    default: return m->post_norm[layer];
    }
}

void orc_llama_reset(void *p, int cap) {
    orc_llama *m = (orc_llama *)p;
    free(m->kc), free(m->vc);
    const int64_t n = (int64_t)m->L * m->kvh * cap * m->D;
    m->kc = alloc_f(n), m->vc = alloc_f(n);
    m->cap = cap;
    m->length = 0;
}

/* LlamaModelBF16 (include/models/llama.cuh:290-291, runtime/weights.cuh:16-94):
 * projections and the tied embedding are stored as bf16, and so are the norm
 * weights of a bf16 pack (widened to fp32 on load); every weight is therefore
 * rounded to bf16 (nearest-even) in place. The forward then follows
 * linear_dispatch (models/llama.cuh:190-199). */
void orc_llama_set_bf16(void *p) {
    orc_llama *m = (orc_llama *)p;
    const int64_t H = m->H, I = m->I, qw = (int64_t)m->qh * m->D, kw = (int64_t)m->kvh * m->D;
    orc_round_bf16(m->embed, m->embed, NULL, (int64_t)m->V * H);
    orc_round_bf16(m->final_norm, m->final_norm, NULL, H);
    for (int l = 0; l < m->L; ++l) {
        orc_round_bf16(m->wq[l], m->wq[l], NULL, qw * H);
        orc_round_bf16(m->wk[l], m->wk[l], NULL, kw * H);
        orc_round_bf16(m->wv[l], m->wv[l], NULL, kw * H);
        orc_round_bf16(m->wo[l], m->wo[l], NULL, H * qw);
        orc_round_bf16(m->wg[l], m->wg[l], NULL, I * H);
        orc_round_bf16(m->wu[l], m->wu[l], NULL, I * H);
        orc_round_bf16(m->wd[l], m->wd[l], NULL, H * I);
        orc_round_bf16(m->in_norm[l], m->in_norm[l], NULL, H);
        orc_round_bf16(m->post_norm[l], m->post_norm[l], NULL, H);
    }
    m->bf16 = 1;
}

/* linear_dispatch: a bf16 model with rows >= 16 takes the tensor-core GEMM,
 * which rounds X to bf16 (ops/linear_mma.cuh:49); otherwise ops::linear. */
static void llama_project(const orc_llama *m, const float *X, const float *W, float *Y, int rows, int in, int out) {
    if (m->bf16 && rows >= 16) {
        float *xr = alloc_f((int64_t)rows * in);
        orc_round_bf16(X, xr, NULL, (int64_t)rows * in);
        orc_linear_exact(xr, W, Y, rows, in, out);
        free(xr);
    } else {
        orc_linear(X, W, Y, rows, in, out);
    }
}

/* argmax_kernel (include/ops/argmax.cuh:9-51): lowest index on ties, NaN never wins. */
int orc_argmax(const float *x, int n) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = 0; i < n; ++i)
        if (x[i] > best || (x[i] == best && i < bi))
            best = x[i], bi = i;
    return bi;
}

/* LlamaModelT::forward (include/models/llama.cuh:216-285) for `rows` tokens at
 * positions [length, length + rows). logits (V floats) of the last row;
 * captures (optional) receive hidden after the embedding and each layer. */
static int llama_forward(orc_llama *m, const int *ids, int rows, float *logits, float *captures) {
    const int H = m->H, I = m->I, D = m->D, qh = m->qh, kvh = m->kvh, rep = qh / kvh;
    const int pos0 = m->length, S = pos0 + rows;
    const int64_t qw = (int64_t)qh * D, kw = (int64_t)kvh * D;
    float *hidden = alloc_f((int64_t)rows * H), *normed = alloc_f((int64_t)rows * H);
    float *q = alloc_f(rows * qw), *k = alloc_f(rows * kw), *v = alloc_f(rows * kw);
    float *attn = alloc_f(rows * qw), *gate = alloc_f((int64_t)rows * I), *up = alloc_f((int64_t)rows * I);
    float *qheads = alloc_f(rows * qw), *aheads = alloc_f(rows * qw);
    for (int r = 0; r < rows; ++r)
        memcpy(hidden + (int64_t)r * H, m->embed + (int64_t)ids[r] * H, sizeof(float) * H);
    if (captures)
        memcpy(captures, hidden, sizeof(float) * rows * H);
    for (int l = 0; l < m->L; ++l) {
        float *kc = m->kc + (int64_t)l * kvh * m->cap * D, *vc = m->vc + (int64_t)l * kvh * m->cap * D;
        orc_rms_norm_rows(hidden, m->in_norm[l], normed, rows, H, m->eps);
        llama_project(m, normed, m->wq[l], q, rows, H, (int)qw);
        llama_project(m, normed, m->wk[l], k, rows, H, (int)kw);
        llama_project(m, normed, m->wv[l], v, rows, H, (int)kw);
        orc_rope(q, m->inv_freq, rows, qh, D, pos0);
        orc_rope(k, m->inv_freq, rows, kvh, D, pos0);
        for (int r = 0; r < rows; ++r) /* split_heads into the cache (include/ops/split_heads.cuh:9-18) */
            for (int h = 0; h < kvh; ++h)
                for (int d = 0; d < D; ++d) {
                    kc[((int64_t)h * m->cap + pos0 + r) * D + d] = k[(int64_t)r * kw + h * D + d];
                    vc[((int64_t)h * m->cap + pos0 + r) * D + d] = v[(int64_t)r * kw + h * D + d];
                }
        if (rows == 1) {
            orc_attention_decode(q, kc, vc, attn, qh, rep, D, S, m->cap);
        } else {
            for (int r = 0; r < rows; ++r)
                for (int h = 0; h < qh; ++h)
                    memcpy(qheads + ((int64_t)h * rows + r) * D, q + (int64_t)r * qw + h * D, sizeof(float) * D);
            orc_attention_explicit(qheads, kc, vc, aheads, NULL, rows, S, qh, rep, D, m->cap, NULL, 0);
            for (int r = 0; r < rows; ++r)
                for (int h = 0; h < qh; ++h)
                    memcpy(attn + (int64_t)r * qw + h * D, aheads + ((int64_t)h * rows + r) * D, sizeof(float) * D);
        }
        llama_project(m, attn, m->wo[l], normed, rows, (int)qw, H);
        for (int64_t i = 0; i < (int64_t)rows * H; ++i) /* add_kernel */
            hidden[i] = hidden[i] + normed[i];
        orc_rms_norm_rows(hidden, m->post_norm[l], normed, rows, H, m->eps);
        llama_project(m, normed, m->wg[l], gate, rows, H, I);
        llama_project(m, normed, m->wu[l], up, rows, H, I);
        for (int64_t i = 0; i < (int64_t)rows * I; ++i) { /* swiglu_kernel (include/ops/swiglu.cuh:7-12) */
            const float g = gate[i];
            gate[i] = g / (1.f + expf(-g)) * up[i];
        }
        llama_project(m, gate, m->wd[l], normed, rows, I, H);
        for (int64_t i = 0; i < (int64_t)rows * H; ++i)
            hidden[i] = hidden[i] + normed[i];
        if (captures)
            memcpy(captures + (int64_t)(l + 1) * rows * H, hidden, sizeof(float) * rows * H);
    }
    orc_rms_norm_rows(hidden + (int64_t)(rows - 1) * H, m->final_norm, normed, 1, H, m->eps);
    orc_gemv(normed, m->embed, logits, H, m->V);
    m->length = S;
    free(hidden), free(normed), free(q), free(k), free(v), free(attn), free(gate), free(up), free(qheads);
    free(aheads);
    return orc_argmax(logits, m->V);
}

int orc_llama_prefill(void *p, const int *ids, int n, float *logits, float *captures) {
    orc_llama *m = (orc_llama *)p;
    m->length = 0;
    return llama_forward(m, ids, n, logits, captures);
}

int orc_llama_decode(void *p, int token, float *logits) { return llama_forward((orc_llama *)p, &token, 1, logits, NULL); }

/* ---- Scan / Transform / GatherScatter (semantics stated in oracle.h) ---- */
void orc_scan(const float *in, float *out, double *abs_prefix, int64_t n, int op, int inclusive) {
    double run = 0.0, run_abs = 0.0;
    float best = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        const float x = in[i];
        if (!inclusive) {
            out[i] = op == 1 ? best : (float)run;
            if (abs_prefix)
                abs_prefix[i] = run_abs;
        }
        run += (double)x;
        run_abs += fabs((double)x);
        best = fmaxf(best, x);
        if (inclusive) {
            out[i] = op == 1 ? best : (float)run;
            if (abs_prefix)
                abs_prefix[i] = run_abs;
        }
    }
}

struct transpose_ctx {
    const float *in;
    float *out;
    int rows, cols;
};
static void transpose_range(void *p, int64_t r0, int64_t r1) {
    const struct transpose_ctx *t = (const struct transpose_ctx *)p;
    for (int64_t r = r0; r < r1; ++r)
        for (int c = 0; c < t->cols; ++c)
            t->out[(int64_t)c * t->rows + r] = t->in[r * t->cols + c];
}
void orc_transpose(const float *in, float *out, int rows, int cols) {
    struct transpose_ctx t = {in, out, rows, cols};
    parallel_for(rows, transpose_range, &t);
}

struct gather_ctx {
    const float *in;
    int64_t in_size;
    const int *idx;
    float *out;
};
static void gather_range(void *p, int64_t i0, int64_t i1) {
    const struct gather_ctx *g = (const struct gather_ctx *)p;
    for (int64_t i = i0; i < i1; ++i)
        g->out[i] = (g->idx[i] >= 0 && g->idx[i] < g->in_size) ? g->in[g->idx[i]] : NAN;
}
void orc_gather(const float *in, int64_t in_size, const int *idx, float *out, int64_t count) {
    struct gather_ctx g = {in, in_size, idx, out};
    parallel_for(count, gather_range, &g);
}

void orc_scatter(const float *in, const int *idx, float *out, int64_t out_size, int64_t count) {
    for (int64_t i = 0; i < count; ++i)
        if (idx[i] >= 0 && idx[i] < out_size)
            out[idx[i]] = in[i];
}
