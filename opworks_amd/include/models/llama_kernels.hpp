#pragma once

// Kernels of the Llama decode step and prefill glue (fp32 weights).
//
// Decode step per layer (5 launches; every kernel reads the step position from
// device memory, so one captured HIP graph replays every token):
//   1. qkv_rope_kernel   RMSNorm(hidden) -> fused [q;k;v] GEMV -> RoPE on q, k ->
//                        q to the workspace, k and v appended to the KV cache
//   2. decode_attention_kernel  split-KV partials; the last workgroup of each
//                        kv head merges the chunks (no second launch)
//   3. gemv_residual_kernel   hidden += W_o attn
//   4. norm_gemv_kernel<SwiGLU>  RMSNorm(hidden) -> interleaved [gate;up] GEMV ->
//                        act = silu(gate) * up
//   5. down_residual_kernel   hidden += W_down act (K split over 4 waves)
// then final RMSNorm + LM-head GEMV with a fused argmax (last-workgroup reduce).
//
// GEMV shape: a wave owns kRows output rows; each lane streams 16-byte packs
// of those rows at columns 4*(lane + 64*u) with all loads issued before the
// FMAs; the normalised input vector lives in registers (kV packs per lane);
// one DPP reduction per row. Weight bytes are read once per token.

#include <cmath>
#include <cstdint>

#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "../ops/attention.hpp"
#include "../ops/elementwise.hpp"

namespace opworks::llama {

using detail::f32x4;

// Device-resident state of the decode step.
struct StepState {
    int32_t token; // input token id of this step
    int32_t pos;   // its position (= KV length before the step)
    int32_t next;  // argmax result
    int32_t pad;
};

constexpr int kRows = 4;       // GEMV rows per wave
constexpr int kBlock = 256;    // threads per GEMV workgroup
constexpr int kWavesPerBlock = kBlock / kWaveSize;

// x (H = 256 * kV floats) -> registers, optionally RMS-normalised with gamma:
// xn = x * rsqrtf(mean(x^2) + eps) * gamma, same expression order as ops::rms_norm.
template <int kV>
__device__ __forceinline__ void load_vector(const float *__restrict__ x, const float *__restrict__ gamma, float eps,
                                            int lane, f32x4 (&xn)[kV]) {
    const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
#pragma unroll
    for (int u = 0; u < kV; ++u)
        xn[u] = x4[lane + kWaveSize * u];
    if (gamma) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < kV; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ss = fmaf(xn[u][j], xn[u][j], ss);
        const float inv = rsqrtf(wave::sum(ss) / (256 * kV) + eps);
        const f32x4 *g4 = reinterpret_cast<const f32x4 *>(gamma);
#pragma unroll
        for (int u = 0; u < kV; ++u) {
            const f32x4 g = g4[lane + kWaveSize * u];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xn[u][j] = xn[u][j] * inv * g[j];
        }
    }
}

// y[r] = dot(W[row_r, :], xn) for kRows rows, wave-uniform results.
template <int kV>
__device__ __forceinline__ void gemv_rows(const float *__restrict__ W, const int (&row)[kRows], const f32x4 (&xn)[kV],
                                          int lane, float (&y)[kRows]) {
    constexpr int H = 256 * kV;
    f32x4 w[kRows][kV];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int u = 0; u < kV; ++u)
            w[r][u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(W + int64_t(row[r]) * H) + lane +
                                                 kWaveSize * u);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < kV; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = fmaf(w[r][u][j], xn[u][j], acc);
        y[r] = wave::sum(acc);
    }
}

// ---- 1. QKV + RoPE + cache append ------------------------------------------
// Fused weight rows: [q heads | k heads | v heads], each head D rows. Wave w
// owns rotary pairs (j, j + D/2) and (j+1, j+1 + D/2) of head slot w / (D/4),
// j = 2 * (w % (D/4)). Layer 0 reads its input from the embedding row of the
// step token and also writes it to the residual stream.
struct QkvArgs {
    const float *hidden_in; // residual stream (or nullptr: use embed[token])
    const float *embed;     // [V][H]
    float *hidden_out;      // written only when reading from the embedding
    const float *gamma;     // input RMSNorm weight
    const float *wqkv;      // [(qh + 2 kvh) * D][H]
    const float *inv_freq;  // [D/2]
    float *q_out;           // [qh][D]
    float *kcache, *vcache; // this layer: [kvh][cap][D]
    const StepState *state;
    float eps;
    int qh, kvh, D, cap;
};

template <int kV>
__global__ __launch_bounds__(kBlock) void qkv_rope_kernel(QkvArgs a) {
    constexpr int H = 256 * kV;
    const int lane = threadIdx.x % kWaveSize;
    const int w = blockIdx.x * kWavesPerBlock + threadIdx.x / kWaveSize;
    const int waves_per_head = a.D / 4;
    const int slot = w / waves_per_head;
    if (slot >= a.qh + 2 * a.kvh)
        return;
    const int pos = a.state->pos;
    const float *src = a.hidden_in ? a.hidden_in : a.embed + int64_t(a.state->token) * H;
    f32x4 xn[kV];
    if (!a.hidden_in && w == 0) { // layer 0: residual stream = embedding row
        const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src);
        f32x4 *h4 = reinterpret_cast<f32x4 *>(a.hidden_out);
#pragma unroll
        for (int u = 0; u < kV; ++u)
            h4[lane + kWaveSize * u] = s4[lane + kWaveSize * u];
    }
    load_vector<kV>(src, a.gamma, a.eps, lane, xn);
    const int half = a.D / 2;
    const int j = 2 * (w % waves_per_head);
    const int base = slot * a.D;
    const int row[kRows] = {base + j, base + j + 1, base + j + half, base + j + 1 + half};
    float y[kRows];
    gemv_rows<kV>(a.wqkv, row, xn, lane, y);
    if (lane != 0)
        return;
    if (slot < a.qh + a.kvh) { // rotate q and k: (lo, hi) = (a c - b s, b c + a s)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const float freq = static_cast<float>(pos) * a.inv_freq[j + p];
            const float c = cosf(freq), s = sinf(freq);
            const float lo = y[p], hi = y[p + 2];
            y[p] = lo * c - hi * s;
            y[p + 2] = hi * c + lo * s;
        }
    }
    float *dst;
    if (slot < a.qh)
        dst = a.q_out + int64_t(slot) * a.D;
    else if (slot < a.qh + a.kvh)
        dst = a.kcache + (int64_t(slot - a.qh) * a.cap + pos) * a.D;
    else
        dst = a.vcache + (int64_t(slot - a.qh - a.kvh) * a.cap + pos) * a.D;
    dst[j] = y[0];
    dst[j + 1] = y[1];
    dst[j + half] = y[2];
    dst[j + 1 + half] = y[3];
}

// ---- 2. decode attention with an in-kernel merge -----------------------------
// grid (kvh, max_chunks), block kv_rep waves. Partial records [qh][max_chunks][D + 2]
// (max, sum, unnormalised output); counters[kvh] start at zero and are
// returned to zero by the merging workgroup.
struct DecodeAttnArgs {
    const float *q;                  // [qh][D]
    const float *kcache, *vcache;    // [kvh][cap][D]
    float *out;                      // [qh][D]
    float *partial;                  // [qh][max_chunks][D + 2]
    unsigned *counters;              // [kvh]
    const StepState *state;          // len = pos + 1
    int kv_rep, D, cap, max_chunks;
    float scale;
};

__global__ __launch_bounds__(16 * kWaveSize) static void decode_attention_kernel(DecodeAttnArgs a) {
    constexpr int C = detail::kAttnChunk;
    int len = a.state->pos + 1;
    len = len < a.cap ? len : a.cap;
    len = len < a.max_chunks * C ? len : a.max_chunks * C;
    const int nchunks = (len + C - 1) / C;
    const int kvh = blockIdx.x, chunk = blockIdx.y;
    if (chunk >= nchunks)
        return;
    const int k0 = chunk * C;
    const int n = len - k0 < C ? len - k0 : C;
    const int D = a.D;
    __shared__ __attribute__((aligned(16))) float Ks[C][64 + 4];
    __shared__ __attribute__((aligned(16))) float Vs[C][64];
    __shared__ __attribute__((aligned(16))) float Qs[16][64];
    __shared__ float Ps[16][C];
    __shared__ bool merge;
    const float *kh = a.kcache + (int64_t(kvh) * a.cap + k0) * D;
    const float *vh = a.vcache + (int64_t(kvh) * a.cap + k0) * D;
    for (int i = threadIdx.x; i < C * D; i += blockDim.x) {
        const int r = i / D, d = i % D;
        Ks[r][d] = r < n ? kh[i] : 0.f;
        Vs[r][d] = r < n ? vh[i] : 0.f;
    }
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int h = kvh * a.kv_rep + wave;
    if (lane < D)
        Qs[wave][lane] = a.q[int64_t(h) * D + lane];
    __syncthreads();
    // lane = key
    float s = 0.f;
    for (int d = 0; d < D; d += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4 *>(&Ks[lane][d]);
        const f32x4 qv = *reinterpret_cast<const f32x4 *>(&Qs[wave][d]);
        s = fmaf(qv[0], kv[0], s);
        s = fmaf(qv[1], kv[1], s);
        s = fmaf(qv[2], kv[2], s);
        s = fmaf(qv[3], kv[3], s);
    }
    s = lane < n ? s * a.scale : kNegInf;
    const float m = wave::max(s);
    const float p = lane < n ? expf(s - m) : 0.f;
    const float l = wave::sum(p);
    Ps[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    // lane = head-dim element
    float o = 0.f;
    if (lane < D) {
        for (int key = 0; key < n; ++key)
            o = fmaf(Ps[wave][key], Vs[key][lane], o);
    }
    float *rec = a.partial + (int64_t(h) * a.max_chunks + chunk) * (D + 2);
    if (lane == 0) {
        rec[0] = m;
        rec[1] = l;
    }
    if (lane < D)
        rec[2 + lane] = o;
    // last workgroup of this kv head merges the chunks
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
        merge = atomicAdd(&a.counters[kvh], 1u) == static_cast<unsigned>(nchunks - 1);
    __syncthreads();
    if (!merge)
        return;
    __threadfence();
    const float *base = a.partial + int64_t(h) * a.max_chunks * (D + 2);
    float M = kNegInf;
    for (int c = lane; c < nchunks; c += kWaveSize)
        M = fmaxf(M, __hip_atomic_load(base + int64_t(c) * (D + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    M = wave::max(M);
    float L = 0.f;
    for (int c = lane; c < nchunks; c += kWaveSize) {
        const float mc = __hip_atomic_load(base + int64_t(c) * (D + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float lc = __hip_atomic_load(base + int64_t(c) * (D + 2) + 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        L = fmaf(lc, expf(mc - M), L);
    }
    L = wave::sum(L);
    float acc = 0.f;
    if (lane < D) {
        for (int c = 0; c < nchunks; ++c) {
            const float mc = __hip_atomic_load(base + int64_t(c) * (D + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float oc = __hip_atomic_load(base + int64_t(c) * (D + 2) + 2 + lane, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
            acc = fmaf(oc, expf(mc - M), acc);
        }
        a.out[int64_t(h) * D + lane] = L > 0.f ? acc / L : 0.f;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        a.counters[kvh] = 0u;
}

// ---- 3. hidden += W x (in = H) -----------------------------------------------
template <int kV>
__global__ __launch_bounds__(kBlock) void gemv_residual_kernel(const float *__restrict__ W,
                                                               const float *__restrict__ x, float *__restrict__ hidden,
                                                               int out) {
    const int lane = threadIdx.x % kWaveSize;
    const int w = blockIdx.x * kWavesPerBlock + threadIdx.x / kWaveSize;
    const int r0 = w * kRows;
    if (r0 >= out)
        return;
    f32x4 xv[kV];
    load_vector<kV>(x, nullptr, 0.f, lane, xv);
    int row[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
        row[r] = r0 + r < out ? r0 + r : r0;
    float y[kRows];
    gemv_rows<kV>(W, row, xv, lane, y);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kRows; ++r)
            if (r0 + r < out)
                hidden[r0 + r] += y[r];
    }
}

// ---- 4. act = silu(gate) * up, interleaved [gate_i; up_i] rows ----------------
template <int kV>
__global__ __launch_bounds__(kBlock) void swiglu_gemv_kernel(const float *__restrict__ hidden,
                                                             const float *__restrict__ gamma, float eps,
                                                             const float *__restrict__ wgu, float *__restrict__ act,
                                                             int inter) {
    const int lane = threadIdx.x % kWaveSize;
    const int w = blockIdx.x * kWavesPerBlock + threadIdx.x / kWaveSize;
    const int i0 = w * (kRows / 2); // two (gate, up) pairs per wave
    if (i0 >= inter)
        return;
    f32x4 xn[kV];
    load_vector<kV>(hidden, gamma, eps, lane, xn);
    const int row[kRows] = {2 * i0, 2 * i0 + 1, 2 * i0 + 2, 2 * i0 + 3};
    float y[kRows];
    gemv_rows<kV>(wgu, row, xn, lane, y);
    if (lane == 0) {
        act[i0] = y[0] / (1.f + expf(-y[0])) * y[1];
        act[i0 + 1] = y[2] / (1.f + expf(-y[2])) * y[3];
    }
}

// ---- 5. hidden += W_down act (in = I = 1024 * kV2), K split across 4 waves ----
template <int kV2>
__global__ __launch_bounds__(kBlock) void down_residual_kernel(const float *__restrict__ W,
                                                               const float *__restrict__ act,
                                                               float *__restrict__ hidden, int out) {
    constexpr int I = 1024 * kV2;
    constexpr int Kw = I / kWavesPerBlock; // columns per wave
    __shared__ float part[kWavesPerBlock][kRows];
    const int lane = threadIdx.x % kWaveSize, wave = threadIdx.x / kWaveSize;
    const int r0 = blockIdx.x * kRows;
    const int c0 = wave * Kw;
    f32x4 xv[kV2];
    const f32x4 *a4 = reinterpret_cast<const f32x4 *>(act + c0);
#pragma unroll
    for (int u = 0; u < kV2; ++u)
        xv[u] = a4[lane + kWaveSize * u];
    f32x4 wv[kRows][kV2];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int row = r0 + r < out ? r0 + r : r0;
        const f32x4 *w4 = reinterpret_cast<const f32x4 *>(W + int64_t(row) * I + c0);
#pragma unroll
        for (int u = 0; u < kV2; ++u)
            wv[r][u] = __builtin_nontemporal_load(w4 + lane + kWaveSize * u);
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < kV2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = fmaf(wv[r][u][j], xv[u][j], acc);
        acc = wave::sum(acc);
        if (lane == 0)
            part[wave][r] = acc;
    }
    __syncthreads();
    if (threadIdx.x < kRows && r0 + threadIdx.x < out) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < kWavesPerBlock; ++k)
            t += part[k][threadIdx.x];
        hidden[r0 + threadIdx.x] += t;
    }
}

// ---- LM head + argmax ----------------------------------------------------------
// logits[v] = dot(E[v], RMSNorm(hidden_row)); each workgroup records its best
// (value, index); the last workgroup reduces the records. Ties go to the lowest
// index and NaN never wins (reference: include/ops/argmax.cuh:8-14); an all-NaN
// input yields 0x7fffffff.
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_argmax(float &v, int &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off);
        const int i2 = __shfl_xor(i, off);
        argmax_merge(v, i, v2, i2);
    }
}

struct LmHeadArgs {
    const float *hidden_row; // [H]
    const float *gamma;      // final norm
    const float *embed;      // [V][H]
    float *logits;           // [V]
    float *best_val;         // [grid]
    int *best_idx;           // [grid]
    unsigned *counter;       // zero-initialised, reset by the last workgroup
    StepState *state;        // next <- argmax
    int *argmax_out;         // [1]
    float eps;
    int vocab;
};

template <int kV>
__global__ __launch_bounds__(kBlock) void lm_head_argmax_kernel(LmHeadArgs a) {
    __shared__ float sv[kWavesPerBlock];
    __shared__ int si[kWavesPerBlock];
    __shared__ bool last;
    const int lane = threadIdx.x % kWaveSize, wave = threadIdx.x / kWaveSize;
    const int r0 = (blockIdx.x * kWavesPerBlock + wave) * kRows;
    float bv = kNegInf;
    int bi = 0x7fffffff;
    if (r0 < a.vocab) {
        f32x4 xn[kV];
        load_vector<kV>(a.hidden_row, a.gamma, a.eps, lane, xn);
        int row[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r)
            row[r] = r0 + r < a.vocab ? r0 + r : r0;
        float y[kRows];
        gemv_rows<kV>(a.embed, row, xn, lane, y);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            if (r0 + r < a.vocab) {
                if (lane == 0)
                    a.logits[r0 + r] = y[r];
                argmax_merge(bv, bi, y[r], r0 + r);
            }
        }
    }
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 0; k < kWavesPerBlock; ++k)
            argmax_merge(bv, bi, sv[k], si[k]);
        a.best_val[blockIdx.x] = bv;
        a.best_idx[blockIdx.x] = bi;
        __threadfence();
        last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last)
        return;
    __threadfence();
    bv = kNegInf;
    bi = 0x7fffffff;
    for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += blockDim.x)
        argmax_merge(bv, bi, __hip_atomic_load(a.best_val + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                     __hip_atomic_load(a.best_idx + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    wave_argmax(bv, bi);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 0; k < kWavesPerBlock; ++k)
            argmax_merge(bv, bi, sv[k], si[k]);
        a.argmax_out[0] = bi;
        a.state->next = bi;
        *a.counter = 0u;
    }
}

// ---- prefill glue ------------------------------------------------------------
// hidden[t][:] = embed[ids[t]][:]
__global__ __launch_bounds__(256) static void embedding_kernel(const float *__restrict__ embed,
                                                               const int *__restrict__ ids, float *__restrict__ hidden,
                                                               int rows, int H) {
    OPWORKS_GRID_LOOP(i, int64_t(rows) * H / 4) {
        const int64_t t = i / (H / 4), c = i % (H / 4);
        reinterpret_cast<f32x4 *>(hidden)[i] =
            reinterpret_cast<const f32x4 *>(embed + int64_t(ids[t]) * H)[c];
    }
}

// qkv [T][(qh + 2 kvh) D] -> RoPE(q) into q_heads [qh][T][D]; RoPE(k) and v
// appended to the caches at positions pos_start + t. One thread per rotary pair.
__global__ __launch_bounds__(256) static void rope_split_kernel(const float *__restrict__ qkv,
                                                                const float *__restrict__ inv_freq,
                                                                float *__restrict__ q_heads, float *__restrict__ kcache,
                                                                float *__restrict__ vcache, int T, int qh, int kvh,
                                                                int D, int cap, int pos_start) {
    const int half = D / 2;
    const int slots = qh + 2 * kvh;
    const int width = slots * D;
    OPWORKS_GRID_LOOP(i, int64_t(T) * slots * half) {
        const int j = static_cast<int>(i % half);
        const int slot = static_cast<int>((i / half) % slots);
        const int t = static_cast<int>(i / (int64_t(half) * slots));
        const int pos = pos_start + t;
        const float *src = qkv + int64_t(t) * width + slot * D;
        float lo = src[j], hi = src[j + half];
        if (slot < qh + kvh) {
            const float freq = static_cast<float>(pos) * inv_freq[j];
            const float c = cosf(freq), s = sinf(freq);
            const float a = lo, b = hi;
            lo = a * c - b * s;
            hi = b * c + a * s;
        }
        float *dst;
        if (slot < qh)
            dst = q_heads + (int64_t(slot) * T + t) * D;
        else if (slot < qh + kvh)
            dst = kcache + (int64_t(slot - qh) * cap + pos) * D;
        else
            dst = vcache + (int64_t(slot - qh - kvh) * cap + pos) * D;
        dst[j] = lo;
        dst[j + half] = hi;
    }
}

// attn_heads [qh][T][D] -> packed rows [T][qh * D]
__global__ __launch_bounds__(256) static void merge_heads_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                                 int T, int qh, int D) {
    OPWORKS_GRID_LOOP(i, int64_t(T) * qh * D) {
        const int d = static_cast<int>(i % D);
        const int h = static_cast<int>((i / D) % qh);
        const int t = static_cast<int>(i / (int64_t(D) * qh));
        out[i] = in[(int64_t(h) * T + t) * D + d];
    }
}

} // namespace opworks::llama
