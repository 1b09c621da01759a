#pragma once

// Kernels of the Llama decode step and prefill glue (fp32 weights).
//
// Decode step per layer (every kernel reads the step position from device
// memory, so one captured HIP graph replays every token):
//   1. qkv_rope_kernel   RMSNorm(hidden) -> fused [q;k;v] GEMV -> RoPE on q, k ->
//                        q to the workspace, k and v appended to the KV cache
//   2. decode_attention_kernel + decode_combine_kernel  split-KV partial
//                        records per 64-key chunk, merged in fixed order
//   3. gemv_residual_kernel   hidden += W_o attn
//   4. swiglu_gemv_kernel     RMSNorm(hidden) -> interleaved [gate;up] GEMV ->
//                        act = silu(gate) * up
//   5. down_residual_kernel   hidden += W_down act (K split over 4 waves)
// then lm_head_kernel (final RMSNorm + tied-embedding GEMV + per-workgroup
// argmax records) and argmax_records_kernel.
//
// GEMV shape: a wave owns one output row (LM head: four; o_proj: a quarter of
// the columns of four rows); each lane streams 16-byte packs of its rows with
// every load issued before the FMAs, and the (normalised) input vector is
// staged once per workgroup in LDS. Weight bytes are read once per token.

#include <cmath>
#include <cstdint>

#include <type_traits>

#include "../core/bf16.hpp"
#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "../core/weight_pack.hpp"
#include "../ops/argmax.hpp"
#include "../ops/attention.hpp"
#include "../ops/elementwise.hpp"

namespace opworks::llama {

using detail::f32x4;

// Device-resident state of the decode step.
struct StepState {
    int32_t token; // input token id of this step
    int32_t pos;   // its position (= KV length before the step)
    int32_t next;  // argmax result
    int32_t chain; // nonzero: the argmax kernel also records `next` in gen[pos] and advances to it
};

constexpr int kRows = 4;       // rows per workgroup of the o_proj / down GEMVs (fp32 weights)
constexpr int kLmRows = 1;     // rows per LM-head wave (fp32 weights): sizes the argmax records
constexpr int kBlock = 256;    // threads per GEMV workgroup
constexpr int kWavesPerBlock = kBlock / kWaveSize;

// Weights are streamed in 16-byte packs (core/weight_pack.hpp).
using detail::dot_wpack;
using detail::load_wpack;
using detail::u32x4;
using detail::widen;
using detail::WPack;

// Rows per wave of the two long GEMVs (gate/up, LM head) relative to fp32: a bf16 row is half
// the bytes of an fp32 row, so with bf16 weights a wave takes two rows and streams as many
// bytes as an fp32 wave, and the per-workgroup costs (staging and normalising the input
// vector, the reductions, the stores) are spread over twice the bytes (bf16 LM head 88.4 ->
// 80.5 us, gate/up 12.8 -> 12.4 us). The short matrices (qkv, o_proj, down: 2048-3072 rows)
// keep one row's share per wave: halving their workgroup count leaves CUs idle (qkv 5.26 ->
// 5.37 us, o_proj 3.90 -> 4.00 us when doubled).
template <typename WT> constexpr int kRowScale = std::is_same_v<WT, bf16> ? 2 : 1;

// GEMV of a 4-wave workgroup: each wave owns kR rows of a [*, H] matrix,
// H = 256 * kV. The input vector is staged once per workgroup: its loads are
// issued first, then every weight pack of the wave, so with in-order vmcnt
// accounting the RMS statistics are computed while the weights stream in.
// That holds only while the loads are straight-line code: a load under a
// branch (a per-lane bound, a wave that has no row) leaves the compiler
// unable to count what is outstanding at the join, and it waits for every
// load before the first use. So every load is issued, from a valid address
// (the callers give inactive waves a valid row), the barriers order LDS only,
// and the copy of x is stored after the dot products.
// The (optionally RMS-normalised) vector goes to LDS and each wave reads its
// kV packs from there. Waves with active == false still take part in the
// barriers. xn = x * rsqrtf(mean(x^2) + eps) * gamma, ops::rms_norm's order.
// The input x is fp32, or (XT = bf16: a bf16 model's embedding row at layer 0)
// bf16 widened exactly as it is loaded; copy_x_to receives the widened row.
template <typename XT> __device__ __forceinline__ f32x4 load_x4(const XT *x, int c) {
    if constexpr (std::is_same_v<XT, float>) {
        return reinterpret_cast<const f32x4 *>(x)[c];
    } else {
        const uint2 b = reinterpret_cast<const uint2 *>(x)[c]; // elements 4c .. 4c+3, low half first
        return f32x4{__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xffff0000u), __uint_as_float(b.y << 16),
                     __uint_as_float(b.y & 0xffff0000u)};
    }
}

template <int kV, int kR = kRows, typename WT = float, typename XT = float>
__device__ __forceinline__ void block_gemv(const XT *__restrict__ x, const float *__restrict__ gamma, float eps,
                                           const WT *__restrict__ W, const int (&row)[kR], bool active,
                                           float *__restrict__ copy_x_to, float (&y)[kR]) {
    constexpr int H = 256 * kV;
    constexpr int kPacks = H / 4;
    constexpr int kX = (kPacks + kBlock - 1) / kBlock; // input packs per thread
    constexpr int E = WPack<WT>::kElems;
    constexpr int kP = H / (kWaveSize * E); // weight packs per lane per row
    static_assert(kP * kWaveSize * E == H, "row width must be a multiple of 64 weight packs");
    __shared__ __attribute__((aligned(16))) float xs[H];
    __shared__ float red[kWavesPerBlock];
    const int tid = threadIdx.x, lane = tid % kWaveSize, wave = tid / kWaveSize;
    const f32x4 *g4 = reinterpret_cast<const f32x4 *>(gamma);
    f32x4 xv[kX], gv[kX];
#pragma unroll
    for (int i = 0; i < kX; ++i) {
        const int c = tid + kBlock * i, cc = c < kPacks ? c : kPacks - 1;
        xv[i] = load_x4(x, cc);
        if (gamma) // uniform
            gv[i] = g4[cc];
    }
    typename WPack<WT>::type w[kR][kP];
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int u = 0; u < kP; ++u)
            w[r][u] = load_wpack(W + int64_t(row[r]) * H, lane + kWaveSize * u);
    __builtin_amdgcn_sched_barrier(0);
    float inv = 1.f;
    if (gamma) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kX; ++i)
            if (tid + kBlock * i < kPacks)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ss = fmaf(xv[i][j], xv[i][j], ss);
        ss = wave::sum(ss);
        if (lane == 0)
            red[wave] = ss;
        detail::lds_barrier(); // the weight loads stay in flight
        inv = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / H + eps);
    }
#pragma unroll
    for (int i = 0; i < kX; ++i) {
        const int c = tid + kBlock * i;
        if (c < kPacks) {
            f32x4 v = xv[i];
            if (gamma)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[j] = v[j] * inv * gv[i][j];
            *reinterpret_cast<f32x4 *>(&xs[4 * c]) = v;
        }
    }
    detail::lds_barrier(); // each dot product waits for its own weight pack only
    if (active) {
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < kP; ++u) {
                f32x4 xl[E / 4];
#pragma unroll
                for (int q = 0; q < E / 4; ++q)
                    xl[q] = *reinterpret_cast<const f32x4 *>(&xs[E * (lane + kWaveSize * u) + 4 * q]);
                acc = dot_wpack<WT>(w[r][u], xl, acc);
            }
            y[r] = wave::sum(acc);
        }
    }
    if (copy_x_to) { // uniform; after the dot products, so no store sits between the weight loads and their uses
#pragma unroll
        for (int i = 0; i < kX; ++i) {
            const int c = tid + kBlock * i;
            if (c < kPacks)
                reinterpret_cast<f32x4 *>(copy_x_to)[c] = xv[i];
        }
    }
}

// GEMV of kRows rows by a whole workgroup, the columns split across its four
// waves: thread t owns input packs t + kBlock * i (i < kV / 4), so wave w
// covers packs w * 64 + lane + 256 * i of every row. The thread's input packs
// are exactly the ones its dot products need, so only the per-wave partial
// sums go through LDS, combined in the fixed order (w0 + w1) + (w2 + w3).
// Serves short matrices (o_proj), where it measured faster than one row per
// wave.
template <int kV, int kR, typename WT = float>
__device__ __forceinline__ void block_gemv_split(const float *__restrict__ x, const WT *__restrict__ W,
                                                 const int (&row)[kR], float (&y)[kR]) {
    constexpr int H = 256 * kV;
    constexpr int E = WPack<WT>::kElems;
    constexpr int kX = H / (kBlock * E); // weight packs per thread
    static_assert(kX * kBlock * E == H, "the split GEMV needs H to be a multiple of 256 weight packs");
    __shared__ float part[kWavesPerBlock][kR];
    const int tid = threadIdx.x, lane = tid % kWaveSize, wave = tid / kWaveSize;
    const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
    f32x4 xv[kX][E / 4];
#pragma unroll
    for (int i = 0; i < kX; ++i)
#pragma unroll
        for (int q = 0; q < E / 4; ++q)
            xv[i][q] = x4[(E / 4) * (tid + kBlock * i) + q];
    typename WPack<WT>::type w[kR][kX];
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int i = 0; i < kX; ++i)
            w[r][i] = load_wpack(W + int64_t(row[r]) * H, tid + kBlock * i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < kX; ++i)
            acc = dot_wpack<WT>(w[r][i], xv[i], acc);
        acc = wave::sum(acc);
        if (lane == 0)
            part[wave][r] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kR; ++r)
        y[r] = (part[0][r] + part[1][r]) + (part[2][r] + part[3][r]);
}

// ---- 1. QKV + RoPE + cache append ------------------------------------------
// Fused weight rows: [q heads | k heads | v heads], each head D rows.
// Workgroup g owns rotary pairs (j, j + D/2) and (j+1, j+1 + D/2) of head
// slot g / (D/4), j = 2 * (g % (D/4)). Layer 0 reads its input from the
// embedding row of the step token and also writes it to the residual stream.
template <typename WT> struct QkvArgs {
    const float *hidden_in; // residual stream (or nullptr: layer 0 reads embed[token])
    const WT *embed;        // [V][H]
    float *hidden_out;      // written only when reading from the embedding
    const float *gamma;     // input RMSNorm weight
    const WT *wqkv;         // [(qh + 2 kvh) * D][H]
    const float *inv_freq;  // [D/2]
    float *q_out;           // [qh][D]
    float *kcache, *vcache; // this layer: [kvh][cap][D]
    const StepState *state;
    float eps;
    int qh, kvh, D, cap;
};

// Rotary pair p (0 or 1) of the group: elements (j + p, j + p + D/2) of the head slot, with
// (lo, hi) = (lo c - hi s, hi c + lo s) for q and k. Each of the group's two pairs is stored by
// its own thread, so the two sincosf calls (large arguments: pos up to 8191) run side by side
// at the end of the kernel rather than four trigonometric calls one after another.
template <typename WT>
__device__ __forceinline__ void qkv_store_pair(const QkvArgs<WT> &a, int slot, int j, int pos, int p, float lo,
                                               float hi) {
    if (slot < a.qh + a.kvh) {
        const float freq = static_cast<float>(pos) * a.inv_freq[j + p];
        float s, c;
        sincosf(freq, &s, &c);
        const float rlo = lo * c - hi * s, rhi = hi * c + lo * s;
        lo = rlo;
        hi = rhi;
    }
    float *dst;
    if (slot < a.qh)
        dst = a.q_out + int64_t(slot) * a.D;
    else if (slot < a.qh + a.kvh)
        dst = a.kcache + (int64_t(slot - a.qh) * a.cap + pos) * a.D;
    else
        dst = a.vcache + (int64_t(slot - a.qh - a.kvh) * a.cap + pos) * a.D;
    dst[j + p] = lo;
    dst[j + p + a.D / 2] = hi;
}

// One workgroup per 4-row group (grid = (qh + 2 kvh) * D / 4), one row per
// wave: wave w computes row j + (w & 1) + (w >> 1) * D/2 of the head slot.
template <int kV, typename WT>
__global__ __launch_bounds__(kBlock) void qkv_rope_kernel(QkvArgs<WT> a) {
    constexpr int H = 256 * kV;
    __shared__ float res[kWavesPerBlock];
    const int g = blockIdx.x, wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int groups_per_head = a.D / 4;
    const int slot = g / groups_per_head;
    const int j = 2 * (g % groups_per_head);
    const int pos = a.state->pos;
    const int row[1] = {slot * a.D + j + (wave & 1) + (wave >> 1) * (a.D / 2)};
    float y[1];
    if (a.hidden_in)
        block_gemv<kV, 1, WT>(a.hidden_in, a.gamma, a.eps, a.wqkv, row, true, nullptr, y);
    else // layer 0: the step token's embedding row (widened if bf16); workgroup 0 also writes it into the residual stream
        block_gemv<kV, 1, WT, WT>(a.embed + int64_t(a.state->token) * H, a.gamma, a.eps, a.wqkv, row, true,
                                  g == 0 ? a.hidden_out : nullptr, y);
    if (lane == 0)
        res[wave] = y[0];
    __syncthreads();
    if (threadIdx.x < 2) // wave w holds row j + (w & 1) + (w >> 1) * D/2: pair p is (res[p], res[p + 2])
        qkv_store_pair(a, slot, j, pos, threadIdx.x, res[threadIdx.x], res[threadIdx.x + 2]);
}

// ---- 2. decode attention: split-KV partials + combine ---------------------
// ops/attention.hpp's decode kernels with the length read from the step
// state on the device (len = pos + 1), so the captured graph replays it.
using detail::DecodeAttnArgs;

// ---- 3. hidden += W x (in = H) -----------------------------------------------
template <int kV, typename WT>
__global__ __launch_bounds__(kBlock) void gemv_residual_kernel(const WT *__restrict__ W,
                                                               const float *__restrict__ x, float *__restrict__ hidden,
                                                               int out) {
    if constexpr (kV % WPack<WT>::kElems == 0) { // kRows rows per workgroup, columns split across the waves
        constexpr int kR = kRows;
        const int r0 = blockIdx.x * kR;
        const bool owner = threadIdx.x < kR && r0 + threadIdx.x < out;
        // the residual is read at the start, so its load is not a round trip in the tail
        const float resid = owner ? hidden[r0 + threadIdx.x] : 0.f;
        int row[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r)
            row[r] = r0 + r < out ? r0 + r : r0;
        float y[kR];
        block_gemv_split<kV, kR, WT>(x, W, row, y);
        if (owner) {
            float v = y[0];
#pragma unroll
            for (int r = 1; r < kR; ++r)
                v = threadIdx.x == r ? y[r] : v;
            hidden[r0 + threadIdx.x] = resid + v;
        }
    } else { // one row per wave
        const int r = blockIdx.x * kWavesPerBlock + threadIdx.x / kWaveSize;
        const bool active = r < out;
        const bool owner = active && threadIdx.x % kWaveSize == 0;
        const float resid = owner ? hidden[r] : 0.f;
        const int row[1] = {active ? r : 0};
        float y[1];
        block_gemv<kV, 1, WT>(x, nullptr, 0.f, W, row, active, nullptr, y);
        if (owner)
            hidden[r] = resid + y[0];
    }
}

// ---- 4. act = silu(gate) * up, interleaved [gate_i; up_i] rows ----------------
// fp32: workgroup b computes pairs 2b and 2b + 1, one row per wave (rows 4b .. 4b+3).
// bf16 (two rows per wave): wave w of workgroup b computes both rows of pair 4b + w.
template <int kV, typename WT>
__global__ __launch_bounds__(kBlock) void swiglu_gemv_kernel(const float *__restrict__ hidden,
                                                             const float *__restrict__ gamma, float eps,
                                                             const WT *__restrict__ wgu, float *__restrict__ act,
                                                             int inter) {
    const int wave = threadIdx.x / kWaveSize;
    if constexpr (kRowScale<WT> == 2) {
        const int i = blockIdx.x * kWavesPerBlock + wave;
        const bool active = i < inter;
        const int row[2] = {active ? 2 * i : 0, active ? 2 * i + 1 : 1};
        float y[2];
        block_gemv<kV, 2, WT>(hidden, gamma, eps, wgu, row, active, nullptr, y);
        if (active && threadIdx.x % kWaveSize == 0)
            act[i] = y[0] / (1.f + expf(-y[0])) * y[1];
        return;
    }
    __shared__ float res[kWavesPerBlock];
    const int r = blockIdx.x * kWavesPerBlock + wave;
    const bool active = r < 2 * inter;
    const int row[1] = {active ? r : 0};
    float y[1];
    block_gemv<kV, 1, WT>(hidden, gamma, eps, wgu, row, active, nullptr, y);
    if (threadIdx.x % kWaveSize == 0)
        res[wave] = y[0];
    __syncthreads();
    const int i = 2 * blockIdx.x + threadIdx.x;
    if (threadIdx.x < 2 && i < inter) {
        const float g = res[2 * threadIdx.x], u = res[2 * threadIdx.x + 1];
        act[i] = g / (1.f + expf(-g)) * u;
    }
}

// ---- 5. hidden += W_down act (in = I = 1024 * kV2), K split across 4 waves ----
template <int kV2, typename WT>
__global__ __launch_bounds__(kBlock) void down_residual_kernel(const WT *__restrict__ W,
                                                               const float *__restrict__ act,
                                                               float *__restrict__ hidden, int out) {
    constexpr int I = 1024 * kV2;
    constexpr int Kw = I / kWavesPerBlock; // columns per wave
    constexpr int E = WPack<WT>::kElems;
    constexpr int kP = Kw / (kWaveSize * E); // weight packs per lane per row
    constexpr int kR = kRows;
    static_assert(kP * kWaveSize * E == Kw, "intermediate size must split into 64-lane weight packs");
    __shared__ float part[kWavesPerBlock][kR];
    const int lane = threadIdx.x % kWaveSize, wave = threadIdx.x / kWaveSize;
    const int r0 = blockIdx.x * kR;
    const int c0 = wave * Kw;
    const bool owner = threadIdx.x < kR && r0 + threadIdx.x < out;
    const float resid = owner ? hidden[r0 + threadIdx.x] : 0.f; // read first: no round trip in the tail
    f32x4 xv[kP][E / 4];
    const f32x4 *a4 = reinterpret_cast<const f32x4 *>(act + c0);
#pragma unroll
    for (int u = 0; u < kP; ++u)
#pragma unroll
        for (int q = 0; q < E / 4; ++q)
            xv[u][q] = a4[(E / 4) * (lane + kWaveSize * u) + q];
    typename WPack<WT>::type wv[kR][kP];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int row = r0 + r < out ? r0 + r : r0;
#pragma unroll
        for (int u = 0; u < kP; ++u)
            wv[r][u] = load_wpack(W + int64_t(row) * I + c0, lane + kWaveSize * u);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < kP; ++u)
            acc = dot_wpack<WT>(wv[r][u], xv[u], acc);
        acc = wave::sum(acc);
        if (lane == 0)
            part[wave][r] = acc;
    }
    __syncthreads();
    if (owner) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < kWavesPerBlock; ++k)
            t += part[k][threadIdx.x];
        hidden[r0 + threadIdx.x] = resid + t;
    }
}

// ---- LM head + argmax ----------------------------------------------------------
// logits[v] = dot(E[v], RMSNorm(hidden_row)); each workgroup records its best
// (value, index); the last workgroup reduces the records. Ties go to the lowest
// index and NaN never wins (reference: include/ops/argmax.cuh:8-14); an all-NaN
// input yields 0x7fffffff.
using detail::argmax_merge;
using detail::wave_argmax;

template <typename WT> struct LmHeadArgs {
    const float *hidden_row; // [H]
    const float *gamma;      // final norm
    const WT *embed;         // [V][H]
    float *logits;           // [V]
    float *best_val;         // [grid]
    int *best_idx;           // [grid]
    float eps;
    int vocab;
};

template <int kV, typename WT>
__global__ __launch_bounds__(kBlock) void lm_head_kernel(LmHeadArgs<WT> a) {
    __shared__ float sv[kWavesPerBlock];
    __shared__ int si[kWavesPerBlock];
    const int lane = threadIdx.x % kWaveSize, wave = threadIdx.x / kWaveSize;
    constexpr int kLR = kLmRows * kRowScale<WT>;
    const int r0 = (blockIdx.x * kWavesPerBlock + wave) * kLR;
    int row[kLR];
#pragma unroll
    for (int r = 0; r < kLR; ++r)
        row[r] = r0 + r < a.vocab ? r0 + r : 0;
    float y[kLR];
    block_gemv<kV, kLR, WT>(a.hidden_row, a.gamma, a.eps, a.embed, row, r0 < a.vocab, nullptr, y);
    float bv = kNegInf;
    int bi = 0x7fffffff;
    if (r0 < a.vocab) {
#pragma unroll
        for (int r = 0; r < kLR; ++r) {
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
    }
}

// kArgmaxGroups workgroups of 256 lanes reduce the LM head's per-workgroup
// records: workgroup g takes records [g * per, (g + 1) * per) down to one
// (value, index) partial and publishes it with agent-coherent stores; once
// they have completed it counts itself in on `counter`, and the last to arrive
// merges the partials (agent-coherent loads), resets the counter and advances
// the step state. This is the protocol of the fused decode-attention merge.
// The merge is order-independent (largest value, then lowest index), so the
// result does not depend on which workgroup arrives last. (One 1024-lane
// workgroup over the 32064 records of the fp32 LM head took 8.1 us.)
// A chained step whose logits hold no winner (every logit NaN: index 0x7fffffff) or any index
// outside [0, vocab) records it in gen[pos] and stops the chain instead of advancing: the token
// and position stay those of the step just run, so the steps still queued behind it recompute
// that step in place (same inputs, same cache row) and no kernel reads an embedding row past
// the table. The host sees chain == 0 with that index in `next`.
constexpr int kArgmaxGroups = 64;
__global__ __launch_bounds__(256) static void argmax_records_kernel(const float *__restrict__ best_val,
                                                                    const int *__restrict__ best_idx, int count,
                                                                    float *part_val, int *part_idx, int *counter,
                                                                    StepState *state, int *gen, int vocab) {
    __shared__ float sv[256 / kWaveSize];
    __shared__ int si[256 / kWaveSize];
    __shared__ int last;
    const int lane = threadIdx.x % kWaveSize, wave = threadIdx.x / kWaveSize;
    const int per = (count + kArgmaxGroups - 1) / kArgmaxGroups;
    const int b0 = blockIdx.x * per, b1 = b0 + per < count ? b0 + per : count;
    float bv = kNegInf;
    int bi = 0x7fffffff;
    constexpr int kBatch = 4;
    for (int base = b0 + threadIdx.x; base < b1; base += kBatch * 256) {
        float v[kBatch];
        int ix[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int b = base + u * 256;
            v[u] = b < b1 ? best_val[b] : kNegInf;
            ix[u] = b < b1 ? best_idx[b] : 0x7fffffff;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            argmax_merge(bv, bi, v[u], ix[u]);
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 0; k < 256 / kWaveSize; ++k)
            argmax_merge(bv, bi, sv[k], si[k]);
        __hip_atomic_store(part_val + blockIdx.x, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part_idx + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(detail::kWaitVmcnt0); // the partial has completed
        last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kArgmaxGroups - 1;
    }
    __syncthreads();
    if (!last || wave != 0)
        return;
    float v = kNegInf;
    int ix = 0x7fffffff;
    if (lane < kArgmaxGroups) {
        v = __hip_atomic_load(part_val + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ix = __hip_atomic_load(part_idx + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wave_argmax(v, ix);
    if (lane == 0) {
        __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        state->next = ix;
        if (state->chain) { // greedy chaining: the next launch decodes this token at pos + 1
            gen[state->pos] = ix;
            if (ix >= 0 && ix < vocab) {
                state->token = ix;
                state->pos += 1;
            } else {
                state->chain = 0;
            }
        }
    }
}
static_assert(kArgmaxGroups <= kWaveSize, "one wave merges the partials");

// ---- prefill glue ------------------------------------------------------------
// hidden[t][:] = embed[ids[t]][:] (bf16 rows widened), one 16-byte pack of
// the table per thread
template <typename WT>
__global__ __launch_bounds__(256) void embedding_kernel(const WT *__restrict__ embed, const int *__restrict__ ids,
                                                        float *__restrict__ hidden, int rows, int H) {
    constexpr int E = WPack<WT>::kElems;
    const int per_row = H / E;
    OPWORKS_GRID_LOOP(i, int64_t(rows) * per_row) {
        const int64_t t = i / per_row, c = i % per_row;
        const typename WPack<WT>::type v =
            reinterpret_cast<const typename WPack<WT>::type *>(embed + int64_t(ids[t]) * H)[c];
        f32x4 *dst = reinterpret_cast<f32x4 *>(hidden + t * H + c * E);
#pragma unroll
        for (int q = 0; q < E / 4; ++q)
            dst[q] = f32x4{WPack<WT>::at(v, 4 * q), WPack<WT>::at(v, 4 * q + 1), WPack<WT>::at(v, 4 * q + 2),
                           WPack<WT>::at(v, 4 * q + 3)};
    }
}

// hidden = embed[state.token] widened to fp32: the "after embedding" capture of a
// bf16 model's single-row debug prefill (the decode step itself reads the row in
// layer 0's qkv kernel).
template <typename WT>
__global__ __launch_bounds__(256) void embed_token_kernel(const WT *__restrict__ embed,
                                                          const StepState *__restrict__ state,
                                                          float *__restrict__ hidden, int H) {
    const WT *row = embed + int64_t(state->token) * H;
    OPWORKS_GRID_LOOP(i, H) { hidden[i] = widen(row[i]); }
}

// qkv [T][(qh + 2 kvh) D] -> RoPE(q) into q_heads [qh][T][D]; RoPE(k) and v
// appended to the caches at positions pos_start + t. One thread per rotary pair.
// splits > 0: qkv holds the split-K partials of the projection instead, `splits`
// slices of [T][width], summed here in split order and then + 0.f, exactly as
// splitk_reduce_kernel would have stored them (one pass and one launch fewer).
__global__ __launch_bounds__(256) static void rope_split_kernel(const float *__restrict__ qkv, int splits,
                                                                const float *__restrict__ inv_freq,
                                                                float *__restrict__ q_heads, float *__restrict__ kcache,
                                                                float *__restrict__ vcache, int T, int qh, int kvh,
                                                                int D, int cap, int pos_start) {
    const int half = D / 2;
    const int slots = qh + 2 * kvh;
    const int width = slots * D;
    const int64_t slice = int64_t(T) * width;
    OPWORKS_GRID_LOOP(i, int64_t(T) * slots * half) {
        const int j = static_cast<int>(i % half);
        const int slot = static_cast<int>((i / half) % slots);
        const int t = static_cast<int>(i / (int64_t(half) * slots));
        const int pos = pos_start + t;
        const float *src = qkv + int64_t(t) * width + slot * D;
        float lo = src[j], hi = src[j + half];
        if (splits > 0) { // uniform
            for (int sp = 1; sp < splits; ++sp) {
                lo = lo + src[sp * slice + j];
                hi = hi + src[sp * slice + j + half];
            }
            lo = lo + 0.f;
            hi = hi + 0.f;
        }
        if (slot < qh + kvh) {
            const float freq = static_cast<float>(pos) * inv_freq[j];
            float s, c;
            sincosf(freq, &s, &c); // as the decode step's qkv_store_pair, so both fill the cache alike
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

} // namespace opworks::llama
