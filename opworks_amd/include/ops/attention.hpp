#pragma once

// Causal GQA attention over a KV cache, fp32.
//
// Layouts (reference: include/ops/attention_prefill.cuh:21-24,
// include/ops/attention_decode.cuh:8-11):
//   q_heads [qh][T][D]   queries at absolute positions q_offset + [0, T)
//   k/v cache [kvh][cap][D], S valid entries; kv head of q head h = h / kv_rep
//   out [qh][T][D]
// A query at position p sees keys 0..min(p, S-1); scores are scaled by
// 1/sqrt(D); a row that sees no key writes zeros.
//
// ---- prefill (flash) -----------------------------------------------------
// One workgroup = one kv head x one 32-query tile, with one wave per q head of
// the GQA group, so each K/V tile is read from HBM once per group and shared
// through LDS (double buffered). Each wave computes the transposed products
//   S^T = K Q^T  and  O^T += V^T P^T
// on v_mfma_f32_32x32x2_f32. In that orientation lane l owns query l % 32:
// the online-softmax max and sum are register reductions plus one exchange
// between the two lane halves, and the rescale of O is a
// per-lane multiply. Inside an MFMA chain, step s = 4g + j of lane half h
// uses reduction index 8g + 4h + j; with that order the S^T accumulator
// register r = 4g + j of a lane is exactly the P^T operand that lane supplies
// at step s of the P V chain, so P never moves. Q stays in registers.
// Workgroups start with the longest (last) query tiles.
//
// ---- decode (split-KV) ---------------------------------------------------
// One workgroup = one kv head x one chunk of kAttnChunk keys: the chunk's K/V
// rows are read once for all q heads of the group, each wave (one q head)
// produces a partial (max, sum, unnormalised output) for the chunk, and a
// combine kernel merges the chunks. The valid length can be read from device
// memory, so one graph serves every decode position.

#include <cmath>
#include <cstdint>

#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "elementwise.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

constexpr int kAttnTile = 32;      // queries per wave, keys per KV tile
constexpr int kAttnMaxD = 64;
constexpr int kAttnLdK = 64 + 4;   // padded K row (floats)
constexpr int kAttnLdV = 64 + 8;   // padded V row (floats)
constexpr int kAttnMaxRep = 16;    // q heads per kv head (waves per workgroup)

// v[l] (+) v[l ^ 32] in every lane (ds_bpermute exchange between the lane halves).
template <typename Combine> __device__ __forceinline__ float half_combine(float v, Combine c) {
    return c(v, __shfl_xor(v, 32));
}

// kDT = number of 32-wide head-dim tiles (D padded to 32 * kDT); kWaves = q
// heads handled by one workgroup (a GQA group, or an 8-head slice of a larger one).
template <int kDT, int kWaves> struct PrefillShape {
    static constexpr int kDp = 32 * kDT;
    static constexpr int kStage = kAttnTile * (kAttnLdK + kAttnLdV); // floats per K/V stage
    static constexpr int kOut = kWaves * kAttnTile * (kDp + 1);      // floats of the output transpose
    static constexpr int kLdsFloats = 2 * kStage > kOut ? 2 * kStage : kOut;
    static constexpr int kChunks = kAttnTile * kDp / 4;               // float4 chunks per K (or V) tile
    static constexpr int kPerThread = (kChunks + kWaves * kWaveSize - 1) / (kWaves * kWaveSize);
};

template <int kDT, int kWaves>
__global__ __launch_bounds__(kWaves *kWaveSize) void attention_prefill_kernel(
    const float *__restrict__ q_heads, const float *__restrict__ kcache, const float *__restrict__ vcache,
    float *__restrict__ out, int T, int S, int q_offset, int head_dim, int kv_rep, int num_kv_heads, int cap,
    float scale) {
    using Shape = PrefillShape<kDT, kWaves>;
    constexpr int kDp = Shape::kDp;
    constexpr int kStage = Shape::kStage;
    extern __shared__ __attribute__((aligned(16))) float lds[];

    const int slices = (kv_rep + kWaves - 1) / kWaves; // workgroups per GQA group
    const int ntq = (T + kAttnTile - 1) / kAttnTile;
    const int per_tile = num_kv_heads * slices;
    const int qt = ntq - 1 - static_cast<int>(blockIdx.x) / per_tile; // longest tiles first
    const int kvh = (static_cast<int>(blockIdx.x) % per_tile) / slices;
    const int slice = static_cast<int>(blockIdx.x) % slices;
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int l32 = lane % 32, half = lane / 32;
    const int rep = slice * kWaves + wave;               // head within the group
    const bool head_ok = rep < kv_rep;                   // idle waves still join barriers
    const int h = kvh * kv_rep + (head_ok ? rep : 0);
    const int q0 = qt * kAttnTile;

    const float *kh = kcache + int64_t(kvh) * cap * head_dim;
    const float *vh = vcache + int64_t(kvh) * cap * head_dim;

    // Q^T operand: lane (q = l32, half) keeps Q[q][8g + 4*half + 0..3].
    constexpr int kG = kDp / 8;
    f32x4 qreg[kG];
    {
        const int q = q0 + l32;
        const float *qrow = q_heads + (int64_t(h) * T + (q < T ? q : 0)) * head_dim;
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const int d = 8 * g + 4 * half;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                qreg[g][j] = (q < T && d + j < head_dim) ? qrow[d + j] : 0.f;
        }
    }

    const int kv_end = (q_offset + q0 + kAttnTile) < S ? (q_offset + q0 + kAttnTile) : S;
    const int ntiles = (kv_end + kAttnTile - 1) / kAttnTile;

    // K/V tile staging through registers: chunk c = tid + i * threads covers row c / (kDp/4).
    constexpr int kChunksPerRow = kDp / 4;
    const bool vec = (head_dim % 4 == 0);
    f32x4 kst[Shape::kPerThread], vst[Shape::kPerThread];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < Shape::kPerThread; ++i) {
            const int c = threadIdx.x + i * kWaves * kWaveSize;
            const int r = c / kChunksPerRow, d = (c % kChunksPerRow) * 4;
            const int key = kt * kAttnTile + r;
            kst[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            vst[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (c < Shape::kChunks && key < S) {
                if (vec) {
                    if (d < head_dim) {
                        kst[i] = *reinterpret_cast<const f32x4 *>(kh + int64_t(key) * head_dim + d);
                        vst[i] = *reinterpret_cast<const f32x4 *>(vh + int64_t(key) * head_dim + d);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        kst[i][j] = d + j < head_dim ? kh[int64_t(key) * head_dim + d + j] : 0.f;
                        vst[i][j] = d + j < head_dim ? vh[int64_t(key) * head_dim + d + j] : 0.f;
                    }
                }
            }
        }
    };
    auto commit = [&](int buf) {
        float *Ks = lds + buf * kStage;
        float *Vs = Ks + kAttnTile * kAttnLdK;
#pragma unroll
        for (int i = 0; i < Shape::kPerThread; ++i) {
            const int c = threadIdx.x + i * kWaves * kWaveSize;
            if (c < Shape::kChunks) {
                const int r = c / kChunksPerRow, d = (c % kChunksPerRow) * 4;
                *reinterpret_cast<f32x4 *>(Ks + r * kAttnLdK + d) = kst[i];
                *reinterpret_cast<f32x4 *>(Vs + r * kAttnLdV + d) = vst[i];
            }
        }
    };

    f32x16 oacc[kDT];
#pragma unroll
    for (int t = 0; t < kDT; ++t)
        oacc[t] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;
    const int qpos = q_offset + q0 + l32; // this lane's query position

    if (ntiles > 0) {
        fetch(0);
        commit(0);
        __syncthreads();
    }
    for (int kt = 0; kt < ntiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ntiles)
            fetch(kt + 1); // global loads in flight during this tile's MFMAs
        const float *Ks = lds + buf * kStage;
        const float *Vs = Ks + kAttnTile * kAttnLdK;

        // S^T[key][q] = sum_d K[key][d] Q[q][d]
        f32x16 sacc = f32x16{};
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            const f32x4 kv = *reinterpret_cast<const f32x4 *>(Ks + l32 * kAttnLdK + 8 * g + 4 * half);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[j], qreg[g][j], sacc, 0, 0, 0);
        }
        // scale, mask, online softmax (register r holds key 8*(r/4) + 4*half + r%4 of this tile)
        float tmax = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kt * kAttnTile + 8 * (r / 4) + 4 * half + (r % 4);
            const float s = (key < S && key <= qpos) ? sacc[r] * scale : kNegInf;
            sacc[r] = s;
            tmax = fmaxf(tmax, s);
        }
        tmax = half_combine(tmax, wave::Max{});
        const float m_new = fmaxf(m_run, tmax);
        const float corr = m_run == kNegInf ? 0.f : expf(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = sacc[r] == kNegInf ? 0.f : expf(sacc[r] - m_new);
            sacc[r] = p;
            psum += p;
        }
        psum = half_combine(psum, wave::Add{});
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < kDT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                oacc[t][r] *= corr;
        // O^T[d][q] += sum_key V[key][d] P^T[key][q]
#pragma unroll
        for (int t = 0; t < kDT; ++t) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float v = Vs[(8 * g + 4 * half + j) * kAttnLdV + 32 * t + l32];
                    oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(v, sacc[4 * g + j], oacc[t], 0, 0, 0);
                }
            }
        }
        if (kt + 1 < ntiles)
            commit(buf ^ 1); // that buffer was last read before the previous barrier
        __syncthreads();
    }

    // Transpose O^T through LDS (a private 32 x kDp block per wave), then store rows.
    float *Os = lds + wave * kAttnTile * (kDp + 1);
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int t = 0; t < kDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            Os[l32 * (kDp + 1) + 32 * t + 8 * (r / 4) + 4 * half + (r % 4)] = oacc[t][r] * inv;
    __syncthreads();
    if (head_ok) {
        for (int i = lane; i < kAttnTile * head_dim; i += kWaveSize) {
            const int q = i / head_dim, d = i % head_dim;
            if (q0 + q < T)
                out[(int64_t(h) * T + q0 + q) * head_dim + d] = Os[q * (kDp + 1) + d];
        }
    }
}

template <int kDT, int kWaves>
inline void attention_prefill_launch(const float *q, const float *k, const float *v, float *out, int T, int S,
                                     int q_offset, int head_dim, int kv_rep, int kvh, int cap, float scale,
                                     hipStream_t stream) {
    using Shape = PrefillShape<kDT, kWaves>;
    const int slices = (kv_rep + kWaves - 1) / kWaves;
    const int grid = static_cast<int>(blocks_for64(T, kAttnTile)) * kvh * slices;
    launch_async_lds(stream, sizeof(float) * Shape::kLdsFloats, attention_prefill_kernel<kDT, kWaves>, grid,
                     kWaves * kWaveSize, q, k, v, out, T, S, q_offset, head_dim, kv_rep, kvh, cap, scale);
}

template <int kDT>
inline void attention_prefill_dispatch(const float *q, const float *k, const float *v, float *out, int T, int S,
                                       int q_offset, int head_dim, int kv_rep, int kvh, int cap, float scale,
                                       hipStream_t stream) {
    if (kv_rep == 1)
        attention_prefill_launch<kDT, 1>(q, k, v, out, T, S, q_offset, head_dim, kv_rep, kvh, cap, scale, stream);
    else if (kv_rep == 2)
        attention_prefill_launch<kDT, 2>(q, k, v, out, T, S, q_offset, head_dim, kv_rep, kvh, cap, scale, stream);
    else if (kv_rep <= 4)
        attention_prefill_launch<kDT, 4>(q, k, v, out, T, S, q_offset, head_dim, kv_rep, kvh, cap, scale, stream);
    else
        attention_prefill_launch<kDT, 8>(q, k, v, out, T, S, q_offset, head_dim, kv_rep, kvh, cap, scale, stream);
}

// ---------------------------------------------------------------- decode
constexpr int kAttnChunk = 64;       // keys per decode workgroup
constexpr int kAttnDecodeMaxLen = 8192;
constexpr int kAttnMaxChunks = kAttnDecodeMaxLen / kAttnChunk;

// Partial record per (q head, chunk): [0] max, [1] sum, [2..2+D) unnormalised output.
inline int attention_decode_workspace_floats(int num_q_heads, int max_len, int head_dim) {
    const int chunks = (max_len + kAttnChunk - 1) / kAttnChunk;
    return num_q_heads * chunks * (head_dim + 2);
}

// Split-KV decode ("flash-decoding"): one workgroup per (kv head, chunk of
// kAttnChunk keys) stages the chunk's K/V rows in LDS with 16-byte loads
// (all issued before the LDS stores); wave w handles q head kvh * kv_rep + w:
// lane = key for the scores (four partial dot products), then lane = head-dim
// element for P V. Each chunk leaves a record (max, sum, unnormalised
// output[D]); the combine kernel (one wave per q head) merges a head's
// records in chunk order: M = max m_c, L = sum l_c e^(m_c - M),
// out = sum acc_c e^(m_c - M) / L, loading 16 chunk rows per round trip.
// The length is a host value or, for graph replay, read on the device.
struct DecodeAttnArgs {
    const float *q;               // [qh][D]
    const float *kcache, *vcache; // [kvh][cap][D]
    float *out;                   // [qh][D]
    float *partial;               // [qh][max_chunks][D + 2]
    const int *len_ptr;           // if set, length = *len_ptr + len_bias
    int len, len_bias;
    int kv_rep, D, cap, max_chunks;
    float scale;
};

__device__ __forceinline__ int decode_len(const DecodeAttnArgs &a) {
    int len = a.len_ptr ? *a.len_ptr + a.len_bias : a.len;
    len = len < a.cap ? len : a.cap;
    return len < a.max_chunks * kAttnChunk ? len : a.max_chunks * kAttnChunk;
}

template <int kWaves>
__global__ __launch_bounds__(kWaves *kWaveSize) void attention_decode_partial_kernel(DecodeAttnArgs a) {
    constexpr int C = kAttnChunk;
    const int len = decode_len(a);
    const int nchunks = (len + C - 1) / C;
    const int kvh = blockIdx.x, chunk = blockIdx.y;
    if (chunk >= nchunks)
        return;
    const int k0 = chunk * C;
    const int n = len - k0 < C ? len - k0 : C;
    const int D = a.D;
    __shared__ __attribute__((aligned(16))) float Ks[C][kAttnMaxD + 4];
    __shared__ __attribute__((aligned(16))) float Vs[C][kAttnMaxD];
    __shared__ __attribute__((aligned(16))) float Qs[kWaves][kAttnMaxD];
    __shared__ __attribute__((aligned(16))) float Ps[kWaves][C];
    const float *kh = a.kcache + (int64_t(kvh) * a.cap + k0) * D;
    const float *vh = a.vcache + (int64_t(kvh) * a.cap + k0) * D;
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const bool head_ok = wave < a.kv_rep;
    const int h = kvh * a.kv_rep + (head_ok ? wave : 0);
    {
        constexpr int kMaxPer = C * kAttnMaxD / 4 / (kWaves * kWaveSize);
        constexpr int nthreads = kWaves * kWaveSize;
        const int packs = C * D / 4;
        f32x4 kv[kMaxPer], vv[kMaxPer];
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int c = threadIdx.x + i * nthreads;
            const int r = (4 * c) / D;
            kv[i] = vv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (c < packs && r < n) {
                kv[i] = reinterpret_cast<const f32x4 *>(kh)[c];
                vv[i] = reinterpret_cast<const f32x4 *>(vh)[c];
            }
        }
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int c = threadIdx.x + i * nthreads;
            if (c < packs) {
                const int r = (4 * c) / D, d = (4 * c) % D;
                *reinterpret_cast<f32x4 *>(&Ks[r][d]) = kv[i];
                *reinterpret_cast<f32x4 *>(&Vs[r][d]) = vv[i];
            }
        }
    }
    if (lane < D)
        Qs[wave][lane] = a.q[int64_t(h) * D + lane];
    __syncthreads();
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    for (int d = 0; d < D; d += 4) {
        const f32x4 kq = *reinterpret_cast<const f32x4 *>(&Ks[lane][d]);
        const f32x4 qv = *reinterpret_cast<const f32x4 *>(&Qs[wave][d]);
        s0 = fmaf(qv[0], kq[0], s0);
        s1 = fmaf(qv[1], kq[1], s1);
        s2 = fmaf(qv[2], kq[2], s2);
        s3 = fmaf(qv[3], kq[3], s3);
    }
    const float s = lane < n ? ((s0 + s1) + (s2 + s3)) * a.scale : kNegInf;
    const float m = wave::max(s);
    const float p = lane < n ? expf(s - m) : 0.f;
    const float l = wave::sum(p);
    Ps[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    // lane = head-dim element; keys past n have p = 0 and zero V rows
    if (lane < D) {
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll 4
        for (int key = 0; key < C; key += 4) {
            const f32x4 pv = *reinterpret_cast<const f32x4 *>(&Ps[wave][key]);
            o0 = fmaf(pv[0], Vs[key][lane], o0);
            o1 = fmaf(pv[1], Vs[key + 1][lane], o1);
            o2 = fmaf(pv[2], Vs[key + 2][lane], o2);
            o3 = fmaf(pv[3], Vs[key + 3][lane], o3);
        }
        if (head_ok) {
            float *rec = a.partial + (int64_t(h) * a.max_chunks + chunk) * (D + 2);
            if (lane == 0) {
                rec[0] = m;
                rec[1] = l;
            }
            rec[2 + lane] = (o0 + o1) + (o2 + o3);
        }
    }
}

// grid kvh, block kv_rep waves; wave w merges q head kvh * kv_rep + w.
__global__ __launch_bounds__(kAttnMaxRep *kWaveSize) static void attention_decode_combine_kernel(DecodeAttnArgs a) {
    constexpr int C = kAttnChunk;
    const int len = decode_len(a);
    const int nchunks = (len + C - 1) / C; // <= max_chunks <= 2 * kWaveSize
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int h = blockIdx.x * a.kv_rep + wave;
    const int D = a.D;
    const float *base = a.partial + int64_t(h) * a.max_chunks * (D + 2);
    float m0 = kNegInf, l0 = 0.f, m1 = kNegInf, l1 = 0.f;
    if (lane < nchunks) {
        m0 = base[int64_t(lane) * (D + 2)];
        l0 = base[int64_t(lane) * (D + 2) + 1];
    }
    if (lane + kWaveSize < nchunks) {
        m1 = base[int64_t(lane + kWaveSize) * (D + 2)];
        l1 = base[int64_t(lane + kWaveSize) * (D + 2) + 1];
    }
    const float M = wave::max(fmaxf(m0, m1));
    const float w0 = lane < nchunks ? expf(m0 - M) : 0.f;
    const float w1 = lane + kWaveSize < nchunks ? expf(m1 - M) : 0.f;
    const float L = wave::sum(l0 * w0 + l1 * w1);
    constexpr int kBatch = 16;
    float acc = 0.f;
    for (int c0 = 0; c0 < nchunks; c0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            v[j] = c0 + j < nchunks && lane < D ? base[int64_t(c0 + j) * (D + 2) + 2 + lane] : 0.f;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int c = c0 + j;
            const float wc = wave::readlane(c < kWaveSize ? w0 : w1, c % kWaveSize);
            acc = c < nchunks ? fmaf(v[j], wc, acc) : acc;
        }
    }
    if (lane < D)
        a.out[int64_t(h) * D + lane] = L > 0.f ? acc / L : 0.f;
}

// Enqueues the partial and combine kernels: grid (kvh, max_chunks) with
// kv_rep rounded up to a power of two waves per workgroup.
inline void attention_decode_launch(const DecodeAttnArgs &a, int kvh, hipStream_t stream) {
    const dim3 grid(kvh, a.max_chunks);
    const int rep = a.kv_rep;
    if (rep <= 1)
        launch_async(stream, attention_decode_partial_kernel<1>, grid, kWaveSize, a);
    else if (rep <= 2)
        launch_async(stream, attention_decode_partial_kernel<2>, grid, 2 * kWaveSize, a);
    else if (rep <= 4)
        launch_async(stream, attention_decode_partial_kernel<4>, grid, 4 * kWaveSize, a);
    else if (rep <= 8)
        launch_async(stream, attention_decode_partial_kernel<8>, grid, 8 * kWaveSize, a);
    else
        launch_async(stream, attention_decode_partial_kernel<16>, grid, 16 * kWaveSize, a);
    launch_async(stream, attention_decode_combine_kernel, kvh, rep * kWaveSize, a);
}

} // namespace opworks::detail

namespace opworks::ops {

// Flash-style causal prefill over the cache (reference:
// ops::attention_prefill_chunked, include/ops/attention_prefill.cuh:164-177).
inline void attention_prefill(const float *q_heads, const float *kcache, const float *vcache, float *out, int T,
                              int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap,
                              hipStream_t stream = nullptr) {
    detail::require(T > 0 && S >= T && q_offset == S - T, "attention_prefill: bad shape/offset");
    detail::require(num_q_heads > 0 && kv_rep > 0 && num_q_heads % kv_rep == 0, "attention_prefill: bad head shape");
    detail::require(head_dim > 0 && head_dim <= detail::kAttnMaxD && head_dim % 16 == 0,
                    "attention_prefill supports head_dim in {16,32,48,64}");
    detail::require(cap >= S, "attention_prefill: length exceeds cache capacity");
    detail::require(q_heads && kcache && vcache && out, "attention_prefill requires non-null pointers");
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    const int kvh = num_q_heads / kv_rep;
    if (head_dim <= 32)
        detail::attention_prefill_dispatch<1>(q_heads, kcache, vcache, out, T, S, q_offset, head_dim, kv_rep, kvh, cap,
                                              scale, stream);
    else
        detail::attention_prefill_dispatch<2>(q_heads, kcache, vcache, out, T, S, q_offset, head_dim, kv_rep, kvh, cap,
                                              scale, stream);
}

// Same contract as the reference's chunked prefill (name kept for drop-in callers).
inline void attention_prefill_chunked(const float *q_heads, const float *kcache, const float *vcache, float *out,
                                      int T, int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap,
                                      hipStream_t stream = nullptr) {
    attention_prefill(q_heads, kcache, vcache, out, T, S, q_offset, num_q_heads, kv_rep, head_dim, cap, stream);
}

inline int attention_decode_workspace_size(int num_q_heads, int max_len, int head_dim) {
    return detail::attention_decode_workspace_floats(num_q_heads, max_len, head_dim);
}

// Single-query GQA attention over the first len cache entries, workspace form
// (no allocation; graph-capturable). If len_ptr is non-null the length is
// *len_ptr + len_bias, read on the device, and max_len bounds it.
inline void attention_decode_ws(const float *q, const float *kcache, const float *vcache, float *out,
                                int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                int workspace_size, const int *len_ptr = nullptr, int len_bias = 0,
                                int max_len = 0, hipStream_t stream = nullptr) {
    detail::require(num_q_heads > 0 && kv_rep > 0 && head_dim > 0 && num_q_heads % kv_rep == 0,
                    "attention_decode requires positive head shape");
    detail::require(kv_rep <= detail::kAttnMaxRep, "attention_decode supports at most 16 q heads per kv head");
    detail::require(head_dim <= 64, "attention_decode supports head_dim <= 64");
    const int bound = len_ptr ? max_len : len;
    detail::require(bound > 0 && bound <= max_seq, "attention_decode length outside the cache capacity");
    detail::require(bound <= detail::kAttnDecodeMaxLen, "attention_decode length exceeds 8192");
    detail::require(q && kcache && vcache && out && workspace, "attention_decode requires non-null pointers");
    const int max_chunks = (bound + detail::kAttnChunk - 1) / detail::kAttnChunk;
    detail::require(workspace_size >= num_q_heads * max_chunks * (head_dim + 2), "attention_decode workspace is too small");
    detail::require(head_dim % 4 == 0, "attention_decode needs head_dim to be a multiple of 4");
    detail::require(detail::aligned16(q) && detail::aligned16(kcache) && detail::aligned16(vcache),
                    "attention_decode needs 16-byte aligned q and caches");
    detail::DecodeAttnArgs a{};
    a.q = q;
    a.kcache = kcache;
    a.vcache = vcache;
    a.out = out;
    a.partial = workspace;
    a.len_ptr = len_ptr;
    a.len = len;
    a.len_bias = len_bias;
    a.kv_rep = kv_rep;
    a.D = head_dim;
    a.cap = max_seq;
    a.max_chunks = max_chunks;
    a.scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    detail::attention_decode_launch(a, num_q_heads / kv_rep, stream);
}

// Reference signature (include/ops/attention_decode.cuh:99-109): scratch comes
// from stream-ordered allocation.
inline void attention_decode(const float *q, const float *kcache, const float *vcache, float *out, int num_q_heads,
                             int kv_rep, int head_dim, int len, int max_seq, hipStream_t stream = nullptr) {
    detail::require(num_q_heads > 0 && kv_rep > 0 && head_dim > 0, "attention_decode requires positive head shape");
    detail::require(len > 0 && len <= max_seq, "attention_decode length outside the cache capacity");
    detail::require(len <= detail::kAttnDecodeMaxLen, "attention_decode length exceeds the shared-memory kernel limit");
    const int ws = attention_decode_workspace_size(num_q_heads, len, head_dim);
    float *scratch = nullptr;
    OPWORKS_HIP_CHECK(hipMallocAsync(reinterpret_cast<void **>(&scratch), sizeof(float) * ws, stream));
    attention_decode_ws(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq, scratch, ws, nullptr, 0,
                        0, stream);
    OPWORKS_HIP_CHECK(hipFreeAsync(scratch, stream));
}

} // namespace opworks::ops
