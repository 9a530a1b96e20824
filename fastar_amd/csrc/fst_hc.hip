// fst_hc.hip — Hyper-Connections (HC) around the MoE for gfx950.
//
// The residual of an HC model is 4 streams of width d per token
// (include/fst_engine.h:98-106).  Around the FFN (src/fst_engine.cpp:2734-2740,
// :2914-2917) the engine runs
//   hc_pre  (:2350-2392): flat = rms_norm_no_weight(h) over 4d, mix = flat . fn
//            (24 outputs, the NPU control matvec :694-742), a Sinkhorn split
//            into pre[4], post[4], comb[4x4], and cur = sum_h pre[h] h[h];
//   hc_post (:2394-2414): h'[dst] = bo * post[dst] + sum_src comb[dst + 4 src] h[src];
// and before the LM head output_hc_head (:2416-2459) collapses the streams
// with sigmoid weights from a 4-output control matvec.
//
// Fixed orders where the reference leaves them to the NPU or libm (restated
// by the CPU oracle, so results are bit-identical to it):
//   sum of squares in double: 64 partials of contiguous chunks + halving tree;
//   control matvec: per 1024-wide K chunk, 16 sequential-fmaf partials of 64
//   products and a halving tree, the chunk sum rounded to bf16, chunk sums
//   added in order in float, the total rounded to bf16;
//   exp is fst_expf; bf16 rounding is RNE; no floating contraction.
#include "fst_internal.h"
#include "../../include/fst_exact_math.h"

namespace fst {

#pragma clang fp contract(off)

constexpr int kHcN = 4;
constexpr int kHcMix = 2 * kHcN + kHcN * kHcN;  // 24
constexpr int kHcIters = 20;
constexpr float kHcEps = 1e-6f;
constexpr int kHcMaxK = 4 * 8192;
constexpr int kHcThreads = 256;

__device__ __forceinline__ float bf(uint16_t v) { return fst_bf16_to_f32(v); }
__device__ __forceinline__ uint16_t rb(float v) { return fst_f32_to_bf16(v); }

// flat = bf16(r * inv_rms(r)) into LDS (K values of the token's 4 streams).
__device__ void hc_flat(const uint16_t* __restrict__ r, int K, uint16_t* flat) {
    __shared__ double part[64];
    __shared__ float s_inv;
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int C = K / 64;
        double a = 0.0;
        for (int i = 0; i < C; ++i) {
            const double v = (double)bf(r[tid * C + i]);
            a = a + v * v;
        }
        part[tid] = a;
    }
    __syncthreads();
    if (tid == 0) {
        for (int off = 32; off >= 1; off >>= 1)
            for (int j = 0; j < off; ++j) part[j] = part[j] + part[j + off];
        s_inv = 1.0f / sqrtf((float)(part[0] / (double)K) + kHcEps);
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = tid; i < K; i += kHcThreads) flat[i] = rb(bf(r[i]) * inv);
    __syncthreads();
}

// mix[n] (bf16-valued floats) = flat . fnT[n] for n < nout, in the fixed order.
__device__ void hc_mix(const uint16_t* flat, const uint16_t* __restrict__ fnT, int K, int nout, float* mix) {
    __shared__ float chunk_sum[kHcMix][kHcMaxK / 1024];
    const int tid = threadIdx.x, lane = tid & 15, grp = tid >> 4;
    constexpr int NGRP = kHcThreads / 16;
    const int nch = K / 1024, tasks = nout * nch;
    for (int t = grp; t < tasks; t += NGRP) {
        const int n = t / nch, c = t - n * nch;
        const int k0 = c * 1024 + lane * 64;
        const uint16_t* w = fnT + (size_t)n * K + k0;
        float a = 0.0f;
        for (int i = 0; i < 64; ++i) a = fmaf(bf(flat[k0 + i]), bf(w[i]), a);
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) a = a + __shfl_down(a, off, 16);
        if (lane == 0) chunk_sum[n][c] = bf(rb(a));
    }
    __syncthreads();
    if (tid < nout) {
        float acc = 0.0f;
        for (int c = 0; c < nch; ++c) acc = acc + chunk_sum[tid][c];
        mix[tid] = bf(rb(acc));
    }
    __syncthreads();
}

// hc_split_sinkhorn (src/fst_engine.cpp:2286-2342), one thread.
__device__ void hc_split(const float* mix, const float* scale, const float* base, float* split) {
    constexpr int n = kHcN;
    const float pre_scale = scale[0], post_scale = scale[1], comb_scale = scale[2];
    for (int i = 0; i < n; ++i) {
        const float z = mix[i] * pre_scale + base[i];
        split[i] = 1.0f / (1.0f + fst_expf(-z)) + kHcEps;
    }
    for (int i = 0; i < n; ++i) {
        const int off = n + i;
        const float z = mix[off] * post_scale + base[off];
        split[off] = 2.0f / (1.0f + fst_expf(-z));
    }
    float c[16];
    for (int dst = 0; dst < n; ++dst) {
        float row_max = -1e30f;
        for (int src = 0; src < n; ++src) {
            const int idx = src + dst * n;
            const float v = mix[2 * n + idx] * comb_scale + base[2 * n + idx];
            c[idx] = v;
            if (v > row_max) row_max = v;
        }
        float row_sum = 0.0f;
        for (int src = 0; src < n; ++src) {
            const int idx = src + dst * n;
            c[idx] = fst_expf(c[idx] - row_max);
            row_sum += c[idx];
        }
        const float inv = 1.0f / row_sum;
        for (int src = 0; src < n; ++src) c[src + dst * n] = c[src + dst * n] * inv + kHcEps;
    }
    for (int src = 0; src < n; ++src) {
        float sum = 0.0f;
        for (int dst = 0; dst < n; ++dst) sum += c[src + dst * n];
        const float inv = 1.0f / (sum + kHcEps);
        for (int dst = 0; dst < n; ++dst) c[src + dst * n] *= inv;
    }
    for (int it = 1; it < kHcIters; ++it) {
        for (int dst = 0; dst < n; ++dst) {
            float sum = 0.0f;
            for (int src = 0; src < n; ++src) sum += c[src + dst * n];
            const float inv = 1.0f / (sum + kHcEps);
            for (int src = 0; src < n; ++src) c[src + dst * n] *= inv;
        }
        for (int src = 0; src < n; ++src) {
            float sum = 0.0f;
            for (int dst = 0; dst < n; ++dst) sum += c[src + dst * n];
            const float inv = 1.0f / (sum + kHcEps);
            for (int dst = 0; dst < n; ++dst) c[src + dst * n] *= inv;
        }
    }
    for (int i = 0; i < n * n; ++i) split[2 * n + i] = c[i];
}

// One workgroup per token: cur[d], post[4], comb[16].
__global__ __launch_bounds__(kHcThreads) void hc_pre_kernel(const uint16_t* __restrict__ h_hc,
                                                            const uint16_t* __restrict__ fnT,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ base, int d,
                                                            uint16_t* __restrict__ cur, float* __restrict__ post,
                                                            float* __restrict__ comb) {
    __shared__ uint16_t flat[kHcMaxK];
    __shared__ float mix[kHcMix], split[kHcMix];
    const int m = blockIdx.x, tid = threadIdx.x, K = kHcN * d;
    const uint16_t* r = h_hc + (size_t)m * K;
    hc_flat(r, K, flat);
    hc_mix(flat, fnT, K, kHcMix, mix);
    if (tid == 0) hc_split(mix, scale, base, split);
    __syncthreads();
    if (tid < kHcN) post[(size_t)m * kHcN + tid] = split[kHcN + tid];
    if (tid < kHcN * kHcN) comb[(size_t)m * kHcN * kHcN + tid] = split[2 * kHcN + tid];
    for (int j = tid; j < d; j += kHcThreads) {
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < kHcN; ++h) acc = acc + split[h] * bf(r[(size_t)h * d + j]);
        cur[(size_t)m * d + j] = rb(acc);
    }
}

// h'[dst][j] = bf16(bo[j] * post[dst] + sum_src comb[dst + 4 src] h[src][j]); each
// thread owns one j of one token for all 4 streams, so h_hc is updated in place.
__global__ __launch_bounds__(kHcThreads) void hc_post_kernel(const uint16_t* __restrict__ bo,
                                                             uint16_t* __restrict__ h_hc,
                                                             const float* __restrict__ post,
                                                             const float* __restrict__ comb, int d) {
    const int m = blockIdx.y, j = blockIdx.x * kHcThreads + threadIdx.x;
    if (j >= d) return;
    uint16_t* r = h_hc + (size_t)m * kHcN * d;
    float rv[kHcN];
#pragma unroll
    for (int s = 0; s < kHcN; ++s) rv[s] = bf(r[(size_t)s * d + j]);
    const float b = bf(bo[(size_t)m * d + j]);
    const float* p = post + (size_t)m * kHcN;
    const float* c = comb + (size_t)m * kHcN * kHcN;
#pragma unroll
    for (int dst = 0; dst < kHcN; ++dst) {
        float acc = b * p[dst];
#pragma unroll
        for (int s = 0; s < kHcN; ++s) acc = acc + c[dst + s * kHcN] * rv[s];
        r[(size_t)dst * d + j] = rb(acc);
    }
}

// output_hc_head: plain[j] = bf16(sum_h w[h] h[h][j]), w = sigmoid(mix*scale + base) + eps.
__global__ __launch_bounds__(kHcThreads) void hc_head_kernel(const uint16_t* __restrict__ h_hc,
                                                             const uint16_t* __restrict__ fnT, float scale,
                                                             const float* __restrict__ base, int d,
                                                             uint16_t* __restrict__ plain) {
    __shared__ uint16_t flat[kHcMaxK];
    __shared__ float mix[kHcN], w[kHcN];
    const int m = blockIdx.x, tid = threadIdx.x, K = kHcN * d;
    const uint16_t* r = h_hc + (size_t)m * K;
    hc_flat(r, K, flat);
    hc_mix(flat, fnT, K, kHcN, mix);
    if (tid < kHcN) {
        const float z = mix[tid] * scale + (base ? base[tid] : 0.0f);
        w[tid] = 1.0f / (1.0f + fst_expf(-z)) + kHcEps;
    }
    __syncthreads();
    for (int j = tid; j < d; j += kHcThreads) {
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < kHcN; ++h) acc = acc + w[h] * bf(r[(size_t)h * d + j]);
        plain[(size_t)m * d + j] = rb(acc);
    }
}

#pragma clang fp contract(on)

void launch_hc_pre(hipStream_t st, const uint16_t* h_hc, const uint16_t* fnT, const float* scale, const float* base,
                   int M, int d, uint16_t* cur, float* post, float* comb) {
    hipLaunchKernelGGL(hc_pre_kernel, dim3(M), dim3(kHcThreads), 0, st, h_hc, fnT, scale, base, d, cur, post, comb);
}

void launch_hc_post(hipStream_t st, const uint16_t* bo, uint16_t* h_hc, const float* post, const float* comb, int M,
                    int d) {
    hipLaunchKernelGGL(hc_post_kernel, dim3((d + kHcThreads - 1) / kHcThreads, M), dim3(kHcThreads), 0, st, bo, h_hc,
                       post, comb, d);
}

void launch_hc_head(hipStream_t st, const uint16_t* h_hc, const uint16_t* fnT, float scale, const float* base, int M,
                    int d, uint16_t* plain) {
    hipLaunchKernelGGL(hc_head_kernel, dim3(M), dim3(kHcThreads), 0, st, h_hc, fnT, scale, base, d, plain);
}

}  // namespace fst
