// fst_accept.hip — greedy and rejection-sampling acceptance for gfx950.
//
// Rows: target rows r = s*(k+1)+i (i = 0..k) of n_seq sequences, then (for
// rejection sampling) draft rows n_seq*(k+1) + s*k + i.  Each row of V logits
// is split into kChunks chunks processed by one workgroup each.
//
// Greedy (src/fst_engine.cpp:6021-6063): argmax per target row with the
// reference's sequential semantics (first maximum wins, NaN skipped, a NaN at
// index 0 pins the result to 0), then the longest matching prefix and bonus.
//
// Rejection sampling: probabilities in exact 2^-32 fixed point
// E = floor(exp(l - max) * 2^32) with the shared fst_expf, integer sums, and
// 128-bit integer comparisons/prefix sums, so the accept decisions and the
// resampled token are identical to the CPU oracle for identical logits.
#include <atomic>
#include <mutex>
#include <string>

#include "fst_internal.h"
#include "../../include/fst_hip.h"
#include "../../include/fst_exact_math.h"

namespace fst {

constexpr int kChunks = 64;
// threads of the per-sequence residual and sampling workgroups (two
// exponentials and 128-bit products per element, few workgroups: compute
// bound per thread; the per-row sums keep 256, their grid is large)
constexpr int kProbThreads = 1024;
typedef unsigned __int128 u128;

// Rejection-sampling tail launch (acc_tail_kernel): chunks per sequence,
// threads, rows (2k + 1 <= 17), elements per thread at most, and the
// arrival counters: kTailGroups16 groups of 16 chunks, then one top counter,
// each on its own 256-byte line.
constexpr int kTailThreads = 512;
constexpr int kTailChunks = 256;
constexpr int kTailRows = 17;
constexpr int kTailPerMax = 2;  // chunk length <= 1024
constexpr int kTailArrGroups = kTailChunks / 16;
constexpr int kTailCntStride = 32;  // u64 words between counters
// [n_seq][kTailChunks][3] chunk sums (residual lo, hi; target E), then
// [n_seq][kTailArrGroups + 1] counters.
static size_t tail_words(int n_seq) {
    return (size_t)n_seq * kTailChunks * 3 + (size_t)n_seq * (kTailArrGroups + 1) * kTailCntStride;
}

struct AccWs {
    float* part_max;          // [R][kChunks]
    int* part_idx;            // [R][kChunks]
    unsigned long long* part_sum;  // [R][kChunks]
    unsigned long long* part_res;  // [n_seq][kChunks][2] (u128 as lo, hi)
    unsigned long long* dec;       // [n_seq][8]
    unsigned long long* gslot;     // [R][kChunks] greedy chunk partials (zero between calls)
    float* xsel;                   // [R] each row's logit at its position's draft token (acc_sums_kernel)
    unsigned long long* tail;      // acc_tail_kernel: chunk sums and counters (counters zero between calls)
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static AccWs carve(void* ws, int n_seq, int k) {
    const int R = n_seq * (k + 1) + n_seq * k;
    char* p = (char*)ws;
    AccWs w;
    w.part_max = (float*)p; p += align256(sizeof(float) * R * kChunks);
    w.part_idx = (int*)p; p += align256(sizeof(int) * R * kChunks);
    w.part_sum = (unsigned long long*)p; p += align256(8ull * R * kChunks);
    w.part_res = (unsigned long long*)p; p += align256(16ull * n_seq * kChunks);
    w.dec = (unsigned long long*)p; p += align256(64ull * n_seq);
    w.gslot = (unsigned long long*)p; p += align256(8ull * R * kChunks);
    w.xsel = (float*)p; p += align256(sizeof(float) * R);
    w.tail = (unsigned long long*)p;
    return w;
}

size_t accept_ws_bytes(int n_seq, int k, int V) {
    (void)V;
    const int R = n_seq * (k + 1) + n_seq * k;
    return align256(sizeof(float) * R * kChunks) + align256(sizeof(int) * R * kChunks) +
           align256(8ull * R * kChunks) + align256(16ull * n_seq * kChunks) + align256(64ull * n_seq) +
           align256(8ull * R * kChunks) + align256(sizeof(float) * R) + align256(8ull * tail_words(n_seq)) + 256;
}

// Calls f(x, v) for v = v0, v0 + stride, ... < v1 in that order, with the
// loads of each batch of NB elements issued before any of them is used (a
// plain loop waits for every load in turn); addresses past v1 are clamped to
// v1 - 1 and their values unused.
template <int NB, typename F>
__device__ __forceinline__ void for_strided(const float* __restrict__ p, int v0, int v1, int stride, F&& f) {
    for (int base = v0; base < v1; base += NB * stride) {
        float x[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) x[u] = p[min(base + u * stride, v1 - 1)];
#pragma unroll
        for (int u = 0; u < NB; ++u)
            if (base + u * stride < v1) f(x[u], base + u * stride);
    }
}
// Two rows at once (the same indices of p and q).
template <int NB, typename F>
__device__ __forceinline__ void for_strided2(const float* __restrict__ p, const float* __restrict__ q, int v0,
                                             int v1, int stride, F&& f) {
    for (int base = v0; base < v1; base += NB * stride) {
        float x[NB], y[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int v = min(base + u * stride, v1 - 1);
            x[u] = p[v];
            y[u] = q ? q[v] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < NB; ++u)
            if (base + u * stride < v1) f(x[u], y[u], base + u * stride);
    }
}

__device__ __forceinline__ const float* row_ptr(const float* target, const float* draft, int n_tgt_rows,
                                                int r, int V) {
    return r < n_tgt_rows ? target + (size_t)r * V : draft + (size_t)(r - n_tgt_rows) * V;
}

// (max over non-NaN of x*inv_t, lowest index attaining it) per (row, chunk).
__global__ __launch_bounds__(256) void acc_stats_kernel(const float* __restrict__ target,
                                                        const float* __restrict__ draft, int n_tgt_rows,
                                                        int V, float inv_t, float* __restrict__ part_max,
                                                        int* __restrict__ part_idx) {
    const int c = blockIdx.x, r = blockIdx.y;
    const float* row = row_ptr(target, draft, n_tgt_rows, r, V);
    const int clen = (V + kChunks - 1) / kChunks;
    const int b0 = c * clen, b1 = min(V, b0 + clen);
    float best = 0.0f;
    int bi = 0x7fffffff;
    for_strided<8>(row, b0 + (int)threadIdx.x, b1, 256, [&](float x, int v) {
        const float l = x * inv_t;
        if (l != l) return;
        if (bi == 0x7fffffff || l > best) { best = l; bi = v; }
    });
    if (bi == 0x7fffffff) bi = -1;
    wave_argmax(best, bi);
    __shared__ float sm[4];
    __shared__ int si[4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int q = 1; q < 4; ++q) argmax_merge(best, bi, sm[q], si[q]);
        part_max[(size_t)r * kChunks + c] = best;
        part_idx[(size_t)r * kChunks + c] = bi;
    }
}

// Wave-parallel reduction of the kChunks (= 64) chunk partials of row r: lane
// c reads chunk c.  Returns (max, lowest index attaining it, -1 if the row
// has no number) in every lane.
__device__ __forceinline__ void wave_row_argmax(const float* part_max, const int* part_idx, int r, float* mx,
                                                int* idx) {
    const int lane = threadIdx.x & 63;
    float m = part_max[(size_t)r * kChunks + lane];
    int i = part_idx[(size_t)r * kChunks + lane];
    wave_argmax(m, i);
    *mx = m;
    *idx = i;
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) { return wave_sum_u64_dpp(v); }

// Wave-wide sum of a u128 as four 32-bit limbs summed exactly in u64, then
// recombined (result in every lane).
__device__ __forceinline__ u128 wave_sum_u128(u128 v) {
    u128 t = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) t += (u128)wave_sum_u64_dpp((uint32_t)(v >> (32 * k))) << (32 * k);
    return t;
}


__device__ __forceinline__ unsigned long long fixed_prob(float x, float inv_t, float mx, int any) {
    const float l = x * inv_t;
    if (!any || l != l) return 0ull;
    if (l == mx) return 4294967296ull;
    const float d = l - mx;
    if (d != d) return 0ull;
    return (unsigned long long)fst_prob_fixed(d);
}

__device__ __forceinline__ void wave_row_max_any(const float* part_max, const int* part_idx, int r, float* mx,
                                                 int* any) {
    int idx;
    wave_row_argmax(part_max, part_idx, r, mx, &idx);
    *any = idx >= 0;
}

// Chunk sums of E for every row.  With xsel given, the workgroup whose chunk
// holds the row's draft token (position i of sequence s: draft[s*k + i], for
// target rows i < k and every draft row) also writes that logit to xsel[r],
// so that the decisions need no dependent load of it later.
__global__ __launch_bounds__(256) void acc_sums_kernel(const float* __restrict__ target,
                                                       const float* __restrict__ draft, int n_tgt_rows,
                                                       int V, float inv_t,
                                                       const float* __restrict__ part_max,
                                                       const int* __restrict__ part_idx,
                                                       unsigned long long* __restrict__ part_sum,
                                                       const int32_t* __restrict__ dtok, int k,
                                                       float* __restrict__ xsel) {
    const int c = blockIdx.x, r = blockIdx.y;
    const float* row = row_ptr(target, draft, n_tgt_rows, r, V);
    const int clen = (V + kChunks - 1) / kChunks;
    const int b0 = c * clen, b1 = min(V, b0 + clen);
    if (xsel && threadIdx.x == 0 && k > 0) {
        const int seq = r < n_tgt_rows ? r / (k + 1) : (r - n_tgt_rows) / k;
        const int pos = r < n_tgt_rows ? r % (k + 1) : (r - n_tgt_rows) % k;
        if (pos < k) {
            const int x = dtok[seq * k + pos];
            if (x >= b0 && x < b1) xsel[r] = row[x];
        }
    }
    // the first 8 elements of each thread are loaded before the row maximum
    // is known (they do not depend on it), so both round trips overlap
    constexpr int NB = 8;
    const int v0 = b0 + (int)threadIdx.x;
    float x0[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) x0[u] = row[max(min(v0 + u * 256, b1 - 1), 0)];
    __shared__ float s_mx;
    __shared__ int s_any;
    if (threadIdx.x < 64) {
        float mx;
        int any;
        wave_row_max_any(part_max, part_idx, r, &mx, &any);
        if (threadIdx.x == 0) {
            s_mx = mx;
            s_any = any;
        }
    }
    __syncthreads();
    const float mx = s_mx;
    const int any = s_any;
    unsigned long long acc = 0;
#pragma unroll
    for (int u = 0; u < NB; ++u)
        if (v0 + u * 256 < b1) acc += fixed_prob(x0[u], inv_t, mx, any);
    for_strided<8>(row, v0 + NB * 256, b1, 256, [&](float x, int) { acc += fixed_prob(x, inv_t, mx, any); });
    // integer sums: any order gives the same total
    __shared__ unsigned long long sm[256 / 64];
    acc = wave_sum_u64_dpp(acc);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < 256 / 64; ++w) t += sm[w];
        part_sum[(size_t)r * kChunks + c] = t;
    }
}

// dec layout per sequence: [0] n_acc, [1] sampling target row, [2] mode
// (0: residual vs draft row, 1: sample from target row), [3] U', [4] Sp, [5] Sq,
// [6] draft row, [7] unused.
// One workgroup per sequence; wave w decides positions w, w+NW, ... in
// parallel (each decision is independent given the logits and uniforms).
constexpr int kDecideWaves = 8;
__global__ __launch_bounds__(64 * kDecideWaves) void acc_decide_kernel(
    const float* __restrict__ target, const float* __restrict__ draftl, int n_seq, int k, int V,
    float inv_t, const int32_t* __restrict__ draft, uint64_t seed, uint64_t seq_base,
    const float* __restrict__ part_max, const int* __restrict__ part_idx,
    const unsigned long long* __restrict__ part_sum, unsigned long long* __restrict__ dec,
    int32_t* __restrict__ n_acc, int32_t* __restrict__ tokens) {
    const int s = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n_tgt = n_seq * (k + 1);
    __shared__ int accept[64];
    __shared__ unsigned long long Sp_s[65], Sq_s[64];
    for (int i = wave; i <= k; i += kDecideWaves) {
        const int rt = s * (k + 1) + i;
        const unsigned long long Sp = wave_sum_u64(part_sum[(size_t)rt * kChunks + lane]);
        if (i == k) {
            if (lane == 0) Sp_s[k] = Sp;
            continue;
        }
        const int rd = n_tgt + s * k + i;
        const unsigned long long Sq = wave_sum_u64(part_sum[(size_t)rd * kChunks + lane]);
        float mp, mq;
        int ap, aq;
        wave_row_max_any(part_max, part_idx, rt, &mp, &ap);
        wave_row_max_any(part_max, part_idx, rd, &mq, &aq);
        if (lane == 0) {
            const int x = draft[s * k + i];
            int ok = 0;
            if (x >= 0 && x < V) {
                const unsigned long long P = fixed_prob(target[(size_t)rt * V + x], inv_t, mp, ap);
                const unsigned long long Q = fixed_prob(draftl[(size_t)(rd - n_tgt) * V + x], inv_t, mq, aq);
                const uint32_t U = fst_uniform24(seed, seq_base + (uint64_t)s, (uint32_t)i, 0);
                const u128 lhs = (u128)U * (u128)Q * (u128)Sp;
                const u128 rhs = ((u128)P * (u128)Sq) << 24;
                ok = lhs < rhs;
            }
            accept[i] = ok;
            Sp_s[i] = Sp;
            Sq_s[i] = Sq;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int n = 0;
        while (n < k && accept[n]) ++n;
        unsigned long long* d = dec + (size_t)s * 8;
        d[0] = (unsigned long long)n;
        d[1] = (unsigned long long)(s * (k + 1) + n);
        d[3] = fst_uniform24(seed, seq_base + (uint64_t)s, (uint32_t)n, 1);
        d[4] = Sp_s[n];
        if (n < k) {
            d[2] = 0;
            d[5] = Sq_s[n];
            d[6] = (unsigned long long)(n_tgt + s * k + n);
        } else {
            d[2] = 1;
            d[5] = 0;
            d[6] = 0;
        }
        for (int i = 0; i < n; ++i) tokens[s * (k + 1) + i] = draft[s * k + i];
        for (int i = n; i <= k; ++i) tokens[s * (k + 1) + i] = -1;
        n_acc[s] = n;
    }
}

// Residual weight of one element from its target (xt) and draft (xd) logits.
__device__ __forceinline__ u128 res_of(float xt, float xd, float inv_t, float mp, int ap, float mq, int aq,
                                       unsigned long long Sp, unsigned long long Sq, int mode) {
    const unsigned long long P = fixed_prob(xt, inv_t, mp, ap);
    if (mode) return (u128)P;
    const unsigned long long Q = fixed_prob(xd, inv_t, mq, aq);
    const u128 a = (u128)P * Sq, b = (u128)Q * Sp;
    return a > b ? a - b : (u128)0;
}
__device__ __forceinline__ u128 res_value(const float* trow, const float* drow, int v, float inv_t,
                                          float mp, int ap, float mq, int aq, unsigned long long Sp,
                                          unsigned long long Sq, int mode) {
    return res_of(trow[v], mode ? 0.0f : drow[v], inv_t, mp, ap, mq, aq, Sp, Sq, mode);
}

struct RowCtx {
    const float* trow;
    const float* drow;
    float mp, mq;
    int ap, aq, mode;
    unsigned long long Sp, Sq;
};

// Called by all lanes of the first wave; lane 0 stores the context.
__device__ void load_rowctx_wave(const float* target, const float* draftl, int n_tgt, int V,
                                 const float* part_max, const int* part_idx, const unsigned long long* d,
                                 RowCtx& rc) {
    const int rt = (int)d[1];
    const int mode = (int)d[2];
    float mp, mq = 0.0f;
    int ap, aq = 0;
    wave_row_max_any(part_max, part_idx, rt, &mp, &ap);
    const int rd = (int)d[6];
    if (mode == 0) wave_row_max_any(part_max, part_idx, rd, &mq, &aq);
    if ((threadIdx.x & 63) == 0) {
        rc.mode = mode;
        rc.Sp = d[4];
        rc.Sq = d[5];
        rc.trow = target + (size_t)rt * V;
        rc.drow = mode == 0 ? draftl + (size_t)(rd - n_tgt) * V : nullptr;
        rc.mp = mp;
        rc.ap = ap;
        rc.mq = mq;
        rc.aq = aq;
    }
}

// Residual (or target) chunk sums for the one sampling row of each sequence.
__global__ __launch_bounds__(kProbThreads) void acc_res_chunks_kernel(
    const float* __restrict__ target, const float* __restrict__ draftl, int n_seq, int k, int V,
    float inv_t, const float* __restrict__ part_max, const int* __restrict__ part_idx,
    const unsigned long long* __restrict__ dec, unsigned long long* __restrict__ part_res) {
    const int c = blockIdx.x, s = blockIdx.y;
    const unsigned long long* d = dec + (size_t)s * 8;
    const int clen = (V + kChunks - 1) / kChunks;
    const int b0 = c * clen, b1 = min(V, b0 + clen);
    // the thread's first elements are loaded as soon as the sampling rows are
    // known, before their maxima (round trips overlap)
    constexpr int NB = 2;
    const int v0 = b0 + (int)threadIdx.x;
    const int mode0 = (int)d[2];
    const float* trow0 = target + (size_t)d[1] * V;
    const float* drow0 = mode0 == 0 ? draftl + ((size_t)d[6] - (size_t)n_seq * (k + 1)) * V : trow0;
    float xt0[NB], xd0[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int v = max(min(v0 + u * kProbThreads, b1 - 1), 0);
        xt0[u] = trow0[v];
        xd0[u] = drow0[v];
    }
    __shared__ RowCtx rc;
    if (threadIdx.x < 64) load_rowctx_wave(target, draftl, n_seq * (k + 1), V, part_max, part_idx, d, rc);
    __syncthreads();
    u128 acc = 0;
#pragma unroll
    for (int u = 0; u < NB; ++u)
        if (v0 + u * kProbThreads < b1)
            acc += res_of(xt0[u], rc.mode ? 0.0f : xd0[u], inv_t, rc.mp, rc.ap, rc.mq, rc.aq, rc.Sp, rc.Sq, rc.mode);
    for_strided2<8>(rc.trow, rc.mode ? nullptr : rc.drow, v0 + NB * kProbThreads, b1, kProbThreads,
                    [&](float xt, float xd, int) {
                        acc += res_of(xt, xd, inv_t, rc.mp, rc.ap, rc.mq, rc.aq, rc.Sp, rc.Sq, rc.mode);
                    });
    // integer sums: any order gives the same total
    __shared__ u128 sm[kProbThreads / 64];
    acc = wave_sum_u128(acc);
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        u128 tot = 0;
        for (int w = 0; w < kProbThreads / 64; ++w) tot += sm[w];
        unsigned long long* o = part_res + ((size_t)s * kChunks + c) * 2;
        o[0] = (unsigned long long)tot;
        o[1] = (unsigned long long)(tot >> 64);
    }
}

__device__ __forceinline__ u128 shfl_u128(u128 v, int src) {
    const uint64_t lo = (uint64_t)v, hi = (uint64_t)(v >> 64);
    const uint32_t a = __shfl((uint32_t)lo, src, 64), b = __shfl((uint32_t)(lo >> 32), src, 64);
    const uint32_t c = __shfl((uint32_t)hi, src, 64), d = __shfl((uint32_t)(hi >> 32), src, 64);
    return ((u128)(((uint64_t)d << 32) | c) << 64) | (u128)(((uint64_t)b << 32) | a);
}

// Inclusive prefix sum over the 64 lanes of a wave (exact, unsigned 128-bit).
__device__ __forceinline__ u128 wave_incl_scan_u128(u128 v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const u128 o = shfl_u128(v, max(lane - off, 0));
        if (lane >= off) v += o;
    }
    return v;
}

// Inverse-CDF pick: the first v whose inclusive prefix exceeds
// target = (U' * total) >> 24.  Chunk sums are scanned by one wave (lane c
// = chunk c), then the chosen chunk by the whole workgroup (thread t owns a
// contiguous run), and only the owning thread walks its few elements.
__global__ __launch_bounds__(kProbThreads) void acc_sample_kernel(
    const float* __restrict__ target, const float* __restrict__ draftl, int n_seq, int k, int V,
    float inv_t, const float* __restrict__ part_max, const int* __restrict__ part_idx,
    const unsigned long long* __restrict__ part_sum, unsigned long long* __restrict__ dec,
    const unsigned long long* __restrict__ part_res, int32_t* __restrict__ tokens) {
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ RowCtx rc;
    __shared__ u128 s_target, s_before;
    __shared__ int s_chunk;
    __shared__ u128 wtot[kProbThreads / 64];
    __shared__ int s_owner;
    __shared__ u128 s_run;
    __shared__ int s_tok;
    unsigned long long* d = dec + (size_t)s * 8;
    // the chunk totals do not depend on the row context: load them first so
    // that both round trips overlap
    unsigned long long o0 = 0, o1 = 0;
    if (tid < 64) {
        const unsigned long long* o = part_res + ((size_t)s * kChunks + lane) * 2;
        o0 = o[0];
        o1 = o[1];
        load_rowctx_wave(target, draftl, n_seq * (k + 1), V, part_max, part_idx, d, rc);
    }
    __syncthreads();
    if (tid < 64) {
        const unsigned long long U2 = d[3];
        u128 cs = ((u128)o1 << 64) | (u128)o0;
        u128 pre = wave_incl_scan_u128(cs);
        u128 tot = shfl_u128(pre, 63);
        int mode = rc.mode;
        if (mode == 0 && tot == 0) {
            // residual is identically zero: sample from the target row instead
            mode = 1;
            cs = (u128)part_sum[(size_t)((int)d[1]) * kChunks + lane];
            pre = wave_incl_scan_u128(cs);
            tot = shfl_u128(pre, 63);
        }
        int chunk = -1;
        u128 tg = 0;
        if (tot != 0) {
            tg = ((u128)U2 * tot) >> 24;
            const unsigned long long hit = __ballot(pre > tg);
            chunk = hit ? __ffsll((long long)hit) - 1 : -1;
        }
        const u128 before = chunk > 0 ? shfl_u128(pre, chunk - 1) : (u128)0;
        if (lane == 0) {
            rc.mode = mode;
            s_chunk = chunk;
            s_target = tg;
            s_before = before;
            s_tok = 0;
        }
    }
    __syncthreads();
    const int c = s_chunk;
    if (c >= 0) {
        const int clen = (V + kChunks - 1) / kChunks;
        const int b0 = c * clen, b1 = min(V, b0 + clen);
        const int per = (clen + kProbThreads - 1) / kProbThreads;
        const int v0 = b0 + tid * per, v1 = min(b1, v0 + per);
        // the thread's residual values stay in registers for the owner's walk
        // (runs of up to kCache elements; longer ones are recomputed there)
        constexpr int kCache = 16;
        u128 cache[kCache];
        u128 acc = 0;
        if (per <= kCache) {
            // slots past the run length `per` (uniform) are skipped, not
            // computed and discarded: each slot costs two exponentials and
            // 128-bit products
            float xt[kCache], xd[kCache];
#pragma unroll
            for (int u = 0; u < kCache; ++u) {
                if (u >= per) break;
                const int v = max(min(v0 + u, v1 - 1), 0);
                xt[u] = rc.trow[v];
                xd[u] = rc.mode ? 0.0f : rc.drow[v];
            }
#pragma unroll
            for (int u = 0; u < kCache; ++u) {
                cache[u] = 0;
                if (u >= per) continue;
                if (v0 + u < v1)
                    cache[u] = res_of(xt[u], xd[u], inv_t, rc.mp, rc.ap, rc.mq, rc.aq, rc.Sp, rc.Sq, rc.mode);
                acc += cache[u];
            }
        } else {
            for_strided2<8>(rc.trow, rc.mode ? nullptr : rc.drow, v0, v1, 1, [&](float xt, float xd, int) {
                acc += res_of(xt, xd, inv_t, rc.mp, rc.ap, rc.mq, rc.aq, rc.Sp, rc.Sq, rc.mode);
            });
        }
        const u128 pre = wave_incl_scan_u128(acc);
        if (lane == 63) wtot[wave] = pre;
        if (tid == 0) s_owner = 0x7fffffff;
        __syncthreads();
        u128 base = s_before;
        for (int w2 = 0; w2 < wave; ++w2) base += wtot[w2];
        const unsigned long long hit = __ballot(base + pre > s_target);
        if (hit && lane == __ffsll((long long)hit) - 1) atomicMin(&s_owner, tid);
        __syncthreads();
        if (tid == s_owner) s_run = base + pre - acc;  // prefix before this thread's run
        __syncthreads();
        if (tid == s_owner) {
            u128 run = s_run;
            int tok = v1 - 1;
            if (per <= kCache) {
#pragma unroll
                for (int u = 0; u < kCache; ++u) {
                    if (v0 + u >= v1) break;
                    run += cache[u];
                    if (run > s_target) {
                        tok = v0 + u;
                        break;
                    }
                }
            } else {
                for (int v = v0; v < v1; ++v) {
                    run += res_value(rc.trow, rc.drow, v, inv_t, rc.mp, rc.ap, rc.mq, rc.aq, rc.Sp, rc.Sq,
                                     rc.mode);
                    if (run > s_target) {
                        tok = v;
                        break;
                    }
                }
            }
            s_tok = tok;
        }
        __syncthreads();
        if (tid == 0) tokens[s * (k + 1) + (int)d[0]] = s_owner == 0x7fffffff ? 0 : s_tok;
    } else if (tid == 0) {
        tokens[s * (k + 1) + (int)d[0]] = 0;
    }
}

// Greedy acceptance in one launch, without counters.  Every (row, chunk)
// workgroup reduces its chunk to (max, lowest index) and publishes it as one
// 64-bit word {tag, max bits}, tag = epoch << 20 | (index + 1): a word is
// valid for this call only when its tag carries the call's epoch (1..4095),
// so words left by an earlier or abandoned call are never taken.  The
// workgroup with the highest linear id of a sequence (last chunk of its last
// row) then collects the sequence's (k+1)*CH words with coherent loads,
// resolves each row's argmax with the reference's rules, the longest
// matching prefix and the bonus token, and clears the words.  Workgroups are
// dispatched in linear-id order on each XCD, so every workgroup it waits for
// is resident or finished (the lowest unfinished id never waits), and the
// wait ends.  The wait is still bounded (spin_limit polls): past it the
// owner gives up, writes n_acc = -1 and tokens = -1 for its sequence (the
// host turns that into FST_EHIP) and exits normally.  (Counters instead of
// flags serialise: increments of one device-scope counter complete a few
// hundred ns apart at the memory side.)
constexpr int kGreedyIdxBits = 20;
#ifndef FST_GREEDY_CHUNKS
#define FST_GREEDY_CHUNKS 16
#endif
static_assert(FST_GREEDY_CHUNKS == kGreedyChunks, "greedy chunk count");  // index + 1 < 2^20: V <= kMaxAcceptVocab

template <int CH>
__device__ __forceinline__ void greedy_chunk(const float* __restrict__ row, int V, int c, float& best, int& bi) {
    const int clen = ((V + CH - 1) / CH + 3) & ~3;  // multiple of 4 elements
    const int b0 = min(V, c * clen), b1 = min(V, b0 + clen);
    best = 0.0f;
    bi = 0x7fffffff;
    auto take = [&](float l, int v) {
        if (l != l) return;
        if (bi == 0x7fffffff || l > best) {
            best = l;
            bi = v;
        }
    };
    if ((V & 3) == 0) {
        // 16-byte loads: thread t takes elements b0 + 4(t + 256 j) .. +3, in
        // index order; each batch of 8 loads is issued before any is used
        // (b1 - b0 is a multiple of 4 here, so b1 - 4 is a valid clamp)
        constexpr int NB = 8;
        for (int base = b0 + 4 * (int)threadIdx.x; base < b1; base += NB * 1024) {
            float4 q[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) q[u] = *reinterpret_cast<const float4*>(row + min(base + u * 1024, b1 - 4));
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int v = base + u * 1024;
                if (v < b1) {
                    take(q[u].x, v);
                    take(q[u].y, v + 1);
                    take(q[u].z, v + 2);
                    take(q[u].w, v + 3);
                }
            }
        }
    } else {
        for_strided<8>(row, b0 + (int)threadIdx.x, b1, 256, [&](float x, int v) { take(x, v); });
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (bi == 0x7fffffff) bi = -1;
    wave_argmax(best, bi);
    __shared__ float sm[4];
    __shared__ int si[4];
    if (lane == 0) {
        sm[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    for (int q = 1; q < 4; ++q) argmax_merge(best, bi, sm[q], si[q]);
}

template <int CH, int NU>
__global__ __launch_bounds__(256) void acc_greedy_kernel(const float* __restrict__ target, int k, int V,
                                                         const int32_t* __restrict__ draft,
                                                         unsigned long long* __restrict__ gslot, uint32_t epoch,
                                                         int spin_limit, int32_t* __restrict__ n_acc,
                                                         int32_t* __restrict__ tokens) {
    static_assert(CH == 16, "a row's chunk words fill one 16-lane DPP row");
    const int c = blockIdx.x, r = blockIdx.y;
    const int s = r / (k + 1);
    const int lane = threadIdx.x & 63;
    const bool owner = c == CH - 1 && r == s * (k + 1) + k;
    // the owner's row-0 values and draft tokens, loaded before anything waits
    int32_t dv = 0;
    float x0 = 0.0f;
    if (owner && threadIdx.x < 64) {
        if (lane < k) dv = draft[s * k + lane];
        if (lane <= k) x0 = target[(size_t)(s * (k + 1) + lane) * V];
    }
    float best;
    int bi;
    greedy_chunk<CH>(target + (size_t)r * V, V, c, best, bi);
    unsigned long long* words = gslot + (size_t)s * (k + 1) * CH;
    const int me = (r - s * (k + 1)) * CH + c;
    if (threadIdx.x == 0) {
        const uint32_t tag = (epoch << kGreedyIdxBits) | (uint32_t)(bi + 1);
        st_coherent_u64(&words[me], ((unsigned long long)tag << 32) | fst_f32_bits(best));
        publish_wait();
    }
    if (!owner || threadIdx.x >= 64) return;
    // collect: lane l holds words l + 64u (row 4u + l/16, chunk l%16)
    const int nw = (k + 1) * CH;
    unsigned long long v[NU];
    uint32_t pend = 0;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        v[u] = 0ull;
        if (lane + 64 * u < nw) pend |= 1u << u;
    }
    bool timed_out = false;
    for (int spin = 0;; ++spin) {
        unsigned long long t[NU];
#pragma unroll
        for (int u = 0; u < NU; ++u) t[u] = ld_coherent_u64(&words[min(lane + 64 * u, nw - 1)]);
#pragma unroll
        for (int u = 0; u < NU; ++u)
            if (((pend >> u) & 1u) && (uint32_t)(t[u] >> (32 + kGreedyIdxBits)) == epoch) {
                v[u] = t[u];
                pend &= ~(1u << u);
            }
        if (!__any(pend != 0u)) break;
        if (spin >= spin_limit) {
            timed_out = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (timed_out) {
        // late words carry this call's epoch, which the next call does not accept
#pragma unroll
        for (int u = 0; u < NU; ++u)
            if (lane + 64 * u < nw) st_coherent_u64(&words[lane + 64 * u], 0ull);
        if (lane <= k) tokens[s * (k + 1) + lane] = -1;
        if (lane == 0) n_acc[s] = -1;
        return;
    }
    // per row: argmax over its 16 chunk words (one DPP row); lane l then
    // takes row l's result from lane 16 (l % 4) of iteration l / 4
    int pv = 0;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        float m = fst_bits_f32((uint32_t)v[u]);
        int i = (lane + 64 * u < nw) ? (int)((v[u] >> 32) & ((1u << kGreedyIdxBits) - 1u)) - 1 : -1;
        argmax_step<0xb1>(m, i);
        argmax_step<0x4e>(m, i);
        argmax_step<0x124>(m, i);
        argmax_step<0x128>(m, i);
        const int ti = __shfl(i, 16 * (lane & 3), 64);
        if ((lane >> 2) == u) pv = ti;
        if (lane + 64 * u < nw) st_coherent_u64(&words[lane + 64 * u], 0ull);
    }
    // the reference's rules: first max wins, a NaN at index 0 pins row 0
    if (lane <= k) pv = (x0 != x0 || pv < 0) ? 0 : pv;
    const unsigned long long match = __ballot(lane < k && pv == dv);
    const int n = min(k, __ffsll((long long)~match) - 1);
    const int bonus = __shfl(pv, n, 64);
    if (lane <= k) tokens[s * (k + 1) + lane] = lane < n ? dv : (lane == n ? bonus : -1);
    if (lane == 0) n_acc[s] = n;
}

void* accept_greedy_words(void* ws, int n_seq, int k) { return carve(ws, n_seq, k).gslot; }

void launch_accept_greedy(hipStream_t st, const float* target, int n_seq, int k, int V,
                          const int32_t* draft, int32_t* n_acc, int32_t* tokens, void* words, uint32_t epoch,
                          int spin_limit) {
    const int R = n_seq * (k + 1);
    constexpr int CH = FST_GREEDY_CHUNKS;
    // words per sequence (k+1)*16 <= 1024: NU = 64-lane passes
    const int nu = ((k + 1) * CH + 63) / 64;
#define FST_GK(NUV) \
    hipLaunchKernelGGL((acc_greedy_kernel<CH, NUV>), dim3(CH, R), dim3(256), 0, st, target, k, V, draft, \
                       static_cast<unsigned long long*>(words), epoch, spin_limit, n_acc, tokens)
    if (nu <= 1)
        FST_GK(1);
    else if (nu <= 2)
        FST_GK(2);
    else if (nu <= 4)
        FST_GK(4);
    else if (nu <= 8)
        FST_GK(8);
    else
        FST_GK(16);
#undef FST_GK
}


// ------------------------------- rejection sampling: decide, residual, pick
//
// The last three steps of the chain in one launch.  Workgroup (c, s) of
// kTailChunks chunks per sequence:
//   - loads chunk c of every row of sequence s, the draft tokens' logits and
//     the row partials of the maxima and sums launches, all at once;
//   - takes the accept decisions (every workgroup alike, as acc_decide_kernel);
//   - sums the residual of its chunk (and the target row's E, for the case
//     of an identically zero residual), writes the sums with device-coherent
//     stores and counts itself in with one atomic per workgroup;
//   - the last workgroup of the sequence to arrive (the counter is left at
//     zero) finds the chunk holding the inverse-CDF target, loads it and
//     picks the token, then writes n_acc and the tokens.
// No workgroup waits for another, so any grid size is safe.  The arithmetic
// is the chain's, and the results are identical to it and to the CPU oracle.
// The two searches ("first index whose inclusive prefix exceeds t") run over
// LDS: sums of 16-element groups and of 16-group super-groups, then one wave
// locates the super-group, the group and the element, each level by a
// ballot over per-lane prefix sums of at most 16 terms (no u128 wave scans).
#define TAIL_STAMP(i) \
    do {              \
    } while (0)
#define TAIL_FLUSH(i0, i1) \
    do {                   \
    } while (0)
constexpr int kTailWaves = kTailThreads / 64;
constexpr int kTailMaxN = kTailPerMax * kTailThreads;  // longest array searched
constexpr int kTailGroups = kTailMaxN / 16;            // 16-element groups
static_assert(kTailChunks <= kTailThreads && kTailGroups <= 64, "search levels");


// u128 as four 32-bit limbs, each held in 64 bits so that sums over up to
// 2^32 terms need no carries until recombined.
struct Limbs {
    unsigned long long l[4];
};
__device__ __forceinline__ Limbs to_limbs(u128 v) {
    Limbs r;
#pragma unroll
    for (int q = 0; q < 4; ++q) r.l[q] = (uint32_t)(v >> (32 * q));
    return r;
}
__device__ __forceinline__ u128 from_limbs(const Limbs& r) {
    u128 t = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) t += (u128)r.l[q] << (32 * q);
    return t;
}
// Sum over the 16 lanes of each DPP row, in every lane of the row.
__device__ __forceinline__ u128 row_sum_u128(u128 v) {
    Limbs r = to_limbs(v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r.l[q] += dpp_u64<0xb1>(r.l[q]);   // quad_perm [1,0,3,2]
        r.l[q] += dpp_u64<0x4e>(r.l[q]);   // quad_perm [2,3,0,1]
        r.l[q] += dpp_u64<0x124>(r.l[q]);  // row_ror 4
        r.l[q] += dpp_u64<0x128>(r.l[q]);  // row_ror 8
    }
    return from_limbs(r);
}
// Inclusive prefix sum within each DPP row (row_shr 1, 2, 4, 8; lanes
// without a source add 0).
__device__ __forceinline__ u128 row_scan_u128(u128 v) {
    Limbs r = to_limbs(v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r.l[q] += dpp_u64<0x111>(r.l[q]);
        r.l[q] += dpp_u64<0x112>(r.l[q]);
        r.l[q] += dpp_u64<0x114>(r.l[q]);
        r.l[q] += dpp_u64<0x118>(r.l[q]);
    }
    return from_limbs(r);
}
__device__ __forceinline__ u128 readlane_u128(u128 v, int j) {
    u128 t = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        t |= (u128)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> (32 * q)), j) << (32 * q);
    return t;
}

// The search arrays of NU values per thread (value u of thread t is element
// u*kTailThreads + t, zero at or past n): the elements in a[], the sums of
// 16-element groups in g[] (a DPP row sum: 16 consecutive threads hold 16
// consecutive elements) and of 16-group super-groups in sg[] (wave 0).
// Every thread calls it; a barrier at the start and at the end.
template <int NU>
__device__ __forceinline__ void tail_sums(const u128 (&vals)[NU], int n, u128* a, u128* g, u128* sg) {
    const int tid = threadIdx.x;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const u128 r = row_sum_u128(vals[u]);
        const int i = u * kTailThreads + tid;
        a[i] = vals[u];
        if ((tid & 15) == 0) g[i >> 4] = r;
    }
    __syncthreads();
    if (tid < 64) {
        const int ng = (n + 15) >> 4;
        const u128 r = row_sum_u128(tid < ng ? g[tid] : (u128)0);
        if ((tid & 15) == 0) sg[tid >> 4] = r;
    }
    __syncthreads();
}

// One level of the search, called by a whole wave: among v[0..m) (m <= 16),
// the first j whose running sum, started at run, exceeds t; run becomes the
// sum before j.  -1 if none.  One LDS load per lane and a DPP row scan.
__device__ __forceinline__ int tail_level(const u128* v, int m, u128 t, u128& run) {
    const int lane = threadIdx.x & 63;
    const u128 own = lane < m ? v[lane] : (u128)0;
    const u128 pre = row_scan_u128(own) + run;
    const unsigned long long hit = __ballot(lane < m && pre > t);
    if (!hit) return -1;
    const int j = __ffsll((long long)hit) - 1;
    run = readlane_u128(pre - own, j);
    return j;
}

// First index of a[0..n) (n <= 1024) whose inclusive prefix exceeds t
// (tail_sums done), and in *before the sum of the elements before it; -1 if
// none.  Called by a whole wave; the results are uniform.
__device__ __forceinline__ int tail_pick(const u128* a, int n, const u128* g, const u128* sg, u128 t,
                                         u128* before) {
    const int ng = (n + 15) >> 4, ns = (ng + 15) >> 4;
    u128 run = 0;
    int J = 0;
    if (ns > 1) {
        J = tail_level(sg, ns, t, run);
        if (J < 0) return -1;
    }
    const int Q = tail_level(g + J * 16, min(16, ng - J * 16), t, run);
    if (Q < 0) return -1;
    const int q = J * 16 + Q;
    const int e = tail_level(a + q * 16, min(16, n - q * 16), t, run);
    if (e < 0) return -1;
    *before = run;
    return q * 16 + e;
}

template <int PER>
__global__ __launch_bounds__(kTailThreads) void acc_tail_kernel(
    const float* __restrict__ target, const float* __restrict__ draftl, int n_seq, int k, int V, float inv_t,
    const int32_t* __restrict__ draft, uint64_t seed, uint64_t seq_base, const float* __restrict__ part_max,
    const int* __restrict__ part_idx, const unsigned long long* __restrict__ part_sum,
    const float* __restrict__ xsel, unsigned long long* __restrict__ tw, int32_t* __restrict__ n_acc,
    int32_t* __restrict__ tokens) {
    const int c = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_tgt = n_seq * (k + 1), NR = 2 * k + 1;
    const int clen = (V + kTailChunks - 1) / kTailChunks, b0 = min(V, c * clen), b1 = min(V, b0 + clen);
    unsigned long long* cw = tw + (size_t)s * kTailChunks * 3;  // this sequence's chunk sums
    // arrival counters: this chunk's group, then the sequence's top counter
    unsigned long long* cbase = tw + (size_t)n_seq * kTailChunks * 3 + (size_t)s * (kTailArrGroups + 1) * kTailCntStride;
    int* gcnt = reinterpret_cast<int*>(cbase + (size_t)(c >> 4) * kTailCntStride);
    int* tcnt = reinterpret_cast<int*>(cbase + (size_t)kTailArrGroups * kTailCntStride);
    auto grow = [&](int rr) { return rr <= k ? s * (k + 1) + rr : n_tgt + s * k + (rr - k - 1); };
    auto rowp = [&](int rr) {
        return rr <= k ? target + (size_t)(s * (k + 1) + rr) * V : draftl + (size_t)(s * k + rr - k - 1) * V;
    };
    __shared__ float s_M[kTailRows];
    __shared__ int s_any[kTailRows];
    __shared__ unsigned long long s_S[kTailRows];
    __shared__ uint32_t s_U2[kTailRows];
    __shared__ int s_n, s_last, s_chunk;
    __shared__ u128 s_wtot[kTailWaves], s_rem;
    __shared__ unsigned long long s_ew[kTailWaves];
    // the last workgroup's searches (s_sg padded to one 16-lane level)
    __shared__ u128 s_a[kTailMaxN], s_g[kTailGroups], s_sg[16];

    TAIL_STAMP(0);
    // ---- loads, all issued before the first use: the row partials and the
    // draft tokens' logits first (the decisions wait for these only), then the
    // chunk of every row (unconditional loads from clamped addresses: no
    // branch per load; V >= 1)
    // wave w: rows w, w + 8, w + 16
    constexpr int kRowsPerWave = (kTailRows + kTailWaves - 1) / kTailWaves;
    float pm[kRowsPerWave];
    int pi[kRowsPerWave];
    unsigned long long ps[kRowsPerWave];
#pragma unroll
    for (int q = 0; q < kRowsPerWave; ++q) {
        const int rr = min(wave + q * kTailWaves, NR - 1);
        const size_t o = (size_t)grow(rr) * kChunks + lane;
        pm[q] = part_max[o];
        pi[q] = part_idx[o];
        ps[q] = part_sum[o];
    }
    float xp = 0.0f, xq = 0.0f;
    int xt_id = -1;
    if (wave == 0 && lane < k) {
        xt_id = draft[s * k + lane];
        xp = xsel[grow(lane)];
        xq = xsel[grow(k + 1 + lane)];
    }
    float xv[kTailRows][PER];
#pragma unroll
    for (int rr = 0; rr < kTailRows; ++rr)
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int v = b0 + tid + u * kTailThreads;
            xv[rr][u] = rowp(min(rr, NR - 1))[min(v, max(b1 - 1, 0))];
            if (rr >= NR || v >= b1) xv[rr][u] = __builtin_nanf("");
        }
    // the uniforms (no memory operands: computed while the loads are in
    // flight): U for the decision at position lane, U2 for a resample at
    // position lane
    uint32_t U = 0;
    if (wave == 0 && lane <= k) {
        U = fst_uniform24(seed, seq_base + (uint64_t)s, (uint32_t)lane, 0);
        s_U2[lane] = fst_uniform24(seed, seq_base + (uint64_t)s, (uint32_t)lane, 1);
    }
#pragma unroll
    for (int q = 0; q < kRowsPerWave; ++q) {
        const int rr = wave + q * kTailWaves;
        if (rr < NR) {
            wave_argmax(pm[q], pi[q]);
            const unsigned long long S = wave_sum_u64(ps[q]);
            if (lane == 0) {
                s_M[rr] = pm[q];
                s_any[rr] = pi[q] >= 0;
                s_S[rr] = S;
            }
        }
    }
    __syncthreads();
    TAIL_STAMP(1);
    // ---- the decisions (acc_decide_kernel's): lane i < k decides position i
    if (wave == 0) {
        int ok = 0;
        if (lane < k && xt_id >= 0 && xt_id < V) {
            const int rt = lane, rd = k + 1 + lane;
            const unsigned long long P = fixed_prob(xp, inv_t, s_M[rt], s_any[rt]);
            const unsigned long long Q = fixed_prob(xq, inv_t, s_M[rd], s_any[rd]);
            const u128 lhs = (u128)U * (u128)Q * (u128)s_S[rt];
            const u128 rhs = ((u128)P * (u128)s_S[rd]) << 24;
            ok = lhs < rhs;
        }
        const unsigned long long rej = __ballot(lane < k && !ok);
        if (lane == 0) s_n = rej ? __ffsll((long long)rej) - 1 : k;
    }
    __syncthreads();
    const int n = s_n, mode0 = n < k ? 0 : 1, tr = n, dr = min(k + 1 + n, NR - 1);
    const unsigned long long Sp = s_S[tr], Sq = mode0 == 0 ? s_S[dr] : 0ull;
    const float mp = s_M[tr], mq = mode0 == 0 ? s_M[dr] : 0.0f;
    const int ap = s_any[tr], aq = mode0 == 0 ? s_any[dr] : 0;
    // this thread's values of the sampling rows (uniform branches: no
    // dynamic register indexing)
    float xt[PER], xd[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) xt[u] = xd[u] = 0.0f;
#pragma unroll
    for (int rr = 0; rr < kTailRows; ++rr)
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            if (rr == tr) xt[u] = xv[rr][u];
            if (mode0 == 0 && rr == dr) xd[u] = xv[rr][u];
        }
    // ---- the chunk's residual and target-E sums (exact, any order)
    u128 ra = 0;
    unsigned long long ea = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        ra += res_of(xt[u], xd[u], inv_t, mp, ap, mq, aq, Sp, Sq, mode0);
        ea += fixed_prob(xt[u], inv_t, mp, ap);
    }
    ra = wave_sum_u128(ra);
    ea = wave_sum_u64(ea);
    if (lane == 0) {
        s_wtot[wave] = ra;
        s_ew[wave] = ea;
    }
    __syncthreads();
    TAIL_STAMP(2);
    if (tid == 0) {
        u128 rt = 0;
        unsigned long long et = 0;
        for (int w = 0; w < kTailWaves; ++w) {
            rt += s_wtot[w];
            et += s_ew[w];
        }
        st_coherent_u64(cw + (size_t)c * 3, (unsigned long long)rt);
        st_coherent_u64(cw + (size_t)c * 3 + 1, (unsigned long long)(rt >> 64));
        st_coherent_u64(cw + (size_t)c * 3 + 2, et);
        publish_wait();
        // the 16th arrival of a group of 16 chunks counts the group in at the
        // top; the last group to arrive makes this workgroup the last one
        // (both counters are left at zero)
        int last = 0;
        if (__hip_atomic_fetch_add(gcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 15) {
            __hip_atomic_store(gcnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = __hip_atomic_fetch_add(tcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kTailArrGroups - 1;
            if (last) __hip_atomic_store(tcnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last;
    }
    __syncthreads();
    TAIL_STAMP(3);
    if (!s_last) {
        TAIL_FLUSH(0, 4);
        return;
    }

    // ---- the last workgroup: the chunk holding the inverse-CDF target
    // (thread i < kTailChunks holds chunk i's sums)
    u128 cv[1] = {0};
    unsigned long long ce = 0;
    if (tid < kTailChunks) {
        const unsigned long long lo = ld_coherent_u64(cw + (size_t)tid * 3), hi = ld_coherent_u64(cw + (size_t)tid * 3 + 1);
        cv[0] = ((u128)hi << 64) | (u128)lo;
        ce = ld_coherent_u64(cw + (size_t)tid * 3 + 2);
    }
    tail_sums(cv, kTailChunks, s_a, s_g, s_sg);
    TAIL_STAMP(4);
    constexpr int kNs = (kTailChunks + 255) / 256;
    u128 tot = 0;
#pragma unroll
    for (int j = 0; j < kNs; ++j) tot += s_sg[j];
    int mode = mode0;
    if (mode == 0 && tot == 0) {
        // the residual is identically zero: sample from the target row
        mode = 1;
        cv[0] = (u128)ce;
        tail_sums(cv, kTailChunks, s_a, s_g, s_sg);
        tot = 0;
#pragma unroll
        for (int j = 0; j < kNs; ++j) tot += s_sg[j];
    }
    if (wave == 0) {
        int chunk = -1;
        u128 rem = 0;
        if (tot != 0) {
            const u128 tg = ((u128)s_U2[n] * tot) >> 24;
            u128 before;
            chunk = tail_pick(s_a, kTailChunks, s_g, s_sg, tg, &before);
            if (chunk >= 0) rem = tg - before;  // tg minus the mass before the chunk
        }
        if (lane == 0) {
            s_chunk = chunk;
            s_rem = rem;
        }
    }
    __syncthreads();
    TAIL_STAMP(5);
    const int cc = s_chunk;
    int tok = 0;  // (as the chain: no crossing in the chunk gives token 0)
    if (cc >= 0) {
        // ---- the token: the first v of the chunk (index order) whose
        // inclusive prefix exceeds the remaining target
        const int cb0 = min(V, cc * clen), cb1 = min(V, cb0 + clen);
        float a[PER], b[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int v = min(cb0 + tid + u * kTailThreads, cb1 - 1);
            a[u] = rowp(tr)[v];
            b[u] = mode == 0 ? rowp(dr)[v] : 0.0f;
        }
        u128 rv[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u)
            rv[u] = cb0 + tid + u * kTailThreads < cb1 ? res_of(a[u], b[u], inv_t, mp, ap, mq, aq, Sp, Sq, mode)
                                                      : (u128)0;
        tail_sums(rv, cb1 - cb0, s_a, s_g, s_sg);
        TAIL_STAMP(6);
        if (wave == 0) {
            u128 before;
            const int e = tail_pick(s_a, cb1 - cb0, s_g, s_sg, s_rem, &before);
            if (e >= 0) tok = cb0 + e;
        }
    }
    if (tid == 0) {
        for (int i = 0; i < n; ++i) tokens[s * (k + 1) + i] = draft[s * k + i];
        tokens[s * (k + 1) + n] = tok;
        for (int i = n + 1; i <= k; ++i) tokens[s * (k + 1) + i] = -1;
        n_acc[s] = n;
    }
    TAIL_STAMP(7);
    TAIL_FLUSH(0, 8);
}


// The tail launch applies when every row's chunk fits the registers.
static bool tail_fits(int k, int V) {
    return k >= 0 && 2 * k + 1 <= kTailRows && (V + kTailChunks - 1) / kTailChunks <= kTailPerMax * kTailThreads;
}

void launch_accept_stochastic(hipStream_t st, const float* target, const float* draft_logits,
                              int n_seq, int k, int V, const int32_t* draft, float inv_t,
                              uint64_t seed, uint64_t seq_base, int32_t* n_acc, int32_t* tokens,
                              void* ws, bool tail) {
    AccWs w = carve(ws, n_seq, k);
    const int n_tgt = n_seq * (k + 1);
    const int R = n_tgt + n_seq * k;
    const bool use_tail = tail && tail_fits(k, V);
    hipLaunchKernelGGL(acc_stats_kernel, dim3(kChunks, R), dim3(256), 0, st, target, draft_logits, n_tgt, V,
                       inv_t, w.part_max, w.part_idx);
    hipLaunchKernelGGL(acc_sums_kernel, dim3(kChunks, R), dim3(256), 0, st, target, draft_logits, n_tgt, V,
                       inv_t, w.part_max, w.part_idx, w.part_sum, draft, k, use_tail ? w.xsel : nullptr);
    if (use_tail) {
        // one element per thread while the chunks fit, else two
        auto kern = (V + kTailChunks - 1) / kTailChunks <= kTailThreads ? acc_tail_kernel<1> : acc_tail_kernel<2>;
        hipLaunchKernelGGL(kern, dim3(kTailChunks, n_seq), dim3(kTailThreads), 0, st, target, draft_logits, n_seq,
                           k, V, inv_t, draft, seed, seq_base, w.part_max, w.part_idx, w.part_sum, w.xsel, w.tail,
                           n_acc, tokens);
        return;
    }
    hipLaunchKernelGGL(acc_decide_kernel, dim3(n_seq), dim3(64 * kDecideWaves), 0, st, target, draft_logits, n_seq, k, V,
                       inv_t, draft, seed, seq_base, w.part_max, w.part_idx, w.part_sum, w.dec, n_acc,
                       tokens);
    hipLaunchKernelGGL(acc_res_chunks_kernel, dim3(kChunks, n_seq), dim3(kProbThreads), 0, st, target, draft_logits,
                       n_seq, k, V, inv_t, w.part_max, w.part_idx, w.dec, w.part_res);
    hipLaunchKernelGGL(acc_sample_kernel, dim3(n_seq), dim3(kProbThreads), 0, st, target, draft_logits, n_seq, k, V,
                       inv_t, w.part_max, w.part_idx, w.part_sum, w.dec, w.part_res, tokens);
}

// ---------------------------------------------------------- sample_token
//
// FSTEngine::sample_token (src/fst_engine.cpp:4491-4528) on the device, one
// workgroup per row of logits.  temperature <= 0 is the reference's plain
// argmax (first maximum, NaN skipped, a NaN at index 0 pins 0).  Otherwise
// the build's reproducible form of its softmax / top-p / draw (the reference
// draws from an unseeded mt19937): E[v] = floor(exp(x_v*(1/T) - max)*2^32),
// S = sum E; tokens ordered by E descending, ties by lower index; the kept
// set is the shortest prefix whose mass C has C*2^32 >= q*S (q = top_p in
// 2^-32 units), at least one token; the token is the first of the kept
// prefix whose running mass exceeds (U*C) >> 24, U = uniform24(seed, seq, 0,
// stream 2).  Both searches ("first position of the descending order whose
// running mass reaches T") run as radix selects over the 33-bit E values:
// E = 2^32 (the maxima) first, then 4 levels of 8-bit digits with LDS
// histograms of the digit's mass, then the rank among equal values in index
// order.  Integer sums: any reduction order gives the same result.
constexpr int kSampleThreads = 1024;
constexpr unsigned long long kOne32 = 4294967296ull;

__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long v, unsigned long long* red) {
    const int tid = threadIdx.x;
    v = wave_sum_u64_dpp(v);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    unsigned long long t = 0;
#pragma unroll
    for (int w = 0; w < kSampleThreads / 64; ++w) t += red[w];
    return t;
}

struct Cross {
    unsigned long long t;  // value E of the position
    unsigned long long G;  // mass of all values above t
    unsigned long long r;  // 1-based rank of the position among values == t
};

// First position of the (E desc, index asc) order whose running mass reaches
// T (1 <= T <= S); n_top = number of E == 2^32.
__device__ Cross find_cross(const unsigned long long* __restrict__ E, int V, unsigned long long T,
                            unsigned long long n_top, unsigned long long* hist, unsigned long long* bc) {
    const int tid = threadIdx.x;
    Cross c;
    if ((u128)T <= (u128)n_top * kOne32) {
        c.t = kOne32;
        c.G = 0;
        c.r = (T + kOne32 - 1) >> 32;
        return c;
    }
    unsigned long long G = n_top * kOne32, rem = T - G, prefix = 0;
    for (int lvl = 0; lvl < 4; ++lvl) {
        const int shift = 24 - 8 * lvl;
        __syncthreads();
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int v = tid; v < V; v += kSampleThreads) {
            const unsigned long long e = E[v];
            if (e < kOne32 && (e >> (shift + 8)) == prefix) atomicAdd(&hist[(e >> shift) & 255u], e);
        }
        __syncthreads();
        if (tid == 0) {
            unsigned long long acc = 0;
            int b = 255;
            for (; b > 0; --b) {
                if (acc + hist[b] >= rem) break;
                acc += hist[b];
            }
            bc[0] = acc;
            bc[1] = (unsigned long long)b;
        }
        __syncthreads();
        rem -= bc[0];
        G += bc[0];
        prefix = (prefix << 8) | bc[1];
    }
    c.t = prefix;
    c.G = G;
    c.r = prefix ? (rem + prefix - 1) / prefix : 1;
    return c;
}

// Index of the r-th (1-based) element with E == t, in index order.
__device__ int nth_equal(const unsigned long long* __restrict__ E, int V, unsigned long long t,
                         unsigned long long r, int* cnt, int* bc) {
    const int tid = threadIdx.x;
    const int per = (V + kSampleThreads - 1) / kSampleThreads;
    const int v0 = min(V, tid * per), v1 = min(V, v0 + per);
    int n = 0;
    for (int v = v0; v < v1; ++v) n += E[v] == t;
    __syncthreads();
    cnt[tid] = n;
    if (tid == 0) bc[0] = V - 1;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < kSampleThreads; ++i) {
            const int c = cnt[i];
            cnt[i] = run;
            run += c;
        }
    }
    __syncthreads();
    const long long want = (long long)r - 1;  // 0-based
    const int pre = cnt[tid];
    if (want >= pre && want < pre + n) {
        int k = pre;
        for (int v = v0; v < v1; ++v)
            if (E[v] == t) {
                if (k == want) {
                    bc[0] = v;
                    break;
                }
                ++k;
            }
    }
    __syncthreads();
    return bc[0];
}

__global__ __launch_bounds__(kSampleThreads) void sample_token_kernel(const float* __restrict__ logits, int V,
                                                                      float inv_t, int greedy, unsigned long long q,
                                                                      uint64_t seed, uint64_t seq_base,
                                                                      unsigned long long* __restrict__ Ews,
                                                                      int32_t* __restrict__ tokens) {
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* x = logits + (size_t)row * V;
    unsigned long long* E = Ews + (size_t)row * V;
    __shared__ float s_m[kSampleThreads / 64];
    __shared__ int s_i[kSampleThreads / 64];
    __shared__ unsigned long long red[kSampleThreads / 64];
    __shared__ unsigned long long hist[256];
    __shared__ unsigned long long bc[2];
    __shared__ int cnt[kSampleThreads];
    __shared__ int ibc[1];
    // (max, lowest index) of l = x*inv_t over non-NaN values (greedy: of x)
    const float sc = greedy ? 1.0f : inv_t;
    float best = 0.0f;
    int bi = -1;
    for_strided<8>(x, tid, V, kSampleThreads, [&](float xv, int v) {
        const float l = xv * sc;
        if (l != l) return;
        if (bi < 0 || l > best) {
            best = l;
            bi = v;
        }
    });
    wave_argmax(best, bi);
    if (lane == 0) {
        s_m[wave] = best;
        s_i[wave] = bi;
    }
    __syncthreads();
    for (int w = 0; w < kSampleThreads / 64; ++w) argmax_merge(best, bi, s_m[w], s_i[w]);
    if (greedy) {
        if (tid == 0) tokens[row] = (bi < 0 || x[0] != x[0]) ? 0 : bi;
        return;
    }
    const int any = bi >= 0;
    unsigned long long s = 0, ntop = 0;
    for_strided<8>(x, tid, V, kSampleThreads, [&](float xv, int v) {
        const unsigned long long e = fixed_prob(xv, inv_t, best, any);
        E[v] = e;
        s += e;
        ntop += e == kOne32;
    });
    const unsigned long long S = block_sum_u64(s, red);
    const unsigned long long n_top = block_sum_u64(ntop, red);
    if (S == 0) {
        if (tid == 0) tokens[row] = 0;
        return;
    }
    __syncthreads();  // E stores of every thread are visible to the searches
    u128 need = ((u128)q * S + (kOne32 - 1)) >> 32;
    const unsigned long long Tp = need == 0 ? 1ull : (unsigned long long)need;
    const Cross k = find_cross(E, V, Tp, n_top, hist, bc);
    const unsigned long long C = k.G + k.r * k.t;
    const uint32_t U = fst_uniform24(seed, seq_base + (uint64_t)row, 0u, 2u);
    const unsigned long long tgt = (unsigned long long)(((u128)U * C) >> 24);
    const Cross d = find_cross(E, V, tgt + 1, n_top, hist, bc);
    const int tok = nth_equal(E, V, d.t, d.r, cnt, ibc);
    if (tid == 0) tokens[row] = tok;
}

void launch_sample_token(hipStream_t st, const float* logits, int n_rows, int V, float temperature, float top_p,
                         uint64_t seed, uint64_t seq_base, void* ws, int32_t* tokens) {
    const int greedy = !(temperature > 0.0f);
    const float inv_t = greedy ? 1.0f : 1.0f / temperature;
    unsigned long long q;
    if (!(top_p > 0.0f))
        q = 0;
    else if (top_p >= 1.0f)
        q = kOne32;
    else
        q = (unsigned long long)((double)top_p * 4294967296.0);  // exact product, truncated
    hipLaunchKernelGGL(sample_token_kernel, dim3(n_rows), dim3(kSampleThreads), 0, st, logits, V, inv_t, greedy, q,
                       seed, seq_base, static_cast<unsigned long long*>(ws), tokens);
}

size_t sample_ws_bytes(int n_rows, int V) { return (size_t)n_rows * V * 8 + 256; }

// ---- scratch of the allocation-free greedy entry point ----
// The greedy hand-off words of fst_accept_greedy_dev_noalloc live in this
// fixed device array instead of a context workspace: kStaticGreedyRows rows
// of kGreedyChunks words (256 KiB), held by every device the library runs on
// until the process ends.  Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// handed to kernels: in host code the array's name is not a device address.
// Every call on a device shares the array; calls that overlap on one device
// race.  Each call takes the next epoch of the device (1..4095), so no
// clearing is needed between calls (zero-initialised words carry epoch 0,
// never used); the array is cleared with a fill kernel before each call
// that takes epoch 1, so that late words of a timed-out call cannot match
// a reused epoch.
static __device__ __align__(256) unsigned long long scratch[kStaticGreedyRows * kGreedyChunks];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];
std::atomic<uint32_t> g_scratch_epoch[kMaxDevices];
}  // namespace

int accept_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return set_error(FST_ENODEV, "device ordinal beyond the scratch table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return 0;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_error(FST_EHIP, (std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e)).c_str());
    g_scratch_ptr[device] = p;
    return 0;
}

void* accept_scratch_ptr(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[device];
}

__global__ __launch_bounds__(256) void fill_zero_u64_kernel(unsigned long long* __restrict__ p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0ull;
}

void accept_scratch_clear(hipStream_t st, void* words) {
    constexpr int n = kStaticGreedyRows * kGreedyChunks;
    hipLaunchKernelGGL(fill_zero_u64_kernel, dim3(64), dim3(256), 0, st, static_cast<unsigned long long*>(words), n);
}

uint32_t accept_scratch_epoch(int device) {
    // 1..4095 in turn (the tag field of a greedy word holds 12 bits)
    const uint32_t n = g_scratch_epoch[device].fetch_add(1u, std::memory_order_relaxed);
    return n % 4095u + 1u;
}

}  // namespace fst
