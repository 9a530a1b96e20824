// fst_accept.hip — greedy and rejection-sampling acceptance for gfx950.
//
// Rows: target rows r = s*(k+1)+i (i = 0..k) of n_seq sequences, then (for
// rejection sampling) draft rows n_seq*(k+1) + s*k + i.
//
// Greedy (src/fst_engine.cpp:6021-6063): argmax per target row with the
// reference's sequential semantics (first maximum wins, NaN skipped, a NaN at
// index 0 pins the result to 0), then the longest matching prefix and bonus.
//
// Rejection sampling (defined by this build; the reference is greedy-only):
// each row's softmax (max, sum) in binary32 with a fixed chunking and
// summation order, u < p/q decided as u*q < p, and the resampled (or bonus)
// token drawn by an exponential race (argmin of -log(u_v)/r_v over the
// residual r = p - q > 0, per-element Philox uniforms), as Gumbel-max
// sampling draws; every operation is the CPU oracle's, in the same order, so
// the accepted lengths and tokens are identical to it for identical logits.
#include <atomic>
#include <mutex>
#include <string>

#include "fst_internal.h"
#include "../../include/fst_hip.h"
#include "../../include/fst_exact_math.h"

namespace fst {

typedef unsigned __int128 u128;

// Rejection sampling: softmax-statistics chunks per row, race chunks per
// sequence (the tail launch's workgroups), threads of the tail launch, and
// the tail's arrival counters: kRsArrGroups groups of 16 race chunks, then
// one top counter, each on its own 256-byte line.
constexpr int kRsChunks = 64;
constexpr int kRsRaceChunks = 256;
constexpr int kRsTailThreads = 512;
constexpr int kRsArrGroups = kRsRaceChunks / 16;
constexpr int kRsCntStride = 32;  // u64 words between counters
constexpr int kRsMaxRows = 2 * 63 + 1;  // rows of one sequence (k <= 63)
// [n_seq][kRsRaceChunks][2] chunk race results, then [n_seq][kRsArrGroups + 1] counters.
static size_t rs_tail_words(int n_seq) {
    return (size_t)n_seq * kRsRaceChunks * 2 + (size_t)n_seq * (kRsArrGroups + 1) * kRsCntStride;
}

struct AccWs {
    unsigned long long* gslot;     // [R][kGreedySlots] greedy chunk words (zero between calls)
    float2* rs_part;               // [R][kRsChunks] rejection sampling: chunk (max, sum)
    float* xsel;                   // [R] each row's scaled logit at its position's draft token
    unsigned long long* tail;      // acc_rs_tail_kernel: chunk race results and counters (counters zero between calls)
};
constexpr int kGreedySlots = 64;   // >= the greedy launch's chunks per row

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static AccWs carve(void* ws, int n_seq, int k) {
    const int R = n_seq * (k + 1) + n_seq * k;
    char* p = (char*)ws;
    AccWs w;
    w.gslot = (unsigned long long*)p; p += align256(8ull * R * kGreedySlots);
    w.rs_part = (float2*)p; p += align256(8ull * R * kRsChunks);
    w.xsel = (float*)p; p += align256(sizeof(float) * R);
    w.tail = (unsigned long long*)p;
    return w;
}

size_t accept_ws_bytes(int n_seq, int k, int V) {
    (void)V;
    const int R = n_seq * (k + 1) + n_seq * k;
    return align256(8ull * R * kGreedySlots) + align256(8ull * R * kRsChunks) + align256(sizeof(float) * R) +
           align256(8ull * rs_tail_words(n_seq)) + 256;
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


// ------------------------------------------------- rejection sampling
//
// Two launches per call, with the CPU oracle's arithmetic in its order
// (fo_rs_row_stats, fo_rs_race, fo_accept_stochastic):
//   acc_rs_stats_kernel  workgroup (c, r): chunk c of row r (kRsChunks chunks
//                        of L = ceil(V/64) rounded up to 4 elements) reduced
//                        to its softmax partial (m_c, s_c): thread t adds
//                        e(x | m_c) over elements b0 + 4t + 1024i + {0..3}
//                        in that order, the waves' partials by the halving
//                        tree, the four wave sums left to right; the
//                        workgroup whose chunk holds the row's draft token
//                        also stores that scaled logit (xsel);
//   acc_rs_tail_kernel   workgroup (c, s): every workgroup merges the
//                        sequence's row partials into (M, S) per row (the
//                        halving tree over the 64 chunks), takes the accept
//                        decisions (wave 0, one lane per position), runs the
//                        exponential race over race chunk c of the first
//                        rejected position (or the bonus row), publishes the
//                        chunk's two minimum keys with device-coherent stores
//                        and counts itself in (the 16th arrival of a group of
//                        16 chunks counts the group in at a top counter, each
//                        on its own line); the last workgroup takes the
//                        minimum over the chunks and writes n_acc and the
//                        tokens.  With at most 16 rows per sequence (k <= 7)
//                        and short race chunks, every row's chunk is loaded
//                        with the partials, so the race does not wait for a
//                        second round trip after the decisions.
// No workgroup waits for another, so any grid is safe; the counters are
// left at zero by their last arrival.
__device__ __forceinline__ int rs_chunk_len(int V) { return ((V + kRsChunks - 1) / kRsChunks + 3) & ~3; }

// e(x | M) of a scaled logit: 0 for NaN, -inf, or a row with no number
__device__ __forceinline__ float rs_e(float x, float M) {
    if (x != x || M == fst_bits_f32(0xff800000u)) return 0.0f;
    return fst_rel_exp(x, M);
}

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long x) { return ~wave_max_u64(~x); }

// fst_softmax_merge with one exponential: the larger maximum's weight is
// exactly 1 and s*1 = s, so a = s1*w1, b = s2*w2, a + b come out bit for bit.
__device__ __forceinline__ void rs_merge(float& m1, float& s1, float m2, float s2) {
    const float ninf = fst_bits_f32(0xff800000u);
    const bool first = m1 >= m2 || m2 != m2;
    const float M = first ? m1 : m2;
    const float lo = first ? m2 : m1, slo = first ? s2 : s1, shi = first ? s1 : s2;
    const float w = lo == M ? 1.0f : fst_exp_nonpos(lo - M);
    const float b = slo * w;
    s1 = M == ninf ? 0.0f : shi + b;
    m1 = M;
}
// Two rows' merges in one wave, each the halving tree over its 64 chunk
// partials: lanes 0..31 hold row A's chunks j and j + 32 (tree level 32 is
// their local merge), lanes 32..63 row B's; levels 16..1 then run in both
// halves at once (the row-pair swap and DPP row shifts stay inside a half).
// Results in lanes 0 (row A) and 32 (row B).
__device__ __forceinline__ void rs_tree_merge2(float& m, float& s, float m_hi, float s_hi) {
    auto take = [&](float om, float os) { rs_merge(m, s, om, os); };
    take(m_hi, s_hi);
    {
        const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, m), false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, s), __builtin_bit_cast(uint32_t, s), false, false);
        take(__builtin_bit_cast(float, (uint32_t)a[1]), __builtin_bit_cast(float, (uint32_t)b[1]));
    }
    take(fdpp<0x108>(m), fdpp<0x108>(s));  // row_shl 8
    take(fdpp<0x104>(m), fdpp<0x104>(s));  // row_shl 4
    take(fdpp<0x102>(m), fdpp<0x102>(s));  // row_shl 2
    take(fdpp<0x101>(m), fdpp<0x101>(s));  // row_shl 1
}

// Chunk partial of thread-ordered values xv (NaN: no element), rounds of 4.
template <int NI>
__device__ __forceinline__ float rs_thread_sum(const float (&xv)[NI][4], float m, float acc) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = xv[i][e];
            if (x == x) acc = acc + fst_rel_exp(x, m);
        }
    return acc;
}

// Loads rounds [i0, i0 + NI) of this thread's elements of [b0, b1), scaled;
// NaN past b1.
template <int NI>
__device__ __forceinline__ void rs_load_rounds(const float* __restrict__ row, int V, int b0, int b1, int i0,
                                               float inv_t, float (&xv)[NI][4]) {
    const int tid = threadIdx.x;
    const float nan = __builtin_nanf("");
    if ((V & 3) == 0) {
        // 16-byte loads, all issued before any is used (b1 - 4 >= 0: V >= 4)
        float4 q[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            q[i] = *reinterpret_cast<const float4*>(row + min(b0 + 4 * tid + 1024 * (i0 + i), b1 - 4));
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int v = b0 + 4 * tid + 1024 * (i0 + i);
            xv[i][0] = v < b1 ? q[i].x * inv_t : nan;
            xv[i][1] = v + 1 < b1 ? q[i].y * inv_t : nan;
            xv[i][2] = v + 2 < b1 ? q[i].z * inv_t : nan;
            xv[i][3] = v + 3 < b1 ? q[i].w * inv_t : nan;
        }
    } else {
        float q[NI][4];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) q[i][e] = row[min(b0 + 4 * tid + 1024 * (i0 + i) + e, V - 1)];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = b0 + 4 * tid + 1024 * (i0 + i) + e < b1 ? q[i][e] * inv_t : nan;
    }
}

// REG: the chunk fits the registers (L <= 4096: four rounds), one pass over
// memory; else two passes (maximum, then the sum from the device cache).
template <bool REG>
__global__ __launch_bounds__(256) void acc_rs_stats_kernel(const float* __restrict__ target,
                                                           const float* __restrict__ draftl, int n_seq, int k,
                                                           int V, float inv_t, const int32_t* __restrict__ draft,
                                                           float2* __restrict__ part, float* __restrict__ xsel) {
    const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_tgt = n_seq * (k + 1);
    const float* row = r < n_tgt ? target + (size_t)r * V : draftl + (size_t)(r - n_tgt) * V;
    int di = r - n_tgt;  // this row's draft token: draft[di] (draft rows s*k+i, target rows s*(k+1)+i, i < k)
    if (r < n_tgt) {
        const int s = r / (k + 1), i = r - s * (k + 1);
        di = i < k ? s * k + i : -1;
    }
    const int x_id = di >= 0 ? draft[di] : -1;
    const int L = rs_chunk_len(V), b0 = min(V, c * L), b1 = min(V, b0 + L);
    const int nrounds = (L + 1023) / 1024;
    __shared__ float s_m[4], s_s[4];
    float m = fst_bits_f32(0xff800000u), acc = 0.0f;
    constexpr int NI = 4;
    float xv[NI][4];
    if (REG) rs_load_rounds<NI>(row, V, b0, b1, 0, inv_t, xv);
    for (int i0 = 0; i0 < (REG ? NI : nrounds); i0 += NI) {
        if (!REG) rs_load_rounds<NI>(row, V, b0, b1, i0, inv_t, xv);
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) m = fmaxf(m, xv[i][e]);  // fmaxf skips NaN
    }
    m = wave_fmax(m);
    if (lane == 0) s_m[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    if (REG) {
        acc = rs_thread_sum<NI>(xv, m, acc);
    } else {
        for (int i0 = 0; i0 < nrounds; i0 += NI) {
            rs_load_rounds<NI>(row, V, b0, b1, i0, inv_t, xv);
            acc = rs_thread_sum<NI>(xv, m, acc);
        }
    }
    acc = tree_sum64(acc);
    if (lane == 0) s_s[wave] = acc;
    __syncthreads();
    if (tid == 0) {
        part[(size_t)r * kRsChunks + c] = make_float2(m, ((s_s[0] + s_s[1]) + s_s[2]) + s_s[3]);
        if (x_id >= b0 && x_id < b1) xsel[r] = row[x_id] * inv_t;
    }
}

// PRE: every row's race chunk is loaded with the partials (at most kPreRows
// rows per sequence, race chunks of at most kRsTailThreads elements).
constexpr int kPreRows = 16;
template <bool PRE>
__global__ __launch_bounds__(kRsTailThreads) void acc_rs_tail_kernel(
    const float* __restrict__ target, const float* __restrict__ draftl, int n_seq, int k, int V, float inv_t,
    const int32_t* __restrict__ draft, uint64_t seed, uint64_t seq_base, const float2* __restrict__ part,
    const float* __restrict__ xsel, unsigned long long* __restrict__ tw, int32_t* __restrict__ n_acc,
    int32_t* __restrict__ tokens) {
    constexpr int NW = kRsTailThreads / 64;
    const int c = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_tgt = n_seq * (k + 1), NR = 2 * k + 1;
    const uint64_t seq = seq_base + (uint64_t)s;
    unsigned long long* cw = tw + (size_t)s * kRsRaceChunks * 2;  // this sequence's chunk results
    unsigned long long* cbase =
        tw + (size_t)n_seq * kRsRaceChunks * 2 + (size_t)s * (kRsArrGroups + 1) * kRsCntStride;
    int* gcnt = reinterpret_cast<int*>(cbase + (size_t)(c >> 4) * kRsCntStride);
    int* tcnt = reinterpret_cast<int*>(cbase + (size_t)kRsArrGroups * kRsCntStride);
    auto grow = [&](int rr) { return rr <= k ? s * (k + 1) + rr : n_tgt + s * k + (rr - k - 1); };
    auto rowp = [&](int rr) -> const float* {
        return rr <= k ? target + (size_t)(s * (k + 1) + rr) * V : draftl + (size_t)(s * k + rr - k - 1) * V;
    };
    __shared__ float s_M[kRsMaxRows], s_S[kRsMaxRows];
    __shared__ int s_n, s_last;
    __shared__ unsigned long long s_kr[NW], s_kp[NW];
    const int Lr = (V + kRsRaceChunks - 1) / kRsRaceChunks, b0 = min(V, c * Lr), b1 = min(V, b0 + Lr);

    // the decision inputs (wave 0, lane i < k: position i), loaded first
    int x_id = -1;
    float xp = 0.0f, xq = 0.0f;
    if (wave == 0 && lane < k) {
        x_id = draft[s * k + lane];
        xp = xsel[grow(lane)];
        xq = xsel[grow(k + 1 + lane)];
    }
    // every row's (M, S): wave w merges rows 2w and 2w + 1, then 2w + 16, ...
    // (lane j < 32: chunks j and j + 32 of the first row, lane 32 + j those
    // of the second), the first pass's loads issued before the row values
    const int hrow = lane >> 5, hl = lane & 31;
    float2 pa[2];
    {
        const int rr = min(2 * wave + hrow, NR - 1);
        pa[0] = part[(size_t)grow(rr) * kRsChunks + hl];
        pa[1] = part[(size_t)grow(rr) * kRsChunks + hl + 32];
    }
    // PRE: this thread's element of race chunk c in every row
    float pre[PRE ? kPreRows : 1];
    if constexpr (PRE) {
        const int v = min(b0 + tid, V - 1);
#pragma unroll
        for (int rr = 0; rr < kPreRows; ++rr) pre[rr] = rowp(min(rr, NR - 1))[v];
    }
    for (int rr0 = 2 * wave; rr0 < NR; rr0 += 2 * NW) {
        if (rr0 != 2 * wave) {
            const int rr = min(rr0 + hrow, NR - 1);
            pa[0] = part[(size_t)grow(rr) * kRsChunks + hl];
            pa[1] = part[(size_t)grow(rr) * kRsChunks + hl + 32];
        }
        float m = pa[0].x, sm = pa[0].y;
        rs_tree_merge2(m, sm, pa[1].x, pa[1].y);
        const int rr = rr0 + hrow;
        if (hl == 0 && rr < NR) {
            s_M[rr] = m;
            s_S[rr] = sm;
        }
    }
    uint32_t U = 0;
    if (wave == 0 && lane < k) U = fst_uniform24(seed, seq, (uint32_t)lane, 0);
    __syncthreads();
    // the decisions: lane i < k decides position i; n = the first reject
    if (wave == 0) {
        int ok = 0;
        if (lane < k && x_id >= 0 && x_id < V) {
            const float St = s_S[lane], Sd = s_S[k + 1 + lane];
            const float et = rs_e(xp, s_M[lane]), ed = rs_e(xq, s_M[k + 1 + lane]);
            const float u = (float)U * 5.9604644775390625e-8f;
            const float lhs = (u * ed) * St, rhs = et * Sd;
            ok = lhs < rhs;
        }
        const unsigned long long rej = __ballot(lane < k && !ok);
        if (lane == 0) s_n = rej ? __ffsll((long long)rej) - 1 : k;
    }
    __syncthreads();
    const int n = s_n;
    const bool has_d = n < k;
    const float Mt = s_M[n], St = s_S[n];
    const float Md = has_d ? s_M[k + 1 + n] : 0.0f, Sd = has_d ? s_S[k + 1 + n] : 0.0f;
    const float* trow = rowp(n);
    const float* drow = has_d ? rowp(k + 1 + n) : trow;
    // the race over chunk c: keys (bits of E/r << 32 | v) over r > 0 and
    // (fallback) E/e_t over e_t > 0
    unsigned long long kr = ~0ull, kp = ~0ull;
    for (int v = b0 + tid; v < b1; v += kRsTailThreads) {
        float tv, dv;
        if constexpr (PRE) {
            // (uniform selects: no dynamic register indexing)
            tv = dv = 0.0f;
#pragma unroll
            for (int rr = 0; rr < kPreRows; ++rr) {
                if (rr == n) tv = pre[rr];
                if (has_d && rr == k + 1 + n) dv = pre[rr];
            }
        } else {
            tv = trow[v];
            dv = drow[v];
        }
        const float et = rs_e(tv * inv_t, Mt);
        float r = et;
        if (has_d) {
            const float ed = rs_e(dv * inv_t, Md);
            const float a = et * Sd, b = ed * St;
            r = a - b;
        }
        fst_philox_ctr ctr;
        ctr.v[0] = (uint32_t)v;
        ctr.v[1] = 0x52430000u ^ (uint32_t)n;
        ctr.v[2] = (uint32_t)seq;
        ctr.v[3] = (uint32_t)(seq >> 32);
        const fst_philox_ctr w = fst_philox4x32_10(ctr, (uint32_t)seed, (uint32_t)(seed >> 32));
        const float u = (float)(2u * (w.v[0] >> 9) + 1u) * 5.9604644775390625e-8f;
        const float E = -fst_logf(u);
        if (r > 0.0f) {
            const unsigned long long key = ((unsigned long long)fst_f32_bits(E / r) << 32) | (uint32_t)v;
            kr = key < kr ? key : kr;
        }
        if (et > 0.0f) {
            const unsigned long long key = ((unsigned long long)fst_f32_bits(E / et) << 32) | (uint32_t)v;
            kp = key < kp ? key : kp;
        }
    }
    kr = wave_min_u64(kr);
    kp = wave_min_u64(kp);
    if (lane == 0) {
        s_kr[wave] = kr;
        s_kp[wave] = kp;
    }
    __syncthreads();
    // publish the chunk's keys and count in
    if (tid == 0) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            kr = s_kr[w] < kr ? s_kr[w] : kr;
            kp = s_kp[w] < kp ? s_kp[w] : kp;
        }
        st_coherent_u64(cw + 2 * c, kr);
        st_coherent_u64(cw + 2 * c + 1, kp);
        publish_wait();
        int last = 0;
        if (__hip_atomic_fetch_add(gcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 15) {
            __hip_atomic_store(gcnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = __hip_atomic_fetch_add(tcnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kRsArrGroups - 1;
            if (last) __hip_atomic_store(tcnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // the last workgroup: the minimum keys over the chunks give the token
    unsigned long long a = ~0ull, b = ~0ull;
    if (tid < kRsRaceChunks) {
        a = ld_coherent_u64(cw + 2 * tid);
        b = ld_coherent_u64(cw + 2 * tid + 1);
    }
    a = wave_min_u64(a);
    b = wave_min_u64(b);
    __syncthreads();
    if (lane == 0) {
        s_kr[wave] = a;
        s_kp[wave] = b;
    }
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            a = s_kr[w] < a ? s_kr[w] : a;
            b = s_kp[w] < b ? s_kp[w] : b;
        }
        const int tok = a != ~0ull ? (int)(uint32_t)a : (b != ~0ull ? (int)(uint32_t)b : 0);
        for (int i = 0; i < n; ++i) tokens[s * (k + 1) + i] = draft[s * k + i];
        tokens[s * (k + 1) + n] = tok;
        for (int i = n + 1; i <= k; ++i) tokens[s * (k + 1) + i] = -1;
        n_acc[s] = n;
    }
}

void launch_accept_stochastic(hipStream_t st, const float* target, const float* draft_logits,
                              int n_seq, int k, int V, const int32_t* draft, float inv_t,
                              uint64_t seed, uint64_t seq_base, int32_t* n_acc, int32_t* tokens, void* ws) {
    AccWs w = carve(ws, n_seq, k);
    const int R = n_seq * (2 * k + 1);
    const int L = ((V + kRsChunks - 1) / kRsChunks + 3) & ~3;
    if (L <= 4096)
        hipLaunchKernelGGL(acc_rs_stats_kernel<true>, dim3(kRsChunks, R), dim3(256), 0, st, target, draft_logits,
                           n_seq, k, V, inv_t, draft, w.rs_part, w.xsel);
    else
        hipLaunchKernelGGL(acc_rs_stats_kernel<false>, dim3(kRsChunks, R), dim3(256), 0, st, target, draft_logits,
                           n_seq, k, V, inv_t, draft, w.rs_part, w.xsel);
    const bool pre = 2 * k + 1 <= kPreRows && (V + kRsRaceChunks - 1) / kRsRaceChunks <= kRsTailThreads;
    auto tail = pre ? acc_rs_tail_kernel<true> : acc_rs_tail_kernel<false>;
    hipLaunchKernelGGL(tail, dim3(kRsRaceChunks, n_seq), dim3(kRsTailThreads), 0, st, target, draft_logits, n_seq,
                       k, V, inv_t, draft, seed, seq_base, w.rs_part, w.xsel, w.tail, n_acc, tokens);
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
// E = floor(exp(x*inv_t - max) * 2^32) of one logit (0 for NaN or a row
// without numbers), the fixed-point mass of sample_token.
__device__ __forceinline__ unsigned long long fixed_prob(float x, float inv_t, float mx, int any) {
    const float l = x * inv_t;
    if (!any || l != l) return 0ull;
    if (l == mx) return 4294967296ull;
    const float d = l - mx;
    if (d != d) return 0ull;
    return (unsigned long long)fst_prob_fixed(d);
}
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
