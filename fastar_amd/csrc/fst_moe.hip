// fst_moe.hip — MoE-layer verify kernels for gfx950 (MI355X).
//
// One MoE layer call is a fixed chain of stream-ordered launches with no host
// round trip:
//   router_prep     h[M,K] . W_r (canonical fp32 order, bit-exact vs the CPU
//                   oracle) and, in extra workgroups, h -> prescaled fp16 operand
//   route_bucket    top-k + weights; the last workgroup groups (token, expert)
//                   pairs per expert slot
//   q4k_linear<1>   gate||up: fused Q4_K decode + MFMA; each workgroup pairs 64
//                   gate rows with the same 64 up rows -> h = silu(g)*u
//   prep_act        h -> prescaled fp16 operand (one workgroup per pair)
//   q4k_linear<2>   down; the last contribution to each (token, 128-row tile)
//                   combines it: out[t] = sum_j w[t][j] y[pair(t,j)] + y[shared(t)]
//
// The Q4_K contraction (reference semantics: kernels/fst_dequant_q4k_kernel.cc
// w = d*sc*q - dmin*m, GEMM orientation A.B^T from scripts/fst_validate_gemms.py:174)
// is factored so that no per-weight floating multiply by d or dmin is needed:
//   sum_k w_k x_k = d * sum_k (sc_j(k) q_k) x_k  -  dmin * sum_j m_j Sx_j
// sc*q <= 945 is an exact fp16 integer, built from the nibble with one
// v_and_or (fp16 1024+q) and one v_pk_fma_f16 ((1024+q)*sc - 1024*sc, exact),
// and fed to v_mfma_f32_16x16x32_f16 with the tokens as the A operand.  The
// min term is a second MFMA over the per-sub-block activation sums (split
// hi+lo in fp16).  d and dmin scale once per 256-weight super-block.
// Activations are prescaled per token by a power of two (exact) so the fp16
// operand covers their range.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "fst_internal.h"
#include <hip/hip_ext.h>
#include "fst_q4k_dev.h"
#include "../../include/fst_exact_math.h"

namespace fst {


// ---------------------------------------------------------------- router

// Router logits: one wave per (expert, TPW tokens); lane j owns the
// contiguous K/64 chunk j (NV = K/512 16-byte pieces), sums it with a
// sequential fmaf chain, then the 64 partials are combined by the halving
// tree p[j] += p[j+off] (off = 32..1) that lane 0 sees through shfl_down.
// Lane 0 stores the logit's score (sigmoid or sqrt(softplus), after the
// optional bf16 rounding).
//  - weights: the router is stored lane-interleaved per expert (piece i of
//    lane j at 16-byte index 64 i + j, router_interleave), so load i of a
//    wave is one contiguous kilobyte;
//  - activations: the workgroup copies its TPW rows once into LDS (sm) with
//    the same interleave, rows padded to 65 pieces per i so that both the
//    copy and the per-lane reads spread over the banks; the 4 waves share it.
// Workgroups past the router part each prepare one token row of the expert
// operand (prep_row), so both consumers of h share one launch.
template <int NV, int TPW>
__device__ void router_block(const uint4* __restrict__ w_il, const uint16_t* __restrict__ h, int M, int E,
                             int bx, int by, int score_func, int round_bf16, float* __restrict__ scores,
                             uint4* sm) {
    constexpr int RU = 64 * NV;                      // 16-byte pieces per row
    constexpr int NL = (TPW * RU + 255) / 256;       // copy loads per thread
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int e = bx * 4 + wave;
    const int t0 = by * TPW;
    uint4 wq[NV];
    if (e < E) {
        const uint4* wp = w_il + (size_t)e * RU + lane;
#pragma unroll
        for (int i = 0; i < NV; ++i) wq[i] = wp[i * 64];
    }
    {
        const uint4* h4 = reinterpret_cast<const uint4*>(h);
        uint4 v[NL];
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int q = tid + 256 * u, t = q / RU;
            v[u] = make_uint4(0u, 0u, 0u, 0u);
            if (q < TPW * RU && t0 + t < M) v[u] = h4[(size_t)(t0 + t) * RU + (q - t * RU)];
        }
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int q = tid + 256 * u, t = q / RU, qq = q - t * RU;
            const int j = qq / NV, i = qq - j * NV;
            if (q < TPW * RU) sm[(t * NV + i) * 65 + j] = v[u];
        }
    }
    __syncthreads();
    if (e >= E) return;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        if (t0 + t >= M) continue;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint4 xq = sm[(t * NV + i) * 65 + lane];
            const uint32_t wv[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
            const uint32_t xv[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc = fmaf(fst_bits_f32(xv[k] << 16), fst_bits_f32(wv[k] << 16), acc);
                acc = fmaf(fst_bits_f32(xv[k] & 0xffff0000u), fst_bits_f32(wv[k] & 0xffff0000u), acc);
            }
        }
        acc = tree_sum64(acc);
        if (lane == 0) {
            // the score of the logit (src/fst_engine.cpp:974-983), computed
            // where the logit is produced so the top-k only compares
            float x = acc;
            if (round_bf16) x = fst_bf16_to_f32(fst_f32_to_bf16(x));
            scores[(size_t)(t0 + t) * E + e] = score_func == 0 ? fst_sigmoidf(x) : fst_sqrtsoftplusf(x);
        }
    }
}

// ------------------------------------------------------------ route + bucket

constexpr int kMaxExperts = 1024;

// Total order used for top-k: larger score first, then lower expert id; NaN
// scores rank below every number (and among themselves by id).  Encoded as a
// 64-bit key: (order-preserving bits of the score) << 32 | (0xffffffff - id).
// -0 is folded into +0 so that equal scores compare equal as in float math.
__device__ __forceinline__ unsigned long long topk_key(float sel, int id) {
    uint32_t u = fst_f32_bits(sel == 0.0f ? 0.0f : sel);
    uint32_t o;
    if (sel != sel)
        o = 0u;
    else
        o = (u >> 31) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (0xffffffffu - (uint32_t)id);
}

// (token, expert) pairs grouped per slot: the shared expert (if used) is slot
// 0 with all M tokens (so its work starts first), then the routed experts in
// ascending id, tokens ascending within an expert.  Also counts each token's
// distinct pairs (the number of down contributions its combine waits for).
// eids_s: the call's [M][tk] expert ids, already in LDS.  One workgroup of NT
// threads.
template <int NT, int MAXE = kMaxExperts>
__device__ void bucket_block(int M, int E, int tk, int use_shared, const int* eids_s, int topk_err,
                             int* __restrict__ meta, int* __restrict__ slot_eid, int* __restrict__ slot_M,
                             int* __restrict__ slot_off, int* __restrict__ pair_tok,
                             int* __restrict__ pair_of, int* __restrict__ pair_shared) {
    __shared__ unsigned long long hitmask[MAXE];
    __shared__ int eoff[MAXE];
    __shared__ int err;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) err = 0;
    for (int e = tid; e < E; e += NT) hitmask[e] = 0ull;
    __syncthreads();
    for (int i = tid; i < M * tk; i += NT) {
        const int t = i / tk;
        const int e = eids_s[i];
        if (e < 0 || e >= E)
            atomicOr(&err, 1);
        else
            atomicOr(&hitmask[e], 1ull << t);
    }
    __syncthreads();
    const int s0 = use_shared ? 1 : 0, p0 = use_shared ? M : 0;
    // Slots and pairs numbered in ascending expert id, one expert per
    // thread: exclusive prefix counts within each wave from ballots (a count
    // of at most 64 tokens summed bit-plane by bit-plane), then the totals of
    // the waves before it.
    constexpr int NW = NT / 64;
    __shared__ int s_wtot[2][NW];
    int slot_base = s0, pair_base = p0;
    for (int e0 = 0; e0 < E; e0 += NT) {
        const int e = e0 + tid;
        const int cnt = (e < E) ? __popcll(hitmask[e]) : 0;
        const unsigned long long ba = __ballot(cnt > 0);
        int ex_a = lane_prefix(ba, lane), ex_c = 0, tot_c = 0;
#pragma unroll
        for (int bit = 0; bit < 7; ++bit) {
            const unsigned long long bb = __ballot((cnt >> bit) & 1);
            ex_c += lane_prefix(bb, lane) << bit;
            tot_c += __popcll(bb) << bit;
        }
        if (lane == 0) {
            s_wtot[0][wave] = __popcll(ba);
            s_wtot[1][wave] = tot_c;
        }
        __syncthreads();
        int ta = 0, tc = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int a = s_wtot[0][w], c = s_wtot[1][w];
            if (w < wave) {
                ex_a += a;
                ex_c += c;
            }
            ta += a;
            tc += c;
        }
        ex_a += slot_base;
        ex_c += pair_base;
        if (cnt > 0) {
            slot_eid[ex_a] = e;
            slot_M[ex_a] = cnt;
            slot_off[ex_a] = ex_c;
        }
        if (e < E) eoff[e] = ex_c;
        slot_base += ta;
        pair_base += tc;
        __syncthreads();
    }
    for (int i = tid; i < M * tk; i += NT) {
        const int t = i / tk;
        const int e = eids_s[i];
        int p = -1;
        if (e >= 0 && e < E) {
            p = eoff[e] + __popcll(hitmask[e] & ((1ull << t) - 1ull));
            pair_tok[p] = t;
        }
        pair_of[i] = p;
    }
    if (use_shared)
        for (int t = tid; t < M; t += NT) {
            pair_tok[t] = t;
            pair_shared[t] = t;
        }
    if (use_shared && tid == 0) {
        slot_eid[0] = E;
        slot_M[0] = M;
        slot_off[0] = 0;
    }
    __syncthreads();
    if (tid == 0) {
        meta[META_N_ROUTED] = slot_base - s0;
        meta[META_N_SLOTS] = slot_base;
        meta[META_N_ROUTED_PAIRS] = pair_base - p0;
        meta[META_N_PAIRS] = pair_base;
        meta[META_ERROR] = err | topk_err;
        sticky_or(meta, err | topk_err);
    }
}

constexpr int kRouteThreads = 1024;

// Caller-given routing: eids [M][tk] in global memory.
__global__ __launch_bounds__(kRouteThreads) void bucket_kernel(
    int M, int E, int tk, int use_shared, const int32_t* __restrict__ eids, int* __restrict__ meta,
    int* __restrict__ slot_eid, int* __restrict__ slot_M, int* __restrict__ slot_off, int* __restrict__ pair_tok,
    int* __restrict__ pair_of, int* __restrict__ pair_shared) {
    __shared__ int s_eids[kMaxTokens * kMaxTopK];
    for (int i = threadIdx.x; i < M * tk; i += kRouteThreads) s_eids[i] = eids[i];
    __syncthreads();
    bucket_block<kRouteThreads>(M, E, tk, use_shared, s_eids, 0, meta, slot_eid, slot_M, slot_off, pair_tok,
                                pair_of, pair_shared);
}

// Arguments of the routing step (top-k or hash rows, then bucketing).
struct RouteArgs {
    int M, E, tk, score_func, round_bf16;
    float route_scale;
    const float* scores;  // [M][E] router scores (router_block)
    const float* bias;
    const int32_t* hash;
    const int32_t* ids;
    int vocab, use_shared;
    int32_t* eids;
    float* wts;
    int* meta;
    int* slot_eid;
    int* slot_M;
    int* slot_off;
    int* pair_tok;
    int* pair_of;
    int* pair_shared;
    const int32_t* given;  // caller-given eids [M][tk] (process_expert_ffn): no top-k, no eids/wts written
};

// One workgroup of NT threads: wave w selects the top-k of tokens w, w+NT/64,
// ... (src/fst_engine.cpp:974-1061 semantics with the order of topk_key) or
// reads their hash-table rows (:1015-1021) and writes eids/wts; after one
// barrier the same workgroup groups all tokens' (token, expert) pairs.  PER =
// experts per lane.  gw: write eids/wts (the bucket tables always go to the
// pointers in ra, global or LDS).
template <int PER, int NT, int MAXT = kMaxTokens>
__device__ void topk_bucket_block(const RouteArgs& ra, bool gw = true) {
    const int M = ra.M, E = ra.E, tk = ra.tk;
    const float route_scale = ra.route_scale;
    const float* __restrict__ scores = ra.scores;
    const float* __restrict__ bias = ra.bias;
    const int32_t* __restrict__ hash = ra.hash;
    const int32_t* __restrict__ ids = ra.ids;
    const int vocab = ra.vocab;
    int32_t* __restrict__ eids = ra.eids;
    float* __restrict__ wts = ra.wts;
    constexpr int NW = NT / 64;
    __shared__ int s_eids[MAXT * kMaxTopK];
    __shared__ int s_err;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float zero_score = ra.score_func == 0 ? fst_sigmoidf(0.0f) : fst_sqrtsoftplusf(0.0f);
    if (tid == 0) s_err = 0;
    __syncthreads();
    if (ra.given) {
        for (int i = tid; i < M * tk; i += NT) s_eids[i] = ra.given[i];
        __syncthreads();
        bucket_block<NT, (PER * 64 < kMaxExperts ? PER * 64 : kMaxExperts)>(M, E, tk, ra.use_shared, s_eids, 0, ra.meta,
                         ra.slot_eid, ra.slot_M, ra.slot_off, ra.pair_tok, ra.pair_of, ra.pair_shared);
        return;
    }
    for (int t = wave; t < M; t += NW) {
        const float* row = scores + (size_t)t * E;
        if (hash) {
            if (lane == 0) {
                const int tok = ids ? ids[t] : -1;
                if (tok < 0 || tok >= vocab) {
                    atomicOr(&s_err, 2);
                    for (int k = 0; k < tk; ++k) {
                        s_eids[t * tk + k] = -1;
                        if (gw) {
                            eids[(size_t)t * tk + k] = -1;
                            wts[(size_t)t * tk + k] = 0.0f;
                        }
                    }
                } else {
                    float sc[kMaxTopK];
                    float sum = 0.0f;
                    for (int k = 0; k < tk; ++k) {
                        const int e = hash[(size_t)tok * tk + k];
                        // an out-of-range id scores as a zero logit
                        sc[k] = (e >= 0 && e < E) ? row[e] : zero_score;
                        sum += sc[k];
                        s_eids[t * tk + k] = e;
                        if (gw) eids[(size_t)t * tk + k] = e;
                    }
                    const float inv = 1.0f / (sum + 1e-12f);
                    if (gw)
                        for (int k = 0; k < tk; ++k) wts[(size_t)t * tk + k] = sc[k] * inv * route_scale;
                }
            }
            continue;
        }
        // Exact top-k by extraction in rank order (topk_key: order bits of
        // score+bias descending, then lower id; 1 + order bits here so that
        // 0 marks a retired slot below every live one).  Each lane keeps its
        // experts sorted, so its head is slot 0; each round the wave takes
        // the largest head (DPP + lane swaps), an exact tie going to the
        // lowest id, and that lane retires its head.  Lane r keeps rank r;
        // the weight sum runs in selection order as the reference sums.
        uint32_t key[PER];
        float sc[PER];
        int id[PER];
        {
            float x[PER], bv[PER];
#pragma unroll
            for (int i = 0; i < PER; ++i) x[i] = row[min(lane + 64 * i, E - 1)];
#pragma unroll
            for (int i = 0; i < PER; ++i) bv[i] = bias ? bias[min(lane + 64 * i, E - 1)] : 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int e = lane + 64 * i;
                sc[i] = x[i];
                id[i] = e;
                key[i] = e < E ? (uint32_t)(topk_key(x[i] + bv[i], e) >> 32) + 1u : 0u;
            }
        }
        // stable sort descending by key (ids ascend within a lane)
#pragma unroll
        for (int i = 0; i < PER; ++i)
#pragma unroll
            for (int j = 0; j + 1 < PER - i; ++j)
                if (key[j + 1] > key[j]) {
                    const uint32_t a = key[j];
                    key[j] = key[j + 1];
                    key[j + 1] = a;
                    const float b = sc[j];
                    sc[j] = sc[j + 1];
                    sc[j + 1] = b;
                    const int c = id[j];
                    id[j] = id[j + 1];
                    id[j + 1] = c;
                }
        float wsum = 0.0f, my_sc = 0.0f;
        int my_id = -1;
        for (int r = 0; r < tk; ++r) {
            const uint32_t m = wave_max_u32_all(key[0]);
            const unsigned long long tie = __ballot(key[0] == m);
            int wl = __ffsll((long long)tie) - 1;
            if (__popcll(tie) > 1) wl = (int)(wave_min_u32_all((tie >> lane) & 1ull ? (uint32_t)id[0] : 0xffffffffu) & 63u);
            const float wsc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc[0]), wl));
            const int wid = __builtin_amdgcn_readlane(id[0], wl);
            if (lane == wl) {  // retire the head: shift the list up
#pragma unroll
                for (int i = 0; i + 1 < PER; ++i) {
                    key[i] = key[i + 1];
                    sc[i] = sc[i + 1];
                    id[i] = id[i + 1];
                }
                key[PER - 1] = 0u;
            }
            wsum += wsc;
            if (lane == r) {
                my_id = wid;
                my_sc = wsc;
            }
        }
        if (lane < tk) {
            const float inv = 1.0f / (wsum + 1e-12f);
            s_eids[t * tk + lane] = my_id;
            if (gw) {
                eids[(size_t)t * tk + lane] = my_id;
                wts[(size_t)t * tk + lane] = my_sc * inv * route_scale;
            }
        }
    }
    __syncthreads();
    bucket_block<NT, (PER * 64 < kMaxExperts ? PER * 64 : kMaxExperts)>(M, E, tk, ra.use_shared, s_eids, s_err, ra.meta, ra.slot_eid, ra.slot_M, ra.slot_off,
                     ra.pair_tok, ra.pair_of, ra.pair_shared);
}

template <int PER>
__global__ __launch_bounds__(kRouteThreads) void topk_bucket_kernel(RouteArgs ra) {
    topk_bucket_block<PER, kRouteThreads>(ra);
}

static RouteArgs route_args(const Geometry& g, const LayerView& L, int M, const float* logits,
                            const int32_t* input_ids, int use_hash, int use_shared, int32_t* eids, float* wts,
                            const Scratch& s) {
    return RouteArgs{M,          g.E,         g.tk,       g.score_func,
                     g.round_logits_bf16, g.route_scale, logits, L.router_bias,
                     use_hash ? L.hash : nullptr, input_ids, g.vocab, use_shared,
                     eids,       wts,         s.meta,     s.slot_eid,
                     s.slot_M,   s.slot_off,  s.pair_tok, s.pair_of,
                     s.pair_shared, nullptr};
}

void launch_bucket(hipStream_t st, const Geometry& g, int M, int use_shared, const int32_t* eids,
                   const Scratch& s) {
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(kRouteThreads), 0, st, M, g.E, g.tk, use_shared, eids, s.meta,
                       s.slot_eid, s.slot_M, s.slot_off, s.pair_tok, s.pair_of, s.pair_shared);
}


// -------------------------------------------------------------- operand prep

// Element sources for the prep kernel: bf16 activations, or the fp32
// h = silu(gate)*up rows written by the gate/up kernel.
// (kVec: elements per 16-byte vector load; vec() loads vector q of a row,
// unpack() widens it to floats)
struct SrcBf16 {
    static constexpr int kVec = 8;
    const uint16_t* p;
    __device__ __forceinline__ float at(size_t row, int K, int i) const {
        return fst_bf16_to_f32(p[row * K + i]);
    }
    __device__ __forceinline__ uint4 vec(size_t row, int K, int q) const {
        return reinterpret_cast<const uint4*>(p + row * K)[q];
    }
    __device__ __forceinline__ void unpack(const uint4& v, float* f) const {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = fst_bits_f32(w[i] << 16);
            f[2 * i + 1] = fst_bits_f32(w[i] & 0xffff0000u);
        }
    }
};
struct SrcF32 {
    static constexpr int kVec = 4;
    const float* p;
    __device__ __forceinline__ float at(size_t row, int K, int i) const { return p[row * K + i]; }
    __device__ __forceinline__ uint4 vec(size_t row, int K, int q) const {
        return reinterpret_cast<const uint4*>(p + row * K)[q];
    }
    __device__ __forceinline__ void unpack(const uint4& v, float* f) const {
        f[0] = fst_bits_f32(v.x);
        f[1] = fst_bits_f32(v.y);
        f[2] = fst_bits_f32(v.z);
        f[3] = fst_bits_f32(v.w);
    }
};
// h = silu(gate) * up from the split-K partials of the gate||up launch:
// part[ks][row][2*inter] (gate in [0, inter), up in [inter, 2*inter)), the S
// partials added in ks order, then the same SwiGLU (and clamp) as the
// unsplit launch's epilogue.
template <int S>
struct SrcSplit {
    static constexpr int kVec = 4;
    const float* part;
    int rows, inter;
    float lim;
    __device__ __forceinline__ float4 ld(int ks, size_t row, int off) const {
        return *reinterpret_cast<const float4*>(part + ((size_t)ks * rows + row) * (2 * inter) + off);
    }
    __device__ __forceinline__ uint4 vec(size_t row, int, int q) const {
        // all 2S loads issued before the sums
        float4 g[S], u[S];
#pragma unroll
        for (int ks = 0; ks < S; ++ks) {
            g[ks] = ld(ks, row, 4 * q);
            u[ks] = ld(ks, row, inter + 4 * q);
        }
        float4 gs = g[0], us = u[0];
#pragma unroll
        for (int ks = 1; ks < S; ++ks) {
            gs.x += g[ks].x; gs.y += g[ks].y; gs.z += g[ks].z; gs.w += g[ks].w;
            us.x += u[ks].x; us.y += u[ks].y; us.z += u[ks].z; us.w += u[ks].w;
        }
        const float gv[4] = {gs.x, gs.y, gs.z, gs.w}, uv[4] = {us.x, us.y, us.z, us.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float a = gv[e], b = uv[e];
            if (lim > 0.0f) {
                a = fminf(a, lim);
                b = fminf(fmaxf(b, -lim), lim);
            }
            o[e] = fst_f32_bits((a / (1.0f + expf(-a))) * b);
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
    }
    __device__ __forceinline__ void unpack(const uint4& v, float* f) const {
        f[0] = fst_bits_f32(v.x);
        f[1] = fst_bits_f32(v.y);
        f[2] = fst_bits_f32(v.z);
        f[3] = fst_bits_f32(v.w);
    }
};
constexpr int kMaxPrepK = 8192;

// One row by one workgroup of NT threads (xv: K floats of LDS): amax ->
// exponent s so that amax*2^-s lies in [2^9, 2^10); then the k-interleaved
// fp16 operand (per super-block, lane group g, MFMA c: elements
// 64g+4c+{0,2,1,3} and 64g+32+4c+{0,2,1,3}, the order q4k_bop produces the
// weights in) and the per-sub-block sums split hi+lo.
template <int NT, typename Src>
__device__ void prep_row(const Src& src, int row, int K, float* xv, _Float16* __restrict__ x16p,
                         uint4* __restrict__ sxp, int* __restrict__ xs) {
    __shared__ float red[NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float m = 0.0f;
    if constexpr (Src::kVec > 0) {
        // 16-byte loads, each thread's batch issued before any is used
        constexpr int VE = Src::kVec, NB = 4;
        const int nv = K / VE;
        for (int q0 = tid; q0 < nv; q0 += NB * NT) {
            uint4 v[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) v[u] = src.vec(row, K, min(q0 + u * NT, nv - 1));
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int q = q0 + u * NT;
                if (q < nv) {
                    float f[VE];
                    src.unpack(v[u], f);
#pragma unroll
                    for (int e = 0; e < VE; ++e) {
                        xv[q * VE + e] = f[e];
                        m = fmaxf(m, fabsf(f[e]));
                    }
                }
            }
        }
    } else {
        for (int i = tid; i < K; i += NT) {
            const float v = src.at(row, K, i);
            xv[i] = v;
            m = fmaxf(m, fabsf(v));
        }
    }
    m = wave_fmax(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float a = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) a = fmaxf(a, red[w]);
    const int s = prescale_exp(a);
    if (tid == 0) xs[row] = s;
    // One pass over the operand chunks: chunk q = 32 sb + 8g + c holds the
    // fp16 values (exact power-of-two scaling, one rounding) of elements
    // 64g+4c+{0,2,1,3} and 64g+32+4c+{0,2,1,3} of super-block sb; the 8
    // lanes of one (sb, g) then reduce the two sub-block sums (hi+lo split).
    // K/8 is a multiple of 8, so each 8-lane group runs the same iterations.
    _Float16* dst = x16p + (size_t)row * K;
    uint4* sx = sxp + (size_t)row * (K / 256) * 4;
    for (int q = tid; q < K / 8; q += NT) {
        const int sb = q >> 5, g = (q >> 3) & 3, c = q & 7;
        const int base = sb * 256 + 64 * g + 4 * c;
        const float4 lo4 = *reinterpret_cast<const float4*>(xv + base);
        const float4 hi4 = *reinterpret_cast<const float4*>(xv + base + 32);
        h8_t v;
        v[0] = (_Float16)ldexpf(lo4.x, -s);
        v[1] = (_Float16)ldexpf(lo4.z, -s);
        v[2] = (_Float16)ldexpf(lo4.y, -s);
        v[3] = (_Float16)ldexpf(lo4.w, -s);
        v[4] = (_Float16)ldexpf(hi4.x, -s);
        v[5] = (_Float16)ldexpf(hi4.z, -s);
        v[6] = (_Float16)ldexpf(hi4.y, -s);
        v[7] = (_Float16)ldexpf(hi4.w, -s);
        *reinterpret_cast<h8_t*>(dst + (size_t)q * 8) = v;
        float s0 = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
        float s1 = ((float)v[4] + (float)v[5]) + ((float)v[6] + (float)v[7]);
        // butterfly over the 8 lanes of the group; lane c == 0 holds
        // ((l0 + l1) + (l2 + l3)) + ((l4 + l5) + (l6 + l7))
        s0 = s0 + fdpp<0xb1>(s0);  // quad_perm [1,0,3,2]
        s1 = s1 + fdpp<0xb1>(s1);
        s0 = s0 + fdpp<0x4e>(s0);  // quad_perm [2,3,0,1]
        s1 = s1 + fdpp<0x4e>(s1);
        s0 = s0 + fdpp<0x104>(s0);  // row_shl 4
        s1 = s1 + fdpp<0x104>(s1);
        if (c == 0) {
            const _Float16 h0 = (_Float16)s0, h1 = (_Float16)s1;
            const _Float16 l0 = (_Float16)(s0 - (float)h0), l1 = (_Float16)(s1 - (float)h1);
            const _Float16 z = (_Float16)0.0f;
            *reinterpret_cast<h8_t*>(sx + sb * 4 + g) = h8_t{h0, h1, l0, l1, z, z, z, z};
        }
    }
    __syncthreads();
}

template <typename Src>
__global__ __launch_bounds__(256) void prep_kernel(Src src, const int* __restrict__ nrows_dev, int nrows_host,
                                                   int K, _Float16* __restrict__ x16p,
                                                   uint4* __restrict__ sxp, int* __restrict__ xs,
                                                   const uint4* __restrict__ pf, size_t pf_pieces) {
    const int row = blockIdx.x;
    if (row >= nrows_host) {
        // workgroups past the rows read pf (the weights the next launch
        // streams first) into the device-wide cache while this latency-bound
        // launch leaves HBM idle; the loads land in a scratch LDS line
        __shared__ __attribute__((aligned(16))) uint4 pf_lds[64];
        const size_t step = (size_t)(gridDim.x - nrows_host) * 256;
        for (size_t q = (size_t)(row - nrows_host) * 256 + threadIdx.x; q < pf_pieces; q += step)
            __builtin_amdgcn_global_load_lds((const void*)(pf + q), (__attribute__((address_space(3))) void*)pf_lds,
                                             16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }
    const int nrows = nrows_dev ? nrows_dev[0] : nrows_host;
    if (row >= nrows) return;
    __shared__ float xv[kMaxPrepK];
    prep_row<256>(src, row, K, xv, x16p, sxp, xs);
}

// Caller-given routing (process_expert_ffn): workgroup 0 buckets the eids
// (bucket_block), workgroups 1..M prepare each token row's fp16 operand
// (Q4_K only), in one launch.  When the down launch writes the result
// itself (o1/o2 given: one routed pair per token, no shared expert),
// workgroup 0 also zeroes the output rows of tokens whose expert id is
// invalid, which the combine would have written as zeros.
__global__ __launch_bounds__(kRouteThreads) void bucket_prep_kernel(
    int M, int E, int tk, int use_shared, const int32_t* __restrict__ eids, Scratch s, const uint16_t* h, int K,
    uint16_t* o1, uint16_t* o2, int hd, int nprep, const uint4* __restrict__ pf, size_t pf_pieces, int bucket) {
    // the fused launch that may follow claims work from this counter
    if (blockIdx.x == 0 && threadIdx.x == 0) *s.fused_claim = 0;
    if ((int)blockIdx.x > nprep) {
        // workgroups past the prep rows read pf (the shared expert's gate||up
        // weights, streamed first by the next launch) into the device-wide
        // cache while this latency-bound launch leaves HBM idle
        __shared__ __attribute__((aligned(16))) uint4 pf_lds[64];
        const size_t step = (size_t)(gridDim.x - 1 - nprep) * kRouteThreads;
        for (size_t q = (size_t)(blockIdx.x - 1 - nprep) * kRouteThreads + threadIdx.x; q < pf_pieces; q += step)
            __builtin_amdgcn_global_load_lds((const void*)(pf + q), (__attribute__((address_space(3))) void*)pf_lds,
                                             16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }
    if (blockIdx.x > 0) {
        __shared__ float xv[kMaxPrepK];
        prep_row<kRouteThreads>(SrcBf16{h}, blockIdx.x - 1, K, xv, s.x16p, s.sxp, s.xs);
        return;
    }
    if (!bucket) return;
    __shared__ int s_eids[kMaxTokens * kMaxTopK];
    for (int i = threadIdx.x; i < M * tk; i += kRouteThreads) s_eids[i] = eids[i];
    __syncthreads();
    bucket_block<kRouteThreads>(M, E, tk, use_shared, s_eids, 0, s.meta, s.slot_eid, s.slot_M, s.slot_off,
                                s.pair_tok, s.pair_of, s.pair_shared);
    if (o1 || o2)
        for (int i = threadIdx.x; i < M * (hd / 8); i += kRouteThreads) {
            const int t = i / (hd / 8), q = i - t * (hd / 8);
            const int e = s_eids[t * tk];
            if (e >= 0 && e < E) continue;
            const uint4 z = make_uint4(0u, 0u, 0u, 0u);
            if (o1) reinterpret_cast<uint4*>(o1 + (size_t)t * hd)[q] = z;
            if (o2) reinterpret_cast<uint4*>(o2 + (size_t)t * hd)[q] = z;
        }
}

void launch_bucket_prep(hipStream_t st, const Geometry& g, int M, int use_shared, const int32_t* eids,
                        const Scratch& s, const uint16_t* h, uint16_t* o1, uint16_t* o2, const void* pf,
                        size_t pf_bytes, bool bucket) {
    const int nprep = h ? M : 0;
    const int extra = pf ? 32 : 0;  // 1024-thread prefetch workgroups
    hipLaunchKernelGGL(bucket_prep_kernel, dim3(1 + nprep + extra), dim3(kRouteThreads), 0, st, M, g.E, g.tk,
                       use_shared, eids, s, h, g.hd, o1, o2, g.hd, nprep, static_cast<const uint4*>(pf),
                       pf_bytes / 16, bucket ? 1 : 0);
}

// Router logits (workgroups [0, nrb), router_block) and the fp16 expert
// operand of each token row (workgroups [nrb, nrb + nprep), prep_row; Q4_K
// only) in one launch.  The top-k and bucketing of the call follow in the
// gate||up launch's prologue (the fused launch, or the chain's gate||up launch:
// every workgroup routes the call into LDS), or in topk_bucket_kernel when the
// layer has more experts than that prologue handles.  (A single launch whose last router
// workgroup runs the top-k was measured slower: the hand-off through
// device-coherent stores and a contended completion counter costs more than
// the kernel boundary.)
template <int NV, int TPW>
__global__ __launch_bounds__(256) void router_prep_kernel(const uint4* __restrict__ w_il,
                                                          const uint16_t* __restrict__ h, int M, int K, int E,
                                                          int score_func, int round_bf16,
                                                          float* __restrict__ scores, int nbx, int nrb,
                                                          _Float16* __restrict__ x16p, uint4* __restrict__ sxp,
                                                          int* __restrict__ xs, int* __restrict__ zero_word) {
    static_assert(TPW >= 2, "the router stage must also hold a prep row (K floats)");
    // the fused launch that follows claims work from this counter
    if (zero_word && blockIdx.x == 0 && threadIdx.x == 0) *zero_word = 0;
    __shared__ uint4 sm[TPW * NV * 65];
    const int b = blockIdx.x;
    if (b >= nrb) {
        prep_row<256>(SrcBf16{h}, b - nrb, K, reinterpret_cast<float*>(sm), x16p, sxp, xs);
        return;
    }
    router_block<NV, TPW>(w_il, h, M, E, b % nbx, b / nbx, score_func, round_bf16, scores, sm);
}

void launch_route(hipStream_t st, const Geometry& g, const LayerView& L, const uint16_t* h, int M, int prep,
                  const int32_t* input_ids, int use_hash, int use_shared, int32_t* eids, float* wts,
                  const Scratch& s, int topk) {
#ifndef FST_RTPW
#define FST_RTPW 2
#endif
    constexpr int TPW = FST_RTPW;  // tokens per router wave
    const int nbx = (g.E + 3) / 4, nby = (M + TPW - 1) / TPW, nrb = nbx * nby;
    const dim3 grid(nrb + (prep ? M : 0));
#define FST_RP(NVV)                                                                                        \
    case NVV:                                                                                              \
        hipLaunchKernelGGL((router_prep_kernel<NVV, TPW>), grid, dim3(256), 0, st,                         \
                           reinterpret_cast<const uint4*>(L.router_nk), h, M, g.hd, g.E, g.score_func,     \
                           g.round_logits_bf16, s.logits, nbx, nrb, s.x16p, s.sxp, s.xs, s.fused_claim);    \
        break
    // hidden_dim is a multiple of 512 in [512, 8192] (checked at context creation)
    switch (g.hd / 512) {
        FST_RP(1); FST_RP(2); FST_RP(3); FST_RP(4); FST_RP(5); FST_RP(6); FST_RP(7); FST_RP(8);
        FST_RP(9); FST_RP(10); FST_RP(11); FST_RP(12); FST_RP(13); FST_RP(14); FST_RP(15); FST_RP(16);
        default: break;
    }
#undef FST_RP
    if (!topk) return;
    const RouteArgs ra = route_args(g, L, M, s.logits, input_ids, use_hash, use_shared, eids, wts, s);
    const int per = (g.E + 63) / 64;
#define FST_TOPK(PERV) hipLaunchKernelGGL(topk_bucket_kernel<PERV>, dim3(1), dim3(kRouteThreads), 0, st, ra)
    if (per <= 1)
        FST_TOPK(1);
    else if (per <= 2)
        FST_TOPK(2);
    else if (per <= 4)
        FST_TOPK(4);
    else if (per <= 8)
        FST_TOPK(8);
    else
        FST_TOPK(16);
#undef FST_TOPK
}

void launch_prep_bf16(hipStream_t st, const uint16_t* x, int rows, int K, _Float16* x16p, uint4* sxp,
                      int* xs) {
    hipLaunchKernelGGL(prep_kernel<SrcBf16>, dim3(rows), dim3(256), 0, st, SrcBf16{x}, nullptr, rows, K,
                       x16p, sxp, xs, nullptr, (size_t)0);
}
// ---------------------------------------------------- residual + RMSNorm

// Element source reading a row already held in LDS.
struct SrcRow {
    static constexpr int kVec = 0;  // already in LDS: element loads
    const float* p;
    __device__ __forceinline__ float at(size_t, int, int i) const { return p[i]; }
};

// One workgroup per token row (process_layer's non-HC residual and norm,
// src/fst_engine.cpp:2913-2917 and :2738-2741; rms_cpu :89-90):
//   x   = y ? bf16(h + y) : h          (the previous sublayer's residual add)
//   ss  = sum_j x_j^2 in double, canonical order: lane p of 64 sums the
//         contiguous chunk p sequentially, then p[j] += p[j+off], off = 32..1
//   r   = (float)(1 / sqrt(ss/d + eps))
//   out = bf16((x * r) * w)            (fp32 products, no contraction, RNE)
// x is written back to h_out (when given); out goes to normed (when given)
// and, when x16p is given, straight into the linear kernel's fp16 operand
// (prep_row).  Block 0 also writes a one-slot table for a dense linear call
// over the M rows (when slot_tab is given: meta, slot_eid, slot_M, slot_off).
#pragma clang fp contract(off)
__global__ __launch_bounds__(256) void resid_norm_kernel(const uint16_t* __restrict__ h,
                                                         const uint16_t* __restrict__ y,
                                                         const uint16_t* __restrict__ w, int M, int d,
                                                         float eps, uint16_t* __restrict__ h_out,
                                                         uint16_t* __restrict__ normed, _Float16* __restrict__ x16p,
                                                         uint4* __restrict__ sxp, int* __restrict__ xs,
                                                         int* __restrict__ slot_tab) {
    // x in LDS with one pad word per 64 (xi): lane p's sequential pass over
    // its contiguous chunk then reads 64 different banks at each step, not one
    __shared__ float xrow[kMaxPrepK + kMaxPrepK / 64];
    __shared__ float nrow[kMaxPrepK];
    __shared__ float s_r;
    const int t = blockIdx.x, tid = threadIdx.x;
    auto xi = [](int e) { return e + (e >> 6); };
    if (slot_tab && t == 0 && tid == 0) {
        slot_tab[META_N_SLOTS] = 1;
        slot_tab[META_WORDS + 0] = 0;  // slot_eid
        slot_tab[META_WORDS + 1] = M;  // slot_M
        slot_tab[META_WORDS + 2] = 0;  // slot_off
    }
    // 8 elements per 16-byte load (d is a multiple of 512, at most 8192: at
    // most NB loads of each row per thread); every load, the norm weights
    // included, is issued before any is used
    const int nv = d / 8;
    constexpr int NB = 4;
    uint4 hv[NB], yv[NB], wv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int q = min(tid + u * 256, nv - 1);
        hv[u] = reinterpret_cast<const uint4*>(h + (size_t)t * d)[q];
        yv[u] = y ? reinterpret_cast<const uint4*>(y + (size_t)t * d)[q] : make_uint4(0u, 0u, 0u, 0u);
        wv[u] = reinterpret_cast<const uint4*>(w)[q];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int q = tid + u * 256;
        if (q >= nv) continue;
        const uint32_t hw[4] = {hv[u].x, hv[u].y, hv[u].z, hv[u].w};
        const uint32_t yw[4] = {yv[u].x, yv[u].y, yv[u].z, yv[u].w};
        uint32_t ow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t o2 = 0u;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float x = fst_bf16_to_f32((uint16_t)(hw[i] >> (16 * hh)));
                if (y) x = fst_bf16_to_f32(fst_f32_to_bf16(x + fst_bf16_to_f32((uint16_t)(yw[i] >> (16 * hh)))));
                xrow[xi(8 * q + 2 * i + hh)] = x;
                o2 |= (uint32_t)fst_f32_to_bf16(x) << (16 * hh);
            }
            ow[i] = o2;
        }
        if (h_out) reinterpret_cast<uint4*>(h_out + (size_t)t * d)[q] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
    __syncthreads();
    if (tid < 64) {
        const int C = d / 64;
        double a = 0.0;
#pragma unroll 8
        for (int i = 0; i < C; ++i) {
            const double v = (double)xrow[xi(tid * C + i)];
            a = a + v * v;
        }
        // halving tree p[j] += p[j+off], off = 32..1: lane j < off adds
        // lane j+off's partial (the upper lanes' values are not used again)
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) a = a + __shfl_down(a, off, 64);
        if (tid == 0) s_r = (float)(1.0 / sqrt(a / (double)d + (double)eps));
    }
    __syncthreads();
    const float r = s_r;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int q = tid + u * 256;
        if (q >= nv) continue;
        const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
        uint32_t ow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t o2 = 0u;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int j = 8 * q + 2 * i + hh;
                const uint16_t o = fst_f32_to_bf16((xrow[xi(j)] * r) * fst_bf16_to_f32((uint16_t)(ww[i] >> (16 * hh))));
                nrow[j] = fst_bf16_to_f32(o);
                o2 |= (uint32_t)o << (16 * hh);
            }
            ow[i] = o2;
        }
        if (normed) reinterpret_cast<uint4*>(normed + (size_t)t * d)[q] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
    __syncthreads();
    if (x16p) prep_row<256>(SrcRow{nrow}, t, d, xrow, x16p, sxp, xs);
}
#pragma clang fp contract(on)

void launch_resid_norm(hipStream_t st, const uint16_t* h, const uint16_t* y, const uint16_t* w, int M, int d,
                       float eps, uint16_t* h_out, uint16_t* normed, const Scratch* prep, int* slot_tab) {
    hipLaunchKernelGGL(resid_norm_kernel, dim3(M), dim3(256), 0, st, h, y, w, M, d, eps, h_out, normed,
                       prep ? prep->x16p : nullptr, prep ? prep->sxp : nullptr, prep ? prep->xs : nullptr,
                       slot_tab);
}

// prefetch workgroups added to a prep launch (when pf is given)
constexpr int kPrepPrefetchWGs = 128;

void launch_prep_act(hipStream_t st, const float* h, const int* meta, int max_rows, int K, _Float16* a16p,
                     uint4* sxp, int* xs, const void* pf, size_t pf_bytes) {
    const int extra = pf ? kPrepPrefetchWGs : 0;
    hipLaunchKernelGGL(prep_kernel<SrcF32>, dim3(max_rows + extra), dim3(256), 0, st, SrcF32{h},
                       meta + META_N_PAIRS, max_rows, K, a16p, sxp, xs, static_cast<const uint4*>(pf), pf_bytes / 16);
}

void launch_prep_act_split(hipStream_t st, const float* part, int S, int rows, float swiglu_limit, const int* meta,
                           int inter, _Float16* a16p, uint4* sxp, int* xs, const void* pf, size_t pf_bytes) {
    const int extra = pf ? kPrepPrefetchWGs : 0;
#define FST_PS(SV)                                                                                          \
    hipLaunchKernelGGL(prep_kernel<SrcSplit<SV>>, dim3(rows + extra), dim3(256), 0, st,                     \
                       SrcSplit<SV>{part, rows, inter, swiglu_limit}, meta + META_N_PAIRS, rows, inter, a16p, sxp, \
                       xs, static_cast<const uint4*>(pf), pf_bytes / 16)
    if (S <= 2)
        FST_PS(2);
    else if (S <= 4)
        FST_PS(4);
    else
        FST_PS(8);
#undef FST_PS
}

// ------------------------------------------------------- Q4_K linear kernel

// MXFP4 chunk (fst_layout.cpp): 2176 bytes = [0,1024) block 2g of row r at
// lane slot 16g+r, [1024,2048) block 2g+1, [2048,2176) the 8 scale bytes of
// each row (h.x, h.y of the lane's row).
__device__ __forceinline__ WRaw load_wraw_mx(const uint8_t* chunk, int lane) {
    WRaw w;
    w.a = ld_stream(chunk + 16 * lane);
    w.b = ld_stream(chunk + 1024 + 16 * lane);
    typedef uint32_t u2v_t __attribute__((ext_vector_type(2)));
    const u2v_t hv = __builtin_nontemporal_load(reinterpret_cast<const u2v_t*>(chunk + 2048 + 8 * (lane & 15)));
    w.h = u4v_t{hv.x, hv.y, 0u, 0u};
    return w;
}

// e8m0 block scale as float: 2^(e-127); the reference kernel maps e = 0 and
// e = 255 to 0 (kernels/fst_dequant_v4_vectorized_kernel.cc:19-37,60-80).
__device__ __forceinline__ float e8m0_scale(uint32_t e) {
    return (e == 0u || e == 255u) ? 0.0f : __uint_as_float(e << 23);
}

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));

// LDS activation stage: per token 36 uint4 (32 operand chunks, 4 min-term
// chunks; MXFP4 uses the 32 operand chunks only), padded to kTokStride.
constexpr int kTokStride = 37;

// Y[pair][row] = 2^xs[a] * sum_k W[row][k] * A[a][k] for the rows of one
// Q4_K matrix (N rows x K/256 super-blocks per row) of the slot's expert.
// Grid: max_slots * N/64 workgroups of 4 waves; wave w of tile T owns rows
// T*64 + 16w .. +15 and all tokens of its slot.  Weights stream through
// registers two super-blocks ahead (ping-pong pair, loop unrolled by two);
// the slot's activation operands are staged per super-block in a
// double-buffered LDS ring shared by the 4 waves.
#ifndef FST_Q4K_WAVES_PER_EU
#define FST_Q4K_WAVES_PER_EU 4
#endif
#ifndef FST_Q4K_WPE_MID
#define FST_Q4K_WPE_MID 4
#endif
#ifndef FST_MF32_WPE
#define FST_MF32_WPE 2
#endif
#ifndef FST_MF32_PF
#define FST_MF32_PF 1
#endif
// What a linear-kernel launch does besides Y = W.A (mode 1, gate||up:
// workgroup tile T holds gate rows [64T, 64T+64) in waves 0..3 and the
// matching up rows in waves 4..7; it writes h = silu(gate) * up for its 64
// rows, fp32 for Q4_K, bf16 for MXFP4 (the down operand as is)).
struct EpiArgs {
    float swiglu_limit;
    float* h;
    uint16_t* h16;
    // mode 2 with one routed pair per token and no shared expert: write
    // out = bf16(w[token] * y) to o1/o2 (either may be null) instead of y
    const float* wts;
    const int* pair_tok;
    uint16_t* o1;
    uint16_t* o2;
    // mode 1 split-K: S > 1 items per (slot, tile), partial sums written to
    // part[ks][pair][N] (part_rows pairs per split) instead of h
    int ksplit;
    float* part;
    int part_rows;
};

#ifndef FST_Q4K_PF
#define FST_Q4K_PF 1
#endif
#ifndef FST_WNT
#define FST_WNT 2
#endif
#ifndef FST_SHARED_PREFETCH
#define FST_SHARED_PREFETCH 1
#endif
#ifndef FST_SKIP_DEAD_SLOTS
#define FST_SKIP_DEAD_SLOTS 1
#endif
#ifndef FST_UNROLL_X
#define FST_UNROLL_X 1
#endif
// Y[pair][row] = 2^xs[a] * sum_k W[row][k] * A[a][k] for the rows of one
// Q4_K matrix (N rows x K/256 super-blocks per row) of each slot's expert.
// Work item t = (slot, tile) covers 16*WAVES rows: wave w owns 16 rows and up
// to TOKS tokens of the slot.  The grid is persistent (a few workgroups per
// CU) and walks t = blockIdx.x, +gridDim.x, ...; the first weights of the
// next item are fetched while the current one finishes.
//  - weights stream through a ring of PF+1 register sets (PF super-blocks
//    ahead), the ring unrolled so each set keeps fixed registers;
//  - the slot's activation operands are staged into LDS in macro-stages of MS
//    super-blocks (double-buffered, prefetched one macro-stage ahead into
//    registers), one workgroup barrier per macro-stage.
//  - RPER > 0 (gate||up only): the launch routes the call itself first
//    (topk_bucket_block over ra.scores with RPER experts per lane) into LDS
//    tables, which then replace meta/slot_*/a_row; workgroup 0 also writes
//    eids/wts and the tables to the global arrays of ra for later launches.
// MF (mode 0, Q4_K, 17..32 tokens): each wave owns 32 rows (two 16-row
// tiles) and computes with v_mfma_f32_32x32x16_f16: one 16-byte LDS read per
// lane feeds 32 rows x 16 k x 32 tokens, half the operand reads per weight of
// two 16x16x32 token groups.  Lane (n = lane % 32, h = lane / 32) takes row n
// and bytes [64h, 64h+64) of its nibbles (sub-blocks 4h..4h+3); MFMA j of a
// super-block uses nibble dword j of that range, whose weights are the
// elements of operand chunk 16h + j (the layout prep_row writes), so the
// staged operand is read as it is.
template <int TOKS, int MS, int WAVES, int MODE, int CODEC = 0, int RPER = 0, int PF = FST_Q4K_PF, bool MF = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(MF ? FST_MF32_WPE : (TOKS <= 8 ? FST_Q4K_WAVES_PER_EU : (TOKS <= 32 ? FST_Q4K_WPE_MID : 2))))) void q4k_linear_kernel(
    const uint8_t* __restrict__ bank, size_t expert_stride, size_t mat_offset, int K, int N,
    const int* meta_g, const int* slot_eid_g, const int* slot_M_g,
    const int* slot_off_g, const int* a_row_g, const _Float16* __restrict__ A,
    const uint4* __restrict__ SX, const int* __restrict__ xs, float* __restrict__ out, EpiArgs ep, RouteArgs ra) {
    static_assert(MODE != 1 || WAVES % 2 == 0, "gate||up pairs waves");
    static_assert(!MF || (MODE == 0 && CODEC == 0 && TOKS == 32), "32x32 tiles: mode 0, Q4_K, 32 tokens");
    constexpr int WROWS = MF ? 32 : 16;              // rows per wave
    constexpr bool MX = CODEC == 1;                  // MXFP4 weights, bf16 operand, bf16 MFMA
    constexpr int CHUNK = MX ? 2176 : 2304;          // bytes per (16 rows x 256 weights)
    constexpr int PARTS = MX ? 32 : 36;              // staged 16-byte chunks per token per super-block
    constexpr int NGRP = (TOKS + 15) / 16;
    constexpr int TS = TOKS * kTokStride;            // one super-block of one stage
    constexpr int STAGE = MS * TS;                   // one macro-stage
    constexpr int NT = 64 * WAVES;                   // threads per workgroup
    constexpr int NCH = MS * TOKS * PARTS;           // 16-byte chunks per macro-stage
    constexpr int NS = (NCH + NT - 1) / NT;          // staged chunks per thread
    constexpr int HALF = WAVES / 2;
    constexpr int R = PF + 1;                        // weight register ring
    constexpr int U = FST_UNROLL_X * ((MS % R == 0) ? MS : (R % MS == 0 ? R : MS * R));  // lcm(MS, R)
    static_assert(U % MS == 0 && U % R == 0, "unroll must cover whole stages and ring turns");
    __shared__ uint4 lds[2 * STAGE];

    // in-launch routing tables (one int each when unused)
    constexpr int RPAIR = RPER > 0 ? TOKS * kMaxTopK : 1;  // routed pairs (M <= TOKS)
    constexpr int RTOK = RPER > 0 ? TOKS : 1;
    __shared__ int r_meta[META_WORDS], r_seid[RPAIR + 1], r_sM[RPAIR + 1], r_soff[RPAIR + 1];
    __shared__ int r_ptok[RPAIR + RTOK], r_pof[RPAIR], r_psh[RTOK];
    if constexpr (RPER > 0) {
        static_assert(MODE == 1, "in-launch routing is the gate||up launch's");
        RouteArgs la = ra;
        la.meta = r_meta;
        la.slot_eid = r_seid;
        la.slot_M = r_sM;
        la.slot_off = r_soff;
        la.pair_tok = r_ptok;
        la.pair_of = r_pof;
        la.pair_shared = r_psh;
#if FST_SHARED_PREFETCH
        // The shared expert (slot 0, bank index E) is the one expert known
        // before routing: every workgroup reads its slice of the shared
        // gate||up weights while it routes, so that stream overlaps the
        // routing instead of following it, and the shared-expert items later
        // find the lines in the device-wide cache.  The values are discarded.
        uint4 pfv[3];
        const int npf = ra.use_shared ? 3 : 0;
        {
            const size_t pieces = (size_t)(N / 16) * (K >> 8) * (CHUNK / 16);  // 16-byte pieces of gate||up
            const uint4* src = reinterpret_cast<const uint4*>(bank + (size_t)ra.E * expert_stride + mat_offset);
            const size_t step = (size_t)gridDim.x * (64 * WAVES);
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const size_t q = (size_t)blockIdx.x * (64 * WAVES) + threadIdx.x + i * step;
                pfv[i] = i < npf ? src[q < pieces ? q : 0] : make_uint4(0u, 0u, 0u, 0u);
            }
        }
#endif
        topk_bucket_block<RPER, 64 * WAVES, TOKS>(la, blockIdx.x == 0);
#if FST_SHARED_PREFETCH
#pragma unroll
        for (int i = 0; i < 3; ++i) asm volatile("" ::"v"(pfv[i].x));
#endif
        __syncthreads();
        if (blockIdx.x == 0) {
            const int ns = r_meta[META_N_SLOTS], np = r_meta[META_N_PAIRS];
            const int t = threadIdx.x;
            if (t <= META_N_ROUTED_PAIRS) ra.meta[t] = r_meta[t];
            if (t == 0) sticky_or(ra.meta, r_meta[META_ERROR]);
            for (int i = t; i < ns; i += 64 * WAVES) {
                ra.slot_eid[i] = r_seid[i];
                ra.slot_M[i] = r_sM[i];
                ra.slot_off[i] = r_soff[i];
            }
            for (int i = t; i < np; i += 64 * WAVES) ra.pair_tok[i] = r_ptok[i];
            for (int i = t; i < ra.M * ra.tk; i += 64 * WAVES) ra.pair_of[i] = r_pof[i];
            if (ra.use_shared)
                for (int i = t; i < ra.M; i += 64 * WAVES) ra.pair_shared[i] = r_psh[i];
        }
    }
    const int* meta = RPER > 0 ? r_meta : meta_g;
    const int* slot_eid = RPER > 0 ? r_seid : slot_eid_g;
    const int* slot_M = RPER > 0 ? r_sM : slot_M_g;
    const int* slot_off = RPER > 0 ? r_soff : slot_off_g;
    const int* a_row = RPER > 0 ? r_ptok : a_row_g;

    // split-K (gate||up of calls with few slots, ep.ksplit > 1): work item
    // t = ((slot * tiles) + tile) * S + ks covers super-blocks [ks*nsb,
    // (ks+1)*nsb) of the rows and writes partial sums
    const int S = MODE == 1 ? max(ep.ksplit, 1) : 1;
    const int tiles = N / (WROWS * WAVES);
    const int total = meta[META_N_SLOTS] * tiles * S;
    if ((int)blockIdx.x >= total) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    const int nsb_row = K >> 8;      // super-blocks per row
    const int nsb = nsb_row / S;     // super-blocks per work item
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    const f4_t zf = f4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t magic = 0x64006400u;
    const uint32_t ssel = q4k_scale_sel(g);

    // 16-row tile of the matrix owned by this wave in work item tt; MODE 1
    // pairs gate rows [64T, 64T+64) (waves 0..3) with the same up rows
    auto wave_tile = [&](int tile) -> int {
        if constexpr (MODE == 1)
            return wave < HALF ? tile * HALF + wave : (N / 32) + tile * HALF + (wave - HALF);
        else
            return (tile * WAVES + wave) * (WROWS / 16);
    };
    // wave-tiled device layout (see repack_q4k_matrix): the wave's 16 rows are
    // one contiguous run of nsb 2304-byte chunks read front to back
    auto wave_base = [&](int tt) -> const uint8_t* {
        const int sl = tt / (tiles * S), rm = tt - sl * tiles * S, ti = rm / S, ks = rm - ti * S;
        return bank + (size_t)slot_eid[sl] * expert_stride + mat_offset +
               ((size_t)wave_tile(ti) * nsb_row + (size_t)ks * nsb) * CHUNK;
    };
    // Weight loads go through a buffer resource on the wave's run (uniform:
    // scalar base, the chunk offset in soffset, constant lane offsets), so no
    // per-step 64-bit address arithmetic runs on the vector ALUs.
    auto rsrc = [&](const uint8_t* p) -> __amdgpu_buffer_rsrc_t {
        const uint64_t u = (uint64_t)(uintptr_t)p;
        const uint64_t us = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
        // num_records: the run; dword 3: 32-bit data format (raw loads)
        return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)us, (short)0, (WROWS / 16) * nsb * CHUNK, 0x00020000);
    };
    constexpr int kNT = FST_WNT;  // cache policy: non-temporal (streamed once)
    // MF: lane (n, h) reads row n % 16 of tile n / 16 (the second tile's run
    // follows the first's), nibble bytes [64h, 64h + 64): region-0 and
    // region-1 pieces of lane groups 2h and 2h + 1
    const int mf_n = lane & 31, mf_h = lane >> 5;
    const int mf_t = (mf_n >> 4) * nsb * CHUNK, mf_r = mf_n & 15;
    auto load_w2 = [&](__amdgpu_buffer_rsrc_t rs, int off) -> WRaw2 {
        WRaw2 x;
        x.h = __builtin_amdgcn_raw_buffer_load_b128(rs, mf_t + 2048 + 16 * mf_r, off, kNT);
        x.a = __builtin_amdgcn_raw_buffer_load_b128(rs, mf_t + 16 * (32 * mf_h + mf_r), off, kNT);
        x.b = __builtin_amdgcn_raw_buffer_load_b128(rs, mf_t + 1024 + 16 * (32 * mf_h + mf_r), off, kNT);
        x.a1 = __builtin_amdgcn_raw_buffer_load_b128(rs, mf_t + 16 * (32 * mf_h + 16 + mf_r), off, kNT);
        x.b1 = __builtin_amdgcn_raw_buffer_load_b128(rs, mf_t + 1024 + 16 * (32 * mf_h + 16 + mf_r), off, kNT);
        return x;
    };
    auto load_w = [&](__amdgpu_buffer_rsrc_t rs, int off) -> WRaw {
        WRaw x;
        // (the header first: issued last, its register was taken by a live
        // staging address and got a copy at the loop back-edge, which waits
        // for the load: vmcnt(0) once per loop iteration)
        if constexpr (!MX) x.h = __builtin_amdgcn_raw_buffer_load_b128(rs, 2048 + 16 * (lane & 15), off, kNT);
        x.a = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * lane, off, kNT);
        x.b = __builtin_amdgcn_raw_buffer_load_b128(rs, 1024 + 16 * lane, off, kNT);
        if constexpr (MX) {
            typedef uint32_t u2v_t __attribute__((ext_vector_type(2)));
            const u2v_t hv = __builtin_amdgcn_raw_buffer_load_b64(rs, 2048 + 8 * (lane & 15), off, kNT);
            x.h = u4v_t{hv.x, hv.y, 0u, 0u};
        }
        return x;
    };

    // Every global load below is unconditional, with clamped addresses, and
    // every staging decision is a compile-time function of the unrolled
    // position: the number of loads in flight is then the same on every path
    // and the compiler waits only for the oldest super-block instead of
    // draining the prefetch ring at each step.
    __amdgpu_buffer_rsrc_t wrs = rsrc(wave_base(blockIdx.x));
    using WT = typename std::conditional<MF, WRaw2, WRaw>::type;
    auto load_any = [&](__amdgpu_buffer_rsrc_t rs, int off) -> WT {
        if constexpr (MF)
            return load_w2(rs, off);
        else
            return load_w(rs, off);
    };
    WT w[R];
#pragma unroll
    for (int j = 0; j < PF; ++j) w[j] = load_any(wrs, j * CHUNK);
    for (int i = tid; i < 2 * STAGE; i += NT) lds[i] = z4;

    // Staging map: chunk q = tid + NT*i of a macro-stage -> (super-block u,
    // token tl, part).  Chunks of token rows the slot does not have are not
    // stored: those LDS rows keep whatever an earlier item left there and
    // feed only discarded MFMA output rows (an output row reads only its own
    // operand row).  Their loads read a valid address, and a chunk slot
    // holding no live row at all is not loaded.  The next item's token rows are
    // fetched when an item starts and its map is built (and its first stage
    // loaded) during the current item's last macro-stage.
    int su[NS], stl[NS], spart[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int q = tid + NT * i;
        const int u = q / (TOKS * PARTS), rem = q - u * (TOKS * PARTS);
        su[i] = u;
        stl[i] = q < NCH ? rem / PARTS : TOKS;
        spart[i] = rem - (rem / PARTS) * PARTS;
    }
    auto load_rows = [&](int tt, int* ar) -> int {
        const int sl = tt / (tiles * S);
        const int Mi = min(slot_M[sl], TOKS), offi = slot_off[sl];
#pragma unroll
        for (int i = 0; i < NS; ++i)
            ar[i] = stl[i] < Mi ? (a_row ? a_row[offi + stl[i]] : offi + stl[i]) : -1;
        return Mi;
    };
    // Lowest token row that chunk slot i of any thread covers (0 when the
    // slot spans two super-blocks): an item with at most that many tokens
    // has nothing live in slot i, and its loads are skipped (uniformly).
    auto slot_minrow = [](int i) constexpr -> int {
        const int q0 = NT * i, q1 = (NT * i + NT < NCH ? NT * i + NT : NCH) - 1;
        return q0 / (TOKS * PARTS) != q1 / (TOKS * PARTS) ? 0 : (q0 % (TOKS * PARTS)) / PARTS;
    };
    int st_me = 0;  // token count of the item the staging map belongs to
    // The map keeps one int per chunk slot: the chunk's offset (16-byte
    // units) in A (parts 0..31) or SX (parts 32..35) for the item's first
    // macro-stage, or -1 when the slot has no live row.  Base, step and LDS
    // destination follow from the slot's (u, token, part), which are fixed
    // per thread, so they are formed at each use instead of being held in
    // registers across the super-block loop.
    int soff[NS];
    u4v_t sv[NS];
    // sbo: the item's first super-block within the row
    auto build_map = [&](const int* ar, int me, int sbo) {
        st_me = me;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int u = su[i], part = spart[i];
            soff[i] = ar[i] < 0 ? -1
                      : part < 32 ? ar[i] * (K / 8) + (sbo + u) * 32 + part
                                  : (ar[i] * nsb_row + sbo + u) * 4 + (part - 32);
        }
    };
    // past nsb inside a partial macro-stage a chunk re-reads its first
    // super-block (a valid address; the value is unused); a slot without a
    // live row reads the first chunk of its array
    auto stage_load = [&](int m) {
#pragma unroll
        for (int i = 0; i < NS; ++i) {
#if FST_SKIP_DEAD_SLOTS
            if (i > 0 && st_me <= slot_minrow(i)) continue;
#endif
            const int part = spart[i];
            const bool live = m * MS + su[i] < nsb;
            const int o = soff[i] < 0 ? 0 : soff[i] + (live ? m * (part < 32 ? 32 * MS : 4 * MS) : 0);
            const u4v_t* base = part < 32 ? reinterpret_cast<const u4v_t*>(A) : reinterpret_cast<const u4v_t*>(SX);
            sv[i] = base[o];
        }
    };
    auto stage_store = [&](int m) {
        const int base = (m & 1) * STAGE;
#pragma unroll
        for (int i = 0; i < NS; ++i)
            if (soff[i] >= 0)
                *reinterpret_cast<u4v_t*>(&lds[base + su[i] * TS + stl[i] * kTokStride + spart[i]]) = sv[i];
    };
    {
        int ar0[NS];
        const int me0 = load_rows(blockIdx.x, ar0);
        build_map(ar0, me0, ((int)blockIdx.x % S) * nsb);
        stage_load(0);
    }
    const int nms = nsb / MS;

    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        const int slot = t / (tiles * S);
        const int tile = (t - slot * tiles * S) / S;
        const int ks = t % S;
        const int tn = t + (int)gridDim.x;
        const __amdgpu_buffer_rsrc_t nrs = tn < total ? rsrc(wave_base(tn)) : wrs;
        const int Me = min(slot_M[slot], TOKS), off = slot_off[slot];
        const int row = wave_tile(tile) * 16 + r;
        int ar_next[NS];
        const int me_next = load_rows(tn < total ? tn : t, ar_next);

        __syncthreads();  // the previous item's readers of the LDS are done
        stage_store(0);
        __syncthreads();

        f4_t acc[NGRP];
#pragma unroll
        for (int q = 0; q < NGRP; ++q) acc[q] = zf;
        f16v_t acc32 = {};
        const int ngrp_live = (Me + 15) >> 4;

        // 32x32 tiles: 16 MFMAs on the lane's 16 nibble dwords, one for the
        // min term (sub-block sums of chunks 32 + 2h and 33 + 2h against the
        // mins of sub-blocks 4h..4h+3)
        auto compute32 = [&](int sb, const WRaw2& cur) {
            const int m = sb / MS, u = sb - m * MS;
            const uint4* st = lds + (m & 1) * STAGE + u * TS + mf_n * kTokStride;
            Q4kScale S0, S1;
            q4k_scales(cur.h, 2 * mf_h, q4k_scale_sel(2 * mf_h), S0);
            q4k_scales(cur.h, 2 * mf_h + 1, q4k_scale_sel(2 * mf_h + 1), S1);
            const uint32_t Dw[16] = {cur.a.x,  cur.a.y,  cur.a.z,  cur.a.w,  cur.b.x,  cur.b.y,  cur.b.z,  cur.b.w,
                                     cur.a1.x, cur.a1.y, cur.a1.z, cur.a1.w, cur.b1.x, cur.b1.y, cur.b1.z, cur.b1.w};
            f16v_t D = {};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const h8_t b = q4k_bop(Dw[j], j < 8 ? S0 : S1, magic);
                const h8_t a = __builtin_bit_cast(h8_t, st[16 * mf_h + j]);
                D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, D, 0, 0, 0);
            }
            const h8_t s0 = __builtin_bit_cast(h8_t, st[32 + 2 * mf_h]);
            const h8_t s1 = __builtin_bit_cast(h8_t, st[33 + 2 * mf_h]);
            const h8_t am = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
            const h8_t bm = {S0.m[0], S0.m[1], S0.m[2], S0.m[3], S1.m[0], S1.m[1], S1.m[2], S1.m[3]};
            const f16v_t Dm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, f16v_t{}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc32[i] = fmaf(S0.d, D[i], acc32[i]);
                acc32[i] = fmaf(-S0.dmin, Dm[i], acc32[i]);
            }
        };
        auto compute = [&](int sb, const WRaw& cur) {
            const int m = sb / MS, u = sb - m * MS;
            // at a capacity of 8 tokens, MFMA rows 8..15 (discarded) read rows
            // 0..7: the same addresses (a broadcast) instead of 8 more rows
            // whose 37-chunk stride lands on the same LDS banks
            const uint4* st = lds + (m & 1) * STAGE + u * TS + (TOKS < 16 ? (r & (TOKS - 1)) : r) * kTokStride;
            const uint32_t Dw[8] = {cur.a.x, cur.a.y, cur.a.z, cur.a.w, cur.b.x, cur.b.y, cur.b.z, cur.b.w};
            if constexpr (MX) {
                // lane (g, r): blocks 2g (cur.a) and 2g+1 (cur.b) of row r; the
                // hardware FP4 (E2M1) conversion applies the block scale exactly
                const uint32_t sw = g < 2 ? cur.h.x : cur.h.y;
                const float s0 = e8m0_scale((sw >> ((g & 1) * 16)) & 0xffu);
                const float s1 = e8m0_scale((sw >> ((g & 1) * 16 + 8)) & 0xffu);
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const float sc = c < 4 ? s0 : s1;
                    const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 0);
                    const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 1);
                    const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 2);
                    const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 3);
                    const bf8_t b = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
#pragma unroll
                    for (int q = 0; q < NGRP; ++q) {
                        if (q > 0 && q >= ngrp_live) break;
                        const bf8_t a = __builtin_bit_cast(bf8_t, st[q * 16 * kTokStride + 8 * g + c]);
                        acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[q], 0, 0, 0);
                    }
                }
                return;
            } else {
            Q4kScale S;
            q4k_scales(cur.h, g, ssel, S);
            // each decoded weight operand feeds every live 16-token group
            f4_t D[NGRP];
#pragma unroll
            for (int q = 0; q < NGRP; ++q) D[q] = zf;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const h8_t b = q4k_bop(Dw[c], S, magic);
#pragma unroll
                for (int q = 0; q < NGRP; ++q) {
                    if (q > 0 && q >= ngrp_live) break;
                    const h8_t a = __builtin_bit_cast(h8_t, st[q * 16 * kTokStride + 8 * g + c]);
                    D[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, D[q], 0, 0, 0);
                }
            }
#pragma unroll
            for (int q = 0; q < NGRP; ++q) {
                if (q > 0 && q >= ngrp_live) break;
                const h8_t am = __builtin_bit_cast(h8_t, st[q * 16 * kTokStride + 32 + g]);
                const f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, S.m, zf, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[q][i] = fmaf(S.d, D[q][i], acc[q][i]);
                    acc[q][i] = fmaf(-S.dmin, Dm[i], acc[q][i]);
                }
            }
            }
        };
        // U super-blocks per iteration (the launcher guarantees nsb % U == 0):
        // ring slot j % R, stage boundaries at j % MS, all known at compile
        // time.  The last PF prefetches are the next item's first chunks.
        // Every iteration ends on a barrier.
        for (int sb0 = 0; sb0 < nsb; sb0 += U) {
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int sb = sb0 + j;
                if (j % MS == 0) {
                    // one call site for the staging loads: loads issued on two
                    // paths leave their registers to a copy at the merge,
                    // and the copy waits for the load (vmcnt(0))
                    const bool last = sb / MS + 1 >= nms;
                    if (last) build_map(ar_next, me_next, (tn < total ? tn % S : ks) * nsb);
                    stage_load(last ? 0 : sb / MS + 1);
                }
                const int pf = sb + PF;
                // one load call site (resource and offset selected first), for
                // the same reason as the staging loads
                const bool pnx = pf >= nsb;
                w[(j + PF) % R] = load_any(pnx ? nrs : wrs, (pnx ? pf - nsb : pf) * CHUNK);
                // keep the prefetches where they are issued (the scheduler
                // would otherwise sink them next to their use to save registers)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (MF)
                    compute32(sb, w[j % R]);
                else
                    compute(sb, w[j % R]);
                if (j % MS == MS - 1) {
                    if (sb / MS + 1 < nms) stage_store(sb / MS + 1);
                    __syncthreads();
                }
            }
        }
        wrs = nrs;

        // D layout: lane holds token rows 4g+i (i=0..3) of the group, column r.
        auto unscale = [&](int pidx) -> int {
            if constexpr (MX)
                return 0;
            else
                return xs[a_row ? a_row[pidx] : pidx];
        };
        if (MODE == 1 && S > 1) {
            // split-K: this item's partial gate and up sums (rows of the
            // [gate | up] matrix) for the prep launch to add up
#pragma unroll
            for (int q = 0; q < NGRP; ++q) {
                if (q * 16 >= Me) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tl = q * 16 + 4 * g + i;
                    if (tl >= Me) continue;
                    ep.part[((size_t)ks * ep.part_rows + off + tl) * N + row] =
                        ldexpf(acc[q][i], unscale(off + tl));
                }
            }
            continue;
        }
        if constexpr (MODE == 1) {
            // gate waves hand their rows to the up waves through LDS (the
            // staging ring is free: the loop ended on a barrier)
            float* xg = reinterpret_cast<float*>(lds);
            if (wave < HALF) {
#pragma unroll
                for (int q = 0; q < NGRP; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tl = q * 16 + 4 * g + i;
                        xg[((wave * NGRP + q) * 4 + i) * 64 + lane] =
                            tl < Me ? ldexpf(acc[q][i], unscale(off + tl)) : 0.0f;
                    }
            }
            __syncthreads();
            if (wave >= HALF) {
                const int inter = N / 2;
                const int n = (tile * HALF + wave - HALF) * 16 + r;
                const float lim = ep.swiglu_limit;
#pragma unroll
                for (int q = 0; q < NGRP; ++q) {
                    if (q * 16 >= Me) break;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tl = q * 16 + 4 * g + i;
                        if (tl >= Me) continue;
                        float gv = xg[(((wave - HALF) * NGRP + q) * 4 + i) * 64 + lane];
                        float uv = ldexpf(acc[q][i], unscale(off + tl));
                        if (lim > 0.0f) {
                            gv = fminf(gv, lim);
                            uv = fminf(fmaxf(uv, -lim), lim);
                        }
                        const float hv = (gv / (1.0f + expf(-gv))) * uv;
                        if constexpr (MX)
                            ep.h16[(size_t)(off + tl) * inter + n] = fst_f32_to_bf16(hv);
                        else
                            ep.h[(size_t)(off + tl) * inter + n] = hv;
                    }
                }
            }
            continue;
        }
        if constexpr (MF) {
            // D layout (32x32): lane (n, h), value i is token row
            // 8 (i / 4) + 4 h + i % 4 of column n
            const int row32 = wave_tile(tile) * 16 + mf_n;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tl = 8 * (i >> 2) + 4 * mf_h + (i & 3);
                if (tl >= Me) continue;
                const int pidx = off + tl;
                out[(size_t)pidx * N + row32] = ldexpf(acc32[i], unscale(pidx));
            }
            continue;
        }
        const bool direct = MODE == 2 && (ep.o1 || ep.o2);
#pragma unroll
        for (int q = 0; q < NGRP; ++q) {
            if (q * 16 >= Me) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tl = q * 16 + 4 * g + i;
                if (tl >= Me) continue;
                const int pidx = off + tl;
                const float yv = ldexpf(acc[q][i], unscale(pidx));
                if (direct) {
                    // the combine of a single pair: bf16(w * y) (src/fst_engine.cpp:4196-4201)
                    const int tok = ep.pair_tok[pidx];
                    const uint16_t o = fst_f32_to_bf16(ep.wts[tok] * yv);
                    if (ep.o1) ep.o1[(size_t)tok * N + row] = o;
                    if (ep.o2) ep.o2[(size_t)tok * N + row] = o;
                } else {
                    out[(size_t)pidx * N + row] = yv;
                }
            }
        }
    }
}

// --------------------------------------------- fused gate||up + down launch
//
// One persistent launch runs a block-8 MoE layer's expert work after the
// router: the work items are every (slot, 64-row gate||up tile) and then
// every (slot, 128-row down tile), dealt to the workgroups in static rounds
// (t = blockIdx.x + k * gridDim.x).  The down items of the early rounds fill
// the time that workgroups would otherwise spend idle at the end of a
// separate gate||up launch, and no operand-prep launch runs between them.
//  - routing: every workgroup computes the call's top-k and bucketing into
//    LDS first (topk_bucket_block), as the gate||up launch does;
//  - gate||up items: the arithmetic of q4k_linear_kernel MODE 1 (16-row MFMA
//    tiles, 8 waves: 64 gate rows in waves 0..3 paired with the same up rows
//    in waves 4..7), with the item's operand copied into LDS at its start
//    (a slot of 5..8 tokens in two halves of K, of 9..16 tokens in four
//    quarters, rebuilt between them), so that the super-block loop has no
//    staging loads and no per-super-block barrier;
//    the up waves write h = silu(g)*u as 64-bit words {epoch, h bits} with
//    device-coherent stores, and per 16 rows the largest |h| of each token
//    in the same form (the down operand's prescale needs the row maximum);
//  - down items: wait until the slot's maxima and h words carry this call's
//    epoch (coherent loads, bounded polling; for a one-token slot the first
//    poll's words are loaded during the last super-block of the item before),
//    then build the slot's fp16 operand (prescale, k-interleave and sub-block
//    sums exactly as prep_row) in LDS once per item (a slot of 9..16 tokens
//    in two halves of K), and stream the down weights with no staging or
//    barrier inside the super-block loop; y rows go out in fp32 for the
//    combine launch.
// Slots of more than 16 tokens run as several 16-token slot groups.  Calls of
// at most 8 tokens use the SMALL instantiation (no slot above 8 tokens: none
// of the group and phase paths compiled in).
// Deadlock freedom: every workgroup finishes its gate||up items (lower
// indices) before it reaches a down item, and the grid never exceeds the
// workgroups the device holds at once (two per CU), so every item a down
// item waits for is processed.  The waits are still bounded: past
// spin_limit polls a workgroup sets meta[META_TIMEOUT] and the sticky
// timeout bit and carries on (fst_moe_check and the host-pointer entry
// points turn that into FST_EHIP).
// Build-time settings (measured defaults): operand chunks per thread in
// flight when a gate||up item rebuilds its operand inside the super-block
// loop (SMALL and general instantiation), and the token rows of a down slot.
#ifndef FST_FU_NB_SMALL
#define FST_FU_NB_SMALL 1
#endif
#ifndef FST_FU_NB
#define FST_FU_NB 5
#endif
#ifndef FST_FU_TD
#define FST_FU_TD 16
#endif
constexpr int kFuT = 16;                          // token rows of a gate||up slot (the MFMA's 16 rows)
constexpr int kFuTD = FST_FU_TD;                  // token rows of a down slot
constexpr int kFuMaxM = 32;                       // tokens of one call
constexpr int kFuMaxPairs = 256;                  // routed (token, expert) pairs of one call
// slots of one call: every routed pair its own expert, the shared expert,
// and the extra slots of experts split into groups of kFuT tokens
constexpr int kFuMaxSlots = kFuMaxPairs + 1 + (kFuMaxPairs + kFuMaxM) / kFuTD;
constexpr int kFuW = 8;                           // waves per workgroup
constexpr int kFuHalf = kFuW / 2;
constexpr int kFuChunk = 2304;                    // Q4_K bytes per 16 rows x 256 weights
constexpr int kFuParts = 36;                      // staged chunks per token per super-block
constexpr int kFuMaxDnSb = 8;                     // down K (inter) <= 2048
constexpr int kFuOpStride = kFuMaxDnSb * 36 + 1;  // down operand row in LDS, uint4
constexpr int kFuOpStride16 = 16 * 36 + 1;        // gate||up operand row of <= 4 tokens x 16 super-blocks
constexpr int kFuOpStride4 = 4 * 36 + 1;          // operand row of 9..16 tokens, 4 super-blocks per phase
constexpr int kFuOpb = 16 * kFuOpStride4 > 8 * kFuOpStride ? 16 * kFuOpStride4 : 8 * kFuOpStride;

struct FusedArgs {
    const uint8_t* bank;
    size_t expert_stride;         // bytes per expert
    const _Float16* A;            // gate||up operand [T][hd] (router_prep)
    const uint4* SX;              // its sub-block sums
    const int* xs;                // its prescale exponents
    unsigned long long* hbuf;     // [P][inter] {epoch, h bits}
    unsigned long long* amaxw;    // [P][inter/16] {epoch, max |h| over 16 rows}
    size_t hbuf_bytes;
    float* y;                     // [P][hd]
    int* claim;                   // item counter, zero at launch (null: static rounds only)
    float swiglu_limit;
    uint32_t epoch;
    int spin_limit;
    int singles;                  // the last down items handed out one by one
};

// Largest value of the 16 lanes of each DPP row (all 64 lanes active).
__device__ __forceinline__ float row16_fmax(float x) {
    x = fmaxf(x, fdpp<0x128>(x));  // row_ror 8
    x = fmaxf(x, fdpp<0x124>(x));  // row_ror 4
    x = fmaxf(x, fdpp<0x122>(x));  // row_ror 2
    x = fmaxf(x, fdpp<0x121>(x));  // row_ror 1
    return x;
}

// CODEC 0: Q4_K experts, fp16 operands with power-of-two prescales, fp16
// MFMA; 1: MXFP4 experts, bf16 operands (the input rows as they are, h
// rounded to bf16), bf16 MFMA, as in q4k_linear_kernel's MXFP4 path.
// SMALL: calls of at most 8 tokens (no slot above 8 tokens: no slot splits,
// no operand phases for down items, no 9..16-token layout compiled in).
template <int HD, int INTER, int CODEC, bool SMALL>
__global__ __launch_bounds__(64 * kFuW) __attribute__((amdgpu_waves_per_eu(FST_Q4K_WAVES_PER_EU))) void
moe_fused_kernel(FusedArgs fa, RouteArgs ra) {
    constexpr bool MX = CODEC == 1;
    constexpr int CHK = MX ? 2176 : kFuChunk;     // bytes per 16 rows x 256 weights
    constexpr int PARTS = MX ? 32 : kFuParts;     // staged chunks per token per super-block
    static_assert(INTER % 1024 == 0 && INTER <= 256 * kFuMaxDnSb && HD % 512 == 0, "fused geometry");
    constexpr int NT = 64 * kFuW;
    static_assert(4 * kFuOpStride16 <= kFuOpb && HD == 4096, "gate||up operand of 4 tokens fits opb");
    static_assert(HD / 8 == NT, "one operand chunk per thread for a one-token prefetch");
    constexpr int RPER = 4;
    __shared__ float xg[kFuHalf * 4 * 64];  // gate rows handed to the up waves
    __shared__ int s_xs[kFuMaxM];           // prescale exponents of the token rows
    __shared__ uint4 opn[kFuOpStride16];    // the next item's one-token gate||up operand
    __shared__ uint4 opb[kFuOpb];
    __shared__ float s_amax[kFuTD][1];
    __shared__ int s_xs2[kFuTD];
    __shared__ int s_claim;
    __shared__ int s_vn[kFuW];              // slot split: the waves' counts
    __shared__ int r_meta[META_WORDS], r_seid[kFuMaxSlots], r_sM[kFuMaxSlots], r_soff[kFuMaxSlots];
    __shared__ int d_seid[kFuMaxSlots], d_sM[kFuMaxSlots], d_soff[kFuMaxSlots];  // down slots
    __shared__ int s_nds;
    __shared__ int r_ptok[kFuMaxPairs + kFuMaxM], r_pof[kFuMaxPairs], r_psh[kFuMaxM];
    __shared__ int r_yrow[kFuMaxPairs + kFuMaxM];  // pair -> its y row t*(tk+1) + j (shared: j = tk)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int hd = HD, inter = INTER;
    const size_t stride = fa.expert_stride;
    const uint8_t* bank = fa.bank;
    {
        RouteArgs la = ra;
        la.meta = r_meta;
        la.slot_eid = r_seid;
        la.slot_M = r_sM;
        la.slot_off = r_soff;
        la.pair_tok = r_ptok;
        la.pair_of = r_pof;
        la.pair_shared = r_psh;
        // the shared expert's gate||up slice of this workgroup, read while it
        // routes (see q4k_linear_kernel)
        uint4 pfv[3];
        const int npf = ra.use_shared ? 3 : 0;
        {
            const size_t pieces = (size_t)(2 * inter / 16) * (hd >> 8) * (CHK / 16);
            const uint4* src = reinterpret_cast<const uint4*>(bank + (size_t)ra.E * stride);
            const size_t step = (size_t)gridDim.x * NT;
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const size_t q = (size_t)blockIdx.x * NT + tid + i * step;
                pfv[i] = i < npf ? src[q < pieces ? q : 0] : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        topk_bucket_block<RPER, NT, kFuMaxM>(la, blockIdx.x == 0);
#pragma unroll
        for (int i = 0; i < 3; ++i) asm volatile("" ::"v"(pfv[i].x));
        __syncthreads();
        if (blockIdx.x == 0) {
            const int ns = r_meta[META_N_SLOTS], np = r_meta[META_N_PAIRS];
            if (tid <= META_N_ROUTED_PAIRS) ra.meta[tid] = r_meta[tid];
            if (tid == 0) sticky_or(ra.meta, r_meta[META_ERROR]);
            if (tid == META_TIMEOUT) ra.meta[META_TIMEOUT] = 0;
            for (int i = tid; i < ns; i += NT) {
                ra.slot_eid[i] = r_seid[i];
                ra.slot_M[i] = r_sM[i];
                ra.slot_off[i] = r_soff[i];
            }
            for (int i = tid; i < np; i += NT) ra.pair_tok[i] = r_ptok[i];
            for (int i = tid; i < ra.M * ra.tk; i += NT) ra.pair_of[i] = r_pof[i];
            if (ra.use_shared)
                for (int i = tid; i < ra.M; i += NT) ra.pair_shared[i] = r_psh[i];
        }
        // y rows by (token, j), so that the combine reads them without the
        // pair table (one round trip instead of two); the rows of pairs
        // without a valid expert are zeros (workgroup 0 writes them), which
        // the combine adds as the chain's combine skips them
        // (caller-given routing may name one expert twice for a token: two
        // (token, j) share one pair there, so y stays indexed by pair and the
        // pair-table combine follows)
        if (ra.given) {
            for (int i = tid; i < kFuMaxPairs + kFuMaxM; i += NT) r_yrow[i] = i;
        } else {
        for (int i = tid; i < ra.M * ra.tk; i += NT)
            if (r_pof[i] >= 0) r_yrow[r_pof[i]] = (i / ra.tk) * (ra.tk + 1) + i % ra.tk;
        }
        if (blockIdx.x == 0 && r_meta[META_ERROR] && !ra.given)
            for (int i = 0; i < ra.M * ra.tk; ++i)
                if (r_pof[i] < 0) {
                    float4* yz = reinterpret_cast<float4*>(fa.y + (size_t)((i / ra.tk) * (ra.tk + 1) + i % ra.tk) * hd);
                    for (int q = tid; q < hd / 4; q += NT) yz[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
        if (ra.use_shared && !ra.given)
            for (int i = tid; i < ra.M; i += NT) r_yrow[r_psh[i]] = i * (ra.tk + 1) + ra.tk;
        // the tokens' operand prescale exponents, read in LDS by the gate||up
        // epilogue (a global load there would wait, in the in-order count,
        // behind the next item's weight prefetch)
        if (!MX && tid < ra.M) s_xs[tid] = fa.xs[tid];
        __syncthreads();
        // Slots of more than kFuT tokens become several gate||up slots of at
        // most kFuT consecutive pairs each, and slots of more than kFuTD tokens
        // several down slots of at most kFuTD (the expert's matrix streamed
        // once per group).  Each thread reads its slot, the waves count the
        // new slots (shuffle prefix), and every slot writes its groups.
        {
            const int ns0 = r_meta[META_N_SLOTS];
            int e0 = 0, m0 = 0, o0 = 0;
            if (tid < ns0) {
                e0 = r_seid[tid];
                m0 = r_sM[tid];
                o0 = r_soff[tid];
            }
            auto split = [&](int cap, int* se, int* sm, int* so, int* count) {
                const int nv = tid < ns0 ? (m0 + cap - 1) / cap : 0;
                int x = nv;
#pragma unroll
                for (int d = 1; d < 64; d <<= 1) {
                    const int y = __shfl_up(x, d, 64);
                    if (lane >= d) x += y;
                }
                if (lane == 63) s_vn[wave] = x;
                __syncthreads();
                int before = 0, total_v = 0;
#pragma unroll
                for (int w2 = 0; w2 < kFuW; ++w2) {
                    const int c = s_vn[w2];
                    if (w2 < wave) before += c;
                    total_v += c;
                }
                const int first = before + x - nv;
                __syncthreads();
                for (int v = 0; v < nv; ++v) {
                    se[first + v] = e0;
                    sm[first + v] = min(cap, m0 - v * cap);
                    so[first + v] = o0 + v * cap;
                }
                if (tid == 0) *count = total_v;
            };
            // (ns0 <= kFuMaxPairs + 1 <= NT: one slot per thread; without
            // large slots, the down items read the gate||up table)
            const int big = SMALL ? 0 : __syncthreads_or(m0 > kFuTD);
            if (big) {
                if constexpr (kFuT == kFuTD) {
                    // one table for both: the down items read the split gate||up table
                    split(kFuT, r_seid, r_sM, r_soff, &r_meta[META_N_SLOTS]);
                    if (tid == 0) s_nds = -1;
                } else {
                    split(kFuTD, d_seid, d_sM, d_soff, &s_nds);
                    if (__syncthreads_or(m0 > kFuT)) split(kFuT, r_seid, r_sM, r_soff, &r_meta[META_N_SLOTS]);
                }
            } else if (tid == 0) {
                s_nds = -1;
            }
            __syncthreads();
        }
    }
    const int ns = r_meta[META_N_SLOTS], nds = s_nds < 0 ? ns : s_nds;
    // the down slot table: its own when slots were split for the down items
    const int* dtab_e = s_nds < 0 ? r_seid : d_seid;
    const int* dtab_m = s_nds < 0 ? r_sM : d_sM;
    const int* dtab_o = s_nds < 0 ? r_soff : d_soff;
    constexpr int tiles_gu = inter / 64, tiles_dn = hd / 128;
    const int ngu = ns * tiles_gu, total = ngu + nds * tiles_dn;
    const int ndn = total - ngu;
    if ((int)blockIdx.x >= total) return;
    const int r = lane & 15, g = lane >> 4;
    constexpr int nsb_gu = hd >> 8, nsb_dn = inter >> 8;
    constexpr int aw = inter / 16;  // amax words per pair
    constexpr size_t proj = (size_t)inter * (hd / 256) * (MX ? 136 : 144);
    const f4_t zf = f4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t magic = 0x64006400u;
    const uint32_t ssel = q4k_scale_sel(g);
    const uint32_t epoch = fa.epoch;

    // Item order: the gate||up items, then the down items, each in slot-major
    // order, so down items 2p, 2p+1 are the tiles 2x, 2x+1 of one slot.  The
    // first round is static (item blockIdx.x); after it workgroups claim work
    // from the call's counter: claim k = G + counter is gate||up item k, or,
    // past them, a down pair (both tiles, the second reusing the operand the
    // first built in LDS) or, for the last G down items, a single item.  Workgroups that run faster take more
    // work (the second workgroup of a CU runs measurably slower), and the
    // launch ends within about one item of its average.  A claim's answer is
    // needed only at the last super-block of the item before the claimed
    // work: gate||up items and second halves of down pairs claim their
    // successor early enough that thread 0 can store the answer to LDS three
    // super-blocks before the end, where a barrier publishes it.  Work is
    // claimed in increasing order, and a down item waits only for gate||up
    // items of lower index, claimed earlier by running workgroups that never
    // wait: no wait can close a cycle.  Without a counter (or with fewer
    // gate||up items than workgroups) the rounds stay static.
    // The last G down items go out one by one: claimed pairs are about two
    // items long, and single items at the end keep the workgroups' finishing
    // times within about one down item.
    const int G = (int)gridDim.x;
    const bool dyn = fa.claim != nullptr && ngu >= G;
    const int D1 = max(ndn - fa.singles, 0) & ~1;  // down items [0, D1) go in pairs
    auto dn_map = [&](int d, int& sl, int& ti) {
        sl = d / tiles_dn;
        ti = d - sl * tiles_dn;
    };
    auto claim_item = [&](int k) {
        if (k < ngu) return k;
        const int p = k - ngu;
        return p < D1 / 2 ? ngu + 2 * p : ngu + D1 + (p - D1 / 2);
    };
    // the wave's contiguous run of 2304-byte chunks in item tt
    auto wave_base = [&](int tt) -> const uint8_t* {
        if (tt < ngu) {
            const int sl = tt / tiles_gu, ti = tt - sl * tiles_gu;
            const int wt = wave < kFuHalf ? ti * kFuHalf + wave : inter / 16 + ti * kFuHalf + (wave - kFuHalf);
            return bank + (size_t)r_seid[sl] * stride + (size_t)wt * nsb_gu * CHK;
        }
        int sl, ti;
        dn_map(tt - ngu, sl, ti);
        return bank + (size_t)dtab_e[sl] * stride + 2 * proj + (size_t)(ti * kFuW + wave) * nsb_dn * CHK;
    };
    auto rsrc = [&](const uint8_t* p, int nsb) -> __amdgpu_buffer_rsrc_t {
        const uint64_t u = (uint64_t)(uintptr_t)p;
        const uint64_t us = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
        return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)us, (short)0, nsb * CHK, 0x00020000);
    };
    auto item_rsrc = [&](int tt) { return rsrc(wave_base(tt), tt < ngu ? nsb_gu : nsb_dn); };
    constexpr int kNT = FST_WNT;
    auto load_w = [&](__amdgpu_buffer_rsrc_t rs, int off) -> WRaw {
        WRaw x;
        if constexpr (MX) {
            // (the scale bytes first, as the Q4_K header, for the same reason)
            typedef uint32_t u2v_t __attribute__((ext_vector_type(2)));
            const u2v_t hv = __builtin_amdgcn_raw_buffer_load_b64(rs, 2048 + 8 * (lane & 15), off, kNT);
            x.h = u4v_t{hv.x, hv.y, 0u, 0u};
        } else {
            x.h = __builtin_amdgcn_raw_buffer_load_b128(rs, 2048 + 16 * (lane & 15), off, kNT);
        }
        x.a = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * lane, off, kNT);
        x.b = __builtin_amdgcn_raw_buffer_load_b128(rs, 1024 + 16 * lane, off, kNT);
        return x;
    };
    // h words of the call, read with device-coherent 16-byte loads (sc1)
    const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
        fa.hbuf, (short)0, (int)(fa.hbuf_bytes < 0x7fffffffull ? fa.hbuf_bytes : 0x7fffffffull), 0x00020000);
    // the row maxima words, likewise
    static_assert(aw == 128, "one wave's 64 lanes x 2 words cover a row's maxima");
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        fa.amaxw, (short)0, (int)(fa.hbuf_bytes / 16 < 0x7fffffffull ? fa.hbuf_bytes / 16 : 0x7fffffffull), 0x00020000);

    __amdgpu_buffer_rsrc_t wrs = item_rsrc(blockIdx.x);
    WRaw w[2];
    w[0] = load_w(wrs, 0);
    // The gate||up operand of an item, copied once from the call's prepared
    // rows (A: fp16 operand chunks, SX: sub-block sums) into opb: for a slot
    // of at most 4 tokens all nsb_gu super-blocks at once (row stride
    // kFuOpStride16), else 8 super-blocks per phase (row stride kFuOpStride,
    // the down operand's layout).  Per token row and super-block 36 chunks,
    // 32 operand chunks then the 4 sum chunks (MXFP4: the 32 chunks of bf16
    // input only).  Rows past the slot's tokens are left as they are: their
    // MFMA rows are discarded.
    // (NB loads per thread in flight: fewer inside the super-block loop,
    // where the weight ring holds registers)
    auto gu_build = [&](auto nbc, int Me, int off, int sbase, int nph, int ostr) {
        constexpr int NB = decltype(nbc)::value;
        const int per = nph * PARTS, n = Me * per;
        const u4v_t* A4 = reinterpret_cast<const u4v_t*>(fa.A);
        const u4v_t* SX4 = reinterpret_cast<const u4v_t*>(fa.SX);
        for (int q0 = tid; q0 < n; q0 += NB * NT) {
            u4v_t v[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int q = min(q0 + u * NT, n - 1);
                const int tl = q / per, rem = q - tl * per, sbl = rem / PARTS, part = rem - sbl * PARTS;
                const int tok = r_ptok[off + tl];
                v[u] = part < 32 ? A4[tok * (hd / 8) + (sbase + sbl) * 32 + part]
                                 : SX4[tok * nsb_gu * 4 + (sbase + sbl) * 4 + (part - 32)];
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int q = q0 + u * NT;
                if (q < n) {
                    const int tl = q / per, rem = q - tl * per, sbl = rem / PARTS, part = rem - sbl * PARTS;
                    *reinterpret_cast<u4v_t*>(&opb[tl * ostr + sbl * 36 + part]) = v[u];
                }
            }
        }
    };

    // The down operand of a down slot's rows (at most kFuTD): all nsb_dn
    // super-blocks for a slot of at most 8 tokens, else nph super-blocks from
    // sbase per call (the row maxima read with the first phase), built in LDS from the gate||up items' h words: poll until
    // the words and the row maxima words carry this call's epoch
    // (device-coherent loads, bounded), then convert.  Each polling round issues the
    // maxima loads (Me*aw words) and the first pass of h loads together, so a
    // slot of one or two tokens (most routed slots) costs one round trip when
    // its words are in.  Q4_K: the fp16 operand, prescaled, k-interleaved and
    // with the sub-block sums split hi+lo exactly as prep_row builds it;
    // MXFP4: the h words rounded to bf16, 8 per chunk in element order.
    // Each round covers 512 operand chunks as two sub-rounds of 256: thread
    // tid takes chunk base + 256u + (tid & 255) of sub-round u and half
    // tid >> 8 of it (the chunk's elements e0..e0+3, or e0+32..e0+35: two
    // 16-byte h loads), so a one-token slot (256 chunks per row) spreads over
    // all 512 threads.  Chunk q's 8 lanes of a sub-block sit in consecutive
    // lanes of one wave, as the sub-block sums' butterflies need.  `pf`: the
    // first poll of a one-token slot takes sub-round 0's words (pd) and the
    // maxima (pm) that the item before loaded.
    u4v_t pd[2] = {u4v_t{0u, 0u, 0u, 0u}, u4v_t{0u, 0u, 0u, 0u}};
    u4v_t pm = u4v_t{0u, 0u, 0u, 0u};
    // byte offsets of the two h loads of chunk q (chunk-row tl) and half hf
    auto h_off = [&](int off, int tl, int q, int sb, int hf) -> int {
        if constexpr (MX) {
            return ((off + tl) * inter + sb * 256 + 8 * (q & 31)) * 8 + 32 * hf;
        } else {
            const int gg = (q >> 3) & 3, c = q & 7;
            return ((off + tl) * inter + sb * 256 + 64 * gg + 4 * c) * 8 + 256 * hf;
        }
    };
    auto dn_build = [&](int Me, int off, int sbase, int nph, int ostr, bool pf) {
        const int cpr = nph * 32;     // operand chunks per row of this phase
        const int nwd = sbase == 0 ? Me * aw : 0;  // maxima words of the slot's rows (first phase)
        const int nch = Me * cpr;     // operand chunks of the slot's rows
        const int hf = tid >> 8, ql = tid & 255;
        int timed_out = 0;
        for (int spin = 0;; ++spin) {
            int ok = 1;
            const bool use_pf = pf && spin == 0;
            // maxima words: two per thread and load (16 bytes), so that the
            // 128 words of a row are one wave's (aw == 128)
            static_assert(kFuTD * aw <= 4 * NT, "two 16-byte maxima loads per thread");
            u4v_t mv[2];
            if constexpr (!MX) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int i = 2 * tid + 2 * NT * k;
                    mv[k] = (k == 0 || (!SMALL && kFuTD * aw > 2 * NT))
                                ? __builtin_amdgcn_raw_buffer_load_b128(ars, (off * aw + (i < nwd ? i : 0)) * 8, 0, 16)
                                : u4v_t{0u, 0u, 0u, 0u};
                }
                if (use_pf) mv[0] = pm;
            }
            for (int base = 0; base < nch; base += 2 * 256) {
                u4v_t hw[2][2];
                int tlu[2], qu[2];
                bool liveu[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int qq = base + 256 * u + ql;
                    liveu[u] = qq < nch;
                    tlu[u] = liveu[u] ? qq / cpr : 0;
                    qu[u] = qq - (qq / cpr) * cpr;
                    const int o = h_off(off, tlu[u], qu[u], sbase + (qu[u] >> 5), hf);
                    hw[u][0] = __builtin_amdgcn_raw_buffer_load_b128(hrs, o, 0, 16);
                    hw[u][1] = __builtin_amdgcn_raw_buffer_load_b128(hrs, o + 16, 0, 16);
                }
                if (use_pf && base == 0) {
                    hw[0][0] = pd[0];
                    hw[0][1] = pd[1];
                }
                if constexpr (!MX) {
                    if (base == 0 && sbase == 0) {
                        // the row maxima -> prescale exponents (the 128 words
                        // of a row are one wave's)
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            if (k == 1 && (SMALL || kFuTD * aw <= 2 * NT)) break;
                            const int i = 2 * tid + 2 * NT * k;
                            float m = 0.0f;
                            if (i < nwd) {
                                // words {max bits, epoch}
                                if (mv[k].y != epoch || mv[k].w != epoch)
                                    ok = 0;
                                else
                                    m = fmaxf(fst_bits_f32(mv[k].x), fst_bits_f32(mv[k].z));
                            }
                            m = wave_fmax(m);
                            if (lane == 0 && i < nwd) s_amax[i / aw][0] = m;
                        }
                        __syncthreads();
                        if (tid < Me) s_xs2[tid] = prescale_exp(s_amax[tid][0]);
                        __syncthreads();
                    }
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const bool live = liveu[u];
                    const int tl = tlu[u], q = qu[u], sbl = q >> 5;
                    const u4v_t a = hw[u][0], b = hw[u][1];
                    // words {h bits, epoch}: .y / .w hold the tags
                    if (live && (a.y != epoch || a.w != epoch || b.y != epoch || b.w != epoch)) ok = 0;
                    uint2* dst = reinterpret_cast<uint2*>(&opb[tl * ostr + sbl * 36 + (q & 31)]) + hf;
                    if constexpr (MX) {
                        const uint32_t o0 = (uint32_t)fst_f32_to_bf16(fst_bits_f32(a.x)) |
                                            ((uint32_t)fst_f32_to_bf16(fst_bits_f32(a.z)) << 16);
                        const uint32_t o1 = (uint32_t)fst_f32_to_bf16(fst_bits_f32(b.x)) |
                                            ((uint32_t)fst_f32_to_bf16(fst_bits_f32(b.z)) << 16);
                        if (live) *dst = make_uint2(o0, o1);
                    } else {
                        const int gg = (q >> 3) & 3, c = q & 7;
                        const int sx = s_xs2[tl];
                        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
                        h4_t v;
                        v[0] = (_Float16)ldexpf(fst_bits_f32(a.x), -sx);
                        v[1] = (_Float16)ldexpf(fst_bits_f32(b.x), -sx);
                        v[2] = (_Float16)ldexpf(fst_bits_f32(a.z), -sx);
                        v[3] = (_Float16)ldexpf(fst_bits_f32(b.z), -sx);
                        if (live) *dst = __builtin_bit_cast(uint2, v);
                        float sm = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
                        sm = sm + fdpp<0xb1>(sm);  // quad_perm [1,0,3,2]
                        sm = sm + fdpp<0x4e>(sm);  // quad_perm [2,3,0,1]
                        sm = sm + fdpp<0x104>(sm);  // row_shl 4
                        if (live && c == 0) {
                            // the sum chunk {h0, h1, l0, l1, 0, 0, 0, 0}: half 0
                            // holds sub-block 2gg's sum (h0, l0), half 1 the other
                            _Float16* sc = reinterpret_cast<_Float16*>(&opb[tl * ostr + sbl * 36 + 32 + gg]);
                            const _Float16 hs = (_Float16)sm;
                            sc[hf] = hs;
                            sc[2 + hf] = (_Float16)(sm - (float)hs);
                            if (hf == 0) *reinterpret_cast<uint2*>(sc + 4) = make_uint2(0u, 0u);
                        }
                    }
                }
            }
            if (__syncthreads_and(ok)) break;
            if (spin >= fa.spin_limit) {
                timed_out = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (timed_out && tid == 0) {
            atomicOr(&ra.meta[META_TIMEOUT], 1);
            sticky_or(ra.meta, STICKY_TIMEOUT);
        }
    };

    // one 16-row x 256-weight step: Q4_K decode + MFMA against the operand
    // rows at st (row stride rs uint4), accumulated into acc
    auto compute = [&](const uint4* st, const WRaw& cur, f4_t& acc) {
        const uint32_t Dw[8] = {cur.a.x, cur.a.y, cur.a.z, cur.a.w, cur.b.x, cur.b.y, cur.b.z, cur.b.w};
        if constexpr (MX) {
            // lane (g, r): blocks 2g (cur.a) and 2g+1 (cur.b) of row r; the
            // hardware E2M1 conversion applies the block scale exactly
            const uint32_t sw = g < 2 ? cur.h.x : cur.h.y;
            const float s0 = e8m0_scale((sw >> ((g & 1) * 16)) & 0xffu);
            const float s1 = e8m0_scale((sw >> ((g & 1) * 16 + 8)) & 0xffu);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const float sc = c < 4 ? s0 : s1;
                const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 0);
                const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 1);
                const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 2);
                const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(Dw[c], sc, 3);
                const bf8_t b = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
                const bf8_t a = __builtin_bit_cast(bf8_t, st[8 * g + c]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
            }
            return;
        }
        Q4kScale S;
        q4k_scales(cur.h, g, ssel, S);
        f4_t D = zf;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const h8_t b = q4k_bop(Dw[c], S, magic);
            const h8_t a = __builtin_bit_cast(h8_t, st[8 * g + c]);
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, D, 0, 0, 0);
        }
        const h8_t am = __builtin_bit_cast(h8_t, st[32 + g]);
        const f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, S.m, zf, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = fmaf(S.d, D[i], acc[i]);
            acc[i] = fmaf(-S.dmin, Dm[i], acc[i]);
        }
    };

    int opb_key = -1;  // what opb holds: slot (gate||up, one phase), slot | 2^20 (down), -1: neither
    // A gate||up item of a one-token slot gets its operand chunks loaded into
    // registers (pv: chunk tid = 32 sb + part, the 32 operand chunks of each
    // super-block) one super-block before the end of the item before it, and
    // written to opn with the sub-block sums (computed from the same fp16
    // values in prep_row's order) once that item's readers are done: no load
    // latency at its start.  The loads are issued for every item on one
    // straight path (loads on two paths merge into register copies that wait
    // for them), before the weight prefetch of the next item's first
    // super-block, so waiting for them waits for nothing else.
    bool pre = false;  // this item's operand arrives in pv
    u4v_t pv = u4v_t{0u, 0u, 0u, 0u};
    bool pdn = false;  // this down item's first h words and maxima arrive in pd, pm
    int claimed = 0;    // thread 0: the counter value its last claim returned
    for (int t = blockIdx.x, tn = total; t < total; t = tn) {
        const bool dn = t >= ngu;
        __syncthreads();  // the previous item's readers of the LDS are done
        const int nsb = dn ? nsb_dn : nsb_gu;
        int slot = t / tiles_gu, tile = t - slot * tiles_gu;
        if (dn) dn_map(t - ngu, slot, tile);
        const int Me = dn ? dtab_m[slot] : r_sM[slot], off = dn ? dtab_o[slot] : r_soff[slot];
        // the item that follows: the second half of this down pair, or claimed
        const bool pair1 = dyn && dn && t - ngu < D1 && ((t - ngu) & 1) == 0;
        const bool claims = dyn && !pair1;
        __amdgpu_buffer_rsrc_t nrs = wrs;
        f4_t acc = zf;
        // the operand layout of the item: nph super-blocks in opb at once
        // (all of them, or phases rebuilt inside the super-block loop), the
        // row stride, and the operand row a lane's MFMA row reads
        int nph, ostr, rs;
        if (Me <= 4 && !dn) {
            nph = nsb_gu;
            ostr = kFuOpStride16;
            rs = r & 3;
        } else if (SMALL || Me <= 8) {  // (every down slot of at most 8 tokens)
            nph = 8;
            ostr = kFuOpStride;
            rs = r & 7;
        } else {
            nph = 4;
            ostr = kFuOpStride4;
            rs = r;
        }
        const bool multi = nph < nsb;
        if (!dn) {
            if (pre) {
                const int sbl = tid >> 5, part = tid & 31;
                *reinterpret_cast<u4v_t*>(&opn[sbl * 36 + part]) = pv;
                if constexpr (!MX) {
                    const h8_t v = __builtin_bit_cast(h8_t, pv);
                    float s0 = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
                    float s1 = ((float)v[4] + (float)v[5]) + ((float)v[6] + (float)v[7]);
                    s0 = s0 + fdpp<0xb1>(s0);  // quad_perm [1,0,3,2]
                    s1 = s1 + fdpp<0xb1>(s1);
                    s0 = s0 + fdpp<0x4e>(s0);  // quad_perm [2,3,0,1]
                    s1 = s1 + fdpp<0x4e>(s1);
                    s0 = s0 + fdpp<0x104>(s0);  // row_shl 4
                    s1 = s1 + fdpp<0x104>(s1);
                    if ((part & 7) == 0) {
                        const _Float16 h0 = (_Float16)s0, h1 = (_Float16)s1;
                        const _Float16 l0 = (_Float16)(s0 - (float)h0), l1 = (_Float16)(s1 - (float)h1);
                        const _Float16 z = (_Float16)0.0f;
                        opn[sbl * 36 + 32 + (part >> 3)] = __builtin_bit_cast(uint4, h8_t{h0, h1, l0, l1, z, z, z, z});
                    }
                }
            } else {
                const int key = multi ? -1 : slot;
                if (key < 0 || key != opb_key) gu_build(std::integral_constant<int, 5>{}, Me, off, 0, nph, ostr);
                opb_key = key;
            }
            __syncthreads();
        } else {
            // the slot's down operand, unless the previous item built it
            const int key = multi ? -1 : slot | 0x100000;
            if (key < 0 || key != opb_key) dn_build(Me, off, 0, nph, ostr, pdn);
            opb_key = key;
            __syncthreads();
        }
        const uint4* opr = pre && !dn ? opn : opb + rs * ostr;
        // one super-block step; j: the weight ring slot
        auto step = [&](int sb, auto jc) {
            constexpr int j = decltype(jc)::value;
            const int pf = sb + 1;
            const bool pnx = pf >= nsb;
            w[(j + 1) & 1] = load_w(pnx ? nrs : wrs, (pnx ? pf - nsb : pf) * CHK);
            // each item claims its successor four super-blocks before its
            // end (issued after this step's loads; its value is first used
            // at the publication one step later, so the wait for it there
            // leaves the next step's weight loads in flight)
            if (claims && sb == nsb - 4 && tid == 0) claimed = atomicAdd(fa.claim, 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(opr + (sb & (nph - 1)) * 36, w[j], acc);
            if (sb == nsb - 3) {
                if (tid == 0) s_claim = claim_item(G + claimed);
                __syncthreads();  // publishes s_claim
            }
        };
        using J0 = std::integral_constant<int, 0>;
        using J1 = std::integral_constant<int, 1>;
        for (int sb0 = 0; sb0 < nsb - 2; sb0 += 2) {
            if (multi && sb0 > 0 && (sb0 & (nph - 1)) == 0) {
                // the operand's next phase (nph is even: the phases start at
                // even super-blocks, before the last two)
                __syncthreads();
                if (dn) {
                    if constexpr (!SMALL && kFuTD > 8) dn_build(Me, off, sb0, nph, ostr, false);
                } else {
                    gu_build(std::integral_constant<int, SMALL ? FST_FU_NB_SMALL : FST_FU_NB>{}, Me, off, sb0, nph, ostr);
                }
                __syncthreads();
            }
            step(sb0, J0{});
            step(sb0 + 1, J1{});
        }
        step(nsb - 2, J0{});
        // the next item (published two super-blocks earlier) and the operand
        // prefetch of a one-token gate||up item
        tn = pair1 ? t + 1 : (dyn ? s_claim : t + G);
        tn = tn < total ? tn : total;
        if (tn < total) nrs = item_rsrc(tn);
        {
            const int nsl = tn < ngu ? tn / tiles_gu : 0;
            pre = tn < ngu && r_sM[nsl] == 1;
            const int tok = r_ptok[r_soff[nsl]];
            pv = reinterpret_cast<const u4v_t*>(fa.A)[tok * (hd / 8) + tid];
            // a one-token down item of another slot: its first poll's words
            // (one straight path: clamped to word 0 otherwise)
            int dsl = 0, dti = 0;
            if (tn >= ngu && tn < total) dn_map(tn - ngu, dsl, dti);
            // (not in the 8-token instantiation: measured slower there)
            const bool nd = !SMALL && tn >= ngu && tn < total && !(dn && dsl == slot) && dtab_m[dsl] == 1;
            const int doff = nd ? dtab_o[dsl] : 0;
            const int ql = tid & 255;
            const int ho = nd ? h_off(doff, 0, ql, ql >> 5, tid >> 8) : 0;
            pd[0] = __builtin_amdgcn_raw_buffer_load_b128(hrs, ho, 0, 16);
            pd[1] = __builtin_amdgcn_raw_buffer_load_b128(hrs, nd ? ho + 16 : 0, 0, 16);
            if constexpr (!MX) pm = __builtin_amdgcn_raw_buffer_load_b128(ars, nd && 2 * tid < aw ? (doff * aw + 2 * tid) * 8 : 0, 0, 16);
            pdn = nd;
        }
        __builtin_amdgcn_sched_barrier(0);
        step(nsb - 1, J1{});
        wrs = nrs;

        // D layout: lane holds token rows 4g+i (i = 0..3), column r
        if (!dn) {
            // gate waves hand their rows to the up waves through LDS
            if (wave < kFuHalf) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tl = 4 * g + i;
                    xg[(wave * 4 + i) * 64 + lane] =
                        tl < Me ? (MX ? acc[i] : ldexpf(acc[i], s_xs[r_ptok[off + tl]])) : 0.0f;
                }
            }
            __syncthreads();
            if (wave >= kFuHalf) {
                const int n = (tile * kFuHalf + wave - kFuHalf) * 16 + r;
                const float lim = fa.swiglu_limit;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tl = 4 * g + i;
                    float m = 0.0f;
                    if (tl < Me) {
                        float gv = xg[((wave - kFuHalf) * 4 + i) * 64 + lane];
                        float uv = MX ? acc[i] : ldexpf(acc[i], s_xs[r_ptok[off + tl]]);
                        if (lim > 0.0f) {
                            gv = fminf(gv, lim);
                            uv = fminf(fmaxf(uv, -lim), lim);
                        }
                        const float hv = (gv / (1.0f + expf(-gv))) * uv;
                        st_coherent_u64(fa.hbuf + (size_t)(off + tl) * inter + n,
                                        ((unsigned long long)epoch << 32) | fst_f32_bits(hv));
                        m = fabsf(hv);
                    }
                    if (MX) continue;    // bf16 operands: no prescale, no maxima
                    m = row16_fmax(m);  // the 16 rows of this wave
                    if (r == 0 && tl < Me)
                        st_coherent_u64(fa.amaxw + (size_t)(off + tl) * aw + (n >> 4),
                                        ((unsigned long long)epoch << 32) | fst_f32_bits(m));
                }
            }
        } else {
            const int row = (tile * kFuW + wave) * 16 + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tl = 4 * g + i;
                if (tl < Me) fa.y[(size_t)r_yrow[off + tl] * hd + row] = MX ? acc[i] : ldexpf(acc[i], s_xs2[tl]);
            }
        }
    }
}

int launch_moe_fused(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                     const RouteReq& rq, uint32_t epoch, int spin_limit, const uint16_t* h, hipEvent_t ev0,
                     hipEvent_t ev1) {
    RouteArgs ra = route_args(g, L, M, s.logits, rq.input_ids, rq.use_hash, rq.use_shared, rq.eids, rq.wts, s);
    if (rq.given) ra.given = rq.eids;
    FusedArgs fa{};
    fa.bank = L.bank;
    fa.expert_stride = L.expert_stride;
    // Q4_K: the fp16 operand the router launch prepared; MXFP4: the bf16 input rows
    fa.A = g.codec == 1 ? reinterpret_cast<const _Float16*>(h) : s.x16p;
    fa.SX = s.sxp;
    fa.xs = s.xs;
    fa.hbuf = s.hbuf;
    fa.amaxw = s.amaxw;
    fa.hbuf_bytes = (size_t)s.max_pairs * g.inter * 8;
    fa.y = s.y;
    fa.claim = s.fused_claim;
    fa.swiglu_limit = g.swiglu_limit;
    fa.epoch = epoch;
    fa.spin_limit = spin_limit;
    // as many workgroups per CU as the occupancy calculator says fit (two:
    // the kernel's VGPR and LDS budget allows two), all resident at once
    // (the down items' waits rely on it)
    const unsigned items = (unsigned)s.max_slots * (unsigned)(g.inter / 64 + g.hd / 128);
    const dim3 grid(std::min(items, (unsigned)s.n_cu * (unsigned)std::max(1, s.fused_per_cu)));
    fa.singles = (int)grid.x;
    // with events: they take the dispatch's own start and end times (the
    // kernel's duration, without the gap to the previous launch)
#define FST_FU(C, SM)                                                                                         \
    do {                                                                                                        \
        if (ev0)                                                                                                \
            hipExtLaunchKernelGGL((moe_fused_kernel<4096, 2048, C, SM>), grid, dim3(64 * kFuW), 0, st, ev0, ev1, 0, \
                                  fa, ra);                                                                      \
        else                                                                                                    \
            hipLaunchKernelGGL((moe_fused_kernel<4096, 2048, C, SM>), grid, dim3(64 * kFuW), 0, st, fa, ra);     \
    } while (0)
    // (at most 8 tokens: no slot holds more than 8)
    const bool small = M <= 8;
    if (g.hd == 4096 && g.inter == 2048 && g.codec == 1) {
        if (small)
            FST_FU(1, true);
        else
            FST_FU(1, false);
    } else if (g.hd == 4096 && g.inter == 2048) {
        if (small)
            FST_FU(0, true);
        else
            FST_FU(0, false);
    } else {
        return set_error(1, "fused MoE launch: geometry without an instantiation");
    }
#undef FST_FU
    return 0;
}

int moe_fused_occupancy(int codec) {
    int n = 0;
    // (the smaller of the two instantiations' figures)
    int n2 = 0;
    const hipError_t e =
        codec == 1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, moe_fused_kernel<4096, 2048, 1, false>, 64 * kFuW, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, moe_fused_kernel<4096, 2048, 0, false>, 64 * kFuW, 0);
    const hipError_t e2 =
        codec == 1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n2, moe_fused_kernel<4096, 2048, 1, true>, 64 * kFuW, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n2, moe_fused_kernel<4096, 2048, 0, true>, 64 * kFuW, 0);
    if (e != hipSuccess || e2 != hipSuccess) return 0;
    return std::min(std::min(n, n2), 2);
}

bool moe_fused_supported(const Geometry& g, int M) {
    // instantiated for the DeepSeek-V4-Flash-like expert (4096 -> 2048 -> 4096)
    return (g.codec == 0 || g.codec == 1) && M <= kFuMaxM && M * g.tk <= kFuMaxPairs &&
           g.E <= kFusedRouteMaxExperts && g.hd == 4096 && g.inter == 2048;
}

// Token capacity of the launch (the call's M bounds every slot's M_e): 8, 16,
// 32 or 64 tokens; smaller capacities stage more super-blocks per barrier.
#ifndef FST_Q4K_WG_PER_CU
#define FST_Q4K_WG_PER_CU 2
#endif
#ifndef FST_Q4K_W
#define FST_Q4K_W 8
#endif
#ifndef FST_Q4K_W16
#define FST_Q4K_W16 16
#endif
#ifndef FST_Q4K_W32
#define FST_Q4K_W32 16
#endif
// Waves per workgroup of the linear kernel by token capacity (larger
// capacities stage more operand chunks per super-block; more threads hold
// fewer each), when N is a multiple of the workgroup's 16*W rows.
static int linear_waves(int M, int N) {
    const int WC = M <= 8 ? FST_Q4K_W : (M <= 16 ? FST_Q4K_W16 : (M <= 32 ? FST_Q4K_W32 : FST_Q4K_W));
    return N % (16 * WC) == 0 ? WC : FST_Q4K_W;
}
// Resident waves per CU the persistent grid is sized for.
static int linear_waves_per_cu(int M) {
    return 8 * (M <= 8 ? FST_Q4K_WG_PER_CU : (M <= 32 && FST_Q4K_WPE_MID >= 4 ? 2 : 1));
}

template <int MODE, int CODEC = 0, int RPER = 0>
static void launch_q4k_linear(hipStream_t st, int M, unsigned slots, const uint8_t* bank, size_t stride,
                              size_t mat_off, int K, int N, const Scratch& s, const int* a_row,
                              const _Float16* A, const uint4* SX, const int* xs, float* out, const EpiArgs& ep,
                              const RouteArgs& ra = RouteArgs{}) {

    if constexpr (MODE == 0 && CODEC == 0 && RPER == 0) {
        if (M > 16 && M <= 32 && N % 256 == 0) {
            // 32x32 tiles: 8 waves x 32 rows per item, one workgroup per CU (the
            // tile's accumulators need more than 128 VGPRs)
            const unsigned items32 = slots * (unsigned)(N / 256);
            hipLaunchKernelGGL((q4k_linear_kernel<32, 1, 8, MODE, CODEC, RPER, FST_MF32_PF, true>),
                               dim3(std::min(items32, (unsigned)s.n_cu * (FST_MF32_WPE >= 4 ? 2u : 1u))), dim3(512), 0, st, bank, stride,
                               mat_off, K, N, s.meta, s.slot_eid, s.slot_M, s.slot_off, a_row, A, SX, xs, out, ep,
                               ra);
            return;
        }
    }
    const int W = linear_waves(M, N);
    // persistent grid: FST_Q4K_WG_PER_CU workgroups per CU at most
    const unsigned items = slots * (unsigned)(N / (16 * W)) * (unsigned)(MODE == 1 ? std::max(ep.ksplit, 1) : 1);
    const unsigned waves_per_cu = (unsigned)linear_waves_per_cu(M);
    const dim3 grid(std::min(items, (unsigned)s.n_cu * std::max(1u, waves_per_cu / (unsigned)W)));
#define FST_Q4K_LAUNCH_W(T, MSV, WV)                                                                         \
    hipLaunchKernelGGL((q4k_linear_kernel<T, MSV, WV, MODE, CODEC, RPER>), grid, dim3(64 * WV), 0, st, bank,    \
                       stride, mat_off, K, N, s.meta, s.slot_eid, s.slot_M, s.slot_off, a_row, A, SX, xs, out, ep, \
                       ra)
#define FST_Q4K_LAUNCH(T, MSV) FST_Q4K_LAUNCH_W(T, MSV, FST_Q4K_W)
    // K is a multiple of 512 (checked at context creation): nsb is even
#ifndef FST_MS8
#define FST_MS8 1
#endif
#ifndef FST_MS8_DN
#define FST_MS8_DN 2
#endif
    constexpr int ms8 = MODE == 2 ? FST_MS8_DN : FST_MS8;
    if (M <= 8 && (K >> 8) % ms8 == 0)
        FST_Q4K_LAUNCH(8, ms8);
    else if (M <= 8)
        FST_Q4K_LAUNCH(8, 2);
#ifndef FST_MS16
#define FST_MS16 2
#endif
#ifndef FST_MS32
#define FST_MS32 1
#endif
    else if (M <= 16 && W == FST_Q4K_W16)
        FST_Q4K_LAUNCH_W(16, FST_MS16, FST_Q4K_W16);
    else if (M <= 16)
        FST_Q4K_LAUNCH(16, 2);
    else if (M <= 32 && W == FST_Q4K_W32)
        FST_Q4K_LAUNCH_W(32, FST_MS32, FST_Q4K_W32);
    else if (M <= 32)
        FST_Q4K_LAUNCH(32, 1);
    else
        FST_Q4K_LAUNCH(64, 1);
#undef FST_Q4K_LAUNCH
#undef FST_Q4K_LAUNCH_W
}

// gate||up: the two [inter][hd/K-block] matrices are contiguous; each
// workgroup takes 64 gate rows and the same 64 up rows and writes
// h = silu(gate)*up (fp32 for Q4_K, bf16 for MXFP4).  The Q4_K operand is the
// prescaled fp16 one (router_prep); MXFP4 stages the bf16 rows of h_in as is.
int launch_q4k_gate_up(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                       const uint16_t* h_in, const RouteReq* rq, int slots_bound, int pairs_bound) {
    // split-K when the call's (slot, tile) items would leave most of the
    // persistent grid idle: more, shorter items (each wave's chain of
    // dependent super-block loads gets shorter); Q4_K only (the prep launch
    // adds the partials up), at most 8 ways, 2 super-blocks per item at least
    int ksplit = 1;
    if (g.codec == 0 && slots_bound > 0 && pairs_bound > 0) {
        const int N = 2 * g.inter, W = linear_waves(M, N);
        const long items = (long)slots_bound * (N / (16 * W));
        const long cap = (long)s.n_cu * std::max(1, linear_waves_per_cu(M) / W);
        const int nsb_row = g.hd >> 8;
        while (ksplit < 8 && items * ksplit * 2 <= cap && 2L * ksplit * 2 * pairs_bound <= s.max_pairs &&
               nsb_row % (ksplit * 4) == 0)
            ksplit *= 2;
    }
    const int part_rows = pairs_bound;
    EpiArgs ep{};
    ep.swiglu_limit = g.swiglu_limit;
    ep.h = s.act;
    ep.h16 = reinterpret_cast<uint16_t*>(s.a16p);
    ep.ksplit = ksplit;
    ep.part = s.act;
    ep.part_rows = part_rows;
    const unsigned S = (unsigned)s.max_slots;
    const _Float16* hx = reinterpret_cast<const _Float16*>(h_in);
    if (rq && g.E <= kFusedRouteMaxExperts) {
        static_assert(kFusedRouteMaxExperts == 64 * 4, "4 experts per lane");
        const RouteArgs ra = route_args(g, L, M, s.logits, rq->input_ids, rq->use_hash, rq->use_shared, rq->eids,
                                        rq->wts, s);
        if (g.codec == 1)
            launch_q4k_linear<1, 1, 4>(st, M, S, L.bank, L.expert_stride, 0, g.hd, 2 * g.inter, s, s.pair_tok, hx,
                                       nullptr, nullptr, nullptr, ep, ra);
        else
            launch_q4k_linear<1, 0, 4>(st, M, S, L.bank, L.expert_stride, 0, g.hd, 2 * g.inter, s, s.pair_tok,
                                       s.x16p, s.sxp, s.xs, nullptr, ep, ra);
        return ksplit;
    }
    if (g.codec == 1)
        launch_q4k_linear<1, 1>(st, M, S, L.bank, L.expert_stride, 0, g.hd, 2 * g.inter, s, s.pair_tok, hx, nullptr,
                                nullptr, nullptr, ep);
    else
        launch_q4k_linear<1>(st, M, S, L.bank, L.expert_stride, 0, g.hd, 2 * g.inter, s, s.pair_tok, s.x16p, s.sxp,
                             s.xs, nullptr, ep);
    return ksplit;
}

// down: y[pair][n] (fp32) for every (token, expert) pair of the call.
void launch_q4k_down(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                     const float* wts, uint16_t* o1, uint16_t* o2) {
    const size_t proj = g.codec == 1 ? (size_t)g.inter * (g.hd / 32) * 17 : (size_t)g.inter * (g.hd / 256) * 144;
    EpiArgs ep{};
    if (o1 || o2) {
        ep.wts = wts;
        ep.pair_tok = s.pair_tok;
        ep.o1 = o1;
        ep.o2 = o2;
    }
    if (g.codec == 1)
        launch_q4k_linear<2, 1>(st, M, (unsigned)s.max_slots, L.bank, L.expert_stride, 2 * proj, g.inter, g.hd,
                                s, nullptr, s.a16p, nullptr, nullptr, s.y, ep);
    else
        launch_q4k_linear<2>(st, M, (unsigned)s.max_slots, L.bank, L.expert_stride, 2 * proj, g.inter, g.hd, s,
                             nullptr, s.a16p, s.sx2p, s.xs2, s.y, ep);
}

// Dense Q4_K linear over M rows (the LM head): logits[m][n] = sum_k W[n][k] x[m][k],
// operand prepared by launch_resid_norm with `prep` and `slot_tab`.
void launch_q4k_dense(hipStream_t st, const uint8_t* W, int M, int K, int N, const Scratch& s, int* slot_tab,
                      float* out) {
    Scratch t = s;
    t.meta = slot_tab;
    t.slot_eid = slot_tab + META_WORDS;
    t.slot_M = slot_tab + META_WORDS + 1;
    t.slot_off = slot_tab + META_WORDS + 2;
    launch_q4k_linear<0>(st, M, 1u, W, 0, 0, K, N, t, nullptr, s.x16p, s.sxp, s.xs, out, EpiArgs{});
}


// ------------------------------------------------------------------ combine

// src/fst_engine.cpp:4196-4201 and :2851-2852: out = bf16(sum_j w[t][j] y[pair(t,j)]
// + y_shared[t]), fp32 accumulation in slot order j = 0..tk-1, then the shared
// term (weight 1.0), one RNE rounding.  The shared term is its pair's row of y,
// or row t of ys when the shared expert ran from bf16 weights.  One thread per
// 4 consecutive columns of one token.
template <int TK>
__global__ __launch_bounds__(256) void combine_kernel(int M, int hd, int tk, int use_shared,
                                                      const float* __restrict__ y,
                                                      const int* __restrict__ pair_of,
                                                      const int* __restrict__ pair_shared,
                                                      const float* __restrict__ ys,
                                                      const float* __restrict__ wts,
                                                      uint16_t* __restrict__ out,
                                                      uint16_t* __restrict__ out_routed,
                                                      uint16_t* __restrict__ out_shared) {
    const int t = blockIdx.y;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (t >= M || n >= hd) return;
    // every load issued before the sums (slots past tk or without a pair
    // read row 0 of y and are not summed; with tk = 0, a shared-only call,
    // no routing entry is read at all)
    int p[TK];
    float w[TK];
#pragma unroll
    for (int j = 0; j < TK; ++j) {
        const int jj = t * tk + max(min(j, tk - 1), 0);
        p[j] = tk > 0 ? pair_of[jj] : -1;
        w[j] = tk > 0 ? wts[jj] : 0.0f;
    }
    float4 v[TK];
#pragma unroll
    for (int j = 0; j < TK; ++j) v[j] = *reinterpret_cast<const float4*>(y + (size_t)max(p[j], 0) * hd + n);
    const float4 vs = use_shared ? *reinterpret_cast<const float4*>((ys ? ys + (size_t)t * hd : y + (size_t)pair_shared[t] * hd) + n)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < TK; ++j) {
        if (j >= tk || p[j] < 0) continue;
        a.x = a.x + w[j] * v[j].x;
        a.y = a.y + w[j] * v[j].y;
        a.z = a.z + w[j] * v[j].z;
        a.w = a.w + w[j] * v[j].w;
    }
    auto put = [&](uint16_t* o, const float4& v) {
        if (!o) return;
        const uint32_t lo = fst_f32_to_bf16(v.x) | ((uint32_t)fst_f32_to_bf16(v.y) << 16);
        const uint32_t hi = fst_f32_to_bf16(v.z) | ((uint32_t)fst_f32_to_bf16(v.w) << 16);
        *reinterpret_cast<uint2*>(o + (size_t)t * hd + n) = make_uint2(lo, hi);
    };
    put(out_routed, a);
    if (use_shared) {
        put(out_shared, vs);
        a.x = a.x + vs.x;
        a.y = a.y + vs.y;
        a.z = a.z + vs.z;
        a.w = a.w + vs.w;
    }
    put(out, a);
}

// The combine of the fused launch: y rows by (token, j) (j = tk: the shared
// expert), so every load is issued at once; same arithmetic as combine_kernel.
// Columns n..n+3 of token t: a = the routed pairs' weighted sum (slot order
// j = 0..tk-1), vs = the shared term.
template <int TK>
__device__ __forceinline__ void combine_tj_cols(int t, int n, int hd, int tk, int use_shared,
                                                const float* __restrict__ y, const float* __restrict__ ys,
                                                const float* __restrict__ wts, float4& a, float4& vs) {
    float w[TK];
    float4 v[TK];
#pragma unroll
    for (int j = 0; j < TK; ++j) {
        const int jj = max(min(j, tk - 1), 0);
        w[j] = tk > 0 ? wts[t * tk + jj] : 0.0f;
        v[j] = *reinterpret_cast<const float4*>(y + ((size_t)t * (tk + 1) + jj) * hd + n);
    }
    vs = use_shared ? *reinterpret_cast<const float4*>((ys ? ys + (size_t)t * hd : y + ((size_t)t * (tk + 1) + tk) * hd) + n)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < TK; ++j) {
        if (j >= tk) continue;
        a.x = a.x + w[j] * v[j].x;
        a.y = a.y + w[j] * v[j].y;
        a.z = a.z + w[j] * v[j].z;
        a.w = a.w + w[j] * v[j].w;
    }
}

template <int TK>
__global__ __launch_bounds__(256) void combine_tj_kernel(int M, int hd, int tk, int use_shared,
                                                         const float* __restrict__ y, const float* __restrict__ ys,
                                                         const float* __restrict__ wts, uint16_t* __restrict__ out,
                                                         uint16_t* __restrict__ out_routed,
                                                         uint16_t* __restrict__ out_shared) {
    const int t = blockIdx.y;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (t >= M || n >= hd) return;
    float4 a, vs;
    combine_tj_cols<TK>(t, n, hd, tk, use_shared, y, ys, wts, a, vs);
    auto put = [&](uint16_t* o, const float4& q) {
        if (!o) return;
        const uint32_t lo = fst_f32_to_bf16(q.x) | ((uint32_t)fst_f32_to_bf16(q.y) << 16);
        const uint32_t hi = fst_f32_to_bf16(q.z) | ((uint32_t)fst_f32_to_bf16(q.w) << 16);
        *reinterpret_cast<uint2*>(o + (size_t)t * hd + n) = make_uint2(lo, hi);
    };
    put(out_routed, a);
    if (use_shared) {
        put(out_shared, vs);
        a.x = a.x + vs.x;
        a.y = a.y + vs.y;
        a.z = a.z + vs.z;
        a.w = a.w + vs.w;
    }
    put(out, a);
}

// The combine of a verify-forward layer with the next layer's residual add
// and RMSNorm folded in (process_layer's order, include/fst_engine.h:308:
// h += out, then mn = RMSNorm(h) for the next layer).  Grid (hd / 1024, M):
// workgroup c of token t combines columns [1024c, 1024c + 1024) as
// combine_tj_kernel does, rounds out to bf16, forms x = bf16(h + out) as
// resid_norm_kernel does, writes x back to h (device-coherent 8-byte stores)
// and the double sums of squares of its hd/64-element lane chunks (lanes
// 1024c/(hd/64) on; each chunk summed in order, as resid_norm_kernel's lane
// does) to npart.  The token's last workgroup to arrive (ncnt, left at zero)
// runs resid_norm_kernel's halving tree over the 64 partials and writes
// mn = bf16((x * r) * w) for the whole row: the same bits as combine_tj_kernel
// followed by resid_norm_kernel.
template <int TK>
__global__ __launch_bounds__(256) void combine_norm_tj_kernel(int M, int hd, int tk, int use_shared,
                                                              const float* __restrict__ y,
                                                              const float* __restrict__ ys,
                                                              const float* __restrict__ wts, uint16_t* h,
                                                              const uint16_t* __restrict__ w, float eps,
                                                              uint16_t* __restrict__ normed,
                                                              unsigned long long* npart, int* ncnt) {
    __shared__ float xl[1024 + 1024 / 64];  // this workgroup's x, one pad word per 64
    __shared__ int s_last;
    __shared__ float s_r;
    auto xi = [](int e) { return e + (e >> 6); };
    const int t = blockIdx.y, tid = threadIdx.x;
    const int n = blockIdx.x * 1024 + tid * 4;
    float4 a, vs;
    combine_tj_cols<TK>(t, n, hd, tk, use_shared, y, ys, wts, a, vs);
    if (use_shared) {
        a.x = a.x + vs.x;
        a.y = a.y + vs.y;
        a.z = a.z + vs.z;
        a.w = a.w + vs.w;
    }
    const float av[4] = {a.x, a.y, a.z, a.w};
    unsigned long long* hrow = reinterpret_cast<unsigned long long*>(h + (size_t)t * hd);
    const unsigned long long hv = hrow[n / 4];
    unsigned long long xw = 0ull;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float o = fst_bf16_to_f32(fst_f32_to_bf16(av[k]));
        const uint16_t xb = fst_f32_to_bf16(fst_bf16_to_f32((uint16_t)(hv >> (16 * k))) + o);
        xl[xi(4 * tid + k)] = fst_bf16_to_f32(xb);
        xw |= (unsigned long long)xb << (16 * k);
    }
    st_coherent_u64(hrow + n / 4, xw);
    __syncthreads();
    const int C = hd / 64, nl = 1024 / C;  // elements per lane chunk, chunks of this workgroup
    if (tid < nl) {
        double s = 0.0;
        for (int i = 0; i < C; ++i) {
            const double v = (double)xl[xi(tid * C + i)];
            s = __dadd_rn(s, __dmul_rn(v, v));
        }
        st_coherent_u64(npart + (size_t)t * 64 + blockIdx.x * nl + tid, (unsigned long long)__double_as_longlong(s));
    }
    publish_wait();
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(ncnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (int)gridDim.x - 1;
        if (s_last) __hip_atomic_store(ncnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    if (tid < 64) {
        double s = __longlong_as_double((long long)ld_coherent_u64(npart + (size_t)t * 64 + tid));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_down(s, off, 64);
        if (tid == 0) s_r = (float)(1.0 / sqrt(s / (double)hd + (double)eps));
    }
    __syncthreads();
    const float r = s_r;
    for (int q = tid; q < hd / 4; q += 256) {
        const unsigned long long xq = ld_coherent_u64(hrow + q);
        const uint2 wq = reinterpret_cast<const uint2*>(w)[q];
        const uint32_t ww[2] = {wq.x, wq.y};
        uint32_t o[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t o2 = 0u;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const float x = fst_bf16_to_f32((uint16_t)(xq >> (32 * i + 16 * hh)));
                o2 |= (uint32_t)fst_f32_to_bf16((x * r) * fst_bf16_to_f32((uint16_t)(ww[i] >> (16 * hh)))) << (16 * hh);
            }
            o[i] = o2;
        }
        reinterpret_cast<uint2*>(normed + (size_t)t * hd)[q] = make_uint2(o[0], o[1]);
    }
}

bool combine_norm_supported(const Geometry& g) { return g.hd % 1024 == 0 && 65536 % g.hd == 0; }

void launch_combine_norm_tj(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s,
                            const float* wts, const float* ys, uint16_t* h, const uint16_t* w, float eps,
                            uint16_t* normed) {
    dim3 grid(g.hd / 1024, M);
#define FST_CN(T)                                                                                              \
    hipLaunchKernelGGL(combine_norm_tj_kernel<T>, grid, dim3(256), 0, st, M, g.hd, g.tk, use_shared, s.y, ys, wts, \
                       h, w, eps, normed, s.norm_part, s.norm_cnt)
    if (g.tk <= 8)
        FST_CN(8);
    else
        FST_CN(kMaxTopK);
#undef FST_CN
}

void launch_combine_tj(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s, const float* wts,
                       const float* ys, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared) {
    dim3 grid((g.hd / 4 + 255) / 256, M);
#define FST_COMB(T)                                                                                        \
    hipLaunchKernelGGL(combine_tj_kernel<T>, grid, dim3(256), 0, st, M, g.hd, g.tk, use_shared, s.y, ys, wts, \
                       out, out_routed, out_shared)
    if (g.tk <= 8)
        FST_COMB(8);
    else
        FST_COMB(kMaxTopK);
#undef FST_COMB
}

void launch_combine(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s,
                    const float* wts, const float* ys, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared) {
    dim3 grid((g.hd / 4 + 255) / 256, M);
#define FST_COMB(T)                                                                                              \
    hipLaunchKernelGGL(combine_kernel<T>, grid, dim3(256), 0, st, M, g.hd, g.tk, use_shared, s.y, s.pair_of, \
                       s.pair_shared, ys, wts, out, out_routed, out_shared)
    if (g.tk <= 8)
        FST_COMB(8);
    else
        FST_COMB(kMaxTopK);
#undef FST_COMB
}

// --------------------------------------------------------------------- copy

__global__ __launch_bounds__(256) void copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                   size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        dst[i] = src[i];
}

void launch_copy(hipStream_t st, void* dst, const void* src, size_t bytes) {
    const size_t n16 = bytes / 16;
    const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256, 256 * 64);
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, st, (uint4*)dst, (const uint4*)src, n16);
}

// ------------------------------------------------------------------ dequant

// kernels/fst_dequant_q4k_kernel.cc:40-100 semantics in binary32 (see oracle).
__global__ __launch_bounds__(256) void dequant_q4k_kernel(const uint8_t* __restrict__ blocks,
                                                          size_t nblocks, float* __restrict__ of,
                                                          uint16_t* __restrict__ ob) {
    const size_t b = blockIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = blocks + b * 144;
    const int i = threadIdx.x, j = i >> 5, ii = i & 31;
    const float d = fst_fp16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float dmin = fst_fp16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    const uint8_t* q = blk + 4;
    int sc, m;
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
    const uint8_t byte = blk[16 + 32 * (j >> 1) + ii];
    const int nib = (j & 1) ? (byte >> 4) : (byte & 15);
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
    const float v = __fsub_rn(__fmul_rn(d1, (float)nib), m1);
    if (of) of[b * 256 + i] = v;
    if (ob) ob[b * 256 + i] = fst_f32_to_bf16(v);
}

__global__ __launch_bounds__(256) void dequant_mxfp4_kernel(const uint8_t* __restrict__ blocks,
                                                            size_t nblocks, float* __restrict__ of,
                                                            uint16_t* __restrict__ ob) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t b = idx >> 5;
    if (b >= nblocks) return;
    const int i = idx & 31;
    const uint8_t* blk = blocks + b * 17;
    const int e = blk[0];
    const float s = (e == 0 || e == 255) ? 0.0f : ldexpf(1.0f, e - 127);
    const uint8_t byte = blk[1 + (i >> 1)];
    const int nib = (i & 1) ? (byte >> 4) : (byte & 15);
    const float lut[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const float mag = lut[nib & 7];
    const float sv = (nib & 8) ? (0.0f - mag) : mag;  // code 8 is +0 as in the kernel LUT
    const float v = __fmul_rn(sv, s);
    if (of) of[idx] = v;
    if (ob) ob[idx] = fst_f32_to_bf16(v);
}

void launch_dequant(hipStream_t st, int codec, const uint8_t* blocks, size_t nblocks, float* out_f32,
                    uint16_t* out_bf16) {
    if (codec == 0) {
        hipLaunchKernelGGL(dequant_q4k_kernel, dim3((unsigned)nblocks), dim3(256), 0, st, blocks, nblocks,
                           out_f32, out_bf16);
    } else {
        size_t n = nblocks * 32;
        hipLaunchKernelGGL(dequant_mxfp4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           blocks, nblocks, out_f32, out_bf16);
    }
}

}  // namespace fst
