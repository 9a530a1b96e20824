// fst_moe.hip — MoE-layer verify kernels for gfx950 (MI355X).
//
// One MoE layer call is a fixed chain of stream-ordered launches with no host
// round trip:
//   router_logits   h[M,K] . W_r  (canonical fp32 order, bit-exact vs the CPU oracle)
//   route_bucket    top-k + weights, then (token, expert) pairs grouped per expert
//   prep_bf16       activations -> power-of-two prescaled fp16 operand tiles
//   q4k_ffn<gate|up> fused Q4_K decode + MFMA gate/up + SiLU*up  -> act[pair][inter]
//   prep_act        act -> fp16 operand tiles
//   q4k_ffn<down>   fused Q4_K decode + MFMA down                  -> y[pair][hidden]
//   combine         out[t] = sum_j w[t][j] y[pair(t,j)] + y[shared(t)]  (fixed order)
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
#include "fst_internal.h"
#include "../../include/fst_exact_math.h"

namespace fst {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ float half_bits_to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// ---------------------------------------------------------------- router

// One wave per expert: lane j owns the contiguous K/64 chunk j, sums it with a
// sequential fmaf chain, then the 64 partials are combined by the halving
// tree p[j] += p[j+off] (off = 32..1) that lane 0 sees through shfl_down.
template <int CH>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ w_nk,
                                                            const uint16_t* __restrict__ h, int M,
                                                            int K, int E, float* __restrict__ logits) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + wave;
    if (e >= E) return;
    float wv[CH];
    const uint4* wp = reinterpret_cast<const uint4*>(w_nk + (size_t)e * K + (size_t)lane * CH);
#pragma unroll
    for (int i = 0; i < CH / 8; ++i) {
        uint4 u = wp[i];
        uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            wv[8 * i + 2 * k] = fst_bits_f32(q[k] << 16);
            wv[8 * i + 2 * k + 1] = fst_bits_f32(q[k] & 0xffff0000u);
        }
    }
    for (int t = 0; t < M; ++t) {
        const uint4* xp = reinterpret_cast<const uint4*>(h + (size_t)t * K + (size_t)lane * CH);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < CH / 8; ++i) {
            uint4 u = xp[i];
            uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc = fmaf(fst_bits_f32(q[k] << 16), wv[8 * i + 2 * k], acc);
                acc = fmaf(fst_bits_f32(q[k] & 0xffff0000u), wv[8 * i + 2 * k + 1], acc);
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_down(acc, off, 64);
        if (lane == 0) logits[(size_t)t * E + e] = acc;
    }
}

void launch_router_logits(hipStream_t st, const Geometry& g, const LayerView& L, const uint16_t* h,
                          int M, float* logits) {
    dim3 grid((g.E + 3) / 4);
    if (g.hd == 4096)
        hipLaunchKernelGGL(router_logits_kernel<64>, grid, dim3(256), 0, st, L.router_nk, h, M, g.hd,
                           g.E, logits);
    else if (g.hd == 2048)
        hipLaunchKernelGGL(router_logits_kernel<32>, grid, dim3(256), 0, st, L.router_nk, h, M, g.hd,
                           g.E, logits);
    else if (g.hd == 1024)
        hipLaunchKernelGGL(router_logits_kernel<16>, grid, dim3(256), 0, st, L.router_nk, h, M, g.hd,
                           g.E, logits);
    else
        hipLaunchKernelGGL(router_logits_kernel<8>, grid, dim3(256), 0, st, L.router_nk, h, M, g.hd,
                           g.E, logits);
}

// ------------------------------------------------------------ route + bucket

struct Cand {
    float sel, score;
    int id;  // INT_MAX: empty
};

__device__ __forceinline__ bool cand_better(const Cand& a, const Cand& b) {
    if (a.id == 0x7fffffff) return false;
    if (b.id == 0x7fffffff) return true;
    bool an = a.sel != a.sel, bn = b.sel != b.sel;
    if (an != bn) return bn;  // a number beats NaN
    if (!an && a.sel != b.sel) return a.sel > b.sel;
    return a.id < b.id;
}

constexpr int kMaxExperts = 1024;

// Single workgroup of 256 threads.  Part A: per-token top-k and weights
// (src/fst_engine.cpp:974-1061 semantics; ties toward the lower expert id).
// Part B: (token, expert) pairs grouped by expert in ascending expert id,
// tokens ascending within an expert; the shared expert gets the last slot.
__global__ __launch_bounds__(256) void route_bucket_kernel(
    int M, int E, int tk, int score_func, int round_bf16, float route_scale,
    const float* __restrict__ logits, const float* __restrict__ bias,
    const int32_t* __restrict__ hash, const int32_t* __restrict__ ids, int vocab, int do_topk,
    int use_shared, int32_t* __restrict__ eids, float* __restrict__ wts, int* __restrict__ meta,
    int* __restrict__ slot_eid, int* __restrict__ slot_M, int* __restrict__ slot_off,
    int* __restrict__ pair_tok, int* __restrict__ pair_of, int* __restrict__ pair_shared) {
    __shared__ unsigned long long hitmask[kMaxExperts];
    __shared__ int eoff[kMaxExperts];
    __shared__ int wave_tot[2][4];
    __shared__ int err;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) err = 0;

    if (do_topk) {
        for (int t = wave; t < M; t += 4) {
            const float* row = logits + (size_t)t * E;
            if (hash) {
                int tok = ids ? ids[t] : -1;
                if (lane == 0) {
                    if (tok < 0 || tok >= vocab) {
                        atomicOr(&err, 2);
                        for (int k = 0; k < tk; ++k) {
                            eids[(size_t)t * tk + k] = -1;
                            wts[(size_t)t * tk + k] = 0.0f;
                        }
                    } else {
                        float sc[kMaxTopK];
                        float sum = 0.0f;
                        for (int k = 0; k < tk; ++k) {
                            int e = hash[(size_t)tok * tk + k];
                            float x = (e >= 0 && e < E) ? row[e] : 0.0f;
                            if (e < 0 || e >= E) atomicOr(&err, 1);
                            if (round_bf16) x = fst_bf16_to_f32(fst_f32_to_bf16(x));
                            sc[k] = score_func == 0 ? fst_sigmoidf(x) : fst_sqrtsoftplusf(x);
                            sum += sc[k];
                            eids[(size_t)t * tk + k] = e;
                        }
                        float inv = 1.0f / (sum + 1e-12f);
                        for (int k = 0; k < tk; ++k) wts[(size_t)t * tk + k] = sc[k] * inv * route_scale;
                    }
                }
                continue;
            }
            constexpr int PER = kMaxExperts / 64;
            Cand c[PER];
            int nper = (E + 63) / 64;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                int e = lane + 64 * i;
                c[i].id = 0x7fffffff;
                if (i < nper && e < E) {
                    float x = row[e];
                    if (round_bf16) x = fst_bf16_to_f32(fst_f32_to_bf16(x));
                    float s = score_func == 0 ? fst_sigmoidf(x) : fst_sqrtsoftplusf(x);
                    c[i].score = s;
                    c[i].sel = s + (bias ? bias[e] : 0.0f);
                    c[i].id = e;
                }
            }
            float chosen_sc[kMaxTopK];
            int chosen_id[kMaxTopK];
            for (int k = 0; k < tk; ++k) {
                Cand b;
                b.id = 0x7fffffff;
                b.sel = 0.0f;
                b.score = 0.0f;
#pragma unroll
                for (int i = 0; i < PER; ++i)
                    if (cand_better(c[i], b)) b = c[i];
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) {
                    Cand o;
                    o.sel = __shfl_xor(b.sel, off, 64);
                    o.score = __shfl_xor(b.score, off, 64);
                    o.id = __shfl_xor(b.id, off, 64);
                    if (cand_better(o, b)) b = o;
                }
                chosen_sc[k] = b.score;
                chosen_id[k] = b.id;
#pragma unroll
                for (int i = 0; i < PER; ++i)
                    if (c[i].id == b.id) c[i].id = 0x7fffffff;
            }
            if (lane == 0) {
                float sum = 0.0f;
                for (int k = 0; k < tk; ++k) sum += chosen_sc[k];
                float inv = 1.0f / (sum + 1e-12f);
                for (int k = 0; k < tk; ++k) {
                    eids[(size_t)t * tk + k] = chosen_id[k];
                    wts[(size_t)t * tk + k] = chosen_sc[k] * inv * route_scale;
                }
            }
        }
        __threadfence_block();
    }
    for (int e = tid; e < E; e += 256) hitmask[e] = 0ull;
    __syncthreads();
    for (int i = tid; i < M * tk; i += 256) {
        int t = i / tk;
        int e = eids[i];
        if (e < 0 || e >= E)
            atomicOr(&err, 1);
        else
            atomicOr(&hitmask[e], 1ull << t);
    }
    __syncthreads();
    // exclusive scans over experts of (active) and (count), 256 experts per pass
    int slot_base = 0, pair_base = 0;
    for (int e0 = 0; e0 < E; e0 += 256) {
        int e = e0 + tid;
        int cnt = (e < E) ? __popcll(hitmask[e]) : 0;
        int act = cnt > 0;
        int sa = act, sc = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            int ua = __shfl_up(sa, off, 64), uc = __shfl_up(sc, off, 64);
            if (lane >= off) { sa += ua; sc += uc; }
        }
        if (lane == 63) { wave_tot[0][wave] = sa; wave_tot[1][wave] = sc; }
        __syncthreads();
        int pa = slot_base, pc = pair_base;
        for (int w = 0; w < wave; ++w) { pa += wave_tot[0][w]; pc += wave_tot[1][w]; }
        int ex_a = pa + sa - act, ex_c = pc + sc - cnt;
        if (act) {
            slot_eid[ex_a] = e;
            slot_M[ex_a] = cnt;
            slot_off[ex_a] = ex_c;
            unsigned long long mk = hitmask[e];
            int r = 0;
            while (mk) {
                int t = __ffsll((long long)mk) - 1;
                pair_tok[ex_c + r] = t;
                ++r;
                mk &= mk - 1;
            }
        }
        if (e < E) eoff[e] = ex_c;
        int tot_a = 0, tot_c = 0;
        for (int w = 0; w < 4; ++w) { tot_a += wave_tot[0][w]; tot_c += wave_tot[1][w]; }
        slot_base += tot_a;
        pair_base += tot_c;
        __syncthreads();
    }
    for (int i = tid; i < M * tk; i += 256) {
        int t = i / tk;
        int e = eids[i];
        pair_of[i] = (e >= 0 && e < E) ? eoff[e] + __popcll(hitmask[e] & ((1ull << t) - 1ull)) : -1;
    }
    if (use_shared) {
        for (int t = tid; t < M; t += 256) {
            pair_tok[pair_base + t] = t;
            pair_shared[t] = pair_base + t;
        }
        if (tid == 0) {
            slot_eid[slot_base] = E;
            slot_M[slot_base] = M;
            slot_off[slot_base] = pair_base;
        }
    }
    __syncthreads();
    if (tid == 0) {
        meta[META_N_ROUTED] = slot_base;
        meta[META_N_SLOTS] = slot_base + (use_shared ? 1 : 0);
        meta[META_N_ROUTED_PAIRS] = pair_base;
        meta[META_N_PAIRS] = pair_base + (use_shared ? M : 0);
        meta[META_ERROR] = err;
    }
}

void launch_route_bucket(hipStream_t st, const Geometry& g, const LayerView& L, int M,
                         const float* logits, const int32_t* input_ids, int use_hash, int do_topk,
                         int use_shared, int32_t* eids, float* wts, const Scratch& s) {
    hipLaunchKernelGGL(route_bucket_kernel, dim3(1), dim3(256), 0, st, M, g.E, g.tk, g.score_func,
                       g.round_logits_bf16, g.route_scale, logits, L.router_bias,
                       use_hash ? L.hash : nullptr, input_ids, g.vocab, do_topk, use_shared, eids, wts,
                       s.meta, s.slot_eid, s.slot_M, s.slot_off, s.pair_tok, s.pair_of, s.pair_shared);
}

// -------------------------------------------------------------- operand prep

__device__ __forceinline__ float load_elem(const uint16_t* p, size_t i) {
    return fst_bf16_to_f32(p[i]);
}
__device__ __forceinline__ float load_elem(const float* p, size_t i) { return p[i]; }

// Per row: amax -> exponent s so that amax*2^-s lies in [2^9, 2^10); then the
// k-interleaved fp16 operand (per super-block, lane group g, MFMA c: elements
// 64g+4c+{0..3} and 64g+32+4c+{0..3}) and per-sub-block sums split hi+lo.
template <typename T>
__global__ __launch_bounds__(256) void prep_kernel(const T* __restrict__ x, const int* __restrict__ nrows_dev,
                                                   int nrows_host, int K, _Float16* __restrict__ x16p,
                                                   uint4* __restrict__ sxp, int* __restrict__ xs) {
    const int row = blockIdx.x;
    const int nrows = nrows_dev ? nrows_dev[0] : nrows_host;
    if (row >= nrows) return;
    __shared__ float red[4];
    __shared__ int s_sh;
    const T* xr = x + (size_t)row * K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float m = 0.0f;
    for (int i = tid; i < K; i += 256) m = fmaxf(m, fabsf(load_elem(xr, i)));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (tid == 0) {
        float a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        int s = 0;
        if (a > 0.0f && a < INFINITY) {
            int e;
            frexpf(a, &e);  // a = f*2^e, f in [0.5,1)
            s = e - 10;
        }
        s_sh = s;
        xs[row] = s;
    }
    __syncthreads();
    const int s = s_sh;
    _Float16* dst = x16p + (size_t)row * K;
    const int nchunk = K / 8;
    for (int q = tid; q < nchunk; q += 256) {
        int sb = q >> 5, gc = q & 31, g = gc >> 3, c = gc & 7;
        size_t base = (size_t)sb * 256 + 64 * g + 4 * c;
        h8_t v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = (_Float16)ldexpf(load_elem(xr, base + i), -s);
            v[4 + i] = (_Float16)ldexpf(load_elem(xr, base + 32 + i), -s);
        }
        *reinterpret_cast<h8_t*>(dst + (size_t)q * 8) = v;
    }
    // sub-block sums (32 consecutive elements, natural order, of the fp16 values)
    const int nsub = K / 32;
    uint16_t* sx16 = reinterpret_cast<uint16_t*>(sxp + (size_t)row * (K / 256) * 4);
    for (int j = tid; j < nsub; j += 256) {
        float S = 0.0f;
        for (int i = 0; i < 32; ++i) S += (float)(_Float16)ldexpf(load_elem(xr, (size_t)j * 32 + i), -s);
        _Float16 hi = (_Float16)S;
        _Float16 lo = (_Float16)(S - (float)hi);
        int sb = j >> 3, jj = j & 7, g = jj >> 1, odd = jj & 1;
        uint16_t* e = sx16 + ((size_t)sb * 4 + g) * 8;
        e[odd] = __builtin_bit_cast(uint16_t, hi);
        e[2 + odd] = __builtin_bit_cast(uint16_t, lo);
        if (!odd) { e[4] = 0; e[5] = 0; e[6] = 0; e[7] = 0; }
    }
}

void launch_prep_bf16(hipStream_t st, const uint16_t* x, int rows, int K, _Float16* x16p, uint4* sxp,
                      int* xs) {
    hipLaunchKernelGGL(prep_kernel<uint16_t>, dim3(rows), dim3(256), 0, st, x, nullptr, rows, K, x16p,
                       sxp, xs);
}
void launch_prep_act(hipStream_t st, const float* act, const int* meta, int max_rows, int K,
                     _Float16* a16p, uint4* sxp, int* xs) {
    hipLaunchKernelGGL(prep_kernel<float>, dim3(max_rows), dim3(256), 0, st, act, meta + META_N_PAIRS,
                       max_rows, K, a16p, sxp, xs);
}

// ---------------------------------------------------------- Q4_K FFN kernel

struct Q4kB {
    h8_t w[8];  // sc*q as fp16, 8 MFMA B operands (one per 8-column chunk c)
    h8_t m;     // {m_a, m_b, m_a, m_b, 0...}
    float d, dmin;
};

// Lane (row r = lane&15, group g = lane>>4) owns qs bytes [32g, 32g+32) of the
// row's super-block: low nibbles are sub-block 2g, high nibbles 2g+1.
__device__ __forceinline__ void q4k_build(const uint4 hdr, const uint4 qa, const uint4 qb, int g,
                                          Q4kB& B) {
    B.d = half_bits_to_f32(hdr.x & 0xffffu);
    B.dmin = half_bits_to_f32(hdr.x >> 16);
    const uint32_t y = hdr.y, z = hdr.z, w = hdr.w;
    // get_scale_min_k4 for all 8 sub-blocks, byte-parallel
    const uint32_t sc_lo = y & 0x3F3F3F3Fu, m_lo = z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
    const uint32_t SC = g < 2 ? sc_lo : sc_hi;
    const uint32_t MM = g < 2 ? m_lo : m_hi;
    const int sh = (g & 1) * 16;
    const float sca = (float)((SC >> sh) & 0xffu), scb = (float)((SC >> (sh + 8)) & 0xffu);
    const _Float16 ma = (_Float16)(float)((MM >> sh) & 0xffu);
    const _Float16 mb = (_Float16)(float)((MM >> (sh + 8)) & 0xffu);
    const _Float16 fa = (_Float16)sca, na = (_Float16)(-1024.0f * sca);
    const _Float16 fb = (_Float16)(scb * 0.0625f), nb = (_Float16)(-64.0f * scb);
    const h2_t SCA = {fa, fa}, NEGA = {na, na}, SCB = {fb, fb}, NEGB = {nb, nb};
    const uint32_t D[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t E0 = __builtin_amdgcn_perm(0u, D[c], 0x0C010C00u);  // [0,b1,0,b0]
        const uint32_t E1 = __builtin_amdgcn_perm(0u, D[c], 0x0C030C02u);  // [0,b3,0,b2]
        const h2_t l0 = __builtin_elementwise_fma(as_h2((E0 & 0x000F000Fu) | 0x64006400u), SCA, NEGA);
        const h2_t l1 = __builtin_elementwise_fma(as_h2((E1 & 0x000F000Fu) | 0x64006400u), SCA, NEGA);
        const h2_t u0 = __builtin_elementwise_fma(as_h2((E0 & 0x00F000F0u) | 0x64006400u), SCB, NEGB);
        const h2_t u1 = __builtin_elementwise_fma(as_h2((E1 & 0x00F000F0u) | 0x64006400u), SCB, NEGB);
        B.w[c] = h8_t{l0.x, l0.y, l1.x, l1.y, u0.x, u0.y, u1.x, u1.y};
    }
    const _Float16 z0 = (_Float16)0.0f;
    B.m = h8_t{ma, mb, ma, mb, z0, z0, z0, z0};
}

// Grid: (max_slots * N/64) workgroups of 4 waves; wave w of tile T computes rows
// T*64 + w*16 .. +15 of NPROJ projections for all tokens of its slot (expert).
// MODE 0: gate/up, epilogue silu(g)*u.  MODE 1: down, epilogue scaling.
template <int NPROJ, int NGRP, int MODE>
__global__ __launch_bounds__(256) void q4k_ffn_kernel(
    const uint8_t* __restrict__ bank, size_t expert_stride, size_t mat_offset, size_t proj_stride,
    int K, int N, const int* __restrict__ meta, const int* __restrict__ slot_eid,
    const int* __restrict__ slot_M, const int* __restrict__ slot_off, const int* __restrict__ a_row,
    const _Float16* __restrict__ A, const uint4* __restrict__ SX, const int* __restrict__ xs,
    float* __restrict__ out, float swiglu_limit) {
    const int tiles = N >> 6;
    const int slot = blockIdx.x / tiles;
    const int tile = blockIdx.x - slot * tiles;
    if (slot >= meta[META_N_SLOTS]) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int Me = slot_M[slot], off = slot_off[slot];
    const int row = tile * 64 + wave * 16 + r;
    const int nsb = K >> 8;
    const size_t rowbytes = (size_t)nsb * 144;
    const uint8_t* wbase =
        bank + (size_t)slot_eid[slot] * expert_stride + mat_offset + (size_t)row * rowbytes;

    const h8_t* arow[NGRP];
    const uint4* sxrow[NGRP];
    bool aval[NGRP];
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
        const int tl = q * 16 + r;
        aval[q] = tl < Me;
        int ar = 0;
        if (aval[q]) ar = a_row ? a_row[off + tl] : off + tl;
        arow[q] = reinterpret_cast<const h8_t*>(A + (size_t)ar * K) + g * 8;
        sxrow[q] = SX + (size_t)ar * nsb * 4 + g;
    }

    f4_t acc[NPROJ][NGRP];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int q = 0; q < NGRP; ++q) acc[p][q] = f4_t{0.f, 0.f, 0.f, 0.f};

    uint4 nh[NPROJ], na[NPROJ], nb[NPROJ];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
        const uint8_t* blk = wbase + p * proj_stride;
        nh[p] = *reinterpret_cast<const uint4*>(blk);
        na[p] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g);
        nb[p] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * g);
    }
    const h8_t hz = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    for (int sb = 0; sb < nsb; ++sb) {
        uint4 ch[NPROJ], ca[NPROJ], cb[NPROJ];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) { ch[p] = nh[p]; ca[p] = na[p]; cb[p] = nb[p]; }
        if (sb + 1 < nsb) {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) {
                const uint8_t* blk = wbase + p * proj_stride + (size_t)(sb + 1) * 144;
                nh[p] = *reinterpret_cast<const uint4*>(blk);
                na[p] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g);
                nb[p] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * g);
            }
        }
        h8_t a[NGRP][8], am[NGRP];
#pragma unroll
        for (int q = 0; q < NGRP; ++q) {
            if (q * 16 < Me) {
#pragma unroll
                for (int c = 0; c < 8; ++c) a[q][c] = aval[q] ? arow[q][(size_t)sb * 32 + c] : hz;
                am[q] = aval[q] ? __builtin_bit_cast(h8_t, sxrow[q][(size_t)sb * 4]) : hz;
            }
        }
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
            Q4kB B;
            q4k_build(ch[p], ca[p], cb[p], g, B);
#pragma unroll
            for (int q = 0; q < NGRP; ++q) {
                if (q * 16 < Me) {
                    f4_t D = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < 8; ++c)
                        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[q][c], B.w[c], D, 0, 0, 0);
                    f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am[q], B.m,
                                                                     f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc[p][q][i] = fmaf(B.d, D[i], acc[p][q][i]);
                        acc[p][q][i] = fmaf(-B.dmin, Dm[i], acc[p][q][i]);
                    }
                }
            }
        }
    }

    // D layout: lane holds token rows 4g+i (i=0..3) of the group, column r.
#pragma unroll
    for (int q = 0; q < NGRP; ++q) {
        if (q * 16 >= Me) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tl = q * 16 + 4 * g + i;
            if (tl >= Me) continue;
            const int pidx = off + tl;
            const int ar = a_row ? a_row[pidx] : pidx;
            const int sh = xs[ar];
            if (MODE == 0) {
                float gv = ldexpf(acc[0][q][i], sh);
                float uv = ldexpf(acc[NPROJ - 1][q][i], sh);
                if (swiglu_limit > 0.0f) {
                    gv = fminf(gv, swiglu_limit);
                    uv = fminf(fmaxf(uv, -swiglu_limit), swiglu_limit);
                }
                out[(size_t)pidx * N + row] = (gv / (1.0f + expf(-gv))) * uv;
            } else {
                out[(size_t)pidx * N + row] = ldexpf(acc[0][q][i], sh);
            }
        }
    }
}

template <int NPROJ, int MODE>
static void launch_q4k(hipStream_t st, int ngrp, dim3 grid, const uint8_t* bank, size_t stride,
                       size_t mat_off, size_t proj_stride, int K, int N, const Scratch& s,
                       const int* a_row, const _Float16* A, const uint4* SX, const int* xs, float* out,
                       float lim) {
#define FST_Q4K_LAUNCH(NG)                                                                            \
    hipLaunchKernelGGL((q4k_ffn_kernel<NPROJ, NG, MODE>), grid, dim3(256), 0, st, bank, stride,       \
                       mat_off, proj_stride, K, N, s.meta, s.slot_eid, s.slot_M, s.slot_off, a_row, A, \
                       SX, xs, out, lim)
    if (ngrp <= 1)
        FST_Q4K_LAUNCH(1);
    else if (ngrp == 2)
        FST_Q4K_LAUNCH(2);
    else
        FST_Q4K_LAUNCH(4);
#undef FST_Q4K_LAUNCH
}

void launch_q4k_gate_up(hipStream_t st, const Geometry& g, const LayerView& L, int ngrp,
                        const Scratch& s) {
    const size_t proj = (size_t)g.inter * (g.hd / 256) * 144;
    dim3 grid((unsigned)s.max_slots * (g.inter / 64));
    launch_q4k<2, 0>(st, ngrp, grid, L.bank, L.expert_stride, 0, proj, g.hd, g.inter, s, s.pair_tok,
                     s.x16p, s.sxp, s.xs, s.act, g.swiglu_limit);
}

void launch_q4k_down(hipStream_t st, const Geometry& g, const LayerView& L, int ngrp,
                     const Scratch& s) {
    const size_t proj = (size_t)g.inter * (g.hd / 256) * 144;
    dim3 grid((unsigned)s.max_slots * (g.hd / 64));
    launch_q4k<1, 1>(st, ngrp, grid, L.bank, L.expert_stride, 2 * proj, 0, g.inter, g.hd, s, nullptr,
                     s.a16p, s.sx2p, s.xs2, s.y, 0.0f);
}

// ------------------------------------------------------------------ combine

// src/fst_engine.cpp:4196-4201 and :2851-2852: fp32 accumulation in slot
// order j = 0..tk-1, then + shared, one bf16 rounding (RNE).
__global__ __launch_bounds__(256) void combine_kernel(int M, int hd, int tk, int use_shared,
                                                      const float* __restrict__ y,
                                                      const int* __restrict__ pair_of,
                                                      const int* __restrict__ pair_shared,
                                                      const float* __restrict__ wts,
                                                      uint16_t* __restrict__ out,
                                                      uint16_t* __restrict__ out_routed,
                                                      uint16_t* __restrict__ out_shared) {
    const int t = blockIdx.y;
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (t >= M || n >= hd) return;
    float acc = 0.0f;
    for (int j = 0; j < tk; ++j) {
        const int p = pair_of[t * tk + j];
        if (p < 0) continue;
        acc = acc + wts[t * tk + j] * y[(size_t)p * hd + n];
    }
    if (out_routed) out_routed[(size_t)t * hd + n] = fst_f32_to_bf16(acc);
    if (use_shared) {
        const float sv = y[(size_t)pair_shared[t] * hd + n];
        if (out_shared) out_shared[(size_t)t * hd + n] = fst_f32_to_bf16(sv);
        acc = acc + sv;
    }
    if (out) out[(size_t)t * hd + n] = fst_f32_to_bf16(acc);
}

void launch_combine(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s,
                    const float* wts, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared) {
    dim3 grid((g.hd + 255) / 256, M);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, st, M, g.hd, g.tk, use_shared, s.y,
                       s.pair_of, s.pair_shared, wts, out, out_routed, out_shared);
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
