// fst_gemv.hip — the small-M expert FFN: caller-given routing (process_expert_ffn,
// src/fst_engine.cpp:4068-4371, with process_shared_expert :4373-4489 as one more
// slot and the combine :4196-4201, :2851-2852) for calls of at most two tokens, in
// ONE launch.
//
// At one or two tokens the launch chain of the MFMA path (bucketing + operand
// prep, gate||up, h prep, down) is four dependent launches, each a few
// microseconds of dispatch and memory latency around a sub-microsecond stream
// of one expert's 14 MB.  Here every workgroup finds the call's slots itself,
// and the work is cut so that one expert spreads over the whole chip:
//
//   workgroups [0, S*2*inter/16): (slot, gate or up, 16-row tile): each of the
//     8 waves takes two super-blocks of K, stages its own fp16 operand (per
//     (token, super-block) a power-of-two prescale, k-interleaved, sub-block
//     sums split hi+lo) and runs 8 v_mfma_f32_16x16x32_f16 over the exact fp16
//     sc*q decode of the weights plus one for the min term; partials are summed
//     across the waves through LDS in wave order, and the rows go out as 64-bit
//     words {epoch, value} with device-coherent stores.
//   workgroups [S*2*inter/16, +S*hd/16): (slot, 16-row down tile): the weights
//     are loaded first, then each wave waits for its super-block of the gate
//     and up words (the epoch marks this call's words), forms h = silu(g)*u and
//     runs the same tile.  The down rows then go out with device-coherent
//     stores, and the last slot's workgroup to finish a row tile (a per-tile
//     counter, left at zero) sums the tile in the reference's order: routed
//     pairs in slot order j = 0..tk-1, weighted, then the shared term; one RNE
//     bf16 rounding (the combine kernel's arithmetic).
//
// Weight tile layout (16 rows x one super-block, 2304 bytes): lane 16g+r holds
// bytes [32g, 32g+16) and [32g+16, 32g+32) of row r's nibbles, so its 64 weights
// are sub-block 2g (low nibbles) and 2g+1 (high nibbles), and the headers
// (fp16 d, fp16 dmin, 12 scale bytes) follow at byte 2048 + 16r
// (kernels/fst_dequant_q4k_kernel.cc:40-100 for the block decode).
//
// Waits: a down workgroup waits only for gate||up workgroups, which have lower
// ids and never wait; workgroups are dispatched in id order on each XCD, so
// every awaited workgroup is resident or done.  The wait is bounded by the
// context's spin limit (past it: the sticky timeout bit of the meta words,
// and the call completes).
#include <algorithm>
#include <cstdlib>
#include "fst_internal.h"
#include "fst_q4k_dev.h"
#include "../../include/fst_exact_math.h"

namespace fst {

namespace {

constexpr int kGvW = 8;             // waves per workgroup
constexpr int kGvNT = 64 * kGvW;
constexpr int kGvMaxM = 2;          // tokens per call
constexpr int kGvMaxK = 4096;       // hd and inter bounds (LDS)
constexpr int kGvMaxPairs = kGvMaxM * kMaxTopK;
constexpr int kGvMaxSlots = kGvMaxPairs + 1;
// s_sleep argument between the down waves' one-lane polls
constexpr int kGvPollSleep = 4;


// s_sleep(8) rounds before the down workgroups' first weight loads, so that
// the gate||up weights, which every down workgroup waits for, get the memory
// bandwidth first (measured best at 8-10 rounds).
constexpr int kGvDnDelay = 9;

struct GemvArgs {
    const uint8_t* bank;
    size_t expert_stride;
    int hd, inter, E, M, tk, use_shared, smax;
    const int32_t* eids;   // [M][tk] (caller's routing)
    const float* wts;      // [M][tk]
    const uint16_t* h;     // bf16 [M][hd]
    unsigned long long* hbuf;  // [smax*M][inter] {epoch, value} words: h (VALU variant) or gate rows
    unsigned long long* ubuf;  // [smax*M][inter] {epoch, value} words: up rows (MFMA variant)
    float* y;              // [smax*M][hd] down rows
    int* cnt;              // [hd/16] per-tile arrival counters, zero between calls
    int* meta;
    uint16_t *out, *out_routed, *out_shared;
    float swiglu_limit;
    uint32_t epoch;
    int spin_limit;
    int dn_delay;          // s_sleep(8) rounds before the down workgroups' weight loads
};

__device__ __forceinline__ void st_coherent_f32(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), fst_f32_bits(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent_f32(const float* p) {
    return fst_bits_f32(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT));
}

// The call's slots as every workgroup derives them: distinct valid experts in
// order of first use over (token, j), then the shared expert.
struct GvSlots {
    int eid[kGvMaxPairs], slot_e[kGvMaxSlots], slot_mask[kGvMaxSlots], pslot[kGvMaxPairs];
    int ns, last;
};

__device__ __forceinline__ void gemv_slots(const GemvArgs& a, GvSlots& S, int tid) {
    const int M = a.M, tk = a.tk;
    if (tid < M * tk) S.eid[tid] = a.eids[tid];  // the ids in one round trip
    __syncthreads();
    if (tid == 0) {
        int ns = 0, err = 0;
        for (int i = 0; i < M * tk; ++i) {
            const int e = S.eid[i];
            int sl = -1;
            if (e < 0 || e >= a.E) {
                err = 1;
            } else {
                for (int q = 0; q < ns; ++q)
                    if (S.slot_e[q] == e) sl = q;
                if (sl < 0) {
                    sl = ns++;
                    S.slot_e[sl] = e;
                    S.slot_mask[sl] = 0;
                }
                S.slot_mask[sl] |= 1 << (i / tk);
            }
            S.pslot[i] = sl;
        }
        if (a.use_shared) {
            S.slot_e[ns] = a.E;
            S.slot_mask[ns] = (1 << M) - 1;
            ++ns;
        }
        S.ns = ns;
        if (blockIdx.x == 0) {
            a.meta[META_ERROR] = err;
            a.meta[META_TIMEOUT] = 0;
            sticky_or(a.meta, err);
        }
    }
    __syncthreads();
}

// The end of a down workgroup: v = this slot's down row rt*16 + (tid & 15) of
// token tid >> 4 (threads tid < M*16).  A one-slot call combines at once;
// otherwise the rows go out to y with device-coherent stores and the tile's
// last slot to arrive (per-tile counter, left at zero) combines the tile in
// the reference's order (src/fst_engine.cpp:4196-4201, :2851-2852): routed
// pairs j = 0..tk-1 weighted in fp32, then the shared term, one RNE rounding.
__device__ __forceinline__ void gemv_tile_out(const GemvArgs& a, GvSlots& S, float (*ystage)[16], int ns, int slot,
                                              int mask, int rt, int tid, float v) {
    const int M = a.M, tk = a.tk, hd = a.hd;
    if (tid < M * 16) {
        const int t = tid >> 4, rr = tid & 15;
        if (ns == 1)
            ystage[t][rr] = v;
        else if ((mask >> t) & 1)
            st_coherent_f32(a.y + (size_t)(slot * M + t) * hd + rt * 16 + rr, v);
    }
    if (ns > 1) {
        publish_wait();
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(a.cnt + rt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            S.last = old == ns - 1;
            if (S.last) __hip_atomic_store(a.cnt + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!S.last) return;
    } else {
        __syncthreads();
    }
    if (tid < M * 16) {
        const int t = tid >> 4, rr = tid & 15;
        const int n = rt * 16 + rr;
        auto yv = [&](int sl) {
            return ns == 1 ? ystage[t][rr] : ld_coherent_f32(a.y + (size_t)(sl * M + t) * hd + n);
        };
        float acc = 0.0f;
        for (int j = 0; j < tk; ++j) {
            const int sl = S.pslot[t * tk + j];
            if (sl < 0) continue;
            acc = fmaf(a.wts[t * tk + j], yv(sl), acc);
        }
        const size_t o = (size_t)t * hd + n;
        if (a.out_routed) a.out_routed[o] = fst_f32_to_bf16(acc);
        if (a.use_shared) {
            const float vs = yv(ns - 1);
            if (a.out_shared) a.out_shared[o] = fst_f32_to_bf16(vs);
            acc = acc + vs;
        }
        if (a.out) a.out[o] = fst_f32_to_bf16(acc);
    }
}

// h = silu(g) * u with the optional clamp (swiglu_limit > 0).
__device__ __forceinline__ float swiglu(float gv, float uv, float lim) {
    if (lim > 0.0f) {
        gv = fminf(gv, lim);
        uv = fminf(fmaxf(uv, -lim), lim);
    }
    return (gv / (1.0f + expf(-gv))) * uv;
}


// 16 lanes' max (DPP within the row), then the row pair's (rows 0+1, 2+3).
__device__ __forceinline__ float max32(float x) {
    x = fmaxf(x, fdpp<0xb1>(x));   // quad_perm [1,0,3,2]
    x = fmaxf(x, fdpp<0x4e>(x));   // quad_perm [2,3,0,1]
    x = fmaxf(x, fdpp<0x124>(x));  // row_ror 4
    x = fmaxf(x, fdpp<0x128>(x));  // row_ror 8
    const uint32_t u = fst_f32_bits(x);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(fst_bits_f32((uint32_t)p[0]), fst_bits_f32((uint32_t)p[1]));
}

constexpr int kGvMaxSb = kGvMaxK / 256;
constexpr int kGvOpSb = 36;  // 32 operand chunks + 4 sub-block-sum chunks per super-block

// The launch: each wave stages its
// own super-blocks' operand (no workgroup barrier before the dot products):
// per (token, super-block) a power-of-two prescale from the 256 values' max,
// the fp16 operand k-interleaved to match q4k_bop, and the sub-block sums
// split hi+lo for the min term.  Each tile is then 8 v_mfma_f32_16x16x32_f16
// on the decoded weights (the MFMA path's exact fp16 sc*q decode) plus one
// for the min term; token rows t < M of the result are used.
__global__ __launch_bounds__(kGvNT) __attribute__((amdgpu_waves_per_eu(4))) void expert_gemv_mfma_kernel(GemvArgs a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int hd = a.hd, inter = a.inter, M = a.M;
    __shared__ uint4 opb[kGvMaxM][kGvMaxSb * kGvOpSb];
    __shared__ int s_exp[kGvMaxM][kGvMaxSb];
    __shared__ float red[2][kGvW][kGvMaxM][16];
    __shared__ GvSlots S;
    __shared__ float ystage[kGvMaxM][16];

    gemv_slots(a, S, tid);
    const int ns = __builtin_amdgcn_readfirstlane(S.ns);
    // workgroups: (slot, gate or up, 16-row tile), then (slot, down tile)
    const int tiles_gu = inter / 16, tiles_dn = hd / 16;
    const int ngu = a.smax * 2 * tiles_gu;
    const bool dn = (int)blockIdx.x >= ngu;
    const int b = dn ? (int)blockIdx.x - ngu : (int)blockIdx.x;
    const int slot = dn ? b / tiles_dn : b / (2 * tiles_gu);
    const int rem = dn ? b - slot * tiles_dn : b - slot * 2 * tiles_gu;
    const int up = dn ? 0 : (rem & 1);
    const int rt = dn ? rem : rem >> 1;
    const size_t proj = (size_t)inter * (hd / 256) * 144;
    if (ns == 0) {
        if (dn && slot == 0 && tid < M * 16) {
            const size_t o = (size_t)(tid >> 4) * hd + rt * 16 + (tid & 15);
            if (a.out) a.out[o] = 0;
            if (a.out_routed) a.out_routed[o] = 0;
        }
        return;
    }
    if (slot >= ns) return;
    const int mask = __builtin_amdgcn_readfirstlane(S.slot_mask[slot]);
    const uint8_t* ex = a.bank + (size_t)__builtin_amdgcn_readfirstlane(S.slot_e[slot]) * a.expert_stride;
    const int K = dn ? inter : hd, nsb = K >> 8;
    const uint8_t* wbase = ex + (dn ? 2 * proj : up * proj) + (size_t)rt * nsb * 2304;

    // ---- this wave's weight tiles (super-blocks wave, wave + 8)
    WRaw w0[2];
    auto load_weights = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int sb = wave + kGvW * i;
            if (sb < nsb) w0[i] = load_wraw(wbase + (size_t)sb * 2304, lane);
        }
    };
    // down workgroups start their weight loads after the gate||up ones have
    // had a head start (dn_delay sleeps), so the gate||up weights, which the
    // whole launch waits on, do not share the memory bandwidth at first
    if (dn)
        for (int i = 0; i < a.dn_delay; ++i) __builtin_amdgcn_s_sleep(8);
    load_weights();

    // ---- this wave's operand: (token, super-block) pairs, two per pass
    // (lanes 0-31 and 32-63), lane q = 8 gq + c builds chunk (gq, c)
    const int nT = mask == 3 ? 2 : 1, t0 = mask == 2 ? 1 : 0;
    const int nsw = (wave < nsb ? 1 : 0) + (wave + kGvW < nsb ? 1 : 0);
    const int np = nT * nsw;
    const int q = lane & 31, gq = q >> 3, c = q & 7;
    int timed_out = 0;
    // polls of this wave so far: the one-lane pre-poll and every later poll
    // draw on one budget of spin_limit polls
    int spent = 0;
    if (dn && np > 0) {
        // first wait on one word (the last row of the last gate and up tiles
        // of this wave's first super-block) with one lane: device-coherent
        // loads from every lane (or from one lane per source tile) slow the
        // gate||up weight streams measurably for the whole wait
        const size_t wo = (size_t)(slot * M + t0) * inter + wave * 256 + 255;
        for (; spent < a.spin_limit; ++spent) {
            int ready = 1;
            if (lane == 0) {
                const unsigned long long gv = ld_coherent_u64(a.hbuf + wo), uv = ld_coherent_u64(a.ubuf + wo);
                ready = (uint32_t)(gv >> 32) == a.epoch && (uint32_t)(uv >> 32) == a.epoch;
            }
            if (__builtin_amdgcn_readfirstlane(ready)) break;
            __builtin_amdgcn_s_sleep(kGvPollSleep);
        }
    }
    for (int p0 = 0; p0 < np; p0 += 2) {
        const int p = p0 + (lane >> 5);
        const bool live = p < np;
        const int pp = live ? p : p0;
        const int t = nT == 2 ? (pp & 1) : t0;
        const int sb = wave + kGvW * (nT == 2 ? (pp >> 1) : pp);
        const int e0 = sb * 256 + 64 * gq + 4 * c;
        float x[8];
        if (!dn) {
            const uint16_t* hx = a.h + (size_t)t * hd + e0;
            const uint2 lo = *reinterpret_cast<const uint2*>(hx);
            const uint2 hi = *reinterpret_cast<const uint2*>(hx + 32);
            x[0] = fst_bits_f32(lo.x << 16);
            x[1] = fst_bits_f32(lo.x & 0xffff0000u);
            x[2] = fst_bits_f32(lo.y << 16);
            x[3] = fst_bits_f32(lo.y & 0xffff0000u);
            x[4] = fst_bits_f32(hi.x << 16);
            x[5] = fst_bits_f32(hi.x & 0xffff0000u);
            x[6] = fst_bits_f32(hi.y << 16);
            x[7] = fst_bits_f32(hi.y & 0xffff0000u);
        } else {
            // poll this lane's 8 gate and 8 up words (device-coherent loads)
            // until every lane of the wave holds words of this call's epoch;
            // then h = silu(g) * u
            const size_t wo = (size_t)(slot * M + t) * inter + e0;
            const unsigned long long* gw = a.hbuf + wo;
            const unsigned long long* uw = a.ubuf + wo;
            unsigned long long gv[8], uv[8];
            for (;;) {
                int ok = 1;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int o = (k & 3) + (k >> 2) * 32;
                    gv[k] = ld_coherent_u64(gw + o);
                    uv[k] = ld_coherent_u64(uw + o);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if ((uint32_t)(gv[k] >> 32) != a.epoch || (uint32_t)(uv[k] >> 32) != a.epoch) ok = 0;
                if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                if (++spent > a.spin_limit) {
                    timed_out = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k)
                x[k] = swiglu(fst_bits_f32((uint32_t)gv[k]), fst_bits_f32((uint32_t)uv[k]), a.swiglu_limit);
        }
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(x[k]));
        const int se = prescale_exp(max32(m));
        h8_t v;
        v[0] = (_Float16)ldexpf(x[0], -se);
        v[1] = (_Float16)ldexpf(x[2], -se);
        v[2] = (_Float16)ldexpf(x[1], -se);
        v[3] = (_Float16)ldexpf(x[3], -se);
        v[4] = (_Float16)ldexpf(x[4], -se);
        v[5] = (_Float16)ldexpf(x[6], -se);
        v[6] = (_Float16)ldexpf(x[5], -se);
        v[7] = (_Float16)ldexpf(x[7], -se);
        float s0 = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
        float s1 = ((float)v[4] + (float)v[5]) + ((float)v[6] + (float)v[7]);
        s0 = s0 + fdpp<0xb1>(s0);  // quad_perm [1,0,3,2]
        s1 = s1 + fdpp<0xb1>(s1);
        s0 = s0 + fdpp<0x4e>(s0);  // quad_perm [2,3,0,1]
        s1 = s1 + fdpp<0x4e>(s1);
        s0 = s0 + fdpp<0x104>(s0);  // row_shl 4: lane c == 0 holds the 8 lanes' sum
        s1 = s1 + fdpp<0x104>(s1);
        if (live) {
            opb[t][sb * kGvOpSb + q] = __builtin_bit_cast(uint4, v);
            if (c == 0) {
                const _Float16 h0 = (_Float16)s0, h1 = (_Float16)s1;
                const _Float16 l0 = (_Float16)(s0 - (float)h0), l1 = (_Float16)(s1 - (float)h1);
                const _Float16 z = (_Float16)0.0f;
                opb[t][sb * kGvOpSb + 32 + gq] = __builtin_bit_cast(uint4, h8_t{h0, h1, l0, l1, z, z, z, z});
            }
            if (q == 0) s_exp[t][sb] = se;
        }
    }
    if (timed_out && lane == 0) sticky_or(a.meta, STICKY_TIMEOUT);
    // the wave reads back only what it wrote: LDS keeps one wave's accesses
    // in order, the compiler must too
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    // ---- dot products: rows r of the tile for token rows 0..M-1 (A rows r
    // read token r & (M-1): broadcast reads; rows >= M are discarded)
    const uint32_t ssel = q4k_scale_sel(g), magic = 0x64006400u;
    const int tr = r & (M - 1);
    float acc0[kGvMaxM] = {0.0f, 0.0f};
    auto tile = [&](const WRaw& W, int sb, float* acc) {
        Q4kScale Sc;
        q4k_scales(W.h, g, ssel, Sc);
        const uint32_t Dw[8] = {W.a.x, W.a.y, W.a.z, W.a.w, W.b.x, W.b.y, W.b.z, W.b.w};
        const uint4* op = opb[tr] + sb * kGvOpSb;
        f4_t D = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const h8_t bo = q4k_bop(Dw[cc], Sc, magic);
            const h8_t ao = __builtin_bit_cast(h8_t, op[8 * g + cc]);
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, bo, D, 0, 0, 0);
        }
        const h8_t am = __builtin_bit_cast(h8_t, op[32 + g]);
        const f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, Sc.m, f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < kGvMaxM; ++i) {
            const float part = fmaf(Sc.d, D[i], -Sc.dmin * Dm[i]);
            acc[i] += ldexpf(part, s_exp[i < M ? i : 0][sb]);
        }
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int sb = wave + kGvW * i;
        if (sb >= nsb) continue;
        tile(w0[i], sb, acc0);
    }
    if (g == 0)
        for (int t = 0; t < M; ++t) red[0][wave][t][r] = acc0[t];
    __syncthreads();
    if (!dn) {
        // the tile's gate (or up) rows as {epoch, value} words
        if (tid < M * 16) {
            const int t = tid >> 4, rr = tid & 15;
            if ((mask >> t) & 1) {
                float v = 0.0f;
                for (int w = 0; w < kGvW; ++w) v += red[0][w][t][rr];
                st_coherent_u64((up ? a.ubuf : a.hbuf) + (size_t)(slot * M + t) * inter + rt * 16 + rr,
                                ((unsigned long long)a.epoch << 32) | fst_f32_bits(v));
            }
        }
        return;
    }
    float v = 0.0f;
    if (tid < M * 16)
        for (int w = 0; w < kGvW; ++w) v += red[0][w][tid >> 4][tid & 15];
    gemv_tile_out(a, S, ystage, ns, slot, mask, rt, tid, v);
}

}  // namespace


bool gemv_supported(const Geometry& g, int M, int tk, int use_shared, const Scratch& s) {
    if (g.codec != 0 || M < 1 || M > kGvMaxM || tk < 0 || tk > kMaxTopK) return false;
    if (g.hd % 256 || g.inter % 256 || g.hd > kGvMaxK || g.inter > kGvMaxK) return false;
    const int smax = std::max(1, std::min(g.E, M * tk) + (use_shared ? 1 : 0));
    return smax * M <= s.max_pairs;
}

int launch_expert_gemv(hipStream_t st, const Geometry& g, const LayerView& L, int M, int tk, const int32_t* eids,
                       const float* wts, int use_shared, const uint16_t* h, const Scratch& s, uint32_t epoch,
                       int spin_limit, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared) {
    GemvArgs a{};
    a.bank = L.bank;
    a.expert_stride = L.expert_stride;
    a.hd = g.hd;
    a.inter = g.inter;
    a.E = g.E;
    a.M = M;
    a.tk = tk;
    a.use_shared = use_shared;
    a.smax = std::max(1, std::min(g.E, M * tk) + (use_shared ? 1 : 0));
    a.eids = eids;
    a.wts = wts;
    a.h = h;
    a.hbuf = s.hbuf;
    a.y = s.y;
    a.cnt = s.gemv_cnt;
    a.meta = s.meta;
    a.out = out;
    a.out_routed = out_routed;
    a.out_shared = out_shared;
    a.swiglu_limit = g.swiglu_limit;
    a.epoch = epoch;
    a.spin_limit = spin_limit;
    a.dn_delay = kGvDnDelay;
    a.ubuf = s.hbuf + (size_t)s.max_pairs * g.inter;
    hipLaunchKernelGGL(expert_gemv_mfma_kernel, dim3((unsigned)a.smax * (unsigned)(2 * g.inter / 16 + g.hd / 16)),
                       dim3(kGvNT), 0, st, a);
    return 0;
}

}  // namespace fst
