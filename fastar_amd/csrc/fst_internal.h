// fst_internal.h — device-side layouts and kernel launchers shared by the
// HIP translation units of libfst_hip.so.  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fst {

// Records the message returned by fst_last_error() and returns code.
int set_error(int code, const char* msg);

// Q4_K super-block: 256 weights in 144 bytes (fp16 d, fp16 dmin, 12 bytes of
// packed 6-bit scales/mins, 128 bytes of nibbles).
constexpr int kQ4kBlockElems = 256;
constexpr int kQ4kBlockBytes = 144;
// MXFP4 block: 32 weights in 17 bytes (e8m0 scale + 16 nibble bytes).
constexpr int kMxBlockElems = 32;
constexpr int kMxBlockBytes = 17;

constexpr int kMaxTokens = 64;      // tokens per call (4 groups of 16 MFMA rows)
constexpr int kMaxTopK = 16;

// Meta words written by the bucketing kernel and read by later kernels.
enum MetaIdx {
    META_N_SLOTS = 0,      // routed active slots + shared slot
    META_N_ROUTED = 1,     // routed active slots
    META_N_PAIRS = 2,      // (token, expert) pairs incl. shared
    META_ERROR = 3,        // nonzero: invalid expert id seen
    META_N_ROUTED_PAIRS = 4,
    META_TIMEOUT = 5,      // this call: a cross-workgroup hand-off wait gave up
    META_STICKY = 6,       // kernels only OR into it; only the host clears it
    META_WORDS = 8
};
// Bits of meta[META_STICKY]: every error a launch of the MoE path detects on
// the device, kept until the host reads and clears it (fst_moe_check and the
// host-pointer entry points), so that an error of an earlier stream-ordered
// call is not overwritten by the calls after it.
enum StickyBits {
    STICKY_EXPERT_ID = 1,  // an expert id out of range in the routing
    STICKY_HASH_ID = 2,    // an input id out of the vocabulary for hash routing
    STICKY_TIMEOUT = 4     // a hand-off wait gave up (spin limit)
};
// ORs a routing error word (META_ERROR bits 1 and 2) and a timeout flag into
// the sticky word; meta may be any address space the caller holds.
__device__ __forceinline__ void sticky_or(int* meta, int bits) {
    if (bits) atomicOr(&meta[META_STICKY], bits);
}

// Device scratch owned by a context, sized for max_tokens.
struct Scratch {
    int max_tokens, max_pairs, max_slots;
    int n_cu;              // compute units of the device (persistent grids)
    int fused_per_cu;      // workgroups of the fused MoE launch resident per CU (0: launch unused)
    uint16_t* h;           // bf16 [T][hd] staging for host-pointer calls
    uint16_t* out;         // bf16 [T][hd]
    uint16_t* out_routed;  // bf16 [T][hd]
    uint16_t* out_shared;  // bf16 [T][hd]
    int32_t* ids;          // [T]
    float* logits;         // [T][E]
    int32_t* eids;         // [T][tk]
    float* wts;            // [T][tk]
    int* meta;             // [META_WORDS]
    int* slot_eid;         // [S]
    int* slot_M;           // [S]
    int* slot_off;         // [S]
    int* pair_tok;         // [P]
    int* pair_of;          // [T][tk]
    int* pair_shared;      // [T]
    _Float16* x16p;        // [T][hd]    k-interleaved, power-of-two prescaled
    uint4* sxp;            // [T][hd/256][4] sub-block sums (hi,lo) per lane group
    int* xs;               // [T] prescale exponent
    float* act;            // [P][inter] h = silu(gate) * up
    _Float16* a16p;        // [P][inter] h as the down projection's operand
    uint4* sx2p;           // [P][inter/256][4]
    int* xs2;              // [P]
    float* y;              // [P][hd]
    uint16_t* sh_h16;      // [T][inter] bf16 shared-expert h (bf16 shared expert)
    float* ys;             // [T][hd] fp32 shared-expert output (bf16 shared expert)
    // fused gate||up + down launch: {epoch, value} words handed between
    // workgroups (h rows and their per-16-row maxima)
    unsigned long long* hbuf;   // [2][P][inter] (the small-M launch uses both halves)
    unsigned long long* amaxw;  // [P][inter/16]
    int* fused_claim;           // down-pair counter of the fused launch (zeroed by the router launch)
    int* gemv_cnt;              // [hd/16] arrival counters of the small-M launch (zero between calls)
    // combine with the next layer's residual + RMSNorm folded in (verify forward)
    unsigned long long* norm_part;  // [T][64] double sums of squares of the row's lane chunks
    int* norm_cnt;                  // [T] arrival counters (zero between calls)
};

// Device expert bank: n_layers x (n_experts + 1) packed experts.
struct LayerView {
    const uint8_t* bank;       // expert 0 of the layer; expert e at bank + e*expert_stride
    size_t expert_stride;
    const uint16_t* router_nk; // bf16 [E][hd], transposed and lane-interleaved at upload (router_interleave)
    const float* router_bias;  // [E] or null
    const int32_t* hash;       // [vocab][tk] or null
};

struct Geometry {
    int hd, inter, E, tk, codec;
    int score_func, round_logits_bf16;
    float route_scale, swiglu_limit;
    int vocab;
};

// ---- cross-workgroup hand-off inside one launch ----
// On this multi-XCD GPU each XCD has its own L2; an agent-scope fence
// (__threadfence) writes back and invalidates the whole L2, which is far too
// expensive to issue per workgroup.  Data handed to another workgroup is
// instead written with device-coherent stores (sc1) that carry their own
// "written" marker, the writer waits for its stores to complete, and the
// reader polls with device-coherent loads.
__device__ __forceinline__ void st_coherent_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_coherent_u64(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's stores are complete (and keep the compiler from
// moving memory operations across the point).
__device__ __forceinline__ void publish_wait() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- wave-level DPP reductions (all 64 lanes active) ----
// Wave-wide max / min of a uint32 held by every lane (all 64 lanes active):
// DPP within each row of 16 lanes, then the four row results.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t x) {  // bound_ctrl off: lanes without a source read 0
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float fdpp(float x) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(uint32_t, x)));
}
// Wave-wide fmaxf (order-free: fmaxf ignores NaN operands).
__device__ __forceinline__ float wave_fmax(float x) {
    x = fmaxf(x, fdpp<0xb1>(x));
    x = fmaxf(x, fdpp<0x4e>(x));
    x = fmaxf(x, fdpp<0x124>(x));
    x = fmaxf(x, fdpp<0x128>(x));
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    x = max(x, dpp<0xb1>(x));   // quad_perm [1,0,3,2]
    x = max(x, dpp<0x4e>(x));   // quad_perm [2,3,0,1]
    x = max(x, dpp<0x124>(x));  // row_ror 4
    x = max(x, dpp<0x128>(x));  // row_ror 8
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
    return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
    x = min(x, dpp<0xb1>(x));
    x = min(x, dpp<0x4e>(x));
    x = min(x, dpp<0x124>(x));
    x = min(x, dpp<0x128>(x));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
    return min(min(a, b), min(c, d));
}

// Sum of the 64 lanes' values in the canonical halving-tree order, as lane 0
// sees it: p[j] += p[j + off] for off = 32, 16, ..., 1.  The cross-row steps
// use gfx950's permlane32/16 swaps (lanes j < 32 read lane j + 32; lanes of
// even rows read the next row), the in-row steps DPP row shifts (lane j reads
// lane j + off).  Only lane 0's result is meaningful.
__device__ __forceinline__ float tree_sum64(float acc) {
    const uint32_t a = __builtin_bit_cast(uint32_t, acc);
    const auto s32 = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    acc = acc + __builtin_bit_cast(float, (uint32_t)s32[1]);
    const uint32_t b = __builtin_bit_cast(uint32_t, acc);
    const auto s16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    acc = acc + __builtin_bit_cast(float, (uint32_t)s16[1]);
    acc = acc + __builtin_bit_cast(float, dpp<0x108>(__builtin_bit_cast(uint32_t, acc)));  // row_shl 8
    acc = acc + __builtin_bit_cast(float, dpp<0x104>(__builtin_bit_cast(uint32_t, acc)));  // row_shl 4
    acc = acc + __builtin_bit_cast(float, dpp<0x102>(__builtin_bit_cast(uint32_t, acc)));  // row_shl 2
    acc = acc + __builtin_bit_cast(float, dpp<0x101>(__builtin_bit_cast(uint32_t, acc)));  // row_shl 1
    return acc;
}

// Wave-wide max of a uint64 held by every lane, in every lane: DPP within
// each row of 16 lanes, then gfx950's row-pair and half swaps (with both
// operands x, permlane16_swap returns {x of the even row, x of the odd row}
// of each row pair in both rows, permlane32_swap the same for the halves).
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    return ((unsigned long long)dpp<CTRL>((uint32_t)(v >> 32)) << 32) | dpp<CTRL>((uint32_t)v);
}
__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
    x = max_u64(x, dpp_u64<0xb1>(x));   // quad_perm [1,0,3,2]
    x = max_u64(x, dpp_u64<0x4e>(x));   // quad_perm [2,3,0,1]
    x = max_u64(x, dpp_u64<0x124>(x));  // row_ror 4
    x = max_u64(x, dpp_u64<0x128>(x));  // row_ror 8
    {
        const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
        const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        x = max_u64(((unsigned long long)(uint32_t)h[0] << 32) | (uint32_t)l[0],
                    ((unsigned long long)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
    }
    {
        const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
        const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        x = max_u64(((unsigned long long)(uint32_t)h[0] << 32) | (uint32_t)l[0],
                    ((unsigned long long)(uint32_t)h[1] << 32) | (uint32_t)l[1]);
    }
    return ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((int)(x >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
}
// Wave-wide max / min of a uint32, in every lane (DPP within rows, then the
// row-pair and half swaps as in wave_max_u64).
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext_u32_all(uint32_t x) {
    auto f = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    x = f(x, dpp<0xb1>(x));
    x = f(x, dpp<0x4e>(x));
    x = f(x, dpp<0x124>(x));
    x = f(x, dpp<0x128>(x));
    const auto p16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = f((uint32_t)p16[0], (uint32_t)p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    x = f((uint32_t)p32[0], (uint32_t)p32[1]);
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
__device__ __forceinline__ uint32_t wave_max_u32_all(uint32_t x) { return wave_ext_u32_all<true>(x); }
__device__ __forceinline__ uint32_t wave_min_u32_all(uint32_t x) { return wave_ext_u32_all<false>(x); }
// Number of set bits of mask below bit `lane` (mbcnt).
__device__ __forceinline__ int lane_prefix(unsigned long long mask, int lane) {
    (void)lane;
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Wave-wide argmax over (m, i) pairs, i < 0 meaning "no element": larger m
// first, then lower i.  The merge is associative and commutative, so the
// DPP tree gives the same result as any other order.  Result in every lane.
__device__ __forceinline__ void argmax_merge(float& m, int& i, float om, int oi) {
    if (oi >= 0 && (i < 0 || om > m || (om == m && oi < i))) {
        m = om;
        i = oi;
    }
}
template <int CTRL>
__device__ __forceinline__ void argmax_step(float& m, int& i) {
    const float om = fdpp<CTRL>(m);
    const int oi = (int)dpp<CTRL>((uint32_t)i);
    argmax_merge(m, i, om, oi);
}
__device__ __forceinline__ void wave_argmax(float& m, int& i) {
    argmax_step<0xb1>(m, i);
    argmax_step<0x4e>(m, i);
    argmax_step<0x124>(m, i);
    argmax_step<0x128>(m, i);
    float rm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 0));
    int ri = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        argmax_merge(rm, ri, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), r)),
                     __builtin_amdgcn_readlane(i, r));
    m = rm;
    i = ri;
}
// Wave-wide sum of a uint64 (integer: any order gives the same result).
__device__ __forceinline__ unsigned long long wave_sum_u64_dpp(unsigned long long v) {
    v += dpp_u64<0xb1>(v);
    v += dpp_u64<0x4e>(v);
    v += dpp_u64<0x124>(v);
    v += dpp_u64<0x128>(v);
    unsigned long long t = 0;
#pragma unroll
    for (int r = 0; r < 64; r += 16)
        t += ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), r) << 32) |
             (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, r);
    return t;
}

// ---- launchers (each enqueues on `st`) ----
// Router logits with the fp16 operand prep of h (prep, Q4_K), then top-k (or
// hash rows) and the bucketing of the call (two launches).
// With topk = 0 only the logits (and the operand prep) are launched: the
// top-k and bucketing then run in the gate||up launch (RouteReq).
void launch_route(hipStream_t st, const Geometry& g, const LayerView& L, const uint16_t* h, int M, int prep,
                  const int32_t* input_ids, int use_hash, int use_shared, int32_t* eids, float* wts,
                  const Scratch& s, int topk = 1);
// Routing that the gate||up launch performs itself from s.logits (every
// workgroup computes the call's top-k and bucket tables into LDS; workgroup 0
// also writes eids/wts and the tables to global memory for later launches).
struct RouteReq {
    const int32_t* input_ids;
    int use_hash, use_shared;
    int32_t* eids;
    float* wts;
    int given;  // eids/wts are the caller's routing (no router)
};
// Largest expert count the in-launch routing handles (4 experts per lane).
constexpr int kFusedRouteMaxExperts = 256;
// Bucketing of caller-given routing eids [M][tk].
void launch_bucket(hipStream_t st, const Geometry& g, int M, int use_shared, const int32_t* eids,
                   const Scratch& s);
void launch_prep_bf16(hipStream_t st, const uint16_t* x, int rows, int K, _Float16* x16p,
                      uint4* sxp, int* xs);
// launch_bucket and (h given: Q4_K) launch_prep_bf16 of the M rows in one
// launch; o1/o2: the outputs the down launch will write directly (their
// rows of tokens with an invalid expert id are zeroed here); pf/pf_bytes
// (optional): weights read into the device-wide cache by extra workgroups.
// bucket = false: no bucketing (the fused launch buckets the ids itself).
// Also zeroes the fused launch's claim counter.
void launch_bucket_prep(hipStream_t st, const Geometry& g, int M, int use_shared, const int32_t* eids,
                        const Scratch& s, const uint16_t* h, uint16_t* o1, uint16_t* o2, const void* pf = nullptr,
                        size_t pf_bytes = 0, bool bucket = true);
// Residual add + RMSNorm per token row (see resid_norm_kernel); optional
// outputs: h_out (x), normed (bf16), the fp16 operand in prep->x16p/sxp/xs,
// and a one-slot table for launch_q4k_dense in slot_tab (META_WORDS + 3 ints).
void launch_resid_norm(hipStream_t st, const uint16_t* h, const uint16_t* y, const uint16_t* w, int M, int d,
                       float eps, uint16_t* h_out, uint16_t* normed, const Scratch* prep, int* slot_tab);
// logits[M][N] = x . W^T for one resident Q4_K matrix W (device layout).
void launch_q4k_dense(hipStream_t st, const uint8_t* W, int M, int K, int N, const Scratch& s, int* slot_tab,
                      float* out);
// Linear layers over plain bf16 [N][K] weights (fst_dense.hip).
int bf16_linear_rows_per_wg(int K, int gate_up);
void launch_bf16_linear(hipStream_t st, const uint16_t* W, int K, int N, const uint16_t* x, int M, float* y32,
                        uint16_t* y16a, uint16_t* y16b);
void launch_bf16_gate_up(hipStream_t st, const uint16_t* W, int K, int inter, const uint16_t* x, int M,
                         float swiglu_limit, uint16_t* h);
// Hyper-Connections (4 residual streams of width d; see fst_hc.hip).
void launch_hc_pre(hipStream_t st, const uint16_t* h_hc, const uint16_t* fnT, const float* scale, const float* base,
                   int M, int d, uint16_t* cur, float* post, float* comb);
void launch_hc_post(hipStream_t st, const uint16_t* bo, uint16_t* h_hc, const float* post, const float* comb, int M,
                    int d);
void launch_hc_head(hipStream_t st, const uint16_t* h_hc, const uint16_t* fnT, float scale, const float* base, int M,
                    int d, uint16_t* plain);
// h rows -> the down projection's operand (one workgroup per pair).
// pf/pf_bytes (optional): weights the next launch streams first, read into
// the device-wide cache by extra workgroups of this latency-bound launch.
void launch_prep_act(hipStream_t st, const float* h, const int* meta, int max_rows, int K, _Float16* a16p,
                     uint4* sxp, int* xs, const void* pf = nullptr, size_t pf_bytes = 0);
// Weights must be in the wave-tiled device layout (repack_q4k_expert).
// gate/up writes h = silu(gate)*up; down writes y[pair] (fp32), combined by
// launch_combine.
// slots_bound / pairs_bound: upper bounds of the call's slots and (token,
// expert) pairs (0: unknown).  Returns the split-K factor it chose: with
// ksplit > 1 (Q4_K only) each (slot, tile) is split into ksplit super-block
// ranges that write partial gate and up sums over s.act
// ([ksplit][pairs_bound][2*inter]), and the caller runs
// launch_prep_act_split (which adds them up and applies the SwiGLU) instead
// of launch_prep_act.
int launch_q4k_gate_up(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                       const uint16_t* h_in, const RouteReq* route = nullptr, int slots_bound = 0,
                       int pairs_bound = 0);
void launch_prep_act_split(hipStream_t st, const float* part, int S, int rows, float swiglu_limit, const int* meta,
                           int inter, _Float16* a16p, uint4* sxp, int* xs, const void* pf = nullptr,
                           size_t pf_bytes = 0);
// The expert work of a routed block of at most 8 tokens in one persistent
// launch (gate||up then down items, see moe_fused_kernel), after launch_route
// with topk = 0; y rows go to s.y for launch_combine.  epoch: a new nonzero
// value per call (tags the h words); spin_limit bounds each hand-off wait.
bool moe_fused_supported(const Geometry& g, int M);
// Workgroups of the fused MoE launch (codec's instantiation) that one CU holds
// at once, by the occupancy calculator, capped at 2 (0 on error).
int moe_fused_occupancy(int codec);
// Small-M expert FFN with caller-given routing (M <= 2, Q4_K): one launch
// from the eids to the combined bf16 rows.
bool gemv_supported(const Geometry& g, int M, int tk, int use_shared, const Scratch& s);
int launch_expert_gemv(hipStream_t st, const Geometry& g, const LayerView& L, int M, int tk, const int32_t* eids,
                       const float* wts, int use_shared, const uint16_t* h, const Scratch& s, uint32_t epoch,
                       int spin_limit, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared);
// The fused launch's combine: y rows indexed (token, j), j = tk the shared expert.
// The combine of a verify-forward layer with the next layer's h += out and
// RMSNorm (weights w) folded in: h is updated in place and normed written,
// bit-identical to launch_combine_tj followed by launch_resid_norm.
bool combine_norm_supported(const Geometry& g);
void launch_combine_norm_tj(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s,
                            const float* wts, const float* ys, uint16_t* h, const uint16_t* w, float eps,
                            uint16_t* normed);
void launch_combine_tj(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s, const float* wts,
                       const float* ys, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared);
int launch_moe_fused(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                     const RouteReq& rq, uint32_t epoch, int spin_limit, const uint16_t* h,
                     hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
// With o1/o2 (one routed pair per token, no shared expert) it writes
// out = bf16(wts[token] * y) there instead of y, and no combine is needed.
void launch_q4k_down(hipStream_t st, const Geometry& g, const LayerView& L, int M, const Scratch& s,
                     const float* wts = nullptr, uint16_t* o1 = nullptr, uint16_t* o2 = nullptr);
// Host-side reorder of one packed Q4_K expert (gate|up|down, each [N][K/256]
// blocks of 144 B) into the device layout the linear kernel streams.
void repack_q4k_expert(const uint8_t* src, uint8_t* dst, int hd, int inter);
void repack_q4k_matrix(const uint8_t* src, uint8_t* dst, int N, int K);
// The same for an MXFP4 expert (2176-byte chunks of 16 rows x 256 weights).
void repack_mx_expert(const uint8_t* src, uint8_t* dst, int hd, int inter);
// Synthetic Q4_K matrix [N][K/256] (blocks b0.. of generator stream `id`)
// written in the device layout at dst.
void launch_synth_q4k_tiled(hipStream_t st, uint64_t seed, uint64_t id, uint64_t b0, int N, int K, float sigma,
                            uint8_t* dst);
void launch_synth_mx_tiled(hipStream_t st, uint64_t seed, uint64_t id, uint64_t b0, int N, int K, int e_lo,
                           int e_hi, uint8_t* dst);
// out = bf16(sum_j w_j y[pair(t,j)] + shared) per token (see combine_kernel).
void launch_combine(hipStream_t st, const Geometry& g, int M, int use_shared, const Scratch& s,
                    const float* wts, const float* ys, uint16_t* out, uint16_t* out_routed, uint16_t* out_shared);
void launch_copy(hipStream_t st, void* dst, const void* src, size_t bytes);
void launch_dequant(hipStream_t st, int codec, const uint8_t* blocks, size_t nblocks,
                    float* out_f32, uint16_t* out_bf16);

// Acceptance.  Work buffers are carved from `ws` (bytes given by accept_ws_bytes).
size_t accept_ws_bytes(int n_seq, int k, int V);
// Greedy acceptance: chunk words at `words` (n_seq*(k+1)*kGreedyChunks
// 64-bit words; accept_greedy_words gives them inside a workspace), tagged
// with epoch (1..4095, a new one per call on the same words); the owner's
// wait gives up after spin_limit polls and reports n_acc = -1.
constexpr int kGreedyChunks = 16;
constexpr int kMaxAcceptVocab = (1 << 20) - 2;   // index + 1 fits the word's 20-bit field
constexpr int kDefaultSpinLimit = 1 << 20;
void* accept_greedy_words(void* ws, int n_seq, int k);
void launch_accept_greedy(hipStream_t st, const float* target, int n_seq, int k, int V,
                          const int32_t* draft, int32_t* n_acc, int32_t* tokens, void* words, uint32_t epoch,
                          int spin_limit);
// sample_token over n_rows rows of V logits (one token per row; row r draws
// with Philox (seed, seq_base + r)); ws holds sample_ws_bytes.
size_t sample_ws_bytes(int n_rows, int V);
void launch_sample_token(hipStream_t st, const float* logits, int n_rows, int V, float temperature, float top_p,
                         uint64_t seed, uint64_t seq_base, void* ws, int32_t* tokens);
// The allocation-free greedy entry point's fixed device scratch (rows =
// n_seq*(k+1) at most kStaticGreedyRows): accept_scratch_init looks its
// address up for `device` (which must be current), once; accept_scratch_ptr
// returns it (null before init); accept_scratch_epoch hands out the device's
// next epoch.
constexpr int kStaticGreedyRows = 2048;
int accept_scratch_init(int device);
void* accept_scratch_ptr(int device);
uint32_t accept_scratch_epoch(int device);
// Zeroes the whole fixed greedy array of the device with a fill kernel on st
// (no memset node, so the call stays capturable).  Run before the call that
// takes epoch 1 again: words a timed-out call wrote after its owner left
// carry that call's epoch and may sit at offsets later shapes do not
// rewrite; clearing at every wrap keeps them from matching a reused epoch.
void accept_scratch_clear(hipStream_t st, void* words);
// Rejection sampling in two launches: every row's chunk softmax partials,
// then the decisions, the exponential race and the token.
void launch_accept_stochastic(hipStream_t st, const float* target, const float* draft_logits,
                              int n_seq, int k, int V, const int32_t* draft, float inv_t,
                              uint64_t seed, uint64_t seq_base, int32_t* n_acc, int32_t* tokens,
                              void* ws);

}  // namespace fst
