// fst_dense.hip — linear layers over plain bf16 weight matrices for gfx950.
//
// The reference keeps two matrices of the verify path in bf16 rather than in
// an expert codec: the shared expert (TID_SHARED_GATE/UP/DOWN, run by
// process_shared_expert, src/fst_engine.cpp:4373-4489, "same chain with
// preloaded BF16 weights") and the LM head (apply_final_norm_and_lm_head,
// :2115-2160).  Both are stored [N][K] row-major (scripts/fst_converter.py
// _parse_state_dict; "[N,K] native", src/fst_engine.cpp:1613-1616), and this
// kernel reads them in that layout straight from HBM.
//
// Y[m][n] = sum_k W[n][k] x[m][k] with v_mfma_f32_16x16x32_bf16: weights are
// the B operand (16 rows per wave), tokens the A operand (16 per group, up to
// 4 groups).  A workgroup of 8 waves owns one to four 16-row tiles and splits
// K between the waves of a tile (gate||up: waves 0-3 take the gate rows,
// waves 4-7 the same up rows), and sums the wave partials through LDS in wave
// order, so results do not depend on scheduling.
//
// Each lane streams 64 contiguous bytes (32 k values) of its row per
// 128-wide K step; the four MFMAs of the step take the lane's values in
// 8-wide pieces.  The A operand takes the same k permutation, so the product
// is unchanged.  Two steps are in flight per wave; every load is
// unconditional and none reads past the wave's part of K.
#include "fst_internal.h"
#include "../../include/fst_exact_math.h"

namespace fst {

typedef __bf16 bf8v_t __attribute__((ext_vector_type(8)));
typedef float f4v_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4x_t __attribute__((ext_vector_type(4)));

constexpr int kDnWaves = 8;
constexpr int kDnThreads = 64 * kDnWaves;

struct DenseOut {
    float* y32;       // fp32 [M][N] (mode 0)
    uint16_t* y16a;   // bf16 [M][N] (mode 0), or h = silu(g)*u [M][N/2] (mode 1)
    uint16_t* y16b;   // second bf16 copy (mode 0)
    float swiglu_limit;
};

__device__ __forceinline__ bf8v_t as_bf8(u4x_t v) { return __builtin_bit_cast(bf8v_t, v); }

// The waves of a matrix half split K into SPLIT parts (a power of two that
// divides K/256, so each part is an even number of 128-wide steps) and the
// half's 16-row tiles (TPW of them per workgroup) among themselves.
__host__ __device__ constexpr int dense_split(int K, int waves) {
    return (K / 256) % waves == 0 ? waves : ((K / 256) % (waves / 2) == 0 ? waves / 2 : 2);
}

// MODE 0: Y = W x.  MODE 1: W holds N/2 gate rows then N/2 up rows; the
// output is h[m][j] = bf16(silu(g) * u) for j < N/2.
template <int NG, int MODE>
__global__ __launch_bounds__(kDnThreads) void bf16_linear_kernel(const uint16_t* __restrict__ W, int K, int N,
                                                                 const uint16_t* __restrict__ x, int M,
                                                                 DenseOut o) {
    __shared__ f4v_t red[kDnWaves][NG][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    constexpr int HW = MODE == 1 ? kDnWaves / 2 : kDnWaves;  // waves per matrix half
    const int split = dense_split(K, HW), tpw = HW / split;
    const int hw = MODE == 1 ? (wave & (HW - 1)) : wave;
    const int tile = hw / split, part = hw % split;
    const int row0 = (MODE == 1 && wave >= HW ? N / 2 : 0) + (blockIdx.x * tpw + tile) * 16;
    const int nst = (K >> 7) / split;  // even, >= 2
    const u4x_t* wrow = reinterpret_cast<const u4x_t*>(W + (size_t)(row0 + r) * K) + (size_t)part * nst * 16 + g * 4;
    const u4x_t* xrow[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        const int m = min(q * 16 + r, M - 1);  // rows >= M are computed and dropped
        xrow[q] = reinterpret_cast<const u4x_t*>(x + (size_t)m * K) + (size_t)part * nst * 16 + g * 4;
    }
    f4v_t acc[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) acc[q] = f4v_t{0.f, 0.f, 0.f, 0.f};

    u4x_t wr[2][4];
    u4x_t xr[2][NG][4];
    auto load = [&](int slot, int s) {
        const size_t off = (size_t)s * 16;  // 16 x 16 B per 128 k
#pragma unroll
        for (int j = 0; j < 4; ++j) wr[slot][j] = __builtin_nontemporal_load(wrow + off + j);
#pragma unroll
        for (int q = 0; q < NG; ++q)
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[slot][q][j] = xrow[q][off + j];
    };
    auto mma = [&](int slot) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < NG; ++q)
                acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xr[slot][q][j]), as_bf8(wr[slot][j]),
                                                                acc[q], 0, 0, 0);
    };
    load(0, 0);
    load(1, 1);
    for (int s = 0; s < nst - 2; s += 2) {
        mma(0);
        load(0, s + 2);
        mma(1);
        load(1, s + 3);
    }
    mma(0);
    mma(1);
#pragma unroll
    for (int q = 0; q < NG; ++q) red[wave][q][lane] = acc[q];
    __syncthreads();

    // lane layout of a 16x16 result: token 4g+i of group q, row r of the tile
    for (int it = wave; it < tpw * NG; it += kDnWaves) {
        const int t = it / NG, q = it % NG;
        const int n = (blockIdx.x * tpw + t) * 16 + r;
        if constexpr (MODE == 0) {
            f4v_t a = red[t * split][q][lane];
            for (int p = 1; p < split; ++p) a = a + red[t * split + p][q][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = q * 16 + 4 * g + i;
                if (m >= M) continue;
                if (o.y32) o.y32[(size_t)m * N + n] = a[i];
                if (o.y16a) o.y16a[(size_t)m * N + n] = fst_f32_to_bf16(a[i]);
                if (o.y16b) o.y16b[(size_t)m * N + n] = fst_f32_to_bf16(a[i]);
            }
        } else {
            f4v_t gs = red[t * split][q][lane], us = red[HW + t * split][q][lane];
            for (int p = 1; p < split; ++p) {
                gs = gs + red[t * split + p][q][lane];
                us = us + red[HW + t * split + p][q][lane];
            }
            const int inter = N / 2;
            const float lim = o.swiglu_limit;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = q * 16 + 4 * g + i;
                if (m >= M) continue;
                float gv = gs[i], uv = us[i];
                if (lim > 0.0f) {
                    gv = fminf(gv, lim);
                    uv = fminf(fmaxf(uv, -lim), lim);
                }
                o.y16a[(size_t)m * inter + n] = fst_f32_to_bf16((gv / (1.0f + expf(-gv))) * uv);
            }
        }
    }
}

template <int MODE>
static void launch_bf16_linear_mode(hipStream_t st, const uint16_t* W, int K, int N, const uint16_t* x, int M,
                                    const DenseOut& o) {
    constexpr int HW = MODE == 1 ? kDnWaves / 2 : kDnWaves;
    const int tpw = HW / dense_split(K, HW);
    const dim3 grid((MODE == 1 ? N / 2 : N) / (16 * tpw)), block(kDnThreads);
    if (M <= 16)
        hipLaunchKernelGGL((bf16_linear_kernel<1, MODE>), grid, block, 0, st, W, K, N, x, M, o);
    else if (M <= 32)
        hipLaunchKernelGGL((bf16_linear_kernel<2, MODE>), grid, block, 0, st, W, K, N, x, M, o);
    else
        hipLaunchKernelGGL((bf16_linear_kernel<4, MODE>), grid, block, 0, st, W, K, N, x, M, o);
}

// Rows per workgroup of a launch over K: the caller's N must be a multiple.
int bf16_linear_rows_per_wg(int K, int gate_up) {
    const int hw = gate_up ? kDnWaves / 2 : kDnWaves;
    return 16 * (hw / dense_split(K, hw));
}

// Y = W x over bf16 W [N][K] (K % 512 == 0, N a multiple of
// bf16_linear_rows_per_wg, 1 <= M <= 64): any of y32 (fp32), y16a, y16b
// (bf16) may be null.
void launch_bf16_linear(hipStream_t st, const uint16_t* W, int K, int N, const uint16_t* x, int M, float* y32,
                        uint16_t* y16a, uint16_t* y16b) {
    DenseOut o{y32, y16a, y16b, 0.0f};
    launch_bf16_linear_mode<0>(st, W, K, N, x, M, o);
}

// h[m][j] = bf16(silu(g) * u) with gate rows W[0, inter) and up rows
// W[inter, 2 inter).
void launch_bf16_gate_up(hipStream_t st, const uint16_t* W, int K, int inter, const uint16_t* x, int M,
                         float swiglu_limit, uint16_t* h) {
    DenseOut o{nullptr, h, nullptr, swiglu_limit};
    launch_bf16_linear_mode<1>(st, W, K, 2 * inter, x, M, o);
}

}  // namespace fst
