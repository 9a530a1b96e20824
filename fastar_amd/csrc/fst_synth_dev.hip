// fst_synth_dev.hip — synthetic Q4_K weights generated directly in HBM, in
// the wave-tiled device layout (see fst_layout.cpp), with the same bytes as
// the host generator (fst_synth_gen.h).  Used to fill multi-gigabyte expert
// banks without a host round trip.
#include "fst_internal.h"
#include "fst_synth_gen.h"

namespace fst {

// One thread per 144-byte block of one [N][K/256] matrix whose first block is
// block b0 of generator stream `id`.  Word k of the block (4-byte little
// endian) is d | dmin << 16 for k = 0 and Philox word k-1 for k = 1..35.
__global__ __launch_bounds__(256) void synth_q4k_tiled_kernel(uint64_t seed, uint64_t id, uint64_t b0, int N,
                                                              int nsb, float sigma, uint8_t* __restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * nsb) return;
    const int n = (int)(i / nsb), sb = (int)(i - (size_t)n * nsb);
    const uint64_t b = b0 + i;
    const uint64_t lane = kFstSynthTagQ4k ^ (id << 8);
    uint32_t w[36];
#pragma unroll
    for (int j = 0; j < 9; ++j) {
        const fst_philox_ctr r = fst_synth_philox(seed, b, lane | (uint64_t)j);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (1 + 4 * j + k < 36) w[1 + 4 * j + k] = r.v[k];
    }
    const uint16_t d = fst_f32_to_f16_bits((float)(fst_synth_halfnormal(seed, b, lane | 16u) * (double)sigma));
    const uint16_t dm = fst_f32_to_f16_bits((float)(fst_synth_halfnormal(seed, b, lane | 32u) * (double)sigma));
    w[0] = (uint32_t)d | ((uint32_t)dm << 16);
    uint8_t* chunk = dst + ((size_t)(n >> 4) * nsb + sb) * 2304;
    const int r = n & 15;
    *reinterpret_cast<uint4*>(chunk + 2048 + 16 * r) = make_uint4(w[0], w[1], w[2], w[3]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int L = 16 * g + r;
        *reinterpret_cast<uint4*>(chunk + 16 * L) = make_uint4(w[4 + 8 * g], w[5 + 8 * g], w[6 + 8 * g], w[7 + 8 * g]);
        *reinterpret_cast<uint4*>(chunk + 1024 + 16 * L) =
            make_uint4(w[8 + 8 * g], w[9 + 8 * g], w[10 + 8 * g], w[11 + 8 * g]);
    }
}

void launch_synth_q4k_tiled(hipStream_t st, uint64_t seed, uint64_t id, uint64_t b0, int N, int K, float sigma,
                            uint8_t* dst) {
    const size_t nblk = (size_t)N * (K / 256);
    hipLaunchKernelGGL(synth_q4k_tiled_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, seed, id, b0,
                       N, K / 256, sigma, dst);
}

// MXFP4: one thread per 17-byte block of one [N][K/32] matrix (blocks b0..
// of stream `id`), written in the MXFP4 device layout (fst_layout.cpp).
__global__ __launch_bounds__(256) void synth_mx_tiled_kernel(uint64_t seed, uint64_t id, uint64_t b0, int N,
                                                             int bpr, int e_lo, int e_hi, uint8_t* __restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * bpr) return;
    const int n = (int)(i / bpr), kb = (int)(i - (size_t)n * bpr);
    uint8_t blk[17];
    fst_synth_mx_block(seed, id, b0 + i, e_lo, e_hi, blk);
    const int nsb = bpr / 8, sb = kb >> 3, j = kb & 7, r = n & 15;
    uint8_t* chunk = dst + ((size_t)(n >> 4) * nsb + sb) * 2176;
    chunk[2048 + 8 * r + j] = blk[0];
    uint8_t* q = chunk + (j & 1) * 1024 + 16 * (16 * (j >> 1) + r);
    uint32_t w[4];
    for (int k = 0; k < 4; ++k)
        w[k] = (uint32_t)blk[1 + 4 * k] | ((uint32_t)blk[2 + 4 * k] << 8) | ((uint32_t)blk[3 + 4 * k] << 16) |
               ((uint32_t)blk[4 + 4 * k] << 24);
    *reinterpret_cast<uint4*>(q) = make_uint4(w[0], w[1], w[2], w[3]);
}

void launch_synth_mx_tiled(hipStream_t st, uint64_t seed, uint64_t id, uint64_t b0, int N, int K, int e_lo,
                           int e_hi, uint8_t* dst) {
    const size_t nblk = (size_t)N * (K / 32);
    hipLaunchKernelGGL(synth_mx_tiled_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, st, seed, id, b0,
                       N, K / 32, e_lo, e_hi, dst);
}

}  // namespace fst
