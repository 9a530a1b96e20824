// fst_layout.cpp — device layout of resident Q4_K experts.
//
// The packed expert handed over at the ABI is the reference's byte format:
// gate | up | down, each a row-major [N rows][K/256] array of 144-byte Q4_K
// super-blocks (scripts/fst_converter.py:64-92 orientation, block format of
// kernels/fst_dequant_q4k_kernel.cc).  On upload each matrix is reordered so
// the linear kernel's 64-lane wave reads it with contiguous, fully coalesced
// 1 KiB loads, front to back:
//
//   matrix = [N/16 row tiles][K/256 super-blocks] chunks of 2304 bytes;
//   chunk (t, sb) holds super-block sb of rows 16t .. 16t+15:
//     [0,    1024)  lane L = 16g + r: qs bytes [32g,    32g+16) of row r
//     [1024, 2048)  lane L = 16g + r: qs bytes [32g+16, 32g+32) of row r
//     [2048, 2304)  row r: the 16-byte header (d, dmin, 12 scale bytes)
//
// Every byte of every block is kept; only their order changes, so the device
// copy holds exactly the packed expert's 14,155,776 bytes (4096/2048 shape).
#include <cstring>
#include <thread>
#include <vector>

#include "fst_internal.h"

namespace fst {

static void repack_matrix(const uint8_t* src, uint8_t* dst, int N, int K) {
    const int nsb = K / 256;
    for (int t = 0; t < N / 16; ++t)
        for (int sb = 0; sb < nsb; ++sb) {
            uint8_t* chunk = dst + ((size_t)t * nsb + sb) * 2304;
            for (int r = 0; r < 16; ++r) {
                const uint8_t* b = src + ((size_t)(t * 16 + r) * nsb + sb) * 144;
                std::memcpy(chunk + 2048 + 16 * r, b, 16);
                for (int g = 0; g < 4; ++g) {
                    const int L = 16 * g + r;
                    std::memcpy(chunk + 16 * L, b + 16 + 32 * g, 16);
                    std::memcpy(chunk + 1024 + 16 * L, b + 32 + 32 * g, 16);
                }
            }
        }
}

// Large matrices (the LM head) are split over row tiles between threads.
void repack_q4k_matrix(const uint8_t* src, uint8_t* dst, int N, int K) {
    const int tiles = N / 16, nt = 8;
    const size_t tile_src = (size_t)16 * (K / 256) * 144;
    std::vector<std::thread> th;
    for (int i = 0; i < nt; ++i) {
        const int t0 = tiles * i / nt, t1 = tiles * (i + 1) / nt;
        if (t0 >= t1) continue;
        th.emplace_back([=] { repack_matrix(src + t0 * tile_src, dst + t0 * tile_src, (t1 - t0) * 16, K); });
    }
    for (auto& t : th) t.join();
}

void repack_q4k_expert(const uint8_t* src, uint8_t* dst, int hd, int inter) {
    const size_t proj = (size_t)inter * (hd / 256) * 144;
    std::thread a([&] { repack_matrix(src, dst, inter, hd); });
    std::thread b([&] { repack_matrix(src + proj, dst + proj, inter, hd); });
    repack_matrix(src + 2 * proj, dst + 2 * proj, hd, inter);
    a.join();
    b.join();
}

// MXFP4 (17-byte blocks of 32 weights: e8m0 scale byte, then 16 bytes with
// elements 2i / 2i+1 in the low / high nibble of byte i) in the same spirit:
//
//   matrix = [N/16 row tiles][K/256] chunks of 2176 bytes; chunk (t, sb)
//   holds the 8 blocks of K range [256 sb, 256 sb + 256) of rows 16t..16t+15:
//     [0,    1024)  lane L = 16g + r: the 16 nibble bytes of block 2g   of row r
//     [1024, 2048)  lane L = 16g + r: the 16 nibble bytes of block 2g+1 of row r
//     [2048, 2176)  row r: the 8 scale bytes of its blocks 0..7
//
// so lane (g, r) holds the 64 consecutive weights [64g, 64g+64) of the
// super-block range, and the expert keeps exactly its packed size.
static void repack_mx_matrix(const uint8_t* src, uint8_t* dst, int N, int K) {
    const int nsb = K / 256, bpr = K / 32;
    for (int t = 0; t < N / 16; ++t)
        for (int sb = 0; sb < nsb; ++sb) {
            uint8_t* chunk = dst + ((size_t)t * nsb + sb) * 2176;
            for (int r = 0; r < 16; ++r) {
                const uint8_t* row = src + (size_t)(t * 16 + r) * bpr * 17;
                for (int j = 0; j < 8; ++j) {
                    const uint8_t* b = row + (size_t)(sb * 8 + j) * 17;
                    chunk[2048 + 8 * r + j] = b[0];
                    const int g = j >> 1, L = 16 * g + r;
                    std::memcpy(chunk + (j & 1) * 1024 + 16 * L, b + 1, 16);
                }
            }
        }
}

void repack_mx_expert(const uint8_t* src, uint8_t* dst, int hd, int inter) {
    const size_t proj = (size_t)inter * (hd / 32) * 17;
    std::thread a([&] { repack_mx_matrix(src, dst, inter, hd); });
    std::thread b([&] { repack_mx_matrix(src + proj, dst + proj, inter, hd); });
    repack_mx_matrix(src + 2 * proj, dst + 2 * proj, hd, inter);
    a.join();
    b.join();
}

}  // namespace fst
