// fst_synth_gen.h — the synthetic Q4_K block generator, shared by the host
// (fst_synth_q4k_*) and the device (bank fill) so both produce the same bytes.
//
// Block b of matrix/expert `id` under `seed`:
//   bytes 4..143 (12 scale/min bytes, 128 nibble bytes): Philox-4x32-10
//     words of counters (b, tag ^ id<<8 | j), j = 0..8, in order;
//   d, dmin = fp16(|z| * sigma), z ~ N(0,1) by Irwin-Hall: the sum of twelve
//     24-bit uniforms / 2^24 - 6.  Every step is exact or one IEEE rounding
//     (integer sum, exact scaling, one double multiply, one float cast, one
//     fp16 rounding), so host and device agree bit for bit.
#pragma once
#include <stdint.h>

#include "../../include/fst_exact_math.h"

FST_HD fst_philox_ctr fst_synth_philox(uint64_t seed, uint64_t a, uint64_t b) {
    fst_philox_ctr c;
    c.v[0] = (uint32_t)a;
    c.v[1] = (uint32_t)(a >> 32);
    c.v[2] = (uint32_t)b;
    c.v[3] = (uint32_t)(b >> 32);
    return fst_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
}

// binary32 -> binary16 bits, round to nearest even (subnormals, overflow, NaN).
FST_HD uint16_t fst_f32_to_f16_bits(float f) {
    const uint32_t x = fst_f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (ax < 0x33000000u) return (uint16_t)sign;               // < 2^-25 -> 0
    const int e = (int)(ax >> 23) - 127;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    if (e < -14) {
        // subnormal: value = m * 2^(e-23); target unit 2^-24
        const int shift = -14 - e + 13;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = m >> 13;
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    uint32_t he = (uint32_t)(e + 15);
    if (q == 0x800u) {
        q = 0x400u;
        ++he;
    }
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (he << 10) | (q & 0x3ffu));
}

// |N(0,1)| by Irwin-Hall over the 12 words of three Philox outputs.
FST_HD double fst_synth_halfnormal(uint64_t seed, uint64_t a, uint64_t lane) {
    uint32_t s = 0;
    for (uint64_t k = 0; k < 3; ++k) {
        const fst_philox_ctr r = fst_synth_philox(seed, a, lane | k);
        s += (r.v[0] >> 8) + (r.v[1] >> 8) + (r.v[2] >> 8) + (r.v[3] >> 8);
    }
    const double z = (double)s * (1.0 / 16777216.0) - 6.0;
    return z < 0.0 ? -z : z;
}

constexpr uint64_t kFstSynthTagQ4k = 0x51344bull << 40;

// One 144-byte Q4_K block (see the header comment).
FST_HD void fst_synth_q4k_block(uint64_t seed, uint64_t id, uint64_t b, float d_sigma, uint8_t* blk) {
    const uint64_t lane = kFstSynthTagQ4k ^ (id << 8);
    for (int j = 0; j < 9; ++j) {
        const fst_philox_ctr r = fst_synth_philox(seed, b, lane | (uint64_t)j);
        for (int w = 0; w < 4; ++w)
            for (int k = 0; k < 4; ++k) {
                const int o = 16 * j + 4 * w + k;
                if (o < 140) blk[4 + o] = (uint8_t)(r.v[w] >> (8 * k));
            }
    }
    const uint16_t d = fst_f32_to_f16_bits((float)(fst_synth_halfnormal(seed, b, lane | 16u) * (double)d_sigma));
    const uint16_t dmin = fst_f32_to_f16_bits((float)(fst_synth_halfnormal(seed, b, lane | 32u) * (double)d_sigma));
    blk[0] = (uint8_t)d;
    blk[1] = (uint8_t)(d >> 8);
    blk[2] = (uint8_t)dmin;
    blk[3] = (uint8_t)(dmin >> 8);
}

constexpr uint64_t kFstSynthTagMx = 0x4d5846ull << 40;

// One 17-byte MXFP4 block b of expert `id`: scale byte e_lo + (word % (e_hi -
// e_lo)) from counter (b, tag ^ id<<8 | 1), then the 16 nibble bytes = the
// Philox words of counter (b, tag ^ id<<8).
FST_HD void fst_synth_mx_block(uint64_t seed, uint64_t id, uint64_t b, int e_lo, int e_hi, uint8_t* blk) {
    const uint64_t lane = kFstSynthTagMx ^ (id << 8);
    const fst_philox_ctr r0 = fst_synth_philox(seed, b, lane);
    const fst_philox_ctr r1 = fst_synth_philox(seed, b, lane | 1u);
    blk[0] = (uint8_t)(e_lo + (int)(r1.v[0] % (uint32_t)(e_hi - e_lo)));
    for (int w = 0; w < 4; ++w)
        for (int k = 0; k < 4; ++k) blk[1 + 4 * w + k] = (uint8_t)(r0.v[w] >> (8 * k));
}
