// fst_synth.cpp — deterministic synthetic inputs for the benchmark configs.
//
// Every byte is a pure function of (seed, tensor id, element index) through
// Philox-4x32-10, so the workload can be regenerated on any host from the
// repository alone and generation parallelises without changing the result.
// Normals come from Box-Muller in double precision.
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/fst_exact_math.h"
#include "../../include/fst_hip.h"

namespace {

inline fst_philox_ctr philox(uint64_t seed, uint64_t a, uint64_t b) {
    fst_philox_ctr c;
    c.v[0] = (uint32_t)a;
    c.v[1] = (uint32_t)(a >> 32);
    c.v[2] = (uint32_t)b;
    c.v[3] = (uint32_t)(b >> 32);
    return fst_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
}

// binary32 -> binary16 bits, round to nearest even (subnormals and overflow handled).
uint16_t f32_to_f16(float f) {
    uint32_t x = fst_f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (ax < 0x33000000u) return (uint16_t)sign;               // < 2^-25 -> 0
    int e = (int)(ax >> 23) - 127;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    if (e < -14) {
        // subnormal: value = m * 2^(e-23); target unit 2^-24
        int shift = -14 - e + 13;  // bits to drop from the 24-bit significand to units of 2^-24
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = m >> 13;
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    uint32_t he = (uint32_t)(e + 15);
    if (q == 0x800u) {
        q = 0x400u;
        ++he;
    }
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (he << 10) | (q & 0x3ffu));
}

void normal_pair(fst_philox_ctr r, double* z0, double* z1) {
    const double u1 = ((double)r.v[0] + 1.0) * (1.0 / 4294967296.0);  // (0,1]
    const double u2 = (double)r.v[1] * (1.0 / 4294967296.0);          // [0,1)
    const double rad = std::sqrt(-2.0 * std::log(u1));
    *z0 = rad * std::cos(2.0 * M_PI * u2);
    *z1 = rad * std::sin(2.0 * M_PI * u2);
}

template <typename F>
void parallel_for(size_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < 4096 || nt == 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> th;
    size_t per = (n + nt - 1) / nt;
    for (unsigned i = 0; i < nt; ++i) {
        size_t b = i * per, e = std::min(n, b + per);
        if (b >= e) break;
        th.emplace_back([=] { f(b, e); });
    }
    for (auto& t : th) t.join();
}

constexpr uint64_t kTagQ4k = 0x51344bull << 40;
constexpr uint64_t kTagMx = 0x4d5846ull << 40;

}  // namespace

extern "C" {

int fst_synth_q4k_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, float d_sigma, uint8_t* out) {
    if (!out || hd <= 0 || inter <= 0 || hd % 256 || inter % 256) return FST_EINVAL;
    const size_t nblk = 3 * (size_t)hd * inter / 256;
    parallel_for(nblk, [&](size_t b0, size_t b1) {
        for (size_t b = b0; b < b1; ++b) {
            uint8_t* blk = out + b * 144;
            const uint64_t lane = kTagQ4k ^ (expert_id << 8);
            // 140 random bytes: scales[12] then qs[128]
            uint8_t rnd[144];
            for (int j = 0; j < 9; ++j) {
                fst_philox_ctr r = philox(seed, b, lane | (uint64_t)j);
                std::memcpy(rnd + 16 * j, r.v, 16);
            }
            double z0, z1;
            normal_pair(philox(seed, b, lane | 9u), &z0, &z1);
            const uint16_t d = f32_to_f16((float)std::fabs(z0 * d_sigma));
            const uint16_t dmin = f32_to_f16((float)std::fabs(z1 * d_sigma));
            blk[0] = (uint8_t)d;
            blk[1] = (uint8_t)(d >> 8);
            blk[2] = (uint8_t)dmin;
            blk[3] = (uint8_t)(dmin >> 8);
            std::memcpy(blk + 4, rnd, 140);
        }
    });
    return FST_OK;
}

int fst_synth_mxfp4_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, int e_lo, int e_hi,
                           uint8_t* out) {
    if (!out || hd <= 0 || inter <= 0 || hd % 32 || inter % 32 || e_lo < 0 || e_hi > 256 || e_lo >= e_hi)
        return FST_EINVAL;
    const size_t nblk = 3 * (size_t)hd * inter / 32;
    parallel_for(nblk, [&](size_t b0, size_t b1) {
        for (size_t b = b0; b < b1; ++b) {
            uint8_t* blk = out + b * 17;
            const uint64_t lane = kTagMx ^ (expert_id << 8);
            fst_philox_ctr r0 = philox(seed, b, lane);
            fst_philox_ctr r1 = philox(seed, b, lane | 1u);
            blk[0] = (uint8_t)(e_lo + (int)(r1.v[0] % (uint32_t)(e_hi - e_lo)));
            std::memcpy(blk + 1, r0.v, 16);
        }
    });
    return FST_OK;
}

int fst_synth_normal_f32(uint64_t seed, uint64_t stream, size_t n, float mean, float std_, float* out) {
    if (!out) return FST_EINVAL;
    const size_t np = (n + 1) / 2;
    parallel_for(np, [&](size_t p0, size_t p1) {
        for (size_t p = p0; p < p1; ++p) {
            double z0, z1;
            normal_pair(philox(seed, p, stream), &z0, &z1);
            out[2 * p] = (float)(mean + std_ * z0);
            if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std_ * z1);
        }
    });
    return FST_OK;
}

int fst_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t n, float mean, float std_, uint16_t* out) {
    if (!out) return FST_EINVAL;
    const size_t np = (n + 1) / 2;
    parallel_for(np, [&](size_t p0, size_t p1) {
        for (size_t p = p0; p < p1; ++p) {
            double z0, z1;
            normal_pair(philox(seed, p, stream), &z0, &z1);
            out[2 * p] = fst_f32_to_bf16((float)(mean + std_ * z0));
            if (2 * p + 1 < n) out[2 * p + 1] = fst_f32_to_bf16((float)(mean + std_ * z1));
        }
    });
    return FST_OK;
}

}  // extern "C"
