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
#include "fst_synth_gen.h"

namespace {

inline fst_philox_ctr philox(uint64_t seed, uint64_t a, uint64_t b) {
    fst_philox_ctr c;
    c.v[0] = (uint32_t)a;
    c.v[1] = (uint32_t)(a >> 32);
    c.v[2] = (uint32_t)b;
    c.v[3] = (uint32_t)(b >> 32);
    return fst_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
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


}  // namespace

extern "C" {

int fst_synth_q4k_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, float d_sigma, uint8_t* out) {
    if (!out || hd <= 0 || inter <= 0 || hd % 256 || inter % 256) return FST_EINVAL;
    return fst_synth_q4k_blocks(seed, expert_id, 3 * (size_t)hd * inter / 256, d_sigma, out);
}

int fst_synth_q4k_blocks(uint64_t seed, uint64_t id, size_t nblocks, float d_sigma, uint8_t* out) {
    if (!out) return FST_EINVAL;
    parallel_for(nblocks, [&](size_t b0, size_t b1) {
        for (size_t b = b0; b < b1; ++b) fst_synth_q4k_block(seed, id, b, d_sigma, out + b * 144);
    });
    return FST_OK;
}

int fst_synth_mxfp4_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, int e_lo, int e_hi,
                           uint8_t* out) {
    if (!out || hd <= 0 || inter <= 0 || hd % 32 || inter % 32 || e_lo < 0 || e_hi > 256 || e_lo >= e_hi)
        return FST_EINVAL;
    const size_t nblk = 3 * (size_t)hd * inter / 32;
    parallel_for(nblk, [&](size_t b0, size_t b1) {
        for (size_t b = b0; b < b1; ++b) fst_synth_mx_block(seed, expert_id, b, e_lo, e_hi, out + b * 17);
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
