// fst_q4k_dev.h — device helpers shared by the Q4_K kernels: vector types,
// the power-of-two operand prescale and the exact per-lane Q4_K decode into
// fp16 MFMA operands.  Not part of the public ABI.
#pragma once
#include "fst_internal.h"

namespace fst {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ float half_bits_to_f32(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// Power-of-two prescale of a row whose largest finite |x| is a: the s with
// a*2^-s in [2^9, 2^10) (0 for a zero, infinite or NaN maximum).
__device__ __forceinline__ int prescale_exp(float a) {
    int s = 0;
    if (a > 0.0f && a < INFINITY) {
        int e;
        frexpf(a, &e);  // a = f*2^e, f in [0.5,1)
        s = e - 10;
    }
    return s;
}

// Per-lane decode of one super-block row slice.  Lane (row r = lane&15, group
// g = lane>>4) owns qs bytes [32g, 32g+32): low nibbles are sub-block 2g,
// high nibbles 2g+1; B operand c holds elements 64g+4c+{0,2,1,3}, 64g+32+4c+{0,2,1,3}.
typedef uint32_t u4v_t __attribute__((ext_vector_type(4)));

struct Q4kScale {
    h8_t SC8, NEG8;  // {sc_a x4, sc_b/16 x4}, {-1024 sc_a x4, -64 sc_b x4}
    h8_t m;
    float d, dmin;
};

// perm selector placing bytes 2(g&1) and 2(g&1)+1 of a dword into the low
// byte of each 16-bit half (v_perm_b32: 0..3 pick source bytes, 0x0C gives 0)
__device__ __forceinline__ uint32_t q4k_scale_sel(int g) {
    const uint32_t a = 2u * (uint32_t)(g & 1);
    return 0x0C000C00u | ((a + 1u) << 16) | a;
}

// The two 6-bit fields of lane group g as an exact fp16 pair: (x & 63) | fp16
// 1024 (one v_and_or_b32 on the spread bytes), minus 1024 (one v_pk_add_f16).
__device__ __forceinline__ h2_t q4k_field_pair(uint32_t bytes, uint32_t sel) {
    const uint32_t spread = __builtin_amdgcn_perm(0u, bytes, sel);
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(spread), "v"(0x003F003Fu), "v"(0x64006400u));
    return as_h2(r) - h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
}

__device__ __forceinline__ void q4k_scales(const u4v_t hdr, int g, uint32_t sel, Q4kScale& S) {
    S.d = half_bits_to_f32(hdr.x & 0xffffu);
    S.dmin = half_bits_to_f32(hdr.x >> 16);
    const uint32_t y = hdr.y, z = hdr.z, w = hdr.w;
    // get_scale_min_k4 byte-parallel: sub-blocks 0..3 in the low 6 bits of
    // q[0..3] / q[4..7]; 4..7 from q[8..11] nibbles and the top bits of q[0..7]
    const uint32_t SC = g < 2 ? y : ((w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u));
    const uint32_t MM = g < 2 ? z : (((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u));
    const h2_t sc = q4k_field_pair(SC, sel), mm = q4k_field_pair(MM, sel);
    const h2_t f = sc * h2_t{(_Float16)1.0f, (_Float16)0.0625f};          // sc_a, sc_b/16
    const h2_t n = sc * h2_t{(_Float16)-1024.0f, (_Float16)-64.0f};       // -1024 sc_a, -64 sc_b
    S.SC8 = h8_t{f.x, f.x, f.x, f.x, f.y, f.y, f.y, f.y};
    S.NEG8 = h8_t{n.x, n.x, n.x, n.x, n.y, n.y, n.y, n.y};
    const _Float16 z0 = (_Float16)0.0f;
    S.m = h8_t{mm.x, mm.y, mm.x, mm.y, z0, z0, z0, z0};
}

// Exact fp16 sc*q for the 8 weights held in one dword D = [b3 b2 b1 b0] of
// nibble bytes.  (x & m) | MAGIC (one v_and_or_b32) turns a nibble pair into
// fp16 (1024 + q) (low nibbles) or (1024 + 16q) (high nibbles); one
// v_pk_fma_f16 then gives (1024+q)*sc - 1024*sc = q*sc exactly (<= 945).
// Slot order of the result: elements {0,2,1,3} of the low nibbles, then
// {0,2,1,3} of the high nibbles (the activation operand is laid out to match).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

__device__ __forceinline__ h8_t q4k_bop(uint32_t D, const Q4kScale& S, uint32_t magic) {
    const uint32_t D8 = D >> 8;
    const u4v_t X = {and_or(D, 0x000F000Fu, magic), and_or(D8, 0x000F000Fu, magic),
                     and_or(D, 0x00F000F0u, magic), and_or(D8, 0x00F000F0u, magic)};
    return __builtin_elementwise_fma(__builtin_bit_cast(h8_t, X), S.SC8, S.NEG8);
}

// (ext-vector members: HIP's uint4 struct copies defeat scalar replacement
// and put the register ring in scratch)
struct WRaw {
    u4v_t h, a, b;
};
// The 32x32 tile's lane data: header and four 16-byte nibble pieces.
struct WRaw2 {
    u4v_t h, a, b, a1, b1;
};
typedef float f16v_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ u4v_t ld_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u4v_t*>(p));
}

// One 2304-byte chunk = 16 rows x one super-block: [0,1024) nibble bytes
// [32g, 32g+16) of row r at lane slot 16g+r, [1024,2048) bytes [32g+16,
// 32g+32), [2048,2304) the 16-byte headers (d, dmin, scales) of rows 0..15.
// Each of the three loads is one contiguous span across the wave.
__device__ __forceinline__ WRaw load_wraw(const uint8_t* chunk, int lane) {
    WRaw w;
    w.a = ld_stream(chunk + 16 * lane);
    w.b = ld_stream(chunk + 1024 + 16 * lane);
    w.h = ld_stream(chunk + 2048 + 16 * (lane & 15));
    return w;
}

}  // namespace fst
