// Shared device helpers for the gfx950 MatMulNBits kernels.
//
// Unpacking follows ORT's MatMulNBits layout (reference: docs/OP_COVERAGE.md:4210-4230,
// rust/shaders/glsl/templates/q_gemv.comp:284-338): 4-bit weights low nibble first, zero points
// packed like B with per-column byte padding, implied zero point 1 << (bits-1).
//
// The fp16 dequantisation is exact by construction: a nibble or byte q is placed in the low
// mantissa bits of the fp16 value 1024 (0x6400), which makes the half 1024 + q (or 1024 + 16q for
// a high nibble kept in place); one packed FMA with (1, 1/16) and -(1024 + z, 64 + z) then yields
// the small integer q - z with no rounding, and a single packed multiply by the fp16 scale rounds
// once to nearest even: fp16_rne((q - z) * s), the bit-exact dequant definition.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnb {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// (a & m) | o in one v_and_or_b32.  gfx9 VOP3 cannot encode a literal and may read one SGPR,
// so the two constants are passed in VGPRs; left to itself the compiler emits v_and + v_or.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
    return r;
}

// Byte `i` of `w` copied into bits 0-7 and 16-23; bits 8-15 and 24-31 zero (v_perm_b32,
// selector 0x0c yields a zero byte).
template <int I>
__device__ __forceinline__ uint32_t dup_byte(uint32_t w) {
    constexpr uint32_t sel = (uint32_t)I | (0x0Cu << 8) | ((uint32_t)I << 16) | (0x0Cu << 24);
    return __builtin_amdgcn_perm(w, w, sel);
}

// The constant pair (1024 + z, 64 + z) that turns 4-bit magic halves into q - z.
__device__ __forceinline__ f16x2 zoff4(int z) {
    // z in 0..15: -(1024 + z) is 0xE400 | z and -(64 + z) is 0xD400 | (z << 4) in fp16 (the
    // exponent fields of 1024 and 64, z in the mantissa), formed without a conversion
    return as_h2(0xD400E400u | (uint32_t)z | ((uint32_t)z << 20));
}

// Four exact (q - z) pairs from one dword of eight 4-bit weights, natural element order:
// out[i] = (q[2i] - z, q[2i+1] - z).
template <int I>
__device__ __forceinline__ f16x2 nib_pair(uint32_t w, f16x2 zo) {
    const uint32_t t = and_or(dup_byte<I>(w), 0x00F0000Fu, 0x64006400u);
    const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
    return __builtin_elementwise_fma(as_h2(t), mul, zo);
}

// Eight exact fp16 (q - z) from one dword of the MFMA-native strip copy (launch_strip_pack with native set):
// its nibbles hold k0 k2 k4 k6 in bits 0-15 and k1 k3 k5 k7 in bits 16-31, so each pair (k_2p,
// k_2p+1) sits at one nibble position of the two halves -- (k0, k1), (k4, k5) at bits 0-3 of w
// and of w >> 8, giving 1024 + q less (1024 + z); (k2, k3), (k6, k7) at bits 4-7, giving
// 1024 + 16 q, times 1/16, less (64 + z).  One shift, four and-ors and four packed fp16 ops per
// dword (the ORT layout needs a byte duplicate per pair besides).
__device__ __forceinline__ f16x8 native_pairs(uint32_t w, f16x2 zlo, f16x2 zhi) {
    const uint32_t wh = w >> 8;
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    f16x8 r;
    r.s01 = as_h2(and_or(w, 0x000F000Fu, 0x64006400u)) + zlo;
    r.s23 = __builtin_elementwise_fma(as_h2(and_or(w, 0x00F000F0u, 0x64006400u)), sixteenth, zhi);
    r.s45 = as_h2(and_or(wh, 0x000F000Fu, 0x64006400u)) + zlo;
    r.s67 = __builtin_elementwise_fma(as_h2(and_or(wh, 0x00F000F0u, 0x64006400u)), sixteenth, zhi);
    return r;
}

// Eight fp16 dequantised weights (natural order) from one dword of 4-bit weights.
__device__ __forceinline__ f16x8 dequant8_4b(uint32_t w, f16x2 zo, f16x2 s2) {
    const f16x2 p0 = nib_pair<0>(w, zo) * s2;
    const f16x2 p1 = nib_pair<1>(w, zo) * s2;
    const f16x2 p2 = nib_pair<2>(w, zo) * s2;
    const f16x2 p3 = nib_pair<3>(w, zo) * s2;
    f16x8 r;
    r.s01 = p0;
    r.s23 = p1;
    r.s45 = p2;
    r.s67 = p3;
    return r;
}

// Two exact (q - z) pairs from one dword of four 8-bit weights: (q0-z, q1-z), (q2-z, q3-z).
__device__ __forceinline__ f16x2 byte_pair_lo(uint32_t w, f16x2 zo) {
    // bytes [b0, 0x64, b1, 0x64]
    const uint32_t t = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    return as_h2(t) + zo;
}
__device__ __forceinline__ f16x2 byte_pair_hi(uint32_t w, f16x2 zo) {
    // bytes [b2, 0x64, b3, 0x64]
    const uint32_t t = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    return as_h2(t) + zo;
}
__device__ __forceinline__ f16x2 zoff8(int z) {
    f16x2 r;
    r.x = (f16)(-(1024 + z));
    r.y = r.x;
    return r;
}

// Eight fp16 dequantised weights from two dwords of 8-bit weights.
__device__ __forceinline__ f16x8 dequant8_8b(uint32_t w0, uint32_t w1, f16x2 zo, f16x2 s2) {
    f16x8 r;
    r.s01 = byte_pair_lo(w0, zo) * s2;
    r.s23 = byte_pair_hi(w0, zo) * s2;
    r.s45 = byte_pair_lo(w1, zo) * s2;
    r.s67 = byte_pair_hi(w1, zo) * s2;
    return r;
}

// Zero point of (column n, block blk); implied 1 << (bits-1) when Z is null.
template <int BITS, bool HAS_ZP>
__device__ __forceinline__ int load_zp(const uint8_t* __restrict__ Z, int64_t n, int blk, int zpb) {
    if constexpr (!HAS_ZP) {
        return 1 << (BITS - 1);
    } else if constexpr (BITS == 4) {
        const uint32_t byte = Z[n * zpb + (blk >> 1)];
        return (int)((byte >> ((blk & 1) * 4)) & 0xFu);
    } else {
        return (int)Z[n * zpb + blk];
    }
}

// DPP lane permutation of a float (gfx9 dpp_ctrl encodings: quad_perm 0x00-0xFF,
// row_mirror 0x140, row_half_mirror 0x141).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                                0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G = 1, 2, 4, ..., 64); every lane of a group receives the
// group's sum.  Quad permutes and row mirrors are DPP modifiers on the add; the 16- and 32-lane
// steps exchange rows / half-waves with v_permlane16_swap / v_permlane32_swap.  The pairing is
// fixed, so the result is deterministic.
__device__ __forceinline__ float group_sum(float v, int G) {
    if (G >= 2) v += dpp_f<0xB1>(v);     // quad_perm [1,0,3,2]: lane ^ 1
    if (G >= 4) v += dpp_f<0x4E>(v);     // quad_perm [2,3,0,1]: lane ^ 2
    if (G >= 8) v += dpp_f<0x141>(v);    // row_half_mirror: lane i <-> 7 - i within 8
    if (G >= 16) v += dpp_f<0x140>(v);   // row_mirror: lane i <-> 15 - i within 16
    if (G >= 32) {
        const uint32_t x = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        v = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    }
    if (G >= 64) {
        const uint32_t x = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        v = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    }
    return v;
}

// Maximum over the 64 lanes of a wavefront, received by every lane (the exchanges of
// group_sum; fmaxf ignores a NaN operand).
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    uint32_t x = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    v = fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
    x = __builtin_bit_cast(uint32_t, v);
    const auto r2 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r2[0]),
                 __builtin_bit_cast(float, (uint32_t)r2[1]));
}

// 4 x 4 transpose of dwords across the lane rows (16 lanes each) of a wavefront: on return,
// v[t] of a lane in row g is what v[g] of the same column lane in row t held.
__device__ __forceinline__ void transpose_rows(uint32_t& v0, uint32_t& v1, uint32_t& v2,
                                               uint32_t& v3) {
    auto a = __builtin_amdgcn_permlane32_swap(v0, v2, false, false);
    v0 = a[0];
    v2 = a[1];
    auto b = __builtin_amdgcn_permlane32_swap(v1, v3, false, false);
    v1 = b[0];
    v3 = b[1];
    auto c = __builtin_amdgcn_permlane16_swap(v0, v1, false, false);
    v0 = c[0];
    v1 = c[1];
    auto d = __builtin_amdgcn_permlane16_swap(v2, v3, false, false);
    v2 = d[0];
    v3 = d[1];
}

// Eight int4 weights (one dword, natural order e0..e7) as int8 (q - z) in the order
// [e0, e2, e4, e6, e1, e3, e5, e7]; zb = (128 - z) in every byte.
__device__ __forceinline__ i32x2 qz_i8(uint32_t w, uint32_t zb) {
    // per byte: (q + 128 - z) has no carry for q, z in 0..15; XOR 0x80 gives (q - z) mod 256
    const uint32_t lo = ((w & 0x0F0F0F0Fu) + zb) ^ 0x80808080u;
    const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) + zb) ^ 0x80808080u;
    return i32x2{(int32_t)lo, (int32_t)hi};
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace mnb
