// Streaming decode GEMV for MatMulNBits with fp32 activations, scales and output (M <= 4 rows,
// 4- or 8-bit weights, blocks 16-128): the form ORT's CPU-exported int4 models use, which the
// reference's shader also serves (rust/shaders/glsl/templates/q_gemv.comp, float A/scales).
//
// Same launch design as the fp16 streaming GEMV (mnb_gemv_stream.hpp): one to four workgroups per
// CU; every thread first requests its share of the MR activation rows, then each lane its own
// chunks' block scales and zero points, then its first weight chunk; the activations are staged
// in LDS as they arrive and the rest of the lane's weights are issued at once; one workgroup
// barrier precedes the compute.  A lane group of G lanes owns one column and lane i takes the
// 16-byte chunks i, i + G, ... of it (32 int4 or 16 int8 weights each), so one load instruction
// covers 64/G runs of G*16 contiguous bytes.
//
// Staged in LDS: each chunk's activations as fp32 (128 or 64 bytes) followed by the fp32 sum of
// its activations per quant-block segment, padded to 144 / 80 bytes per chunk so that the 16
// lanes of a read quarter land in 16 distinct 4-bank groups (36 i mod 64 and 20 i mod 64 are
// distinct multiples of 4 for i = 0..15).
//
// Arithmetic.  The reference forms, per (column, quant block), the fp32 sum of a * (q - zp) and
// scales it once (q_gemv.comp:571-579).  Here the weights enter fp32 FMAs as fp16 subnormals
// q * 2^-24 (one AND per pair), which v_fma_mix_f32 reads as exact fp32 operands: one mixed FMA
// per weight, no conversion.  The chunk's partial over a block segment is recovered as
// sum a*q - zp * sum a  (the activation sum from the staging) and scaled by the block's scale in
// fp32.  The G lane accumulators of a column are summed by a fixed butterfly (run-to-run
// deterministic).
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

template <int BITS>
constexpr int f32_chunk_weights() { return 128 / BITS; }

// LDS bytes of one staged chunk: its activations and up to four segment sums.
template <int BITS>
__host__ __device__ constexpr int f32_chunk_stride() { return 4 * (128 / BITS) + 16; }

constexpr int kF32MaxCpl = 8;
constexpr int64_t kF32MaxRows = 64;                    // row-tiles of up to four rows above that
constexpr int64_t kF32MaxLds = 96 * 1024;
constexpr int kF32AU = 2;                               // 16-byte activation units per thread and batch

template <int BITS, int BS, bool HAS_ZP, int MR, int CPL>
__global__ void __launch_bounds__(kStreamMaxThreads)
gemv_stream_f32(const float* __restrict__ A, const uint8_t* __restrict__ B,
                const float* __restrict__ S, const uint8_t* __restrict__ Z, float* __restrict__ Y,
                int M, int N, int K, int log2g) {
    constexpr int WPC = f32_chunk_weights<BITS>();
    constexpr int UPC = WPC / 4;                         // 16-byte activation units per chunk
    constexpr int SEGS = WPC > BS ? WPC / BS : 1;        // quant-block segments per chunk
    constexpr int UPS = UPC / SEGS;                      // units per segment: 4 or 8
    constexpr int WPS = WPC / SEGS;                      // weights per segment
    constexpr int CST = f32_chunk_stride<BITS>();
    extern __shared__ __align__(16) uint8_t smem[];

    const int T = (int)blockDim.x;
    const int tid = (int)threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = 1 << log2g;
    const int ng = 64 >> log2g;
    const int grp = lane >> log2g;
    const int gi = lane & (G - 1);
    const int cpc = K / WPC;                             // chunks per column
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const int C = (T >> 6) * ng;                         // columns per workgroup
    const int col0 = (int)blockIdx.x * C;
    const int lc = wave * ng + grp;                      // this lane group's column
    const int col = min(col0 + lc, N - 1);
    const int m0 = (int)blockIdx.y * MR;
    const int upr = K / 4;                               // activation units per row
    const int a_units = MR * upr;

    // ---- 1. the first batch of activation units (clamped, unpredicated addresses: waiting
    // for them does not wait for the requests made after them) --------------------------------
    auto unit_src = [&](int u) {
        int r = 0;
#pragma unroll
        for (int rr = 1; rr < MR; ++rr) r += u >= rr * upr ? 1 : 0;
        return A + (int64_t)min(m0 + r, M - 1) * K + 4 * (int64_t)(u - r * upr);
    };
    u32x4 av[kF32AU];
#pragma unroll
    for (int i = 0; i < kF32AU; ++i)
        av[i] = *reinterpret_cast<const u32x4*>(unit_src(min(tid + i * T, a_units - 1)));

    // ---- 2. the lane's own block scales and zero points, then its first weight chunk ----------
    auto chunk_of = [&](int j) { return min(gi + j * G, cpc - 1); };
    float sc[CPL][SEGS], zf[CPL][SEGS];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int s = 0; s < SEGS; ++s) {
            const int blk = (chunk_of(j) * WPC + s * BS) / BS;
            sc[j][s] = S[(int64_t)col * bpc + blk];
            if constexpr (HAS_ZP) {
                const uint32_t zb = Z[(int64_t)col * zpb + (BITS == 4 ? blk >> 1 : blk)];
                zf[j][s] = (float)(BITS == 4 ? (zb >> ((blk & 1) * 4)) & 0xFu : zb);
            } else {
                zf[j][s] = (float)(1 << (BITS - 1));
            }
        }
    const uint8_t* bcol = B + (int64_t)col * ((int64_t)K * BITS / 8);
    u32x4 bw[CPL];
    bw[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bcol + 16 * chunk_of(0)));
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. stage the activations: unit u is chunk u / UPC (of its row), quarter u % UPC; the
    // UPS units of one segment sit in UPS consecutive lanes, whose sums are combined there ------
    auto stage = [&](int u, u32x4 x) {
        const bool live = u < a_units;
        const int uu = min(u, a_units - 1);
        int r = 0;
#pragma unroll
        for (int rr = 1; rr < MR; ++rr) r += uu >= rr * upr ? 1 : 0;
        const int w = uu - r * upr;
        const int c = w / UPC;
        const int q = w - c * UPC;
        uint8_t* dst = smem + (r * cpc + c) * CST;
        if (live) *reinterpret_cast<u32x4*>(dst + 16 * q) = x;
        // (the whole vector is reinterpreted: a bit cast of one element of an ext_vector
        // operand was compiled as a read of element 0 by this compiler)
        const f32x4 fx = __builtin_bit_cast(f32x4, x);
        float t = (fx[0] + fx[1]) + (fx[2] + fx[3]);
        t = live ? t : 0.f;
        t += dpp_f<0xB1>(t);                             // lane ^ 1
        t += dpp_f<0x4E>(t);                             // lane ^ 2
        if constexpr (UPS == 8) t += dpp_f<0x141>(t);    // the other quad of 8
        if (live && q % UPS == 0) reinterpret_cast<float*>(dst + 4 * WPC)[q / UPS] = t;
    };
#pragma unroll
    for (int i = 0; i < kF32AU; ++i) stage(tid + i * T, av[i]);
    for (int base = kF32AU * T; base < a_units; base += kF32AU * T) {
        u32x4 x[kF32AU];
#pragma unroll
        for (int i = 0; i < kF32AU; ++i)
            x[i] = *reinterpret_cast<const u32x4*>(unit_src(min(base + tid + i * T, a_units - 1)));
#pragma unroll
        for (int i = 0; i < kF32AU; ++i) stage(base + tid + i * T, x[i]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 4. the rest of the lane's weights, at once ------------------------------------------
#pragma unroll
    for (int j = 1; j < CPL; ++j)
        bw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bcol + 16 * chunk_of(j)));
    __syncthreads();

    // ---- 5. compute: per chunk, its weights as fp32 once, then each row's dot products -------
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const bool live = gi + j * G < cpc;
        const int c = chunk_of(j);
        // The chunk's weights as fp16 subnormal pairs q * 2^-24 (one AND each), read by
        // v_fma_mix_f32 as exact fp32 operands: int4 dword d gives (w[8d], w[8d+4]) and, masked in
        // place at 16 q * 2^-24, (w[8d+1], w[8d+5]); w >> 8 the same for 8d+2 / 8d+6 and
        // 8d+3 / 8d+7.  int8: bytes (0, 2) and, after a shift, (1, 3).
        const uint32_t wd[4] = {bw[j].x, bw[j].y, bw[j].z, bw[j].w};
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const uint8_t* src = smem + (r * cpc + c) * CST;
            float a[WPC];
#pragma unroll
            for (int v = 0; v < WPC / 4; ++v) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(src + 16 * v);
                a[4 * v + 0] = x[0];
                a[4 * v + 1] = x[1];
                a[4 * v + 2] = x[2];
                a[4 * v + 3] = x[3];
            }
            const float* asum = reinterpret_cast<const float*>(src + 4 * WPC);
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                float t = 0.f, t16 = 0.f;
#pragma unroll
                for (int d = 4 * s / SEGS; d < 4 * (s + 1) / SEGS; ++d) {
                    if constexpr (BITS == 4) {
                        const uint32_t wh = wd[d] >> 8;
                        const f16x2 p0 = as_h2(wd[d] & 0x000F000Fu), p1 = as_h2(wd[d] & 0x00F000F0u);
                        const f16x2 p2 = as_h2(wh & 0x000F000Fu), p3 = as_h2(wh & 0x00F000F0u);
                        t = __builtin_fmaf(a[8 * d + 0], (float)p0.x, t);
                        t = __builtin_fmaf(a[8 * d + 4], (float)p0.y, t);
                        t16 = __builtin_fmaf(a[8 * d + 1], (float)p1.x, t16);
                        t16 = __builtin_fmaf(a[8 * d + 5], (float)p1.y, t16);
                        t = __builtin_fmaf(a[8 * d + 2], (float)p2.x, t);
                        t = __builtin_fmaf(a[8 * d + 6], (float)p2.y, t);
                        t16 = __builtin_fmaf(a[8 * d + 3], (float)p3.x, t16);
                        t16 = __builtin_fmaf(a[8 * d + 7], (float)p3.y, t16);
                    } else {
                        const f16x2 p0 = as_h2(wd[d] & 0x00FF00FFu);
                        const f16x2 p1 = as_h2((wd[d] >> 8) & 0x00FF00FFu);
                        t = __builtin_fmaf(a[4 * d + 0], (float)p0.x, t);
                        t = __builtin_fmaf(a[4 * d + 2], (float)p0.y, t);
                        t = __builtin_fmaf(a[4 * d + 1], (float)p1.x, t);
                        t = __builtin_fmaf(a[4 * d + 3], (float)p1.y, t);
                    }
                }
                // sum a*q over the segment: 2^24 t + 2^20 t16 (exact power-of-two scalings)
                float p = __builtin_fmaf(t16, 0.0625f, t) * 16777216.0f;
                p = __builtin_fmaf(-zf[j][s], asum[s], p);
                acc[r] = __builtin_fmaf(live ? sc[j][s] : 0.f, p, acc[r]);
            }
        }
        // finish the chunk here (the compiler would otherwise hold every chunk's activations)
#pragma unroll
        for (int r = 0; r < MR; ++r) asm volatile("" : "+v"(acc[r]));
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = group_sum(acc[r], G);
    if (gi == 0 && col0 + lc < N) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (m0 + r < M) Y[(int64_t)(m0 + r) * N + col0 + lc] = acc[r];
    }
}

template <int BITS, int BS, bool HAS_ZP, int MR, int CPL>
hipError_t f32_go(const StreamConfig& c, const float* A, const uint8_t* B, const float* S,
                  const uint8_t* Z, float* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    auto kern = gemv_stream_f32<BITS, BS, HAS_ZP, MR, CPL>;
    const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), (size_t)c.lds);
    if (ea != hipSuccess) return ea;
    const dim3 grid((unsigned)c.groups, (unsigned)((m + MR - 1) / MR), 1);
    const dim3 block((unsigned)(64 * c.waves_per_group), 1, 1);
    hipLaunchKernelGGL(kern, grid, block, (size_t)c.lds, st, A, B, S, Z, Y, (int)m, (int)n, (int)k,
                       __builtin_ctz((unsigned)c.g));
    return hipGetLastError();
}

template <int BITS, int BS, bool HAS_ZP, int MR>
hipError_t f32_cpl(const StreamConfig& c, const float* A, const uint8_t* B, const float* S,
                   const uint8_t* Z, float* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    if (c.cpl <= 1) return f32_go<BITS, BS, HAS_ZP, MR, 1>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 2) return f32_go<BITS, BS, HAS_ZP, MR, 2>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 3) return f32_go<BITS, BS, HAS_ZP, MR, 3>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 4) return f32_go<BITS, BS, HAS_ZP, MR, 4>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 6) return f32_go<BITS, BS, HAS_ZP, MR, 6>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 8) return f32_go<BITS, BS, HAS_ZP, MR, 8>(c, A, B, S, Z, Y, m, n, k, st);
    return hipErrorInvalidValue;
}

template <int BITS, int BS, bool HAS_ZP>
hipError_t f32_mr(const StreamConfig& c, const float* A, const uint8_t* B, const float* S,
                  const uint8_t* Z, float* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    switch (c.mr) {
        case 1: return f32_cpl<BITS, BS, HAS_ZP, 1>(c, A, B, S, Z, Y, m, n, k, st);
        case 2: return f32_cpl<BITS, BS, HAS_ZP, 2>(c, A, B, S, Z, Y, m, n, k, st);
        case 3: return f32_cpl<BITS, BS, HAS_ZP, 3>(c, A, B, S, Z, Y, m, n, k, st);
        case 4: return f32_cpl<BITS, BS, HAS_ZP, 4>(c, A, B, S, Z, Y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

template <int BITS, int BS>
hipError_t f32_zp(const StreamConfig& c, const float* A, const uint8_t* B, const float* S,
                  const uint8_t* Z, float* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    if (Z) return f32_mr<BITS, BS, true>(c, A, B, S, Z, Y, m, n, k, st);
    return f32_mr<BITS, BS, false>(c, A, B, S, Z, Y, m, n, k, st);
}

template <int BITS>
hipError_t f32_bs(const StreamConfig& c, int bs, const float* A, const uint8_t* B, const float* S,
                  const uint8_t* Z, float* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    switch (bs) {
        case 16: return f32_zp<BITS, 16>(c, A, B, S, Z, Y, m, n, k, st);
        case 32: return f32_zp<BITS, 32>(c, A, B, S, Z, Y, m, n, k, st);
        case 64: return f32_zp<BITS, 64>(c, A, B, S, Z, Y, m, n, k, st);
        case 128: return f32_zp<BITS, 128>(c, A, B, S, Z, Y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// The fp16 streaming GEMV's launch shape (lane-group width, chunks per lane, wavefronts per
// workgroup) for a row-tile of up to four rows -- the largest whose staged fp32 chunks fit the
// LDS cap -- and this kernel's LDS.  Above one tile the grid's y dimension walks the row-tiles,
// each streaming the weights again: up to 64 rows, still far fewer weight reads than the
// generic kernel's (one pass per four rows, every activation element loaded per weight).
bool gemv_stream_f32_config(int64_t m, int64_t n, int64_t k, int bits, int bs, StreamConfig* out) {
    if (m < 1 || m > kF32MaxRows) return false;
    const int64_t wpc = 128 / bits;
    for (int64_t mr = std::min<int64_t>(m, 4); mr >= 1; --mr) {
        if (!gemv_stream_supported(mr, n, k, bits, bs)) continue;
        StreamConfig c = gemv_stream_config(mr, n, k, bits, bs);
        const int64_t cpc = k / wpc;
        if (c.u != 1 || c.cpl < 1 || c.cpl > kF32MaxCpl || (int64_t)c.g * c.cpl < cpc) return false;
        const int64_t cols = (int64_t)c.waves_per_group * (64 / c.g);
        c.groups = (n + cols - 1) / cols;
        c.lds = c.mr * cpc * (bits == 4 ? f32_chunk_stride<4>() : f32_chunk_stride<8>());
        if (c.groups > 0x7fffffff) return false;
        if (c.lds > kF32MaxLds) continue;
        if ((m + c.mr - 1) / c.mr > 65535) return false;
        if (out) *out = c;
        return true;
    }
    return false;
}

hipError_t launch_gemv_stream_f32(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                                  void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                                  hipStream_t st) {
    if (m == 0) return hipSuccess;
    StreamConfig c{};
    if (m < 0 || !gemv_stream_f32_config(m, n, k, bits, bs, &c)) return hipErrorInvalidValue;
    const float* A = static_cast<const float*>(a);
    const float* S = static_cast<const float*>(s);
    float* Y = static_cast<float*>(y);
    if (bits == 4) return f32_bs<4>(c, bs, A, b, S, z, Y, m, n, k, st);
    if (bits == 8) return f32_bs<8>(c, bs, A, b, S, z, Y, m, n, k, st);
    return hipErrorInvalidValue;
}

}  // namespace mnb
