// Streaming decode GEMV for MatMulNBits on gfx950 (fp16 A, M <= 4 rows, K % (128/bits) == 0).
//
// Design.  The packed weight of column n is K*bits/8 contiguous bytes (B is [N][K/bs][bs*bits/8]),
// so the kernel reads it in 16-byte "chunks" (32 int4 or 16 int8 weights) with one dwordx4 load
// per lane: a lane group of G lanes (G = 16, 32 or 64) owns one column at a time and lane i of the
// group takes chunks i, i+G, i+2G, ... .  One load instruction therefore covers 64/G runs of
// G*16 contiguous bytes, the coalescing HBM wants, and the chunk set of a lane is the same for
// every column, so the activation values it multiplies are loaded once into registers and reused
// for every column the wavefront visits.
//
// Arithmetic.  The reference forms, per (column, quant block), the fp32 sum of a * (q - zp) and
// scales it once (rust/shaders/glsl/templates/q_gemv.comp:571-579).  Here each chunk's weights are
// turned into fp16 *subnormals* q * 2^-24 with a single AND (the nibble lands in the mantissa of
// an exponent-zero half), multiplied by the fp16 activations with v_dot2_f32_f16 (products are
// exact in fp32), and the chunk's block partial is recovered exactly as
//     sum a*(q - zp) = 2^24 * sum a*(q*2^-24) - zp * sum a,
// with sum a over the chunk's block segment computed once per lane when A is loaded.  The block
// partial is then scaled by the block's scale in fp32 and added to the lane's accumulator; the G
// lane accumulators of a column are summed by a fixed butterfly, so results are run-to-run
// deterministic.  A chunk that lies inside one quant block (bs >= 32 for int4) contributes a
// partial of part of the block; the sum over the block is the same value up to fp32 rounding.
#pragma once

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

// Weights of one 16-byte chunk.
template <int BITS>
constexpr int chunk_weights() { return 128 / BITS; }

// fp16 pairs per chunk (one v_dot2 each).
template <int BITS>
constexpr int chunk_pairs() { return chunk_weights<BITS>() / 2; }

// Quant-block segments inside one chunk: 2 for int4 with block 16, else 1.
template <int BITS, int BS>
constexpr int chunk_segs() { return chunk_weights<BITS>() > BS ? chunk_weights<BITS>() / BS : 1; }

// Pair p of dword d, as two fp16 subnormals (q * 2^-24).  int4: p = 0..3 gives elements
// (8d + p, 8d + p + 4); int8: p = 0..1 gives (4d + p, 4d + p + 2).
template <int BITS, int P>
__device__ __forceinline__ f16x2 sub_pair(uint32_t w) {
    if constexpr (BITS == 4) {
        return as_h2((w >> (4 * P)) & 0x000F000Fu);
    } else {
        return as_h2((w >> (8 * P)) & 0x00FF00FFu);
    }
}

// Rearranges 8 (int4) or 4 (int8) consecutive fp16 activations, given as dwords x[0..] of
// natural pairs, into the pair order sub_pair produces.
template <int BITS>
__device__ __forceinline__ void pair_activations(const uint32_t* x, f16x2* out) {
    if constexpr (BITS == 4) {
        // x0 = (a0,a1) x1 = (a2,a3) x2 = (a4,a5) x3 = (a6,a7) -> (a0,a4) (a1,a5) (a2,a6) (a3,a7)
        out[0] = as_h2(__builtin_amdgcn_perm(x[2], x[0], 0x05040100u));
        out[1] = as_h2(__builtin_amdgcn_perm(x[2], x[0], 0x07060302u));
        out[2] = as_h2(__builtin_amdgcn_perm(x[3], x[1], 0x05040100u));
        out[3] = as_h2(__builtin_amdgcn_perm(x[3], x[1], 0x07060302u));
    } else {
        // x0 = (a0,a1) x1 = (a2,a3) -> (a0,a2) (a1,a3)
        out[0] = as_h2(__builtin_amdgcn_perm(x[1], x[0], 0x05040100u));
        out[1] = as_h2(__builtin_amdgcn_perm(x[1], x[0], 0x07060302u));
    }
}

}  // namespace

// Weight-side registers of one pass: U columns x CPL chunks per lane.  Scales and zero points
// are kept raw (the fp16 bits and the packed byte) so that issuing the loads never waits for
// them; they are decoded when the pass is computed.
template <int SEGS, int CPL, int U>
struct StreamPass {
    u32x4 bw[U][CPL];
    uint16_t sraw[U][CPL][SEGS];
    uint32_t zraw[U][CPL][SEGS];
    int cols[U];
};

// Loads of one pass.  Out-of-range chunks and columns read a clamped, in-bounds address; their
// contribution is removed at compute time (scale forced to zero), so no load sits behind a
// branch and every request of the pass is in flight at once.
template <int BITS, int BS, bool HAS_ZP, int CPL, int U, bool NT>
__device__ __forceinline__ void stream_fetch(StreamPass<chunk_segs<BITS, BS>(), CPL, U>& p,
                                             const uint8_t* __restrict__ B,
                                             const f16* __restrict__ S,
                                             const uint8_t* __restrict__ Z, int task, int ng,
                                             int grp, int gi, int G, int N, int K) {
    constexpr int WPC = chunk_weights<BITS>();
    constexpr int SEGS = chunk_segs<BITS, BS>();
    const int cpc = K / WPC;
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const int64_t col_bytes = (int64_t)K * BITS / 8;
    const int base = task * ng * U;
    const uint16_t* __restrict__ Sr = reinterpret_cast<const uint16_t*>(S);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int col = base + grp * U + u;
        p.cols[u] = col;
        const int cc = col < N ? col : N - 1;
        const uint8_t* bcol = B + (int64_t)cc * col_bytes;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            int c = gi + j * G;
            c = c < cpc ? c : cpc - 1;
            const u32x4* q = reinterpret_cast<const u32x4*>(bcol + (int64_t)c * 16);
            p.bw[u][j] = NT ? __builtin_nontemporal_load(q) : *q;
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                const int blk = (c * WPC + s * BS) / BS;
                p.sraw[u][j][s] = Sr[(int64_t)cc * bpc + blk];
                if constexpr (HAS_ZP) {
                    p.zraw[u][j][s] = BITS == 4 ? (uint32_t)Z[(int64_t)cc * zpb + (blk >> 1)]
                                                : (uint32_t)Z[(int64_t)cc * zpb + blk];
                } else {
                    p.zraw[u][j][s] = 0u;
                }
            }
        }
    }
}

// One wavefront = 64/G lane groups; a "task" is the NG*U consecutive columns a wavefront
// handles in one pass (group g takes columns base + g*U + u, u < U).  Waves loop over tasks with
// a grid stride, fetching the next pass's weights before computing the current one; the first
// pass's weights are requested before the activations, so the HBM stream starts at once.  MR
// rows of A (rows m0 .. m0+MR-1, m0 = blockIdx.y * MR) are held in registers for the lane's
// chunk set; CPL chunks per lane at most.  G is a power of two passed as log2(G).
template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U, bool NT>
__global__ void __launch_bounds__(kStreamMaxThreads)
gemv_stream(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
            const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K, int log2g,
            int tasks, int total_waves) {
    constexpr int WPC = chunk_weights<BITS>();
    constexpr int NP = chunk_pairs<BITS>();
    constexpr int SEGS = chunk_segs<BITS, BS>();
    constexpr int DW_PER_SEG = 4 / SEGS;                 // dwords of a chunk per block segment
    const int G = 1 << log2g;
    const int lane = threadIdx.x & 63;
    // wave-uniform: in a scalar register, the task loop and its column base stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(
        (int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
    const int grp = lane >> log2g;
    const int gi = lane & (G - 1);
    const int ng = 64 >> log2g;
    const int cpc = K / WPC;                             // chunks per column
    const int m0 = blockIdx.y * MR;
    int task = wave;
    if (task >= tasks) return;                           // no barriers below: safe to leave

    StreamPass<SEGS, CPL, U> cur;
    stream_fetch<BITS, BS, HAS_ZP, CPL, U, NT>(cur, B, S, Z, task, ng, grp, gi, G, N, K);

    // ---- activations for this lane's chunks, paired to match sub_pair, plus segment sums ----
    f16x2 ap[MR][CPL][NP];
    float asum[MR][CPL][SEGS];
    bool live[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c0 = gi + j * G;
        live[j] = c0 < cpc;
        const int c = live[j] ? c0 : cpc - 1;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const int row = (m0 + r) < M ? (m0 + r) : M - 1;
            const uint32_t* src =
                reinterpret_cast<const uint32_t*>(A + (int64_t)row * K + (int64_t)c * WPC);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t x[4] = {0u, 0u, 0u, 0u};
                if constexpr (BITS == 4) {               // 8 activations = 16 bytes
                    const u32x4 v = *reinterpret_cast<const u32x4*>(src + 4 * d);
                    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
                    pair_activations<4>(x, &ap[r][j][4 * d]);
                } else {                                 // 4 activations = 8 bytes
                    const u32x2 v = *reinterpret_cast<const u32x2*>(src + 2 * d);
                    x[0] = v.x; x[1] = v.y;
                    pair_activations<8>(x, &ap[r][j][2 * d]);
                }
            }
            const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                float t = 0.f;
#pragma unroll
                for (int p = s * (NP / SEGS); p < (s + 1) * (NP / SEGS); ++p)
                    t = __builtin_amdgcn_fdot2(ap[r][j][p], one2, t, false);
                asum[r][j][s] = t;
            }
        }
    }

    while (true) {
        const int next = task + total_waves;
        const bool more = next < tasks;                  // wave-uniform
        StreamPass<SEGS, CPL, U> nxt;
        if (more) stream_fetch<BITS, BS, HAS_ZP, CPL, U, NT>(nxt, B, S, Z, next, ng, grp, gi, G, N, K);

        float acc[MR][U];
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) acc[r][u] = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t w[4] = {cur.bw[u][j].x, cur.bw[u][j].y, cur.bw[u][j].z,
                                       cur.bw[u][j].w};
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const int blk = ((gi + j * G) * WPC + s * BS) / BS;
                    float sv = (float)__builtin_bit_cast(f16, cur.sraw[u][j][s]);
                    sv = live[j] ? sv : 0.f;
                    float zv;
                    if constexpr (!HAS_ZP) {
                        zv = (float)(1 << (BITS - 1));
                    } else if constexpr (BITS == 4) {
                        zv = (float)((cur.zraw[u][j][s] >> ((blk & 1) * 4)) & 0xFu);
                    } else {
                        zv = (float)cur.zraw[u][j][s];
                    }
                    const float s24 = sv * 16777216.0f;
                    const float sz = -sv * zv;
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        float t = 0.f;
                        float t16 = 0.f;
#pragma unroll
                        for (int d = s * DW_PER_SEG; d < (s + 1) * DW_PER_SEG; ++d) {
                            if constexpr (BITS == 4) {
                                // Nibble pairs 0 and 2 sit in bits 0-3 of each half (q * 2^-24);
                                // pairs 1 and 3 are masked in place at bits 4-7 (16q * 2^-24,
                                // still subnormal) and summed apart, scaled by 1/16 below:
                                // one shift per dword instead of three.
                                const uint32_t wh = w[d] >> 8;
                                t = __builtin_amdgcn_fdot2(as_h2(w[d] & 0x000F000Fu), ap[r][j][4 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(as_h2(wh & 0x000F000Fu), ap[r][j][4 * d + 2], t, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(w[d] & 0x00F000F0u), ap[r][j][4 * d + 1], t16, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(wh & 0x00F000F0u), ap[r][j][4 * d + 3], t16, false);
                            } else {
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 0>(w[d]), ap[r][j][2 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 1>(w[d]), ap[r][j][2 * d + 1], t, false);
                            }
                        }
                        t = __builtin_fmaf(t16, 0.0625f, t);
                        acc[r][u] = __builtin_fmaf(s24, t, acc[r][u]);
                        acc[r][u] = __builtin_fmaf(sz, asum[r][j][s], acc[r][u]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) acc[r][u] = group_sum(acc[r][u], G);
        if (gi == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (cur.cols[u] >= N) continue;
#pragma unroll
                for (int r = 0; r < MR; ++r)
                    if (m0 + r < M) Y[(int64_t)(m0 + r) * N + cur.cols[u]] = (f16)acc[r][u];
            }
        }
        if (!more) break;
        cur = nxt;
        task = next;
    }
}

template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U, bool NT>
hipError_t stream_go(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                            const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    const int64_t wpg = c.waves_per_group;
    const dim3 grid((unsigned)((c.total_waves + wpg - 1) / wpg), (unsigned)((m + MR - 1) / MR), 1);
    const dim3 block((unsigned)(64 * wpg), 1, 1);
    hipLaunchKernelGGL((gemv_stream<BITS, BS, HAS_ZP, MR, CPL, U, NT>), grid, block, 0, st, A, B,
                       S, Z, Y, (int)m, (int)n, (int)k, __builtin_ctz((unsigned)c.g), (int)c.tasks,
                       (int)(grid.x * wpg));
    return hipGetLastError();
}

template <int BITS, int BS, bool HAS_ZP, int MR, int U, bool NT>
hipError_t stream_cpl(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                             const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k,
                             hipStream_t st) {
    // Register arrays are sized by the instantiated CPL; the runtime count selects the
    // smallest instantiation that holds it.
    if (c.cpl <= 1) return stream_go<BITS, BS, HAS_ZP, MR, 1, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 2) return stream_go<BITS, BS, HAS_ZP, MR, 2, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
    if constexpr (MR <= 2) {
        if (c.cpl <= 3) return stream_go<BITS, BS, HAS_ZP, MR, 3, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
        if (c.cpl <= 4) return stream_go<BITS, BS, HAS_ZP, MR, 4, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
    }
    if constexpr (MR == 1) {
        if (c.cpl <= 6) return stream_go<BITS, BS, HAS_ZP, MR, 6, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
        if (c.cpl <= 8) return stream_go<BITS, BS, HAS_ZP, MR, 8, U, NT>(c, A, B, S, Z, Y, m, n, k, st);
    }
    return hipErrorInvalidValue;
}

template <int BITS, int BS, bool HAS_ZP>
hipError_t stream_rows(const StreamConfig& c, const f16* A, const uint8_t* B,
                              const f16* S, const uint8_t* Z, f16* Y, int64_t m, int64_t n,
                              int64_t k, hipStream_t st) {
    const bool nt = c.nontemporal != 0;
#define MNB_STREAM_U(MR_)                                                                         \
    do {                                                                                          \
        if (c.u == 1)                                                                             \
            return nt ? stream_cpl<BITS, BS, HAS_ZP, MR_, 1, true>(c, A, B, S, Z, Y, m, n, k, st) \
                      : stream_cpl<BITS, BS, HAS_ZP, MR_, 1, false>(c, A, B, S, Z, Y, m, n, k, st); \
        if (c.u == 2)                                                                             \
            return nt ? stream_cpl<BITS, BS, HAS_ZP, MR_, 2, true>(c, A, B, S, Z, Y, m, n, k, st) \
                      : stream_cpl<BITS, BS, HAS_ZP, MR_, 2, false>(c, A, B, S, Z, Y, m, n, k, st); \
        return hipErrorInvalidValue;                                                              \
    } while (0)
    switch (c.mr) {
        case 1: MNB_STREAM_U(1);
        case 2: MNB_STREAM_U(2);
        case 3: MNB_STREAM_U(3);
        case 4: MNB_STREAM_U(4);
        default: return hipErrorInvalidValue;
    }
#undef MNB_STREAM_U
}

template <int BITS, int BS>
hipError_t stream_zp(const StreamConfig& c, const void* a, const uint8_t* b, const void* s,
                            const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    const f16* A = static_cast<const f16*>(a);
    const f16* S = static_cast<const f16*>(s);
    f16* Y = static_cast<f16*>(y);
    if (z) return stream_rows<BITS, BS, true>(c, A, b, S, z, Y, m, n, k, st);
    return stream_rows<BITS, BS, false>(c, A, b, S, z, Y, m, n, k, st);
}

// All block sizes of one bit width (instantiated once per width, in its own translation unit).
template <int BITS>
hipError_t stream_bits(const StreamConfig& c, const void* a, const uint8_t* b, const void* s,
                       const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bs,
                       hipStream_t st) {
    switch (bs) {
        case 16: return stream_zp<BITS, 16>(c, a, b, s, z, y, m, n, k, st);
        case 32: return stream_zp<BITS, 32>(c, a, b, s, z, y, m, n, k, st);
        case 64: return stream_zp<BITS, 64>(c, a, b, s, z, y, m, n, k, st);
        case 128: return stream_zp<BITS, 128>(c, a, b, s, z, y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mnb
