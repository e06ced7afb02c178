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

template <int BITS, bool HAS_ZP>
__device__ __forceinline__ float zp_value(const uint8_t* __restrict__ Z, int64_t n, int blk,
                                          int zpb) {
    if constexpr (!HAS_ZP) {
        return (float)(1 << (BITS - 1));
    } else if constexpr (BITS == 4) {
        const uint32_t byte = Z[n * zpb + (blk >> 1)];
        return (float)((byte >> ((blk & 1) * 4)) & 0xFu);
    } else {
        return (float)Z[n * zpb + blk];
    }
}

}  // namespace

// One wavefront = 64/G lane groups; a "task" is the NG*U consecutive columns a wavefront
// handles in one pass (group g takes columns base + g*U + u, u < U).  Waves loop over tasks with
// a grid stride.  MR rows of A (rows m0 .. m0+MR-1, m0 = blockIdx.y * MR) are held in registers
// for the lane's chunk set; CPL chunks per lane at most.
template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U, bool NT>
__global__ void __launch_bounds__(256)
gemv_stream(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
            const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K, int G,
            int tasks, int total_waves) {
    constexpr int WPC = chunk_weights<BITS>();
    constexpr int NP = chunk_pairs<BITS>();
    constexpr int SEGS = chunk_segs<BITS, BS>();
    constexpr int DW_PER_SEG = 4 / SEGS;                 // dwords of a chunk per block segment
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int grp = lane / G;
    const int gi = lane - grp * G;
    const int ng = 64 / G;
    const int cpc = K / WPC;                             // chunks per column
    const int bpc = K / BS;
    const int zpb = (bpc * BITS + 7) / 8;
    const int64_t col_bytes = (int64_t)K * BITS / 8;
    const int m0 = blockIdx.y * MR;

    // ---- activations for this lane's chunks, paired to match sub_pair, plus segment sums ----
    f16x2 ap[MR][CPL][NP];
    float asum[MR][CPL][SEGS];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = gi + j * G;
        const bool ok = c < cpc;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const bool rok = ok && (m0 + r) < M;
            const uint32_t* src =
                reinterpret_cast<const uint32_t*>(A + (int64_t)(m0 + r) * K + (int64_t)c * WPC);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                // WPC fp16 = 4 * (WPC/8) dwords ... loaded as 16-byte pieces
                uint32_t x[4] = {0u, 0u, 0u, 0u};
                if constexpr (BITS == 4) {
                    if (rok) {
                        const u32x4 v = *reinterpret_cast<const u32x4*>(src + 4 * d);
                        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
                    }
                    pair_activations<4>(x, &ap[r][j][4 * d]);
                } else {
                    if (rok) {
                        const u32x2 v = *reinterpret_cast<const u32x2*>(src + 2 * d);
                        x[0] = v.x; x[1] = v.y;
                    }
                    pair_activations<8>(x, &ap[r][j][2 * d]);
                }
            }
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                float t = 0.f;
#pragma unroll
                for (int p = s * (NP / SEGS); p < (s + 1) * (NP / SEGS); ++p)
                    t += (float)ap[r][j][p].x + (float)ap[r][j][p].y;
                asum[r][j][s] = t;
            }
        }
    }

    for (int task = wave; task < tasks; task += total_waves) {
        const int base = task * ng * U;
        u32x4 bw[U][CPL];
        float sc[U][CPL][SEGS];
        float zs[U][CPL][SEGS];
        int cols[U];
        // Issue every weight, scale and zero-point load of the pass first.
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int col = base + grp * U + u;
            cols[u] = col;
            const int cc = col < N ? col : N - 1;
            const uint8_t* bcol = B + (int64_t)cc * col_bytes;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = gi + j * G;
                const bool ok = c < cpc;
                bw[u][j] = u32x4{0u, 0u, 0u, 0u};
                if (ok) {
                    const u32x4* p = reinterpret_cast<const u32x4*>(bcol + (int64_t)c * 16);
                    bw[u][j] = NT ? __builtin_nontemporal_load(p) : *p;
                }
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const int blk = (c * WPC + s * BS) / BS;
                    sc[u][j][s] = 0.f;
                    zs[u][j][s] = 0.f;
                    if (ok) {
                        sc[u][j][s] = (float)S[(int64_t)cc * bpc + blk];
                        zs[u][j][s] = zp_value<BITS, HAS_ZP>(Z, cc, blk, zpb);
                    }
                }
            }
        }
        float acc[MR][U];
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) acc[r][u] = 0.f;

#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t w[4] = {bw[u][j].x, bw[u][j].y, bw[u][j].z, bw[u][j].w};
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const float s24 = sc[u][j][s] * 16777216.0f;
                    const float sz = -sc[u][j][s] * zs[u][j][s];
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        float t = 0.f;
#pragma unroll
                        for (int d = s * DW_PER_SEG; d < (s + 1) * DW_PER_SEG; ++d) {
                            if constexpr (BITS == 4) {
                                t = __builtin_amdgcn_fdot2(sub_pair<4, 0>(w[d]), ap[r][j][4 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<4, 1>(w[d]), ap[r][j][4 * d + 1], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<4, 2>(w[d]), ap[r][j][4 * d + 2], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<4, 3>(w[d]), ap[r][j][4 * d + 3], t, false);
                            } else {
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 0>(w[d]), ap[r][j][2 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 1>(w[d]), ap[r][j][2 * d + 1], t, false);
                            }
                        }
                        acc[r][u] = __builtin_fmaf(s24, t, acc[r][u]);
                        acc[r][u] = __builtin_fmaf(sz, asum[r][j][s], acc[r][u]);
                    }
                }
            }
        }
        // Butterfly over the G lanes of each group (offsets stay inside the group).
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float v = acc[r][u];
                for (int off = G >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
                acc[r][u] = v;
            }
        if (gi == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (cols[u] >= N) continue;
#pragma unroll
                for (int r = 0; r < MR; ++r)
                    if (m0 + r < M) Y[(int64_t)(m0 + r) * N + cols[u]] = (f16)acc[r][u];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Launch configuration
// ------------------------------------------------------------------------------------------

namespace {

constexpr int kNumCUs = 256;

// Chunks-per-lane capacity for MR rows held in registers.
int cpl_cap(int mr) { return mr == 1 ? 8 : (mr == 2 ? 4 : 2); }

int rows_tile(int64_t m) { return m <= 1 ? 1 : (m == 2 ? 2 : (m == 3 ? 3 : 4)); }

}  // namespace

bool gemv_stream_supported(int64_t m, int64_t k, int bits, int bs) {
    if (bits != 4 && bits != 8) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    const int wpc = 128 / bits;
    if (k <= 0 || k % wpc || k % bs) return false;
    const int mr = rows_tile(m);
    if (m < 1 || m > 4) return false;
    const int64_t cpc = k / wpc;
    return cpc <= (int64_t)64 * cpl_cap(mr);
}

StreamConfig gemv_stream_config(int64_t m, int64_t n, int64_t k, int bits, int bs) {
    (void)bs;
    StreamConfig c{};
    c.mr = rows_tile(m);
    const int64_t cpc = k / (128 / bits);
    const int cap = cpl_cap(c.mr);
    // Smallest lane group whose chunk count per lane fits the register budget; prefer groups
    // that divide the chunk count evenly (no idle lanes).
    int g = 64;
    for (int cand : {16, 32, 64}) {
        if ((cpc + cand - 1) / cand <= cap) { g = cand; break; }
    }
    if (g < 64 && cpc % g && cpc % (2 * g) == 0) g *= 2;
    c.g = g;
    c.cpl = (int)((cpc + g - 1) / g);
    c.u = 2;
    c.waves_per_group = 4;
    const int ng = 64 / g;
    const int64_t tasks = (n + (int64_t)ng * c.u - 1) / ((int64_t)ng * c.u);
    c.tasks = tasks;
    c.total_waves = tasks;   // one pass per wavefront
    (void)kNumCUs;
    return c;
}

template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U, bool NT>
static hipError_t stream_go(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                            const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    const int64_t wpg = c.waves_per_group;
    const dim3 grid((unsigned)((c.total_waves + wpg - 1) / wpg), (unsigned)((m + MR - 1) / MR), 1);
    const dim3 block((unsigned)(64 * wpg), 1, 1);
    hipLaunchKernelGGL((gemv_stream<BITS, BS, HAS_ZP, MR, CPL, U, NT>), grid, block, 0, st, A, B,
                       S, Z, Y, (int)m, (int)n, (int)k, c.g, (int)c.tasks,
                       (int)(grid.x * wpg));
    return hipGetLastError();
}

template <int BITS, int BS, bool HAS_ZP, int MR, int U, bool NT>
static hipError_t stream_cpl(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
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
static hipError_t stream_rows(const StreamConfig& c, const f16* A, const uint8_t* B,
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
static hipError_t stream_zp(const StreamConfig& c, const void* a, const uint8_t* b, const void* s,
                            const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t st) {
    const f16* A = static_cast<const f16*>(a);
    const f16* S = static_cast<const f16*>(s);
    f16* Y = static_cast<f16*>(y);
    if (z) return stream_rows<BITS, BS, true>(c, A, b, S, z, Y, m, n, k, st);
    return stream_rows<BITS, BS, false>(c, A, b, S, z, Y, m, n, k, st);
}

hipError_t launch_gemv_stream_cfg(const StreamConfig& c, const void* a, const uint8_t* b,
                                  const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                  int64_t k, int bits, int bs, hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (c.g != 16 && c.g != 32 && c.g != 64) return hipErrorInvalidValue;
    if ((int64_t)c.g * c.cpl * (128 / bits) < k) return hipErrorInvalidValue;
    if (bits == 4) {
        switch (bs) {
            case 16: return stream_zp<4, 16>(c, a, b, s, z, y, m, n, k, st);
            case 32: return stream_zp<4, 32>(c, a, b, s, z, y, m, n, k, st);
            case 64: return stream_zp<4, 64>(c, a, b, s, z, y, m, n, k, st);
            case 128: return stream_zp<4, 128>(c, a, b, s, z, y, m, n, k, st);
        }
    } else if (bits == 8) {
        switch (bs) {
            case 16: return stream_zp<8, 16>(c, a, b, s, z, y, m, n, k, st);
            case 32: return stream_zp<8, 32>(c, a, b, s, z, y, m, n, k, st);
            case 64: return stream_zp<8, 64>(c, a, b, s, z, y, m, n, k, st);
            case 128: return stream_zp<8, 128>(c, a, b, s, z, y, m, n, k, st);
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_stream(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                              void* y, int64_t m, int64_t n, int64_t k, int bits, int bs,
                              hipStream_t st) {
    const StreamConfig c = gemv_stream_config(m, n, k, bits, bs);
    return launch_gemv_stream_cfg(c, a, b, s, z, y, m, n, k, bits, bs, st);
}

}  // namespace mnb
