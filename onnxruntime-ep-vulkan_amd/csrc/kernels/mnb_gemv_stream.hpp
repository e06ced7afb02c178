// Streaming decode GEMV for MatMulNBits on gfx950 (fp16 A, M <= 4 rows, K % (128/bits) == 0).
//
// Design.  At M <= 4 one launch streams 5-30 MB of weights, and once the whole chip has its
// weight loads in flight every memory request -- an L2 hit included -- waits behind that burst
// (measured on MI355X: a 6 KB L2-resident read takes 0.4 us alone and 1.6-2.7 us while the other
// workgroups stream).  Whatever a wavefront needs besides its own weights must therefore arrive
// before the burst starts.  The launch is one to four workgroups per CU (up to 16 wavefronts
// each); every thread first requests its share of what the workgroup's wavefronts share -- the
// MR activation rows (an L2 / MALL hit) and the columns' scale and zero-point bytes (cold in
// HBM; with at most four chunks per lane each lane instead loads its own chunks' scales and
// zero points into registers) -- and each wavefront stages its activation share in LDS as soon
// as it arrives and then issues its weights at once (all activation requests of the launch are
// out by then); the scale and zero-point bytes reach LDS while the weights are in flight, and
// one workgroup barrier precedes the compute.  Everything but the pairing and the stores -- the LDS offsets of the
// staged units, the weight addresses -- is formed before the activations arrive: a wavefront's
// VALU work between its activations' arrival and its weight requests delays the whole stream.
// Each wavefront makes exactly one pass: it owns U
// columns per lane group (written for U, launched with U = 1) and issues all of their 16-byte
// weight loads at once.  The packed weight
// of column n is K*bits/8 contiguous bytes (B is [N][K/bs][bs*bits/8]); a lane group of G lanes
// (G = 16, 32 or 64) owns a column and lane i of the group takes chunks i, i+G, i+2G, ... (a
// "chunk" is 16 bytes: 32 int4 or 16 int8 weights), so one load instruction covers 64/G runs of
// G*16 contiguous bytes, the coalescing HBM wants.
//
// Staged in LDS: the activations in the pair order the unpack produces, each chunk with the fp32
// sum of its activations per quant-block segment, and the workgroup's scale and zero-point bytes,
// which for its C consecutive columns are one contiguous byte range each, copied with 16-byte
// loads.  A lane reads its chunks' activations, scales and zero points from LDS (broadcast reads,
// a padded chunk stride that keeps 8 consecutive chunks in 8 different bank groups).
//
// Arithmetic.  The reference forms, per (column, quant block), the fp32 sum of a * (q - zp) and
// scales it once (rust/shaders/glsl/templates/q_gemv.comp:571-579).  Here each chunk's weights are
// turned into fp16 *subnormals* q * 2^-24 with a single AND (the nibble lands in the mantissa of
// an exponent-zero half), multiplied by the fp16 activations with v_dot2_f32_f16 (products are
// exact in fp32), and the chunk's block partial is recovered exactly as
//     sum a*(q - zp) = 2^24 * sum a*(q*2^-24) - zp * sum a,
// with sum a over the chunk's block segment taken from the staged activations.  The block
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

// Rearranges 8 consecutive fp16 activations, given as 4 dwords x[0..3] of natural pairs, into
// the pair order sub_pair produces: int4 (a0,a4) (a1,a5) (a2,a6) (a3,a7); int8 (a0,a2) (a1,a3)
// (a4,a6) (a5,a7).
template <int BITS>
__device__ __forceinline__ u32x4 pair_activations(u32x4 x) {
    if constexpr (BITS == 4) {
        return u32x4{__builtin_amdgcn_perm(x.z, x.x, 0x05040100u),
                     __builtin_amdgcn_perm(x.z, x.x, 0x07060302u),
                     __builtin_amdgcn_perm(x.w, x.y, 0x05040100u),
                     __builtin_amdgcn_perm(x.w, x.y, 0x07060302u)};
    } else {
        return u32x4{__builtin_amdgcn_perm(x.y, x.x, 0x05040100u),
                     __builtin_amdgcn_perm(x.y, x.x, 0x07060302u),
                     __builtin_amdgcn_perm(x.w, x.z, 0x05040100u),
                     __builtin_amdgcn_perm(x.w, x.z, 0x07060302u)};
    }
}

}  // namespace

// LDS bytes of one staged activation chunk: its fp16 pairs (64 bytes int4, 32 bytes int8) and
// the fp32 segment sums, padded to 80 / 48 bytes so that 8 consecutive chunks start in 8
// distinct 16-byte bank groups (5c mod 8 and 3c mod 8 are permutations of 0..7).
template <int BITS>
__host__ __device__ constexpr int stream_chunk_stride() { return BITS == 4 ? 80 : 48; }

// Units (16 bytes) a thread loads per staging batch: activations (per row of the row-tile, so
// that the first batch covers all of A whenever a workgroup has K / 16 threads), scale bytes,
// zero-point bytes.
constexpr int kStreamAU = 2;
constexpr int kStreamSU = 2;
constexpr int kStreamZU = 1;

// Whether a lane loads its chunks' block scales and zero points itself, straight into registers
// (at most four (chunk, column, segment) triples: one 2-byte and one 1-byte load each), rather
// than the workgroup staging its columns' scale and zero-point bytes in LDS.  The lane's own
// loads keep the workgroup barrier from waiting for those HBM reads, but every load instruction
// costs address-unit time whatever its width; measured on MI355X: qkv (three chunks per lane)
// 5.25 -> 5.00 us, o (three) 3.61 -> 3.48 us, gate_up (six) 6.64 -> 6.72 us.
__host__ __device__ constexpr bool stream_lane_scales(int cpl, int u, int segs) {
    return cpl * u * segs <= 4;
}

// One workgroup = `waves` wavefronts (blockDim.x / 64) = C = waves * (64/G) * U consecutive
// columns, col0 = blockIdx.x * C; MR rows of A (m0 = blockIdx.y * MR).  vec_s / vec_z: the
// workgroup's scale / zero-point byte ranges may be copied with 16-byte loads (the host checked
// the base alignment and that C * row bytes is a multiple of 16); otherwise 2-byte / 1-byte loads.
template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U>
__global__ void __launch_bounds__(kStreamMaxThreads)
gemv_stream(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
            const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K, int log2g,
            int vec_s, int vec_z) {
    constexpr int WPC = chunk_weights<BITS>();
    constexpr int NP = chunk_pairs<BITS>();
    constexpr int SEGS = chunk_segs<BITS, BS>();
    constexpr int DW_PER_SEG = 4 / SEGS;                 // dwords of a chunk per block segment
    constexpr int UPC = WPC / 8;                         // 16-byte activation units per chunk
    constexpr int CST = stream_chunk_stride<BITS>();
    constexpr bool REG = stream_lane_scales(CPL, U, SEGS);
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
    const int C = (T >> 6) * ng * U;
    const int col0 = (int)blockIdx.x * C;
    const int ncols = min(C, N - col0);
    const int m0 = (int)blockIdx.y * MR;
    const int64_t col_bytes = (int64_t)K * BITS / 8;

    uint8_t* sA = smem;
    uint8_t* sS = smem + MR * cpc * CST;
    uint8_t* sZ = sS + ((C * bpc * 2 + 15) & ~15);
    const int s_bytes = ncols * bpc * 2;
    const int z_bytes = HAS_ZP ? ncols * zpb : 0;
    const uint8_t* gS = reinterpret_cast<const uint8_t*>(S) + (int64_t)col0 * bpc * 2;
    const uint8_t* gZ = HAS_ZP ? Z + (int64_t)col0 * zpb : nullptr;

    // ---- first staging batch: activation units, scale and zero-point units --------------------
    const int upr = K / 8;                               // activation units per row
    const int a_units = MR * upr;
    // Every load of this batch is made by every thread (indices past the end are clamped to an
    // in-bounds unit whose value is not used), so the number of loads in flight is the same on
    // every path and waiting for the activations does not wait for the later requests.  With
    // lanes loading their own scales, a batch entirely past the end is skipped (a branch taken
    // alike by the whole workgroup; measured qkv 4.84 -> 4.74 us, down 4.46 -> 4.40 us; with the
    // workgroup-staged scales it measured slower).
    constexpr int AU = kStreamAU * MR;
    // Unit u is row r = u / upr (found by comparisons: MR <= 4), chunk c = w / UPC and quarter
    // (int4) or half (int8) q of that chunk, w = u - r upr.  Its LDS offsets -- the activations
    // and its chunk's segment-sum slot -- are formed here, from the thread index alone, so that
    // nothing but the pairing and the stores is left for when the activations arrive.
    struct Place {
        const f16* src;                                  // the unit's 8 activations
        int dst;                                         // LDS offset of its pairs
        int sum;                                         // LDS offset of its segment's sum
        bool own;                                        // the unit stores that sum
    };
    auto place = [&](int u) {
        int r = 0;
#pragma unroll
        for (int rr = 1; rr < MR; ++rr) r += u >= rr * upr ? 1 : 0;
        const int w = u - r * upr;
        const int c = w / UPC;
        const int q = w - c * UPC;
        const int cb = (r * cpc + c) * CST;
        Place p;
        p.src = A + (int64_t)min(m0 + r, M - 1) * K + (int64_t)w * 8;
        p.dst = cb + 16 * q;
        if constexpr (BITS == 4 && SEGS == 2) {          // block 16: two units per segment
            p.sum = cb + 4 * NP + 4 * (q >> 1);
            p.own = (q & 1) == 0;
        } else {
            p.sum = cb + 4 * NP;
            p.own = q == 0;
        }
        return p;
    };
    u32x4 av[AU];
    Place pl[AU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        pl[i] = place(min(tid + i * T, a_units - 1));
        if (!REG || i == 0 || i * T < a_units) av[i] = *reinterpret_cast<const u32x4*>(pl[i].src);
    }
    const int s_units = vec_s && !REG ? s_bytes / 16 : 0;
    const int z_units = vec_z && !REG ? z_bytes / 16 : 0;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(s_units > 0 ? gS : reinterpret_cast<const uint8_t*>(A));
    const u32x4* z4 = reinterpret_cast<const u32x4*>(z_units > 0 ? gZ : reinterpret_cast<const uint8_t*>(A));
    u32x4 sv[kStreamSU], zv[kStreamZU];
    if constexpr (!REG) {
#pragma unroll
        for (int i = 0; i < kStreamSU; ++i) sv[i] = s4[min(tid + i * T, max(s_units - 1, 0))];
        if constexpr (HAS_ZP) {
#pragma unroll
            for (int i = 0; i < kStreamZU; ++i) zv[i] = z4[min(tid + i * T, max(z_units - 1, 0))];
        }
    }

    // The wavefront's weight addresses: lane (group grp, index gi) takes chunks gi, gi + G, ...
    // of its U columns (clamped to the column's last chunk; a clamped chunk is not summed).
    int lcol[U];
    const uint8_t* bcol[U];
    int boff[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        boff[j] = 16 * min(gi + j * G, cpc - 1);
        asm volatile("" : "+v"(boff[j]));                // formed here, not after the staging
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int lc = (wave * ng + grp) * U + u;        // column within the workgroup
        lcol[u] = lc;
        bcol[u] = B + (int64_t)min(col0 + lc, N - 1) * col_bytes;
    }
    auto chunk_of = [&](int j) { return min(gi + j * G, cpc - 1); };
    // With few chunks per lane, the lane's own block scales and zero points: for fixed (chunk,
    // column, segment) the G lanes of a group read consecutive scale bytes of one column.
    uint16_t sraw[REG ? CPL : 1][U][SEGS];
    uint8_t zraw[REG ? CPL : 1][U][SEGS];
    if constexpr (REG) {
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const int64_t cc = min(col0 + lcol[u], N - 1);
                    const int blk = (chunk_of(j) * WPC + s * BS) / BS;
                    sraw[REG ? j : 0][u][s] = reinterpret_cast<const uint16_t*>(S)[cc * bpc + blk];
                    if constexpr (HAS_ZP)
                        zraw[REG ? j : 0][u][s] = Z[cc * zpb + (BITS == 4 ? blk >> 1 : blk)];
                }
    }

    // With the lane's own scales, its first weight chunk is requested here, ahead of the
    // activation staging: the stream starts earlier, while the activation requests, made first,
    // stay ahead of it (measured: qkv 5.01 -> 4.89 us, o 3.48 -> 3.34, down 4.67 -> 4.48; two
    // early chunks, or one with the workgroup-staged scales, measured slower).
    constexpr int EW = REG ? (CPL < 1 ? CPL : 1) : 0;
    u32x4 bw[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < EW; ++j)
            bw[u][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bcol[u] + boff[j]));
    __builtin_amdgcn_sched_barrier(0);

    // ---- stage the first batch into LDS ------------------------------------------------------
    const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
    // The pairing and the unit's sum are computed on every lane (a clamped unit past the end
    // included, so that the loads above are used unconditionally and stay where they are); only
    // real units are stored.  Segment sums across the units of a chunk: the units of one chunk
    // sit in UPC consecutive threads (T and the units per row are multiples of UPC), combined in
    // a fixed order.
    auto stage_a = [&](bool live, const Place& p, u32x4 x) {
        const u32x4 pr = pair_activations<BITS>(x);
        if (live) *reinterpret_cast<u32x4*>(sA + p.dst) = pr;
        float t = 0.f;
        t = __builtin_amdgcn_fdot2(as_h2(pr.x), one2, t, false);
        t = __builtin_amdgcn_fdot2(as_h2(pr.y), one2, t, false);
        t = __builtin_amdgcn_fdot2(as_h2(pr.z), one2, t, false);
        t = __builtin_amdgcn_fdot2(as_h2(pr.w), one2, t, false);
        t = live ? t : 0.f;
        // partner sums over the lane's quad (int4) or pair (int8); out-of-range units add 0
        t += dpp_f<0xB1>(t);                             // lane ^ 1
        if constexpr (BITS == 4 && SEGS == 1) t += dpp_f<0x4E>(t);   // lane ^ 2
        if (live && p.own) *reinterpret_cast<float*>(sA + p.sum) = t;
    };
#pragma unroll
    for (int i = 0; i < AU; ++i)
        if (!REG || i == 0 || i * T < a_units) stage_a(tid + i * T < a_units, pl[i], av[i]);
    // ---- what the first batch did not cover (long K, several rows, unaligned tensors) -------
    for (int base = tid + AU * T; base < a_units; base += AU * T) {
        u32x4 x[AU];
        Place px[AU];
#pragma unroll
        for (int i = 0; i < AU; ++i) {
            px[i] = place(min(base + i * T, a_units - 1));
            x[i] = *reinterpret_cast<const u32x4*>(px[i].src);
        }
#pragma unroll
        for (int i = 0; i < AU; ++i) stage_a(base + i * T < a_units, px[i], x[i]);
    }
    if constexpr (!REG) {
        for (int u = tid + kStreamSU * T; u < s_units; u += T)
            reinterpret_cast<u32x4*>(sS)[u] = reinterpret_cast<const u32x4*>(gS)[u];
        for (int i = 2 * (tid + s_units * 8); i < s_bytes; i += 2 * T)   // 2-byte remainder / path
            *reinterpret_cast<uint16_t*>(sS + i) = *reinterpret_cast<const uint16_t*>(gS + i);
        if constexpr (HAS_ZP) {
            for (int u = tid + kStreamZU * T; u < z_units; u += T)
                reinterpret_cast<u32x4*>(sZ)[u] = reinterpret_cast<const u32x4*>(gZ)[u];
            for (int i = tid + z_units * 16; i < z_bytes; i += T) sZ[i] = gZ[i];
        }
    }
    // The weights are issued as soon as this wavefront has staged its activations -- not after
    // a workgroup barrier -- and are kept below the staging (the activation loads, issued
    // first, are not queued behind them).
    __builtin_amdgcn_sched_barrier(0);

    // ---- the wavefront's weights: every load of the pass, issued at once (addresses formed
    // before the activations arrived) --------------------------------------------------------
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = EW; j < CPL; ++j)
            bw[u][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bcol[u] + boff[j]));

    // ---- the scale and zero-point bytes (requested before the weights, from HBM) ------------
    if constexpr (!REG) {
#pragma unroll
        for (int i = 0; i < kStreamSU; ++i) {
            const int u = tid + i * T;
            if (u < s_units) reinterpret_cast<u32x4*>(sS)[u] = sv[i];
        }
        if constexpr (HAS_ZP) {
#pragma unroll
            for (int i = 0; i < kStreamZU; ++i) {
                const int u = tid + i * T;
                if (u < z_units) reinterpret_cast<u32x4*>(sZ)[u] = zv[i];
            }
        }
    }
    __syncthreads();

    // ---- compute: chunk by chunk, its activations read from LDS once for all U columns ------
    float acc[MR][U];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) acc[r][u] = 0.f;
    const uint16_t* sSr = reinterpret_cast<const uint16_t*>(sS);
    // Per chunk j, column u and block segment s: the block's scale (0 for a chunk past the
    // column's end), its zero point, and row r's activation sum over the segment.
    auto scale_of = [&](int j, int u, int s) {
        const int blk = (chunk_of(j) * WPC + s * BS) / BS;
        const uint16_t raw = REG ? sraw[REG ? j : 0][u][s] : sSr[min(lcol[u], C - 1) * bpc + blk];
        return gi + j * G < cpc ? (float)__builtin_bit_cast(f16, raw) : 0.f;
    };
    auto zp_of = [&](int j, int u, int s) {
        const int blk = (chunk_of(j) * WPC + s * BS) / BS;
        const int lc = min(lcol[u], C - 1);
        const int zb = REG ? zraw[REG ? j : 0][u][s] : sZ[lc * zpb + (BITS == 4 ? blk >> 1 : blk)];
        if constexpr (!HAS_ZP) return (float)(1 << (BITS - 1));
        else if constexpr (BITS == 4) return (float)((zb >> ((blk & 1) * 4)) & 0xF);
        else return (float)zb;
    };
    auto asum_of = [&](int j, int r, int s) {
        return reinterpret_cast<const float*>(sA + (r * cpc + chunk_of(j)) * CST + 4 * NP)[s];
    };
    // What does not depend on the weights is formed first, while they are still in flight:
    // each chunk's 2^24 * scale, and the zero-point terms -scale * zp * (activation sum) added
    // into the accumulators; once a chunk's weights arrive only its unpack, dot products and
    // one scaled add are left.
    float s24[CPL][U][SEGS];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                const float sv1 = scale_of(j, u, s);
                s24[j][u][s] = sv1 * 16777216.0f;
                const float sz = -sv1 * zp_of(j, u, s);
#pragma unroll
                for (int r = 0; r < MR; ++r) acc[r][u] = __builtin_fmaf(sz, asum_of(j, r, s), acc[r][u]);
            }
    __builtin_amdgcn_sched_barrier(0);
    // chunk j's (column u, segment s) partial t, scaled
    auto add_partial = [&](int j, int u, int s, int r, float t) {
        acc[r][u] = __builtin_fmaf(s24[j][u][s], t, acc[r][u]);
    };
    if constexpr (MR == 1) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c0 = gi + j * G;
            const bool live = c0 < cpc;
            const int c = live ? c0 : cpc - 1;
            f16x2 ap[MR][NP];
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const uint8_t* src = sA + (r * cpc + c) * CST;
#pragma unroll
                for (int q = 0; q < NP / 4; ++q) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * q);
                    ap[r][4 * q + 0] = as_h2(v.x);
                    ap[r][4 * q + 1] = as_h2(v.y);
                    ap[r][4 * q + 2] = as_h2(v.z);
                    ap[r][4 * q + 3] = as_h2(v.w);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t w[4] = {bw[u][j].x, bw[u][j].y, bw[u][j].z, bw[u][j].w};
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        float t = 0.f;
                        float t16 = 0.f;
#pragma unroll
                        for (int d = s * DW_PER_SEG; d < (s + 1) * DW_PER_SEG; ++d) {
                            if constexpr (BITS == 4) {
                                // Nibble pairs 0 and 2 sit in bits 0-3 of each half (q * 2^-24);
                                // pairs 1 and 3 are masked in place at bits 4-7 (16q * 2^-24, still
                                // subnormal) and summed apart, scaled by 1/16 below: one shift per
                                // dword instead of three.
                                const uint32_t wh = w[d] >> 8;
                                t = __builtin_amdgcn_fdot2(as_h2(w[d] & 0x000F000Fu), ap[r][4 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(as_h2(wh & 0x000F000Fu), ap[r][4 * d + 2], t, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(w[d] & 0x00F000F0u), ap[r][4 * d + 1], t16, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(wh & 0x00F000F0u), ap[r][4 * d + 3], t16, false);
                            } else {
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 0>(w[d]), ap[r][2 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(sub_pair<8, 1>(w[d]), ap[r][2 * d + 1], t, false);
                            }
                        }
                        t = __builtin_fmaf(t16, 0.0625f, t);
                        add_partial(j, u, s, r, t);
                    }
                }
            }
        }
    } else {
        // Several rows: the chunk's weights are unpacked and its scale terms formed once, then
        // each row's activations are read from LDS and used for all U columns.
        constexpr int QPD = BITS == 4 ? 4 : 2;           // fp16 pairs per weight dword
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            // keep the scheduler from hoisting every chunk's activation reads to the top
            __builtin_amdgcn_sched_barrier(0);
            const int c0 = gi + j * G;
            const bool live = c0 < cpc;
            const int c = live ? c0 : cpc - 1;
            // The chunk's weights as fp16 subnormal pairs.  int4: for dword d, pairs 0 and 2 sit in
            // bits 0-3 of each half (q * 2^-24) and pairs 1 and 3 are masked in place at bits 4-7
            // (16q * 2^-24, still subnormal), summed apart and scaled by 1/16: one shift per dword.
            uint32_t q[U][4][QPD];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t w[4] = {bw[u][j].x, bw[u][j].y, bw[u][j].z, bw[u][j].w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    if constexpr (BITS == 4) {
                        const uint32_t wh = w[d] >> 8;
                        q[u][d][0] = w[d] & 0x000F000Fu;
                        q[u][d][1] = w[d] & 0x00F000F0u;
                        q[u][d][2] = wh & 0x000F000Fu;
                        q[u][d][3] = wh & 0x00F000F0u;
                    } else {
                        q[u][d][0] = w[d] & 0x00FF00FFu;
                        q[u][d][1] = (w[d] >> 8) & 0x00FF00FFu;
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const uint8_t* src = sA + (r * cpc + c) * CST;
                f16x2 ap[NP];
#pragma unroll
                for (int qq = 0; qq < NP / 4; ++qq) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * qq);
                    ap[4 * qq + 0] = as_h2(v.x);
                    ap[4 * qq + 1] = as_h2(v.y);
                    ap[4 * qq + 2] = as_h2(v.z);
                    ap[4 * qq + 3] = as_h2(v.w);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
#pragma unroll
                    for (int s = 0; s < SEGS; ++s) {
                        float t = 0.f;
                        float t16 = 0.f;
#pragma unroll
                        for (int d = s * DW_PER_SEG; d < (s + 1) * DW_PER_SEG; ++d) {
                            if constexpr (BITS == 4) {
                                t = __builtin_amdgcn_fdot2(as_h2(q[u][d][0]), ap[4 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(as_h2(q[u][d][2]), ap[4 * d + 2], t, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(q[u][d][1]), ap[4 * d + 1], t16, false);
                                t16 = __builtin_amdgcn_fdot2(as_h2(q[u][d][3]), ap[4 * d + 3], t16, false);
                            } else {
                                t = __builtin_amdgcn_fdot2(as_h2(q[u][d][0]), ap[2 * d + 0], t, false);
                                t = __builtin_amdgcn_fdot2(as_h2(q[u][d][1]), ap[2 * d + 1], t, false);
                            }
                        }
                        t = __builtin_fmaf(t16, 0.0625f, t);
                        add_partial(j, u, s, r, t);
                    }
                }
            }
            // The compiler would otherwise sink rows 1.. of every chunk below the last chunk and
            // hold all of their activations (227 VGPRs at four int4 rows and three chunks: two
            // wavefronts per SIMD, 3-4x slower): the chunk's sums are finished here.
#pragma unroll
            for (int r = 0; r < MR; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) asm volatile("" : "+v"(acc[r][u]));
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) acc[r][u] = group_sum(acc[r][u], G);
    if (gi == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (lcol[u] >= ncols) continue;
#pragma unroll
            for (int r = 0; r < MR; ++r)
                if (m0 + r < M) Y[(int64_t)(m0 + r) * N + col0 + lcol[u]] = (f16)acc[r][u];
        }
    }
}

template <int BITS, int BS, bool HAS_ZP, int MR, int CPL, int U>
hipError_t stream_go(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                     const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    auto kern = gemv_stream<BITS, BS, HAS_ZP, MR, CPL, U>;
    const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), (size_t)c.lds);
    if (ea != hipSuccess) return ea;
    const dim3 grid((unsigned)c.groups, (unsigned)((m + MR - 1) / MR), 1);
    const dim3 block((unsigned)(64 * c.waves_per_group), 1, 1);
    hipLaunchKernelGGL(kern, grid, block, (size_t)c.lds, st, A, B, S, Z, Y, (int)m, (int)n, (int)k,
                       __builtin_ctz((unsigned)c.g), c.vec_s, c.vec_z);
    return hipGetLastError();
}

template <int BITS, int BS, bool HAS_ZP, int MR, int U>
hipError_t stream_cpl(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                      const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    // Register arrays are sized by the instantiated CPL; the runtime count selects the
    // smallest instantiation that holds it.
    if (c.cpl <= 1) return stream_go<BITS, BS, HAS_ZP, MR, 1, U>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 2) return stream_go<BITS, BS, HAS_ZP, MR, 2, U>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 3) return stream_go<BITS, BS, HAS_ZP, MR, 3, U>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 4) return stream_go<BITS, BS, HAS_ZP, MR, 4, U>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 6) return stream_go<BITS, BS, HAS_ZP, MR, 6, U>(c, A, B, S, Z, Y, m, n, k, st);
    if (c.cpl <= 8) return stream_go<BITS, BS, HAS_ZP, MR, 8, U>(c, A, B, S, Z, Y, m, n, k, st);
    return hipErrorInvalidValue;
}

template <int BITS, int BS, bool HAS_ZP>
hipError_t stream_rows(const StreamConfig& c, const f16* A, const uint8_t* B, const f16* S,
                       const uint8_t* Z, f16* Y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
    // one column per lane group (derive() refuses others): two per group measured slower once
    // lanes load their own scales, and would not fit the registers with several rows
    switch (c.mr) {
        case 1: return stream_cpl<BITS, BS, HAS_ZP, 1, 1>(c, A, B, S, Z, Y, m, n, k, st);
        case 2: return stream_cpl<BITS, BS, HAS_ZP, 2, 1>(c, A, B, S, Z, Y, m, n, k, st);
        case 3: return stream_cpl<BITS, BS, HAS_ZP, 3, 1>(c, A, B, S, Z, Y, m, n, k, st);
        case 4: return stream_cpl<BITS, BS, HAS_ZP, 4, 1>(c, A, B, S, Z, Y, m, n, k, st);
        default: return hipErrorInvalidValue;
    }
}

template <int BITS, int BS>
hipError_t stream_zp(const StreamConfig& c, const void* a, const uint8_t* b, const void* s,
                     const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, hipStream_t st) {
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
