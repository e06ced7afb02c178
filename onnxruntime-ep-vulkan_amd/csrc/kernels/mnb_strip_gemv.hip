// Strip GEMV: MatMulNBits with at most 16 rows per group on gfx950 MFMA -- dense decode batches,
// routed experts (rows grouped by expert) and the accuracy_level = 4 int8 path.  int4 weights,
// block_size >= 32, fp16 activations (or their int8 codes) and fp16 output.
//
// Work split.  A workgroup of W wavefronts owns one group (expert), one 16-row tile and a run of
// S strips of 16 output columns.  K is cut into 128-k quads that are split over the W
// wavefronts; each wavefront loads the MFMA A operands of its quads once, keeps them in
// registers for the whole run and streams the weights of its quads strip after strip, so the
// activations are read once per workgroup rather than once per strip.
//
// Loads.  For quad q, lane (n = l % 16, g = l / 16) reads the 16 bytes of chunk 4q + g (32 int4
// weights) of column n: one instruction covers 16 runs of 64 contiguous bytes.  A 4 x 4 dword
// transpose across the lane rows turns the four chunks of a quad into the B operands of four
// 16x16x32 MFMAs (lane (n, g) supplies k = 8g .. 8g + 7 of each chunk).  The weights of the
// next two strips (one, where registers are short) are in flight while a strip is computed.  The run's scales and zero points
// are one contiguous byte range per tensor (ORT's [N][K/bs] layouts); the workgroup copies them
// into LDS with 16-byte loads issued behind the first strip's weights.
//
// Arithmetic.  fp16: exact (q - zp) operands on v_mfma_f32_16x16x32_f16, the fp32 partial of a
// block scaled once by the block's scale (the reference kernel's per-block fp32 partial,
// rust/shaders/glsl/templates/q_gemv.comp:571-579).  int8: the activations arrive as the codes
// of quantize_a_int8 (written once per call in the weights' [0,2,4,6,1,3,5,7] order, and within
// each whole quad with a lane row's four chunks as two 16-byte pieces, so one load covers 64
// contiguous bytes of each row -- quantising inside every workgroup would repeat it per run of
// strips) with block-major scales over 16 rows; v_mfma_i32_16x16x64_i8 (x32 for block 32) gives
// exact int32 block dots, scaled by a_scale * b_scale in fp32.
//
// Reduction.  Each wavefront's 16 x 16 partial tile of a strip goes to LDS; every four strips
// the W partials are summed in wavefront order (run-to-run deterministic) and stored, so the
// LDS buffer does not grow with the run and runs can be long.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

// Threads per workgroup the instantiation is compiled for, 0 where it would not fit its
// registers without spilling: the arrays grow with QW (A operands 16 VGPRs per quad in fp16, 8
// in int8 plus a 4-row scale vector per block; the strips of weights in flight 4 per quad
// each), and 1024 threads leave each wavefront 128 VGPRs, 512 threads 256.
__host__ __device__ constexpr int strip_max_threads(bool i8, int bs, int qw) {
    if (!i8) return qw <= 2 ? 1024 : (qw <= 6 ? 512 : 0);
    if (bs == 32) return qw <= 2 ? 1024 : (qw <= 4 ? 512 : 0);
    if (bs == 64) return qw <= 3 ? 1024 : (qw <= 6 ? 512 : 0);
    return qw <= 4 ? 1024 : 512;
}

// Strips whose partial tiles are summed together: W x period KB of LDS, 32 KB.
__host__ __device__ constexpr int strip_period(int waves) { return waves >= 32 ? 1 : 32 / waves; }

namespace {

// A copy of `bytes` bytes from global memory into LDS in two halves: issue() requests the first
// kEarly 16-byte pieces of each thread (when `vec`: source 16-byte aligned), so the requests
// are in flight while other loads are issued; finish() stores them and copies the rest.
template <int kEarly>
struct LdsCopy {
    u32x4 v[kEarly];
    __device__ __forceinline__ void issue(const uint8_t* __restrict__ src, int bytes, bool vec) {
        const int nvec = vec ? bytes >> 4 : 0;
        const u32x4* __restrict__ s4 = reinterpret_cast<const u32x4*>(src);
#pragma unroll
        for (int b = 0; b < kEarly; ++b) {
            const int i = (int)threadIdx.x + b * (int)blockDim.x;
            if (i < nvec) v[b] = s4[i];
        }
    }
    __device__ __forceinline__ void finish(uint8_t* __restrict__ dst,
                                           const uint8_t* __restrict__ src, int bytes, bool vec) {
        const int nvec = vec ? bytes >> 4 : 0;
        u32x4* __restrict__ d4 = reinterpret_cast<u32x4*>(dst);
#pragma unroll
        for (int b = 0; b < kEarly; ++b) {
            const int i = (int)threadIdx.x + b * (int)blockDim.x;
            if (i < nvec) d4[i] = v[b];
        }
        const u32x4* __restrict__ s4 = reinterpret_cast<const u32x4*>(src);
        for (int i = (int)threadIdx.x + kEarly * (int)blockDim.x; i < nvec; i += (int)blockDim.x)
            d4[i] = s4[i];
        for (int i = (nvec << 4) + (int)threadIdx.x; i < bytes; i += (int)blockDim.x)
            dst[i] = src[i];
    }
};

}  // namespace

// SWIGLU: the stored tile is SwiGLU of its interleaved (gate, linear) column pairs (StripSwiglu).
// NATIVE (fp16 only): Bs is the MFMA-native strip copy (no lane transpose, reordered nibbles).
template <bool I8, int BS, bool HAS_ZP, int QW, bool SWIGLU, bool NATIVE>
__global__ void __launch_bounds__(strip_max_threads(I8, BS, QW) ? strip_max_threads(I8, BS, QW) : 256)
strip_gemv(const void* __restrict__ Av, const float* __restrict__ a_scale,
           const int32_t* __restrict__ row_index,
           const int32_t* __restrict__ offsets, const uint8_t* __restrict__ B,
           const f16* __restrict__ Sc, const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M,
           int N, int K, int S, int vec_s, int vec_z, StripSwiglu sw,
           const uint8_t* __restrict__ Bs) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int CPB = BS / 32;                         // 32-k chunks per block: 1, 2 or 4
    constexpr int BPQ = 4 / CPB;                         // blocks per quad
    const int lane = threadIdx.x & 63;
    // wave-uniform by construction; in an SGPR, the K share, its quad count and every
    // per-quad condition below are scalar (branches, not lane masks) and address bases scalar
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int W = blockDim.x >> 6;
    const int kPeriod = strip_period(W);
    const int nl = lane & 15;
    const int g = lane >> 4;
    const int chunks = K >> 5;
    const int Q = (chunks + 3) >> 2;
    const int bpc = K / BS;
    const int zpb = (bpc + 1) >> 1;
    const int n0 = blockIdx.x * S * 16;
    const int ns = min(S, (N - n0 + 15) >> 4);           // strips of this run (>= 1)

    const int e = offsets ? (int)blockIdx.y : 0;
    const int64_t wb = (int64_t)e * N * (K / 2);
    const int64_t ws = (int64_t)e * N * bpc;
    const int64_t wz = (int64_t)e * N * zpb;
    const int q_lo = (wave * Q) / W;
    const int q_n = ((wave + 1) * Q) / W - q_lo;         // quads of this wavefront, <= QW
    const uint8_t* __restrict__ Bg = B + wb;

    // Lane (n, g) takes chunk 4 q + g of column n: from ORT's layout, or from the strip-major
    // copy (launch_strip_pack: per group, strip and quad one 1 KB run in this lane order, the
    // chunks past K zero; chunks past K are never used either way).
    const int nst = (N + 15) >> 4;
    auto fetch = [&](int s, u32x4(&buf)[QW]) {
        const uint8_t* bc;
        int64_t step;
        if (Bs) {
            const int st = min((n0 >> 4) + s, nst - 1);
            bc = Bs + (((int64_t)e * nst + st) * Q + q_lo) * 1024 + 64 * nl + 16 * g;
            step = 1024;
        } else {
            const int col = min(n0 + 16 * s + nl, N - 1);
            bc = Bg + (int64_t)col * (K / 2) + 16 * (4 * q_lo + g);
            step = 64;
        }
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            if (j < q_n) {                               // wave-uniform
                // ORT's layout: the last quad's chunks past K are clamped onto the last chunk
                const int64_t off = Bs || 4 * (q_lo + j) + g < chunks
                                        ? step * j
                                        : 16 * (int64_t)(chunks - 1 - (4 * q_lo + g));
                buf[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bc + off));
            }
        }
    };

    // Strips in flight ahead of the one computed: two, fewer where the registers are short
    // (the int8 path's runs are usually a single strip).
    constexpr int AHEAD = I8 ? (QW >= 4 ? 0 : 1) : (QW > 3 ? 1 : 2);
    u32x4 b0[QW], b1[AHEAD > 0 ? QW : 1], b2[AHEAD > 1 ? QW : 1];

    // The run's scales and zero points (LDS copies), requested with the first strips' weights.
    const int ncols = min(16 * S, N - n0);
    const int s_bytes = (16 * S * bpc * 2 + 15) & ~15;
    const int z_bytes = HAS_ZP ? ((16 * S * zpb + 15) & ~15) : 0;
    f16* const sS = reinterpret_cast<f16*>(smem);
    uint8_t* const sZ = smem + s_bytes;
    f32x4* const red = reinterpret_cast<f32x4*>(smem + s_bytes + z_bytes);
    const uint8_t* const s_src = reinterpret_cast<const uint8_t*>(Sc + ws + (int64_t)n0 * bpc);
    const uint8_t* const z_src = HAS_ZP ? Z + wz + (int64_t)n0 * zpb : nullptr;
    LdsCopy<4> scopy;
    LdsCopy<1> zcopy;
    auto request = [&]() {
        fetch(0, b0);
        if constexpr (AHEAD > 1) {
            if (ns > 1) fetch(1, b1);
        }
        scopy.issue(s_src, ncols * bpc * 2, vec_s != 0);
        if constexpr (HAS_ZP) zcopy.issue(z_src, ncols * zpb, vec_z != 0);
    };

    // Rows of this workgroup.  The first row tile of a group almost always has rows, so its
    // requests go out before the group's row range is read (a dependent round trip, and for
    // gathered rows a second one before the activations); later tiles read it first.
    const bool eager = blockIdx.z == 0;
    // Rows from the routing itself (StripSwiglu): the expert ids are requested before the
    // weights, so that waiting for them does not wait for the weights (loads complete in order)
    constexpr int kChunks = 16;                          // R <= 1024
    const bool routed = SWIGLU && sw.expert_of;
    int xv[SWIGLU ? kChunks : 1];
    if constexpr (SWIGLU) {
        if (routed) {
#pragma unroll
            for (int c = 0; c < kChunks; ++c)            // clamped, unpredicated: issued together
                xv[c] = sw.expert_of[min(64 * c + lane, sw.R - 1)];
        }
    }
    if (eager) request();
    int row_lo = 0, row_hi = M;
    int arow;
    if constexpr (SWIGLU) {
      if (routed) {
        // Every wavefront scans the R assignments in 64-lane chunks -- a ballot for "expert
        // below e" counts row_lo, one for "expert e" ranks this expert's assignments -- and
        // keeps the tokens of this tile's rows in its own 16 LDS slots (the partial-tile
        // buffer, not used before the first strip).
        int32_t* const s_tok = reinterpret_cast<int32_t*>(smem + s_bytes + z_bytes) + 16 * wave;
        int n_lt = 0, n_eq = 0;
        const int t0 = 16 * (int)blockIdx.z;
        const bool publish = blockIdx.x == 0 && blockIdx.z == 0 && wave == 0;
        int rank[kChunks];
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            if (64 * c >= sw.R) break;                   // wave-uniform
            const bool valid = 64 * c + lane < sw.R;
            const uint64_t m_lt = __ballot(valid && xv[c] < e);
            const uint64_t m_eq = __ballot(valid && xv[c] == e);
            rank[c] = n_eq + (int)__builtin_amdgcn_mbcnt_hi(
                                 (uint32_t)(m_eq >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m_eq, 0));
            if (valid && xv[c] == e && rank[c] >= t0 && rank[c] < t0 + 16)
                s_tok[rank[c] - t0] = (64 * c + lane) / sw.k;
            n_lt += __popcll(m_lt);
            n_eq += __popcll(m_eq);
        }
        row_lo = n_lt;
        row_hi = n_lt + n_eq;
        if (publish) {                                   // before any early exit
            if (lane == 0) {
                sw.offsets[e] = row_lo;
                if (e == (int)gridDim.y - 1) sw.offsets[e + 1] = sw.R;
            }
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                if (64 * c >= sw.R) break;
                if (64 * c + lane < sw.R && xv[c] == e) sw.pos_of[64 * c + lane] = row_lo + rank[c];
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int r0 = row_lo + t0;
        if (r0 >= row_hi) return;                        // the whole workgroup, before a barrier
        if (!eager) request();
        arow = s_tok[min(nl, row_hi - r0 - 1)];
      }
    }
    if (!routed) {
        if (offsets) {
            row_lo = offsets[e];
            row_hi = offsets[e + 1];
        }
        const int r0 = row_lo + blockIdx.z * 16;
        if (r0 >= row_hi) return;                        // the whole workgroup, before a barrier
        if (!eager) request();
        // ---- this lane's row of the tile (row nl) ----
        int rr = r0 + nl;
        rr = rr < row_hi ? rr : row_hi - 1;
        arow = row_index ? row_index[rr] : rr;
    }
    const int r0 = row_lo + blockIdx.z * 16;

    // ---- A operands of this wavefront's quads: row nl of the tile, k = 32c + 8g .. + 8 ----
    f16x8 af[I8 ? 1 : QW][4];
    i32x2 aq[I8 ? QW : 1][4];
    f32x4 sao[I8 ? QW : 1][I8 ? BPQ : 1];                // int8: a_scale of rows 4g .. 4g + 3
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        if (I8 && j < q_n && 4 * (q_lo + j) + 3 < chunks) {
            // whole quad in the quantiser's quad-interleaved layout: chunks 0, 1 of this lane
            // row at 16 g, chunks 2, 3 at 64 + 16 g -- two loads, each 64 contiguous bytes of
            // every row of the tile
            const int8_t* p = static_cast<const int8_t*>(Av) + (int64_t)arow * K +
                              128 * (q_lo + j) + 16 * g;
            const u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
            const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 64);
            aq[j][0] = i32x2{(int32_t)v0.x, (int32_t)v0.y};
            aq[j][1] = i32x2{(int32_t)v0.z, (int32_t)v0.w};
            aq[j][2] = i32x2{(int32_t)v1.x, (int32_t)v1.y};
            aq[j][3] = i32x2{(int32_t)v1.z, (int32_t)v1.w};
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int c = 4 * (q_lo + j) + t;
                const bool live = j < q_n && c < chunks;
                const int64_t off = (int64_t)arow * K + 32 * (int64_t)min(c, chunks - 1) + 8 * g;
                if constexpr (!I8) {
                    const f16x8 v = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(Av) + off);
                    af[j][t] = live ? v : f16x8{};
                } else {
                    // a partial last quad (natural order) or a quad past this wavefront's share
                    const u32x2 v = *reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(Av) + off);
                    aq[j][t] = live ? i32x2{(int32_t)v.x, (int32_t)v.y} : i32x2{0, 0};
                }
            }
        }
        if constexpr (I8) {
            // block-major scales over the 16 rows of the tile: rows 4g .. 4g + 3 in one load
#pragma unroll
            for (int b = 0; b < BPQ; ++b) {
                const int blk = min((128 * (q_lo + j) + BS * b) / BS, bpc - 1);
                sao[j][b] = *reinterpret_cast<const f32x4*>(a_scale + (int64_t)blk * 16 + 4 * g);
            }
        }
    }

    scopy.finish(smem, s_src, ncols * bpc * 2, vec_s != 0);
    if constexpr (HAS_ZP) zcopy.finish(sZ, z_src, ncols * zpb, vec_z != 0);

    __syncthreads();

    auto compute = [&](int s, const u32x4(&buf)[QW]) {
        const int cl = 16 * s + nl;                      // column within the run
        const f16* __restrict__ ls = sS + cl * bpc;
        const uint8_t* __restrict__ lz = sZ + cl * zpb;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            if (j >= q_n) break;                         // wave-uniform
            uint32_t v0 = buf[j].x, v1 = buf[j].y, v2 = buf[j].z, v3 = buf[j].w;
            if constexpr (!NATIVE) transpose_rows(v0, v1, v2, v3);
            const uint32_t wt[4] = {v0, v1, v2, v3};
            if constexpr (!I8) {
                // one accumulator per block of the quad, scaled after the quad's MFMAs
                f32x4 d[BPQ];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int c = 4 * (q_lo + j) + t;
                    const int blk = min((32 * c) / BS, bpc - 1);
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((lz[blk >> 1] >> ((blk & 1) * 4)) & 0xFu);
                    f16x8 bop;
                    if constexpr (NATIVE) {
                        bop = native_pairs(wt[t], as_h2(0xE400E400u + (uint32_t)z * 0x10001u),
                                           as_h2(0xD400D400u + (uint32_t)z * 0x100010u));
                    } else {
                        const f16x2 zo = zoff4(z);
                        bop.s01 = nib_pair<0>(wt[t], zo);
                        bop.s23 = nib_pair<1>(wt[t], zo);
                        bop.s45 = nib_pair<2>(wt[t], zo);
                        bop.s67 = nib_pair<3>(wt[t], zo);
                    }
                    d[t / CPB] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        af[j][t], bop, t % CPB == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[t / CPB], 0, 0, 0);
                }
#pragma unroll
                for (int b = 0; b < BPQ; ++b) {          // each block's partial, scaled once
                    const int blk = min((32 * (4 * (q_lo + j) + CPB * b)) / BS, bpc - 1);
                    const float sc = (float)ls[blk];
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(d[b][q], sc, acc[q]);
                }
            } else {
                i32x4 dot = {0, 0, 0, 0};
                i32x2 bq[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int c = 4 * (q_lo + j) + t;
                    const int blk = min((32 * c) / BS, bpc - 1);
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((lz[blk >> 1] >> ((blk & 1) * 4)) & 0xFu);
                    bq[t] = qz_i8(wt[t], (uint32_t)(128 - z) * 0x01010101u);
                }
#pragma unroll
                for (int t = 0; t < 4; t += (CPB >= 2 ? 2 : 1)) {
                    if constexpr (CPB >= 2) {
                        // two chunks of one block in one 16x16x64 MFMA: A and B place the
                        // same k in the same (lane row, slot)
                        const i32x4 a4 = {aq[j][t].x, aq[j][t].y, aq[j][t + 1].x, aq[j][t + 1].y};
                        const i32x4 b4 = {bq[t].x, bq[t].y, bq[t + 1].x, bq[t + 1].y};
                        dot = __builtin_amdgcn_mfma_i32_16x16x64_i8(a4, b4, dot, 0, 0, 0);
                    } else {
                        dot = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            __builtin_bit_cast(long, aq[j][t]), __builtin_bit_cast(long, bq[t]), dot,
                            0, 0, 0);
                    }
                    const int te = t + (CPB >= 2 ? 1 : 0);   // last chunk covered so far
                    if ((te + 1) % CPB == 0) {               // block end: scale it
                        const int c = 4 * (q_lo + j) + te;
                        const int blk = min((32 * c) / BS, bpc - 1);
                        const float sb = (float)ls[blk];
                        const int b = te / CPB;
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            acc[q] = __builtin_fmaf((float)dot[q], sao[j][b][q] * sb, acc[q]);
                        dot = i32x4{0, 0, 0, 0};
                    }
                }
            }
        }
        red[(wave * kPeriod + s % kPeriod) * 64 + lane] = acc;
    };

    for (int s = 0; s < ns; ++s) {
        if constexpr (AHEAD > 1) {
            if (s + 2 < ns) fetch(s + 2, b2);
        } else if constexpr (AHEAD == 1) {
            if (s + 1 < ns) fetch(s + 1, b1);
        } else {
            if (s > 0) fetch(s, b0);
        }
        compute(s, b0);
        if constexpr (AHEAD > 0) {
#pragma unroll
            for (int j = 0; j < QW; ++j) {
                b0[j] = b1[j];
                if constexpr (AHEAD > 1) b1[j] = b2[j];
            }
        }
        // Every kPeriod strips (and at the end of the run): fixed-order sum of the W partial
        // tiles of those strips, stored, then the partial buffer is free again.  The weights
        // of the next strips stay in flight across the two barriers.
        if ((s + 1) % kPeriod == 0 || s + 1 == ns) {
            const int p0 = s - s % kPeriod;
            const int np = s + 1 - p0;
            __syncthreads();
            for (int idx = threadIdx.x; idx < np * 64; idx += blockDim.x) {
                const int i = idx >> 6;
                const int ll = idx & 63;
                f32x4 sum = red[i * 64 + ll];
                for (int w = 1; w < W; ++w) sum += red[(w * kPeriod + i) * 64 + ll];
                const int col = n0 + 16 * (p0 + i) + (ll & 15);
                if constexpr (SWIGLU) {
                    // the odd column's (linear) sums from lane ll ^ 1, with every lane active
                    f32x4 lin;
#pragma unroll
                    for (int q = 0; q < 4; ++q) lin[q] = dpp_f<0xB1>(sum[q]);
                    if (col >= N || (ll & 1)) continue;
                    const f16* bb = static_cast<const f16*>(sw.bias);
                    const float bg = bb ? (float)bb[(int64_t)e * N + col] : 0.f;
                    const float bl = bb ? (float)bb[(int64_t)e * N + col + 1] : 0.f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int r = r0 + 4 * (ll >> 4) + q;
                        // h is rounded to fp16 before its bias, as where h is stored
                        float gt = (float)(f16)sum[q] + bg;
                        float lt = (float)(f16)lin[q] + bl;
                        if (sw.has_limit) {
                            gt = fminf(gt, sw.limit);
                            lt = fminf(fmaxf(lt, -sw.limit), sw.limit);
                        }
                        const float a = gt / (1.f + expf(-sw.alpha * gt)) * (lt + sw.beta);
                        if (r < row_hi) Y[(int64_t)r * (N >> 1) + (col >> 1)] = (f16)a;
                    }
                } else {
                    if (col >= N) continue;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int r = r0 + 4 * (ll >> 4) + q;
                        if (r < row_hi) Y[(int64_t)r * N + col] = (f16)sum[q];
                    }
                }
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

namespace {

constexpr int kQW[] = {1, 2, 3, 4, 6, 8};

int round_qw(int64_t q) {
    for (int v : kQW)
        if (q <= v) return v;
    return 0;
}

}  // namespace

bool strip_gemv_forced_off() {
    const char* v = std::getenv("MNB_FORCE_KERNEL");
    return v && !std::strcmp(v, "group");
}

bool strip_geometry(int64_t n, int64_t k, int64_t groups, int64_t rows_bound, bool i8, int bs,
                    bool has_zp, StripGeom* out) {
    if (bs != 32 && bs != 64 && bs != 128) return false;
    if (k <= 0 || k % 32 || k % bs || n <= 0 || groups <= 0) return false;
    const int64_t q = (k / 32 + 3) / 4;
    if (i8 && rows_bound > 16) return false;             // block-major scales cover 16 rows
    StripGeom g{};
    // The fewest wavefronts that keep a wavefront's quads at 4 or fewer, else the most that
    // the instantiation's register budget allows.
    for (int pass = 0; pass < 2 && g.waves == 0; ++pass) {
        for (int w : {4, 8, 16}) {
            const int ww = pass == 0 ? w : 20 - w;       // second pass: 16, 12, 8, 4
            const int qw = round_qw((q + ww - 1) / ww);
            if (qw == 0 || (pass == 0 && qw > 4)) continue;
            if (64 * ww > strip_max_threads(i8, bs, qw)) continue;
            g.waves = ww;
            g.qw = qw;
            break;
        }
    }
    if (g.waves == 0) return false;
    const int64_t nstrips = (n + 15) / 16;
    const int64_t bpc = k / bs;
    const int64_t zpb = (bpc + 1) / 2;
    // Runs as long as 80 KB of LDS (partial tiles, then staged scales and zero points: two
    // workgroups per CU) allow, sized so that the launch fills whole rounds of resident workgroups (by registers
    // and LDS).
    const int64_t per_strip = 16 * (bpc * 2 + (has_zp ? zpb : 0)) + 32;
    const int64_t red_bytes = (int64_t)g.waves * strip_period(g.waves) * 64 * sizeof(f32x4);
    const int64_t s_max =
        std::max<int64_t>(1, std::min<int64_t>(32, (80 * 1024 - red_bytes) / per_strip));
    const int waves_per_simd = g.qw <= 3 ? 4 : (g.qw == 4 ? 3 : (g.qw == 6 ? 2 : 1));
    const int64_t by_regs = std::max(1, 4 * waves_per_simd / g.waves);
    const int64_t by_lds = std::max<int64_t>(1, (160 * 1024) / (s_max * per_strip + red_bytes + 64));
    const int64_t slots = 256 * std::min(by_regs, by_lds);
    const int64_t total = groups * nstrips;
    const int64_t rounds = std::max<int64_t>(1, (total + slots * s_max - 1) / (slots * s_max));
    int64_t s = (total + rounds * slots - 1) / (rounds * slots);
    s = std::max<int64_t>(1, std::min<int64_t>(s, std::min<int64_t>(s_max, nstrips)));
    g.strips = (int)s;
    g.gx = (nstrips + s - 1) / s;
    g.gy = groups;
    g.gz = (std::max<int64_t>(rows_bound, 1) + 15) / 16;
    g.lds = (size_t)((16 * s * bpc * 2 + 15) & ~15) + (has_zp ? (size_t)((16 * s * zpb + 15) & ~15) : 0) +
            (size_t)red_bytes;
    if (g.lds > 80 * 1024) return false;
    if (g.gx > 0x7fffffff || g.gy > 65535 || g.gz > 65535) return false;
    *out = g;
    return true;
}

namespace {

template <bool I8, int BS, bool HAS_ZP, int QW, bool SWIGLU>
hipError_t strip_go(const StripGeom& g, const void* a, const float* a_scale,
                    const int32_t* row_index,
                    const int32_t* offsets, const uint8_t* b, const void* s, const uint8_t* z,
                    void* y, int64_t m, int64_t n, int64_t k, int vec_s, int vec_z,
                    const StripSwiglu& sw, hipStream_t st, const uint8_t* bs_) {
    if constexpr (strip_max_threads(I8, BS, QW) == 0 || (SWIGLU && (I8 || HAS_ZP))) {
        return hipErrorInvalidValue;                     // not instantiated (see above)
    } else {
    // the fp16 path reads a strip copy in the MFMA-native order (the only copies passed to it
    // are the QMoE experts', packed that way); the int8 path is never given one
    auto kern = !I8 && bs_ ? strip_gemv<I8, BS, HAS_ZP, QW, SWIGLU, !I8>
                           : strip_gemv<I8, BS, HAS_ZP, QW, SWIGLU, false>;
    if (g.lds > 80 * 1024 || 64 * g.waves > strip_max_threads(I8, BS, QW))
        return hipErrorInvalidValue;
    const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), g.lds);
    if (ea != hipSuccess) return ea;
    const dim3 grid((unsigned)g.gx, (unsigned)g.gy, (unsigned)g.gz);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
    hipLaunchKernelGGL(kern, grid, block, g.lds, st, a, a_scale, row_index,
                       offsets, b, static_cast<const f16*>(s), z, static_cast<f16*>(y), (int)m,
                       (int)n, (int)k, g.strips, vec_s, vec_z, sw, bs_);
    return hipGetLastError();
    }
}

template <bool I8, int BS, bool HAS_ZP, bool SWIGLU>
hipError_t strip_qw(const StripGeom& g, const void* a, const float* a_scale,
                    const int32_t* row_index,
                    const int32_t* offsets, const uint8_t* b, const void* s, const uint8_t* z,
                    void* y, int64_t m, int64_t n, int64_t k, int vec_s, int vec_z,
                    const StripSwiglu& sw, hipStream_t st, const uint8_t* bs_) {
#define MNB_STRIP_GO(QW_)                                                                          \
    case QW_:                                                                                      \
        return strip_go<I8, BS, HAS_ZP, QW_, SWIGLU>(g, a, a_scale, row_index, offsets, b, s, z, y, \
                                                     m, n, k, vec_s, vec_z, sw, st, bs_)
    switch (g.qw) {
        MNB_STRIP_GO(1);
        MNB_STRIP_GO(2);
        MNB_STRIP_GO(3);
        MNB_STRIP_GO(4);
        MNB_STRIP_GO(6);
        MNB_STRIP_GO(8);
        default: return hipErrorInvalidValue;
    }
#undef MNB_STRIP_GO
}

template <bool I8>
hipError_t strip_bs(int bs, const StripGeom& g, const void* a, const float* a_scale,
                    const int32_t* row_index,
                    const int32_t* offsets, const uint8_t* b, const void* s, const uint8_t* z,
                    void* y, int64_t m, int64_t n, int64_t k, int vec_s, int vec_z,
                    const StripSwiglu* sw, hipStream_t st, const uint8_t* bs_) {
    const StripSwiglu none{};
#define MNB_STRIP_ZP(BS_)                                                                          \
    if (sw) return strip_qw<I8, BS_, false, true>(g, a, a_scale, row_index, offsets, b, s, z, y,   \
                                                  m, n, k, vec_s, vec_z, *sw, st, bs_);            \
    return z ? strip_qw<I8, BS_, true, false>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, \
                                              k, vec_s, vec_z, none, st, bs_)                      \
             : strip_qw<I8, BS_, false, false>(g, a, a_scale, row_index, offsets, b, s, z, y, m,   \
                                               n, k, vec_s, vec_z, none, st, bs_)
    switch (bs) {
        case 32: MNB_STRIP_ZP(32);
        case 64: MNB_STRIP_ZP(64);
        case 128: MNB_STRIP_ZP(128);
        default: return hipErrorInvalidValue;
    }
#undef MNB_STRIP_ZP
}

}  // namespace

bool strip_gemv_aligned(const void* a, const uint8_t* b, const void* s, const uint8_t* z,
                        bool i8) {
    (void)s;
    (void)z;                                             // staged element-wise when sub-aligned
    return reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

hipError_t launch_strip_gemv(const StripGeom& g, bool i8, const void* a, const float* a_scale,
                             const int32_t* row_index,
                             const int32_t* offsets, const uint8_t* b, const void* s,
                             const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bs,
                             hipStream_t st, const StripSwiglu* swiglu, const uint8_t* b_strips) {
    if (m == 0) return hipSuccess;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(b) % 16 ||
        reinterpret_cast<uintptr_t>(b_strips) % 16 || (i8 && !a_scale) ||
        (swiglu && (i8 || z || n % 2)))
        return hipErrorInvalidValue;
    const int64_t bpc = k / bs;
    const int64_t zpb = (bpc + 1) / 2;
    // 16-byte copies of the scales / zero points need every run's first byte aligned: the
    // tensor base, and each group's slice when there are several groups.
    const bool multi = offsets != nullptr && g.gy > 1;
    const int vec_s = reinterpret_cast<uintptr_t>(s) % 16 == 0 && (!multi || (n * bpc * 2) % 16 == 0);
    const int vec_z = z && reinterpret_cast<uintptr_t>(z) % 16 == 0 && (!multi || (n * zpb) % 16 == 0);
    if (i8) return strip_bs<true>(bs, g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, vec_s, vec_z, nullptr, st, b_strips);
    return strip_bs<false>(bs, g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, vec_s, vec_z, swiglu, st, b_strips);
}

}  // namespace mnb

