// Batched decode at 4..16 fp16 rows: fp16 activations x int4 weights on gfx950 MFMA, S 16-column
// strips per workgroup over the whole of K.
//
// A workgroup of KW wavefronts owns S consecutive strips of 16 columns; wavefront w owns quads
// [w R, w R + R) of K (a quad is 128 k; KW R = K / 128) of all S strips.  Every lane first
// requests the activations of the wavefront's quads -- one load per 4 rows x 256 bytes of a quad
// (rows past M repeat row M - 1 and are never stored) -- then its columns' block scales and zero
// points for those quads (one contiguous run per column), then its S R 16-byte weight loads
// (lane (n, g): chunk 4 q + g of column n of each strip, streamed past the caches), so the
// activations, needed first, are not queued behind the weights.  Quad by quad the activations
// pass through the wavefront's own LDS slot into the v_mfma_f32_16x16x32_f16 A operand layout
// (lane (n, g): row n, k = 32 c + 8 g .. + 7 of each 32-k chunk c), kept in registers for all S
// strips; nothing waits for another wavefront until the end.
// Per quad a 4 x 4 dword transpose across the lane rows leaves lane (n, g) holding, for each chunk
// c, the eight weights k = 32 c + 8 g .. + 7 of column n -- the B operand -- which become exact
// fp16 (q - zp) values; the MFMAs of one quant block accumulate its exact-product fp32 partial,
// scaled by the block's scale into the lane's accumulator (the reference's per-block fp32 partial
// scaled once, rust/shaders/glsl/templates/q_gemv.comp:571-579).  The KW partial tiles are added
// in LDS in wavefront order (run-to-run deterministic) and stored as fp16.
//
// Each workgroup reads all of A (16 rows x K x 2 bytes, from L2): the price of having no
// cross-workgroup reduction; S strips per workgroup divide that traffic by S (one strip per
// workgroup read 96 KB of A per 24 KB of weights at K = 3072 and ran the 16-row gate_up at
// 19 us, slower than the strip GEMV).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

constexpr int kBatchMaxWaves = 16;
// Bytes per row of a wavefront's LDS slot: one quad of fp16 activations (256 bytes) padded by 16
// so that the 16 rows' operand reads start in distinct bank groups.
constexpr int kBatchSlotRow = 256 + 16;

template <int BS, bool HAS_ZP, int R, int S, bool NATIVE>
__global__ void __launch_bounds__(64 * kBatchMaxWaves)
batch_stream(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ Sc,
             const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K,
             const uint8_t* __restrict__ Bs) {
    constexpr int CPB = BS / 32;                         // 32-k chunks per block: 1, 2 or 4
    constexpr int BPQ = 4 / CPB;                         // blocks per quad
    extern __shared__ f32x4 sRed[];                      // [KW][S][64], then KW slots
    const int lane = threadIdx.x & 63;
    const int kw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int KW = blockDim.x >> 6;
    const int nl = lane & 15;
    const int g = lane >> 4;
    const int bpc = K / BS;                              // a multiple of 4
    const int zpb = bpc >> 1;
    const int strip0 = blockIdx.x * S;
    const int q0 = kw * R;                               // this wavefront's first quad

    // ---- 1. the activations of the wavefront's quads: each load covers 4 rows x 256 bytes of
    // one quad (whole lines; loading the MFMA operands directly touched 16 half lines per load)
    const int lrow = lane >> 4;
    const int lpc = lane & 15;
    // A load whose four rows all lie past M (4 c >= M: uniform over the wavefront) is not made;
    // those rows take zeros and their MFMA output rows are never stored.
    f16x8 raw[R][4];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            raw[j][c] = 4 * c < M ? *reinterpret_cast<const f16x8*>(
                                        A + (int64_t)min(4 * c + lrow, M - 1) * K +
                                        128 * (q0 + j) + 8 * lpc)
                                  : f16x8{};
    // ---- 2. the columns' block scales and zero points for those quads ----------------------
    constexpr int NS = R * BPQ;                          // blocks of the wavefront's quads
    constexpr int NZ = (NS + 1) / 2;
    const int b0 = q0 * BPQ;                             // first block; even unless NS == 1
    uint16_t sv[S][NS];
    uint8_t zv[S][NZ];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        const int col = min(16 * (strip0 + t) + nl, N - 1);
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(Sc) + (int64_t)col * bpc + b0;
        const uint8_t* zp = HAS_ZP ? Z + (int64_t)col * zpb + (b0 >> 1) : nullptr;
        if constexpr (NS % 4 == 0) {
            // 8-byte and 2-byte aligned: bpc % 4 == 0, b0 % 4 == 0, the launcher checks the bases
#pragma unroll
            for (int i = 0; i < NS / 4; ++i) {
                const u32x2 v = *reinterpret_cast<const u32x2*>(sp + 4 * i);
                sv[t][4 * i] = (uint16_t)v.x;
                sv[t][4 * i + 1] = (uint16_t)(v.x >> 16);
                sv[t][4 * i + 2] = (uint16_t)v.y;
                sv[t][4 * i + 3] = (uint16_t)(v.y >> 16);
            }
            if constexpr (HAS_ZP) {
#pragma unroll
                for (int i = 0; i < NZ / 2; ++i) {
                    const uint16_t v = *reinterpret_cast<const uint16_t*>(zp + 2 * i);
                    zv[t][2 * i] = (uint8_t)v;
                    zv[t][2 * i + 1] = (uint8_t)(v >> 8);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NS; ++i) sv[t][i] = sp[i];
            if constexpr (HAS_ZP) {
#pragma unroll
                for (int i = 0; i < NZ; ++i) zv[t][i] = zp[i];
            }
        }
    }

    // ---- 3. the wavefront's weights: lane (n, g) takes chunk 4 q + g of column n, either from
    // ORT's layout (16 columns x 64 bytes per load instruction) or from the strip-major copy made
    // at upload (mnb_weights_prepack: the same 16 x 64 bytes stored as one 1 KB run per strip
    // and quad, in this lane order) ----------------------------------------------------------------
    u32x4 bw[S][R];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        const uint8_t* bc;
        if constexpr (NATIVE) {
            const int st = min(strip0 + t, (N + 15) / 16 - 1);
            bc = Bs + (int64_t)st * (K / 128) * 1024 + 64 * nl + 16 * g;
        } else {
            const int col = min(16 * (strip0 + t) + nl, N - 1);
            bc = B + (int64_t)col * (K / 2) + 16 * g;
        }
#pragma unroll
        for (int j = 0; j < R; ++j)
            bw[t][j] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(bc + (NATIVE ? 1024 : 64) * (int64_t)(q0 + j)));
    }

    // With several strips, every weight request goes out before the first wait (left to itself
    // the compiler issues a strip's weights only after the previous strip's MFMAs, so the weight
    // stream waits on its own arrivals: 16 rows, gate_up 14.4 -> 12.7 us, qkv 11.3 -> 10.5 us);
    // with one strip the compiler's interleaving measured faster (o 6.2 against 6.6 us).
    if constexpr (S > 1) __builtin_amdgcn_sched_barrier(0);

    // ---- the activations into the MFMA operand layout (lane (n, g): row n, k = 32 c + 8 g ..
    // + 7 of each chunk c), quad by quad through the wavefront's own LDS slot: no other
    // wavefront touches it and a wavefront's LDS accesses complete in program order ----------
    uint8_t* const slot = reinterpret_cast<uint8_t*>(sRed) + (size_t)KW * S * 64 * 16 +
                          (size_t)kw * 16 * kBatchSlotRow;
    f16x8 av[R][4];
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            *reinterpret_cast<f16x8*>(slot + (4 * c + lrow) * kBatchSlotRow + 16 * lpc) = raw[j][c];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int c = 0; c < 4; ++c)
            av[j][c] = *reinterpret_cast<const f16x8*>(slot + nl * kBatchSlotRow + 64 * c + 16 * g);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---- 4. each strip's partial tile over this wavefront's quads ----------------------------
    f32x4 acc[S];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < R; ++j) {
            // ORT's layout: lane (n, g) holds chunk g of its column, the 4 x 4 dword transpose
            // gives it dword g of every chunk c; the native copy stores it that way already
            uint32_t v0 = bw[t][j].x, v1 = bw[t][j].y, v2 = bw[t][j].z, v3 = bw[t][j].w;
            if constexpr (!NATIVE) transpose_rows(v0, v1, v2, v3);
            const uint32_t wt[4] = {v0, v1, v2, v3};
            // one accumulator per block of the quad, scaled after all of the quad's MFMAs: the
            // next block's MFMA does not wait for this block's scaled adds to read its result
            f32x4 dot[BPQ];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int bi = j * BPQ + c / CPB;        // block within the wavefront's range
                int z = 8;
                if constexpr (HAS_ZP)
                    z = (int)((zv[t][(bi + (b0 & 1)) >> 1] >> (((b0 + bi) & 1) * 4)) & 0xFu);
                f16x8 bq;
                if constexpr (NATIVE) {
                    // (-(1024 + z), -(1024 + z)) and (-(64 + z), -(64 + z)), z in the mantissas
                    bq = native_pairs(wt[c], as_h2(0xE400E400u + (uint32_t)z * 0x10001u),
                                      as_h2(0xD400D400u + (uint32_t)z * 0x100010u));
                } else {
                    const f16x2 zo = zoff4(z);
                    bq.s01 = nib_pair<0>(wt[c], zo);
                    bq.s23 = nib_pair<1>(wt[c], zo);
                    bq.s45 = nib_pair<2>(wt[c], zo);
                    bq.s67 = nib_pair<3>(wt[c], zo);
                }
                dot[c / CPB] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    av[j][c], bq, c % CPB == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dot[c / CPB], 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < BPQ; ++b) {              // each block's partial, scaled once
                const float sb = (float)__builtin_bit_cast(f16, sv[t][j * BPQ + b]);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[t][q] = __builtin_fmaf(dot[b][q], sb, acc[t][q]);
            }
        }
    }

    // ---- 5. the KW partial tiles added in wavefront order (run-to-run deterministic): every
    // wavefront stores its tiles, then each thread sums its outputs over the KW tiles, so the
    // sum is one short chain per thread instead of (KW - 1) S dependent reads in wavefront 0 -----
    float* const red = reinterpret_cast<float*>(sRed);   // [KW][S][64 lanes][4]
#pragma unroll
    for (int t = 0; t < S; ++t) sRed[(kw * S + t) * 64 + lane] = acc[t];
    __syncthreads();
    for (int o = threadIdx.x; o < S * 256; o += blockDim.x) {
        // output o: strip ot, row orow, column on (fastest, so consecutive threads store along
        // a row); lane (on + 16 (orow / 4)) of every wavefront holds it in element orow % 4
        const int on = o & 15, orow = (o >> 4) & 15, ot = o >> 8;
        const int src = ((ot * 64 + (orow >> 2) * 16 + on) << 2) + (orow & 3);
        float v = red[src];
        for (int w = 1; w < KW; ++w) v += red[w * S * 256 + src];
        const int cc = 16 * (strip0 + ot) + on;
        if (cc < N && orow < M) Y[(int64_t)orow * N + cc] = (f16)v;
    }
}

template <int BS, bool HAS_ZP, int S>
hipError_t batch_go_s(const BatchStreamGeom& g, const void* a, const uint8_t* b, const void* s,
                      const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, hipStream_t st,
                      const uint8_t* bs_) {
    const dim3 grid((unsigned)g.gx, 1, 1);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
    const size_t lds = (size_t)g.waves * S * 64 * sizeof(f32x4) +
                       (size_t)g.waves * 16 * kBatchSlotRow;
    // instantiated for S R <= 8 only (the geometry's register budget)
#define MNB_BS_GO(R_, NAT_)                                                                       \
    {                                                                                             \
        const hipError_t ea = allow_dynamic_lds(                                                  \
            reinterpret_cast<const void*>(batch_stream<BS, HAS_ZP, R_, S, NAT_>), lds);          \
        if (ea != hipSuccess) return ea;                                                          \
        hipLaunchKernelGGL((batch_stream<BS, HAS_ZP, R_, S, NAT_>), grid, block, lds, st,        \
                           static_cast<const f16*>(a), b, static_cast<const f16*>(s), z,          \
                           static_cast<f16*>(y), (int)m, (int)n, (int)k, bs_);                    \
    }
#define MNB_BS(R_)                                                                                \
    if constexpr (S * R_ <= 8) {                                                                  \
        if (bs_) MNB_BS_GO(R_, true) else MNB_BS_GO(R_, false)                                    \
    } else {                                                                                      \
        return hipErrorInvalidValue;                                                              \
    }
    switch (g.r) {
        case 1: MNB_BS(1); break;
        case 2: MNB_BS(2); break;
        case 3: MNB_BS(3); break;
        case 4: MNB_BS(4); break;
        default: return hipErrorInvalidValue;
    }
#undef MNB_BS
#undef MNB_BS_GO
    return hipGetLastError();
}

template <int BS, bool HAS_ZP>
hipError_t batch_go(const BatchStreamGeom& g, const void* a, const uint8_t* b, const void* s,
                    const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, hipStream_t st,
                    const uint8_t* bs_) {
    switch (g.s) {
        case 1: return batch_go_s<BS, HAS_ZP, 1>(g, a, b, s, z, y, m, n, k, st, bs_);
        case 2: return batch_go_s<BS, HAS_ZP, 2>(g, a, b, s, z, y, m, n, k, st, bs_);
        case 3: return batch_go_s<BS, HAS_ZP, 3>(g, a, b, s, z, y, m, n, k, st, bs_);
        case 4: return batch_go_s<BS, HAS_ZP, 4>(g, a, b, s, z, y, m, n, k, st, bs_);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

namespace {

// Wavefronts per SIMD that the instantiations reach, [S - 1][R - 1] (their VGPR counts, 36-126
// for S R <= 8 as the compiler reports them for block 32 with zero points, in 8-register
// granules out of 512); 0 where S R > 8 is not built.
constexpr int kBatchWavesPerSimd[4][4] = {{8, 8, 6, 4}, {8, 7, 4, 4}, {8, 5, 0, 0}, {8, 4, 0, 0}};
constexpr int64_t kBatchCUs = 256;
constexpr int64_t kBatchLdsPerCU = 160 * 1024;
// Activation bytes per CU (every workgroup reads all M rows of A) above which a geometry is
// taken only when nothing else is left, and the per-workgroup size above which fewer, longer
// wavefronts are preferred.
constexpr int64_t kBatchActPerCU = 128 * 1024;
constexpr int64_t kBatchActLongWaves = 64 * 1024;

}  // namespace

bool batch_stream_geometry(int64_t m, int64_t n, int64_t k, int bs, BatchStreamGeom* out) {
    if (m < 1 || m > 16 || n < 1 || k < 128 || k % 128 || (bs != 32 && bs != 64 && bs != 128))
        return false;
    if ((k / bs) % 4) return false;                      // whole 4-block groups of scales
    const int64_t quads = k / 128;
    const int64_t strips = (n + 15) / 16;
    const int64_t act = 2 * m * k;                       // A bytes each workgroup reads
    // S strips per workgroup (each wavefront's activation registers serve all S) and R quads
    // per wavefront (K / (128 R) <= 16 wavefronts; S R <= 8 keeps an instantiation within 128
    // VGPRs), chosen in this order of preference:
    //   1. at most 128 KB of activation reads per CU (the busiest CU's workgroups each read A),
    //      else the fewest;
    //   2. the fewest strips on the busiest CU (ceil(workgroups / 256) workgroups of S strips);
    //   3. all of a CU's workgroups resident at once (by LDS and by the VGPR occupancy above);
    //   4. below 64 KB of A per workgroup the most resident wavefronts per CU, above it the
    //      fewest, longest wavefronts (larger R);
    //   5. the most CUs with work, then the smaller R.
    // Same-run sweep of every S and R on MI355X (Phi-3.5 layer, 3 / 4 / 8 / 16 rows, session
    // calls on the MFMA-native copy; ORT's layout agrees): qkv (576 strips) S = 1, R = 3 at 3-4
    // rows 6.43 us against 7.03 with S = 3, R = 2, which stays best at 8 and 16 rows (6.88 /
    // 7.18 against 7.11 / 9.50); o (192 strips) R = 2 at 3-8 rows 4.01-4.04 us against
    // 4.23-4.33 with R = 4, which stays best at 16 rows (4.36 against 4.55); gate_up (1024
    // strips) S = 2, R = 2 at 3-8 rows 8.00-8.14 us against 8.77-9.01 with S = 4, R = 2, which
    // the activation budget takes at 16 rows (9.36 us; S = 2 measured 9.20); down (K = 8192)
    // S = 1, R = 4 throughout.
    BatchStreamGeom best{};
    int64_t bkey[6] = {0, 0, 0, 0, 0, 0};
    bool have = false;
    for (int s = 1; s <= 4; ++s) {
        for (int r = 1; r <= 4; ++r) {
            if (quads % r || quads / r > kBatchMaxWaves || s * r > 8) continue;
            const int64_t waves = quads / r;
            const int64_t gx = (strips + s - 1) / s;
            const int64_t per_cu = (gx + kBatchCUs - 1) / kBatchCUs;
            const int64_t lds = waves * (1024 * s + 16 * kBatchSlotRow);
            const int64_t occ = std::min<int64_t>(kBatchLdsPerCU / lds,
                                                  4 * kBatchWavesPerSimd[s - 1][r - 1] / waves);
            const int64_t key[6] = {per_cu * act > kBatchActPerCU ? per_cu * act : 0, per_cu * s,
                                    per_cu > occ ? 1 : 0,
                                    act > kBatchActLongWaves ? -r : -std::min(per_cu, occ) * waves,
                                    -std::min(gx, kBatchCUs), r};
            bool better = !have;
            for (int i = 0; i < 6 && !better; ++i) {
                if (key[i] != bkey[i]) {
                    better = key[i] < bkey[i];
                    break;
                }
            }
            if (!better) continue;
            have = true;
            std::copy(key, key + 6, bkey);
            best.s = s;
            best.r = r;
            best.waves = (int)waves;
            best.gx = gx;
        }
    }
    if (!have || best.gx > 0x7fffffff) return false;
    *out = best;
    return true;
}

// ORT's int4 B [groups][N][K / 2] -> the strip-major copy
// [groups][ceil(N / 16)][ceil(K / 128)][16 columns][4 chunks] x 16 bytes that the batched and
// strip kernels read one 1 KB run per load instruction from; columns past N and chunks past K
// (a partial last quad) are zero.  One thread per 16-byte piece.
__global__ void __launch_bounds__(256)
strip_pack(const u32x4* __restrict__ B, u32x4* __restrict__ dst, int64_t N, int64_t K,
           int64_t pieces, int order) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const int64_t kq = (K + 127) / 128, ns = (N + 15) / 16, chunks = K / 32;
    const int g = (int)(i & 3), n = (int)((i >> 2) & 15);
    const int64_t q = (i >> 6) % kq, st = (i >> 6) / kq % ns, grp = (i >> 6) / kq / ns;
    const int64_t col = 16 * st + n;
    auto chunk = [&](int64_t c) {
        return col < N && c < chunks ? B[((grp * N + col) * (K / 2) + 16 * c) / 16]
                                     : u32x4{0u, 0u, 0u, 0u};
    };
    if (order == kStripPlain) {
        dst[i] = chunk(4 * q + g);
        return;
    }
    // MFMA order: dword c of the piece is dword g of chunk 4 q + c (what the ORT layout's 4 x 4
    // transpose across the quad's lanes yields); for the fp16 kernels its nibbles are also
    // reordered from k0..k7 to k0 k2 k4 k6 (bits 0-15) and k1 k3 k5 k7 (bits 16-31)
    u32x4 out;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 v = chunk(4 * q + c);
        const uint32_t d = g == 0 ? v.x : g == 1 ? v.y : g == 2 ? v.z : v.w;
        uint32_t r = d;
        if (order == kStripMfmaF16) {
            r = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                r |= ((d >> (4 * k)) & 0xFu) << ((k & 1) ? 16 + 4 * (k >> 1) : 4 * (k >> 1));
        }
        out[c] = r;
    }
    dst[i] = out;
}

int64_t strip_pack_bytes(int64_t n, int64_t k, int64_t groups) {
    return groups * ((n + 15) / 16) * ((k + 127) / 128) * 1024;
}

hipError_t launch_strip_pack(const uint8_t* b, uint8_t* dst, int64_t n, int64_t k,
                             hipStream_t st, int64_t groups, int order) {
    if (order != kStripPlain && order != kStripMfmaF16 && order != kStripMfmaI8) return hipErrorInvalidValue;
    if (n < 1 || k < 32 || k % 32 || groups < 1 || reinterpret_cast<uintptr_t>(b) % 16 ||
        reinterpret_cast<uintptr_t>(dst) % 16)
        return hipErrorInvalidValue;
    const int64_t pieces = strip_pack_bytes(n, k, groups) / 16;
    const int64_t blocks = (pieces + 255) / 256;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(strip_pack, dim3((unsigned)blocks), dim3(256), 0, st,
                       reinterpret_cast<const u32x4*>(b), reinterpret_cast<u32x4*>(dst), n, k,
                       pieces, order);
    return hipGetLastError();
}

bool batch_stream_aligned(const void* a, const uint8_t* b, const void* s, const uint8_t* z) {
    return reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(s) % 8 == 0 && reinterpret_cast<uintptr_t>(z) % 2 == 0;
}

hipError_t launch_batch_stream(const BatchStreamGeom& g, const void* a, const uint8_t* b,
                               const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                               int64_t k, int bs, hipStream_t st, const uint8_t* b_strips) {
    // waves * R == K / 128: every quad of K belongs to exactly one wavefront
    BatchStreamGeom want{};
    if (!batch_stream_geometry(m, n, k, bs, &want) || want.r != g.r || want.s != g.s ||
        want.waves != g.waves || want.gx != g.gx || !batch_stream_aligned(a, b, s, z) ||
        reinterpret_cast<uintptr_t>(b_strips) % 16)
        return hipErrorInvalidValue;
#define MNB_BS_ZP(BS_)                                                                            \
    return z ? batch_go<BS_, true>(g, a, b, s, z, y, m, n, k, st, b_strips)                       \
             : batch_go<BS_, false>(g, a, b, s, z, y, m, n, k, st, b_strips)
    switch (bs) {
        case 32: MNB_BS_ZP(32);
        case 64: MNB_BS_ZP(64);
        case 128: MNB_BS_ZP(128);
        default: return hipErrorInvalidValue;
    }
#undef MNB_BS_ZP
}

}  // namespace mnb
