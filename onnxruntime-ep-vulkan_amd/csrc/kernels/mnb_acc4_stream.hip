// accuracy_level = 4 at up to 16 rows (batched decode): int8 activations x int4 weights on
// gfx950 MFMA, one 16-column strip per workgroup over the whole of K.
//
// The launch follows the quantiser (quantize_a_int8: the activations' int8 codes in the strip
// layout -- within every 128-k quad a lane row's chunks 0,1 and 2,3 are two 16-byte pieces --
// and their fp32 scales block-major over 16 rows).  A workgroup of KW wavefronts owns one strip
// of 16 columns; wavefront w owns quads [w R, w R + R) of K (KW R = K / 128):
//   * every wavefront first requests its own quads' codes of the 16 rows (2R 16-byte pieces
//     per lane) and their activation scales; one barrier that waits for no load puts all of
//     these requests ahead of any weight request in the CU (whose vector memory returns data in
//     request order); then the wavefront's block scales and zero points, then its R quads of
//     weights (lane (n, g): 16 bytes of column n, chunk 4q + g, streamed past the caches);
//   * each wavefront stages its own codes in LDS (rows padded by 16 bytes: the 16 rows' reads
//     start in distinct bank groups; no workgroup barrier, no other wavefront reads them) and
//     computes quad by quad as its weights arrive: a 4 x 4 dword transpose across the lane
//     rows gives the B operands, weights become exact int8 (q - zp), v_mfma_i32_16x16x64_i8
//     (16x16x32 for block 32) gives exact int32 block dots, scaled by a_scale * b_scale in fp32;
//   * the KW partial tiles are added in LDS in wavefront order (run-to-run deterministic) and
//     stored as fp16.
// Nothing crosses workgroups: no counters and no partial tiles in memory.  Each workgroup reads
// the codes of all of K (16 K bytes, from L2) -- the price of having no cross-workgroup
// reduction, which measured slower on gfx950 (splitting K over 4..16 workgroups per strip adds
// two serialised device-scope round trips, the counter and the partials, at the kernel's end).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

// Wavefronts per workgroup the kernel is compiled for: 8 at R = 8 quads per wavefront (K = 8192;
// its 2R code pieces and R weight chunks per lane need more than the 128 VGPRs of 16 wavefronts),
// 16 below.
constexpr int acc4s_max_waves(int r) { return r == 8 ? 8 : 16; }
constexpr size_t kAcc4sMaxLds = 160 * 1024;

// MFMA: Bs is the strip copy in the int8 MFMA order (launch_strip_pack kStripMfmaI8: each lane's
// 16 bytes are its operand dwords of the quad's four chunks, no lane transpose).
template <int BS, bool HAS_ZP, int R, bool MFMA>
__global__ void __launch_bounds__(64 * acc4s_max_waves(R))
acc4_stream(const int8_t* __restrict__ qa, const float* __restrict__ a_scale,
            const uint8_t* __restrict__ B, const f16* __restrict__ Sc,
            const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K,
            const uint8_t* __restrict__ Bs) {
    constexpr int CPB = BS / 32;                         // 32-k chunks per block: 1, 2 or 4
    constexpr int BPQ = 4 / CPB;                         // blocks per quad
    constexpr int PA = 2 * R;                            // 16-byte code pieces per thread
    constexpr int PS = (R * BPQ + 3) / 4;                // activation scales per thread
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int kw = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int KW = blockDim.x >> 6;
    const int nl = lane & 15;
    const int g = lane >> 4;
    const int quads = K >> 7;                            // = KW * R
    const int bpc = K / BS;                              // a multiple of 4
    const int zpb = bpc >> 1;
    const int strip = blockIdx.x;
    const int q0 = kw * R;                               // this wavefront's first quad
    const int RB = 128 * quads + 16;                     // LDS row stride of the codes
    uint8_t* const sA = smem;
    float* const sSa = reinterpret_cast<float*>(smem + 16 * RB);          // [bpc][16] + 4
    f32x4* const sRed = reinterpret_cast<f32x4*>(smem + 16 * RB + bpc * 64 + 16);

    // ---- 1. this wavefront's own codes and activation scales -------------------------------
    // The wavefront's quads of the 16 rows are 16 x 8R pieces: one load instruction covers 8 / R
    // whole rows of them (8R lanes per row), 2R instructions all 16 rows; rows past M repeat row
    // M - 1 (never stored).  Its activation scales are one contiguous run of 16 R BPQ floats.
    constexpr int LPR = 8 * R;
    constexpr int RPI = 8 / R;
    constexpr int NSA = 16 * R * BPQ;
    constexpr int PSW = (NSA + 63) / 64;
    const int prow = lane / LPR;
    const int ppc = lane % LPR;
    u32x4 va[PA];
#pragma unroll
    for (int i = 0; i < PA; ++i) {
        const int row = min(i * RPI + prow, M - 1);
        va[i] = *reinterpret_cast<const u32x4*>(qa + (int64_t)row * K + 128 * q0 + 16 * ppc);
    }
    const int nsc = bpc * 16;
    const int sbase = 16 * q0 * BPQ;
    float vs[PSW];
#pragma unroll
    for (int i = 0; i < PSW; ++i) vs[i] = a_scale[sbase + min(lane + 64 * i, NSA - 1)];
    // every wavefront's activation requests go out before any wavefront's weight requests (the
    // CU's vector memory returns data in request order, so codes requested behind another
    // wavefront's weights would wait for those); the barrier waits for no load
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. the wavefront's block scales and zero points (contiguous per column) -----------
    const int col = min(16 * strip + nl, N - 1);
    constexpr int NS = R * BPQ;                          // blocks of the wavefront's quads
    constexpr int NZ = (NS + 1) / 2;
    const int b0 = q0 * BPQ;                             // first block; even unless NS == 1
    uint16_t sv[NS];
    uint8_t zv[NZ];
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(Sc) + (int64_t)col * bpc + b0;
    const uint8_t* zp = Z + (int64_t)col * zpb + (b0 >> 1);
    if constexpr (NS % 4 == 0) {
        // 8-byte and 2-byte aligned: bpc % 4 == 0, b0 % 4 == 0, the launcher checks the bases
#pragma unroll
        for (int i = 0; i < NS / 4; ++i) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(sp + 4 * i);
            sv[4 * i] = (uint16_t)v.x;
            sv[4 * i + 1] = (uint16_t)(v.x >> 16);
            sv[4 * i + 2] = (uint16_t)v.y;
            sv[4 * i + 3] = (uint16_t)(v.y >> 16);
        }
        if constexpr (HAS_ZP) {
#pragma unroll
            for (int i = 0; i < NZ / 2; ++i) {
                const uint16_t v = *reinterpret_cast<const uint16_t*>(zp + 2 * i);
                zv[2 * i] = (uint8_t)v;
                zv[2 * i + 1] = (uint8_t)(v >> 8);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < NS; ++i) sv[i] = sp[i];
        if constexpr (HAS_ZP) {
#pragma unroll
            for (int i = 0; i < NZ; ++i) zv[i] = zp[i];
        }
    }

    // ---- 3. the wavefront's weights: lane (n, g) takes chunk 4 q + g of column n, from ORT's
    // layout or from the strip-major copy (one 1 KB run per strip and quad, launch_strip_pack) -
    const uint8_t* const bc = Bs ? Bs + (int64_t)strip * (K / 128) * 1024 + 64 * nl + 16 * g
                                 : B + (int64_t)col * (K / 2) + 16 * g;
    u32x4 bw[R];
#pragma unroll
    for (int j = 0; j < R; ++j)
        bw[j] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(bc + (Bs ? 1024 : 64) * (int64_t)(q0 + j)));

    // all of the loads above are issued before the staging below waits for the first of them
    __builtin_amdgcn_sched_barrier(0);

    // ---- 4. stage the wavefront's own codes and scales: no other wavefront reads them, and a
    // wavefront's LDS accesses complete in program order, so no workgroup barrier ------------
#pragma unroll
    for (int i = 0; i < PA; ++i)
        *reinterpret_cast<u32x4*>(sA + (i * RPI + prow) * RB + 128 * q0 + 16 * ppc) = va[i];
#pragma unroll
    for (int i = 0; i < PSW; ++i) {
        const int u = lane + 64 * i;
        sSa[u < NSA ? sbase + u : nsc + (u & 3)] = vs[i];    // a dummy slot past the end
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- 5. the strip's partial tile over this wavefront's quads -----------------------------
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const uint8_t* ar = sA + nl * RB + 128 * (q0 + j) + 16 * g;
        const u32x4 a01 = *reinterpret_cast<const u32x4*>(ar);        // chunks 0, 1 of row nl
        const u32x4 a23 = *reinterpret_cast<const u32x4*>(ar + 64);   // chunks 2, 3
        const i32x2 aq[4] = {i32x2{(int32_t)a01.x, (int32_t)a01.y}, i32x2{(int32_t)a01.z, (int32_t)a01.w},
                             i32x2{(int32_t)a23.x, (int32_t)a23.y}, i32x2{(int32_t)a23.z, (int32_t)a23.w}};
        uint32_t v0 = bw[j].x, v1 = bw[j].y, v2 = bw[j].z, v3 = bw[j].w;
        if constexpr (!MFMA) transpose_rows(v0, v1, v2, v3);
        const uint32_t wt[4] = {v0, v1, v2, v3};
        i32x2 bq[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int bi = j * BPQ + c / CPB;            // block within the wavefront's range
            int z = 8;
            if constexpr (HAS_ZP)
                z = (int)((zv[(bi + (b0 & 1)) >> 1] >> (((b0 + bi) & 1) * 4)) & 0xFu);
            bq[c] = qz_i8(wt[c], (uint32_t)(128 - z) * 0x01010101u);
        }
        i32x4 dot = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; c += (CPB >= 2 ? 2 : 1)) {
            if constexpr (CPB >= 2) {
                // two chunks of one block in one 16x16x64 MFMA: A and B place the same k in the
                // same (lane row, slot)
                const i32x4 a4 = {aq[c].x, aq[c].y, aq[c + 1].x, aq[c + 1].y};
                const i32x4 b4 = {bq[c].x, bq[c].y, bq[c + 1].x, bq[c + 1].y};
                dot = __builtin_amdgcn_mfma_i32_16x16x64_i8(a4, b4, dot, 0, 0, 0);
            } else {
                dot = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, aq[c]),
                                                            __builtin_bit_cast(long, bq[c]), dot,
                                                            0, 0, 0);
            }
            const int ce = c + (CPB >= 2 ? 1 : 0);       // last chunk covered so far
            if ((ce + 1) % CPB == 0) {                   // block end: scale it
                const int b = ce / CPB;
                const float sb = (float)__builtin_bit_cast(f16, sv[j * BPQ + b]);
                const f32x4 sa =
                    *reinterpret_cast<const f32x4*>(sSa + ((q0 + j) * BPQ + b) * 16 + 4 * g);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf((float)dot[q], sa[q] * sb, acc[q]);
                dot = i32x4{0, 0, 0, 0};
            }
        }
    }

    // ---- 6. the KW partial tiles added in wavefront order (run-to-run deterministic): every
    // wavefront stores its tile, then each thread sums its outputs over them ------------------
    sRed[kw * 64 + lane] = acc;
    __syncthreads();
    const float* const red = reinterpret_cast<const float*>(sRed);
    for (int o = threadIdx.x; o < 256; o += blockDim.x) {
        // output o: row orow, column on (fastest, so consecutive threads store along a row);
        // lane (on + 16 (orow / 4)) of every wavefront holds it in element orow % 4
        const int on = o & 15, orow = o >> 4;
        const int src = (((orow >> 2) * 16 + on) << 2) + (orow & 3);
        float v = red[src];
        for (int w = 1; w < KW; ++w) v += red[w * 256 + src];
        const int cc = 16 * strip + on;
        if (cc < N && orow < M) Y[(int64_t)orow * N + cc] = (f16)v;
    }
}

template <int BS, bool HAS_ZP>
hipError_t acc4s_go(const Acc4StreamGeom& g, const int8_t* qa, const float* sa, const uint8_t* b,
                    const void* s, const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                    hipStream_t st, const uint8_t* bs_) {
    const dim3 grid((unsigned)g.gx, 1, 1);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
#define MNB_A4S(R_)                                                                               \
    do {                                                                                          \
        auto kern = bs_ ? acc4_stream<BS, HAS_ZP, R_, true> : acc4_stream<BS, HAS_ZP, R_, false>;\
        const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), g.lds);     \
        if (ea != hipSuccess) return ea;                                                          \
        hipLaunchKernelGGL(kern, grid, block, g.lds, st, qa, sa, b, static_cast<const f16*>(s),   \
                           z, static_cast<f16*>(y), (int)m, (int)n, (int)k, bs_);                 \
    } while (0)
    switch (g.r) {
        case 1: MNB_A4S(1); break;
        case 2: MNB_A4S(2); break;
        case 4: MNB_A4S(4); break;
        case 8: MNB_A4S(8); break;
        default: return hipErrorInvalidValue;
    }
#undef MNB_A4S
    return hipGetLastError();
}

}  // namespace

bool acc4_stream_geometry(int64_t m, int64_t n, int64_t k, int bs, Acc4StreamGeom* out) {
    if (m < 1 || m > 16 || n < 1 || k < 128 || k % 128 || (bs != 32 && bs != 64 && bs != 128))
        return false;
    if ((k / bs) % 4) return false;                      // whole 4-block groups of scales
    const int64_t quads = k / 128;
    Acc4StreamGeom g{};
    // R quads per wavefront: the largest of 8, 4, 2, 1 that divides K into at least 8
    // wavefronts (into all of its quads when there are fewer than 8), at most 16 wavefronts (8
    // at R = 8: K = 9216 with block 128 now goes to the strip GEMV).
    g.r = 0;
    for (int r : {8, 4, 2, 1}) {
        if (quads % r == 0 && (quads / r >= 8 || r == 1) && quads / r <= acc4s_max_waves(r)) {
            g.r = r;
            break;
        }
    }
    if (g.r == 0) return false;
    g.waves = (int)(quads / g.r);
    g.gx = (n + 15) / 16;
    g.lds = (size_t)16 * (size_t)(128 * quads + 16) + (size_t)(k / bs) * 64 + 16 +
            (size_t)g.waves * 64 * sizeof(f32x4);
    if (g.lds > kAcc4sMaxLds || g.gx > 0x7fffffff) return false;
    *out = g;
    return true;
}

bool acc4_stream_planned(bool a_f16, int64_t m, int64_t n, int64_t k, int bs,
                         Acc4StreamGeom* out) {
    const char* v = std::getenv("MNB_FORCE_KERNEL");
    if (v && (!std::strcmp(v, "strip") || !std::strcmp(v, "group"))) return false;
    return a_f16 && acc4_stream_geometry(m, n, k, bs, out);
}

bool acc4_stream_aligned(const void* qa, const uint8_t* b, const void* s, const uint8_t* z) {
    return reinterpret_cast<uintptr_t>(qa) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(s) % 8 == 0 && reinterpret_cast<uintptr_t>(z) % 2 == 0;
}

hipError_t launch_acc4_stream(const Acc4StreamGeom& g, const int8_t* qa, const float* sa,
                              const uint8_t* b, const void* s, const uint8_t* z, void* y,
                              int64_t m, int64_t n, int64_t k, int bs, hipStream_t st,
                              const uint8_t* b_strips) {
    // the staging covers 16 rows x K exactly with 2R pieces per thread: waves * R == K / 128
    Acc4StreamGeom want{};
    if (!acc4_stream_geometry(m, n, k, bs, &want) || want.r != g.r || want.waves != g.waves ||
        want.gx != g.gx || want.lds != g.lds || !acc4_stream_aligned(qa, b, s, z) ||
        reinterpret_cast<uintptr_t>(b_strips) % 16)
        return hipErrorInvalidValue;
#define MNB_A4S_ZP(BS_)                                                                           \
    return z ? acc4s_go<BS_, true>(g, qa, sa, b, s, z, y, m, n, k, st, b_strips)                 \
             : acc4s_go<BS_, false>(g, qa, sa, b, s, z, y, m, n, k, st, b_strips)
    switch (bs) {
        case 32: MNB_A4S_ZP(32);
        case 64: MNB_A4S_ZP(64);
        case 128: MNB_A4S_ZP(128);
        default: return hipErrorInvalidValue;
    }
#undef MNB_A4S_ZP
}

}  // namespace mnb
