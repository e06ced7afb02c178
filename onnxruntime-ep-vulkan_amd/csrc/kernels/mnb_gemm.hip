// Prefill MatMulNBits on gfx950: dequantise-into-LDS fp16 MFMA GEMM (fp16 A; 4- or 8-bit
// weights; blocks of 16, 32, 64 or 128).
//
// Work split.  One workgroup of 8 wavefronts owns a 256 x 128 tile of Y; the wavefronts form a
// 4 (M) x 2 (N) grid and each owns a 64 x 64 sub-tile of four 32 x 32 MFMA tiles.  K is walked in
// steps of 64 (two 32-k sub-blocks).  Workgroup ids are mapped to tiles XCD by XCD: the eight
// XCDs take consecutive workgroup ids in turn, so each XCD is given one contiguous run of tiles
// (for the prefill shapes: one 256-row band of A, which stays in that XCD's L2, against every
// column tile).
//
// Data movement.  Global -> LDS uses the gfx950 LDS DMA (global_load_lds_dwordx4 / _dword):
// no registers, no LDS write instructions.  Three A stages and three raw-B stages form a ring;
// step s + 2's A and step s + 3's raw B are requested while step s is multiplied, so every load
// has two steps to land.  Each step's raw B (128 columns x 32 or 64 bytes) and its per-column
// scale and zero-point dwords are turned once per workgroup into exact (q - zp) fp16 values and
// the step's block scales in an LDS buffer that all four row-wavefronts then read.  One barrier
// per step.
//
// LDS layouts (16-byte slots):
//   A stage  [256 rows][8 k-chunks], chunk kc of row r at slot 8r + (kc ^ swz(r)): one DMA
//            instruction covers 8 whole rows (8 full 128-byte lines of A), and a wavefront's
//            MFMA operand read (32 rows x one chunk, twice) touches every bank group once.
//   raw B    [128 cols][32 B (4-bit) or 64 B (8-bit)], then the scale dwords (1 per column, 2
//            for blocks of 16) and one zero-point dword per column.
//   (q - z)  [8 k-chunks][128 cols] fp16 (an operand read is 2 x 512 contiguous bytes), then
//            the step's block scales, 4 fp16 per column.
//
// Arithmetic.  Each 32 x 32 tile's partial over one quant block is accumulated by MFMAs over the
// exact (q - zp) operands in fp32 (fp16 a x integer q - zp is exact in fp32) -- the reference
// kernel's per-block fp32 partial (rust/shaders/glsl/templates/q_gemv.comp:571-579) -- and added
// to the tile's accumulator scaled by the block's scale.  The scaled add of one sub-block is
// spread between the MFMAs of the next, so that it runs on the VALU while the matrix core works.
// Blocks of 16 are one MFMA each; blocks of 64 or 128 scale the partial of each 64-k step on
// its own (the same scale twice for a 128 block).
#include <algorithm>
#include <type_traits>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

namespace {

constexpr int kWM = 4, kWN = 2;                  // wavefront grid
constexpr int kBM = 64 * kWM;                    // 256
constexpr int kBN = 64 * kWN;                    // 128
constexpr int kKS = 64;                          // K per step
constexpr int kNA = 3;                           // A stages
constexpr int kNR = 3;                           // raw-B stages
constexpr int kAStage = kBM * kKS * 2;           // 32 KB
constexpr int kFQ = kBN * kKS * 2;               // 16 KB of (q - z) fp16
constexpr int kFStage = kFQ + kBN * 4 * 2;       // + 4 fp16 block scales per column

// Per-form sizes: raw B bytes per stage, scale dwords per column and step, aux dwords per stage
// (scales then zero points, padded to the DMA count), DMAs per step by wavefronts 0-3 (raw B)
// and 4-7 (aux), LDS bytes.
template <int BITS, int BS>
struct GemmForm {
    static constexpr int kRawB = kBN * kKS * BITS / 8;          // 4 or 8 KB
    static constexpr int kSD = BS == 16 ? 2 : 1;
    static constexpr int kAuxUsed = kBN * (kSD + 1);            // 256 or 384 dwords
    static constexpr int kAuxDma = (kAuxUsed + 255) / 256;      // per thread of waves 4-7
    static constexpr int kAux = kAuxDma * 256;                  // dwords, DMA-padded
    static constexpr int kRStage = kRawB + 4 * kAux;
    static constexpr int kRawDma = BITS / 4;                    // per thread of waves 0-3
    static constexpr int kLds = kNA * kAStage + kNR * kRStage + 2 * kFStage;
    static_assert(kLds <= 160 * 1024, "LDS");
};

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)l, 4, 0, 0);
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4));
}

// Workgroup barrier without the release/acquire fence of __syncthreads (which would wait for
// every outstanding DMA); the waits that matter are explicit.
__device__ __forceinline__ void wg_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Two bytes of w (bytes I and I + 1) as the fp16 pair (1024 + b_I, 1024 + b_{I+1}).
template <int I>
__device__ __forceinline__ f16x2 byte_pair(uint32_t w) {
    constexpr uint32_t sel = (uint32_t)I | (0x0Cu << 8) | ((uint32_t)(I + 1) << 16) | (0x0Cu << 24);
    return as_h2(__builtin_amdgcn_perm(w, w, sel) | 0x64006400u);
}

}  // namespace

template <int BITS, int BS, bool HAS_ZP>
__global__ void __launch_bounds__(512)
gemm_f16_mfma(const f16* __restrict__ A, const uint8_t* __restrict__ B, const f16* __restrict__ S,
              const uint8_t* __restrict__ Z, f16* __restrict__ Y, int M, int N, int K,
              int tiles_m, int tiles_n, int ksplit, float* __restrict__ part) {
    static_assert(BITS == 4 || BITS == 8, "bits");
    static_assert(BS == 16 || BS == 32 || BS == 64 || BS == 128, "block size");
    using F = GemmForm<BITS, BS>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const sA = smem;
    uint8_t* const sR = smem + kNA * kAStage;
    uint8_t* const sF = sR + kNR * F::kRStage;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: LDS bases in SGPRs
    const int wm = wave >> 1;
    const int wn = wave & 1;

    // (tile, K split) items, each XCD taking a contiguous run of them
    const int V = tiles_m * tiles_n * ksplit;
    const int per_xcd = (V + 7) >> 3;
    const int item = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (item >= V) return;                           // whole workgroup: before any barrier
    const int tile = item / ksplit;
    const int split = item - tile * ksplit;
    const int tile_m = tile / tiles_n;
    const int tile_n = tile - tile_m * tiles_n;
    const int m0 = tile_m * kBM;
    const int n0 = tile_n * kBN;
    const int bpc = K / BS;
    const int zpb = BITS == 8 ? bpc : (bpc + 1) >> 1;   // zero-point bytes per column
    // this split's 64-k steps s0 .. s0 + steps - 1 (the host keeps every split non-empty); the
    // pipeline below counts steps from 0 and the loaders add s0
    const int per_split = (K / kKS + ksplit - 1) / ksplit;
    const int s0 = split * per_split;
    const int steps = min(K / kKS - s0, per_split);
    const int64_t col_bytes = (int64_t)K * BITS / 8;
    auto gcol = [&](int c) { const int g = n0 + c; return g < N ? g : N - 1; };

    // ---- DMA sources: A (4 instructions per wavefront).  Each address is a uniform base (the
    // step's k offset, in SGPRs) plus this lane's 32-bit byte offset, so a step's requests cost
    // no 64-bit vector adds (the host keeps A and B below 4 GiB). ----
    uint32_t a_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 32 * wave + 8 * j + (lane >> 3);
        const int kc = (lane & 7) ^ swz(row);
        int gm = m0 + row;
        gm = gm < M ? gm : M - 1;                    // clamped rows are never stored
        a_off[j] = (uint32_t)(((int64_t)gm * K + 8 * kc) * 2);
    }
    // raw B (wavefronts 0-3; instruction j of lane l: the 16-byte piece that lands at
    // 1 KB * (kRawDma * wave + j) + 16 l, i.e. column (that offset) / bytes-per-column) or the
    // scale and zero-point dwords (wavefronts 4-7)
    constexpr int kColStep = kKS * BITS / 8;         // raw bytes per column and step: 32 or 64
    uint32_t b_off[F::kRawDma];
#pragma unroll
    for (int j = 0; j < F::kRawDma; ++j) {
        const int off = 1024 * (F::kRawDma * (wave & 3) + j) + 16 * lane;
        b_off[j] = (uint32_t)((int64_t)gcol(off / kColStep) * col_bytes + off % kColStep);
    }

    auto issue_a = [&](int step, int st) {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(A) + (int64_t)(s0 + step) * kKS * 2;
        uint8_t* dst = sA + st * kAStage + wave * 4 * 1024;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(src + a_off[j], dst + j * 1024);
    };
    auto issue_r = [&](int step, int st) {
        uint8_t* base = sR + st * F::kRStage;
        if (wave < 4) {
            const uint8_t* src = B + (int64_t)(s0 + step) * kColStep;
#pragma unroll
            for (int j = 0; j < F::kRawDma; ++j)
                dma16(src + b_off[j], base + 1024 * (F::kRawDma * wave + j));
        } else {
            const int blk0 = ((s0 + step) * kKS) / BS;
#pragma unroll
            for (int j = 0; j < F::kAuxDma; ++j) {
                // aux dword a: scale dword a % kSD of column a / kSD, then zero-point dwords;
                // dwords past the used ones re-read the last zero-point dword (padding)
                const int a = min(256 * j + (tid - 256), F::kAuxUsed - 1);
                const void* src;
                if (HAS_ZP && a >= kBN * F::kSD) {
                    const int gc = gcol(a - kBN * F::kSD);
                    const int64_t zb = BITS == 8 ? (int64_t)gc * zpb + blk0
                                                 : (int64_t)gc * zpb + (blk0 >> 1);
                    src = Z + (zb & ~(int64_t)3);
                } else {
                    const int aa = min(a, kBN * F::kSD - 1);
                    const int gc = gcol(aa / F::kSD);
                    src = S + ((((int64_t)gc * bpc + blk0) & ~(int64_t)1) + 2 * (aa % F::kSD));
                }
                dma4(src, base + F::kRawB + 1024 * j + 4 * (tid - 256));
            }
        }
    };

    // ---- raw stage -> (q - z) fp16 and the step's block scales: thread t takes column
    // t%128, k 16*(t/128) .. +15 ----
    const int dq_col = tid & 127;
    const int dq_seg = tid >> 7;
    auto dequant = [&](int step, int rst, int fst) {
        const uint8_t* base = sR + rst * F::kRStage;
        const uint32_t* aux = reinterpret_cast<const uint32_t*>(base + F::kRawB);
        const int gk = (s0 + step) * kKS + 16 * dq_seg;          // first k of the 16
        const int blk = gk / BS;
        const int blk0 = ((s0 + step) * kKS) / BS;
        uint8_t* f = sF + fst * kFStage;
        if ((16 * dq_seg) % BS == 0) {
            // the first thread of each block in the step stores its scale (slot 16 seg / BS)
            uint32_t sw;
            int half;
            if constexpr (BS == 16) {
                sw = aux[dq_col * 2 + (dq_seg >> 1)];
                half = dq_seg & 1;
            } else {
                sw = aux[dq_col];
                half = (int)((((int64_t)gcol(dq_col) * bpc + blk0) & 1) + (blk - blk0));
            }
            reinterpret_cast<uint16_t*>(f + kFQ)[dq_col * 4 + blk - blk0] =
                (uint16_t)(half ? (sw >> 16) : (sw & 0xFFFFu));
        }
        int z = 1 << (BITS - 1);
        if constexpr (HAS_ZP) {
            const uint32_t zw = aux[kBN * F::kSD + dq_col];
            const int64_t zbase = (int64_t)gcol(dq_col) * zpb;
            if constexpr (BITS == 8) {
                const int byte = (int)((zbase + blk) & 3);
                z = (int)((zw >> (8 * byte)) & 0xFFu);
            } else {
                const int byte = (int)((zbase + (blk >> 1)) & 3);
                z = (int)((zw >> (8 * byte + 4 * (blk & 1))) & 0xFu);
            }
        }
        f16x8 v0, v1;
        if constexpr (BITS == 4) {
            const u32x2 w = *reinterpret_cast<const u32x2*>(base + dq_col * 32 + dq_seg * 8);
            const f16x2 zo = zoff4(z);
            v0.s01 = nib_pair<0>(w.x, zo);
            v0.s23 = nib_pair<1>(w.x, zo);
            v0.s45 = nib_pair<2>(w.x, zo);
            v0.s67 = nib_pair<3>(w.x, zo);
            v1.s01 = nib_pair<0>(w.y, zo);
            v1.s23 = nib_pair<1>(w.y, zo);
            v1.s45 = nib_pair<2>(w.y, zo);
            v1.s67 = nib_pair<3>(w.y, zo);
        } else {
            const u32x4 w = *reinterpret_cast<const u32x4*>(base + dq_col * 64 + dq_seg * 16);
            const f16 zf = (f16)(1024 + z);
            const f16x2 zo = {zf, zf};
            // (1024 + q) - (1024 + z) = q - z, exact
            v0.s01 = byte_pair<0>(w.x) - zo;
            v0.s23 = byte_pair<2>(w.x) - zo;
            v0.s45 = byte_pair<0>(w.y) - zo;
            v0.s67 = byte_pair<2>(w.y) - zo;
            v1.s01 = byte_pair<0>(w.z) - zo;
            v1.s23 = byte_pair<2>(w.z) - zo;
            v1.s45 = byte_pair<0>(w.w) - zo;
            v1.s67 = byte_pair<2>(w.w) - zo;
        }
        *reinterpret_cast<f16x8*>(f + ((2 * dq_seg) * 128 + dq_col) * 16) = v0;
        *reinterpret_cast<f16x8*>(f + ((2 * dq_seg + 1) * 128 + dq_col) * 16) = v1;
    };

    // tile t = 2 * j + i (i: 32-row half, j: 32-column half of the wavefront's sub-tile)
    f32x16 acc[4];
    f32x16 pd[4];          // per tile: running partial, or a finished one awaiting its scale
    float psc[2] = {0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        acc[t] = f32x16{};
        pd[t] = f32x16{};
    }
    auto retire = [&](int t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(pd[t][r], psc[t >> 1], acc[t][r]);
        asm volatile("" : "+v"(acc[t]));             // keep the adds here, beside the MFMAs
    };

    // Lane parts of the operand addresses, fixed for the whole loop, so that a step adds its
    // stage base once per address family and every read takes the rest as an immediate offset.
    // A: row r = 64 wm + 32 i + (lane & 31) holds chunk kc = 2 p + (lane >> 5) (p = 2 sub + h)
    // at slot kc ^ swz(r); swz depends on bits 0-3 of r only, i.e. on the lane, so the 32-row
    // half i is + 4096 bytes and p needs one offset each.  (q - z): chunk kc of column
    // c = 64 wn + 32 j + (lane & 31) at (128 kc + c) * 16 = p * 4096 + j * 512 + lane part.
    // Scales: 8 bytes per column after the (q - z) values, + 256 bytes per j.
    int a_lane[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
        const int r = wm * 64 + (lane & 31);
        a_lane[pp] = (r * 8 + ((2 * pp + (lane >> 5)) ^ swz(r))) * 16;
    }
    const int b_lane = ((lane >> 5) * 128 + wn * 64 + (lane & 31)) * 16;
    const int s_lane = kFQ + (wn * 64 + (lane & 31)) * 8;

    auto compute = [&](int ast, int fst, auto&& between) {
        const uint8_t* a_base = sA + ast * kAStage;
        const uint8_t* f_base = sF + fst * kFStage;
        f16x8 a[2][2][2], b[2][2][2];                // [sub][tile half][k half]
        auto load_sub = [&](int sub) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int pp = 2 * sub + h;
                const uint8_t* ap = a_base + a_lane[pp];
                const uint8_t* bp = f_base + b_lane;
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    a[sub][i][h] = *reinterpret_cast<const f16x8*>(ap + 4096 * i);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    b[sub][j][h] = *reinterpret_cast<const f16x8*>(bp + 4096 * pp + 512 * j);
            }
        };
        // the step's block scales of the wavefront's two 32-column halves, [j][slot]
        u32x2 sw[2];
        auto load_scales = [&]() {
            const uint8_t* sp = f_base + s_lane;
#pragma unroll
            for (int j = 0; j < 2; ++j) sw[j] = *reinterpret_cast<const u32x2*>(sp + 256 * j);
        };
        auto scale_of = [&](int j, int slot) {
            const uint32_t w = slot < 2 ? sw[j].x : sw[j].y;
            return (float)__builtin_bit_cast(f16, (uint16_t)((slot & 1) ? (w >> 16) : (w & 0xFFFFu)));
        };
        // Sub-block 0's operands first; sub-block 1's and the scales are requested behind the
        // first MFMAs, so no more than about 15 LDS reads are ever outstanding (the counter the
        // waits use) and the first MFMA waits only for its own operands.
        load_sub(0);
        __builtin_amdgcn_sched_barrier(0);
        auto after_first = [&](int sub, int t) {
            if (sub == 0 && t == 0) {
                load_sub(1);
                load_scales();
            }
        };
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            if (sub == 1) between();
            if constexpr (BS == 16) {
                // a block per MFMA: each partial is scaled once the next MFMAs are issued
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    f32x16 c[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        c[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][t & 1][h],
                                                                     b[sub][t >> 1][h], f32x16{},
                                                                     0, 0, 0);
                        if (h == 0) after_first(sub, t);
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const float scv = scale_of(t >> 1, 2 * sub + h);
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(c[t][r], scv, acc[t][r]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                continue;
            }
            // A block of 32 starts at every sub-block; blocks of 64 and 128 are scaled per step.
            const bool fresh = BS == 32 || sub == 0;
            if (fresh) {
                // each tile's finished partial is scaled into acc right before its registers
                // take the next partial's first MFMA
                retire(0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = t & 1, j = t >> 1;
                    f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][i][0], b[sub][j][0], f32x16{}, 0, 0, 0);
                    pd[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][i][1], b[sub][j][1], c, 0, 0, 0);
                    if (t < 3) retire(t + 1);
                    after_first(sub, t);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = t & 1, j = t >> 1;
                    f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][i][0], b[sub][j][0], pd[t], 0, 0, 0);
                    pd[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][i][1], b[sub][j][1], c, 0, 0, 0);
                }
            }
            if (BS == 32 || sub == 1) {              // the partial is complete: keep its scales
                psc[0] = scale_of(0, BS == 32 ? sub : 0);
                psc[1] = scale_of(1, BS == 32 ? sub : 0);
                asm volatile("" : "+v"(psc[0]), "+v"(psc[1]));
            }
        }
    };

    // DMAs per step of this wavefront (counted in issue order by vmcnt)
    constexpr int kDmaLo = 4 + F::kRawDma, kDmaHi = 4 + F::kAuxDma;
    auto wait_steps = [&](auto two) {                // two: 0, 1 or 2 steps may stay in flight
        constexpr int n = decltype(two)::value;
        if (wave < 4) wait_vm_lgkm0<n * kDmaLo>(); else wait_vm_lgkm0<n * kDmaHi>();
    };
    using Zero = std::integral_constant<int, 0>;
    using One = std::integral_constant<int, 1>;
    using Two = std::integral_constant<int, 2>;

    // ---- prologue: raw(0) | A(0) raw(1) | A(1) raw(2) ----
    issue_r(0, 0);
    issue_a(0, 0);
    if (steps > 1) { issue_r(1, 1); issue_a(1, 1); }
    if (steps > 2) issue_r(2, 2);
    if (steps > 2) wait_steps(Two{}); else wait_steps(Zero{});
    wg_barrier();
    dequant(0, 0, 0);

    for (int s = 0; s < steps; ++s) {
        // A(s) and raw(s+1) were requested two steps ago; the previous step's requests may
        // still be in flight (all requests are counted in issue order)
        if (s + 2 < steps) wait_steps(One{}); else wait_steps(Zero{});
        wg_barrier();
        if (s + 2 < steps) issue_a(s + 2, (s + 2) % kNA);
        // raw stage (s + 3) % 3 = s % 3: its dequantisation (for step s) finished before the
        // barrier above
        if (s + 3 < steps) issue_r(s + 3, (s + 3) % kNR);
        compute(s % kNA, s & 1, [&]() {
            if (s + 1 < steps) dequant(s + 1, (s + 1) % kNR, (s + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
        });
    }

    if constexpr (BS != 16) {
#pragma unroll
        for (int t = 0; t < 4; ++t) retire(t);
    }

    // ---- store: lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4 of each tile; a K
    // split stores its fp32 partial tile instead, summed by gemm_splitk_sum ----
    float* const pbase = part ? part + (int64_t)split * M * N : nullptr;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int i = t & 1, j = t >> 1;
        const int col = n0 + wn * 64 + 32 * j + (lane & 31);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row >= M) continue;
            if (pbase)
                pbase[(int64_t)row * N + col] = acc[t][r];
            else
                Y[(int64_t)row * N + col] = (f16)acc[t][r];
        }
    }
}

// Y = the sum of the ksplit fp32 partials, in split order (run-to-run deterministic); four
// consecutive outputs per thread (M * N % 4 == 0, Y 8-byte aligned).
__global__ void __launch_bounds__(256)
gemm_splitk_sum(const float* __restrict__ part, f16* __restrict__ Y, int64_t mn, int ksplit) {
    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
    for (int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x); i < mn;
         i += 4 * (int64_t)gridDim.x * 256) {
        f32x4 v = *reinterpret_cast<const f32x4*>(part + i);
        for (int sp = 1; sp < ksplit; ++sp) v += *reinterpret_cast<const f32x4*>(part + sp * mn + i);
        f16x4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = (f16)v[q];
        *reinterpret_cast<f16x4_t*>(Y + i) = o;
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

hipError_t launch_splitk_sum(const float* part, void* y, int64_t mn, int ksplit, hipStream_t st) {
    const unsigned blocks = (unsigned)std::min<int64_t>((mn / 4 + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_sum, dim3(blocks), dim3(256), 0, st, part,
                       static_cast<f16*>(y), mn, ksplit);
    return hipGetLastError();
}

bool gemm_supported(int64_t m, int64_t n, int64_t k, int bits, int bs, bool has_zp) {
    if (m <= 0 || n <= 0 || (bits != 4 && bits != 8) || k <= 0 || k % kKS) return false;
    if (bs != 16 && bs != 32 && bs != 64 && bs != 128) return false;
    if (k % bs) return false;
    const int64_t bpc = k / bs;
    // The scale and zero-point dwords of the last column must not reach past the arrays.
    if (bs > 32 && (n * bpc) % 2) return false;
    const int64_t zpb = bits == 8 ? bpc : (bpc + 1) / 2;
    if (has_zp && (n * zpb) % 4) return false;
    // The DMA sources are a uniform base plus a 32-bit byte offset per lane.
    if (m * k * 2 >= (int64_t)1 << 32 || n * k * bits / 8 >= (int64_t)1 << 32) return false;
    return true;
}

GemmConfig gemm_config(int64_t m, int64_t n, int64_t k) {
    GemmConfig c{};
    c.bm = kBM;
    c.bn = kBN;
    c.tiles_m = (m + kBM - 1) / kBM;
    c.tiles_n = (n + kBN - 1) / kBN;
    // Fewer tiles than the 256 CUs (M = 256: 64 tiles of 8192 columns): split K over up to four
    // workgroups per tile, each split at least eight 64-k steps and none empty.
    const int64_t tiles = c.tiles_m * c.tiles_n;
    const int64_t steps = k / kKS;
    int ks = 1;
    if (tiles < 256 && (m * n) % 4 == 0)
        ks = (int)std::max<int64_t>(1, std::min<int64_t>({4, 256 / tiles, steps / 8}));
    while (ks > 1 && ((steps + ks - 1) / ks) * (ks - 1) >= steps) --ks;
    c.ksplit = ks;
    return c;
}

size_t gemm_workspace_bytes(const GemmConfig& c, int64_t m, int64_t n) {
    return c.ksplit > 1 ? (size_t)c.ksplit * (size_t)m * (size_t)n * sizeof(float) : 0;
}

template <int BITS, int BS, bool HAS_ZP>
static hipError_t gemm_go(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                          const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                          float* part, hipStream_t st) {
    auto kern = gemm_f16_mfma<BITS, BS, HAS_ZP>;
    constexpr int lds = GemmForm<BITS, BS>::kLds;
    // More than 64 KB of dynamic LDS must be allowed explicitly (for the current device).
    const hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
    if (e != hipSuccess) return e;
    const int ks = part ? c.ksplit : 1;
    const int64_t items = c.tiles_m * c.tiles_n * ks;
    const dim3 grid((unsigned)(8 * ((items + 7) / 8)), 1, 1);
    hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, static_cast<const f16*>(a), b,
                       static_cast<const f16*>(s), z, static_cast<f16*>(y), (int)m, (int)n,
                       (int)k, (int)c.tiles_m, (int)c.tiles_n, ks, ks > 1 ? part : nullptr);
    if (ks > 1) return launch_splitk_sum(part, y, m * n, ks, st);
    return hipGetLastError();
}

template <int BITS, int BS>
static hipError_t gemm_zp(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                          const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k,
                          float* part, hipStream_t st) {
    if (z) return gemm_go<BITS, BS, true>(c, a, b, s, z, y, m, n, k, part, st);
    return gemm_go<BITS, BS, false>(c, a, b, s, z, y, m, n, k, part, st);
}

template <int BITS>
static hipError_t gemm_bs(int bs, const GemmConfig& c, const void* a, const uint8_t* b,
                          const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                          int64_t k, float* part, hipStream_t st) {
    switch (bs) {
        case 16: return gemm_zp<BITS, 16>(c, a, b, s, z, y, m, n, k, part, st);
        case 32: return gemm_zp<BITS, 32>(c, a, b, s, z, y, m, n, k, part, st);
        case 64: return gemm_zp<BITS, 64>(c, a, b, s, z, y, m, n, k, part, st);
        case 128: return gemm_zp<BITS, 128>(c, a, b, s, z, y, m, n, k, part, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_cfg(const GemmConfig& c, const void* a, const uint8_t* b, const void* s,
                           const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bits,
                           int bs, hipStream_t st, void* workspace, size_t workspace_bytes) {
    if (m == 0) return hipSuccess;
    if (!gemm_supported(m, n, k, bits, bs, z != nullptr)) return hipErrorInvalidValue;
    if (c.bm != kBM || c.bn != kBN || c.ksplit < 1) return hipErrorInvalidValue;
    // the K split needs the partial buffer and 8-byte aligned output; without them, one pass
    const size_t need = gemm_workspace_bytes(c, m, n);
    float* part = need && workspace && workspace_bytes >= need &&
                          reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                          reinterpret_cast<uintptr_t>(y) % 8 == 0
                      ? static_cast<float*>(workspace)
                      : nullptr;
    return bits == 8 ? gemm_bs<8>(bs, c, a, b, s, z, y, m, n, k, part, st)
                     : gemm_bs<4>(bs, c, a, b, s, z, y, m, n, k, part, st);
}

hipError_t launch_gemm(const void* a, const uint8_t* b, const void* s, const uint8_t* z, void* y,
                       int64_t m, int64_t n, int64_t k, int bits, int bs, hipStream_t st,
                       void* workspace, size_t workspace_bytes) {
    return launch_gemm_cfg(gemm_config(m, n, k), a, b, s, z, y, m, n, k, bits, bs, st, workspace,
                           workspace_bytes);
}

}  // namespace mnb
