// Row-tiled MFMA GEMV for MatMulNBits on gfx950 (int4 weights, block_size >= 32), in two
// arithmetic flavours, both optionally grouped by expert:
//
//   group_gemv_f16   fp16 activations; (q - zp) as exact fp16 on v_mfma_f32_16x16x32_f16, each
//                    32-k partial scaled by its block's scale in fp32 (the reference kernel's
//                    per-block fp32 partial, rust/shaders/glsl/templates/q_gemv.comp:571-579).
//   group_gemv_i8    accuracy_level = 4: activations quantised to int8 per (row, block) by
//                    quantize_a_int8 below; (q - zp) as int8 on v_mfma_i32_16x16x32_i8, exact
//                    int32 block dots, scaled by a_scale * b_scale in fp32.  ORT's CPU EP runs
//                    this level as SQNBIT_CompInt8 (third-party ONNX Runtime; the reference
//                    declines the level, rust/src/ops/quant.rs:191-200): the quantiser here is
//                    this build's declared definition (symmetric, amax / 127, round half even).
//
// Loads.  A wavefront owns 16 columns; lane (n = l%16, g = l/16) reads 16 contiguous bytes of
// column n per iteration -- 32-k chunk 4c+g -- so each load instruction covers 16 runs of 64
// bytes.  A 4 x 4 dword transpose across the four lane rows (v_permlane32_swap then
// v_permlane16_swap) turns that into MFMA operands: afterwards lane (n, g) holds dword g of
// chunks 4c..4c+3, i.e. for chunk t the eight k = 32t + 8g .. +8 that MFMA lane (n, g) supplies,
// so every MFMA covers one chunk of one block.
//
// Grouping.  For the expert-grouped (MoE) form, blockIdx.y is the expert: its rows are
// offsets[e] .. offsets[e+1] of Y, gathered from A through row_index, and its weights are the
// e-th of `experts` consecutive per-expert B / scales / zero_points tensors.  The dense form is
// one group with rows 0 .. M-1.  The W wavefronts of a workgroup split the K iterations and are
// summed in a fixed order through LDS, so results are run-to-run deterministic.
#include <algorithm>
#include <type_traits>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));


// T: activation / scale / output type (f16, or float for the int8 path's fp32 nodes).
// I8: false = fp16 activations (A is f16 [a_rows][K]); true = int8 activations (A is the
// quantiser's qa [a_rows][K] in permuted order, a_scale fp32 [a_rows][K/BS]).
template <typename T, bool I8, int BS, bool HAS_ZP, int MT>
__global__ void __launch_bounds__(kGroupMaxThreads)
group_gemv(const void* __restrict__ Av, const float* __restrict__ a_scale,
           const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
           const uint8_t* __restrict__ B, const T* __restrict__ S, const uint8_t* __restrict__ Z,
           T* __restrict__ Y, int M, int N, int K, int ksplit, int runs_per_split,
           f32x4* __restrict__ part, int* __restrict__ cnt) {
    extern __shared__ f32x4 red[];                       // [W][MT][64]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    const int nl = lane & 15;
    const int g = lane >> 4;
    // blockIdx.x = strip * ksplit + split: the split's workgroups share the strip's K range.
    const int strip = blockIdx.x / ksplit;
    const int split = blockIdx.x - strip * ksplit;
    const int n0 = strip * 16;
    const int col = min(n0 + nl, N - 1);
    const int bpc = K / BS;
    const int zpb = (bpc * 4 + 7) / 8;
    const int chunks = K / 32;                           // 32-k chunks per column
    const int iters = (chunks + 3) / 4;                  // 128-k iterations

    // Rows of this workgroup: group e, row tile blockIdx.z.
    int row_lo = 0, row_hi = M;
    int64_t wofs_b = 0, wofs_s = 0, wofs_z = 0;
    if (offsets) {
        const int e = blockIdx.y;
        row_lo = offsets[e];
        row_hi = offsets[e + 1];
        wofs_b = (int64_t)e * N * (K / 2);
        wofs_s = (int64_t)e * N * bpc;
        wofs_z = (int64_t)e * N * zpb;
    }
    const int r0 = row_lo + blockIdx.z * 16 * MT;
    if (r0 >= row_hi) return;                            // whole workgroup leaves: no barrier yet
    const uint8_t* __restrict__ bcol = B + wofs_b + (int64_t)col * (K / 2) + 16 * g;

    // A row of each 16-row tile this lane feeds (MFMA A operand: row l%16).
    int arow[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        int r = r0 + 16 * i + nl;
        r = r < row_hi ? r : row_hi - 1;
        arow[i] = row_index ? row_index[r] : r;
    }

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int PF = group_pf(I8, BS, MT);
    constexpr int CPB = BS / 32;                         // 32-k chunks per block (1, 2 or 4)
    const int c_lo = split * runs_per_split * PF;
    const int c_hi = min(iters, c_lo + runs_per_split * PF);

    // The strip's scales and zero points over this workgroup's K range are staged in LDS with
    // coalesced loads once: per 32-k chunk each lane then reads them from LDS instead of
    // issuing scattered 1- and 2-byte global loads (which would dominate the kernel).
    const int b_lo = (128 * c_lo) / BS;
    const int b_hi = (32 * min(4 * c_hi, chunks)) / BS;  // K % BS == 0: exact
    const int nblk = b_hi - b_lo;
    const int spitch = (nblk + 3) & ~3;
    const int z_lo = b_lo >> 1;
    const int nz = ((b_hi - 1) >> 1) - z_lo + 1;
    const int zpitch = (nz + 3) & ~3;
    T* const sS = reinterpret_cast<T*>(red + W * MT * 64);
    uint8_t* const sZ = reinterpret_cast<uint8_t*>(sS + 16 * spitch);
    // Staging loads are issued eight at a time before any of them is stored, so a wavefront
    // waits for one memory round trip per batch rather than one per element (with one
    // wavefront per workgroup a strip stages ~20 elements per lane).
    auto stage = [&](int total, auto&& load, auto&& store) {
        constexpr int kB = 8;
        for (int base = (int)threadIdx.x; base < total; base += kB * (int)blockDim.x) {
            decltype(load(0)) v[kB];
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const int idx = base + b * (int)blockDim.x;
                v[b] = load(idx < total ? idx : total - 1);
            }
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const int idx = base + b * (int)blockDim.x;
                if (idx < total) store(idx, v[b]);
            }
        }
    };
    stage(16 * nblk,
          [&](int idx) {
              const int n = idx / nblk;
              const int j = idx - n * nblk;
              const int cc = min(n0 + n, N - 1);
              return S[wofs_s + (int64_t)cc * bpc + b_lo + j];
          },
          [&](int idx, T v) {
              const int n = idx / nblk;
              sS[n * spitch + (idx - n * nblk)] = v;
          });
    if constexpr (HAS_ZP) {
        stage(16 * nz,
              [&](int idx) {
                  const int n = idx / nz;
                  const int j = idx - n * nz;
                  const int cc = min(n0 + n, N - 1);
                  return Z[wofs_z + (int64_t)cc * zpb + z_lo + j];
              },
              [&](int idx, uint8_t v) {
                  const int n = idx / nz;
                  sZ[n * zpitch + (idx - n * nz)] = v;
              });
    }
    // int8 path: the tile rows' activation scales over the same blocks, [block][16 * MT rows],
    // so a lane's four output rows are one 16-byte LDS read.
    float* const sA = reinterpret_cast<float*>(sZ + (HAS_ZP ? 16 * zpitch : 0));
    if constexpr (I8) {
        stage(16 * MT * nblk,
              [&](int idx) {
                  const int b = idx / (16 * MT);
                  const int rr = idx - b * (16 * MT);
                  int r = r0 + rr;
                  r = r < row_hi ? r : row_hi - 1;
                  const int ar = row_index ? row_index[r] : r;
                  return a_scale[(int64_t)ar * bpc + b_lo + b];
              },
              [&](int idx, float v) { sA[idx] = v; });
    }
    __syncthreads();
    const T* __restrict__ lS = sS + nl * spitch;
    const uint8_t* __restrict__ lZ = sZ + nl * zpitch;

    // Each wavefront takes runs of PF consecutive 128-k iterations: all weight loads of a run
    // are issued before any of it is computed.  Out-of-range chunks load a clamped in-bounds
    // address and are dropped by a zero scale at compute time.
    for (int c0 = c_lo + wave * PF; c0 < c_hi; c0 += W * PF) {
        u32x4 raw[PF];
        T sr[PF][4];
        uint8_t zr[PF][4];
        float sa[I8 ? PF : 1][I8 ? 4 : 1][MT][4];        // int8 path: activation scales
        // Activation operands of the run, when they fit in 64 registers (else loaded per chunk).
        constexpr int A_REGS = I8 ? 2 : 4;
        constexpr bool PRE_A = PF * 4 * MT * A_REGS <= 64;
        u32x4 apre[PRE_A ? PF : 1][PRE_A ? 4 : 1][PRE_A ? MT : 1];
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int c = c0 + p;
            if constexpr (PRE_A) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    int kc = 4 * c + t;
                    kc = kc < chunks ? kc : chunks - 1;
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        if constexpr (I8) {
                            const u32x2 v = *reinterpret_cast<const u32x2*>(
                                static_cast<const int8_t*>(Av) + (int64_t)arow[i] * K + 32 * kc + 8 * g);
                            apre[p][t][i] = u32x4{v.x, v.y, 0u, 0u};
                        } else {
                            apre[p][t][i] = *reinterpret_cast<const u32x4*>(
                                static_cast<const f16*>(Av) + (int64_t)arow[i] * K + 32 * kc + 8 * g);
                        }
                    }
                }
            }
            int ch = 4 * c + g;
            const bool ok = ch < chunks;
            ch = ok ? ch : chunks - 1;
            raw[p] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(bcol - 16 * g + 16 * (int64_t)ch));
            if (!ok) raw[p] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int kc = 4 * c + t;
                kc = kc < chunks ? kc : chunks - 1;
                int blk = (32 * kc) / BS;
                blk = blk < b_hi ? blk : b_hi - 1;       // past the range: any staged value
                if (!I8 || (t + 1) % CPB == 0) sr[p][t] = lS[blk - b_lo];
                if constexpr (HAS_ZP) zr[p][t] = lZ[(blk >> 1) - z_lo];
                else zr[p][t] = 0;
                if constexpr (I8) {
                    if ((t + 1) % CPB == 0) {            // block ends: one scale per output row
#pragma unroll
                        for (int i = 0; i < MT; ++i) {
                            const f32x4 v = *reinterpret_cast<const f32x4*>(
                                sA + (blk - b_lo) * (16 * MT) + 16 * i + 4 * g);
#pragma unroll
                            for (int q = 0; q < 4; ++q) sa[p][t][i][q] = v[q];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            // Branch-free: an iteration past the split's range or a chunk past K is computed on
            // clamped in-bounds data and dropped by a zero scale (a branch here would let the
            // compiler sink the prefetched loads into it).
            const int c = c0 + p;
            const bool in_run = c < c_hi;                // wave-uniform
            uint32_t v0 = raw[p].x, v1 = raw[p].y, v2 = raw[p].z, v3 = raw[p].w;
            transpose_rows(v0, v1, v2, v3);
            const uint32_t wt[4] = {v0, v1, v2, v3};
            if constexpr (!I8) {
                const f16* __restrict__ A = static_cast<const f16*>(Av);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int kc = 4 * c + t;
                    const int blk = (32 * kc) / BS;
                    const float s = (in_run && kc < chunks) ? (float)sr[p][t] : 0.f;
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((zr[p][t] >> ((blk & 1) * 4)) & 0xFu);
                    const f16x2 zo = zoff4(z);
                    f16x8 bop;
                    bop.s01 = nib_pair<0>(wt[t], zo);
                    bop.s23 = nib_pair<1>(wt[t], zo);
                    bop.s45 = nib_pair<2>(wt[t], zo);
                    bop.s67 = nib_pair<3>(wt[t], zo);
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        f16x8 aop;
                        if constexpr (PRE_A) aop = __builtin_bit_cast(f16x8, apre[p][t][i]);
                        else aop = *reinterpret_cast<const f16x8*>(A + (int64_t)arow[i] * K + 32 * min(kc, chunks - 1) + 8 * g);
                        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, d, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[i][q] = __builtin_fmaf(d[q], s, acc[i][q]);
                    }
                }
            } else {
                const int8_t* __restrict__ A = static_cast<const int8_t*>(Av);
                i32x4 dot[MT];
#pragma unroll
                for (int i = 0; i < MT; ++i) dot[i] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int kc = 4 * c + t;
                    const int blk = (32 * kc) / BS;
                    int z = 8;
                    if constexpr (HAS_ZP) z = (int)((zr[p][t] >> ((blk & 1) * 4)) & 0xFu);
                    const uint32_t zb = (uint32_t)(128 - z) * 0x01010101u;
                    const i32x2 bop = qz_i8(wt[t], zb);
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        i32x2 aop;
                        if constexpr (PRE_A) aop = i32x2{(int32_t)apre[p][t][i].x, (int32_t)apre[p][t][i].y};
                        else aop = *reinterpret_cast<const i32x2*>(A + (int64_t)arow[i] * K + 32 * min(kc, chunks - 1) + 8 * g);
                        dot[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            __builtin_bit_cast(long, aop), __builtin_bit_cast(long, bop), dot[i], 0, 0, 0);
                    }
                    // K % BS == 0, so a block always ends on a chunk with (t + 1) % CPB == 0,
                    // and a block is either wholly inside K or wholly past it.
                    if ((t + 1) % CPB == 0) {            // end of a block: scale it
                        const float sb = (in_run && kc < chunks) ? (float)sr[p][t] : 0.f;
#pragma unroll
                        for (int i = 0; i < MT; ++i) {
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                acc[i][q] = __builtin_fmaf((float)dot[i][q], sa[p][t][i][q] * sb, acc[i][q]);
                            dot[i] = i32x4{0, 0, 0, 0};
                        }
                    }
                }
            }
        }
    }

    // Fixed-order sum of the W wavefronts' partial tiles.
#pragma unroll
    for (int i = 0; i < MT; ++i) red[(wave * MT + i) * 64 + lane] = acc[i];
    __syncthreads();
    if (ksplit > 1) {
        // K split over workgroups: each writes its partial tile; the last to arrive (device-
        // scope counter) adds the partials in split order and stores Y, then re-arms the
        // counter.  Ordering relies on a property of gfx950 rather than on HIP memory-model
        // fences: the partials are written with agent-scope atomic stores, which are performed
        // at the device coherence point (written through the XCD's L2), s_waitcnt(0) waits
        // until they have completed there, the arrival counter is an agent-scope atomic at the
        // same point, and the last workgroup reads the partials with agent-scope atomic loads.
        // An arriving workgroup that sees the final count therefore sees every partial.  The
        // model-level alternative -- release / acquire fences at agent scope -- compiles on
        // gfx950 to a write-back and an invalidate of the whole L2 (buffer_wbl2 / buffer_inv)
        // per workgroup, which made this launch about ten times slower when measured.
        const int sid = (blockIdx.z * gridDim.y + blockIdx.y) * (gridDim.x / ksplit) + strip;
        float* mine = reinterpret_cast<float*>(part + ((int64_t)sid * ksplit + split) * (MT * 64));
        for (int idx = threadIdx.x; idx < 64 * MT; idx += blockDim.x) {
            f32x4 sum = red[idx];
            for (int w = 1; w < W; ++w) sum += red[w * MT * 64 + idx];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                __hip_atomic_store(mine + 4 * idx + q, sum[q], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);                   // the partial stores have completed
        __syncthreads();
        __shared__ int last;
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(cnt + sid, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == ksplit - 1;
        __syncthreads();
        if (!last) return;
        const float* all = reinterpret_cast<const float*>(part + (int64_t)sid * ksplit * (MT * 64));
        for (int idx = threadIdx.x; idx < 64 * MT; idx += blockDim.x) {
            f32x4 sum;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                sum[q] = __hip_atomic_load(all + 4 * idx + q, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            for (int p = 1; p < ksplit; ++p)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    sum[q] += __hip_atomic_load(all + p * (MT * 64 * 4) + 4 * idx + q,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int i = idx >> 6;
            const int ll = idx & 63;
            const int cc = n0 + (ll & 15);
            if (cc >= N) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = r0 + 16 * i + 4 * (ll >> 4) + q;
                if (r < row_hi) Y[(int64_t)r * N + cc] = (T)sum[q];
            }
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(cnt + sid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    for (int idx = threadIdx.x; idx < 64 * MT; idx += blockDim.x) {
        f32x4 sum = red[idx];
        for (int w = 1; w < W; ++w) sum += red[w * MT * 64 + idx];
        const int i = idx >> 6;
        const int ll = idx & 63;
        const int cc = n0 + (ll & 15);
        if (cc >= N) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = r0 + 16 * i + 4 * (ll >> 4) + q;
            if (r < row_hi) Y[(int64_t)r * N + cc] = (T)sum[q];
        }
    }
}

// accuracy_level = 4 activation quantiser.  One thread per 8 consecutive activations; the
// BS/8 threads of a (row, block) reduce amax with shuffles.  scale = amax / 127,
// qa = clamp(rint(a * (127 / amax)), -127, 127) (0 when amax == 0), all in fp32 with
// round-half-even.  PERMUTED writes each group of eight as [0,2,4,6,1,3,5,7] (the order
// qz_i8 produces weights in); otherwise natural order plus the block sums of qa.
template <typename T, int BS, int LAYOUT, bool VEC>
__global__ void __launch_bounds__(256)
quantize_a_int8(const T* __restrict__ A, int8_t* __restrict__ qa, float* __restrict__ scale,
                int32_t* __restrict__ qsum, int M, int K, int* __restrict__ cnt, int ncnt,
                int s_row, int s_blk) {
    constexpr int G = BS / 8;                            // threads per block: 2..16
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    // the split-K counters of the int8 GEMV that follows start at zero
    for (int64_t i = t; i < ncnt; i += (int64_t)gridDim.x * blockDim.x) cnt[i] = 0;
    const int64_t groups = (int64_t)M * (K / 8);
    const bool live = t < groups;
    const int64_t tt = live ? t : groups - 1;
    const int row = (int)(tt / (K / 8));
    const int k0 = (int)(tt % (K / 8)) * 8;
    float a[8];
    if constexpr (VEC) {                                 // 16-byte aligned rows: wide loads
        const T* src = A + (int64_t)row * K + k0;
        if constexpr (sizeof(T) == 2) {
            const f16x8 v = *reinterpret_cast<const f16x8*>(src);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = (float)v[e];
        } else {
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(src);
            const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) { a[e] = v0[e]; a[e + 4] = v1[e]; }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (float)A[(int64_t)row * K + k0 + e];
    }
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(a[e]));
    // G consecutive threads share a block (G divides 64 and blocks start at multiples of G);
    // their maximum through DPP exchanges within the lane row (G <= 16)
    static_assert(G <= 16, "block of at most 16 threads");
    if constexpr (G >= 2) amax = fmaxf(amax, dpp_f<0xB1>(amax));     // lane ^ 1
    if constexpr (G >= 4) amax = fmaxf(amax, dpp_f<0x4E>(amax));     // lane ^ 2
    if constexpr (G >= 8) amax = fmaxf(amax, dpp_f<0x141>(amax));    // 7 - i within 8
    if constexpr (G >= 16) amax = fmaxf(amax, dpp_f<0x140>(amax));   // 15 - i within 16
    const float inv = amax > 0.f ? 127.0f / amax : 0.f;
    int q[8];
    int s = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float v = rintf(a[e] * inv);
        v = fminf(fmaxf(v, -127.f), 127.f);
        q[e] = (int)v;
        s += q[e];
    }
    if (!live) return;
    const int blk = k0 / BS;
    const int bpc = K / BS;
    constexpr bool PERMUTED = LAYOUT >= 1;
    int kd = k0;
    if constexpr (LAYOUT == 2) {
        // quad-interleaved: in every whole 128-k quad, the 8-byte group of chunk t and lane row
        // g (4t + g in natural order) goes to (t / 2) * 64 + 16 g + (t % 2) * 8, so that a lane
        // row's four chunks are two 16-byte pieces and one 16-byte load per lane covers 64
        // contiguous bytes of each of 16 rows; a partial last quad keeps natural order
        const int qs = k0 & ~127;
        if (qs + 128 <= K) {
            const int t4 = (k0 & 127) >> 5, g4 = (k0 & 31) >> 3;
            kd = qs + (t4 >> 1) * 64 + g4 * 16 + (t4 & 1) * 8;
        }
    }
    int8_t* out = qa + (int64_t)row * K + kd;
    constexpr int order_p[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    int8_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (int8_t)q[PERMUTED ? order_p[e] : e];
    if constexpr (VEC) {
        u32x2 w;
        w.x = (uint32_t)(uint8_t)o[0] | ((uint32_t)(uint8_t)o[1] << 8) |
              ((uint32_t)(uint8_t)o[2] << 16) | ((uint32_t)(uint8_t)o[3] << 24);
        w.y = (uint32_t)(uint8_t)o[4] | ((uint32_t)(uint8_t)o[5] << 8) |
              ((uint32_t)(uint8_t)o[6] << 16) | ((uint32_t)(uint8_t)o[7] << 24);
        *reinterpret_cast<u32x2*>(out) = w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = o[e];
    }
    if (k0 % BS == 0) scale[(int64_t)row * s_row + (int64_t)blk * s_blk] = amax / 127.0f;
    if (qsum) {
        // block sum: the G partial sums meet in the block's first thread
        int bs_sum = s;
        for (int off = G >> 1; off > 0; off >>= 1) bs_sum += __shfl_xor(bs_sum, off, 64);
        if (k0 % BS == 0) qsum[(int64_t)row * bpc + blk] = bs_sum;
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

bool group_gemv_supported(int64_t k, int bits, int bs) {
    return bits == 4 && bs >= 32 && k > 0 && k % 32 == 0 && k % bs == 0;
}

GroupGeom group_geometry(int64_t rows, int64_t n, int64_t k, int64_t groups, bool i8, int bs,
                         bool allow_split) {
    GroupGeom g{};
    g.mt = rows <= 16 ? 1 : (rows <= 32 ? 2 : 4);
    const int64_t iters = (k / 32 + 3) / 4;
    const int pf = group_pf(i8, bs, g.mt);
    const int64_t runs = (iters + pf - 1) / pf;          // runs of pf iterations per wavefront
    g.gx = (n + 15) / 16;
    g.gy = groups;
    g.gz = (rows + 16 * g.mt - 1) / (16 * g.mt);
    // Enough wavefronts on each 16-column strip to fill the chip: about 8 per CU in total.
    const int64_t strips = g.gx * groups * (allow_split ? g.gz : 1);
    int64_t w = (8 * 256 + strips - 1) / strips;
    if (w < 1) w = 1;
    if (w > runs) w = runs;
    // More than 8 wavefronts per strip: split K over workgroups as well.
    int64_t ks = (allow_split && w > 8) ? (w + 7) / 8 : 1;
    int64_t rps = (runs + ks - 1) / ks;
    ks = (runs + rps - 1) / rps;                         // no empty split
    w = ks > 1 ? rps : w;
    if (w > 8) w = 8;
    g.waves = (int)w;
    g.ksplit = (int)ks;
    g.runs_per_split = (int)rps;
    // LDS: the wavefronts' partial tiles, then the strip's staged scales (fp32 at most) and
    // zero points over one split's K range.
    const int64_t nblk = std::min<int64_t>(k / bs, rps * pf * 128 / bs + 1);
    g.lds = (size_t)g.waves * g.mt * 64 * sizeof(f32x4) + 16 * ((nblk + 3) & ~3) * sizeof(float) +
            16 * ((nblk / 2 + 2 + 3) & ~3) + (i8 ? (size_t)16 * g.mt * nblk * sizeof(float) : 0);
    return g;
}

template <typename T, bool I8, int BS, bool HAS_ZP>
static hipError_t group_mt(const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, f32x4* part, int* cnt, hipStream_t st) {
    if (g.waves < 1 || 64 * g.waves > kGroupMaxThreads) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(g.gx * g.ksplit), (unsigned)g.gy, (unsigned)g.gz);
    const dim3 block((unsigned)(64 * g.waves), 1, 1);
    const T* S = static_cast<const T*>(s);
    T* Y = static_cast<T*>(y);
#define MNB_GROUP_GO(MT_)                                                                          \
    do {                                                                                          \
        auto kern = group_gemv<T, I8, BS, HAS_ZP, MT_>;                                           \
        const hipError_t ea = allow_dynamic_lds(reinterpret_cast<const void*>(kern), g.lds);     \
        if (ea != hipSuccess) return ea;                                                          \
        hipLaunchKernelGGL(kern, grid, block, g.lds, st, a, a_scale, row_index, offsets, b, S, z, \
                           Y, (int)m, (int)n, (int)k, g.ksplit, g.runs_per_split, part, cnt);     \
    } while (0)
    switch (g.mt) {
        case 1: MNB_GROUP_GO(1); break;
        case 2: MNB_GROUP_GO(2); break;
        default: MNB_GROUP_GO(4); break;
    }
#undef MNB_GROUP_GO
    return hipGetLastError();
}

template <typename T, bool I8, int BS>
static hipError_t group_zp(const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, f32x4* part, int* cnt, hipStream_t st) {
    if (z) return group_mt<T, I8, BS, true>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, part, cnt, st);
    return group_mt<T, I8, BS, false>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, part, cnt, st);
}

template <typename T, bool I8>
static hipError_t group_bs(int bs, const GroupGeom& g, const void* a, const float* a_scale,
                           const int32_t* row_index, const int32_t* offsets, const uint8_t* b,
                           const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                           int64_t k, f32x4* part, int* cnt, hipStream_t st) {
    switch (bs) {
        case 32: return group_zp<T, I8, 32>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, part, cnt, st);
        case 64: return group_zp<T, I8, 64>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, part, cnt, st);
        case 128: return group_zp<T, I8, 128>(g, a, a_scale, row_index, offsets, b, s, z, y, m, n, k, part, cnt, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_group_gemv_f16(const void* a, const int32_t* row_index, const int32_t* offsets,
                                 int64_t groups, int64_t max_rows, const uint8_t* b,
                                 const void* s, const uint8_t* z, void* y, int64_t m, int64_t n,
                                 int64_t k, int bits, int bs, hipStream_t st) {
    if (!group_gemv_supported(k, bits, bs)) return hipErrorInvalidValue;
    if (m == 0 || groups == 0) return hipSuccess;
    // Up to 16 rows per group (by the mean for grouped rows): the strip GEMV, one 16-row tile
    // per group plus more tiles for the groups that exceed it.
    const int64_t ng = offsets ? groups : 1;
    const int64_t bound = offsets ? max_rows : m;
    const int64_t hint = offsets ? std::min<int64_t>(bound, 2 * ((m + ng - 1) / ng)) : m;
    StripGeom sg;
    if (hint <= 16 && !strip_gemv_forced_off() && strip_gemv_aligned(a, b, s, z, false) &&
        strip_geometry(n, k, ng, bound, false, bs, z != nullptr, &sg))
        return launch_strip_gemv(sg, false, a, nullptr, row_index, offsets, b, s, z, y, m, n, k,
                                 bs, st);
    const GroupGeom g =
        group_geometry(offsets ? max_rows : m, n, k, offsets ? groups : 1, false, bs, false);
    return group_bs<f16, false>(bs, g, a, nullptr, row_index, offsets, b, s, z, y, m, n, k,
                                nullptr, nullptr, st);
}

hipError_t launch_group_gemv_f16_bounded(const void* a, const int32_t* row_index,
                                         const int32_t* offsets, int64_t groups,
                                         int64_t rows_bound, int64_t rows_hint, const uint8_t* b,
                                         const void* s, const uint8_t* z, void* y, int64_t m,
                                         int64_t n, int64_t k, int bits, int bs, hipStream_t st,
                                         const uint8_t* b_strips) {
    if (!group_gemv_supported(k, bits, bs)) return hipErrorInvalidValue;
    if (m == 0 || groups == 0) return hipSuccess;
    StripGeom sg;
    if (rows_hint <= 16 && !strip_gemv_forced_off() && strip_gemv_aligned(a, b, s, z, false) &&
        strip_geometry(n, k, groups, rows_bound, false, bs, z != nullptr, &sg))
        return launch_strip_gemv(sg, false, a, nullptr, row_index, offsets, b, s, z, y, m, n, k,
                                 bs, st, nullptr, b_strips);
    // Tile height from the expected rows per group; enough row tiles for the bound (tiles past
    // a group's last row leave at once).
    GroupGeom g = group_geometry(std::max<int64_t>(1, std::min(rows_hint, rows_bound)), n, k,
                                 groups, false, bs, false);
    g.gz = (rows_bound + 16 * g.mt - 1) / (16 * g.mt);
    return group_bs<f16, false>(bs, g, a, nullptr, row_index, offsets, b, s, z, y, m, n, k,
                                nullptr, nullptr, st);
}

hipError_t launch_quantize_a_int8(const void* a, bool a_f16, int8_t* qa, float* scale,
                                  int32_t* qsum, bool permuted, int64_t m, int64_t k, int bs,
                                  hipStream_t st, int* cnt, int64_t ncnt, int64_t scale_rows,
                                  bool quads) {
    if (m == 0) return hipSuccess;
    if (k % bs || (bs != 16 && bs != 32 && bs != 64 && bs != 128)) return hipErrorInvalidValue;
    const int64_t groups = m * (k / 8);
    // one thread per 8 values; small activations (decode: at most 256 workgroups of 256) in
    // workgroups of one wavefront, so that every CU takes a share of the loads
    const int tpb = groups <= 256 * 256 ? 64 : 256;
    const dim3 grid((unsigned)((groups + tpb - 1) / tpb));
    // scales [m][k/bs], or block-major [k/bs][scale_rows] when scale_rows > 0
    const int s_row = scale_rows > 0 ? 1 : (int)(k / bs);
    const int s_blk = scale_rows > 0 ? (int)scale_rows : 1;
    const bool vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(qa) % 8 == 0);
#define MNB_Q(T_, BS_)                                                                            \
    do {                                                                                          \
        if (quads && vec)                                                                         \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 2, true>), grid, dim3(tpb), 0, st,       \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
        else if (quads)                                                                           \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 2, false>), grid, dim3(tpb), 0, st,      \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
        else if (permuted && vec)                                                                 \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 1, true>), grid, dim3(tpb), 0, st,       \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
        else if (vec)                                                                             \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 0, true>), grid, dim3(tpb), 0, st,       \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
        else if (permuted)                                                                        \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 1, false>), grid, dim3(tpb), 0, st,      \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
        else                                                                                      \
            hipLaunchKernelGGL((quantize_a_int8<T_, BS_, 0, false>), grid, dim3(tpb), 0, st,      \
                               static_cast<const T_*>(a), qa, scale, qsum, (int)m, (int)k, cnt,   \
                               (int)ncnt, s_row, s_blk);                                          \
    } while (0)
#define MNB_QBS(T_)                                                                               \
    switch (bs) {                                                                                 \
        case 16: MNB_Q(T_, 16); break;                                                            \
        case 32: MNB_Q(T_, 32); break;                                                            \
        case 64: MNB_Q(T_, 64); break;                                                            \
        default: MNB_Q(T_, 128); break;                                                           \
    }
    if (a_f16) {
        MNB_QBS(f16);
    } else {
        MNB_QBS(float);
    }
#undef MNB_QBS
#undef MNB_Q
    return hipGetLastError();
}

// accuracy_level = 4 workspace: qa [m][k] int8 | a_scale fp32 ([m][k/bs], or block-major over
// 16 rows) | the row-tiled GEMV's split-K partial tiles | its split-K counters, each part
// 256-byte aligned (the last two empty when another int8 GEMV is planned).
namespace {
struct Acc4Layout {
    size_t qa, sa, part, cnt, total;
    int64_t ncnt;
};
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
Acc4Layout acc4_layout(bool a_f16, int64_t m, int64_t n, int64_t k, int bs, GroupGeom* gout,
                       Acc4StreamGeom* sout, bool* stream, bool* strip) {
    Acc4Layout l{};
    l.qa = 0;
    l.sa = align256((size_t)m * (size_t)k);
    l.part = l.sa + align256((size_t)std::max<int64_t>(m, 16) * (size_t)(k / bs) * sizeof(float));
    size_t part_bytes = 0;
    *stream = acc4_stream_planned(a_f16, m, n, k, bs, sout);
    StripGeom sg;
    *strip = !*stream && a_f16 && m <= 16 && !strip_gemv_forced_off() &&
             strip_geometry(n, k, 1, m, true, bs, true, &sg);   // zero points: the larger LDS
    const GroupGeom g = group_geometry(m, n, k, 1, true, bs, true);
    *gout = g;
    if (!*stream && !*strip) {
        const int64_t nsid = g.gx * g.gy * g.gz;
        part_bytes = g.ksplit > 1 ? (size_t)nsid * g.ksplit * g.mt * 64 * sizeof(f32x4) : 0;
        l.ncnt = g.ksplit > 1 ? nsid : 0;
    }
    l.cnt = l.part + align256(part_bytes);
    l.total = l.cnt + align256((size_t)l.ncnt * sizeof(int));
    return l;
}
}  // namespace

size_t acc4_workspace_bytes(int64_t m, int64_t n, int64_t k, int bs, bool a_f16) {
    GroupGeom g;
    Acc4StreamGeom sg;
    bool stream, strip;
    return acc4_layout(a_f16, m, n, k, bs, &g, &sg, &stream, &strip).total;
}

hipError_t launch_acc4(const void* a, bool a_f16, const uint8_t* b, const void* s,
                       const uint8_t* z, void* y, int64_t m, int64_t n, int64_t k, int bits,
                       int bs, void* workspace, hipStream_t st, const uint8_t* b_strips) {
    if (!group_gemv_supported(k, bits, bs)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    GroupGeom g{};
    Acc4StreamGeom ag{};
    bool stream = false, strip = false;
    const Acc4Layout l = acc4_layout(a_f16, m, n, k, bs, &g, &ag, &stream, &strip);
    uint8_t* const ws = static_cast<uint8_t*>(workspace);
    int8_t* const qa = reinterpret_cast<int8_t*>(ws + l.qa);
    float* const sa = reinterpret_cast<float*>(ws + l.sa);
    // fp16 with at most 16 rows: the quantiser's codes (quad-interleaved) and scales
    // (block-major over 16 rows, the workspace's first two parts) feed the strip-per-workgroup
    // GEMV, or the strip GEMV where that one does not apply
    StripGeom sg;
    if (stream && acc4_stream_aligned(qa, b, s, z)) {
        hipError_t e = launch_quantize_a_int8(a, true, qa, sa, nullptr, true, m, k, bs, st,
                                              nullptr, 0, 16, true);
        if (e != hipSuccess) return e;
        return launch_acc4_stream(ag, qa, sa, b, s, z, y, m, n, k, bs, st, b_strips);
    }
    if (stream || strip) {
        // (the planned kernel, or the fallback of the strip-per-workgroup one for sub-aligned
        // scales or zero points; the workspace has no split-K room for the row-tiled GEMV)
        if (!strip_gemv_aligned(qa, b, s, z, true) ||
            !strip_geometry(n, k, 1, m, true, bs, z != nullptr, &sg))
            return hipErrorInvalidValue;
        hipError_t e = launch_quantize_a_int8(a, true, qa, sa, nullptr, true, m, k, bs, st,
                                              nullptr, 0, 16, true);
        if (e != hipSuccess) return e;
        return launch_strip_gemv(sg, true, qa, sa, nullptr, nullptr, b, s, z, y, m, n, k, bs, st);
    }
    f32x4* part = g.ksplit > 1 ? reinterpret_cast<f32x4*>(ws + l.part) : nullptr;
    int* cnt = g.ksplit > 1 ? reinterpret_cast<int*>(ws + l.cnt) : nullptr;
    hipError_t e = launch_quantize_a_int8(a, a_f16, qa, sa, nullptr, true, m, k, bs, st, cnt,
                                          l.ncnt);
    if (e != hipSuccess) return e;
    if (a_f16)
        return group_bs<f16, true>(bs, g, qa, sa, nullptr, nullptr, b, s, z, y, m, n, k, part, cnt, st);
    return group_bs<float, true>(bs, g, qa, sa, nullptr, nullptr, b, s, z, y, m, n, k, part, cnt, st);
}

}  // namespace mnb
