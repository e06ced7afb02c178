// Fused QMoE (com.microsoft::QMoE, int4 experts, SwiGLU) on gfx950: routing, two expert-grouped
// MatMulNBits GEMVs and the weighted combine, stream-ordered with no host round trip.
//
// The reference registers QMoE without a kernel (rust/src/ops/moe.rs:92-118; its rows are staged,
// top-1/2 only) and records the attribute values of gpt-oss-20b (docs/OP_COVERAGE.md:831-835).
// The op's arithmetic is ONNX Runtime's (third-party, not under the reference); this file
// implements the build's declared reading of it:
//
//   1. qmoe_topk       one wavefront per token: softmax over the E router logits, the k largest
//                      (ties to the lower expert id), optionally renormalised;
//      qmoe_group      one workgroup: counting sort of the T*k (token, slot) assignments by
//                      expert: offsets[E+1], the token of every grouped row, the grouped row of
//                      every assignment.
//      qmoe_group_small the same for T*k <= 1024 and E <= 64 (decode batches), stable; when
//                      fc1 runs on the strip GEMV with SwiGLU it finds its rows itself
//                      (StripSwiglu) and no sort launch runs.
//   2. group_gemv      h = x W1_e^T for every grouped row (the MatMulNBits expert-grouped GEMV,
//                      rows gathered through the sort), fp16 out.
//   3. qmoe_swiglu     act = SwiGLU(h + b1_e): gate/linear interleaved or concatenated,
//                      gate <= limit, |linear| <= limit, gate * sigmoid(alpha gate) * (linear + beta)
//                      in fp32, fp16 out.  For interleaved pairs on the strip GEMV (at most 16
//                      expected rows per expert) steps 2 and 3 are one kernel: the strip GEMV
//                      applies SwiGLU to each (gate, linear) pair as it stores fc1's tiles.
//   4. group_gemv      o = act W2_e^T, fp16 out.
//   5. qmoe_combine    y[t] = sum over the token's k slots of w * (o + b2_e), fp32, in slot order
//                      (deterministic), fp16 out.
//
// Rows per expert are known only on the device, so the GEMV grids cover T rows per expert
// (no expert takes a token twice); tiles past an expert's last row leave at once.
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

constexpr int kRouteThreads = 1024;

template <typename L>
__device__ __forceinline__ float ld(const L* p, int64_t i) {
    return (float)p[i];
}

}  // namespace

// One token's routing by a wavefront when E <= 64: lane e holds logit e.  An expert's rank is
// the number of experts ahead of it (a larger logit, or an equal one with a lower id); the
// experts of rank < k are the k rounds of arg-max with ties to the lower id, in slot order.
// Each lane writes the 64-bit key (logit order, then 63 - lane) to the wavefront's LDS row and
// counts the larger keys of that row, read as broadcasts (lanes past E write 0, below every
// key); logits order as totally ordered keys (-0 as +0, a NaN above +inf or below -inf by its
// sign) so the ranks are always a permutation of 0 .. E-1.  The chosen probabilities pass
// through LDS by slot and are summed in slot order.  Returns the lane's rank (64 past E) and
// routing weight (softmax, renormalised over the k slots when asked).
struct Routed {
    int rank;
    float w;
};

template <int NP>
__device__ __forceinline__ int count_above(const uint64_t* __restrict__ kb, uint64_t mine) {
    typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
    int n = 0;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const u64x2 v = reinterpret_cast<const u64x2*>(kb)[j];
        n += (v.x > mine ? 1 : 0) + (v.y > mine ? 1 : 0);
    }
    return n;
}

__device__ __forceinline__ Routed route_wave64(float v, int lane, int E, int k, int normalize,
                                               uint64_t* __restrict__ kb,
                                               float* __restrict__ kp) {
    const bool live = lane < E;
    v = live ? v + 0.f : -INFINITY;
    const float mx = wave_max64(v);
    const float ev = live ? expf(v - mx) : 0.f;
    const float p = ev / group_sum(ev, 64);
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint64_t mine = ((uint64_t)key << 6) | (uint64_t)(63 - lane);
    kb[lane] = live ? mine : 0;
    __builtin_amdgcn_wave_barrier();
    const int rank = !live ? 64 : E <= 16 ? count_above<8>(kb, mine)
                                : E <= 32 ? count_above<16>(kb, mine) : count_above<32>(kb, mine);
    if (rank < k) kp[rank] = p;
    __builtin_amdgcn_wave_barrier();
    float psum = 0.f;
    for (int s = 0; s < k; ++s) psum += kp[s];
    __builtin_amdgcn_wave_barrier();                     // kb / kp are rewritten by the next token
    return Routed{rank, normalize ? p / psum : p};
}

// Routing, part 1: one wavefront per token (four per workgroup).  E <= 64: route_wave64.
// Otherwise the logits of experts e = lane + 64 j in registers: wave-wide max and sum for the
// softmax, then k rounds of a wave-wide arg-max (the lower id wins a tie) over the experts not
// yet chosen.
template <typename L>
__global__ void __launch_bounds__(256)
qmoe_topk(const L* __restrict__ logits, int T, int E, int k, int normalize,
          int32_t* __restrict__ expert_of, float* __restrict__ weight_of) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;                                  // whole wavefront
    const L* lg = logits + (int64_t)t * E;
    if (E <= 64) {
        __shared__ __align__(16) uint64_t kb[4][64];
        __shared__ float kp[4][8];
        const int w = threadIdx.x >> 6;
        const Routed r = route_wave64(ld(lg, min(lane, E - 1)), lane, E, k, normalize, kb[w],
                                      kp[w]);
        if (r.rank < k) {
            expert_of[t * k + r.rank] = lane;
            weight_of[t * k + r.rank] = r.w;
        }
        return;
    }
    const int nj = (E + 63) / 64;                        // <= 16
    float v[16];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int e = lane + 64 * j;
        const float x = ld(lg, min(e, E - 1));          // clamped, unpredicated: issued together
        v[j] = (j < nj && e < E) ? x : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int e = lane + 64 * j;
        if (j < nj && e < E) sum += expf(v[j] - mx);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    uint32_t taken = 0;                                  // bit j: expert lane + 64 j chosen
    int my_e = 0;                                        // lane s keeps slot s
    float my_p = 0.f, psum = 0.f;
    for (int s = 0; s < k; ++s) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int e = lane + 64 * j;
            if (j < nj && e < E && !((taken >> j) & 1u) && (bi == 0x7fffffff || v[j] > bv)) {
                bv = v[j];
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        const float p = expf(bv - mx) / sum;
        psum += p;
        if (lane == s) {
            my_e = bi;
            my_p = p;
        }
    }
    if (lane < k) {
        expert_of[t * k + lane] = my_e;
        weight_of[t * k + lane] = normalize ? my_p / psum : my_p;
    }
}

// Routing, part 2 (one workgroup): counting sort of the T*k assignments by expert.  An LDS
// atomic gives each assignment its slot within its expert (every grouped row is computed on its
// own, so results do not depend on that order); a scan of the counts gives the offsets.
__global__ void __launch_bounds__(kRouteThreads)
qmoe_group(const int32_t* __restrict__ expert_of, int R, int E, int k,
           int32_t* __restrict__ offsets, int32_t* __restrict__ row_token,
           int32_t* __restrict__ pos_of, int32_t* __restrict__ expert_of_row) {
    __shared__ int32_t cnt[kRouteThreads];
    __shared__ int32_t tmp[kRouteThreads];
    const int tid = threadIdx.x;
    constexpr int kPer = 16;                             // R <= 16 * 1024
    for (int e = tid; e < E; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    int ex[kPer], sl[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int a = tid + kRouteThreads * j;
        const int xv = expert_of[min(a, R - 1)];        // clamped, unpredicated: issued together
        ex[j] = a < R ? xv : -1;
        sl[j] = ex[j] >= 0 ? atomicAdd(&cnt[ex[j]], 1) : 0;
    }
    __syncthreads();
    // inclusive scan of cnt[0..E) (Hillis-Steele), kept beside the counts
    const int c = tid < E ? cnt[tid] : 0;
    int run = c;
    for (int d = 1; d < E; d <<= 1) {
        if (tid < E) tmp[tid] = run;
        __syncthreads();
        if (tid < E && tid >= d) run += tmp[tid - d];
        __syncthreads();
    }
    if (tid < E) {
        cnt[tid] = run - c;                              // exclusive: first row of expert tid
        offsets[tid] = run - c;
        if (tid == E - 1) offsets[E] = run;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int a = tid + kRouteThreads * j;
        if (a >= R) break;
        const int pos = cnt[ex[j]] + sl[j];
        row_token[pos] = a / k;
        pos_of[a] = pos;
        expert_of_row[pos] = ex[j];
    }
}

// Routing, part 2 for T * k <= kSmallR and E <= 64 (decode batches; one workgroup, one
// assignment per thread): a stable counting sort by expert.  Within a wavefront the rank of an
// assignment among those of its expert comes from one ballot per expert; wavefront 0 scans the
// per-wavefront counts in (expert, wavefront) order.  The grouped rows of an expert keep token
// order, independent of timing.
constexpr int kSmallR = 1024;

__global__ void __launch_bounds__(kSmallR)
qmoe_group_small(const int32_t* __restrict__ expert_of, int R, int E, int k,
                 int32_t* __restrict__ offsets, int32_t* __restrict__ row_token,
                 int32_t* __restrict__ pos_of, int32_t* __restrict__ expert_of_row) {
    constexpr int kWaves = kSmallR / 64;
    __shared__ int32_t s_cnt[kWaves][64];                // per wavefront and expert
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int a = threadIdx.x;
    const int x0 = expert_of[min(a, R - 1)];
    const int ex = a < R ? x0 : -1;
    int local = 0;
    if (wave * 64 < R) {                                 // wave-uniform
        for (int x = 0; x < E; ++x) {
            const uint64_t m = __ballot(ex == x);
            const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
            local = ex == x ? below : local;
            if (lane == 0) s_cnt[wave][x] = __popcll(m);
        }
    } else if (lane < E) {
        s_cnt[wave][lane] = 0;
    }
    __syncthreads();
    if (wave == 0) {                                     // offsets, first row of (wave, expert)
        int tot = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tot += lane < E ? s_cnt[w][lane] : 0;
        int incl = tot;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d);
            incl += lane >= d ? o : 0;
        }
        int off = incl - tot;
        if (lane < E) {
            offsets[lane] = off;
            if (lane == E - 1) offsets[E] = incl;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const int c = s_cnt[w][lane];
                s_cnt[w][lane] = off;
                off += c;
            }
        }
    }
    __syncthreads();
    if (a < R) {
        const int pos = s_cnt[wave][ex] + local;
        row_token[pos] = a / k;
        pos_of[a] = pos;
        expert_of_row[pos] = ex;
    }
}

// Thread: four consecutive outputs of one grouped row (inter % 4 == 0).
__global__ void __launch_bounds__(256)
qmoe_swiglu(const f16* __restrict__ h, const f16* __restrict__ b1,
            const int32_t* __restrict__ expert_of_row, f16* __restrict__ act, int64_t rows,
            int64_t inter, int fusion, float alpha, float beta, float limit, int has_limit) {
    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
    const int64_t quads = inter / 4;
    const int64_t total = rows * quads;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t r = idx / quads;
        const int64_t i = (idx - r * quads) * 4;
        const f16* hr = h + r * 2 * inter;
        const f16* br = b1 ? b1 + (int64_t)expert_of_row[r] * 2 * inter : nullptr;
        float g[4], l[4];
        if (fusion == 1) {                               // (gate, linear) pairs at 2i, 2i + 1
            const f16x8 v = *reinterpret_cast<const f16x8*>(hr + 2 * i);
            f16x8 b = {};
            if (br) b = *reinterpret_cast<const f16x8*>(br + 2 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                g[j] = (float)v[2 * j] + (float)b[2 * j];
                l[j] = (float)v[2 * j + 1] + (float)b[2 * j + 1];
            }
        } else {                                         // gates at i, linears at inter + i
            const f16x4_t vg = *reinterpret_cast<const f16x4_t*>(hr + i);
            const f16x4_t vl = *reinterpret_cast<const f16x4_t*>(hr + inter + i);
            f16x4_t bg = {}, bl = {};
            if (br) {
                bg = *reinterpret_cast<const f16x4_t*>(br + i);
                bl = *reinterpret_cast<const f16x4_t*>(br + inter + i);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                g[j] = (float)vg[j] + (float)bg[j];
                l[j] = (float)vl[j] + (float)bl[j];
            }
        }
        f16x4_t out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float gj = g[j], lj = l[j];
            if (has_limit) {
                gj = fminf(gj, limit);
                lj = fminf(fmaxf(lj, -limit), limit);
            }
            out[j] = (f16)(gj / (1.f + expf(-alpha * gj)) * (lj + beta));
        }
        *reinterpret_cast<f16x4_t*>(act + r * inter + i) = out;
    }
}

// Thread: one token, 8 consecutive outputs.  hidden % 8 == 0.
__global__ void __launch_bounds__(256)
qmoe_combine(const f16* __restrict__ o, const f16* __restrict__ b2,
             const int32_t* __restrict__ expert_of, const float* __restrict__ weight_of,
             const int32_t* __restrict__ pos_of, f16* __restrict__ y, int64_t T, int64_t hidden,
             int k) {
    const int64_t chunks = hidden / 8;
    const int64_t total = T * chunks;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t t = idx / chunks;
        const int64_t c = (idx - t * chunks) * 8;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.f;
        // all slots' indices first, then all their rows (k <= 8; slots past k re-read slot k-1
        // and are not added): two dependent round trips instead of two per slot
        int pos[8], ex[8];
        float w[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int64_t a = t * k + min(s, k - 1);
            pos[s] = pos_of[a];
            ex[s] = expert_of[a];
            w[s] = weight_of[a];
        }
        f16x8 v[8], bb[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            v[s] = *reinterpret_cast<const f16x8*>(o + (int64_t)pos[s] * hidden + c);
            bb[s] = b2 ? *reinterpret_cast<const f16x8*>(b2 + (int64_t)ex[s] * hidden + c)
                       : f16x8{};
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (s >= k) break;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += w[s] * ((float)v[s][j] + (float)bb[s][j]);
        }
        f16x8 out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (f16)acc[j];
        *reinterpret_cast<f16x8*>(y + t * hidden + c) = out;
    }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

namespace {

struct QmoeLayout {
    size_t expert_of, weight_of, pos_of, row_token, expert_of_row, offsets, h, act, o, total;
};

QmoeLayout qmoe_layout(const QmoeArgs& q) {
    auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t R = (size_t)(q.rows * q.k);
    QmoeLayout l{};
    size_t off = 0;
    l.expert_of = off;     off += up(R * 4);
    l.weight_of = off;     off += up(R * 4);
    l.pos_of = off;        off += up(R * 4);
    l.row_token = off;     off += up(R * 4);
    l.expert_of_row = off; off += up(R * 4);
    l.offsets = off;       off += up((size_t)(q.experts + 1) * 4);
    l.h = off;             off += up(R * (size_t)(2 * q.inter) * 2);
    l.act = off;           off += up(R * (size_t)q.inter * 2);
    l.o = off;             off += up(R * (size_t)q.hidden * 2);
    l.total = off;
    return l;
}

unsigned grid_for(int64_t total) {
    const int64_t blocks = (total + 255) / 256;
    return (unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 65536);
}

}  // namespace

size_t qmoe_workspace_bytes(const QmoeArgs& q) { return qmoe_layout(q).total; }

hipError_t launch_qmoe(const QmoeArgs& q, const void* x, const void* logits, const uint8_t* fc1,
                       const void* fc1_s, const void* fc1_b, const uint8_t* fc2, const void* fc2_s,
                       const void* fc2_b, void* y, void* workspace, hipStream_t st,
                       const uint8_t* fc1_strips, const uint8_t* fc2_strips) {
    if (q.rows == 0) return hipSuccess;
    const QmoeLayout l = qmoe_layout(q);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int32_t* expert_of = reinterpret_cast<int32_t*>(ws + l.expert_of);
    float* weight_of = reinterpret_cast<float*>(ws + l.weight_of);
    int32_t* pos_of = reinterpret_cast<int32_t*>(ws + l.pos_of);
    int32_t* row_token = reinterpret_cast<int32_t*>(ws + l.row_token);
    int32_t* expert_of_row = reinterpret_cast<int32_t*>(ws + l.expert_of_row);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + l.offsets);
    f16* h = reinterpret_cast<f16*>(ws + l.h);
    f16* act = reinterpret_cast<f16*>(ws + l.act);
    f16* o = reinterpret_cast<f16*>(ws + l.o);
    const int64_t R = q.rows * q.k;
    const unsigned tk_grid = (unsigned)((q.rows + 3) / 4);
    if (q.router_f32)
        hipLaunchKernelGGL(qmoe_topk<float>, dim3(tk_grid), dim3(256), 0, st,
                           static_cast<const float*>(logits), (int)q.rows, (int)q.experts, q.k,
                           q.normalize, expert_of, weight_of);
    else
        hipLaunchKernelGGL(qmoe_topk<f16>, dim3(tk_grid), dim3(256), 0, st,
                           static_cast<const f16*>(logits), (int)q.rows, (int)q.experts, q.k,
                           q.normalize, expert_of, weight_of);
    // expected rows per expert (twice the mean, at least one) sets the GEMV tile height
    const int64_t hint = std::max<int64_t>(1, 2 * ((R + q.experts - 1) / q.experts));
    // Interleaved gate/linear pairs on the strip GEMV: SwiGLU as fc1's tiles are stored; for
    // decode batches fc1 also sorts its own rows out of expert_of and publishes offsets and
    // pos_of, so no sort launch runs.
    StripGeom sg;
    const bool fused = q.fusion == 1 && hint <= 16 && !strip_gemv_forced_off() &&
                       strip_gemv_aligned(x, fc1, fc1_s, nullptr, false) &&
                       strip_geometry(2 * q.inter, q.hidden, q.experts, q.rows, false,
                                      q.block_size, false, &sg);
    const bool self_sort = fused && R <= kSmallR && q.experts <= 64;
    if (self_sort) {
        // sorted inside fc1
    } else if (R <= kSmallR && q.experts <= 64)
        hipLaunchKernelGGL(qmoe_group_small, dim3(1), dim3(kSmallR), 0, st, expert_of, (int)R,
                           (int)q.experts, q.k, offsets, row_token, pos_of, expert_of_row);
    else
        hipLaunchKernelGGL(qmoe_group, dim3(1), dim3(kRouteThreads), 0, st, expert_of, (int)R,
                           (int)q.experts, q.k, offsets, row_token, pos_of, expert_of_row);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (fused) {
        StripSwiglu sw{fc1_b, q.alpha, q.beta, q.limit, q.has_limit, nullptr, nullptr, nullptr,
                       0, 0};
        if (self_sort) {
            sw.expert_of = expert_of;
            sw.offsets = offsets;
            sw.pos_of = pos_of;
            sw.R = (int)R;
            sw.k = q.k;
        }
        e = launch_strip_gemv(sg, false, x, nullptr, row_token, offsets, fc1, fc1_s, nullptr, act,
                              R, 2 * q.inter, q.hidden, q.block_size, st, &sw, fc1_strips);
        if (e != hipSuccess) return e;
    } else {
        e = launch_group_gemv_f16_bounded(x, row_token, offsets, q.experts, q.rows, hint, fc1,
                                          fc1_s, nullptr, h, R, 2 * q.inter, q.hidden, 4,
                                          q.block_size, st);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(qmoe_swiglu, dim3(grid_for(R * q.inter / 4)), dim3(256), 0, st, h,
                           static_cast<const f16*>(fc1_b), expert_of_row, act, R, q.inter,
                           q.fusion, q.alpha, q.beta, q.limit, q.has_limit);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    e = launch_group_gemv_f16_bounded(act, nullptr, offsets, q.experts, q.rows, hint, fc2, fc2_s,
                                      nullptr, o, R, q.hidden, q.inter, 4, q.block_size, st,
                                      fc2_strips);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(qmoe_combine, dim3(grid_for(q.rows * (q.hidden / 8))), dim3(256), 0, st, o,
                       static_cast<const f16*>(fc2_b), expert_of, weight_of, pos_of,
                       static_cast<f16*>(y), q.rows, q.hidden, q.k);
    return hipGetLastError();
}

}  // namespace mnb
