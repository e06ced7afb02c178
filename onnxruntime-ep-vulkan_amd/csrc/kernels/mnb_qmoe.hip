// Fused QMoE (com.microsoft::QMoE, int4 experts, SwiGLU) on gfx950: routing, two expert-grouped
// MatMulNBits GEMVs and the weighted combine, stream-ordered with no host round trip.
//
// The reference registers QMoE without a kernel (rust/src/ops/moe.rs:92-118; its rows are staged,
// top-1/2 only) and records the attribute values of gpt-oss-20b (docs/OP_COVERAGE.md:831-835).
// The op's arithmetic is ONNX Runtime's (third-party, not under the reference); this file
// implements the build's declared reading of it:
//
//   1. qmoe_route      one workgroup: per token softmax over the E router logits, the k largest
//                      (ties to the lower expert id), optionally renormalised; then a stable
//                      counting sort of the T*k (token, slot) assignments by expert: offsets[E+1],
//                      the token of every grouped row, the grouped row of every assignment.
//   2. group_gemv      h = x W1_e^T for every grouped row (the MatMulNBits expert-grouped GEMV,
//                      rows gathered through the sort), fp16 out.
//   3. qmoe_swiglu     act = SwiGLU(h + b1_e): gate/linear interleaved or concatenated,
//                      gate <= limit, |linear| <= limit, gate * sigmoid(alpha gate) * (linear + beta)
//                      in fp32, fp16 out.
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

template <typename L>
__global__ void __launch_bounds__(kRouteThreads)
qmoe_route(const L* __restrict__ logits, int T, int E, int k, int normalize,
           int32_t* __restrict__ expert_of, float* __restrict__ weight_of,
           int32_t* __restrict__ offsets, int32_t* __restrict__ row_token,
           int32_t* __restrict__ pos_of, int32_t* __restrict__ expert_of_row) {
    extern __shared__ int16_t sx[];                      // [T * k] expert of each assignment
    __shared__ int32_t cnt[kRouteThreads];
    const int tid = threadIdx.x;
    for (int t = tid; t < T; t += kRouteThreads) {
        const L* lg = logits + (int64_t)t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; ++e) mx = fmaxf(mx, ld(lg, e));
        float sum = 0.f;
        for (int e = 0; e < E; ++e) sum += expf(ld(lg, e) - mx);
        int sel[8];
        float p[8];
        float psum = 0.f;
        for (int s = 0; s < k; ++s) {
            // the largest logit not yet chosen; strict '>' keeps the lower id on ties
            int best = -1;
            float bv = -INFINITY;
            for (int e = 0; e < E; ++e) {
                bool taken = false;
                for (int j = 0; j < s; ++j) taken |= sel[j] == e;
                const float v = ld(lg, e);
                if (!taken && (best < 0 || v > bv)) {
                    best = e;
                    bv = v;
                }
            }
            sel[s] = best;
            p[s] = expf(bv - mx) / sum;
            psum += p[s];
        }
        for (int s = 0; s < k; ++s) {
            const int a = t * k + s;
            expert_of[a] = sel[s];
            weight_of[a] = normalize ? p[s] / psum : p[s];
            sx[a] = (int16_t)sel[s];
        }
    }
    __syncthreads();
    const int R = T * k;
    for (int e = tid; e < E; e += kRouteThreads) {
        int c = 0;
        for (int a = 0; a < R; ++a) c += sx[a] == e;
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < E; ++e) {
            const int c = cnt[e];
            offsets[e] = run;
            cnt[e] = run;
            run += c;
        }
        offsets[E] = run;
    }
    __syncthreads();
    // assignments of expert e in ascending (token, slot) order
    for (int e = tid; e < E; e += kRouteThreads) {
        int pos = cnt[e];
        for (int a = 0; a < R; ++a) {
            if (sx[a] != e) continue;
            row_token[pos] = a / k;
            pos_of[a] = pos;
            expert_of_row[pos] = e;
            ++pos;
        }
    }
}

__global__ void __launch_bounds__(256)
qmoe_swiglu(const f16* __restrict__ h, const f16* __restrict__ b1,
            const int32_t* __restrict__ expert_of_row, f16* __restrict__ act, int64_t rows,
            int64_t inter, int fusion, float alpha, float beta, float limit, int has_limit) {
    const int64_t total = rows * inter;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t r = idx / inter;
        const int64_t i = idx - r * inter;
        const int64_t gi = fusion == 1 ? 2 * i : i;
        const int64_t li = fusion == 1 ? 2 * i + 1 : inter + i;
        const f16* hr = h + r * 2 * inter;
        float g = (float)hr[gi];
        float l = (float)hr[li];
        if (b1) {
            const f16* br = b1 + (int64_t)expert_of_row[r] * 2 * inter;
            g += (float)br[gi];
            l += (float)br[li];
        }
        if (has_limit) {
            g = fminf(g, limit);
            l = fminf(fmaxf(l, -limit), limit);
        }
        act[idx] = (f16)(g / (1.f + expf(-alpha * g)) * (l + beta));
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
        for (int s = 0; s < k; ++s) {
            const int64_t a = t * k + s;
            const float w = weight_of[a];
            const f16x8 v = *reinterpret_cast<const f16x8*>(o + (int64_t)pos_of[a] * hidden + c);
            if (b2) {
                const f16x8 bb =
                    *reinterpret_cast<const f16x8*>(b2 + (int64_t)expert_of[a] * hidden + c);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] += w * ((float)v[j] + (float)bb[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] += w * (float)v[j];
            }
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
                       const void* fc2_b, void* y, void* workspace, hipStream_t st) {
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
    const size_t route_lds = (size_t)R * sizeof(int16_t);
    if (q.router_f32)
        hipLaunchKernelGGL(qmoe_route<float>, dim3(1), dim3(kRouteThreads), route_lds, st,
                           static_cast<const float*>(logits), (int)q.rows, (int)q.experts, q.k,
                           q.normalize, expert_of, weight_of, offsets, row_token, pos_of,
                           expert_of_row);
    else
        hipLaunchKernelGGL(qmoe_route<f16>, dim3(1), dim3(kRouteThreads), route_lds, st,
                           static_cast<const f16*>(logits), (int)q.rows, (int)q.experts, q.k,
                           q.normalize, expert_of, weight_of, offsets, row_token, pos_of,
                           expert_of_row);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // expected rows per expert (twice the mean, at least one) sets the GEMV tile height
    const int64_t hint = std::max<int64_t>(1, 2 * ((R + q.experts - 1) / q.experts));
    e = launch_group_gemv_f16_bounded(x, row_token, offsets, q.experts, q.rows, hint, fc1, fc1_s,
                                      nullptr, h, R, 2 * q.inter, q.hidden, 4, q.block_size, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(qmoe_swiglu, dim3(grid_for(R * q.inter)), dim3(256), 0, st, h,
                       static_cast<const f16*>(fc1_b), expert_of_row, act, R, q.inter, q.fusion,
                       q.alpha, q.beta, q.limit, q.has_limit);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_group_gemv_f16_bounded(act, nullptr, offsets, q.experts, q.rows, hint, fc2, fc2_s,
                                      nullptr, o, R, q.hidden, q.inter, 4, q.block_size, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(qmoe_combine, dim3(grid_for(q.rows * (q.hidden / 8))), dim3(256), 0, st, o,
                       static_cast<const f16*>(fc2_b), expert_of, weight_of, pos_of,
                       static_cast<f16*>(y), q.rows, q.hidden, q.k);
    return hipGetLastError();
}

}  // namespace mnb
