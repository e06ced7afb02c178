// com.microsoft::GroupQueryAttention, packed QKV with fused half-rotation (neox) RoPE and a KV
// cache, fp16 tensors, fp32 softmax and accumulation.
//
// Semantics follow the reference kernel (rust/shaders/glsl/gqa_f16.comp, dispatched by
// rust/src/ops/attention.rs:388-735):
//   * packed_qkv [B, S, (Nq + 2 Nkv) D]; per batch past_len = seqlens_k[b] + 1 - S (at least 0);
//     query s sits at position tok_pos = past_len + s;
//   * RoPE on Q and the new K: pairs (x[i], x[i + rd/2]), i < rd/2, rotated by the cos/sin cache
//     rows at tok_pos; dims at or past rd are copied;
//   * the new K (rotated) and V are written to present at tok_pos when tok_pos < present_len;
//     under the growing convention (present is a separate buffer) present also receives the past
//     tokens [0, past_len);
//   * each query attends to keys [0, tok_pos] of KV head h / (Nq / Nkv): keys t < past_len from
//     the past buffer, later keys from this call's own (rotated) K and V — never read back from
//     present, so reads and writes never overlap, also when present aliases past.
//
// Bounds the reference leaves to the caller are clamped here so that every access stays inside
// the buffers the problem describes: past_len is clamped to [0, past_stride] and the cos/sin row
// to [0, max_seq - 1].
//
// Three kernels:
//   gqa_prep     RoPE and append: rotated Q in a per-KV-head row order (row r = s * G + g) as
//                fp16 high and low parts, the new K and V in a workspace [B, Nkv, S, D], and the
//                present writes.
//   gqa_attend   flash attention on v_mfma_f32_16x16x32_f16.  A workgroup takes 16 x W query rows
//                of one (batch, KV head) and walks 64-key blocks staged in LDS (K row-major, V
//                transposed).  Scores are computed transposed, S^T = K Q^T, so each lane holds one
//                query's 16 scores of a block: the softmax statistics stay per lane (two
//                shuffles per block) and P^T feeds the second MFMA (O^T = V^T P^T) straight from
//                registers.  Rows of a workgroup are the G query heads of every position, so one
//                K/V block serves all of them.  Long keys with few rows (decode) split the key
//                range over workgroups.  Q and P enter the MFMAs as fp16 high + low pairs (two
//                MFMAs each), so scores and weights keep fp32 precision as in the reference's
//                fp32 kernel; rounding either to one fp16 costs up to 6e-3 relative on outputs.
//   gqa_combine  merges the split partials (max, sum, unnormalised O) into attn_output.
#include <algorithm>

#include "mnb_common.hpp"
#include "mnb_launch.hpp"

namespace mnb {

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kBN = 64;            // keys per block
constexpr int kVP = kBN + 8;       // transposed-V row pitch in halves (conflict-free reads)
constexpr float kMasked = -1.0e30f;

struct GqaDims {
    int64_t S, R;                  // new tokens; query rows per (batch, KV head) = S * G
    int64_t past_stride, present_len, max_seq, chunk;
    int nq, nkv, G, rh, rot, row_blocks, splits, copy_past;
    int64_t work;                  // workgroups of gqa_attend
    int64_t q_elems;               // B * Nq * S * D: offset of the low halves of rotated Q
    float scale_log2;
};

__device__ __forceinline__ int64_t past_len_of(const int32_t* seqlens, int b, const GqaDims& g) {
    const int64_t p = (int64_t)seqlens[b] + 1 - g.S;
    return p < 0 ? 0 : (p > g.past_stride ? g.past_stride : p);
}

// LDS row of key kk within a 64-key block: the 16 keys one score MFMA reads (see gqa_attend)
// sit in 16 consecutive rows.
__device__ __forceinline__ int lds_row(int kk) {
    return (kk & ~31) | (((kk >> 2) & 1) << 4) | (((kk >> 3) & 3) << 2) | (kk & 3);
}

}  // namespace

__global__ void __launch_bounds__(256)
gqa_prep(const f16* __restrict__ qkv, const int32_t* __restrict__ seqlens,
         const f16* __restrict__ cosc, const f16* __restrict__ sinc, f16* __restrict__ qr,
         f16* __restrict__ kn, f16* __restrict__ vn, f16* pres_k, f16* pres_v, int64_t total,
         int D, GqaDims g) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int heads = g.nq + 2 * g.nkv;
    const int d = (int)(i % D);
    int64_t t = i / D;
    const int hh = (int)(t % heads);
    t /= heads;
    const int64_t s = t % g.S;
    const int b = (int)(t / g.S);
    const int64_t tp = past_len_of(seqlens, b, g) + s;
    const f16* row = qkv + (i - d);
    const f16 xv = row[d];
    if (hh >= g.nq + g.nkv) {                            // V: copied
        const int kvh = hh - g.nq - g.nkv;
        const int64_t bk = (int64_t)b * g.nkv + kvh;
        vn[(bk * g.S + s) * D + d] = xv;
        if (tp < g.present_len) pres_v[(bk * g.present_len + tp) * D + d] = xv;
        return;
    }
    float y = (float)xv;
    if (d < g.rot) {
        const int64_t pr = tp < g.max_seq ? tp : g.max_seq - 1;
        const int ri = d < g.rh ? d : d - g.rh;
        const float c = (float)cosc[pr * g.rh + ri];
        const float sn = (float)sinc[pr * g.rh + ri];
        y = d < g.rh ? y * c - (float)row[d + g.rh] * sn : y * c + (float)row[d - g.rh] * sn;
    }
    if (hh < g.nq) {                                     // Q: rotated, rows grouped per KV head
        const int kvh = hh / g.G;
        const int64_t r = s * g.G + (hh % g.G);
        const int64_t o = (((int64_t)b * g.nkv + kvh) * g.R + r) * D + d;
        const f16 hi = (f16)y;
        qr[o] = hi;                                      // y = hi + lo to 2^-22
        qr[o + g.q_elems] = (f16)(y - (float)hi);
        return;
    }
    const int kvh = hh - g.nq;                           // K: rotated
    const int64_t bk = (int64_t)b * g.nkv + kvh;
    kn[(bk * g.S + s) * D + d] = (f16)y;
    if (tp < g.present_len) pres_k[(bk * g.present_len + tp) * D + d] = (f16)y;
}

template <int D, int W>
__global__ void __launch_bounds__(64 * W)
gqa_attend(const f16* __restrict__ qr, const f16* __restrict__ past_k,
           const f16* __restrict__ past_v, const f16* __restrict__ kn,
           const f16* __restrict__ vn, const int32_t* __restrict__ seqlens,
           f16* __restrict__ out, f16* pres_k, f16* pres_v, float* __restrict__ part_o,
           float* __restrict__ part_ml, GqaDims g) {
    constexpr int KS = D / 32;                 // full k-steps of the score MFMA
    constexpr bool TAIL = (D % 32) != 0;       // one 16-deep step more
    constexpr int DT = D / 16;                 // 16-wide d tiles of O
    constexpr int KP = D + 8;                  // K row pitch in halves
    constexpr int CPR = D / 8;                 // 16-byte chunks per key row
    constexpr int NT = 64 * W;
    constexpr int KCH = kBN * CPR;
    constexpr int KIT = (KCH + NT - 1) / NT;
    constexpr int VITEMS = (kBN / 4) * CPR;    // 4 keys x 8 dims each
    constexpr int VIT = (VITEMS + NT - 1) / NT;
    constexpr bool PF = W > 1;                 // prefetch the next block during compute

    __shared__ __align__(16) f16 Ks[kBN * KP];
    __shared__ __align__(16) f16 Vt[D * kVP];

    // Work item: consecutive items (row blocks of one batch and KV head) share K and V, so they
    // are kept on one XCD (workgroups are dealt to the 8 XCDs round-robin).
    int64_t w = blockIdx.x;
    if ((g.work & 7) == 0) w = (w & 7) * (g.work >> 3) + (w >> 3);
    const int rb = g.row_blocks - 1 - (int)(w % g.row_blocks);   // longest rows first
    const int64_t t2 = w / g.row_blocks;
    const int split = (int)(t2 % g.splits);
    const int64_t bk = t2 / g.splits;
    const int b = (int)(bk / g.nkv);

    const int64_t past_len = past_len_of(seqlens, b, g);
    const int64_t r0 = (int64_t)rb * 16 * W;
    const int64_t r_hi = std::min<int64_t>(r0 + 16 * W, g.R);
    const int64_t key_end = past_len + (r_hi - 1) / g.G + 1;
    const int64_t k_begin = (int64_t)split * g.chunk;
    const int64_t k_stop = std::min<int64_t>(k_begin + g.chunk, key_end);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 15;
    const int grp = lane >> 4;
    const int64_t r = r0 + 16 * wave + j;
    const bool rvalid = r < g.R;
    const int64_t wr0 = r0 + 16 * wave;
    const bool wave_active = wr0 < g.R;

    if (k_begin >= k_stop) {                             // no keys in this split
        if (rvalid) {
            const int64_t prow = ((int64_t)split * (g.work / (g.splits * g.row_blocks)) + bk) * g.R + r;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<f32x4*>(part_o + prow * D + 16 * dt + 4 * grp) = f32x4{0, 0, 0, 0};
            if (grp == 0) {
                part_ml[2 * prow] = kMasked;
                part_ml[2 * prow + 1] = 0.f;
            }
        }
        return;
    }

    const int64_t rc = rvalid ? r : g.R - 1;
    const int64_t tp = past_len + rc / g.G;              // this lane's query position
    const int64_t tp_lo = past_len + wr0 / g.G;
    const int64_t tp_hi = past_len + (std::min<int64_t>(wr0 + 15, g.R - 1)) / g.G;

    // Q^T fragments (B operand of the score MFMA): query j, dims 32 ks + 8 grp .. + 7, as fp16
    // high and low parts (two MFMAs), so the scores carry the fp32 rotation of Q.
    f16x8 qf[2][KS > 0 ? KS : 1];
    h4 qt[2] = {};
#pragma unroll
    for (int hl = 0; hl < 2; ++hl) {
        const f16* qrow = qr + hl * g.q_elems + (bk * g.R + rc) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            qf[hl][ks] = rvalid ? *reinterpret_cast<const f16x8*>(qrow + 32 * ks + 8 * grp) : f16x8{};
        if constexpr (TAIL)
            qt[hl] = rvalid ? *reinterpret_cast<const h4*>(qrow + 32 * KS + 4 * grp) : h4{};
    }

    f32x4 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kMasked, l_run = 0.f;

    const bool copy = g.copy_past && rb == 0;
    const f16* pk_base = past_k + bk * g.past_stride * D;
    const f16* pv_base = past_v + bk * g.past_stride * D;
    const f16* kn_base = kn + (bk * g.S - past_len) * D;     // indexed by key t >= past_len
    const f16* vn_base = vn + (bk * g.S - past_len) * D;
    f16* prk = pres_k + bk * g.present_len * D;
    f16* prv = pres_v + bk * g.present_len * D;

    u32x4 kreg[PF ? KIT : 1];
    u32x4 vreg[PF ? VIT : 1][4];

    auto load = [&](int64_t kb) {
#pragma unroll
        for (int it = 0; it < KIT; ++it) {
            const int c = tid + NT * it;
            if (c < KCH) {
                const int64_t t = kb + c / CPR;
                const int part = c % CPR;
                kreg[it] = u32x4{0, 0, 0, 0};
                if (t < k_stop)
                    kreg[it] = *reinterpret_cast<const u32x4*>(
                        (t < past_len ? pk_base : kn_base) + t * D + 8 * part);
            }
        }
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int c = tid + NT * it;
            if (c < VITEMS) {
                const int kg = c & 15;
                const int dc = c >> 4;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t t = kb + 4 * kg + q;
                    vreg[it][q] = u32x4{0, 0, 0, 0};
                    if (t < k_stop)
                        vreg[it][q] = *reinterpret_cast<const u32x4*>(
                            (t < past_len ? pv_base : vn_base) + t * D + 8 * dc);
                }
            }
        }
    };

    auto store = [&](int64_t kb) {
#pragma unroll
        for (int it = 0; it < KIT; ++it) {
            const int c = tid + NT * it;
            if (c < KCH) {
                const int kk = c / CPR;
                const int part = c % CPR;
                *reinterpret_cast<u32x4*>(&Ks[lds_row(kk) * KP + 8 * part]) = kreg[it];
                const int64_t t = kb + kk;
                if (copy && t < past_len)
                    *reinterpret_cast<u32x4*>(prk + t * D + 8 * part) = kreg[it];
            }
        }
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int c = tid + NT * it;
            if (c < VITEMS) {
                const int kg = c & 15;
                const int dc = c >> 4;
                const f16x8 v0 = __builtin_bit_cast(f16x8, vreg[it][0]);
                const f16x8 v1 = __builtin_bit_cast(f16x8, vreg[it][1]);
                const f16x8 v2 = __builtin_bit_cast(f16x8, vreg[it][2]);
                const f16x8 v3 = __builtin_bit_cast(f16x8, vreg[it][3]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const h4 col = {v0[e], v1[e], v2[e], v3[e]};
                    *reinterpret_cast<h4*>(&Vt[(8 * dc + e) * kVP + 4 * kg]) = col;
                }
                if (copy) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int64_t t = kb + 4 * kg + q;
                        if (t < past_len)
                            *reinterpret_cast<u32x4*>(prv + t * D + 8 * dc) = vreg[it][q];
                    }
                }
            }
        }
    };

    auto compute = [&](int64_t kb) {
        // S^T tiles: c2 = 32-key half, a = 16-key MFMA tile.  Lane (j, grp) ends up with the
        // scores of query j and keys kb + 32 c2 + 8 grp + 4 a + i.
        f32x4 sc[2][2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const f16* krow = &Ks[(32 * c2 + 16 * a + j) * KP];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const f16x8 kf = *reinterpret_cast<const f16x8*>(krow + 32 * ks + 8 * grp);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[0][ks], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[1][ks], acc, 0, 0, 0);
                }
                if constexpr (TAIL) {
                    const h4 kf = *reinterpret_cast<const h4*>(krow + 32 * KS + 4 * grp);
                    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kf, qt[0], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kf, qt[1], acc, 0, 0, 0);
                }
                sc[c2][a] = acc;
            }
        const bool need_mask = kb + kBN - 1 > tp_lo;
        float mloc = kMasked;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float x = sc[c2][a][i] * g.scale_log2;
                    if (need_mask && kb + 32 * c2 + 8 * grp + 4 * a + i > tp) x = kMasked;
                    sc[c2][a][i] = x;
                    mloc = fmaxf(mloc, x);
                }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            f16x8 pb, pl;                                // P = pb + pl to 2^-22
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(sc[c2][a][i] - m_new);
                    l_run += p;
                    const f16 hi = (f16)p;
                    pb[4 * a + i] = hi;
                    pl[4 * a + i] = (f16)(p - (float)hi);
                }
            // O^T += V^T P^T over keys kb + 32 c2 + 8 grp .. + 7.
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const f16x8 vf =
                    *reinterpret_cast<const f16x8*>(&Vt[(16 * dt + j) * kVP + 32 * c2 + 8 * grp]);
                oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb, oacc[dt], 0, 0, 0);
                oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl, oacc[dt], 0, 0, 0);
            }
        }
    };

    // Single-wave workgroups copy a block through a few registers at a time (holding a whole
    // block would take 2 x 64 x D / 64 x 2 bytes per lane).
    auto stream_copy = [&](int64_t kb) {
#pragma unroll 4
        for (int c = tid; c < KCH; c += NT) {
            const int kk = c / CPR;
            const int part = c % CPR;
            const int64_t t = kb + kk;
            u32x4 v = {0, 0, 0, 0};
            if (t < k_stop)
                v = *reinterpret_cast<const u32x4*>((t < past_len ? pk_base : kn_base) + t * D +
                                                    8 * part);
            *reinterpret_cast<u32x4*>(&Ks[lds_row(kk) * KP + 8 * part]) = v;
            if (copy && t < past_len) *reinterpret_cast<u32x4*>(prk + t * D + 8 * part) = v;
        }
#pragma unroll 2
        for (int c = tid; c < VITEMS; c += NT) {
            const int kg = c & 15;
            const int dc = c >> 4;
            u32x4 vr[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t t = kb + 4 * kg + q;
                vr[q] = u32x4{0, 0, 0, 0};
                if (t < k_stop)
                    vr[q] = *reinterpret_cast<const u32x4*>((t < past_len ? pv_base : vn_base) +
                                                            t * D + 8 * dc);
            }
            const f16x8 v0 = __builtin_bit_cast(f16x8, vr[0]);
            const f16x8 v1 = __builtin_bit_cast(f16x8, vr[1]);
            const f16x8 v2 = __builtin_bit_cast(f16x8, vr[2]);
            const f16x8 v3 = __builtin_bit_cast(f16x8, vr[3]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const h4 col = {v0[e], v1[e], v2[e], v3[e]};
                *reinterpret_cast<h4*>(&Vt[(8 * dc + e) * kVP + 4 * kg]) = col;
            }
            if (copy) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t t = kb + 4 * kg + q;
                    if (t < past_len) *reinterpret_cast<u32x4*>(prv + t * D + 8 * dc) = vr[q];
                }
            }
        }
    };

    const int64_t nblk = (k_stop - k_begin + kBN - 1) / kBN;
    if constexpr (PF) load(k_begin);
    for (int64_t ib = 0; ib < nblk; ++ib) {
        const int64_t kb = k_begin + ib * kBN;
        if (ib) __syncthreads();                         // the previous block is consumed
        if constexpr (PF) store(kb);
        else stream_copy(kb);
        __syncthreads();
        if constexpr (PF) {
            if (ib + 1 < nblk) load(kb + kBN);
        }
        if (wave_active && kb <= tp_hi) compute(kb);
    }

    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (!rvalid) return;
    if (g.splits == 1) {
        const int64_t s = r / g.G;
        const int h = (int)(bk % g.nkv) * g.G + (int)(r % g.G);
        f16* o = out + (((int64_t)b * g.S + s) * g.nq + h) * D + 4 * grp;
        const float inv = 1.f / l_run;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const h4 v = {(f16)(oacc[dt][0] * inv), (f16)(oacc[dt][1] * inv),
                          (f16)(oacc[dt][2] * inv), (f16)(oacc[dt][3] * inv)};
            *reinterpret_cast<h4*>(o + 16 * dt) = v;
        }
        return;
    }
    const int64_t bks = g.work / ((int64_t)g.splits * g.row_blocks);
    const int64_t prow = ((int64_t)split * bks + bk) * g.R + r;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(part_o + prow * D + 16 * dt + 4 * grp) = oacc[dt];
    if (grp == 0) {
        part_ml[2 * prow] = m_run;
        part_ml[2 * prow + 1] = l_run;
    }
}

// One thread per (batch x KV head x row, 4 dims).
__global__ void __launch_bounds__(256)
gqa_combine(const float* __restrict__ part_o, const float* __restrict__ part_ml,
            f16* __restrict__ out, int64_t rows, int D, GqaDims g) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int quads = D / 4;
    if (i >= rows * quads) return;
    const int64_t row = i / quads;
    const int q = (int)(i % quads);
    float m = kMasked;
    for (int sp = 0; sp < g.splits; ++sp) m = fmaxf(m, part_ml[2 * (sp * rows + row)]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
    for (int sp = 0; sp < g.splits; ++sp) {
        const int64_t pr = sp * rows + row;
        const float wgt = __builtin_amdgcn_exp2f(part_ml[2 * pr] - m);
        l += wgt * part_ml[2 * pr + 1];
        acc += wgt * *reinterpret_cast<const f32x4*>(part_o + pr * D + 4 * q);
    }
    const float inv = 1.f / l;
    const int64_t bk = row / g.R;
    const int64_t r = row % g.R;
    const int b = (int)(bk / g.nkv);
    const int h = (int)(bk % g.nkv) * g.G + (int)(r % g.G);
    const int64_t s = r / g.G;
    const h4 v = {(f16)(acc[0] * inv), (f16)(acc[1] * inv), (f16)(acc[2] * inv),
                  (f16)(acc[3] * inv)};
    *reinterpret_cast<h4*>(out + (((int64_t)b * g.S + s) * g.nq + h) * D + 4 * q) = v;
}

bool gqa_supported(int head_dim) { return head_dim >= 16 && head_dim <= 256 && head_dim % 16 == 0; }

GqaPlan gqa_plan(const GqaArgs& a) {
    GqaPlan p{};
    const int64_t G = a.nq / a.nkv;
    const int64_t R = a.seq * G;
    const int64_t bk = a.batch * a.nkv;
    p.waves = R > 16 ? 4 : 1;
    p.row_blocks = (R + 16 * p.waves - 1) / (16 * p.waves);
    const int64_t base = bk * p.row_blocks;
    const int64_t t_max = a.past_stride + a.seq;        // bound on keys per query
    p.splits = 1;
    p.chunk = (t_max + kBN - 1) / kBN * kBN;
    if (base < 512 && t_max > 2 * kBN) {
        const int64_t want = (512 + base - 1) / base;
        int64_t chunk = (t_max + want - 1) / want;
        chunk = std::max<int64_t>(2 * kBN, (chunk + kBN - 1) / kBN * kBN);
        const int64_t splits = std::min<int64_t>((t_max + chunk - 1) / chunk, 64);
        chunk = std::max<int64_t>(chunk, ((t_max + splits - 1) / splits + kBN - 1) / kBN * kBN);
        p.splits = (int)((t_max + chunk - 1) / chunk);
        p.chunk = chunk;
    }
    return p;
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t gqa_workspace_bytes(const GqaArgs& a) {
    const GqaPlan p = gqa_plan(a);
    const size_t q = (size_t)a.batch * a.nq * a.seq * a.d;
    const size_t kv = (size_t)a.batch * a.nkv * a.seq * a.d;
    size_t n = al256(q * 4) + 2 * al256(kv * 2);     // rotated Q as fp16 high and low parts
    if (p.splits > 1) n += al256((size_t)p.splits * q * 4) + al256((size_t)p.splits * (q / a.d) * 8);
    return n;
}

template <int D, int W>
static void attend_go(const GqaDims& g, const f16* qr, const void* pk, const void* pv,
                      const f16* kn, const f16* vn, const int32_t* seqlens, void* out, void* prk,
                      void* prv, float* po, float* pml, hipStream_t st) {
    hipLaunchKernelGGL((gqa_attend<D, W>), dim3((unsigned)g.work), dim3(64 * W), 0, st, qr,
                       static_cast<const f16*>(pk), static_cast<const f16*>(pv), kn, vn, seqlens,
                       static_cast<f16*>(out), static_cast<f16*>(prk), static_cast<f16*>(prv), po,
                       pml, g);
}

template <int D>
static void attend_w(int waves, const GqaDims& g, const f16* qr, const void* pk, const void* pv,
                     const f16* kn, const f16* vn, const int32_t* seqlens, void* out, void* prk,
                     void* prv, float* po, float* pml, hipStream_t st) {
    if (waves == 4) attend_go<D, 4>(g, qr, pk, pv, kn, vn, seqlens, out, prk, prv, po, pml, st);
    else attend_go<D, 1>(g, qr, pk, pv, kn, vn, seqlens, out, prk, prv, po, pml, st);
}

hipError_t launch_gqa(const GqaArgs& a, const void* qkv, const void* past_k, const void* past_v,
                      const int32_t* seqlens, const void* cos_cache, const void* sin_cache,
                      void* out, void* pres_k, void* pres_v, void* workspace, hipStream_t st) {
    if (!gqa_supported(a.d) || a.nkv <= 0 || a.nq % a.nkv) return hipErrorInvalidValue;
    if (a.batch == 0 || a.seq == 0) return hipSuccess;
    const GqaPlan p = gqa_plan(a);
    GqaDims g{};
    g.S = a.seq;
    g.G = a.nq / a.nkv;
    g.R = a.seq * g.G;
    g.past_stride = a.past_stride;
    g.present_len = a.present_len;
    g.max_seq = a.max_seq;
    g.chunk = p.chunk;
    g.nq = a.nq;
    g.nkv = a.nkv;
    g.rh = a.rot / 2;
    g.rot = a.rot;
    g.row_blocks = (int)p.row_blocks;
    g.splits = p.splits;
    g.copy_past = a.copy_past ? 1 : 0;
    g.work = a.batch * a.nkv * p.row_blocks * p.splits;
    g.scale_log2 = a.scale * 1.4426950408889634f;
    g.q_elems = (int64_t)((size_t)a.batch * a.nq * a.seq * a.d);

    const size_t q = (size_t)a.batch * a.nq * a.seq * a.d;
    const size_t kv = (size_t)a.batch * a.nkv * a.seq * a.d;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    f16* qr = reinterpret_cast<f16*>(ws);
    ws += al256(q * 4);
    f16* kn = reinterpret_cast<f16*>(ws);
    ws += al256(kv * 2);
    f16* vn = reinterpret_cast<f16*>(ws);
    ws += al256(kv * 2);
    float* po = nullptr;
    float* pml = nullptr;
    if (p.splits > 1) {
        po = reinterpret_cast<float*>(ws);
        ws += al256((size_t)p.splits * q * 4);
        pml = reinterpret_cast<float*>(ws);
    }

    const int64_t prep_total = a.batch * a.seq * (int64_t)(a.nq + 2 * a.nkv) * a.d;
    hipLaunchKernelGGL(gqa_prep, dim3((unsigned)((prep_total + 255) / 256)), dim3(256), 0, st,
                       static_cast<const f16*>(qkv), seqlens, static_cast<const f16*>(cos_cache),
                       static_cast<const f16*>(sin_cache), qr, kn, vn, static_cast<f16*>(pres_k),
                       static_cast<f16*>(pres_v), prep_total, a.d, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    switch (a.d) {
#define MNB_GQA_D(DD) \
    case DD: attend_w<DD>(p.waves, g, qr, past_k, past_v, kn, vn, seqlens, out, pres_k, pres_v, po, pml, st); break;
        MNB_GQA_D(16) MNB_GQA_D(32) MNB_GQA_D(48) MNB_GQA_D(64) MNB_GQA_D(80) MNB_GQA_D(96)
        MNB_GQA_D(112) MNB_GQA_D(128) MNB_GQA_D(144) MNB_GQA_D(160) MNB_GQA_D(176)
        MNB_GQA_D(192) MNB_GQA_D(208) MNB_GQA_D(224) MNB_GQA_D(240) MNB_GQA_D(256)
#undef MNB_GQA_D
        default: return hipErrorInvalidValue;
    }
    e = hipGetLastError();
    if (e != hipSuccess || p.splits == 1) return e;
    const int64_t rows = a.batch * a.nkv * g.R;
    const int64_t n = rows * (a.d / 4);
    hipLaunchKernelGGL(gqa_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, po, pml,
                       static_cast<f16*>(out), rows, a.d, g);
    return hipGetLastError();
}

}  // namespace mnb
