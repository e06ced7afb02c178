/*
 * CPU restatement of com.microsoft::MatMulNBits in plain C — TEST INFRASTRUCTURE, NOT PRODUCT.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and
 * only as the checker (or, in bench.py, as the reported CPU baseline of kind "port").  The
 * product path never links it.
 *
 * Semantics (reference paths relative to the reference checkout):
 *   B       [N][bpc][bs*bits/8] bytes, row n is output column n   (docs/OP_COVERAGE.md:4210-4230)
 *   4-bit   element 2i = byte[i] & 0xF, element 2i+1 = byte[i] >> 4  (q_gemv.comp:315-329)
 *   zp      packed like B, per-column runs padded to a byte; absent => 1 << (bits-1)
 *                                                                  (q_gemv.comp:284-306, quant.rs:684-705)
 *   scales  index n*bpc + blk                                      (q_gemv.comp:71-84)
 *   W[n][k] = (q - zp) * s, Y[m][n] = sum_k A[m][k] * W[n][k]
 *
 * Arithmetic order follows ORT's SQNBIT_CompFp32 shape (third-party ONNX Runtime v1.28.0, not in
 * the reference tree): each (column, block) is dequantised to fp32 once, then multiplied into
 * fp32 accumulators for every row.  fp16 inputs are widened with a software fp16->fp32 (exact).
 *
 * Build: see oracle/Makefile (gcc -O3 -fopenmp, shared library).
 */
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Exact IEEE binary16 -> binary32 widening (subnormals, inf and NaN included). */
static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (for writing fp16 outputs). */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax < 0x38800000u) { /* below fp16 min normal: subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        /* a * 2^24 rounded to nearest even integer gives the subnormal mantissa */
        float m = a * 16777216.0f;
        float r = nearbyintf(m);
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static inline int zp_value(const uint8_t* zp, int64_t n, int64_t blk, int64_t bpc, int bits) {
    if (!zp) return 1 << (bits - 1);
    int64_t zpb = (bpc * bits + 7) / 8;
    if (bits == 4) {
        uint8_t b = zp[n * zpb + (blk >> 1)];
        return (blk & 1) ? (b >> 4) : (b & 0xF);
    }
    return zp[n * zpb + blk];
}

/* Dequantise one (column, block) into w[0..bs). */
static inline void dequant_block(const uint8_t* B, const float s, int z, int64_t n, int64_t blk,
                                 int64_t bpc, int bits, int bs, float* w) {
    const int blob = bs * bits / 8;
    const uint8_t* p = B + (n * bpc + blk) * blob;
    if (bits == 4) {
        for (int i = 0; i < blob; ++i) {
            w[2 * i] = (float)((int)(p[i] & 0xF) - z) * s;
            w[2 * i + 1] = (float)((int)(p[i] >> 4) - z) * s;
        }
    } else {
        for (int i = 0; i < blob; ++i) w[i] = (float)((int)p[i] - z) * s;
    }
}

/*
 * Y = A @ dequant(B)^T.  a_is_f16 selects fp16 (uint16 bits) vs fp32 for A, scales and Y.
 * threads <= 0 means "use the OpenMP default".  Returns 0 on success.
 */
int mnb_oracle_matmul(const void* A, const uint8_t* B, const void* scales, const uint8_t* zp,
                      void* Y, int64_t M, int64_t N, int64_t K, int bits, int bs, int a_is_f16,
                      int threads) {
    if (M < 0 || N <= 0 || K <= 0 || (bits != 4 && bits != 8) || bs <= 0 || K % bs) return 1;
    const int64_t bpc = K / bs;
    float* a32 = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M * K : 1));
    if (!a32) return 2;
    for (int64_t i = 0; i < M * K; ++i)
        a32[i] = a_is_f16 ? f16_to_f32(((const uint16_t*)A)[i]) : ((const float*)A)[i];
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        float w[128];
        float* acc = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t m = 0; m < M; ++m) acc[m] = 0.0f;
            for (int64_t blk = 0; blk < bpc; ++blk) {
                float s = a_is_f16 ? f16_to_f32(((const uint16_t*)scales)[n * bpc + blk])
                                   : ((const float*)scales)[n * bpc + blk];
                dequant_block(B, s, zp_value(zp, n, blk, bpc, bits), n, blk, bpc, bits, bs, w);
                for (int64_t m = 0; m < M; ++m) {
                    const float* ar = a32 + m * K + blk * bs;
                    float t = 0.0f;
                    for (int i = 0; i < bs; ++i) t += ar[i] * w[i];
                    acc[m] += t;
                }
            }
            for (int64_t m = 0; m < M; ++m) {
                if (a_is_f16) ((uint16_t*)Y)[m * N + n] = f32_to_f16(acc[m]);
                else ((float*)Y)[m * N + n] = acc[m];
            }
        }
        free(acc);
    }
    free(a32);
    return 0;
}

/* fp16 dequantised weight [N][K] (uint16 bits): fp16_rne(fp32(q - zp) * fp32(s)). */
int mnb_oracle_dequant_f16(const uint8_t* B, const uint16_t* scales, const uint8_t* zp,
                           uint16_t* W, int64_t N, int64_t K, int bits, int bs) {
    if (N <= 0 || K <= 0 || (bits != 4 && bits != 8) || bs <= 0 || K % bs) return 1;
    const int64_t bpc = K / bs;
    float w[128];
    for (int64_t n = 0; n < N; ++n)
        for (int64_t blk = 0; blk < bpc; ++blk) {
            float s = f16_to_f32(scales[n * bpc + blk]);
            dequant_block(B, s, zp_value(zp, n, blk, bpc, bits), n, blk, bpc, bits, bs, w);
            for (int i = 0; i < bs; ++i) W[n * K + blk * bs + i] = f32_to_f16(w[i]);
        }
    return 0;
}

/* Software fp16 conversions exposed for the oracle's own pinning tests. */
float mnb_oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t mnb_oracle_f32_to_f16(float f) { return f32_to_f16(f); }

int mnb_oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
