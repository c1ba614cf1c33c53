/*
 * oracle/orc.c -- CPU restatement of MLXR's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (mlxr_amd/, include/)
 * links, loads or calls this file.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline.
 *
 * What it restates (paths relative to the reference repository root):
 *   - fp16 -> fp32                core/kernels/primitives/q_gemm_dequant_primitive.mm:141-165
 *   - block layouts               q_gemm_dequant_primitive.mm:40-57, q_gemm_dequant.metal:97-131
 *   - Q8_0 dequant                q_gemm_dequant_primitive.mm:218-225 (identical formula)
 *   - Q4_0 / Q4_1 dequant         q_gemm_dequant_primitive.mm:189-216 (same formulas,
 *                                 (q - 8) * d and q * d + m, but in the GGUF element order;
 *                                 the reference's interleaved order is kept as
 *                                 orc_dequant_refcpu_q4 and its relation pinned in tests)
 *   - Q4_K / Q5_K / Q6_K dequant  canonical GGUF block_q4_K / q5_K / q6_K semantics (the
 *                                 reference's only K-quant routines are the Metal ones at
 *                                 q_gemm_dequant.metal:214-286, which are not GGUF-conformant;
 *                                 the GGUF description is the contract these follow)
 *   - eval_cpu                    q_gemm_dequant_primitive.mm:299-365 (dequant all of W to
 *                                 fp32, then a naive single-thread fp32 m/n/k loop, + bias)
 *   - tensor sizes                q_gemm_dequant_primitive.mm:116-135,
 *                                 daemon/registry/gguf_parser.cpp:179-241 (with Q6_K = 210)
 *
 * Pinning (see tests/test_oracle.py): fp16->fp32 exhaustively against numpy;
 * bf16/fp16 RNE against numpy/torch casts; Q8_0/Q4_K/Q6_K dequant against an
 * independent per-element decoder and hand-derived known answers (one-hot scale
 * bits, single-bit ql/qh patterns, extreme scales); GEMM against fp64
 * numpy/torch matmul of the dequantized weights and integer-weight special cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256

enum { Q4_0 = 0, Q4_1 = 1, Q8_0 = 2, Q4_K = 3, Q6_K = 4, Q5_K = 10 };

/* ---------------------------------------------------------------- fp16/bf16 */

/* Exact IEEE binary16 -> binary32 (subnormals, +-0, +-inf; NaN stays NaN).
 * Same results as q_gemm_dequant_primitive.mm:141-165, written on bits. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24 is exact in fp32 */
            float f = (float)m * 0x1p-24f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* The reference's own formulation (powf based), kept to show it agrees with the
 * bit-level conversion on every code (q_gemm_dequant_primitive.mm:141-165). */
float orc_ref_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, exponent = (h >> 10) & 0x1fu, mantissa = h & 0x3ffu;
    if (exponent == 0) {
        if (mantissa == 0) return sign ? -0.0f : 0.0f;
        float r = mantissa / 1024.0f;
        r *= powf(2.0f, -14.0f);
        return sign ? -r : r;
    } else if (exponent == 31) {
        return mantissa ? NAN : (sign ? -INFINITY : INFINITY);
    }
    float r = 1.0f + mantissa / 1024.0f;
    r *= powf(2.0f, (int)exponent - 15);
    return sign ? -r : r;
}

/* fp32 -> binary16, round to nearest even, with subnormals and overflow to inf. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* result is subnormal or zero: value / 2^-24, RNE */
        float a;
        memcpy(&a, &ax, 4);
        double q = (double)a * 16777216.0; /* exact */
        double fl = floor(q);
        double rem = q - fl;
        uint32_t r = (uint32_t)fl;
        if (rem > 0.5 || (rem == 0.5 && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t e = (ax >> 23) - 112u, m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* fp32 -> bfloat16, round to nearest even; NaN -> quiet NaN of the same sign. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

/* ------------------------------------------------------------------- sizes */

int orc_block_elems(int qtype) {
    switch (qtype) {
    case Q4_0: case Q4_1: case Q8_0: return 32;
    case Q4_K: case Q6_K: case Q5_K: return QK_K;
    default: return 0;
    }
}

int orc_block_bytes(int qtype) {
    switch (qtype) {
    case Q4_0: return 18;
    case Q4_1: return 20;
    case Q8_0: return 34;
    case Q4_K: return 144;
    case Q6_K: return 210;
    case Q5_K: return 176;
    default: return 0;
    }
}

/* N * ceil(K / group) * sizeof(block)  (q_gemm_dequant_primitive.mm:116-135). */
uint64_t orc_weight_bytes(int qtype, int N, int K) {
    int g = orc_block_elems(qtype);
    if (g == 0) return 0;
    return (uint64_t)N * (uint64_t)((K + g - 1) / g) * (uint64_t)orc_block_bytes(qtype);
}

/* ------------------------------------------------------------------ dequant */

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* block_q8_0 = { fp16 d; int8 qs[32]; }   w[i] = qs[i] * fp32(d)   (exact) */
static void dq_q8_0(const uint8_t* blk, float* y) {
    float d = orc_f16_to_f32(rd16(blk));
    const int8_t* qs = (const int8_t*)(blk + 2);
    for (int i = 0; i < 32; i++) y[i] = (float)qs[i] * d;
}

/* block_q4_0 = { fp16 d; u8 qs[16]; }  GGUF order: byte j holds element j (low nibble) and
 * element j+16 (high nibble).  w = (q - 8) * fp32(d), exact (q - 8 has 4 bits). */
static void dq_q4_0(const uint8_t* blk, float* y) {
    float d = orc_f16_to_f32(rd16(blk));
    const uint8_t* qs = blk + 2;
    for (int j = 0; j < 16; j++) {
        y[j] = (float)((int)(qs[j] & 0x0f) - 8) * d;
        y[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
    }
}

/* block_q4_1 = { fp16 d; fp16 m; u8 qs[16]; }  GGUF order as Q4_0.  w = q * d + m: the
 * product is exact, so the one rounding is the addition (same with or without fma). */
static void dq_q4_1(const uint8_t* blk, float* y) {
    float d = orc_f16_to_f32(rd16(blk));
    float m = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* qs = blk + 4;
    for (int j = 0; j < 16; j++) {
        y[j] = (float)(qs[j] & 0x0f) * d + m;
        y[j + 16] = (float)(qs[j] >> 4) * d + m;
    }
}

/* The reference's own CPU routines dequant_q4_0_cpu / dequant_q4_1_cpu
 * (q_gemm_dequant_primitive.mm:189-216) read the nibbles interleaved: byte i holds
 * elements 2i (low) and 2i+1 (high).  Same values, different element order from GGUF;
 * kept to document that divergence (tests pin the permutation between the two). */
int orc_dequant_refcpu_q4(int qtype, const uint8_t* blk, float* y) {
    if (qtype != Q4_0 && qtype != Q4_1) return -1;
    float d = orc_f16_to_f32(rd16(blk));
    float m = qtype == Q4_1 ? orc_f16_to_f32(rd16(blk + 2)) : 0.0f;
    const uint8_t* qs = blk + (qtype == Q4_1 ? 4 : 2);
    for (int i = 0; i < 16; i++) {
        if (qtype == Q4_0) {
            y[2 * i] = (float)((int)(qs[i] & 0x0f) - 8) * d;
            y[2 * i + 1] = (float)((int)(qs[i] >> 4) - 8) * d;
        } else {
            y[2 * i] = (float)(qs[i] & 0x0f) * d + m;
            y[2 * i + 1] = (float)(qs[i] >> 4) * d + m;
        }
    }
    return 0;
}

/* 6-bit scale and min of sub-block j (0..7) from the 12 packed bytes. */
void orc_q4k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* block_q4_K = { fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]; }
 * For 64-element chunk c: qs[32c+l] low nibble -> element 64c+l (sub-block 2c),
 * high nibble -> element 64c+32+l (sub-block 2c+1).
 * w = (d*sc)*q - (dmin*m), evaluated in fp32: both products are exact, so the
 * only rounding is the subtraction. */
static void dq_q4_k(const uint8_t* blk, float* y) {
    float d = orc_f16_to_f32(rd16(blk));
    float dmin = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    const uint8_t* q = blk + 16;
    for (int c = 0; c < 4; c++) {
        int sc0, m0, sc1, m1;
        orc_q4k_scale_min(s, 2 * c, &sc0, &m0);
        orc_q4k_scale_min(s, 2 * c + 1, &sc1, &m1);
        float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            y[64 * c + l] = d0 * (float)(q[32 * c + l] & 0x0f) - mm0;
            y[64 * c + 32 + l] = d1 * (float)(q[32 * c + l] >> 4) - mm1;
        }
    }
}

/* block_q5_K = { fp16 d; fp16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]; }
 * As Q4_K (same 12-byte scale/min packing, same qs nibble order), plus a fifth bit:
 * element 64c+l (l < 32) takes bit 2c of qh[l], element 64c+32+l bit 2c+1.
 * w = (d*sc)*q - (dmin*m) with q in 0..31: both products exact, one rounding. */
static void dq_q5_k(const uint8_t* blk, float* y) {
    float d = orc_f16_to_f32(rd16(blk));
    float dmin = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* q = blk + 48;
    for (int c = 0; c < 4; c++) {
        int sc0, m0, sc1, m1;
        orc_q4k_scale_min(s, 2 * c, &sc0, &m0);
        orc_q4k_scale_min(s, 2 * c + 1, &sc1, &m1);
        float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            int lo = (q[32 * c + l] & 0x0f) | (((qh[l] >> (2 * c)) & 1) << 4);
            int hi = (q[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
            y[64 * c + l] = d0 * (float)lo - mm0;
            y[64 * c + 32 + l] = d1 * (float)hi - mm1;
        }
    }
}

/* block_q6_K = { u8 ql[128]; u8 qh[64]; int8 scales[16]; fp16 d; }
 * Two 128-element halves; in half h, for l in 0..31 and quarter t in 0..3 the
 * element 128h+32t+l takes its low 4 bits from ql[64h + l + 32(t&1)] (low nibble
 * for t<2, high nibble for t>=2), its high 2 bits from qh[32h+l] bits 2t..2t+1,
 * and its scale from scales[(128h+32t+l)/16].  w = d * sc * (q - 32), exact. */
static void dq_q6_k(const uint8_t* blk, float* y) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    float d = orc_f16_to_f32(rd16(blk + 208));
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = d * (float)sc[is + 0] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* Dequantize an [N, K] GGUF weight (row-major blocks) to fp32 [N, K].
 * Returns 0 on success, -1 for an unsupported type or K not a block multiple. */
int orc_dequant(int qtype, int N, int K, const uint8_t* w, float* out) {
    int g = orc_block_elems(qtype), bb = orc_block_bytes(qtype);
    if (g == 0 || K % g != 0) return -1;
    int nb = K / g;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)n * nb + b) * bb;
            float* y = out + (size_t)n * K + (size_t)b * g;
            if (qtype == Q8_0) dq_q8_0(blk, y);
            else if (qtype == Q4_0) dq_q4_0(blk, y);
            else if (qtype == Q4_1) dq_q4_1(blk, y);
            else if (qtype == Q4_K) dq_q4_k(blk, y);
            else if (qtype == Q5_K) dq_q5_k(blk, y);
            else dq_q6_k(blk, y);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------- GEMMs */

/* Restatement of QGemmDequantPrimitive::eval_cpu (q_gemm_dequant_primitive.mm:299-365):
 * dequantize ALL of W to fp32, then y[m,n] = sum_k x[m,k]*w[n,k] in fp32, k ascending,
 * single thread, then + bias[n].  The reference supports Q4_0/Q4_1/Q8_0 there and throws
 * for K-quants; this restatement extends it to Q4_K/Q6_K with the canonical dequant so
 * that the same CPU path can be timed on every configuration. */
int orc_eval_cpu(int qtype, int M, int N, int K, const uint8_t* w, const float* x,
                 const float* bias, float* y) {
    float* wd = (float*)malloc(sizeof(float) * (size_t)N * (size_t)K);
    if (!wd) return -2;
    int rc = orc_dequant(qtype, N, K, w, wd);
    if (rc) {
        free(wd);
        return rc;
    }
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            const float* xr = x + (size_t)m * K;
            const float* wr = wd + (size_t)n * K;
            for (int k = 0; k < K; k++) acc += xr[k] * wr[k];
            if (bias) acc += bias[n];
            y[(size_t)m * N + n] = acc;
        }
    }
    free(wd);
    return 0;
}

/* Same as orc_eval_cpu but only output columns [n0, n1) (used to time a bounded
 * sample of a large configuration).  The dequant covers only those rows as well. */
int orc_eval_cpu_cols(int qtype, int M, int N, int K, int n0, int n1, const uint8_t* w,
                      const float* x, const float* bias, float* y) {
    if (n0 < 0 || n1 > N || n0 >= n1) return -1;
    const uint8_t* wsub = w + orc_weight_bytes(qtype, n0, K);
    int ns = n1 - n0;
    float* ysub = (float*)malloc(sizeof(float) * (size_t)M * ns);
    if (!ysub) return -2;
    int rc = orc_eval_cpu(qtype, M, ns, K, wsub, x, bias ? bias + n0 : NULL, ysub);
    if (rc == 0)
        for (int m = 0; m < M; m++) memcpy(y + (size_t)m * N + n0, ysub + (size_t)m * ns, sizeof(float) * ns);
    free(ysub);
    return rc;
}

/* Tolerance oracle: y[m,n] = sum_k x[m,k] * w[n,k] accumulated in fp64 over the fp32
 * dequantized weights (optionally rounded to bf16 first, which is what an MFMA path
 * consumes), plus bias; the fp64 sum is rounded once to fp32.  Rows of y in [m0, m1). */
int orc_gemm_f64(int qtype, int M, int N, int K, const uint8_t* w, const float* x,
                 const float* bias, int w_to_bf16, int m0, int m1, float* y) {
    if (m0 < 0 || m1 > M || m0 > m1) return -1;
    float* wd = (float*)malloc(sizeof(float) * (size_t)N * (size_t)K);
    if (!wd) return -2;
    int rc = orc_dequant(qtype, N, K, w, wd);
    if (rc) {
        free(wd);
        return rc;
    }
    /* w_to_bf16: 1 rounds the weights to bf16 (RNE), 2 to fp16 (RNE): the operands the
       MFMA paths multiply for bf16 and fp16 activations */
    if (w_to_bf16 == 1) {
#pragma omp parallel for schedule(static)
        for (long long i = 0; i < (long long)N * K; i++) wd[i] = orc_bf16_to_f32(orc_f32_to_bf16(wd[i]));
    } else if (w_to_bf16 == 2) {
#pragma omp parallel for schedule(static)
        for (long long i = 0; i < (long long)N * K; i++) wd[i] = orc_f16_to_f32(orc_f32_to_f16(wd[i]));
    }
#pragma omp parallel for schedule(dynamic, 16)
    for (int n = 0; n < N; n++) {
        const float* wr = wd + (size_t)n * K;
        for (int m = m0; m < m1; m++) {
            const float* xr = x + (size_t)m * K;
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += (double)xr[k] * (double)wr[k];
            if (bias) acc += (double)bias[n];
            y[(size_t)(m - m0) * N + n] = (float)acc;
        }
    }
    free(wd);
    return 0;
}
