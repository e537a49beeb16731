/*
 * fg_oracle.c - CPU restatement of fastgguf's quantized weight x Q8-activation hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP backend (see fg_oracle.h). It is
 * never linked into, called by, or used as a fallback of the product library.
 *
 * Written from the reference's formulas; each function cites the fastgguf.c lines it restates.
 * The reference's SIMD kernels keep several fp32 accumulator lanes; this file keeps the same
 * lanes as plain arrays and combines them in the same order, so results are bit-identical to
 * the reference's AVX2 / AVX-VNNI / AVX-512-VNNI builds:
 *   hsum8(v) = ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7))   (hsum_ps, fastgguf.c:797-806)
 *   hsum4(v) = (v0+v1) + (v2+v3)                         (hsum128_ps, fastgguf.c:1089-1095)
 * Compile with -ffp-contract=off: every fused multiply-add below is an explicit fmaf, exactly
 * where the reference uses _mm256_fmadd_ps / _mm256_fnmadd_ps.
 *
 * Parity pins (tests/test_oracle.py): golden vectors written by the compiled reference
 * (tests/golden/), closed-form checks of the quantizers (IEEE division, round-half-even), brute
 * force integer sums over dequantized codes, and the reference selftest relations.
 */
#include "fg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 -> fp32, exact including subnormals (fp16_to_float_sw, fastgguf.c:96-117) ---- */
float fgo_fp16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, f;
    if (ex == 0) {
        if (man == 0) {
            f = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            f = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (ex == 31) {
        f = sign | 0x7f800000u | (man << 13);
    } else {
        f = sign | ((ex + 127 - 15) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

static inline uint16_t rd16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
/* bf16_to_float (fastgguf.c:124-127): the 16 bits above 16 zero bits */
static inline float bf16_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* the activation kind of a weight type (type_uses_q8, fastgguf.c:2167-2173): Q8 blocks of 32 for
 * Q8_0 / Q5_0, Q8_K blocks of 256 for the K-quants */
/* the 256-value types whose row kernels take Q8 (32-value) activations: Q2_K, Q3_K, IQ4_XS
 * (type_uses_q8, 2171) */
static inline int k256q8(uint32_t type) { return type == FGO_T_Q2_K || type == FGO_T_Q3_K || type == FGO_T_IQ4_XS; }
static inline int uses_q8(uint32_t type) {
    return type == FGO_T_Q8_0 || type == FGO_T_Q5_0 || type == FGO_T_Q4_0 || type == FGO_T_Q4_1 ||
           type == FGO_T_Q5_1 || type == FGO_T_IQ4_NL || k256q8(type);
}
/* the float types, whose row kernels take x itself (ACT_F32, type_uses_q8 2172) */
static inline int float_type(uint32_t type) { return type == FGO_T_F32 || type == FGO_T_F16 || type == FGO_T_BF16; }
static inline int k256q8_bytes(uint32_t type) { return type == FGO_T_Q2_K ? 84 : type == FGO_T_Q3_K ? 110 : 136; }
/* the 32-value block types with a min term (d * q + m): Q4_1 / Q5_1 */
static inline int has_min32(uint32_t type) { return type == FGO_T_Q4_1 || type == FGO_T_Q5_1; }

/* FGO_MUTATE (tests only, tests/test_oracle.py) builds a copy of this oracle with one planted
 * mistake, to show that the golden vectors catch it. 0 = the real oracle. */
#ifndef FGO_MUTATE
#define FGO_MUTATE 0
#endif

static inline float hsum8(const float v[8]) {
#if FGO_MUTATE == 1 /* sequential lane sum instead of the hsum_ps tree */
    return ((((((v[0] + v[1]) + v[2]) + v[3]) + v[4]) + v[5]) + v[6]) + v[7];
#else
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
#endif
}
static inline float hsum4(const float v[4]) { return (v[0] + v[1]) + (v[2] + v[3]); }

/* ---- activation quantizers ---- */

/* quantize_q8 (fastgguf.c:746-768): per 32 values d = amax/127, q = lrintf(x/d), two 16-sums */
void fgo_quantize_q8(const float *x, fgo_q8_blk *out, int n) {
    for (int b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
#if FGO_MUTATE == 3 /* reciprocal multiply instead of the IEEE division */
        float d = amax * (1.0f / 127.0f);
#else
        float d = amax / 127.0f;
#endif
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        out[b].d = d;
        int s0 = 0, s1 = 0;
        for (int j = 0; j < 32; j++) {
            int8_t q = (int8_t)lrintf(xb[j] * id);
            out[b].qs[j] = q;
            if (j < 16) s0 += q; else s1 += q;
        }
        out[b].s16[0] = (int16_t)s0;
        out[b].s16[1] = (int16_t)s1;
    }
}

/* quantize_q8k (fastgguf.c:773-793): one d per 256 values, sums of every 16 quants */
void fgo_quantize_q8k(const float *x, fgo_q8k_blk *out, int n) {
    for (int b = 0; b < n / 256; b++) {
        const float *xb = x + b * 256;
        float amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
        out[b].d = d;
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) {
                int v = (int)lrintf(xb[16 * g + j] * id);
                out[b].qs[16 * g + j] = (int8_t)v;
                s += v;
            }
            out[b].bsums[g] = (int16_t)s;
        }
    }
}

/* ---- Q4_K scale/min unpack (scale_min_k4, fastgguf.c:466-472) ---- */
static inline void q4k_scales(const uint8_t *s12, uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = s12[j] & 63;
            mn[j] = s12[j + 4] & 63;
        } else {
            sc[j] = (uint8_t)((s12[j + 4] & 0x0F) | ((s12[j - 4] >> 6) << 4));
            mn[j] = (uint8_t)((s12[j + 4] >> 4) | ((s12[j] >> 6) << 4));
        }
    }
}

/* Q6_K value of element e (0..255) of a block (fastgguf.c:676-690); 0..63, offset 32 not removed */
static inline int q6k_val(const uint8_t *p, int e) {
    int h = e >> 7, r = e & 127, k = r >> 5, l = r & 31;
    const uint8_t *ql = p + 64 * h, *qh = p + 128 + 32 * h;
    int lo = (k & 1) ? ql[l + 32] : ql[l];
    lo = (k & 2) ? (lo >> 4) : (lo & 0x0F);
    int hi = (qh[l] >> (2 * k)) & 3;
    return lo | (hi << 4);
}

/* Q5_0 element j (0..31) of a block, offset 16 not removed (q5_elem, fastgguf.c:939-942): nibble j
 * (low nibbles of qs[0..15] first, then their high nibbles) with bit j of qh as bit 4 */
static inline int q5_0_val(const uint8_t *p, int j) {
    uint32_t qh = rd32(p + 2);
    const uint8_t *qs = p + 6;
    int nib = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
#if FGO_MUTATE == 7 /* the fifth bit taken from the wrong half of qh */
    return nib | (int)(((qh >> ((j + 16) & 31)) & 1u) << 4);
#else
    return nib | (int)(((qh >> j) & 1u) << 4);
#endif
}

/* the non-linear values of IQ4_NL (kvalues_iq4nl, fastgguf.c:475-477) */
static const int8_t IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* nibble j of a 16-byte nibble array in the element order of the 32-value types (nibbles32,
 * fastgguf.c:809-814): low nibbles of qs[0..15], then their high nibbles */
static inline int nib32(const uint8_t *qs, int j) { return j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4); }

/* element j of a 32-value block as the int8 value the reference's row kernel multiplies (bx):
 * Q4_0 nib - 8 (833-857), Q4_1 nib (1020-1031), Q5_0 q5 - 16 (944-959), Q5_1 q5 (973-989),
 * IQ4_NL kvalues[nib] (1547-1562), Q8_0 q (891-902); the block's bytes per type in bb */
static inline int val32(uint32_t type, const uint8_t *p, int j) {
    switch (type) {
    case FGO_T_Q4_0: return nib32(p + 2, j) - 8;
    case FGO_T_Q4_1: return nib32(p + 4, j);
    case FGO_T_Q5_0: return q5_0_val(p, j) - 16;
    case FGO_T_Q5_1: return nib32(p + 8, j) | (int)(((rd32(p + 4) >> j) & 1u) << 4);
    case FGO_T_IQ4_NL: return IQ4NL[nib32(p + 2, j)];
    default: return (int)(int8_t)p[2 + j];
    }
}
static inline int bytes32(uint32_t type) {
    switch (type) {
    case FGO_T_Q4_0: case FGO_T_IQ4_NL: return 18;
    case FGO_T_Q4_1: return 20;
    case FGO_T_Q5_0: return 22;
    case FGO_T_Q5_1: return 24;
    default: return 34;
    }
}

/* Q5_K element e (0..255) of a block (fastgguf.c:1195-1210, scalar form 1216-1221): chunk j = e / 64
 * of ql (bytes 48 + 32 j ..), low nibbles for e % 64 < 32, high nibbles above; bit 2 j (low) or
 * 2 j + 1 (high) of qh[e % 32] as bit 4 */
static inline int q5k_val(const uint8_t *p, int e) {
    int j = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    uint8_t q = p[48 + 32 * j + l];
    int nib = hi ? (q >> 4) : (q & 0x0F);
#if FGO_MUTATE == 8 /* the qh bits of a chunk paired as (j, j + 4) instead of (2j, 2j + 1) */
    return nib | (((p[16 + l] >> (j + 4 * hi)) & 1) << 4);
#else
    return nib | (((p[16 + l] >> (2 * j + hi)) & 1) << 4);
#endif
}

/* ---- B-1: dot_q8_0_q8 (fastgguf.c:891-902) ----
 * lane i of block b: s_i = sum_{t=4i}^{4i+3} w_t x_t;  acc_i = fma(FP16(d)*xd, s_i, acc_i) */
float fgo_dot_q8_0(const uint8_t *row, const fgo_q8_blk *xq, int nb) {
    float acc[8] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 34;
        const int8_t *w = (const int8_t *)(p + 2);
        float d = fgo_fp16(rd16(p)) * xq[b].d;
        for (int i = 0; i < 8; i++) {
            int s = 0;
            for (int t = 4 * i; t < 4 * i + 4; t++) s += (int)w[t] * xq[b].qs[t];
            acc[i] = fmaf(d, (float)s, acc[i]);
        }
    }
    return hsum8(acc);
}

/* ---- B-6: dot_q5_0_q8 (fastgguf.c:944-959), the same lanes as B-1 over the int8 values q5 - 16
 * (bx = nibble | 0xF0 where the fifth bit is clear); the x4 tile dot_q32_q8_x4 (1400-1419) equals
 * it bit for bit (same d * yd, same lanes) */
float fgo_dot_q5_0(const uint8_t *row, const fgo_q8_blk *xq, int nb) {
    float acc[8] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 22;
        float d = fgo_fp16(rd16(p)) * xq[b].d;
        for (int i = 0; i < 8; i++) {
            int s = 0;
            for (int t = 4 * i; t < 4 * i + 4; t++) s += (q5_0_val(p, t) - 16) * xq[b].qs[t];
            acc[i] = fmaf(d, (float)s, acc[i]);
        }
    }
    return hsum8(acc);
}

/* ---- B-8: the other 32-value row kernels, lanes as B-1 over val32:
 *   dot_q4_0_q8 (833-857; its two-row form dot_q4_0_q8_x2 864-889 computes the same per row),
 *   dot_iq4_nl_q8 (1547-1562): acc_i = fma(FP16(d) * xd, s_i, acc_i), out = hsum8(acc);
 *   dot_q4_1_q8 (1020-1031), dot_q5_1_q8 (973-989): the same lanes over the unsigned values plus
 *   one scalar min chain, macc = fma(FP16(m) * xd, s16_0 + s16_1, macc) (the statement
 *   `macc += FP16(m) * xd * (float)(...)`, which gcc contracts to a fused multiply-add at -O3:
 *   the golden vectors of the compiled reference fix it), out = hsum8(acc) + macc */
float fgo_dot_q32(uint32_t type, const uint8_t *row, const fgo_q8_blk *xq, int nb) {
    if (type == FGO_T_Q8_0) return fgo_dot_q8_0(row, xq, nb);
    if (type == FGO_T_Q5_0) return fgo_dot_q5_0(row, xq, nb);
    const int bb = bytes32(type), mn = has_min32(type);
    float acc[8] = {0}, macc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * bb;
        float d = fgo_fp16(rd16(p)) * xq[b].d;
        for (int i = 0; i < 8; i++) {
            int s = 0;
            for (int t = 4 * i; t < 4 * i + 4; t++) s += val32(type, p, t) * xq[b].qs[t];
            acc[i] = fmaf(d, (float)s, acc[i]);
        }
        if (mn) {
#if FGO_MUTATE == 9 /* the min term added without the fused multiply-add */
            volatile float pm = fgo_fp16(rd16(p + 2)) * xq[b].d * (float)(xq[b].s16[0] + xq[b].s16[1]);
            macc = macc + pm;
#else
            macc = fmaf(fgo_fp16(rd16(p + 2)) * xq[b].d, (float)(xq[b].s16[0] + xq[b].s16[1]), macc);
#endif
        }
    }
    return hsum8(acc) + macc;
}

/* ---- B-9: dot_q40x8 (fastgguf.c:2424-2467), the 8-row repacked Q4_0 kernel, one row of it ----
 * per block the whole-block integer isum = sum (nib - 8) y (computed as sum nib y - 8 (s16_0 +
 * s16_1), the same integer); acc = fma(FP16(d) * yd, isum, acc); out = acc. The repack
 * (repack_q40_group 2390-2398) moves bytes only. */
/* ---- the 256-value types on Q8 activations: dot_q2_K_q8 (fastgguf.c:1426-1479), dot_q3_K_q8
 * (1481-1545), dot_iq4_xs_q8 (1580-1614). One fp32 chain per row over its 32-blocks in order
 * (block b, then 32-block c = 0..7 of it, c = 4 half + j for the K-quants):
 *   Q2_K: S = sum_l ((qs[32 half + l] >> 2 j) & 3) * sc(l) * x_l with sc(l) the low nibble of
 *         scales[8 half + 2 j + (l >= 16)], M = m_0 s16_0 + m_1 s16_1 (the high nibbles);
 *         sum = fma(xd, fma(d, S, -(dmin * M)), sum)
 *   Q3_K: qu = lo | 4 hbit (hmask bit 4 half + j of byte l), sc' = 6-bit scale - 32, S = sum
 *         qu * sc'(l) * x_l, off = 4 (sc'_0 s16_0 + sc'_1 s16_1); sum = fma(d * xd, (float)(S - off), sum)
 *   IQ4_XS: si = sum kvalues[nib] * x over the 32-block; sum = fma(d * (ls - 32) * xd, (float)si, sum)
 * These are the contractions gcc makes of the reference's expressions (`sum += xk->d * (d * S -
 * dmin * M)` and its like); they were fixed against the compiled reference, which every other
 * form tried disagrees with on a third or more of random rows. The integers are the AVX2 kernels'
 * (maddubs / madd sums), exact. */
static void q3k_scales(const uint8_t *p, int8_t *scs) {
    uint32_t a0 = rd32(p + 96), a1 = rd32(p + 100), tmp = rd32(p + 104), aux[4];
    aux[0] = (a0 & 0x0f0f0f0fu) | (((tmp >> 0) & 0x03030303u) << 4);
    aux[1] = (a1 & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4);
    aux[2] = ((a0 >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4);
    aux[3] = ((a1 >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4);
    memcpy(scs, aux, 16);
}
static inline int q2k_q(const uint8_t *p, int c, int l) { return (p[16 + 32 * (c >> 2) + l] >> (2 * (c & 3))) & 3; }
static inline int q3k_q(const uint8_t *p, int c, int l) {
#if FGO_MUTATE == 16 /* the hmask bit of the other half */
    return ((p[32 + 32 * (c >> 2) + l] >> (2 * (c & 3))) & 3) | ((p[l] >> (c ^ 4)) & 1) * 4;
#else
    return ((p[32 + 32 * (c >> 2) + l] >> (2 * (c & 3))) & 3) | ((p[l] >> c) & 1) * 4;
#endif
}
static const int8_t IQ4NL_XS[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
static inline int iq4xs_ls(const uint8_t *p, int c) {
#if FGO_MUTATE == 17 /* the high scale bits of scales_h at bit c instead of 2c */
    return ((p[4 + c / 2] >> (4 * (c % 2))) & 0xF) | (((rd16(p + 2) >> c) & 3) << 4);
#else
    return ((p[4 + c / 2] >> (4 * (c % 2))) & 0xF) | (((rd16(p + 2) >> (2 * c)) & 3) << 4);
#endif
}
static inline int iq4xs_q(const uint8_t *p, int c, int l) {
    const uint8_t q = p[8 + 16 * c + (l & 15)];
    return IQ4NL_XS[l < 16 ? (q & 0xF) : (q >> 4)];
}
/* the integers of 32-block c of a block: S (the scaled sum; IQ4_XS: si) and the type's second
 * integer (Q2_K: M; Q3_K: sc'_0 s16_0 + sc'_1 s16_1; IQ4_XS: 0) */
static void k256q8_ints(uint32_t type, const uint8_t *p, int c, const fgo_q8_blk *xb, int *S, int *M) {
    int s = 0, m = 0;
    if (type == FGO_T_Q2_K) {
        const int a = p[2 * c], b = p[2 * c + 1];
        for (int l = 0; l < 32; l++) s += q2k_q(p, c, l) * ((l < 16 ? a : b) & 0xF) * xb->qs[l];
        m = (a >> 4) * xb->s16[0] + (b >> 4) * xb->s16[1];
    } else if (type == FGO_T_Q3_K) {
        int8_t scs[16];
        q3k_scales(p, scs);
        const int a = scs[2 * c] - 32, b = scs[2 * c + 1] - 32;
        for (int l = 0; l < 32; l++) s += q3k_q(p, c, l) * (l < 16 ? a : b) * xb->qs[l];
        m = a * xb->s16[0] + b * xb->s16[1];
    } else {
        for (int l = 0; l < 32; l++) s += iq4xs_q(p, c, l) * xb->qs[l];
    }
    *S = s;
    *M = m;
}
float fgo_dot_k256q8(uint32_t type, const uint8_t *row, const fgo_q8_blk *xq, int nb256) {
    const int bb = k256q8_bytes(type);
    float sum = 0.0f;
    for (int b = 0; b < nb256; b++) {
        const uint8_t *p = row + (size_t)b * bb;
        for (int c = 0; c < 8; c++) {
            const fgo_q8_blk *xb = xq + 8 * b + c;
            int S, M;
            k256q8_ints(type, p, c, xb, &S, &M);
            if (type == FGO_T_Q2_K) {
                const float d = fgo_fp16(rd16(p + 80)), dmin = fgo_fp16(rd16(p + 82));
#if FGO_MUTATE == 15 /* the reference's expression without gcc's contractions */
                sum += xb->d * (d * (float)S - dmin * (float)M);
#else
                sum = fmaf(xb->d, fmaf(d, (float)S, -(dmin * (float)M)), sum);
#endif
            } else if (type == FGO_T_Q3_K) {
                const float d = fgo_fp16(rd16(p + 108));
                sum = fmaf(d * xb->d, (float)(S - 4 * M), sum);
            } else {
                const float d = fgo_fp16(rd16(p));
                sum = fmaf(d * (float)(iq4xs_ls(p, c) - 32) * xb->d, (float)S, sum);
            }
        }
    }
    return sum;
}

float fgo_dot_q4_0_rp(const uint8_t *row, const fgo_q8_blk *xq, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 18;
        int isum = 0;
        for (int t = 0; t < 32; t++) isum += (nib32(p + 2, t) - 8) * xq[b].qs[t];
        acc = fmaf(fgo_fp16(rd16(p)) * xq[b].d, (float)isum, acc);
    }
    return acc;
}

/* ---- B-2: dot_q4_K_q8k (fastgguf.c:1118-1153) ----
 * lane i: sum_j [sc_2j * sum_{t=4i}^{4i+3} lo(32j+t) y(64j+t) + sc_2j+1 * sum hi(32j+t) y(64j+32+t)]
 * min lane p: m_2p (bs_4p + bs_4p+1) + m_2p+1 (bs_4p+2 + bs_4p+3)   (k4_min_vec, 1078-1082) */
float fgo_dot_q4_K(const uint8_t *row, const fgo_q8k_blk *y, int nb) {
    float acc[8] = {0}, macc[4] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 144, *qs = p + 16;
        const int8_t *q8 = y[b].qs;
        uint8_t sc[8], mn[8];
        q4k_scales(p + 4, sc, mn);
        float yd = y[b].d;
        float dd = fgo_fp16(rd16(p)) * yd, dm = fgo_fp16(rd16(p + 2)) * yd;
        for (int i = 0; i < 8; i++) {
            int lane = 0;
            for (int j = 0; j < 4; j++) {
                int il = 0, ih = 0;
                for (int t = 4 * i; t < 4 * i + 4; t++) {
                    il += (qs[32 * j + t] & 0x0F) * q8[64 * j + t];
                    ih += (qs[32 * j + t] >> 4) * q8[64 * j + 32 + t];
                }
                lane += sc[2 * j] * il + sc[2 * j + 1] * ih;
            }
            acc[i] = fmaf(dd, (float)lane, acc[i]);
        }
        for (int pp = 0; pp < 4; pp++) {
            const int16_t *bs = y[b].bsums;
            int s0 = bs[4 * pp] + bs[4 * pp + 1], s1 = bs[4 * pp + 2] + bs[4 * pp + 3];
            int ml = mn[2 * pp] * s0 + mn[2 * pp + 1] * s1;
            macc[pp] = fmaf(dm, (float)ml, macc[pp]);
        }
    }
    return hsum8(acc) - hsum4(macc);
}

/* ---- B-7: dot_q5_K_q8k (fastgguf.c:1178-1230): the lanes, min lanes and final combination of B-2
 * with five-bit values (maddubs pairs, madd with the sub-block scale: lane i sums elements 4i..4i+3
 * of each 32-value sub-block) */
float fgo_dot_q5_K(const uint8_t *row, const fgo_q8k_blk *y, int nb) {
    float acc[8] = {0}, macc[4] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 176;
        const int8_t *q8 = y[b].qs;
        uint8_t sc[8], mn[8];
        q4k_scales(p + 4, sc, mn);
        float yd = y[b].d;
        float dd = fgo_fp16(rd16(p)) * yd, dm = fgo_fp16(rd16(p + 2)) * yd;
        for (int i = 0; i < 8; i++) {
            int lane = 0;
            for (int j = 0; j < 4; j++) {
                int il = 0, ih = 0;
                for (int t = 4 * i; t < 4 * i + 4; t++) {
                    il += q5k_val(p, 64 * j + t) * q8[64 * j + t];
                    ih += q5k_val(p, 64 * j + 32 + t) * q8[64 * j + 32 + t];
                }
                lane += sc[2 * j] * il + sc[2 * j + 1] * ih;
            }
            acc[i] = fmaf(dd, (float)lane, acc[i]);
        }
        for (int pp = 0; pp < 4; pp++) {
            const int16_t *bs = y[b].bsums;
            int s0 = bs[4 * pp] + bs[4 * pp + 1], s1 = bs[4 * pp + 2] + bs[4 * pp + 3];
            macc[pp] = fmaf(dm, (float)(mn[2 * pp] * s0 + mn[2 * pp + 1] * s1), macc[pp]);
        }
    }
    return hsum8(acc) - hsum4(macc);
}

/* per-block Q4_K integers */
static void q4k_block_ints(const uint8_t *p, const fgo_q8k_blk *yb, int32_t *sumi, int32_t *msum) {
    const uint8_t *qs = p + 16;
    uint8_t sc[8], mn[8];
    q4k_scales(p + 4, sc, mn);
    int s = 0, m = 0;
    for (int j = 0; j < 4; j++) {
        int il = 0, ih = 0;
        for (int l = 0; l < 32; l++) {
            il += (qs[32 * j + l] & 0x0F) * yb->qs[64 * j + l];
            ih += (qs[32 * j + l] >> 4) * yb->qs[64 * j + 32 + l];
        }
        s += sc[2 * j] * il + sc[2 * j + 1] * ih;
    }
    for (int j = 0; j < 8; j++) m += mn[j] * (yb->bsums[2 * j] + yb->bsums[2 * j + 1]);
    *sumi = s;
    *msum = m;
}

/* ---- B-3: dot_q4Kx8 (fastgguf.c:2322-2358), the 8-row repacked kernel, one row of it ----
 * per block: sumi, msum (whole-block integers); acc = fma(d*yd, sumi, acc);
 * macc = fma(dmin*yd, msum, macc); result acc - macc. The repack (2268-2282) moves bytes only. */
float fgo_dot_q4_K_rp(const uint8_t *row, const fgo_q8k_blk *y, int nb) {
    float acc = 0.0f, macc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 144;
        int32_t sumi, msum;
        q4k_block_ints(p, &y[b], &sumi, &msum);
        float yd = y[b].d;
#if FGO_MUTATE == 5 /* one chain: the min term subtracted block by block */
        acc = fmaf(fgo_fp16(rd16(p)) * yd, (float)sumi, acc);
        acc = fmaf(-(fgo_fp16(rd16(p + 2)) * yd), (float)msum, acc);
#else
        acc = fmaf(fgo_fp16(rd16(p)) * yd, (float)sumi, acc);
        macc = fmaf(fgo_fp16(rd16(p + 2)) * yd, (float)msum, macc);
#endif
    }
    return acc - macc;
}

/* ---- B-4: dot_q6_K_q8k (fastgguf.c:1232-1264) ----
 * lane i: sum_{h,k} sc[8h+2k+(i>=4)] * sum_{t=4i}^{4i+3} q(128h+32k+t) y(128h+32k+t)
 * correction lane p (q6_corr_vec, 1085-1088):
 *   (sc_2p bs_2p + sc_2p+1 bs_2p+1) + (sc_2p+8 bs_2p+8 + sc_2p+9 bs_2p+9)
 * acc_i = fma(dd, lane_i, acc_i); cacc_p = fma(32*dd, corr_p, cacc_p); hsum8(acc) - hsum4(cacc) */
float fgo_dot_q6_K(const uint8_t *row, const fgo_q8k_blk *y, int nb) {
    float acc[8] = {0}, cacc[4] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *p = row + (size_t)b * 210;
        const int8_t *sc = (const int8_t *)(p + 192);
        float dd = fgo_fp16(rd16(p + 208)) * y[b].d;
        const int8_t *q8 = y[b].qs;
        for (int i = 0; i < 8; i++) {
            int lane = 0;
            for (int h = 0; h < 2; h++)
                for (int k = 0; k < 4; k++) {
                    int s = 0;
                    for (int t = 4 * i; t < 4 * i + 4; t++) {
                        int e = 128 * h + 32 * k + t;
                        s += q6k_val(p, e) * q8[e];
                    }
#if FGO_MUTATE == 4 /* the per-16 scale of the upper half-lane dropped */
                    lane += sc[8 * h + 2 * k] * s;
#else
                    lane += sc[8 * h + 2 * k + (i >= 4)] * s;
#endif
                }
            acc[i] = fmaf(dd, (float)lane, acc[i]);
        }
        const int16_t *bs = y[b].bsums;
        for (int pp = 0; pp < 4; pp++) {
            int c = (sc[2 * pp] * bs[2 * pp] + sc[2 * pp + 1] * bs[2 * pp + 1]) +
                    (sc[2 * pp + 8] * bs[2 * pp + 8] + sc[2 * pp + 9] * bs[2 * pp + 9]);
            cacc[pp] = fmaf(dd * 32.0f, (float)c, cacc[pp]);
        }
    }
    return hsum8(acc) - hsum4(cacc);
}

void fgo_block_ints(uint32_t type, const uint8_t *row, const void *act, int nb,
                    int32_t *sumi, int32_t *msum) {
    for (int b = 0; b < nb; b++) {
        if (type == FGO_T_Q4_K) {
            q4k_block_ints(row + (size_t)b * 144, (const fgo_q8k_blk *)act + b, &sumi[b], &msum[b]);
        } else if (type == FGO_T_Q6_K) {
            const uint8_t *p = row + (size_t)b * 210;
            const int8_t *sc = (const int8_t *)(p + 192);
            const fgo_q8k_blk *yb = (const fgo_q8k_blk *)act + b;
            int s = 0, m = 0;
            for (int g = 0; g < 16; g++) {
                int ig = 0;
                for (int l = 0; l < 16; l++) ig += q6k_val(p, 16 * g + l) * yb->qs[16 * g + l];
                s += sc[g] * ig;
                m += sc[g] * yb->bsums[g];
            }
            sumi[b] = s;
            msum[b] = m;
        } else if (type == FGO_T_Q5_K) {
            const uint8_t *p = row + (size_t)b * 176;
            const fgo_q8k_blk *yb = (const fgo_q8k_blk *)act + b;
            uint8_t sc[8], mn[8];
            q4k_scales(p + 4, sc, mn);
            int s = 0, m = 0;
            for (int g = 0; g < 8; g++) {
                int ig = 0;
                for (int l = 0; l < 32; l++) ig += q5k_val(p, 32 * g + l) * yb->qs[32 * g + l];
                s += sc[g] * ig;
                m += mn[g] * (yb->bsums[2 * g] + yb->bsums[2 * g + 1]);
            }
            sumi[b] = s;
            msum[b] = m;
        } else if (k256q8(type)) { /* b counts 32-blocks here */
            const uint8_t *p = row + (size_t)(b / 8) * k256q8_bytes(type);
            k256q8_ints(type, p, b % 8, (const fgo_q8_blk *)act + b, &sumi[b], &msum[b]);
        } else if (uses_q8(type) && type != FGO_T_Q8_0) {
            const uint8_t *p = row + (size_t)b * bytes32(type);
            const fgo_q8_blk *xb = (const fgo_q8_blk *)act + b;
            int s = 0;
            for (int t = 0; t < 32; t++) s += val32(type, p, t) * xb->qs[t];
            sumi[b] = s;
            msum[b] = 0;
        } else { /* Q8_0 */
            const uint8_t *p = row + (size_t)b * 34;
            const fgo_q8_blk *xb = (const fgo_q8_blk *)act + b;
            int s = 0;
            for (int t = 0; t < 32; t++) s += (int)(int8_t)p[2 + t] * xb->qs[t];
            sumi[b] = s;
            msum[b] = 0;
        }
    }
}

/* ---- dequantize_row (fastgguf.c:518-532, 552-562, 622-667, 669-693) ---- */
int fgo_dequantize_row(uint32_t type, const uint8_t *raw, float *out, int n) {
    if (float_type(type)) { /* dequantize_row 481-489 */
        for (int i = 0; i < n; i++) {
            if (type == FGO_T_F32) memcpy(&out[i], raw + 4 * (size_t)i, 4);
            else out[i] = type == FGO_T_F16 ? fgo_fp16(rd16(raw + 2 * (size_t)i)) : bf16_f32(rd16(raw + 2 * (size_t)i));
        }
        return 0;
    }
    if (k256q8(type)) { /* dequantize_row 563-586 (Q2_K), 587-620 (Q3_K), 709-727 (IQ4_XS) */
        const int bb = k256q8_bytes(type);
        for (int b = 0; b < n / 256; b++) {
            const uint8_t *p = raw + (size_t)b * bb;
            for (int c = 0; c < 8; c++)
                for (int l = 0; l < 32; l++) {
                    float v;
                    if (type == FGO_T_Q2_K) {
                        const int s = p[2 * c + (l >= 16)];
                        v = fgo_fp16(rd16(p + 80)) * (float)(s & 0xF) * (float)q2k_q(p, c, l) -
                            fgo_fp16(rd16(p + 82)) * (float)(s >> 4);
                    } else if (type == FGO_T_Q3_K) {
                        int8_t scs[16];
                        q3k_scales(p, scs);
                        v = fgo_fp16(rd16(p + 108)) * (float)(scs[2 * c + (l >= 16)] - 32) * (float)(q3k_q(p, c, l) - 4);
                    } else {
                        v = fgo_fp16(rd16(p)) * (float)(iq4xs_ls(p, c) - 32) * (float)iq4xs_q(p, c, l);
                    }
                    out[256 * b + 32 * c + l] = v;
                }
        }
        return 0;
    }
    if (uses_q8(type) && type != FGO_T_Q8_0) { /* d * value (+ m for Q4_1 / Q5_1) */
        const int bb = bytes32(type);
        for (int b = 0; b < n / 32; b++) {
            const uint8_t *p = raw + (size_t)b * bb;
            float d = fgo_fp16(rd16(p)), m = has_min32(type) ? fgo_fp16(rd16(p + 2)) : 0.0f;
            for (int j = 0; j < 32; j++) out[32 * b + j] = d * (float)val32(type, p, j) + m;
        }
        return 0;
    }
    if (type == FGO_T_Q5_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t *p = raw + (size_t)b * 176;
            float d = fgo_fp16(rd16(p)), dmin = fgo_fp16(rd16(p + 2));
            uint8_t sc[8], mn[8];
            q4k_scales(p + 4, sc, mn);
            for (int e = 0; e < 256; e++)
                out[256 * b + e] = d * (float)sc[e / 32] * (float)q5k_val(p, e) - dmin * (float)mn[e / 32];
        }
        return 0;
    }
    if (type == FGO_T_Q8_0) {
        for (int b = 0; b < n / 32; b++) {
            const uint8_t *p = raw + (size_t)b * 34;
            float d = fgo_fp16(rd16(p));
            for (int j = 0; j < 32; j++) out[32 * b + j] = d * (float)(int8_t)p[2 + j];
        }
        return 0;
    }
    if (type == FGO_T_Q4_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t *p = raw + (size_t)b * 144;
            float d = fgo_fp16(rd16(p)), dmin = fgo_fp16(rd16(p + 2));
            uint8_t sc[8], mn[8];
            q4k_scales(p + 4, sc, mn);
            for (int j = 0; j < 4; j++) {
                float d1 = d * sc[2 * j], m1 = dmin * mn[2 * j];
                float d2 = d * sc[2 * j + 1], m2 = dmin * mn[2 * j + 1];
                for (int l = 0; l < 32; l++) {
                    uint8_t q = p[16 + 32 * j + l];
                    out[256 * b + 64 * j + l] = d1 * (float)(q & 0x0F) - m1;
                    out[256 * b + 64 * j + 32 + l] = d2 * (float)(q >> 4) - m2;
                }
            }
        }
        return 0;
    }
    if (type == FGO_T_Q6_K) {
        for (int b = 0; b < n / 256; b++) {
            const uint8_t *p = raw + (size_t)b * 210;
            const int8_t *sc = (const int8_t *)(p + 192);
            float d = fgo_fp16(rd16(p + 208));
            for (int e = 0; e < 256; e++)
                out[256 * b + e] = d * (float)sc[e / 16] * (float)(q6k_val(p, e) - 32);
        }
        return 0;
    }
    return -1;
}

int fgo_block_size(uint32_t type, int *elems, int *bytes) {
    switch (type) {
    case FGO_T_F32: *elems = 1; *bytes = 4; return 0;
    case FGO_T_F16: case FGO_T_BF16: *elems = 1; *bytes = 2; return 0;
    case FGO_T_Q8_0: *elems = 32; *bytes = 34; return 0;
    case FGO_T_Q4_K: *elems = 256; *bytes = 144; return 0;
    case FGO_T_Q6_K: *elems = 256; *bytes = 210; return 0;
    case FGO_T_Q5_0: case FGO_T_Q4_0: case FGO_T_Q4_1: case FGO_T_Q5_1: case FGO_T_IQ4_NL:
        *elems = 32; *bytes = bytes32(type); return 0;
    case FGO_T_Q5_K: *elems = 256; *bytes = 176; return 0;
    case FGO_T_Q2_K: case FGO_T_Q3_K: case FGO_T_IQ4_XS: *elems = 256; *bytes = k256q8_bytes(type); return 0;
    default: return -1;
    }
}

/* ---- dot_row dispatch (fastgguf.c:2183-2214), and the repacked kernels of matvec_rp ---- */
static float dot_row3(uint32_t type, int order, const uint8_t *rb, const void *act, int cols) {
    if (float_type(type)) return fgo_dot_float(type, rb, (const float *)act, cols);
    if (type == FGO_T_Q4_K)
        return order == FGO_ORDER_REPACKED ? fgo_dot_q4_K_rp(rb, (const fgo_q8k_blk *)act, cols / 256)
                                           : fgo_dot_q4_K(rb, (const fgo_q8k_blk *)act, cols / 256);
    if (type == FGO_T_Q6_K) return fgo_dot_q6_K(rb, (const fgo_q8k_blk *)act, cols / 256);
    if (type == FGO_T_Q5_K) return fgo_dot_q5_K(rb, (const fgo_q8k_blk *)act, cols / 256);
    if (type == FGO_T_Q4_0 && order == FGO_ORDER_REPACKED) return fgo_dot_q4_0_rp(rb, (const fgo_q8_blk *)act, cols / 32);
    if (k256q8(type)) return fgo_dot_k256q8(type, rb, (const fgo_q8_blk *)act, cols / 256);
    return fgo_dot_q32(type, rb, (const fgo_q8_blk *)act, cols / 32);
}

static int type_ok(uint32_t type, int cols) {
    if (float_type(type)) return cols > 0;
    if (type == FGO_T_Q4_K || type == FGO_T_Q5_K || type == FGO_T_Q6_K || k256q8(type)) return cols > 0 && cols % 256 == 0;
    if (uses_q8(type)) return cols > 0 && cols % 32 == 0;
    return 0;
}

/* quantize one activation vector for the type (type_uses_q8 2167 + quantize_act 2176);
 * returns a malloc'd buffer, NULL on failure */
static void *quantize_for(uint32_t type, const float *x, int cols) {
    if (float_type(type)) { /* x itself (ACT_F32) */
        float *c = (float *)malloc((size_t)cols * sizeof(float));
        if (c) memcpy(c, x, (size_t)cols * sizeof(float));
        return c;
    }
    if (uses_q8(type)) {
        fgo_q8_blk *q = (fgo_q8_blk *)malloc((size_t)(cols / 32) * sizeof(fgo_q8_blk));
        if (q) fgo_quantize_q8(x, q, cols);
        return q;
    }
    fgo_q8k_blk *q = (fgo_q8k_blk *)malloc((size_t)(cols / 256) * sizeof(fgo_q8k_blk));
    if (q) fgo_quantize_q8k(x, q, cols);
    return q;
}

static size_t act_bytes(uint32_t type, int cols) {
    if (float_type(type)) return (size_t)cols * sizeof(float);
    return uses_q8(type) ? (size_t)(cols / 32) * sizeof(fgo_q8_blk) : (size_t)(cols / 256) * sizeof(fgo_q8k_blk);
}

/* matvec (fastgguf.c:2575-2622) and matvec_rp (2540-2545): rows are independent, so the row
 * order of the OpenMP loop does not change any value */
int fgo_matvec(uint32_t type, int order, const uint8_t *w, int64_t rows, int cols,
               const float *x, float *y) {
    if (!type_ok(type, cols)) return -1;
    int eb, bb;
    fgo_block_size(type, &eb, &bb);
    size_t stride = (size_t)(cols / eb) * bb;
    void *act = quantize_for(type, x, cols);
    if (!act) return -1;
#pragma omp parallel for schedule(guided, 32)
    for (int64_t r = 0; r < rows; r++) y[r] = dot_row3(type, order, w + (size_t)r * stride, act, cols);
    free(act);
    return 0;
}

/* ---- B-5: gemmk_kern (fastgguf.c:2756-2797) for Q4_K (GS = MS = 32) and Q6_K (16/16) ----
 * per (row, token) and block b:  a = 0
 *   for g: a = fma(wsc_g, ia_g, a)          wsc_g = FP16(d)*sc_g  (Q6_K: FP16(d)*sc_g)
 *   for g: a = fnmadd(wmn_g, bs_g, a)       wmn_g = FP16(dmin)*m_g (Q6_K: 32*FP16(d)*sc_g)
 *   f = fma(a, yd_b, f)
 * ---- and gemm32_kern (2909-2937) for the 32-value types (unpack_row_q32 2876-2894, gemm_pack_q8
 * 2897-2913; Q4_0 repacked: unpack_row_q40x8 2400-2421, the same values):
 *   per 32-block g: a = fma(d*xd, ia'_g, a); a = fnmadd(m, xd*(s16_0+s16_1), a)
 *   with ia' = sum u*x over the unsigned weights the VNNI kernel multiplies: Q8_0 u = w + 128,
 *   m = 128 d; Q5_0 u = q5, m = 16 d; Q4_0 u = nib, m = 8 d; Q4_1 / Q5_1 u = nib / q5, m = -FP16(m) */
static int has_gemm(uint32_t type) {
    return type != FGO_T_Q5_K && type != FGO_T_IQ4_NL && !k256q8(type) && !float_type(type);
}
static void gemm_row_token(uint32_t type, const uint8_t *rb, const void *act, int cols, float *out) {
    if (uses_q8(type)) {
        const fgo_q8_blk *xq = (const fgo_q8_blk *)act;
        const int bb = bytes32(type);
        float acc = 0.0f;
        for (int g = 0; g < cols / 32; g++) {
            const uint8_t *p = rb + (size_t)g * bb;
            float d = fgo_fp16(rd16(p)), m;
            int off;  /* u = value + off */
            switch (type) {
            case FGO_T_Q8_0: m = 128.0f * d; off = 128; break;
            case FGO_T_Q5_0: m = 16.0f * d; off = 16; break;
            case FGO_T_Q4_0: m = 8.0f * d; off = 8; break;
            default: m = -fgo_fp16(rd16(p + 2)); off = 0; break; /* Q4_1, Q5_1 */
            }
            int ia = 0;
            for (int t = 0; t < 32; t++) ia += (val32(type, p, t) + off) * xq[g].qs[t];
            float ws = d * xq[g].d;
            float ys = xq[g].d * (float)(xq[g].s16[0] + xq[g].s16[1]);
            acc = fmaf(ws, (float)ia, acc);
            acc = fmaf(-m, ys, acc);
        }
        *out = acc;
        return;
    }
    const fgo_q8k_blk *y = (const fgo_q8k_blk *)act;
    float f = 0.0f;
    for (int b = 0; b < cols / 256; b++) {
        float a = 0.0f;
        if (type == FGO_T_Q4_K) {
            const uint8_t *p = rb + (size_t)b * 144;
            uint8_t sc[8], mn[8];
            q4k_scales(p + 4, sc, mn);
            float d = fgo_fp16(rd16(p)), dmin = fgo_fp16(rd16(p + 2));
            for (int g = 0; g < 8; g++) {
                int ia = 0;
                for (int l = 0; l < 32; l++) {
                    int e = 32 * g + l; /* element e: sub-block g = pair j = g/2, nibble g&1 */
                    uint8_t q = p[16 + 32 * (g >> 1) + l];
                    ia += ((g & 1) ? (q >> 4) : (q & 0x0F)) * y[b].qs[e];
                }
#if FGO_MUTATE == 6 /* integer scale sum first, one conversion per block (not the GEMM order) */
                a += 0.0f * (float)ia;
            }
            {
                int isum = 0;
                for (int g = 0; g < 8; g++) {
                    int ia = 0;
                    for (int l = 0; l < 32; l++) {
                        uint8_t q = p[16 + 32 * (g >> 1) + l];
                        ia += ((g & 1) ? (q >> 4) : (q & 0x0F)) * y[b].qs[32 * g + l];
                    }
                    isum += sc[g] * ia;
                }
                a = d * (float)isum;
            }
#else
                a = fmaf(d * (float)sc[g], (float)ia, a);
            }
#endif
            for (int g = 0; g < 8; g++) {
                float bs = (float)(y[b].bsums[2 * g] + y[b].bsums[2 * g + 1]);
                a = fmaf(-(dmin * (float)mn[g]), bs, a);
            }
        } else { /* Q6_K */
            const uint8_t *p = rb + (size_t)b * 210;
            const int8_t *sc = (const int8_t *)(p + 192);
            float d = fgo_fp16(rd16(p + 208));
            for (int g = 0; g < 16; g++) {
                int ia = 0;
                for (int l = 0; l < 16; l++) ia += q6k_val(p, 16 * g + l) * y[b].qs[16 * g + l];
                a = fmaf(d * (float)sc[g], (float)ia, a);
            }
            for (int g = 0; g < 16; g++)
                a = fmaf(-(32.0f * d * (float)sc[g]), (float)y[b].bsums[g], a);
        }
        f = fmaf(a, y[b].d, f);
    }
    *out = f;
}

int fgo_gemm(uint32_t type, const uint8_t *w, int64_t rows, int cols, const void *act,
             int act_stride_blocks, float *Y, int ldy, int nb) {
    if (!type_ok(type, cols)) return -1;
    int eb, bb;
    fgo_block_size(type, &eb, &bb);
    size_t stride = (size_t)(cols / eb) * bb;
    if (!has_gemm(type)) return -1; /* no prompt GEMM: matmul runs the row kernel per token */
    size_t ablk = uses_q8(type) ? sizeof(fgo_q8_blk) : sizeof(fgo_q8k_blk);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int t = 0; t < nb; t++)
            gemm_row_token(type, w + (size_t)r * stride,
                           (const uint8_t *)act + (size_t)t * act_stride_blocks * ablk, cols,
                           &Y[(size_t)t * ldy + r]);
    return 0;
}

/* matmul (fastgguf.c:3004-3093) for the types here, as built for a VNNI CPU:
 *   nb == 1: matvec;  repacked (Q4_K, Q4_0) and nb < 8: per-token matvec;  nb >= 8: the prompt
 *   GEMM (gemm_kquant for Q4_K / Q6_K, gemm_q32 for Q4_0 / Q4_1 / Q5_0 / Q5_1 and, VNNI builds
 *   only, Q8_0 - GEMM_Q8_0 at 2864-2868; Q5_K, IQ4_NL, Q2_K, Q3_K and IQ4_XS have no GEMM: the
 *   row kernel per token);
 *   otherwise the x4 tiles, which equal the single-row kernels bit for bit (selftest 5871-5916). */
int fgo_matmul(uint32_t type, int order, const uint8_t *w, int64_t rows, int cols,
               const float *X, int ldx, float *Y, int ldy, int nb) {
    if (!type_ok(type, cols) || nb < 1) return -1;
    if (nb == 1) return fgo_matvec(type, order, w, rows, cols, X, Y);
    int repacked = (type == FGO_T_Q4_K || type == FGO_T_Q4_0) && order == FGO_ORDER_REPACKED;
    if (repacked && nb < 8) {
        for (int t = 0; t < nb; t++)
            if (fgo_matvec(type, order, w, rows, cols, X + (size_t)t * ldx, Y + (size_t)t * ldy) != 0)
                return -1;
        return 0;
    }
    size_t ab = act_bytes(type, cols);
    uint8_t *act = (uint8_t *)malloc(ab * (size_t)nb);
    if (!act) return -1;
    for (int t = 0; t < nb; t++) {
        if (float_type(type)) memcpy(act + ab * t, X + (size_t)t * ldx, ab);
        else if (uses_q8(type)) fgo_quantize_q8(X + (size_t)t * ldx, (fgo_q8_blk *)(act + ab * t), cols);
        else fgo_quantize_q8k(X + (size_t)t * ldx, (fgo_q8k_blk *)(act + ab * t), cols);
    }
    int eb, bb;
    fgo_block_size(type, &eb, &bb);
    int sblocks = cols / eb;
    if (nb >= 8 && has_gemm(type)) {
        int rc = fgo_gemm(type, w, rows, cols, act, sblocks, Y, ldy, nb);
        free(act);
        return rc;
    }
    size_t stride = (size_t)(cols / eb) * bb;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int t = 0; t < nb; t++)
            Y[(size_t)t * ldy + r] = dot_row3(type, FGO_ORDER_ROW, w + (size_t)r * stride, act + ab * t, cols);
    free(act);
    return 0;
}

/* ---- MoE (moe_ffn, fastgguf.c:4588-4642) ---- */

/* silu_f (fastgguf.c:3118) */
float fgo_silu(float x) { return x / (1.0f + expf(-x)); }

/* the method of ARM optimized-routines' expf (glibc >= 2.27, built with FMA on x86-64): N = 32,
 * z = x N / ln 2, k = round(z) (by adding 1.5 * 2^52), r = fma(N / ln 2, x, -k), 2^(k/N) from a table of the correctly rounded
 * 2^(i/N) with the exponent bits of k/N added, 2^(r/N) ~ (c0 r + c1) r^2 + (c2 r + 1), all in
 * double, one rounding to float. The table is 2^(i/32) rounded to nearest double (computed from
 * the mathematics), stored minus i << 47 as the method stores it. */
static const uint64_t EXP2_TAB[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

float fgo_expf_restated(float x) {
    if (!(x < 128.0f)) return x > 0.0f ? INFINITY : x;
    if (!(x > -128.0f)) return 0.0f;
    const double invln2n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = x, z = invln2n * xd, kd = z + shift;
    uint64_t ki, t;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    double r = fma(invln2n, xd, -kd), s; /* fused as in glibc's FMA build (x86-64 with FMA) */
    t = EXP2_TAB[ki % 32] + (ki << 47);
    memcpy(&s, &t, 8);
    double p = fma(c0, r, c1), r2 = r * r, y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    return (float)(y * s);
}

void fgo_expf_n(const float *x, int n, float *out) {
    for (int i = 0; i < n; i++) out[i] = expf(x[i]);
}

static int64_t f32_key(float f) { /* monotone integer key of a float */
    int32_t i;
    memcpy(&i, &f, 4);
    return i < 0 ? -(int64_t)(i & 0x7fffffff) : (int64_t)i;
}

uint64_t fgo_expf_compare(float lo, float hi, uint32_t stride, uint64_t *n_checked, int *max_ulp) {
    uint64_t bad = 0, n = 0;
    int mu = 0;
    for (int64_t k = f32_key(lo); k <= f32_key(hi); k += stride) {
        int32_t i = k < 0 ? (int32_t)((uint32_t)(-k) | 0x80000000u) : (int32_t)k;
        float x;
        memcpy(&x, &i, 4);
        float a = expf(x), b = fgo_expf_restated(x);
        if (isnan(a) && isnan(b)) continue;
        n++;
        if (memcmp(&a, &b, 4) != 0) {
            bad++;
            int d = (int)llabs(f32_key(a) - f32_key(b));
            if (d > mu) mu = d;
        }
    }
    if (n_checked) *n_checked = n;
    if (max_ulp) *max_ulp = mu;
    return bad;
}

/* softmax_inplace (3147-3156), argmax_f (3328-3332), selection and renormalisation (4594-4604) */
void fgo_moe_route(const float *logits, int n_expert, int k, int32_t *sel, float *w) {
    float *p = (float *)malloc((size_t)n_expert * sizeof(float));
    memcpy(p, logits, (size_t)n_expert * sizeof(float));
    float mx = -INFINITY;
    for (int i = 0; i < n_expert; i++) if (p[i] > mx) mx = p[i];
    float sum = 0.0f;
    for (int i = 0; i < n_expert; i++) { p[i] = expf(p[i] - mx); sum += p[i]; }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n_expert; i++) p[i] *= inv;
    }
    float wsum = 0.0f;
    for (int j = 0; j < k; j++) {
        int best = 0;
        float bv = -INFINITY;
        for (int i = 0; i < n_expert; i++) if (p[i] > bv) { bv = p[i]; best = i; }
        sel[j] = best;
        w[j] = p[best];
        wsum += p[best];
        p[best] = -1.0f;
    }
    if (wsum < 6.103515625e-5f) wsum = 6.103515625e-5f;
    for (int j = 0; j < k; j++) w[j] /= wsum;
    free(p);
}

/* the reference's down loop: s = s + w_j * dot (4626-4635). gcc contracts this statement to a
 * fused multiply-add under -O3 -march=native (fp-contract=fast, the GNU C default); the golden
 * vectors written by the compiled reference fix which form is used. */
static float moe_accum(float s, float wj, float dot) {
#if FGO_MUTATE == 2 /* separately rounded multiply and add */
    volatile float p = wj * dot;
    return s + p;
#else
    return fmaf(wj, dot, s);
#endif
}

int fgo_moe_down(uint32_t type_down, const uint8_t *down, int n_embd, int ff, int k,
                 const int32_t *sel, const float *w, const float *h, float *out) {
    if (!type_ok(type_down, ff)) return -1;
    int eb, bb;
    fgo_block_size(type_down, &eb, &bb);
    size_t sd = (size_t)(ff / eb) * bb, ab = act_bytes(type_down, ff);
    uint8_t *act = (uint8_t *)malloc(ab * (size_t)k);
    if (!act) return -1;
    for (int j = 0; j < k; j++) {
        if (float_type(type_down)) memcpy(act + ab * j, h + (size_t)j * ff, ab);
        else if (uses_q8(type_down)) fgo_quantize_q8(h + (size_t)j * ff, (fgo_q8_blk *)(act + ab * j), ff);
        else fgo_quantize_q8k(h + (size_t)j * ff, (fgo_q8k_blk *)(act + ab * j), ff);
    }
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n_embd; i++) {
        float s = 0.0f;
        for (int j = 0; j < k; j++) {
            size_t row = (size_t)sel[j] * n_embd + i;
            s = moe_accum(s, w[j], dot_row3(type_down, FGO_ORDER_ROW, down + row * sd, act + ab * j, ff));
        }
        out[i] = s;
    }
    free(act);
    return 0;
}

int fgo_moe_ffn(uint32_t type_gate, uint32_t type_up, uint32_t type_down,
                const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                int n_expert, int k, int n_embd, int ff, const float *logits,
                const float *X, float *Y, int n_tok, int32_t *sel_out, float *w_out,
                float *h_out) {
    if (!type_ok(type_gate, n_embd) || !type_ok(type_up, n_embd) || !type_ok(type_down, ff)) return -1;
    if (k < 1 || k > n_expert) return -1;
    int eg, bg, eu, bu;
    fgo_block_size(type_gate, &eg, &bg);
    fgo_block_size(type_up, &eu, &bu);
    size_t sg = (size_t)(n_embd / eg) * bg, su = (size_t)(n_embd / eu) * bu;
    int32_t *sel = (int32_t *)malloc((size_t)k * sizeof(int32_t));
    float *w = (float *)malloc((size_t)k * sizeof(float));
    float *h = (float *)malloc((size_t)k * ff * sizeof(float));
    if (!sel || !w || !h) { free(sel); free(w); free(h); return -1; }
    int rc = 0;
    for (int t = 0; t < n_tok && rc == 0; t++) {
        const float *x = X + (size_t)t * n_embd;
        fgo_moe_route(logits + (size_t)t * n_expert, n_expert, k, sel, w);
        void *ag = quantize_for(type_gate, x, n_embd);
        void *au = type_up == type_gate ? ag : quantize_for(type_up, x, n_embd);
#pragma omp parallel for schedule(static)
        for (int r = 0; r < k * ff; r++) {
            size_t row = (size_t)sel[r / ff] * ff + r % ff;
            float gv = dot_row3(type_gate, FGO_ORDER_ROW, gate + row * sg, ag, n_embd);
            float uv = dot_row3(type_up, FGO_ORDER_ROW, up + row * su, au, n_embd);
            h[r] = fgo_silu(gv) * uv;
        }
        if (au != ag) free(au);
        free(ag);
        rc = fgo_moe_down(type_down, down, n_embd, ff, k, sel, w, h, Y + (size_t)t * n_embd);
        if (sel_out) memcpy(sel_out + (size_t)t * k, sel, (size_t)k * sizeof(int32_t));
        if (w_out) memcpy(w_out + (size_t)t * k, w, (size_t)k * sizeof(float));
        if (h_out) memcpy(h_out + (size_t)t * k * ff, h, (size_t)k * ff * sizeof(float));
    }
    free(sel); free(w); free(h);
    return rc;
}

/* ---- B-10: attention, attn_rows (fastgguf.c:3273-3326): its vector path (hd % 32 == 0) and
 * its per-row path (any other hd, 3313-3325) ----
 * Per query row, over positions st..en of the ring cache (slot p % cap, head offset kvo):
 *   score_p = scale * (((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7))), a_l = fma chain over
 *            m of q[8m + l] * k_p[8m + l]   (att_qk_kern 3227-3246 with hsum4_ps 3187-3190);
 *            other hd: score_p = dot_f32v(q, k_p, hd) * scale (1618-1632 in its AVX2 + FMA form:
 *            8-lane fma chains s0 over values 16 i + l and s1 over 16 i + 8 + l, one more 8-value
 *            group into s0 when 8 remain, hsum_ps(s0 + s1), then the last hd % 8 values one fma
 *            each, as gcc contracts `s += a[i] * b[i]` when FMA is available)
 *   softmax_vec (3194-3219): max; e = exp_neg_ps(s - max) over whole groups of 8 (lane l of the
 *            8-wide sum takes e[8g + l] in order), hsum8 of the lanes, then the tail with libm
 *            expf added in order; every value times 1 / sum
 *   o[c] = fma chain over the positions in order of w_p * v_p[c]   (att_v_kern 3249-3270)
 * The vector path's chain walks the union lo..hi of the ranges of the call's rows (here: the rows
 * with the same kvo) with weight 0 outside the row's own range (3296-3309); for finite V that
 * adds nothing (fma(0, v, acc) = acc), while a non-finite v there makes the output NaN. The
 * per-row path's chain walks the row's own range only (3318-3323). */
static float exp_neg(float x) { /* exp_neg_ps (3168-3184), one lane */
    int keep = x > -87.0f;
    x = x > -87.0f ? x : -87.0f; /* max_ps(x, -87): -87 for a NaN */
    float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
    x = fmaf(-fx, 0.693359375f, x);
    x = fmaf(-fx, -2.12194440e-4f, x);
    float y = 1.9875691500E-4f;
    y = fmaf(y, x, 1.3981999507E-3f);
    y = fmaf(y, x, 8.3334519073E-3f);
    y = fmaf(y, x, 4.1665795894E-2f);
    y = fmaf(y, x, 1.6666665459E-1f);
    y = fmaf(y, x, 5.0000001201E-1f);
    float xx = x * x, x1 = x + 1.0f;
    y = fmaf(y, xx, x1);
    uint32_t eb = (uint32_t)((int32_t)fx + 127) << 23;
    float e;
    memcpy(&e, &eb, 4);
    float r = y * e;
    return keep ? r : 0.0f;
}

float fgo_exp_neg(float x) { return exp_neg(x); }

static void softmax_vec_row(float *s, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) if (s[i] > mx) mx = s[i];
    float vs[8] = {0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            s[i + l] = exp_neg(s[i + l] - mx);
            vs[l] += s[i + l];
        }
    float sum = hsum8(vs);
#if FGO_MUTATE == 11 /* the tail through exp_neg_ps instead of libm's expf */
    for (; i < n; i++) { s[i] = exp_neg(s[i] - mx); sum += s[i]; }
#else
    for (; i < n; i++) { s[i] = expf(s[i] - mx); sum += s[i]; }
#endif
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int j = 0; j < n; j++) s[j] = s[j] * inv;
    }
}

/* dot_f32v (fastgguf.c:1618-1632), AVX2 + FMA form */
static float dot_f32v(const float *a, const float *b, int n) {
    float s0[8] = {0}, s1[8] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
            s1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], s1[l]);
        }
    if (i + 8 <= n) {
        for (int l = 0; l < 8; l++) s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
        i += 8;
    }
    float v[8];
    for (int l = 0; l < 8; l++) v[l] = s0[l] + s1[l];
    float s = hsum8(v);
#if FGO_MUTATE == 14 /* the tail multiplied and added in two roundings instead of one fma */
    for (; i < n; i++) s += a[i] * b[i];
#else
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
#endif
    return s;
}

/* ---- the float weight types (dot_row 2207-2214 with x in fp32) ----
 * F32:  dot_f32v over the row's values (1618-1632, above)
 * F16:  dot_f16_row (1645-1656), F16C + AVX2 form: 8 fma chains, chain l over values 8 i + l
 *       (each converted exactly by vcvtph2ps), hsum_ps, then the last n % 8 values one fma each
 *       (gcc's contraction of `s += FP16(h) * x[i]`)
 * BF16: the loop `s += bf16_to_float(h) * x[i]` (2209-2213): one contracted fma chain over the
 *       row in order */
static float dot_f16_row(const uint8_t *row, const float *x, int n) {
    float acc[8] = {0};
    int i = 0;
#if FGO_MUTATE == 18 /* dot_f32v's two accumulators (values 16 i + l and 16 i + 8 + l) */
    float acc2[8] = {0};
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            acc[l] = fmaf(fgo_fp16(rd16(row + 2 * (i + l))), x[i + l], acc[l]);
            acc2[l] = fmaf(fgo_fp16(rd16(row + 2 * (i + 8 + l))), x[i + 8 + l], acc2[l]);
        }
    for (int l = 0; l < 8; l++) acc[l] += acc2[l];
#endif
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(fgo_fp16(rd16(row + 2 * (i + l))), x[i + l], acc[l]);
    float s = hsum8(acc);
    for (; i < n; i++) s = fmaf(fgo_fp16(rd16(row + 2 * i)), x[i], s);
    return s;
}
static float dot_bf16_row(const uint8_t *row, const float *x, int n) {
    float s = 0.0f;
#if FGO_MUTATE == 19 /* the product rounded before the add (no contraction) */
    for (int i = 0; i < n; i++) {
        volatile float p = bf16_f32(rd16(row + 2 * i)) * x[i];
        s += p;
    }
#else
    for (int i = 0; i < n; i++) s = fmaf(bf16_f32(rd16(row + 2 * i)), x[i], s);
#endif
    return s;
}
float fgo_dot_float(uint32_t type, const uint8_t *row, const float *x, int n) {
    if (type == FGO_T_F16) return dot_f16_row(row, x, n);
    if (type == FGO_T_BF16) return dot_bf16_row(row, x, n);
    float *w = (float *)malloc((size_t)n * sizeof(float));  /* the row's values (rd_f32, unaligned) */
    if (!w) return NAN;
    memcpy(w, row, (size_t)n * sizeof(float));
    float s = dot_f32v(w, x, n);
    free(w);
    return s;
}

int fgo_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const float *ck, const float *cv,
                  int kv_dim, const int *kvo, int cap, int hd, float scale) {
    if (hd <= 0) return -1;
    for (int r = 0; r < nr; r++) {
        int n = en[r] - st[r] + 1;
        if (n < 1 || n > cap) return -1;
        float *s = (float *)malloc((size_t)n * sizeof(float));
        if (!s) return -1;
        const float *qr = q + (size_t)r * hd;
        for (int p = st[r]; p <= en[r]; p++) {
            const float *k = ck + (size_t)(p % cap) * kv_dim + kvo[r];
            if (hd % 32 != 0) { /* the per-row path */
                s[p - st[r]] = dot_f32v(qr, k, hd) * scale;
                continue;
            }
            float a[8] = {0};
            for (int m = 0; m < hd / 8; m++)
                for (int l = 0; l < 8; l++) a[l] = fmaf(qr[8 * m + l], k[8 * m + l], a[l]);
#if FGO_MUTATE == 10 /* the 8 score lanes added in sequence instead of hsum4_ps's tree */
            float t = a[0];
            for (int l = 1; l < 8; l++) t += a[l];
#else
            float t = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
#endif
            s[p - st[r]] = t * scale;
        }
        softmax_vec_row(s, n);
        float *orow = o + (size_t)r * hd;
        int lo = st[r], hi = en[r];
        if (hd % 32 == 0)
            for (int r2 = 0; r2 < nr; r2++)
                if (kvo[r2] == kvo[r] && en[r2] >= st[r2]) {
                    lo = st[r2] < lo ? st[r2] : lo;
                    hi = en[r2] > hi ? en[r2] : hi;
                }
        for (int c = 0; c < hd; c++) {
            float acc = 0.0f;
            for (int p = lo; p <= hi; p++) {
                float w = p >= st[r] && p <= en[r] ? s[p - st[r]] : 0.0f;
                acc = fmaf(w, cv[(size_t)(p % cap) * kv_dim + kvo[r] + c], acc);
            }
            orow[c] = acc;
        }
        free(s);
    }
    return 0;
}

/* ---- B-11: TurboQuant KV cache (fastgguf.c:3341-3513) and its attention step (4760-4846) ----
 * Rotation R x = H(D x) / sqrt(n): D the signs of xorshift64* (rng_next 3333-3338) from seed
 * 0x243F6A8885A308D3, bit 63 set -> +1 (kvq_init 3363-3372); H the in-place Walsh-Hadamard
 * butterflies (a + b, a - b), then every value times 1 / sqrtf(n) (kvq_fwht 3375-3386). Inverse:
 * the same transform, then the signs (kvq_unrotate 3396-3400).
 * Slice records (kvq_quant_slice 3415-3444): a float scale, then the codes.
 *   bits 8: s = amax / 127, q = lrintf(x * (1 / s)) (round half to even)
 *   bits 4 / 2: ss = sum in order of the rounded x_i * x_i, s = sqrtf(ss / hd), code = the first c with
 *     u <= (c_c + c_{c+1}) * 0.5 over the Lloyd-Max centroids (kvq_enc4 / kvq_enc2 3403-3412),
 *     u = x * (1 / s); 4-bit codes low nibble first, 2-bit codes low bits first
 * Scores (kvq_dot_k 3447-3462): 4-bit acc = acc + fma(q_i, c[lo], q_{i+1} * c[hi]) per byte (the
 *   contraction of `acc += q_i c_lo + q_{i+1} c_hi` the compiled reference makes: the golden
 *   vectors fix it), 8-bit acc = fma(q_i, code_i, acc); times s, then times scale.
 * Softmax: softmax_inplace (3147-3156): max, e = expf(s - max), the sum in order, times 1 / sum.
 * Values (kvq_axpy_v 3465-3489 from forward 4829-4836): for each position with w != 0, in order,
 *   o_i = fma(w * s, value_i, o_i) with value_i the centroid (4 / 2 bits) or the int8 code. */
static const float KVQ_C4[16] = {-2.7326f, -2.0690f, -1.6181f, -1.2562f, -0.9424f, -0.6568f, -0.3881f, -0.1284f,
                                 0.1284f,  0.3881f,  0.6568f,  0.9424f,  1.2562f,  1.6181f,  2.0690f,  2.7326f};
static const float KVQ_C2[4] = {-1.5104f, -0.4528f, 0.4528f, 1.5104f};

void fgo_kvq_signs(float *out, int n) {
    uint64_t s = 0x243F6A8885A308D3ULL;
    for (int i = 0; i < n; i++) {
        uint64_t x = s;
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        s = x;
        out[i] = ((x * 0x2545F4914F6CDD1DULL) >> 63) ? 1.0f : -1.0f;
    }
}

static void kvq_hadamard(float *x, int n) {
    for (int len = 1; len < n; len <<= 1)
        for (int i = 0; i < n; i += 2 * len)
            for (int j = i; j < i + len; j++) {
                float a = x[j], b = x[j + len];
                x[j] = a + b;
                x[j + len] = a - b;
            }
    float inv = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;
}

int fgo_kvq_rotate(float *x, int n, int inverse) {
    if (n < 2 || n > 1024 || (n & (n - 1))) return -1;
    float sg[1024];
    fgo_kvq_signs(sg, n);
    if (!inverse)
        for (int i = 0; i < n; i++) x[i] = x[i] * sg[i];
    kvq_hadamard(x, n);
    if (inverse)
        for (int i = 0; i < n; i++) x[i] = x[i] * sg[i];
    return 0;
}

int fgo_kvq_rec_bytes(int hd, int bits) { return 4 + hd * bits / 8; }

static int kvq_code(float u, const float *c, int nc) {
    int k = 0;
    while (k < nc - 1 && u > (c[k] + c[k + 1]) * 0.5f) k++;
    return k;
}

int fgo_kvq_quant(const float *x, int hd, uint8_t *rec, int bits) {
    if (bits != 8 && bits != 4 && bits != 2) return -1;
    uint8_t *q = rec + 4;
    float s;
    if (bits == 8) {
        float amax = 0.0f;
        for (int i = 0; i < hd; i++) if (fabsf(x[i]) > amax) amax = fabsf(x[i]);
        s = amax / 127.0f;
        float inv = s > 0.0f ? 1.0f / s : 0.0f;
        for (int i = 0; i < hd; i++) q[i] = (uint8_t)(int8_t)lrintf(x[i] * inv);
    } else {
        float ss = 0.0f;
#if FGO_MUTATE == 13 /* the sum of squares as an fma chain */
        for (int i = 0; i < hd; i++) ss = fmaf(x[i], x[i], ss);
#else
        for (int i = 0; i < hd; i++) ss = ss + x[i] * x[i]; /* not contracted by the compiled reference */
#endif
        s = sqrtf(ss / (float)hd);
        float inv = s > 0.0f ? 1.0f / s : 0.0f;
        if (bits == 4)
            for (int i = 0; i < hd; i += 2)
                q[i / 2] = (uint8_t)(kvq_code(x[i] * inv, KVQ_C4, 16) | kvq_code(x[i + 1] * inv, KVQ_C4, 16) << 4);
        else
            for (int i = 0; i < hd; i += 4)
                q[i / 4] = (uint8_t)(kvq_code(x[i] * inv, KVQ_C2, 4) | kvq_code(x[i + 1] * inv, KVQ_C2, 4) << 2 |
                                     kvq_code(x[i + 2] * inv, KVQ_C2, 4) << 4 | kvq_code(x[i + 3] * inv, KVQ_C2, 4) << 6);
    }
    memcpy(rec, &s, 4);
    return 0;
}

static float kvq_value(const uint8_t *q, int i, int bits) {
    if (bits == 8) return (float)(int8_t)q[i];
    if (bits == 4) return KVQ_C4[(q[i / 2] >> (4 * (i & 1))) & 15];
    return KVQ_C2[(q[i / 4] >> (2 * (i & 3))) & 3];
}

static float kvq_dot(const float *qh, const uint8_t *rec, int hd, int bits) {
    float s, acc = 0.0f;
    memcpy(&s, rec, 4);
    const uint8_t *q = rec + 4;
    if (bits == 8) {
        for (int i = 0; i < hd; i++) acc = fmaf(qh[i], (float)(int8_t)q[i], acc);
    } else {
        for (int i = 0; i < hd; i += 2) {
#if FGO_MUTATE == 12 /* the pair's products rounded separately, no contraction */
            acc = acc + (qh[i] * KVQ_C4[q[i / 2] & 15] + qh[i + 1] * KVQ_C4[q[i / 2] >> 4]);
#else
            acc = acc + fmaf(qh[i], KVQ_C4[q[i / 2] & 15], qh[i + 1] * KVQ_C4[q[i / 2] >> 4]);
#endif
        }
    }
    return acc * s;
}

int fgo_kvq_attn_rows(int nr, const float *q, float *o, const int *st, const int *en, const uint8_t *kq,
                      const uint8_t *vq, int kqs, int vqs, const int *kvh, int cap, int hd, int kbits, int vbits,
                      float scale) {
    if (hd < 2 || hd > 1024 || (hd & (hd - 1)) || (kbits != 4 && kbits != 8) ||
        (vbits != 2 && vbits != 4 && vbits != 8))
        return -1;
    for (int r = 0; r < nr; r++) {
        int n = en[r] - st[r] + 1;
        if (n < 1 || n > cap) return -1;
        float qh[1024];
        memcpy(qh, q + (size_t)r * hd, (size_t)hd * sizeof(float));
        fgo_kvq_rotate(qh, hd, 0);
        float *sc = (float *)malloc((size_t)n * sizeof(float));
        if (!sc) return -1;
        for (int p = st[r]; p <= en[r]; p++)
            sc[p - st[r]] = kvq_dot(qh, kq + (size_t)(p % cap) * kqs + (size_t)kvh[r] * fgo_kvq_rec_bytes(hd, kbits),
                                    hd, kbits) * scale;
        float mx = -INFINITY, sum = 0.0f;
        for (int i = 0; i < n; i++) if (sc[i] > mx) mx = sc[i];
        for (int i = 0; i < n; i++) { sc[i] = expf(sc[i] - mx); sum += sc[i]; }
        if (sum > 0.0f) {
            float inv = 1.0f / sum;
            for (int i = 0; i < n; i++) sc[i] = sc[i] * inv;
        }
        float *oh = o + (size_t)r * hd;
        for (int i = 0; i < hd; i++) oh[i] = 0.0f;
        for (int p = st[r]; p <= en[r]; p++) {
            float w = sc[p - st[r]];
            if (w == 0.0f) continue;
            const uint8_t *rec = vq + (size_t)(p % cap) * vqs + (size_t)kvh[r] * fgo_kvq_rec_bytes(hd, vbits);
            float s;
            memcpy(&s, rec, 4);
            float ws = w * s;
            for (int i = 0; i < hd; i++) oh[i] = fmaf(ws, kvq_value(rec + 4, i, vbits), oh[i]);
        }
        fgo_kvq_rotate(oh, hd, 1);
        free(sc);
    }
    return 0;
}
