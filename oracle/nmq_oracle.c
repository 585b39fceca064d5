/*
 * CPU oracle for the GGUF quantized mat-vec path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker (or as the timed CPU baseline).  Nothing in the product path calls it.
 *
 * It restates, in plain C with IEEE fp32 semantics (built with -ffp-contract=off, no fast-math),
 * the arithmetic of the reference's CPU path:
 *   - the block layouts and dequantisers of ggufengine/quant.py (Q4_0, Q8_0, Q4_K, Q6_K, IQ2_XXS, TQ2_0),
 *   - the two-stage int8 activation quantiser of ggufengine/mmvq.py (quant32 / quant_q8),
 *   - the integer decomposition used by the int8 kernels (per-16-value int32 sums) and the
 *     fp combine of mmvq.py / cudakern.py, accumulated in fp64,
 *   - the "dequantise + fp32 matmul" path of models/common.py (accumulated in fp64 here).
 *
 * Pinning (which checks fix each function) is listed in the header comment of each function and
 * exercised by tests/test_oracle.py; a function with no such check says "parity unpinned".
 *
 * Format ids are the GGML type ids of ggufengine/gguf.py:64-78.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "iq2xxs_grid.h"

#define OR_Q4_0 2
#define OR_Q8_0 8
#define OR_Q4_K 12
#define OR_Q6_K 14
#define OR_IQ2_XXS 16
#define OR_TQ2_0 35

/* ---- scalar helpers --------------------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact for every input (quant.py:21-23 views bytes as float16 then
 * .float()).  Pinned: exhaustive comparison against numpy's float16 over all 65536 bit patterns. */
float or_half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) & 1u, e = (uint32_t)(h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24); /* zero or subnormal: m * 2^-24, exact */
    } else if (e == 31) {
        uint32_t bits = 0x7f800000u | (m << 13);
        memcpy(&v, &bits, 4);
    } else {
        uint32_t bits = ((e + 112u) << 23) | (m << 13);
        memcpy(&v, &bits, 4);
    }
    return s ? -v : v;
}

/* binary32 -> bfloat16 -> binary32, round to nearest even (torch's .to(torch.bfloat16), used by
 * cudakern.mv / mm at cudakern.py:764, 786 and Eingang at mmvq.py:831).  Pinned against torch. */
float or_round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f; /* NaN passes through */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* ggml get_scale_min_k4: quant.py:99-108 (vectorised) and mmvq.py:333-336 (per sub-block). */
static void scale_min_k4(const uint8_t* sc, int j, int* d, int* m) {
    if (j < 4) {
        *d = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *d = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

static int popcount7(uint32_t s) {
    int c = 0;
    for (int j = 0; j < 7; ++j) c += (s >> j) & 1u;
    return c;
}

int or_format_info(int fmt, int* block_values, int* block_bytes) {
    switch (fmt) {
        case OR_Q4_0: *block_values = 32; *block_bytes = 18; return 0;
        case OR_Q8_0: *block_values = 32; *block_bytes = 34; return 0;
        case OR_Q4_K: *block_values = 256; *block_bytes = 144; return 0;
        case OR_Q6_K: *block_values = 256; *block_bytes = 210; return 0;
        case OR_IQ2_XXS: *block_values = 256; *block_bytes = 66; return 0;
        case OR_TQ2_0: *block_values = 256; *block_bytes = 66; return 0;
        default: return -1;
    }
}

/* ---- dequantisers (quant.py) ------------------------------------------------------------------ */

/* quant.py:60-64 deq_q4_0 with _nibbles (:53-57): the 16 low nibbles of qs are values 0..15, the
 * high nibbles values 16..31; d * (q - 8). */
static void deq_q4_0(const uint8_t* b, float* out) {
    const float d = or_half_to_float(rd16(b));
    for (int j = 0; j < 16; ++j) {
        out[j] = d * (float)((b[2 + j] & 15) - 8);
        out[16 + j] = d * (float)((b[2 + j] >> 4) - 8);
    }
}

/* quant.py:46-50 deq_q8_0: d * q. */
static void deq_q8_0(const uint8_t* b, float* out) {
    const float d = or_half_to_float(rd16(b));
    for (int j = 0; j < 32; ++j) out[j] = d * (float)(int8_t)b[2 + j];
}

/* quant.py:111-120 deq_q4_k: (d*sc)*q - (dmin*mn); sub-block 2i = low nibbles of qs[32i..32i+32),
 * 2i+1 = high nibbles. */
static void deq_q4_k(const uint8_t* b, float* out) {
    const float d = or_half_to_float(rd16(b)), dmin = or_half_to_float(rd16(b + 2));
    for (int i = 0; i < 4; ++i) {
        int sc0, m0, sc1, m1;
        scale_min_k4(b + 4, 2 * i, &sc0, &m0);
        scale_min_k4(b + 4, 2 * i + 1, &sc1, &m1);
        const float a0 = d * (float)sc0, c0 = dmin * (float)m0;
        const float a1 = d * (float)sc1, c1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = b[16 + 32 * i + l];
            out[64 * i + l] = a0 * (float)(q & 15) - c0;
            out[64 * i + 32 + l] = a1 * (float)(q >> 4) - c1;
        }
    }
}

/* quant.py:140-159 deq_q6_k: two halves of 128; q1..q4 from ql/qh; (d*sc)*(q-32). */
static void deq_q6_k(const uint8_t* b, float* out) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = or_half_to_float(rd16(b + 208));
    for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
            const int q1 = (ql[64 * n + l] & 15) | (((qh[32 * n + l] >> 0) & 3) << 4);
            const int q2 = (ql[64 * n + 32 + l] & 15) | (((qh[32 * n + l] >> 2) & 3) << 4);
            const int q3 = (ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4);
            const int q4 = (ql[64 * n + 32 + l] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4);
            const int qq[4] = {q1, q2, q3, q4};
            for (int k = 0; k < 4; ++k) {
                const float s = (float)sc[8 * n + 2 * k + l / 16];
                out[128 * n + 32 * k + l] = (d * s) * (float)(qq[k] - 32);
            }
        }
    }
}

/* quant.py:417-421 deq_tq2_0: value 128n + 32l + m = d * (((qs[32n+m] >> 2l) & 3) - 1). */
static void deq_tq2_0(const uint8_t* b, float* out) {
    const float d = or_half_to_float(rd16(b + 64));
    for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 4; ++l)
            for (int m = 0; m < 32; ++m)
                out[128 * n + 32 * l + m] = d * (float)(((b[32 * n + m] >> (2 * l)) & 3) - 1);
}

/* quant.py:235-245 deq_iq2_xxs with the table of quant.py:170-213:
 * value = (grid byte * sign) * (d * (0.125 + 0.25 * ls)); sign bit 7 = parity of the 7 stored bits
 * (ksigns_iq2xs, cudakern.py:67). */
static void deq_iq2_xxs(const uint8_t* b, float* out) {
    const float d = or_half_to_float(rd16(b));
    for (int ib = 0; ib < 8; ++ib) {
        const uint8_t* q = b + 2 + 8 * ib;
        const uint32_t aux1 = rd32(q + 4);
        const float db = d * (0.125f + 0.25f * (float)(aux1 >> 28));
        for (int l = 0; l < 4; ++l) {
            const unsigned long long g = OR_IQ2XXS_GRID[q[l]];
            uint32_t s = (aux1 >> (7 * l)) & 127u;
            s |= (uint32_t)(popcount7(s) & 1) << 7;
            for (int j = 0; j < 8; ++j) {
                const float v = (float)((g >> (8 * j)) & 255u);
                out[32 * ib + 8 * l + j] = ((s >> j) & 1u ? -v : v) * db;
            }
        }
    }
}

/* quant.py:484-503 dequantize: flat fp32 of n_blocks blocks.  Returns 0 or -1 (unknown format). */
int or_dequant(int fmt, const uint8_t* raw, int64_t n_blocks, float* out) {
    int bv, bb;
    if (or_format_info(fmt, &bv, &bb)) return -1;
    for (int64_t i = 0; i < n_blocks; ++i) {
        const uint8_t* b = raw + i * bb;
        float* o = out + i * bv;
        switch (fmt) {
            case OR_Q4_0: deq_q4_0(b, o); break;
            case OR_Q8_0: deq_q8_0(b, o); break;
            case OR_Q4_K: deq_q4_k(b, o); break;
            case OR_Q6_K: deq_q6_k(b, o); break;
            case OR_IQ2_XXS: deq_iq2_xxs(b, o); break;
            case OR_TQ2_0: deq_tq2_0(b, o); break;
        }
    }
    return 0;
}

/* ---- two-stage int8 activation (mmvq.py:59-83) ------------------------------------------------- */

/* Per 32 values: d = max|x| / 127 (IEEE division), xq = rint(x / d) (half-even, as
 * __float2int_rn), residual r = x - xq*d evaluated as ONE fused multiply-add (the pinned choice;
 * the reference compiles with --use_fast_math where the contraction and the division are not
 * specified), xq2 = clamp(rint(r / (d * (1/254))), -127, 127), xs = sum of the 32 values added in the
 * xor-butterfly order of warp_sum (offsets 16, 8, 4, 2, 1; mmvq.py:42-46).  d == 0 -> xq = xq2 = 0.
 * n % 32 == 0.  Pinned: closed forms (all-equal block, zero block, single spike), the reconstruction
 * bound |x - xq*d - xq2*d/254| <= d/508 (+ rounding), and bit-exact agreement with the GPU kernel. */
void or_quant_q8(const float* x, int64_t n, int8_t* xq, int8_t* xq2, float* xd, float* xs) {
    const float fein = 1.0f / 254.0f;
    for (int64_t g = 0; g < n / 32; ++g) {
        const float* v = x + 32 * g;
        float a = 0.0f;
        for (int j = 0; j < 32; ++j) a = fmaxf(a, fabsf(v[j]));
        const float d = a / 127.0f;
        for (int j = 0; j < 32; ++j) {
            int q = 0, q2 = 0;
            if (d > 0.0f) {
                q = (int)rintf(v[j] / d);
                const float r = fmaf(-(float)q, d, v[j]);
                q2 = (int)rintf(r / (d * fein));
                q2 = q2 < -127 ? -127 : (q2 > 127 ? 127 : q2);
            }
            xq[32 * g + j] = (int8_t)q;
            xq2[32 * g + j] = (int8_t)q2;
        }
        float t[32];
        for (int j = 0; j < 32; ++j) t[j] = v[j];
        for (int o = 16; o > 0; o >>= 1)
            for (int j = 0; j < o; ++j) t[j] = t[j] + t[j + o];
        xd[g] = d;
        xs[g] = t[0];
    }
}

/* ---- integer decomposition ---------------------------------------------------------------------
 * For each format: the int8 weight w of every value (the quantity multiplied with xq / xq2 by the
 * int8 kernels) and the fp32 factors applied per 16 values.
 *   Q4_K  w = nibble 0..15, scale d*sc_s per sub-block s, min term dmin*m_s*xs_s  (mmvq.py:341-419)
 *   Q6_K  w = q - 32, scale d*sc16                                                (mmvq.py:421-482)
 *   Q4_0  w = nibble - 8, scale d                                                 (cudakern.py:315-321)
 *   Q8_0  w = qs, scale d                                                         (cudakern.py:307-313)
 *   TQ2_0 w = code - 1, scale d                                                   (cudakern.py:432-439)
 *   IQ2_XXS w = +-grid byte, scale d*(0.125+0.25*ls) per 32                        (cudakern.py:187-195)
 * wscale[g] is the weight factor for values 16g..16g+15 of the block (fp64, exact products);
 * wmin[s] is the Q4_K min factor dmin*m_s for sub-block s (0 for other formats). */
static void decode_int(int fmt, const uint8_t* b, int8_t* w, double* wscale, double* wmin) {
    switch (fmt) {
        case OR_Q4_0: {
            const double d = or_half_to_float(rd16(b));
            for (int j = 0; j < 16; ++j) {
                w[j] = (int8_t)((b[2 + j] & 15) - 8);
                w[16 + j] = (int8_t)((b[2 + j] >> 4) - 8);
            }
            wscale[0] = wscale[1] = d;
            wmin[0] = 0.0;
            break;
        }
        case OR_Q8_0: {
            const double d = or_half_to_float(rd16(b));
            for (int j = 0; j < 32; ++j) w[j] = (int8_t)b[2 + j];
            wscale[0] = wscale[1] = d;
            wmin[0] = 0.0;
            break;
        }
        case OR_Q4_K: {
            const double d = or_half_to_float(rd16(b)), dmin = or_half_to_float(rd16(b + 2));
            for (int i = 0; i < 4; ++i) {
                for (int l = 0; l < 32; ++l) {
                    w[64 * i + l] = (int8_t)(b[16 + 32 * i + l] & 15);
                    w[64 * i + 32 + l] = (int8_t)(b[16 + 32 * i + l] >> 4);
                }
            }
            for (int s = 0; s < 8; ++s) {
                int sc, m;
                scale_min_k4(b + 4, s, &sc, &m);
                wscale[2 * s] = wscale[2 * s + 1] = d * sc;
                wmin[s] = dmin * m;
            }
            break;
        }
        case OR_Q6_K: {
            const uint8_t* ql = b;
            const uint8_t* qh = b + 128;
            const int8_t* sc = (const int8_t*)(b + 192);
            const double d = or_half_to_float(rd16(b + 208));
            for (int n = 0; n < 2; ++n)
                for (int l = 0; l < 32; ++l) {
                    w[128 * n + l] = (int8_t)(((ql[64 * n + l] & 15) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32);
                    w[128 * n + 32 + l] =
                        (int8_t)(((ql[64 * n + 32 + l] & 15) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32);
                    w[128 * n + 64 + l] = (int8_t)(((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32);
                    w[128 * n + 96 + l] =
                        (int8_t)(((ql[64 * n + 32 + l] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32);
                }
            for (int g = 0; g < 16; ++g) wscale[g] = d * sc[g];
            for (int s = 0; s < 8; ++s) wmin[s] = 0.0;
            break;
        }
        case OR_TQ2_0: {
            const double d = or_half_to_float(rd16(b + 64));
            for (int n = 0; n < 2; ++n)
                for (int l = 0; l < 4; ++l)
                    for (int m = 0; m < 32; ++m)
                        w[128 * n + 32 * l + m] = (int8_t)(((b[32 * n + m] >> (2 * l)) & 3) - 1);
            for (int g = 0; g < 16; ++g) wscale[g] = d;
            for (int s = 0; s < 8; ++s) wmin[s] = 0.0;
            break;
        }
        case OR_IQ2_XXS: {
            const double d = or_half_to_float(rd16(b));
            for (int ib = 0; ib < 8; ++ib) {
                const uint8_t* q = b + 2 + 8 * ib;
                const uint32_t aux1 = rd32(q + 4);
                for (int l = 0; l < 4; ++l) {
                    const unsigned long long g = OR_IQ2XXS_GRID[q[l]];
                    uint32_t s = (aux1 >> (7 * l)) & 127u;
                    s |= (uint32_t)(popcount7(s) & 1) << 7;
                    for (int j = 0; j < 8; ++j) {
                        const int v = (int)((g >> (8 * j)) & 255u);
                        w[32 * ib + 8 * l + j] = (int8_t)((s >> j) & 1u ? -v : v);
                    }
                }
                wscale[2 * ib] = wscale[2 * ib + 1] = d * (0.125 + 0.25 * (double)(aux1 >> 28));
                wmin[ib] = 0.0;
            }
            break;
        }
    }
}

/* int32 sums per 16 weights of each row: s1[r][g] = sum w*xq, s2[r][g] = sum w*xq2 over values
 * 16g..16g+15 (one token; xq/xq2 of length n_in).  Pinned: brute force on tiny inputs in the tests
 * (an independent numpy path over the dequantised integer weights) and the mat-vec identities. */
int or_block_sums(int fmt, const uint8_t* raw, int n_out, int n_in, const int8_t* xq, const int8_t* xq2,
                  int32_t* s1, int32_t* s2) {
    int bv, bb;
    if (or_format_info(fmt, &bv, &bb) || n_in % bv) return -1;
    const int nb = n_in / bv;
    int8_t w[256];
    double ws[16], wm[8];
    for (int r = 0; r < n_out; ++r) {
        for (int blk = 0; blk < nb; ++blk) {
            decode_int(fmt, raw + ((int64_t)r * nb + blk) * bb, w, ws, wm);
            for (int g = 0; g < bv / 16; ++g) {
                int32_t a = 0, c = 0;
                for (int j = 0; j < 16; ++j) {
                    const int k = blk * bv + 16 * g + j;
                    a += (int32_t)w[16 * g + j] * xq[k];
                    c += (int32_t)w[16 * g + j] * xq2[k];
                }
                s1[(int64_t)r * (n_in / 16) + blk * (bv / 16) + g] = a;
                s2[(int64_t)r * (n_in / 16) + blk * (bv / 16) + g] = c;
            }
        }
    }
    return 0;
}

/* Mat-vec through the integer decomposition, combined in fp64:
 *   y[c][r] = sum_g wscale_g * xd_(g/2) * (S1_g + S2_g / 254) - sum_s wmin_s * xs_s
 * for ncols tokens whose two-stage inputs lie at c*n_in (xq, xq2) and c*n_in/32 (xd, xs).
 * This is the arithmetic of the int8 kernels (mmvq.py:395-398, 472-474) without fp32 rounding. */
int or_mv_int(int fmt, const uint8_t* raw, int n_out, int n_in, const int8_t* xq, const int8_t* xq2,
              const float* xd, const float* xs, int ncols, double* y) {
    int bv, bb;
    if (or_format_info(fmt, &bv, &bb) || n_in % bv) return -1;
    const int nb = n_in / bv;
    int8_t w[256];
    double ws[16], wm[8];
    for (int c0 = 0; c0 < ncols; c0 += 64) {  /* tokens in chunks of 64 (one accumulator each) */
        const int nc = ncols - c0 < 64 ? ncols - c0 : 64;
        for (int r = 0; r < n_out; ++r) {
            double acc[64];
            for (int c = 0; c < nc; ++c) acc[c] = 0.0;
            for (int blk = 0; blk < nb; ++blk) {
                decode_int(fmt, raw + ((int64_t)r * nb + blk) * bb, w, ws, wm);
                for (int c = 0; c < nc; ++c) {
                    const int64_t t = c0 + c;
                    const int8_t* q1 = xq + t * n_in + blk * bv;
                    const int8_t* q2 = xq2 + t * n_in + blk * bv;
                    const float* d = xd + (t * n_in + blk * bv) / 32;
                    const float* s = xs + (t * n_in + blk * bv) / 32;
                    for (int g = 0; g < bv / 16; ++g) {
                        int32_t a = 0, e = 0;
                        for (int j = 0; j < 16; ++j) {
                            a += (int32_t)w[16 * g + j] * q1[16 * g + j];
                            e += (int32_t)w[16 * g + j] * q2[16 * g + j];
                        }
                        acc[c] += ws[g] * (double)d[g / 2] * ((double)a + (double)e / 254.0);
                    }
                    if (fmt == OR_Q4_K)
                        for (int sb = 0; sb < 8; ++sb) acc[c] -= wm[sb] * (double)s[sb];
                }
            }
            for (int c = 0; c < nc; ++c) y[(c0 + c) * (int64_t)n_out + r] = acc[c];
        }
    }
    return 0;
}

/* The reference's "dequantise + matmul" path (models/common.py:414-428, 516-527) with fp64
 * accumulation: y[c][r] = sum_k deq(W)[r][k] * x[c][k].  x is taken as given (callers round it to
 * bf16 first where the reference does). */
int or_mv_deq(int fmt, const uint8_t* raw, int n_out, int n_in, const float* x, int ncols, double* y) {
    int bv, bb;
    if (or_format_info(fmt, &bv, &bb) || n_in % bv) return -1;
    const int nb = n_in / bv;
    float row[256];
    for (int r = 0; r < n_out; ++r) {
        for (int c = 0; c < ncols; ++c) y[(int64_t)c * n_out + r] = 0.0;
        for (int blk = 0; blk < nb; ++blk) {
            or_dequant(fmt, raw + ((int64_t)r * nb + blk) * bb, 1, row);
            for (int c = 0; c < ncols; ++c) {
                const float* xc = x + (int64_t)c * n_in + blk * bv;
                double a = 0.0;
                for (int j = 0; j < bv; ++j) a += (double)row[j] * (double)xc[j];
                y[(int64_t)c * n_out + r] += a;
            }
        }
    }
    return 0;
}
