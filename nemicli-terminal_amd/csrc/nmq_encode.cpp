// Host-side GGUF block encoders of libnmq (nmq_encode in include/nmq.h).
//
// The reference reads these formats from GGUF files and ships no quantiser for Q4_K, Q6_K or
// IQ2_XXS; its tests only pack Q8_0 (tests/test_bildmotoren.py:31-37) and the ternary formats
// (tests/test_gguf_ternaer.py:143-154).  These encoders write the block layouts the reference's
// dequantisers read (ggufengine/quant.py), with this library's own choice of scales:
//   Q8_0    d = max|x| / 127, q = round(x / d)                     (as quantize_row_q8_0 in ggml)
//   Q4_0    d = -m / 8 with m the value of largest magnitude, q = min(15, trunc(x / d + 8.5))
//           (as quantize_row_q4_0 in ggml: m itself maps to nibble 0)
//   Q4_K    per 32: least-squares scale and min over a few step candidates, then 6-bit sub-scales
//           relative to fp16 d / dmin
//   Q6_K    per 16: the largest-magnitude value maps to -32; int8 sub-scales relative to fp16 d
//   TQ2_0   d = max|x|, code = round(x / d) + 1 (lossless for ternary input d * {-1, 0, 1})
//   IQ2_XXS per 8 values: signs (even parity), the grid entry of best least-squares fit for the
//           sub-block's scale; per 32 a 4-bit scale relative to fp16 d
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/nmq.h"

namespace {

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

const u64 GRID[256] = {
#include "iq2xxs_grid.inc"
};

// binary32 -> binary16, round to nearest even (overflow to inf, subnormals kept).
u16 f2h(float f) {
    u32 x;
    memcpy(&x, &f, 4);
    const u32 sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return (u16)(sign | 0x7c00u | (x > 0x7f800000u ? 0x200u : 0u));
    if (x >= 0x477ff000u) return (u16)(sign | 0x7c00u);  // rounds to >= 65520: inf
    if (x < 0x38800000u) {                                // below the smallest normal half
        if (x < 0x33000000u) return (u16)sign;            // < 2^-25: rounds to zero
        const u32 e = x >> 23, m = (x & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)e;                   // 14 + (113 - e)
        const u32 r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        return (u16)(sign | (r + (rem > half || (rem == half && (r & 1u)))));
    }
    const u32 r = ((x >> 13) - (112u << 10)), rem = x & 0x1fffu;
    return (u16)(sign | (r + (rem > 0x1000u || (rem == 0x1000u && (r & 1u)))));
}

float h2f(u16 h) {
    const u32 s = (u32)(h >> 15), e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24);
    } else if (e == 31) {
        u32 b = 0x7f800000u | (m << 13);
        memcpy(&v, &b, 4);
    } else {
        u32 b = ((e + 112u) << 23) | (m << 13);
        memcpy(&v, &b, 4);
    }
    return s ? -v : v;
}

inline int nearest(float v) { return (int)lrintf(v); }
inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
inline void put16(u8* p, u16 v) { p[0] = (u8)v; p[1] = (u8)(v >> 8); }
inline void put32(u8* p, u32 v) {
    p[0] = (u8)v; p[1] = (u8)(v >> 8); p[2] = (u8)(v >> 16); p[3] = (u8)(v >> 24);
}

// ---- Q8_0 ----
void enc_q8_0(const float* x, u8* b) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, fabsf(x[j]));
    const float d = amax / 127.f, id = d > 0.f ? 1.f / d : 0.f;
    put16(b, f2h(d));
    for (int j = 0; j < 32; ++j) b[2 + j] = (u8)(int8_t)clampi((int)roundf(x[j] * id), -127, 127);
}

// ---- Q4_0 ----
void enc_q4_0(const float* x, u8* b) {
    float amax = 0.f, m = 0.f;
    for (int j = 0; j < 32; ++j)
        if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); m = x[j]; }
    const float d = m / -8.f, id = d != 0.f ? 1.f / d : 0.f;
    put16(b, f2h(d));
    for (int j = 0; j < 16; ++j) {
        const int lo = std::min(15, (int)(x[j] * id + 8.5f)), hi = std::min(15, (int)(x[j + 16] * id + 8.5f));
        b[2 + j] = (u8)(lo | (hi << 4));
    }
}

// ---- Q4_K ----
// Fit x ~ a*q - bmin (q in 0..15, a >= 0, bmin >= 0) for one sub-block of 32.
void fit_q4(const float* x, float* a_out, float* b_out) {
    float mn = x[0], mx = x[0];
    for (int j = 1; j < 32; ++j) { mn = std::min(mn, x[j]); mx = std::max(mx, x[j]); }
    if (mn > 0.f) mn = 0.f;
    if (mx - mn < 1e-30f) { *a_out = 0.f; *b_out = -mn; return; }
    float best_err = INFINITY, best_a = (mx - mn) / 15.f, best_b = -mn;
    for (int st = -8; st <= 8; ++st) {
        const float iscale = (15.f + 0.1f * st) / (mx - mn);
        int q[32];
        double sq = 0, sq2 = 0, sx = 0, sqx = 0;
        for (int j = 0; j < 32; ++j) {
            q[j] = clampi(nearest(iscale * (x[j] - mn)), 0, 15);
            sq += q[j]; sq2 += (double)q[j] * q[j]; sx += x[j]; sqx += (double)q[j] * x[j];
        }
        // least squares x = a q + c with c = -bmin <= 0
        const double det = 32.0 * sq2 - sq * sq;
        double a, c;
        if (det > 0) {
            a = (32.0 * sqx - sq * sx) / det;
            c = (sq2 * sx - sq * sqx) / det;
        } else {
            a = 0; c = sx / 32.0;
        }
        if (c > 0) { c = 0; a = sq2 > 0 ? sqx / sq2 : 0; }
        if (a < 0) a = 0;
        double err = 0;
        for (int j = 0; j < 32; ++j) {
            const double e = a * q[j] + c - x[j];
            err += e * e;
        }
        if (err < best_err) { best_err = (float)err; best_a = (float)a; best_b = (float)-c; }
    }
    *a_out = best_a;
    *b_out = best_b;
}

void enc_q4_k(const float* x, u8* b) {
    float a[8], bm[8];
    float amax = 0.f, bmax = 0.f;
    for (int s = 0; s < 8; ++s) {
        fit_q4(x + 32 * s, &a[s], &bm[s]);
        amax = std::max(amax, a[s]);
        bmax = std::max(bmax, bm[s]);
    }
    const u16 dh = f2h(amax / 63.f), mh = f2h(bmax / 63.f);
    const float d = h2f(dh), dmin = h2f(mh);
    int sc[8], m[8];
    for (int s = 0; s < 8; ++s) {
        sc[s] = d > 0.f ? clampi(nearest(a[s] / d), 0, 63) : 0;
        m[s] = dmin > 0.f ? clampi(nearest(bm[s] / dmin), 0, 63) : 0;
    }
    put16(b, dh);
    put16(b + 2, mh);
    u8* scales = b + 4;
    for (int j = 0; j < 4; ++j) {
        scales[j] = (u8)(sc[j] | ((sc[j + 4] >> 4) << 6));
        scales[j + 4] = (u8)(m[j] | ((m[j + 4] >> 4) << 6));
        scales[j + 8] = (u8)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    int q[256];
    for (int s = 0; s < 8; ++s) {
        const float ds = d * (float)sc[s], ms = dmin * (float)m[s];
        for (int j = 0; j < 32; ++j)
            q[32 * s + j] = ds > 0.f ? clampi(nearest((x[32 * s + j] + ms) / ds), 0, 15) : 0;
    }
    for (int i = 0; i < 4; ++i)
        for (int l = 0; l < 32; ++l) b[16 + 32 * i + l] = (u8)(q[64 * i + l] | (q[64 * i + 32 + l] << 4));
}

// ---- Q6_K ----
void enc_q6_k(const float* x, u8* b) {
    float s[16];
    float smax = 0.f;
    for (int g = 0; g < 16; ++g) {
        float best = 0.f;
        for (int j = 0; j < 16; ++j)
            if (fabsf(x[16 * g + j]) > fabsf(best)) best = x[16 * g + j];
        s[g] = best / -32.f;
        smax = std::max(smax, fabsf(s[g]));
    }
    const u16 dh = f2h(smax / 127.f);
    const float d = h2f(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = (int8_t)(d > 0.f ? clampi(nearest(s[g] / d), -127, 127) : 0);
    int q[256];
    for (int g = 0; g < 16; ++g) {
        const float f = d * (float)sc[g];
        for (int j = 0; j < 16; ++j) q[16 * g + j] = f != 0.f ? clampi(nearest(x[16 * g + j] / f), -32, 31) + 32 : 32;
    }
    u8* ql = b;
    u8* qh = b + 128;
    memset(b, 0, 192);
    for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
            const int q1 = q[128 * n + l], q2 = q[128 * n + 32 + l], q3 = q[128 * n + 64 + l], q4 = q[128 * n + 96 + l];
            ql[64 * n + l] = (u8)((q1 & 15) | ((q3 & 15) << 4));
            ql[64 * n + 32 + l] = (u8)((q2 & 15) | ((q4 & 15) << 4));
            qh[32 * n + l] = (u8)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    memcpy(b + 192, sc, 16);
    put16(b + 208, dh);
}

// ---- TQ2_0 ----
void enc_tq2_0(const float* x, u8* b) {
    float amax = 0.f;
    for (int j = 0; j < 256; ++j) amax = std::max(amax, fabsf(x[j]));
    const float id = amax > 0.f ? 1.f / amax : 0.f;
    memset(b, 0, 64);
    for (int h = 0; h < 2; ++h)
        for (int l = 0; l < 4; ++l)
            for (int m = 0; m < 32; ++m) {
                const int q = clampi((int)roundf(x[128 * h + 32 * l + m] * id), -1, 1) + 1;
                b[32 * h + m] |= (u8)(q << (2 * l));
            }
    put16(b + 64, f2h(amax));
}

// ---- IQ2_XXS ----
struct Grid {
    float g[256][8];
    float gg[256];
    Grid() {
        for (int e = 0; e < 256; ++e) {
            gg[e] = 0.f;
            for (int j = 0; j < 8; ++j) {
                g[e][j] = (float)((GRID[e] >> (8 * j)) & 255u);
                gg[e] += g[e][j] * g[e][j];
            }
        }
    }
};
const Grid& grid() {
    static const Grid G;
    return G;
}

// One group of 8: sign pattern (even parity) and the dot products of its signed magnitudes with
// every grid entry.
struct Group8 {
    u32 s7;
    float dots[256];
};

void group_prepare(const float* x, Group8& o) {
    u32 neg = 0;
    int cnt = 0, jmin = 0;
    for (int j = 0; j < 8; ++j) {
        if (x[j] < 0.f) { neg |= 1u << j; ++cnt; }
        if (fabsf(x[j]) < fabsf(x[jmin])) jmin = j;
    }
    if (cnt & 1) neg ^= 1u << jmin;  // odd count: flip the smallest value's sign
    float t[8];
    for (int j = 0; j < 8; ++j) t[j] = (neg >> j) & 1u ? -x[j] : x[j];
    const Grid& G = grid();
    for (int e = 0; e < 256; ++e) {
        float s = 0.f;
        for (int j = 0; j < 8; ++j) s += t[j] * G.g[e][j];
        o.dots[e] = s;
    }
    o.s7 = neg & 127u;
}

int group_best(const Group8& g, float sigma, float* score) {
    const Grid& G = grid();
    int best = 0;
    float bs = -INFINITY;
    for (int e = 0; e < 256; ++e) {
        const float v = 2.f * sigma * g.dots[e] - sigma * sigma * G.gg[e];
        if (v > bs) { bs = v; best = e; }
    }
    *score = bs;
    return best;
}

void enc_iq2_xxs(const float* x, u8* b) {
    const Grid& G = grid();
    Group8 grp[32];
    for (int i = 0; i < 32; ++i) group_prepare(x + 8 * i, grp[i]);
    float sig[8];
    for (int s = 0; s < 8; ++s) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, fabsf(x[32 * s + j]));
        float best_sigma = amax / 43.f, best_score = -INFINITY;
        for (int c = 0; c < 12; ++c) {
            float sigma = amax / 43.f * (0.55f + 0.05f * c);
            for (int it = 0; it < 2; ++it) {  // refit sigma to the chosen entries
                double num = 0, den = 0;
                for (int l = 0; l < 4; ++l) {
                    float sc;
                    const int e = group_best(grp[4 * s + l], sigma, &sc);
                    num += grp[4 * s + l].dots[e];
                    den += G.gg[e];
                }
                if (den > 0 && num > 0) sigma = (float)(num / den);
            }
            float tot = 0.f;
            for (int l = 0; l < 4; ++l) {
                float sc;
                group_best(grp[4 * s + l], sigma, &sc);
                tot += sc;
            }
            if (tot > best_score) { best_score = tot; best_sigma = sigma; }
        }
        sig[s] = best_sigma > 0.f ? best_sigma : 0.f;
    }
    float smax = 0.f;
    for (int s = 0; s < 8; ++s) smax = std::max(smax, sig[s]);
    const u16 dh = f2h(smax * 8.f / 31.f);
    const float d = h2f(dh);
    put16(b, dh);
    for (int s = 0; s < 8; ++s) {
        const int ls = d > 0.f ? clampi(nearest((8.f * sig[s] / d - 1.f) * 0.5f), 0, 15) : 0;
        const float sigma = d * (0.125f + 0.25f * (float)ls);
        u32 aux0 = 0, aux1 = (u32)ls << 28;
        for (int l = 0; l < 4; ++l) {
            float sc;
            const int e = group_best(grp[4 * s + l], sigma, &sc);
            aux0 |= (u32)e << (8 * l);
            aux1 |= grp[4 * s + l].s7 << (7 * l);
        }
        put32(b + 2 + 8 * s, aux0);
        put32(b + 6 + 8 * s, aux1);
    }
}

typedef void (*EncFn)(const float*, u8*);

}  // namespace

extern "C" int64_t nmq_encode(int fmt, const float* w, int64_t n, uint8_t* out, int threads) {
    int bv, bb;
    EncFn fn;
    switch (fmt) {
        case NMQ_Q4_0: bv = 32; bb = 18; fn = enc_q4_0; break;
        case NMQ_Q8_0: bv = 32; bb = 34; fn = enc_q8_0; break;
        case NMQ_Q4_K: bv = 256; bb = 144; fn = enc_q4_k; break;
        case NMQ_Q6_K: bv = 256; bb = 210; fn = enc_q6_k; break;
        case NMQ_TQ2_0: bv = 256; bb = 66; fn = enc_tq2_0; break;
        case NMQ_IQ2_XXS: bv = 256; bb = 66; fn = enc_iq2_xxs; break;
        default: return NMQ_ERR_FORMAT;
    }
    if (!w || !out) return NMQ_ERR_ARG;
    if (n <= 0 || n % bv) return NMQ_ERR_SHAPE;
    const int64_t nb = n / bv;
    if (fmt == NMQ_IQ2_XXS) grid();  // build the table before the threads share it
    int nt = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    if ((int64_t)nt > nb) nt = (int)nb;
    std::vector<std::thread> pool;
    for (int t = 0; t < nt; ++t) {
        pool.emplace_back([=]() {
            for (int64_t i = nb * t / nt; i < nb * (t + 1) / nt; ++i) fn(w + i * bv, out + i * bb);
        });
    }
    for (auto& th : pool) th.join();
    return nb * bb;
}
