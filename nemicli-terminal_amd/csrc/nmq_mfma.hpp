// Small-batch mat-vec on the matrix cores: 2..8 tokens per launch with v_mfma_i32_16x16x32_i8.
//
// One MFMA multiplies a 16 x 32 int8 input tile with a 32 x 16 int8 weight tile and produces the
// 16 x 16 int32 sums.  The 16 input rows are the two stages of 8 tokens (row 2t: xq of token t, row
// 2t + 1: xq2 of token t; rows of absent tokens hold whatever LDS holds and their sums are never
// stored); the 16 columns are 16 weight rows.  K = 32 is one scale group of every format here (Q6_K:
// two groups of 16, handled as two MFMAs whose input is masked to one half each), so each MFMA's sums
// get exactly one weight factor per weight row.
//
// Operand layouts (lane l of the wave; checked on gfx950 with an in-bounds probe):
//   A[row = l % 16][k = 8 (l / 16) + j] = byte j of the lane's 64-bit operand
//   B[k = 8 (l / 16) + j][col = l % 16]
//   C[row = 4 (l / 16) + r][col = l % 16] = element r of the 4 x int32 result
// So lane l loads 8 bytes of weight row l % 16 per step, and its C registers hold, for that weight
// row, tokens 2 (l / 16) and 2 (l / 16) + 1 with both stages: the lane combines them with its own
// row's weight factors, without exchanges between lanes.
//
// Work split: a wave owns one 16-row tile and one of KS slices of the row's blocks; a workgroup holds
// TPW tiles x KS slices (W = TPW*KS waves) and stages the input of all tokens once, as ready-made A
// fragments ([step][k-block][input row], 512 bytes per 32 values, conflict-free 64-bit reads).  The
// KS partial sums of a tile are added through LDS.  Up to 16 tokens per launch: G = 2 groups of 8
// share every decoded weight fragment (two MFMAs per fragment).
#pragma once

#include <algorithm>

#include "nmq_device.hpp"

namespace nmq {

typedef int i32x4 __attribute__((ext_vector_type(4)));

struct MvmParams {
    const u8* w;
    const int8_t* xq;
    const int8_t* xq2;
    const float* xd;
    const float* xs;
    float* y;
    int n_out, n_in, nc;
    int ks;       // K slices per tile
    int tpw;      // tiles per workgroup
    int64_t row_bytes;
    int nblk;     // 256-value blocks per row
    int x_stride;  // mvd_kernel: values from one token's input to the next (the whole row of a K range)
    int acc_y;     // mvd_kernel: add the sums to y instead of writing them
    int nr, rb;    // mvd_kernel<..., KL>: K ranges of rb blocks, staged one after another
};

// Per-format pieces of the MFMA path.  Steps are 32 values; GS = values per scale group (Q6_K: 16,
// two groups per step).  load(): the lane's bytes of one 256-value block of its row, k-block kb.
// frag(): the 64-bit weight operand of step s.  fac(): fp32 (weight factor, min factor) of group g.
// NBMAX: blocks one lane holds in registers at once; NBRING: the same for slices cycled through buffers.
// MIN_NC: fewest tokens per launch for which this path beats the dot4 kernel (measured on MI355X at
// 4096 and 12288/14336 rows of 4096 values).
template <int F>
struct Mfma;

template <>
struct Mfma<NMQ_Q4_K> {
    static constexpr int BB = 144, STEPS = 8, GS = 32, NBMAX = 4, NBRING = 4, MIN_NC = 3;
    struct Raw {
        u32x2 q[4];  // [i]: qs[32i + 8kb .. +8]
        u32x4 h;     // d, dmin, scales[12]
    };
    __device__ static void load(const u8* blk, int kb, Raw& r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = *gp<u32x2>(blk + 16 + 32 * i + 8 * kb);
        r.h = ld4a(blk);
    }
    // step s: values 32s + l, nibble (s & 1) of qs[32 (s >> 1) + l]
    __device__ static u64 frag(const Raw& r, int s) {
        const u32x2 v = r.q[s >> 1];
        const int sh = 4 * (s & 1);
        return (u64)((v.x >> sh) & 0x0f0f0f0fu) | ((u64)((v.y >> sh) & 0x0f0f0f0fu) << 32);
    }
    // get_scale_min_k4 on the 12 scale bytes, four groups per dword
    __device__ static float2 fac(const Raw& r, int g) {
        const u32 sv = g < 4 ? (r.h.y & 0x3f3f3f3fu) : ((r.h.w & 0x0f0f0f0fu) | ((r.h.y >> 2) & 0x30303030u));
        const u32 mv = g < 4 ? (r.h.z & 0x3f3f3f3fu) : (((r.h.w >> 4) & 0x0f0f0f0fu) | ((r.h.z >> 2) & 0x30303030u));
        const int b = 8 * (g & 3);
        return make_float2(h2f(r.h.x) * (float)((sv >> b) & 0xffu), h2f(r.h.x >> 16) * (float)((mv >> b) & 0xffu));
    }
};

template <>
struct Mfma<NMQ_Q6_K> {
    static constexpr int BB = 210, STEPS = 8, GS = 16, NBMAX = 4, NBRING = 2, MIN_NC = 4;
    struct Raw {
        u32x2 ql[4];  // [2n + (k&1)]: ql[64n + 32(k&1) + 8kb .. +8]
        u32x2 qh[2];  // [n]: qh[32n + 8kb .. +8]
        u32x4 sc;     // 16 int8 scales
        u32 d;
    };
    __device__ static void load(const u8* blk, int kb, Raw& r) {
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            r.ql[2 * n] = ld2(blk + 64 * n + 8 * kb);
            r.ql[2 * n + 1] = ld2(blk + 64 * n + 32 + 8 * kb);
            r.qh[n] = ld2(blk + 128 + 32 * n + 8 * kb);
        }
        r.sc = ld4(blk + 192);
        r.d = ld16(blk + 208);
    }
    // step s = 4n + k covers values 128n + 32k + l (l = 8kb + j): q = nibble (k >> 1) of
    // ql[64n + 32(k&1) + l] | bits 2k of qh[32n + l] << 4, minus 32
    __device__ static u64 frag(const Raw& r, int s) {
        const int n = s >> 2, k = s & 3;
        const u32x2 l = r.ql[2 * n + (k & 1)], h = r.qh[n];
        const int ls = 4 * (k >> 1), hs = 2 * k;
        const u32 lo = sub32x4(((l.x >> ls) & 0x0f0f0f0fu) | (((h.x >> hs) & 0x03030303u) << 4));
        const u32 hi = sub32x4(((l.y >> ls) & 0x0f0f0f0fu) | (((h.y >> hs) & 0x03030303u) << 4));
        return (u64)lo | ((u64)hi << 32);
    }
    // group g = values 16g .. 16g + 15
    __device__ static float2 fac(const Raw& r, int g) {
        const u32 w = (g >> 2) == 0 ? r.sc.x : (g >> 2) == 1 ? r.sc.y : (g >> 2) == 2 ? r.sc.z : r.sc.w;
        return make_float2(h2f(r.d) * (float)(int8_t)(w >> (8 * (g & 3))), 0.f);
    }
};

template <>
struct Mfma<NMQ_Q8_0> {
    // a 256-value block of this path is 8 GGUF blocks, one step each
    static constexpr int BB = 8 * 34, STEPS = 8, GS = 32, NBMAX = 2, NBRING = 2, MIN_NC = 5;
    struct Raw {
        u32x2 q[8];
        u32 d[8];
    };
    __device__ static void load(const u8* blk, int kb, Raw& r) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            r.q[s] = ld2(blk + 34 * s + 2 + 8 * kb);
            r.d[s] = ld16(blk + 34 * s);
        }
    }
    __device__ static u64 frag(const Raw& r, int s) { return (u64)r.q[s].x | ((u64)r.q[s].y << 32); }
    __device__ static float2 fac(const Raw& r, int g) { return make_float2(h2f(r.d[g]), 0.f); }
};

template <>
struct Mfma<NMQ_Q4_0> {
    // a 256-value block of this path is 8 GGUF blocks, one step each; k-block kb of a step is nibble
    // half kb >> 1 of qs[8 (kb & 1) .. + 8].  Sixteen small loads per lane and 256 values (the blocks
    // are 2-byte aligned): measured on MI355X, this path beats the dot4 kernel only from 8 tokens.
    static constexpr int BB = 8 * 18, STEPS = 8, GS = 32, NBMAX = 4, NBRING = 4, MIN_NC = 8;
    struct Raw {
        u32x2 q[8];
        u32 d[8];
        u32 sh;  // 0: low nibbles, 4: high nibbles
    };
    __device__ static void load(const u8* blk, int kb, Raw& r) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            r.q[s] = ld2(blk + 18 * s + 2 + 8 * (kb & 1));
            r.d[s] = ld16(blk + 18 * s);
        }
        r.sh = 4u * (u32)(kb >> 1);
    }
    __device__ static u64 frag(const Raw& r, int s) {
        const u32x2 v = r.q[s];
        return (u64)sub8x4((v.x >> r.sh) & 0x0f0f0f0fu) | ((u64)sub8x4((v.y >> r.sh) & 0x0f0f0f0fu) << 32);
    }
    __device__ static float2 fac(const Raw& r, int g) { return make_float2(h2f(r.d[g]), 0.f); }
};

template <>
struct Mfma<NMQ_TQ2_0> {
    static constexpr int BB = 66, STEPS = 8, GS = 32, NBMAX = 8, NBRING = 8, MIN_NC = 2;
    struct Raw {
        u32x2 q[2];  // [n]: qs[32n + 8kb .. +8]
        u32 d;
    };
    __device__ static void load(const u8* blk, int kb, Raw& r) {
        r.q[0] = ld2(blk + 8 * kb);
        r.q[1] = ld2(blk + 32 + 8 * kb);
        r.d = ld16(blk + 64);
    }
    // step s = 4n + l: values 128n + 32l + m, codes at shift 2l of qs[32n + m]
    __device__ static u64 frag(const Raw& r, int s) {
        const u32x2 v = r.q[s >> 2];
        const int sh = 2 * (s & 3);
        return (u64)sub1x4((v.x >> sh) & 0x03030303u) | ((u64)sub1x4((v.y >> sh) & 0x03030303u) << 32);
    }
    __device__ static float2 fac(const Raw& r, int) { return make_float2(h2f(r.d), 0.f); }
};

template <>
struct Mfma<NMQ_IQ2_XXS> {
    static constexpr int BB = 66, STEPS = 8, GS = 32, NBMAX = 4, NBRING = 4, MIN_NC = 4;
    struct Raw {
        u32x2 a[8];  // {aux0, aux1} of each 32-value sub-block
        u32 d;
    };
    __device__ static void load(const u8* blk, int /*kb*/, Raw& r) {
#pragma unroll
        for (int s = 0; s < 8; ++s) r.a[s] = ld2(blk + 2 + 8 * s);
        r.d = ld16(blk);
    }
    // k-block kb of sub-block s is grid entry kb: 8 unsigned grid bytes with 8 signs (7 + parity)
    __device__ static u64 frag_iq(const Raw& r, int s, int kb, const u64* tab) {
        const u64 g = tab[bfe(r.a[s].x, 8 * kb, 8)];
        const u64 m = tab[256 + bfe(r.a[s].y, 7 * kb, 7)];
        const u32 glo = (u32)g, ghi = (u32)(g >> 32), mlo = (u32)m, mhi = (u32)(m >> 32);
        return (u64)((glo ^ mlo) + (mlo & 0x01010101u)) | ((u64)((ghi ^ mhi) + (mhi & 0x01010101u)) << 32);
    }
    __device__ static float2 fac(const Raw& r, int g) {
        return make_float2(h2f(r.d) * (0.125f + 0.25f * (float)(r.a[g].y >> 28)), 0.f);
    }
};

// LDS layout of the input, G groups of 8 tokens (group g = tokens 8g .. 8g + 7): A fragments of every
// group, then (xd / 254, xs) pairs of every group.
//   frag_g[s][kb][n] (u64) at g * S * 512 bytes: s = 32-value step of the row; input row n = xq (n even)
//   or xq2 (n odd) of token 8g + n / 2, values 32s + 8kb .. + 8
//   xsc_g[s][t] (float2) at G * S * 512 + g * S * 64 bytes: token 8g + t, step s
// Staged in rounds: per round each thread reads 4 16-byte chunks (16 G input rows x n_in / 16 chunks
// in all, 16 G rows x 4 / G chunks per wave access) and one (xd, xs) pair.  Every read is issued
// (threads with nothing to read re-read the start of xq), so a round's reads can be issued before the
// weight reads and waited for alone.  Rows of absent tokens (t >= nc) are left unwritten.
struct XStage {
    u32x4 v[4];
    float2 f;
};

template <int G>
__device__ __forceinline__ void stage_load(XStage& st, int r, const MvmParams& p) {
    const int T = 64 * p.ks * p.tpw, S = p.n_in / 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = (4 * r + j) * T + (int)threadIdx.x;
        const int na = i & (16 * G - 1), c = i / (16 * G), t = 8 * (na >> 4) + ((na & 15) >> 1);
        const bool ok = i < G * p.n_in && t < p.nc;
        const int8_t* src = ok ? ((na & 1) ? p.xq2 : p.xq) + (int64_t)t * p.n_in + 16 * c : p.xq;
        st.v[j] = *gp<u32x4>(src);
    }
    const int i = r * T + (int)threadIdx.x;
    const int t = i & (8 * G - 1), s = i / (8 * G);
    const int64_t o = (i < 8 * G * S && t < p.nc) ? (int64_t)t * S + s : 0;
    st.f = make_float2(gp<float>(p.xd)[o], gp<float>(p.xs)[o]);
}

template <int G>
__device__ __forceinline__ void stage_store(const XStage& st, int r, u8* lds, const MvmParams& p) {
    const int T = 64 * p.ks * p.tpw, S = p.n_in / 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = (4 * r + j) * T + (int)threadIdx.x;
        const int na = i & (16 * G - 1), c = i / (16 * G), g = na >> 4, n = na & 15, t = 8 * g + (n >> 1);
        if (i < G * p.n_in && t < p.nc) {
            // values 16c .. 16c + 15: step c / 2, k-blocks 2 (c & 1) and 2 (c & 1) + 1
            u64* d = (u64*)(lds + (size_t)g * S * 512) + ((c >> 1) * 4 + 2 * (c & 1)) * 16 + n;
            d[0] = (u64)st.v[j].x | ((u64)st.v[j].y << 32);
            d[16] = (u64)st.v[j].z | ((u64)st.v[j].w << 32);
        }
    }
    const int i = r * T + (int)threadIdx.x;
    const int t = i & (8 * G - 1), s = i / (8 * G);
    if (i < 8 * G * S && t < p.nc) {
        float2* xsc = (float2*)(lds + (size_t)G * S * 512 + (size_t)(t >> 3) * S * 64);
        xsc[s * 8 + (t & 7)] = make_float2(st.f.x * FEIN, st.f.y);
    }
}

// One 256-value block of the lane's weight row into its sums of tokens 8g + 2kb and 8g + 2kb + 1 of
// every group g (the weight fragment of a step is decoded once and meets G input fragments):
//   y += w_g * (xd_g / 254) * (254 S1 + S2) - m_g * xs_g   per 32-value group g (Q6_K: per 16, no m term)
// (254 S1 + S2 is exact in int32: |S1|, |S2| <= 32 * 127 * 63.)
// The LDS operands of each step are read one step ahead.
template <int F, int G>
__device__ __forceinline__ void mvm_block(const typename Mfma<F>::Raw& cur, int b, const u64* tab, const u8* lds, int S,
                                          int lane, float (&acc)[G][2]) {
    using M = Mfma<F>;
    const int kb = lane >> 4, n = lane & 15;
    u64 xv[2][G];
    float4 xf[2][G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const u64* frag = (const u64*)(lds + (size_t)g * S * 512);
        const float2* xsc = (const float2*)(lds + (size_t)G * S * 512 + (size_t)g * S * 64);
        xv[0][g] = frag[(b * M::STEPS * 4 + kb) * 16 + n];
        xf[0][g] = *(const float4*)(xsc + b * M::STEPS * 8 + 2 * kb);
    }
#pragma unroll
    for (int s = 0; s < M::STEPS; ++s) {
        if (s + 1 < M::STEPS) {
            const int gn = b * M::STEPS + s + 1;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const u64* frag = (const u64*)(lds + (size_t)g * S * 512);
                const float2* xsc = (const float2*)(lds + (size_t)G * S * 512 + (size_t)g * S * 64);
                xv[(s + 1) & 1][g] = frag[(gn * 4 + kb) * 16 + n];
                xf[(s + 1) & 1][g] = *(const float4*)(xsc + gn * 8 + 2 * kb);  // tokens 2kb, 2kb + 1
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // the next step's reads stay ahead of this step's work
        u64 wv;
        if constexpr (F == NMQ_IQ2_XXS) wv = M::frag_iq(cur, s, kb, tab);
        else wv = M::frag(cur, s);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const u64 x = xv[s & 1][g];
            const float4 f = xf[s & 1][g];
            if constexpr (M::GS == 16) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const u64 xm = (kb >> 1) == half ? x : 0ull;
                    i32x4 c = {0, 0, 0, 0};
                    c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xm, (long)wv, c, 0, 0, 0);
                    const float w = M::fac(cur, 2 * s + half).x;
                    acc[g][0] = fmaf(w * f.x, (float)__mul24(c[0], 254) + (float)c[1], acc[g][0]);
                    acc[g][1] = fmaf(w * f.z, (float)__mul24(c[2], 254) + (float)c[3], acc[g][1]);
                }
            } else {
                i32x4 c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)wv, c, 0, 0, 0);
                const float2 w = M::fac(cur, s);
                acc[g][0] = fmaf(w.x * f.x, (float)(__mul24(c[0], 254) + c[1]), fmaf(-w.y, f.y, acc[g][0]));
                acc[g][1] = fmaf(w.x * f.z, (float)(__mul24(c[2], 254) + c[3]), fmaf(-w.y, f.w, acc[g][1]));
            }
        }
    }
}

// NB blocks of the wave's slice are held in registers.  RING = false: the slice has exactly NB blocks,
// all requested before the input is staged.  RING = true: any number of blocks, each buffer refilled
// NB blocks ahead once used (requests past the slice re-read its last block, so every wave issues the
// same loads and the waits count exactly).  G: groups of 8 tokens per launch (1 or 2).
template <int F, int NB, bool RING, int G>
__global__ __launch_bounds__(1024) void mvm_kernel(MvmParams p) {
    using M = Mfma<F>;
    // every argument into the first batch of scalar loads (see args_early)
    asm volatile("" ::"s"(p.w), "s"(p.xq), "s"(p.xq2), "s"(p.xd), "s"(p.xs), "s"(p.y), "s"(p.n_out), "s"(p.n_in),
                 "s"(p.nc), "s"(p.ks), "s"(p.tpw), "s"(p.row_bytes), "s"(p.nblk));
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int S = p.n_in / 32;
    float* red = (float*)lds;  // W x 64 x 2G sums, after the blocks

    const int tile_in_wg = wave / p.ks, slice = wave % p.ks;
    const int row0 = (blockIdx.x * p.tpw + tile_in_wg) * 16;
    const int n = lane & 15, kb = lane >> 4;
    const int bpr = p.nblk / p.ks;  // blocks of this wave's slice
    const int b0 = slice * bpr, last = b0 + bpr - 1;
    const u8* rowp = p.w + (int64_t)min(row0 + n, p.n_out - 1) * p.row_bytes;

    // One staging round: the input reads first, then (once every wave has issued them) the weight
    // reads, and the stores wait only for the older input reads.  Several rounds: the input is staged
    // completely before the weight reads (no input read pending where the two paths meet, which would
    // make the compiler wait for all outstanding reads).  The CU's vector cache returns data in request
    // order, so input requested after another wave's weights would wait for them; the barrier between
    // input and weight reads waits for issue only.
    const int nt = 64 * p.ks * p.tpw;  // threads of the workgroup, from the arguments (see args_early)
    const int rounds = (G * p.n_in + 4 * nt - 1) / (4 * nt);
    typename M::Raw buf[NB];
    if (rounds == 1) {
        XStage st;
        stage_load<G>(st, 0, p);
        const u64 gv = tab_load<F>();
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NB; ++u) M::load(rowp + (int64_t)min(b0 + u, last) * M::BB, kb, buf[u]);
        __builtin_amdgcn_sched_barrier(0);
        tab_store<F>(tab, gv, nt);
        stage_store<G>(st, 0, lds, p);
    } else {
        for (int r = 0; r < rounds; ++r) {
            XStage st;
            stage_load<G>(st, r, p);
            stage_store<G>(st, r, lds, p);
        }
        tab_store<F>(tab, tab_load<F>(), nt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NB; ++u) M::load(rowp + (int64_t)min(b0 + u, last) * M::BB, kb, buf[u]);
    }
    lds_barrier();

    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
    if constexpr (RING) {
        for (int j0 = 0; j0 < bpr; j0 += NB) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                if (j0 + u < bpr) mvm_block<F, G>(buf[u], b0 + j0 + u, tab, lds, S, lane, acc);
                M::load(rowp + (int64_t)min(b0 + j0 + u + NB, last) * M::BB, kb, buf[u]);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < NB; ++u) mvm_block<F, G>(buf[u], b0 + u, tab, lds, S, lane, acc);
    }

    // add the KS slices of each tile; lane (n, kb) holds weight row row0 + n, tokens 8g + 2kb, 8g + 2kb + 1
    // (the sums take the place of the staged input, once every wave is done with it)
    lds_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        red[((wave * 64 + lane) * G + g) * 2] = acc[g][0];
        red[((wave * 64 + lane) * G + g) * 2 + 1] = acc[g][1];
    }
    lds_barrier();
    if (slice == 0) {
        const int r = row0 + n;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s0 = 0.f, s1 = 0.f;
            for (int q = 0; q < p.ks; ++q) {
                const int ri = (((tile_in_wg * p.ks + q) * 64 + lane) * G + g) * 2;
                s0 += red[ri];
                s1 += red[ri + 1];
            }
            const int t = 8 * g + 2 * kb;
            if (r < p.n_out) {
                if (t < p.nc) gpw<float>(p.y)[(int64_t)t * p.n_out + r] = s0;
                if (t + 1 < p.nc) gpw<float>(p.y)[(int64_t)(t + 1) * p.n_out + r] = s1;
            }
        }
    }
}

// ---- Q4_K (5..8 tokens), the other formats (2..8 tokens): dense reads straight into LDS -------------
// mvm_kernel reads, per instruction, 8 bytes of each of 16 rows per lane group: 16 short pieces per read.
// A CU issuing those for 16 waves stalls for longer than HBM takes to deliver the bytes (per-wave time
// stamps: 10 us until the last wave has issued its reads, against 6 us with dense reads of the same
// bytes).  mvd_kernel keeps mvm_kernel's work split and arithmetic, but every read is dense (16 bytes per
// lane, consecutive lanes on consecutive bytes), and weights and input move with global_load_lds_dwordx4
// (lane l's 16 bytes land at the LDS address of the instruction + 16 l, no registers in between):
//   - the input rows (xq, xq2 of each present token: 2 nc rows) row-major, 16 + n_in bytes apart, so that
//     the A operands of a step (8 bytes at row n, 32 step + 8 k-block) fall on distinct banks;
//   - the weights, per wave in chunks of CHB 256-value blocks x 16 rows (Q4_K, Q4_0: 2 blocks of 144
//     bytes; Q8_0: 1 block of 272 bytes, 8 GGUF blocks of 34; Q6_K: 1 block of 210; TQ2_0, IQ2_XXS: 2
//     blocks of 66): a chunk row is the 16-byte window from the 16-byte boundary at or below the chunk's
//     first byte (m bytes before it: 0 where CHB blocks fill whole pieces), PR pieces of 16 bytes; slot
//     u = 64 j + lane of instruction j holds piece min(u % SLOTS, PR - 1) of row u / SLOTS (the slots
//     past PR padding copies of the last piece; SLOTS = 19, 15 or 11 puts the 16 rows' operands on
//     distinct banks).  Fields (codes, scales) that sit off a 4-byte boundary in the window are read as
//     dwords and shifted into place with v_alignbyte.
// (xd / 254, xs) per step and token are read densely into registers and stored as mvm_kernel stores them.
// A wave holds one chunk buffer: chunk c + 1 is requested as soon as chunk c's operands are in registers,
// and streams in while chunk c is computed.
typedef __attribute__((address_space(3))) void lds_void;

// global_load_lds_dwordx4 issued by hand, its address a wave-uniform base (SGPR pair) plus an unsigned
// 32-bit per-lane offset: the compiler neither counts it nor sees its LDS write, so it adds no waits of
// its own (with the builtin it waits for every outstanding read before each later LDS access, since it
// cannot tell the buffers apart).  The kernel waits with vm_wait<N> (memory clobber: no LDS access moves
// across the wait).  M0 is set inside the statement; nothing else in the kernel uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is reserved: clobbering it is the point here
__device__ __forceinline__ void dma16s(const void* base, u32 off, void* lds_dst) {
    const u32 m = (u32)(uintptr_t)(lds_void*)lds_dst;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Per-lane offsets of the chunk reads (the same for every chunk), from the window's first byte in row
// rb0 = min(row0, n_out - 1): slot u = 64 j + lane holds piece min(u % SLOTS, PR - 1) of row
// min(row0 + u / SLOTS, n_out - 1) >= rb0, so every offset is non-negative, also for tiles past the matrix.
template <int NI>
struct ChunkOffsets {
    u32 o[NI];
};
template <int PR, int SLOTS, int NI>
__device__ __forceinline__ ChunkOffsets<NI> mvd_offsets(const MvmParams& p, int row0, int lane) {
    ChunkOffsets<NI> c;
    const int rb0 = min(row0, p.n_out - 1);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int u = 64 * j + lane;
        const int r = min(row0 + u / SLOTS, p.n_out - 1) - rb0, k = min(u % SLOTS, PR - 1);
        c.o[j] = (u32)(r * (int)p.row_bytes + 16 * k);
    }
    return c;
}

// chunk of CHB blocks from blk on, rows row0 .. row0 + 15, into buf (NI instructions; the last one with
// 16 SLOTS - 64 (NI - 1) = 48 lanes): the windows start at the 16-byte boundary at or below the chunk
template <int F, int NI>
__device__ __forceinline__ void mvd_chunk(u8* buf, const MvmParams& p, const ChunkOffsets<NI>& co, int row0, int blk,
                                          int lane) {
    const u8* base = p.w + (int64_t)min(row0, p.n_out - 1) * p.row_bytes + (((int64_t)blk * Mfma<F>::BB) & ~15ll);
#pragma unroll
    for (int j = 0; j < NI; ++j)
        if (j < NI - 1 || lane < 48) dma16s(base, co.o[j], buf + 1024 * j);
}

__device__ __forceinline__ u32 lds32(const u8* p) { return *(const u32*)p; }
// 8 bytes at p + sh (p 4-byte aligned, sh in 0..3) from three dwords
__device__ __forceinline__ u32x2 lds8_shifted(const u8* p, u32 sh) {
    const u32 w0 = lds32(p), w1 = lds32(p + 4), w2 = lds32(p + 8);
    return u32x2{__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh)};
}

// Per-format pieces of the dense-read kernel.  CHB: 256-value blocks per chunk, PR: 16-byte pieces of a
// chunk row, SLOTS: its LDS stride in pieces.  frag(): the lane's operands of a whole chunk from the
// buffer (row: the lane's row n, m: the chunk's offset in the window, kb: the lane's k-block).
// block(): block i of the chunk (row block b) into the lane's sums of tokens 2 kb and 2 kb + 1, A operands
// read from the row-major input (ab: the lane's input row n at k-block kb of block b; steps 32 bytes
// apart), (xd / 254, xs) from xb (the block's first step, tokens 2 kb, 2 kb + 1); tab: the IQ2_XXS grid
// and sign tables.
template <int F>
struct Dma;

template <>
struct Dma<NMQ_Q4_K> {
    static constexpr int CHB = 2, PR = 18, SLOTS = 19;
    using M = Mfma<NMQ_Q4_K>;
    struct Raw {
        M::Raw r[2];
    };
    // Mfma<Q4_K>::load from the chunk buffer
    __device__ static void frag(Raw& o, const u8* row, int, int kb) {
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            const u8* b = row + M::BB * bb;
            o.r[bb].h = *(const u32x4*)b;
#pragma unroll
            for (int i = 0; i < 4; ++i) o.r[bb].q[i] = *(const u32x2*)(b + 16 + 32 * i + 8 * kb);
        }
    }
    // The block's scales d, dmin apply once per block:
    //   y += d * sum_g (sc_g (254 S1 + S2)) (xd_g / 254)  -  dmin * sum_g m_g xs_g
    // with sc_g (254 S1 + S2) an exact int32 (|.| <= 63 * 254 * 32 * 127 * 15 * 1.004 < 2^31) rounded once
    // to fp32, where mvm_block forms d sc_g and dmin m_g per group.
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int, const u64*,
                                float (&acc)[2]) {
        const M::Raw& cur = o.r[i];
        // 6-bit scales and mins of groups 0..3 (bytes of lo) and 4..7 (bytes of hi): get_scale_min_k4
        const u32 sc_lo = cur.h.y & 0x3f3f3f3fu, m_lo = cur.h.z & 0x3f3f3f3fu;
        const u32 sc_hi = (cur.h.w & 0x0f0f0f0fu) | ((cur.h.y >> 2) & 0x30303030u);
        const u32 m_hi = ((cur.h.w >> 4) & 0x0f0f0f0fu) | ((cur.h.z >> 2) & 0x30303030u);
        float sd0 = 0.f, sd1 = 0.f, sm0 = 0.f, sm1 = 0.f;
        u64 xv[2];
        float4 xf[2];
        xv[0] = *(const u64*)ab;
        xf[0] = *(const float4*)xb;
#pragma unroll
        for (int s = 0; s < M::STEPS; ++s) {
            if (s + 1 < M::STEPS) {
                xv[(s + 1) & 1] = *(const u64*)(ab + 32 * (s + 1));
                xf[(s + 1) & 1] = *(const float4*)(xb + 8 * (s + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            const u64 wv = M::frag(cur, s);
            const u64 x = xv[s & 1];
            const float4 f = xf[s & 1];
            i32x4 c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)wv, c, 0, 0, 0);
            const u32 scw = s < 4 ? sc_lo : sc_hi, mw = s < 4 ? m_lo : m_hi;
            const int sc = (int)((scw >> (8 * (s & 3))) & 0xffu), sc254 = 254 * sc;
            const float mf = (float)((mw >> (8 * (s & 3))) & 0xffu);
            // sc (254 S1 + S2) as 24-bit products (|S1|, |S2| <= 32 * 127 * 15, sc254 <= 16002)
            sd0 = fmaf((float)(__mul24(c[0], sc254) + __mul24(c[1], sc)), f.x, sd0);
            sd1 = fmaf((float)(__mul24(c[2], sc254) + __mul24(c[3], sc)), f.z, sd1);
            sm0 = fmaf(mf, f.y, sm0);
            sm1 = fmaf(mf, f.w, sm1);
        }
        const float d = h2f(cur.h.x), dm = h2f(cur.h.x >> 16);
        acc[0] = fmaf(d, sd0, fmaf(-dm, sm0, acc[0]));
        acc[1] = fmaf(d, sd1, fmaf(-dm, sm1, acc[1]));
    }
};

// Q4_0 and Q8_0: GGUF blocks of 32 values (one step each, d an fp16 at the block's start, then the codes)
// of BB / 8 bytes, an odd number of 16-bit words: block pairs are 4-byte aligned in the chunk buffer, the
// codes of the pair's first block start 2 bytes past a dword.  The lane's 8 code bytes of a block start
// at lo = 8 (kb & 1) (Q4_0: k-block kb of a step is nibble half kb >> 1 of codes lo .. lo + 7, minus 8)
// or lo = 8 kb (Q8_0: codes lo .. lo + 7).  Per pair the lane reads dwords only: a0..a2 over the first
// block's bytes 2 + lo .. 9 + lo (shifted into place with v_alignbyte), b0, b1 with the second block's
// (4-byte aligned), and the two dwords that hold the d's (first block: low half of the pair's dword 0;
// second block: high half of the dword at byte GB - 2).
// Per step:  y += d * (xd / 254) * (254 S1 + S2)  (254 S1 + S2 exact in int32, rounded once to fp32).
template <int F, int CHB_ = F == NMQ_Q4_0 ? 2 : 1>
struct DmaSmall {
    static constexpr int GB = F == NMQ_Q4_0 ? 18 : 34;  // bytes per GGUF block
    static constexpr int CHB = CHB_, PR = CHB * 8 * GB / 16, SLOTS = PR <= 9 ? 11 : 19;
    static constexpr int NP = CHB * 4;                  // block pairs per chunk
    struct Raw {
        u32x2 q[2 * NP];
        u32 d[NP];  // fp16 d of the pair's first block (low half) and second block (high half)
    };
    __device__ static void frag(Raw& o, const u8* row, int, int kb) {
        const int lo = F == NMQ_Q4_0 ? 8 * (kb & 1) : 8 * kb;  // the lane's code bytes of a block
#pragma unroll
        for (int pr = 0; pr < NP; ++pr) {
            const u8* bp = row + 2 * GB * pr;
            const u32* a = (const u32*)(bp + lo);
            const u32 a0 = a[0], a1 = a[1], a2 = a[2];
            const u32 b0 = a[(GB + 2) / 4], b1 = a[(GB + 2) / 4 + 1];
            const u32 d0 = ((const u32*)bp)[0], d1 = ((const u32*)bp)[GB / 4];
            o.q[2 * pr] = u32x2{__builtin_amdgcn_alignbyte(a1, a0, 2), __builtin_amdgcn_alignbyte(a2, a1, 2)};
            o.q[2 * pr + 1] = u32x2{b0, b1};
            o.d[pr] = (d0 & 0xffffu) | (d1 & 0xffff0000u);
        }
    }
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int kb, const u64*,
                                float (&acc)[2]) {
        const u32 sh = F == NMQ_Q4_0 ? 4u * (u32)(kb >> 1) : 0u;
        u64 xv[2];
        float4 xf[2];
        xv[0] = *(const u64*)ab;
        xf[0] = *(const float4*)xb;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (s + 1 < 8) {
                xv[(s + 1) & 1] = *(const u64*)(ab + 32 * (s + 1));
                xf[(s + 1) & 1] = *(const float4*)(xb + 8 * (s + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            const u32x2 v = o.q[8 * i + s];
            u64 wv;
            if constexpr (F == NMQ_Q4_0)
                wv = (u64)sub8x4((v.x >> sh) & 0x0f0f0f0fu) | ((u64)sub8x4((v.y >> sh) & 0x0f0f0f0fu) << 32);
            else
                wv = (u64)v.x | ((u64)v.y << 32);
            const u64 x = xv[s & 1];
            const float4 f = xf[s & 1];
            i32x4 c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)wv, c, 0, 0, 0);
            const u32 dw = o.d[4 * i + (s >> 1)];
            const float d = h2f((s & 1) ? dw >> 16 : dw);
            // |S1|, |S2| <= 32 * 127 * 128: 254 S1 as a 24-bit product
            acc[0] = fmaf(d * f.x, (float)(__mul24(c[0], 254) + c[1]), acc[0]);
            acc[1] = fmaf(d * f.z, (float)(__mul24(c[2], 254) + c[3]), acc[1]);
        }
    }
};
template <>
struct Dma<NMQ_Q4_0> : DmaSmall<NMQ_Q4_0> {};
template <>
struct Dma<NMQ_Q8_0> : DmaSmall<NMQ_Q8_0> {};

// Q6_K: chunks of one 210-byte block; the window offset m = 2 b mod 16 is even, so the block's fields
// sit 0 or 2 bytes off a dword (sh = m & 3): every 8 bytes are read as three dwords and shifted.  Per
// step two MFMAs, the input masked to one 16-value scale group each (as mvm_kernel).
template <>
struct Dma<NMQ_Q6_K> {
    static constexpr int CHB = 1, PR = 14, SLOTS = 15;
    using M = Mfma<NMQ_Q6_K>;
    using Raw = M::Raw;
    __device__ static void frag(Raw& r, const u8* row, int m, int kb) {
        const u8* b = row + (m & 12);
        const u32 sh = (u32)(m & 3);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            r.ql[2 * n] = lds8_shifted(b + 64 * n + 8 * kb, sh);
            r.ql[2 * n + 1] = lds8_shifted(b + 64 * n + 32 + 8 * kb, sh);
            r.qh[n] = lds8_shifted(b + 128 + 32 * n + 8 * kb, sh);
        }
        const u32x2 s0 = lds8_shifted(b + 192, sh), s1 = lds8_shifted(b + 200, sh);
        r.sc = u32x4{s0.x, s0.y, s1.x, s1.y};
        r.d = lds32(b + 208) >> (8 * sh);
    }
    __device__ static void block(const Raw& cur, int, const u8* ab, const float2* xb, int kb, const u64*,
                                float (&acc)[2]) {
        u64 xv[2];
        float4 xf[2];
        xv[0] = *(const u64*)ab;
        xf[0] = *(const float4*)xb;
#pragma unroll
        for (int s = 0; s < M::STEPS; ++s) {
            if (s + 1 < M::STEPS) {
                xv[(s + 1) & 1] = *(const u64*)(ab + 32 * (s + 1));
                xf[(s + 1) & 1] = *(const float4*)(xb + 8 * (s + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            const u64 wv = M::frag(cur, s);
            const u64 x = xv[s & 1];
            const float4 f = xf[s & 1];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const u64 xm = (kb >> 1) == half ? x : 0ull;
                i32x4 c = {0, 0, 0, 0};
                c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xm, (long)wv, c, 0, 0, 0);
                const float w = M::fac(cur, 2 * s + half).x;
                acc[0] = fmaf(w * f.x, (float)__mul24(c[0], 254) + (float)c[1], acc[0]);
                acc[1] = fmaf(w * f.z, (float)__mul24(c[2], 254) + (float)c[3], acc[1]);
            }
        }
    }
};

// TQ2_0 and IQ2_XXS: chunks of two 66-byte blocks; the window offset m = 132 (b / 2) mod 16 is a
// multiple of 4, so the chunk's first block is dword-aligned and its second sits 2 bytes off (read as
// dwords and shifted by 2).  PR = 9 pieces (m + 132 <= 144 bytes).
template <>
struct Dma<NMQ_TQ2_0> {
    static constexpr int CHB = 2, PR = 9, SLOTS = 11;
    using M = Mfma<NMQ_TQ2_0>;
    struct Raw {
        M::Raw r[2];
    };
    __device__ static void frag(Raw& o, const u8* row, int m, int kb) {
        const u8* b = row + m;  // block 0: codes at 0, d at 64; block 1: codes at 66, d at 130
        o.r[0].q[0] = u32x2{lds32(b + 8 * kb), lds32(b + 8 * kb + 4)};
        o.r[0].q[1] = u32x2{lds32(b + 32 + 8 * kb), lds32(b + 36 + 8 * kb)};
        o.r[0].d = lds32(b + 64);
        o.r[1].q[0] = lds8_shifted(b + 64 + 8 * kb, 2);
        o.r[1].q[1] = lds8_shifted(b + 96 + 8 * kb, 2);
        o.r[1].d = lds32(b + 128) >> 16;
    }
    // one fp16 d per block: the steps' exact sums (|254 S1 + S2| <= 254 * 32 * 127 + 32 * 127 < 2^24)
    // scaled by xd / 254 and added, then d once
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int, const u64*,
                                float (&acc)[2]) {
        const M::Raw& cur = o.r[i];
        float sd0 = 0.f, sd1 = 0.f;
        u64 xv[2];
        float4 xf[2];
        xv[0] = *(const u64*)ab;
        xf[0] = *(const float4*)xb;
#pragma unroll
        for (int s = 0; s < M::STEPS; ++s) {
            if (s + 1 < M::STEPS) {
                xv[(s + 1) & 1] = *(const u64*)(ab + 32 * (s + 1));
                xf[(s + 1) & 1] = *(const float4*)(xb + 8 * (s + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            const u64 wv = M::frag(cur, s);
            const u64 x = xv[s & 1];
            const float4 f = xf[s & 1];
            i32x4 c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)wv, c, 0, 0, 0);
            sd0 = fmaf((float)(__mul24(c[0], 254) + c[1]), f.x, sd0);
            sd1 = fmaf((float)(__mul24(c[2], 254) + c[3]), f.z, sd1);
        }
        const float d = h2f(cur.d);
        acc[0] = fmaf(d, sd0, acc[0]);
        acc[1] = fmaf(d, sd1, acc[1]);
    }
};

template <>
struct Dma<NMQ_IQ2_XXS> {
    static constexpr int CHB = 2, PR = 9, SLOTS = 11;
    using M = Mfma<NMQ_IQ2_XXS>;
    struct Raw {
        M::Raw r[2];
    };
    // block 0: d at 0, sub-block s's {aux0, aux1} at 2 + 8 s (2 bytes off a dword); block 1: d at 66
    // (high half of the dword at 64), its pairs at 68 + 8 s (aligned).  Every lane reads all of them.
    __device__ static void frag(Raw& o, const u8* row, int m, int) {
        const u8* b = row + m;
        u32 w[17];
#pragma unroll
        for (int j = 0; j < 17; ++j) w[j] = lds32(b + 4 * j);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            o.r[0].a[s] = u32x2{__builtin_amdgcn_alignbyte(w[2 * s + 1], w[2 * s], 2),
                                __builtin_amdgcn_alignbyte(w[2 * s + 2], w[2 * s + 1], 2)};
            o.r[1].a[s] = u32x2{lds32(b + 68 + 8 * s), lds32(b + 72 + 8 * s)};
        }
        o.r[0].d = w[0];
        o.r[1].d = w[16] >> 16;
    }
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int kb, const u64* tab,
                                float (&acc)[2]) {
        const M::Raw& cur = o.r[i];
        u64 xv[2];
        float4 xf[2];
        xv[0] = *(const u64*)ab;
        xf[0] = *(const float4*)xb;
#pragma unroll
        for (int s = 0; s < M::STEPS; ++s) {
            if (s + 1 < M::STEPS) {
                xv[(s + 1) & 1] = *(const u64*)(ab + 32 * (s + 1));
                xf[(s + 1) & 1] = *(const float4*)(xb + 8 * (s + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            const u64 wv = M::frag_iq(cur, s, kb, tab);
            const u64 x = xv[s & 1];
            const float4 f = xf[s & 1];
            i32x4 c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)wv, c, 0, 0, 0);
            const float w = M::fac(cur, s).x;
            acc[0] = fmaf(w * f.x, (float)(__mul24(c[0], 254) + c[1]), acc[0]);
            acc[1] = fmaf(w * f.z, (float)(__mul24(c[2], 254) + c[3]), acc[1]);
        }
    }
};

// The long-row form (K ranges of 8 blocks) of TQ2_0 and IQ2_XXS: chunks of one 66-byte block; the window offset m = 2 b mod 16 is even, so the
// block's fields sit 0 or 2 bytes off a dword (sh = m & 3) and are read as dwords and shifted.  PR = 5
// pieces (m + 66 <= 80 bytes; the last block of a row has m = 14 and ends on the row's end).
template <int F>
struct Dma1;

// The long-row form of Q4_K and Q4_0: chunks of one 144-byte block (9 pieces), so that ranges of 14 or
// 16 blocks keep 14 or 16 waves per workgroup.
template <>
struct Dma1<NMQ_Q4_K> {
    static constexpr int CHB = 1, PR = 9, SLOTS = 11;
    using M = Mfma<NMQ_Q4_K>;
    struct Raw {
        M::Raw r[1];
    };
    __device__ static void frag(Raw& o, const u8* row, int, int kb) {
        o.r[0].h = *(const u32x4*)row;
#pragma unroll
        for (int i = 0; i < 4; ++i) o.r[0].q[i] = *(const u32x2*)(row + 16 + 32 * i + 8 * kb);
    }
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int kb, const u64* tab,
                                float (&acc)[2]) {
        Dma<NMQ_Q4_K>::Raw r2;
        r2.r[0] = o.r[i];
        Dma<NMQ_Q4_K>::block(r2, 0, ab, xb, kb, tab, acc);
    }
};
template <>
struct Dma1<NMQ_Q4_0> : DmaSmall<NMQ_Q4_0, 1> {};

template <>
struct Dma1<NMQ_TQ2_0> {
    static constexpr int CHB = 1, PR = 5, SLOTS = 7;
    using M = Mfma<NMQ_TQ2_0>;
    struct Raw {
        M::Raw r[1];
    };
    // codes at 0, d at 64
    __device__ static void frag(Raw& o, const u8* row, int m, int kb) {
        const u8* b = row + (m & 12);
        const u32 sh = (u32)(m & 3);
        o.r[0].q[0] = lds8_shifted(b + 8 * kb, sh);
        o.r[0].q[1] = lds8_shifted(b + 32 + 8 * kb, sh);
        o.r[0].d = lds32(b + 64) >> (8 * sh);
    }
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int kb, const u64* tab,
                                float (&acc)[2]) {
        Dma<NMQ_TQ2_0>::Raw r2;
        r2.r[0] = o.r[i];
        Dma<NMQ_TQ2_0>::block(r2, 0, ab, xb, kb, tab, acc);
    }
};

template <>
struct Dma1<NMQ_IQ2_XXS> {
    static constexpr int CHB = 1, PR = 5, SLOTS = 7;
    using M = Mfma<NMQ_IQ2_XXS>;
    struct Raw {
        M::Raw r[1];
    };
    // d at 0, sub-block s's {aux0, aux1} at 2 + 8 s: from the dword at or below the block's start (shift
    // sh = 0 or 2) the pairs begin 2 + sh bytes in.  Every lane reads all of them.
    __device__ static void frag(Raw& o, const u8* row, int m, int) {
        const u8* b = row + (m & 12);
        const u32 sh = (u32)(m & 3);
        u32 w[18];
#pragma unroll
        for (int j = 0; j < 18; ++j) w[j] = lds32(b + 4 * j);
        const int k = sh >> 1;          // first dword of the pairs
        const u32 shp = 2u - sh;        // their byte shift within it
#pragma unroll
        for (int s = 0; s < 8; ++s)
            o.r[0].a[s] = u32x2{__builtin_amdgcn_alignbyte(w[2 * s + k + 1], w[2 * s + k], shp),
                                __builtin_amdgcn_alignbyte(w[2 * s + k + 2], w[2 * s + k + 1], shp)};
        o.r[0].d = w[0] >> (8 * sh);
    }
    __device__ static void block(const Raw& o, int i, const u8* ab, const float2* xb, int kb, const u64* tab,
                                float (&acc)[2]) {
        Dma<NMQ_IQ2_XXS>::Raw r2;
        r2.r[0] = o.r[i];
        Dma<NMQ_IQ2_XXS>::block(r2, 0, ab, xb, kb, tab, acc);
    }
};

// The chunk layout a kernel form uses: the long-row form of the 66-byte formats takes one block per chunk
// (8-block ranges give twice the waves per workgroup; 4096x14336 at 8 tokens TQ2_0 15.3 -> 12.2 us,
// IQ2_XXS 22.2 -> 17.3), the rows of up to 4096 values keep two (14336x4096 at 8 tokens: one block
// 10.5 / 14.5 us against two 8.6 / 12.6).
template <int F, bool KL>
struct DmaSel {
    using T = Dma<F>;
};
template <>
struct DmaSel<NMQ_TQ2_0, true> {
    using T = Dma1<NMQ_TQ2_0>;
};
template <>
struct DmaSel<NMQ_Q4_K, true> {
    using T = Dma1<NMQ_Q4_K>;
};
template <>
struct DmaSel<NMQ_Q4_0, true> {
    using T = Dma1<NMQ_Q4_0>;
};
template <>
struct DmaSel<NMQ_IQ2_XXS, true> {
    using T = Dma1<NMQ_IQ2_XXS>;
};

// LDS: input rows 2 nc x (n_in + 16), then (xd / 254, xs) [step][token] (64 S bytes), then W chunk buffers.
template <int F, bool KL = false>
__host__ __device__ constexpr size_t mvd_lds(int n_in, int W, int nc) {
    return (size_t)2 * nc * (n_in + 16) + (size_t)2 * n_in + (size_t)W * 256 * DmaSel<F, KL>::T::SLOTS;
}

// KL: rows beyond the LDS's input capacity, as p.nr K ranges of p.rb blocks in one launch (the last one
// the rest of the row, possibly shorter; a wave's slice of every range is 1 or 2 chunks, NCH the most):
// each range's input is staged after every wave is done with the previous one's, the wave's slice of
// each range runs through its chunk buffer, and the sums of all ranges add up in the wave's registers.
template <int F, int NCH, bool KL = false>
__global__ __launch_bounds__(1024) void mvd_kernel(MvmParams p) {
    using D = typename DmaSel<F, KL>::T;
    constexpr int ROW = 16 * D::SLOTS;              // LDS bytes per row of a chunk buffer
    constexpr int NI = (16 * D::SLOTS + 63) / 64;   // chunk read instructions
    static_assert(16 * D::SLOTS - 64 * (NI - 1) == 48, "the last chunk read has 48 lanes");
    asm volatile("" ::"s"(p.w), "s"(p.xq), "s"(p.xq2), "s"(p.xd), "s"(p.xs), "s"(p.y), "s"(p.n_out), "s"(p.n_in),
                 "s"(p.nc), "s"(p.ks), "s"(p.tpw), "s"(p.row_bytes), "s"(p.nblk));
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = p.ks * p.tpw, nt = 64 * W;
    const int KV = KL ? p.rb * 256 : p.n_in;  // values per K range (the whole row without ranges)
    const int S = KV / 32, RS = KV + 16;
    const int tile_in_wg = wave / p.ks, slice = wave % p.ks;
    const int row0 = (blockIdx.x * p.tpw + tile_in_wg) * 16;
    const int n = lane & 15, kb = lane >> 4;
    const int NR = 2 * p.nc;  // input rows in LDS
    float2* xsc = (float2*)(lds + NR * RS);
    u8* buf = lds + NR * RS + 2 * KV + wave * 16 * ROW;
    u32x2 gv = tab_load_hand<F>();  // IQ2_XXS: this thread's grid entry (W >= 4: 256 threads)
    const ChunkOffsets<NI> co = mvd_offsets<D::PR, D::SLOTS, NI>(p, row0, lane);
    const u8* arow = lds + min(n, NR - 1) * RS + 8 * kb;
    float acc[2] = {0.f, 0.f};
    const int nr = KL ? p.nr : 1;
    for (int j = 0; j < nr; ++j) {
    const int k0 = j * KV, jb = j * (KV / 256);  // the range's first value and block
    const int rbj = KL && j == nr - 1 ? p.nblk - jb : KV / 256;  // blocks of this range
    const int KVj = rbj * 256, Sj = KVj / 32;
    const int nchj = KL ? rbj / (p.ks * D::CHB) : NCH;  // chunks of the wave's slice
    const int b0 = slice * D::CHB * nchj;
    if (KL && j > 0) lds_barrier();  // every wave done with the previous range's input

    // input rows: row r = xq (r even) or xq2 (r odd) of token r / 2, 1 KB per instruction, over the waves.
    // Only the present tokens' rows are held: the lanes of absent tokens' A rows read the last row, whose
    // products enter only MFMA result rows of those tokens, which are never stored (their (xd, xs) are 0).
    for (int r = wave; r < NR; r += W) {
        const int t = r >> 1;
        const int8_t* row = ((r & 1) ? p.xq2 : p.xq) + (int64_t)t * p.x_stride + k0;
        for (int m = 0; 1024 * m < KVj; ++m)
            if (1024 * m + 16 * lane < KVj) dma16s(row, (u32)(1024 * m + 16 * lane), lds + r * RS + 1024 * m);
    }
    // (xd, xs): piece i < 4 S = 4 consecutive steps (of S / 4 groups of 4) of token i & 7 of xd
    // (i / 8 < S / 4) or xs, read by hand.  Every thread issues both reads (threads past the pieces and
    // absent tokens re-read xd's first bytes): the code from the reads to their wait is straight-line,
    // so the compiler has no join at which it would copy a register whose read is still outstanding.
    u32x4 xv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = (int)threadIdx.x + k * nt, t = i & 7, g = i >> 3, a = g >= Sj / 4, m = g - a * (Sj / 4);
        const bool ok = i < 4 * Sj && t < p.nc;
        xv[k] = gload16(ok ? (a ? p.xs : p.xd) + (int64_t)t * (p.x_stride / 32) + k0 / 32 + 4 * m : p.xd);
    }
    // the first chunk's reads only once every wave has issued its input reads: the CU returns reads in
    // request order, so input requested after another wave's weights would wait for them (the barrier
    // waits for issue only: the reads are not counted by the compiler's waits)
    lds_barrier();
    mvd_chunk<F, NI>(buf, p, co, row0, jb + b0, lane);
    if constexpr (F == NMQ_IQ2_XXS)
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(xv[0]), "+v"(xv[1]), "+v"(gv) : "n"(NI) : "memory");
    else
        asm volatile("s_waitcnt vmcnt(%2)" : "+v"(xv[0]), "+v"(xv[1]) : "n"(NI) : "memory");
    if (j == 0) tab_store_hand<F>(tab, gv, nt);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = (int)threadIdx.x + k * nt, t = i & 7, g = i >> 3, a = g >= Sj / 4, m = g - a * (Sj / 4);
        if (i < 4 * Sj) {
            const float v[4] = {__uint_as_float(xv[k].x), __uint_as_float(xv[k].y), __uint_as_float(xv[k].z),
                                __uint_as_float(xv[k].w)};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ((float*)xsc)[((4 * m + e) * 8 + t) * 2 + a] = t < p.nc ? (a ? v[e] : v[e] * FEIN) : 0.f;
        }
    }
    lds_barrier();

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (KL && c >= nchj) break;
        vm_wait<0>();  // chunk c in the buffer
        typename D::Raw r;
        D::frag(r, buf + n * ROW, (int)(((int64_t)(jb + b0 + D::CHB * c) * Mfma<F>::BB) & 15), kb);
        if (c + 1 < nchj) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the operands read before the buffer is refilled
            mvd_chunk<F, NI>(buf, p, co, row0, jb + b0 + D::CHB * (c + 1), lane);
        }
#pragma unroll
        for (int i = 0; i < D::CHB; ++i) {
            const int b = b0 + D::CHB * c + i;  // block of the range
            D::block(r, i, arow + 256 * b, xsc + 64 * b + 2 * kb, kb, tab, acc);
        }
    }
    }  // K ranges

    // add the KS slices of each tile (as mvm_kernel)
    float* red = (float*)lds;
    lds_barrier();
    red[(wave * 64 + lane) * 2] = acc[0];
    red[(wave * 64 + lane) * 2 + 1] = acc[1];
    lds_barrier();
    if (slice == 0) {
        const int r = row0 + n;
        float s0 = 0.f, s1 = 0.f;
        for (int q = 0; q < p.ks; ++q) {
            const int ri = ((tile_in_wg * p.ks + q) * 64 + lane) * 2;
            s0 += red[ri];
            s1 += red[ri + 1];
        }
        const int t = 2 * kb;
        if (r < p.n_out) {
            auto* y0 = gpw<float>(p.y) + (int64_t)t * p.n_out + r;
            auto* y1 = y0 + p.n_out;
            if (t < p.nc) *y0 = p.acc_y ? *y0 + s0 : s0;
            if (t + 1 < p.nc) *y1 = p.acc_y ? *y1 + s1 : s1;
        }
    }
}

// ---- host side ------------------------------------------------------------------------------------

struct MvdShape {
    bool ok;
    int ks, tpw, grid_x, nch;
    int nr, rb;  // K ranges (the launch over long rows)
    size_t lds;
};

// MVD_MIN (Q4_K: 5, the others: 2) .. 8 tokens, rows of up to 4096 values (a multiple of 256 CHB, and of
// 16 bytes): tiles of 16 rows, about one workgroup of 4 .. 16 waves per CU, K slices of 1 or 2 chunks of
// CHB blocks.  The weights must start at a 16-byte boundary (global_load_lds_dwordx4).
template <int F>
inline MvdShape plan_mvd(int n_out, int n_in, int nc, int cus, int lds_max, const void* w, int min_nc = 0) {
    constexpr int CHB = Dma<F>::CHB;
    MvdShape s{};
    if (min_nc <= 0) min_nc = tune(TUNE_MVD_MIN, F == NMQ_Q4_K ? 5 : 2);
    if (!tune(TUNE_MVD, 1) || nc < min_nc || nc > 8 || n_in % (256 * CHB) ||
        n_in > 4096 || (uintptr_t)w % 16 || (int64_t)n_in / 256 * Mfma<F>::BB % 16)
        return s;
    const int nblk = n_in / 256;
    const int tiles = (n_out + 15) / 16;
    // workgroups per CU aimed at: two of half the waves for up to 4 tokens on more rows than CUs x 16
    // (the staged input is smaller; 14336x4096 at 2 / 4 tokens: Q6_K 19.3 / 19.5 -> 18.2 / 18.5 us, Q8_0
    // 16.5 / 16.6 -> 15.7 / 16.3, Q4_0 11.4 / 11.6 -> 11.3 / 11.4; TQ2_0 and IQ2_XXS 0.2-0.4 us slower,
    // so they keep one; at 8 tokens every format is slower with two)
    const int wgpc_def = nc <= 4 && tiles > cus && F != NMQ_TQ2_0 && F != NMQ_IQ2_XXS ? 2 : 1;
    const int wgpc = std::max(1, std::min(tune(TUNE_MVD_WGPC, wgpc_def), 4));
    int tpw = tune(TUNE_MVD_TPW, 0);
    if (tpw <= 0) tpw = std::min((tiles + cus * wgpc - 1) / (cus * wgpc), 8);
    int ks = tune(TUNE_MVD_KS, 0);
    if (ks <= 0) {
        ks = 1;
        while (ks * 2 * tpw <= 16 / wgpc && nblk % (ks * 2 * CHB) == 0) ks *= 2;  // slices of at least one chunk
    }
    if (tune(TUNE_MVD_TPW, 0) <= 0 && tune(TUNE_MVD_KS, 0) <= 0) {
        // slices of more than 2 chunks: fewer tiles per workgroup, more slices (Q8_0 14336x4096 at 8
        // tokens: 4 x 4 with 4-chunk slices 27.6 us, 2 x 8 with 2-chunk slices 17.4 us)
        while (nblk / ks > 2 * CHB && tpw > 1 && nblk % (ks * 2) == 0) {
            tpw = (tpw + 1) / 2;
            ks *= 2;
        }
    }
    if (ks < 1 || tpw < 1 || ks * tpw > 16 || ks * tpw < 4 || nblk % ks || (nblk / ks) % CHB) return s;
    s.nch = nblk / ks / CHB;
    if (s.nch != 1 && s.nch != 2) return s;
    s.ks = ks;
    s.tpw = tpw;
    s.grid_x = (tiles + tpw - 1) / tpw;
    s.lds = mvd_lds<F>(n_in, ks * tpw, nc);
    s.ok = s.lds + 4096 <= (size_t)lds_max;
    return s;
}

// Rows of 4097 .. 32768 values, 2..8 tokens, in one launch: nr equal K ranges of rb blocks (below), one
// tile per workgroup when the rows allow, the most slices (up to 16 waves) whose slice of a range is 1
// or 2 chunks.
template <int F>
inline MvdShape plan_mvd_long(int n_out, int n_in, int nc, int cus, int lds_max, const void* w, int64_t row_bytes) {
    constexpr int CHB = DmaSel<F, true>::T::CHB;
    MvdShape s{};
    if (!tune(TUNE_MVD, 1) || nc < 2 || nc > 8 || n_in % 256 || n_in <= 4096 || n_in > 8 * 4096 ||
        (uintptr_t)w % 16 || row_bytes % 16)
        return s;
    // ranges: the most blocks up to 16 that divide the row, fill whole chunks and start on 16-byte
    // boundaries (14336 values: 4 ranges of 14 blocks for Q4_K, Q4_0, Q8_0; 7 of 8 for the 210- and
    // 66-byte blocks); at least 8 blocks
    const int nblk = n_in / 256;
    int rb = 0;
    for (int c = std::min(16, nblk); c >= 8 && rb == 0; --c)
        if (nblk % c == 0 && c % CHB == 0 && (int64_t)c * Mfma<F>::BB % 16 == 0) rb = c;
    // equal ranges below 12 blocks: ranges of 16 and a shorter last one instead, where the same slices
    // fit both (14336 values: 16, 16, 16, 8 blocks for the 210- and 66-byte blocks instead of 7 x 8)
    int last = rb;
    if (rb < 12 && nblk > 16 && 16 * Mfma<F>::BB % 16 == 0 && tune(TUNE_MVD_UNEQ, 1) != 0) {
        const int l = nblk % 16 == 0 ? 16 : nblk % 16;
        if (l % CHB == 0) {
            rb = 16;
            last = l;
        }
    }
    if (rb == 0) return s;
    const int nr = (nblk + rb - 1) / rb;
    const int tiles = (n_out + 15) / 16;
    int tpw = tune(TUNE_MVD_TPW, 0);
    if (tpw <= 0) tpw = std::min((tiles + cus - 1) / cus, 8);
    int ks = tune(TUNE_MVD_KS, 0);
    if (ks <= 0)
        for (int k = 16 / tpw; k >= 1 && ks <= 0; --k)
            if (rb % (k * CHB) == 0 && rb / (k * CHB) <= 2 && last % (k * CHB) == 0) ks = k;
    if (ks < 1 || tpw < 1 || ks * tpw > 16 || ks * tpw < 4 || rb % (ks * CHB) || rb / (ks * CHB) > 2 ||
        last % (ks * CHB) || last / (ks * CHB) < 1)
        return s;
    s.nch = rb / (ks * CHB);
    s.ks = ks;
    s.tpw = tpw;
    s.grid_x = (tiles + tpw - 1) / tpw;
    s.nr = nr;
    s.rb = rb;
    s.lds = mvd_lds<F, true>(rb * 256, ks * tpw, nc);
    s.ok = s.lds + 4096 <= (size_t)lds_max;
    return s;
}

template <int F>
inline int launch_mvd_long(const MvdShape& s, MvmParams p, hipStream_t stream) {
    p.ks = s.ks;
    p.tpw = s.tpw;
    p.nr = s.nr;
    p.rb = s.rb;
    p.x_stride = p.n_in;
    void (*k)(MvmParams) = s.nch == 1 ? mvd_kernel<F, 1, true> : mvd_kernel<F, 2, true>;
    hipLaunchKernelGGL(k, dim3((unsigned)s.grid_x), dim3(64 * s.ks * s.tpw), s.lds, stream, p);
    return (int)hipGetLastError();
}

template <int F>
inline void (*pick_mvd(const MvdShape& s))(MvmParams) {
    return s.nch == 1 ? mvd_kernel<F, 1> : mvd_kernel<F, 2>;
}

template <int F>
inline int launch_mvd(const MvdShape& s, MvmParams p, hipStream_t stream) {
    p.ks = s.ks;
    p.tpw = s.tpw;
    if (p.x_stride == 0) p.x_stride = p.n_in;
    hipLaunchKernelGGL(pick_mvd<F>(s), dim3((unsigned)s.grid_x), dim3(64 * s.ks * s.tpw), s.lds, stream, p);
    return (int)hipGetLastError();
}

struct MvmShape {
    bool ok;
    int ks, tpw, grid_x, nb, g;
    bool ring;
    size_t lds;
};

// Tiles of 16 rows; K slices per tile and tiles per workgroup chosen for about one workgroup of up
// to 16 waves per CU (the staged input takes most of the LDS).  A slice of up to NBMAX blocks is held
// in registers whole; longer slices cycle through NBRING buffers.  9..16 tokens: two groups of 8 in
// one launch when their input fits the LDS.
template <int F>
inline MvmShape plan_mvm(int n_out, int n_in, int nc, int cus, int lds_max) {
    MvmShape s{};
    const int mode = tune(TUNE_MVM, 1);  // 0: never, 1: from MIN_NC tokens, 2: from 2 tokens
    if (mode == 0 || nc < (mode == 2 ? 2 : Mfma<F>::MIN_NC) || nc > 16 || n_in % 256) return s;
    s.g = nc > 8 ? 2 : 1;
    const int nblk = n_in / 256;
    const int tiles = (n_out + 15) / 16;
    int tpw = tune(TUNE_MVM_TPW, 0);
    if (tpw <= 0) tpw = (tiles + cus - 1) / cus;
    if (tpw > 16) tpw = 16;
    int ks = tune(TUNE_MVM_KS, 0);
    if (ks <= 0) {
        ks = 1;
        while (ks * 2 * tpw <= 16 && nblk % (ks * 2) == 0) ks *= 2;
    }
    if (nblk % ks || ks * tpw > 16) return s;
    const int bpr = nblk / ks;
    const int W = ks * tpw;
    s.ks = ks;
    s.tpw = tpw;
    s.grid_x = (tiles + tpw - 1) / tpw;
    s.ring = !(bpr <= Mfma<F>::NBMAX && (bpr & (bpr - 1)) == 0);
    s.nb = s.ring ? Mfma<F>::NBRING : bpr;
    s.lds = std::max((size_t)s.g * (n_in / 32) * 576, (size_t)W * 512 * s.g);
    s.ok = s.lds + 4096 <= (size_t)lds_max;
    return s;
}

template <int F, int G>
inline void (*pick_mvm(const MvmShape& s))(MvmParams) {
    constexpr int NBM = Mfma<F>::NBMAX;
    if (s.ring) return mvm_kernel<F, Mfma<F>::NBRING, true, G>;
    if (s.nb == 1) return mvm_kernel<F, 1, false, G>;
    if (s.nb == 2) return mvm_kernel<F, (NBM >= 2 ? 2 : 1), false, G>;
    if (s.nb == 4) return mvm_kernel<F, (NBM >= 4 ? 4 : 1), false, G>;
    return mvm_kernel<F, NBM, false, G>;
}

template <int F>
int launch_mvm(const MvmShape& s, MvmParams p, hipStream_t stream) {
    p.ks = s.ks;
    p.tpw = s.tpw;
    void (*k)(MvmParams) = s.g == 2 ? pick_mvm<F, 2>(s) : pick_mvm<F, 1>(s);
    hipLaunchKernelGGL(k, dim3((unsigned)s.grid_x), dim3(64 * s.ks * s.tpw), s.lds, stream, p);
    return (int)hipGetLastError();
}

}  // namespace nmq
