// Several tokens per launch (up to 64) on the fp16 matrix cores: v_mfma_f32_16x16x32_f16.
//
// What the reference's MMQ tiles compute (mmvq.py:536-724, 902-920: weights unpacked once per block,
// multiplied with every token's input on the matrix cores, fp32 sums), with more precision than their
// fp16 weights and fp16 input: here the weights stay exact and the input carries about 22 bits.
//
//   input   xs[t] = 2^(e - 8) for max_k |x[t][k]| = f 2^e (f in [.5, 1));  v = x / xs (exact)
//           xh = fp16(v), xl = fp16(v - xh)  (v - xh is exact; xh + xl is v to about 2^-22)
//           X[t][s] = sum of xh + xl over the 32 values of sub-block s (fp32)
//   Q4_K    w = d*sc_s*q - dmin*mn_s:  B = q*sc_s as fp16 (an integer <= 945: exact)
//           y[t][r] = xs[t] * sum_blocks [ d * C - dmin * sum_s mn_s X[t][s] ],  C = sum_k B (xh + xl)
//   Q6_K    w = d*sc_g*(q - 32), q - 32 = 8h + l (h in -4..3, l in 0..7):  B = 8h*sc_g + l*sc_g, each
//           part an fp16 integer of at most 4096 (multiples of 8) or 896 (exact), on the matrix cores
//           as two products;  y = xs * sum_blocks d * C
// C runs over the 8 steps (32 values) of a block on the matrix cores (exact products, fp32 sums) and
// is scaled by d once per block; the min term is one fp32 matrix product per block (16x16x4) added
// straight into the running sum.
//
// Operands (lane l; A and B use the same k mapping, so the order of k inside a step does not matter):
//   A[row = l % 16][k = 8 (l / 16) + j] = input of token l % 16 (8 halves per lane; xh, then xl)
//   B[k = 8 (l / 16) + j][col = l % 16] = weight of row l % 16 without d (8 halves per lane)
//   C[row = 4 (l / 16) + r][col = l % 16]: tokens 4 (l / 16) + r of the lane's own weight row
// So a lane builds 8 weights of its row per step straight from its own loads (the scale of each
// 16- or 32-value group belongs to the lane's own values), and its sums belong to that row: the
// block factors need no exchange between lanes.  Min term, 16x16x4 fp32 (lane l: A = X of token
// l % 16 and sub-block l / 16 (+ 4), B = dmin*mn of the same sub-block of row l % 16).
// The input is stored in operand order (by nmq_mm_input): the A fragment of 16 tokens and one step
// is 1 KB of consecutive memory, one full-width load per wave; X as [group][sub-block][token].
//
// Work split: a workgroup of 4 waves owns T tiles of 16 weight rows and NG groups of 16 tokens
// (blockIdx.y: which NG groups of the launch); wave w takes the w-th quarter of the row's 256-value
// blocks, so every input fragment a wave reads from global memory (the input of all tokens is small
// and shared by every workgroup) serves T tiles.  The 4 partial sums go through LDS and are added in
// wave order.
#pragma once

#include "nmq_mfma.hpp"

namespace nmq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MmhParams {
    const u8* w;
    const u16* xh;    // fp16 input, high part, in operand order (groups of 16 tokens)
    const u16* xl;    // low part
    const float* xsum;  // per token and sub-block: sum of xh + xl, [group][sub-block][16]
    const float* xs;  // per-token scale
    float* y;         // fp32, token-major (nc x n_out)
    int n_out, n_in, nc;
    int64_t row_bytes;
    int nblk;  // 256-value blocks per row
};

// Bytes 0, 1 (codes_lo) or 2, 3 (codes_hi) of v (each < 256) as the fp16 pair (b0 - off, b1 - off):
// 0x64 in the high byte is 1024, the byte the low 8 of the 10 mantissa bits; off >= 1024 (exact).
__device__ __forceinline__ h2 codes_lo(u32 v, _Float16 off) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) - h2{off, off};
}
__device__ __forceinline__ h2 codes_hi(u32 v, _Float16 off) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) - h2{off, off};
}
__device__ __forceinline__ u32 hbits(h2 v) { return __builtin_bit_cast(u32, v); }
// 8 code bytes (each < 256) as 8 fp16 values (byte + 1024 - off) * f
__device__ __forceinline__ u32x4 codes8(u32 lo, u32 hi, _Float16 off, _Float16 f) {
    const h2 f2 = {f, f};
    return u32x4{hbits(codes_lo(lo, off) * f2), hbits(codes_hi(lo, off) * f2), hbits(codes_lo(hi, off) * f2),
                 hbits(codes_hi(hi, off) * f2)};
}

__device__ __forceinline__ f32x4 mfma_h(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

template <int F>
struct Mmh;

template <>
struct Mmh<NMQ_Q4_K> {
    static constexpr bool MIN = true;   // has the dmin * mn * X term
    static constexpr int NB = 1;        // B operands per step
    // per block and lane: sc of the 8 sub-blocks as fp16 pairs, d, and dmin * mn of sub-blocks kb, 4 + kb
    struct Blk {
        h2 sc[4];
        float d, m0, m1;
    };
    __device__ static void block(const Mfma<NMQ_Q4_K>::Raw& r, int kb, Blk& B) {
        // get_scale_min_k4: sub-blocks 0..3 in the low 6 bits of bytes 0..3 (sc) and 4..7 (mn);
        // 4..7 from the nibbles of bytes 8..11 and the top 2 bits of bytes 0..7
        const u32 s_lo = r.h.y & 0x3f3f3f3fu, s_hi = (r.h.w & 0x0f0f0f0fu) | ((r.h.y >> 2) & 0x30303030u);
        const u32 m_lo = r.h.z & 0x3f3f3f3fu, m_hi = ((r.h.w >> 4) & 0x0f0f0f0fu) | ((r.h.z >> 2) & 0x30303030u);
        const _Float16 k = (_Float16)1024.f;
        B.sc[0] = codes_lo(s_lo, k);
        B.sc[1] = codes_hi(s_lo, k);
        B.sc[2] = codes_lo(s_hi, k);
        B.sc[3] = codes_hi(s_hi, k);
        B.d = h2f(r.h.x);
        const float dmin = h2f(r.h.x >> 16);
        B.m0 = dmin * (float)((m_lo >> (8 * kb)) & 0xffu);
        B.m1 = dmin * (float)((m_hi >> (8 * kb)) & 0xffu);
    }
    // step s (sub-block s): q * sc_s for values 8kb .. 8kb + 7, q = nibble (s & 1) of qs[32 (s >> 1) + 8kb ..]
    __device__ static void codes(const Mfma<NMQ_Q4_K>::Raw& r, const Blk& B, int s, int /*kb*/, u32x4 (&b)[1]) {
        const u32x2 v = r.q[s >> 1];
        const int sh = 4 * (s & 1);
        b[0] = codes8((v.x >> sh) & 0x0f0f0f0fu, (v.y >> sh) & 0x0f0f0f0fu, (_Float16)1024.f, B.sc[s >> 1][s & 1]);
    }
};

template <>
struct Mmh<NMQ_Q6_K> {
    static constexpr bool MIN = false;
    static constexpr int NB = 2;        // 8h * sc and l * sc
    // per block and lane: sc of the lane's 16-value group in each of the 8 steps (group 2s + kb / 2)
    struct Blk {
        h2 sc[4];
        float d;
    };
    __device__ static void block(const Mfma<NMQ_Q6_K>::Raw& r, int kb, Blk& B) {
        const u32 sel = (kb >> 1) ? 0x07050301u : 0x06040200u;  // odd or even bytes of the pair
        const u32 lo = __builtin_amdgcn_perm(r.sc.y, r.sc.x, sel) ^ 0x80808080u;  // int8 + 128
        const u32 hi = __builtin_amdgcn_perm(r.sc.w, r.sc.z, sel) ^ 0x80808080u;
        const _Float16 k = (_Float16)1152.f;
        B.sc[0] = codes_lo(lo, k);
        B.sc[1] = codes_hi(lo, k);
        B.sc[2] = codes_lo(hi, k);
        B.sc[3] = codes_hi(hi, k);
        B.d = h2f(r.d);
    }
    // step s = 4n + k: values 128n + 32k + 8kb + j, q = nibble (k >> 1) of ql[64n + 32(k & 1) + l] |
    // bits 2k of qh[32n + l] << 4; q - 32 = 8 ((q >> 3) - 4) + (q & 7)
    __device__ static void codes(const Mfma<NMQ_Q6_K>::Raw& r, const Blk& B, int s, int /*kb*/, u32x4 (&b)[2]) {
        const int n = s >> 2, k = s & 3;
        const u32x2 l = r.ql[2 * n + (k & 1)], h = r.qh[n];
        const int ls = 4 * (k >> 1), hs = 2 * k;
        const u32 lo = ((l.x >> ls) & 0x0f0f0f0fu) | (((h.x >> hs) & 0x03030303u) << 4);
        const u32 hi = ((l.y >> ls) & 0x0f0f0f0fu) | (((h.y >> hs) & 0x03030303u) << 4);
        const _Float16 sc = B.sc[s >> 1][s & 1];
        b[0] = codes8((lo >> 3) & 0x07070707u, (hi >> 3) & 0x07070707u, (_Float16)1028.f, sc * (_Float16)8.f);
        b[1] = codes8(lo & 0x07070707u, hi & 0x07070707u, (_Float16)1024.f, sc);
    }
};

template <int T, int NG>
struct MmhDepth {
    static constexpr int D = T * NG >= 8 ? 2 : 4;  // input steps in flight ahead of the one computed
};

template <int F, int T, int NG>
__global__ __launch_bounds__(256) void mmh_kernel(MmhParams p) {
    using M = Mfma<F>;
    using H = Mmh<F>;
    constexpr int D = MmhDepth<T, NG>::D;
    __shared__ f32x4 red[4 * T * NG * 64];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kb = lane >> 4;
    const int tile0 = blockIdx.x * T;
    const u8* rowp[T];
#pragma unroll
    for (int t = 0; t < T; ++t) rowp[t] = p.w + (int64_t)min((tile0 + t) * 16 + n, p.n_out - 1) * p.row_bytes;
    // the input is stored in operand order: one 512-half fragment per (group of 16 tokens, step)
    const int nsb = p.n_in / 32;  // sub-blocks (steps) per row
    const int ng_all = (p.nc + 15) >> 4, g0 = blockIdx.y * NG;
    int64_t xo[NG];
    int gi[NG];  // groups of this workgroup (past the last one: the last one again, not stored)
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        gi[g] = min(g0 + g, ng_all - 1);
        xo[g] = (int64_t)gi[g] * nsb * 512 + 8 * lane;
    }
    const int per = (p.nblk + 3) >> 2;
    const int b0 = min(wave * per, p.nblk), b1 = min(b0 + per, p.nblk);

    f32x4 acc[T][NG];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < NG; ++g) acc[t][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (b0 < b1) {
        typename M::Raw cur[T], nxt[T];
#pragma unroll
        for (int t = 0; t < T; ++t) M::load(rowp[t] + (int64_t)b0 * M::BB, kb, cur[t]);
        u32x4 xh[D][NG], xl[D][NG];
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                xh[d][g] = *gp<u32x4>(p.xh + xo[g] + 512 * (8 * b0 + d));
                xl[d][g] = *gp<u32x4>(p.xl + xo[g] + 512 * (8 * b0 + d));
            }
        for (int b = b0; b < b1; ++b) {
            const int bn = b + 1 < b1 ? b + 1 : b;  // the last block re-reads itself
#pragma unroll
            for (int t = 0; t < T; ++t) M::load(rowp[t] + (int64_t)bn * M::BB, kb, nxt[t]);
            float X0[NG], X1[NG];  // X of token n, sub-blocks 8b + kb and 8b + 4 + kb
            if constexpr (H::MIN) {
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const float* xp = p.xsum + ((int64_t)gi[g] * nsb + 8 * b + kb) * 16 + n;
                    X0[g] = gp<float>(xp)[0];
                    X1[g] = gp<float>(xp)[64];
                }
            }
            typename H::Blk bk[T];
#pragma unroll
            for (int t = 0; t < T; ++t) H::block(cur[t], kb, bk[t]);
            f32x4 c[T][NG];
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < NG; ++g) c[t][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                u32x4 q[T][H::NB];
#pragma unroll
                for (int t = 0; t < T; ++t) H::codes(cur[t], bk[t], s, kb, q[t]);
#pragma unroll
                for (int i = 0; i < H::NB; ++i)
#pragma unroll
                    for (int t = 0; t < T; ++t)
#pragma unroll
                        for (int g = 0; g < NG; ++g) c[t][g] = mfma_h(xh[s % D][g], q[t][i], c[t][g]);
#pragma unroll
                for (int i = 0; i < H::NB; ++i)
#pragma unroll
                    for (int t = 0; t < T; ++t)
#pragma unroll
                        for (int g = 0; g < NG; ++g) c[t][g] = mfma_h(xl[s % D][g], q[t][i], c[t][g]);
                const int sn = s + D;
                const int bb = sn < 8 ? b : bn;
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    xh[s % D][g] = *gp<u32x4>(p.xh + xo[g] + 512 * (8 * bb + (sn & 7)));
                    xl[s % D][g] = *gp<u32x4>(p.xl + xo[g] + 512 * (8 * bb + (sn & 7)));
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    if constexpr (H::MIN) {  // acc -= sum_s dmin*mn_s * X_s (two fp32 products of K = 4)
                        acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x4f32(X0[g], -bk[t].m0, acc[t][g], 0, 0, 0);
                        acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x4f32(X1[g], -bk[t].m1, acc[t][g], 0, 0, 0);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][g][r] = fmaf(bk[t].d, c[t][g][r], acc[t][g][r]);
                }
#pragma unroll
            for (int t = 0; t < T; ++t) cur[t] = nxt[t];
        }
    }

    // partial sums of the 4 K quarters, added in wave order; lane: row tile*16 + n, tokens 4kb + r
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < NG; ++g) red[((wave * T + t) * NG + g) * 64 + lane] = acc[t][g];
    __syncthreads();
    for (int i = wave; i < T * NG; i += 4) {
        const int t = i / NG, g = i % NG;
        f32x4 s = red[(t * NG + g) * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) s += red[((w * T + t) * NG + g) * 64 + lane];
        const int row = (tile0 + t) * 16 + n;
        if (row < p.n_out) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = 16 * (g0 + g) + 4 * kb + r;
                if (tok < p.nc) gpw<float>(p.y)[(int64_t)tok * p.n_out + row] = s[r] * gp<float>(p.xs)[tok];
            }
        }
    }
}

// ---- host side ------------------------------------------------------------------------------------

constexpr int MMH_MAX_COLS = 64;  // tokens per launch (4 groups of 16)

// Tiles per workgroup: the most (of 4, 2, 1) that still gives nearly every CU a workgroup.
inline int plan_mmh_tiles(int n_out, int cus) {
    const int tiles = (n_out + 15) / 16;
    const int e = tune(TUNE_MMH_T, 0);
    if (e == 1 || e == 2 || e == 4) return e;
    if ((tiles + 3) / 4 >= cus * 7 / 8) return 4;
    if ((tiles + 1) / 2 >= cus * 7 / 8) return 2;
    return 1;
}

template <int F, int T>
inline void (*pick_mmh_ng(int ng))(MmhParams) {
    switch (ng) {
        case 1: return mmh_kernel<F, T, 1>;
        case 2: return mmh_kernel<F, T, 2>;
        case 3: return mmh_kernel<F, T, 3>;
        default: return mmh_kernel<F, T, 4>;
    }
}

// One launch of 1..MMH_MAX_COLS tokens.
template <int F>
int launch_mmh(MmhParams p, hipStream_t stream) {
    const DeviceInfo di = device_info();
    p.nblk = p.n_in / 256;
    p.row_bytes = (int64_t)p.nblk * Mfma<F>::BB;
    const int T = plan_mmh_tiles(p.n_out, di.cus);
    const int ng_all = (p.nc + 15) / 16;
    const int eg = tune(TUNE_MMH_G, 0);  // groups of 16 tokens per workgroup
    const int ng = eg >= 1 && eg <= ng_all ? eg : ng_all;
    void (*k)(MmhParams) = T == 4 ? pick_mmh_ng<F, 4>(ng) : T == 2 ? pick_mmh_ng<F, 2>(ng) : pick_mmh_ng<F, 1>(ng);
    const int tiles = (p.n_out + 15) / 16;
    hipLaunchKernelGGL(k, dim3((unsigned)((tiles + T - 1) / T), (unsigned)((ng_all + ng - 1) / ng)), dim3(256), 0,
                       stream, p);
    return (int)hipGetLastError();
}

}  // namespace nmq
