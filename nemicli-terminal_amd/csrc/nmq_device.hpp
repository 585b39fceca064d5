// Device-side building blocks of the gfx950 GGUF mat-vec kernels: scalar helpers, the two-stage
// int8 input slice a lane works on, and one "unit" decoder per block format.
//
// A unit is the piece of one weight row a lane handles at a time: 64 values, decoded to sixteen
// dwords of four int8 weights each (w[0..15]) plus fp32 factors per 16 values.  The sixteen dwords
// are ordered like the lane's slice of the input, so w[k] pairs with xq dword k.  Two slice shapes:
//   contiguous (Q4_K, Q8_0, IQ2_XXS): the unit covers values 64u .. 64u+63 of the row; runs 0,1
//     (values 0..31) share one weight factor and xd, runs 2,3 the next.
//   strided (Q6_K, TQ2_0): unit u = 4b + 2h + j of block b covers the four 16-value runs at
//     256b + 128h + 32k + 16j (k = 0..3), one weight factor and one xd per run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nmq.h"

namespace nmq {

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

// Loads of weight bytes.  Q6_K (210 B), Q8_0 (34 B), TQ2_0 and IQ2_XXS (66 B) blocks are only
// 2-byte aligned; gfx950 serves dword-multiple global loads at any alignment, and these types tell
// the compiler so (it emits global_load_dwordx4 / dwordx2 / dword for them).
typedef u32 u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef u32 u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef u32 u32_a2 __attribute__((aligned(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));

constexpr float FEIN = 1.0f / 254.0f;  // scale of the second input stage relative to xd

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every global read the wave
// has in flight (on this GPU family reads and writes share one counter and its fence waits for it),
// which would stall a kernel that issues its weight reads before the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Xor butterflies over the 32 lanes of each half-wave with offsets 16, 8, 4, 2, 1 (the tree of the
// reference's warp_sum, mmvq.py:42-46): the xor-16 level by ds_swizzle (bitmask mode, inside 32
// lanes), the others by DPP rotations of 16-lane rows.  After the xor-16 level a lane's partial
// depends only on its index modulo 16, after xor 8 modulo 8, and so on, so rotating the row by 8, 4,
// 2, 1 hands each lane a copy of its xor partner's partial: the same additions (own + partner) as
// the xor butterfly, hence bit-identical sums.  All 32 lanes of a half-wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swz_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
}
__device__ __forceinline__ float swz_xor4(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x101f));
}

__device__ __forceinline__ float half_sum_xor(float v) {
    v += swz_xor16(v);
    v += dpp_f<0x128>(v);  // row_ror:8
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x122>(v);  // row_ror:2
    v += dpp_f<0x121>(v);  // row_ror:1
    return v;
}
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, swz_xor16(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x122>(v));
    v = fmaxf(v, dpp_f<0x121>(v));
    return v;
}

// fp32 -> bf16 (returned as fp32), round to nearest even; NaN stays NaN (torch's .to(torch.bfloat16)).
__device__ __forceinline__ float round_bf16(float f) {
    const u32 u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);  // NaN
    return __uint_as_float((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
}

// The activation of an FFN's gate value g (reference mmvq.py:122-133): silu(g) = g / (1 + exp(-g)) with an
// IEEE division, or the tanh form of gelu.  Every kernel that forms an activation calls these expressions,
// so that they agree bit for bit.
__device__ __forceinline__ float act_value(float g, bool gelu) {
    return gelu ? 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g))) : g / (1.0f + expf(-g));
}

// The gated activation of an expert MLP as its down projection takes it: bf16(silu(g) * u).
__device__ __forceinline__ float silu_mul_bf16(float g, float u) { return round_bf16(act_value(g, false) * u); }

// Two-stage int8 input (reference mmvq.py:59-83) of the value v held by this lane (group = the lane's
// 32-lane half): d = max|v| / 127 over the group, q = rint(v / d), q2 = the rounded residual in units of
// d / 254, and the group's sum (half_max / half_sum_xor).  All 32 lanes of the half-wave take part.
struct Quant32 {
    int q, q2;
    float d, s;
};

__device__ __forceinline__ Quant32 quant32(float v) {
    Quant32 r;
    const float a = half_max(fabsf(v));
    r.d = a / 127.0f;
    r.q = 0;
    r.q2 = 0;
    if (r.d > 0.0f) {
        r.q = (int)rintf(v / r.d);
        const float e = fmaf(-(float)r.q, r.d, v);
        const int q2 = (int)rintf(e / (r.d * FEIN));
        r.q2 = q2 < -127 ? -127 : (q2 > 127 ? 127 : q2);
    }
    r.s = half_sum_xor(v);
    return r;
}

// quant32 of v stored as value index i (i % 32 == lane % 32).
__device__ __forceinline__ void quant32_store(float v, int64_t i, int8_t* __restrict__ xq, int8_t* __restrict__ xq2,
                                              float* __restrict__ xd, float* __restrict__ xs) {
    const Quant32 r = quant32(v);
    xq[i] = (int8_t)r.q;
    xq2[i] = (int8_t)r.q2;
    if ((threadIdx.x & 31) == 0) {
        xd[i >> 5] = r.d;
        xs[i >> 5] = r.s;
    }
}

__device__ __forceinline__ float h2f(u32 bits16) {
    return (float)__builtin_bit_cast(_Float16, (u16)(bits16 & 0xffffu));
}

__device__ __forceinline__ int dot4(u32 a, u32 b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ u32 bfe(u32 v, u32 off, u32 len) { return __builtin_amdgcn_ubfe(v, off, len); }

// Every pointer the kernels dereference in device memory is cast to the global address space, so
// the loads are global_load (counted by vmcnt only) rather than flat loads, whose completion would
// also hold back the waits for LDS reads.
#define NMQ_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const NMQ_GLOBAL T* gp(const void* p) {
    return (const NMQ_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ NMQ_GLOBAL T* gpw(void* p) {
    return (NMQ_GLOBAL T*)p;
}
__device__ __forceinline__ u32x4 ld4(const u8* p) { return *gp<u32x4_a2>(p); }
__device__ __forceinline__ u32x4 ld4a(const u8* p) { return *gp<u32x4>(p); }  // 16-byte aligned
__device__ __forceinline__ u32x2 ld2(const u8* p) { return *gp<u32x2_a2>(p); }
__device__ __forceinline__ u32 ld1(const u8* p) { return *gp<u32_a2>(p); }
__device__ __forceinline__ u32 ld16(const u8* p) { return *gp<u16>(p); }

// Q6_K code bytes (0..63) of group g (0..3) from a dword of ql (la for even g, lb for odd) and of qh:
// low nibbles of ql for g < 2, high ones for g >= 2, and qh bits 2g, 2g+1 of every byte at bits 4, 5
// (qh shifted by 4 - 2g and masked: the same bytes as ((qh >> 2g) & 3) << 4, one instruction fewer).
template <int G>
__device__ __forceinline__ u32 q6k_codes(u32 ql, u32 qh) {
    const u32 hb = G == 0 ? (qh << 4) : (G == 1 ? (qh << 2) : (G == 2 ? qh : (qh >> 2)));
    return ((G >= 2 ? (ql >> 4) : ql) & 0x0f0f0f0fu) | (hb & 0x30303030u);
}

// q - 32 per byte for bytes 0..63 (Q6_K): ((q | 0x80) - 0x20) ^ 0x80 never borrows across bytes.
__device__ __forceinline__ u32 sub32x4(u32 v) { return ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }
// code - 1 per byte for codes 0..3 (TQ2_0): (c + 0x7f) ^ 0x80 never carries across bytes.
__device__ __forceinline__ u32 sub1x4(u32 v) { return (v + 0x7f7f7f7fu) ^ 0x80808080u; }
// q - 8 per byte for nibbles 0..15 (Q4_0): (q + 0x78) ^ 0x80 never carries across bytes.
__device__ __forceinline__ u32 sub8x4(u32 v) { return (v + 0x78787878u) ^ 0x80808080u; }

// The two-stage input of one unit for one token (read from LDS).
struct XSlice {
    u32 q[16];   // xq bytes in unit order
    u32 q2[16];  // xq2 bytes
    float d[4];  // xd: contiguous shape uses d[0], d[1]; strided shape d[0..3]
    float s[2];  // xs (contiguous shape only; Q4_K min term)
};

// Weight factors of one decoded unit.
struct WUnit {
    u32 w[16];
    float ws[4];  // per run (contiguous shape: ws[0] for runs 0,1 and ws[2] for runs 2,3)
    float wm[2];  // Q4_K: dmin*m of the two sub-blocks; 0 otherwise
};

// Integer sums of one unit against one token's slice, run by run (exposed for the diagnostic).
__device__ __forceinline__ void unit_sums(const u32 (&w)[16], const XSlice& x, int (&s1)[4], int (&s2)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int a = 0, b = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a = dot4(w[4 * r + k], x.q[4 * r + k], a);
            b = dot4(w[4 * r + k], x.q2[4 * r + k], b);
        }
        s1[r] = a;
        s2[r] = b;
    }
}

template <bool STRIDED, bool HAS_MIN>
__device__ __forceinline__ float unit_dot(const WUnit& u, const XSlice& x) {
    int s1[4], s2[4];
    unit_sums(u.w, x, s1, s2);
    if (STRIDED) {
        float acc = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc += u.ws[r] * x.d[r] * ((float)s1[r] + FEIN * (float)s2[r]);
        return acc;
    } else {
        const float f0 = (float)(s1[0] + s1[1]) + FEIN * (float)(s2[0] + s2[1]);
        const float f1 = (float)(s1[2] + s1[3]) + FEIN * (float)(s2[2] + s2[3]);
        float acc = u.ws[0] * x.d[0] * f0 + u.ws[2] * x.d[1] * f1;
        if (HAS_MIN) acc -= u.wm[0] * x.s[0] + u.wm[1] * x.s[1];
        return acc;
    }
}

// ---- per-format unit decoders -------------------------------------------------------------------
// Fmt<F>::Raw holds the loaded bytes of one unit; load() never touches memory outside the row
// (row_units = units in the row; a Q8_0 row may end with half a unit).  decode() turns the bytes
// into a WUnit.  `tab` points at the LDS tables (IQ2_XXS only).

template <int F>
struct Fmt;

// Q4_K, 144-byte blocks (reference quant.py:111-120, mmvq.py:333-419): unit u = group i = u % 4
// of block u / 4: qs bytes 32i .. 32i+31 hold sub-block 2i (low nibbles) and 2i+1 (high nibbles).
template <>
struct Fmt<NMQ_Q4_K> {
    static constexpr int BV = 256, BB = 144;
    static constexpr bool STRIDED = false, HAS_MIN = true;
    struct Raw {
        u32x4 a, b, h;
    };
    __device__ static void load(const u8* row, int u, int /*row_units*/, Raw& r) {
        const u8* blk = row + (u >> 2) * BB;
        const int i = u & 3;
        r.h = ld4a(blk);  // d, dmin, scales[12]: 16-byte aligned when the row is
        r.a = ld4a(blk + 16 + 32 * i);
        r.b = ld4a(blk + 32 + 32 * i);
    }
    __device__ static void decode(const Raw& r, int u, const u64* /*tab*/, WUnit& o) {
        const u32 q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o.w[k] = q[k] & 0x0f0f0f0fu;
            o.w[8 + k] = (q[k] >> 4) & 0x0f0f0f0fu;
        }
        // get_scale_min_k4 for sub-blocks j = 2i and 2i+1 (t = j % 4, both in the same half)
        const int i = u & 3;
        const bool hi = i >= 2;
        const u32 t0 = (u32)(2 * i) & 3u;
        float sc[2], mn[2];
#pragma unroll
        for (int z = 0; z < 2; ++z) {
            const u32 sh = 8u * (t0 + z);
            const u32 A = bfe(r.h.y, sh, 8), B = bfe(r.h.z, sh, 8), C = bfe(r.h.w, sh, 8);
            const u32 s = hi ? ((C & 15u) | ((A >> 6) << 4)) : (A & 63u);
            const u32 m = hi ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63u);
            sc[z] = (float)s;
            mn[z] = (float)m;
        }
        const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
        o.ws[0] = o.ws[1] = d * sc[0];
        o.ws[2] = o.ws[3] = d * sc[1];
        o.wm[0] = dmin * mn[0];
        o.wm[1] = dmin * mn[1];
    }
};

// One-token fast path of Q4_K (mv1): decode and dot fused, branch free.  The eight 6-bit scales and
// mins of a block (get_scale_min_k4) are, four at a time inside dwords:
//   sc[0..3] = scales[0..3] & 63              m[0..3] = scales[4..7] & 63
//   sc[4..7] = (scales[8..11] & 15) | (scales[0..3] >> 6) << 4
//   m[4..7]  = (scales[8..11] >> 4) | (scales[4..7] >> 6) << 4
// A lane's unit always takes sub-blocks 2i, 2i+1 = bytes t0, t0 + 1 of the low (i < 2) or high half, so
// the choice of half and byte folds into lane-constant shifts and masks (Q4kLane):
//   sc pair = ((h.w >> sw) & ma) | ((h.y >> sy) & mb),   m pair = ((h.w >> sm) & ma) | ((h.z >> sy) & mb)
// with, low half: ma = 0, mb = 0x3f3f3f3f, sy = 8 t0; high half: ma = 0x0f0f0f0f, mb = 0x30303030,
// sy = 8 t0 + 2, sw = 8 t0, sm = 8 t0 + 4; the scales and mins are then bytes 0 and 1.  Runs 0,1 and
// 2,3 are summed in one dot4 chain each; the two stages combine as an integer 254 S1 + S2 (exact in
// fp32: |254 S1 + S2| < 2^24) times xd / 254.
struct Q4kLane {
    u32 sw, sm, sy, ma, mb;
};

__device__ __forceinline__ Q4kLane q4k_lane(int u) {
    const int i = u & 3;
    const u32 t = 8u * (u32)((2 * i) & 3);
    Q4kLane c;
    if (i >= 2) {
        c.ma = 0x0f0f0f0fu; c.mb = 0x30303030u; c.sy = t + 2u; c.sw = t; c.sm = t + 4u;
    } else {
        c.ma = 0u; c.mb = 0x3f3f3f3fu; c.sy = t; c.sw = 0u; c.sm = 0u;
    }
    return c;
}

__device__ __forceinline__ float q4k_dot1(const Fmt<NMQ_Q4_K>::Raw& r, const XSlice& x, const Q4kLane& c) {
    const u32 sv = ((r.h.w >> c.sw) & c.ma) | ((r.h.y >> c.sy) & c.mb);
    const u32 mv = ((r.h.w >> c.sm) & c.ma) | ((r.h.z >> c.sy) & c.mb);
    const float sc0 = (float)(sv & 0xffu), sc1 = (float)((sv >> 8) & 0xffu);  // v_cvt_f32_ubyte0/1
    const float m0 = (float)(mv & 0xffu), m1 = (float)((mv >> 8) & 0xffu);
    const u32 q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    int a0 = 0, a1 = 0, b0 = 0, b1 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const u32 lo = q[k] & 0x0f0f0f0fu, hn = (q[k] >> 4) & 0x0f0f0f0fu;
        a0 = dot4(lo, x.q[k], a0);
        b0 = dot4(lo, x.q2[k], b0);
        a1 = dot4(hn, x.q[8 + k], a1);
        b1 = dot4(hn, x.q2[8 + k], b1);
    }
    const float g0 = (float)(__mul24(a0, 254) + b0) * (x.d[0] * FEIN);  // |a0| <= 32 * 15 * 127: 24-bit
    const float g1 = (float)(__mul24(a1, 254) + b1) * (x.d[1] * FEIN);
    const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
    return d * (sc0 * g0 + sc1 * g1) - dmin * (m0 * x.s[0] + m1 * x.s[1]);
}

// NC tokens at once (the same weights, NC inputs): the nibble unpacking, scales and mins shared, each
// token's result formed by exactly the expression of q4k_dot1.
template <int NC>
__device__ __forceinline__ void q4k_dotn(const Fmt<NMQ_Q4_K>::Raw& r, const XSlice* x, const Q4kLane& c, float* o) {
    const u32 sv = ((r.h.w >> c.sw) & c.ma) | ((r.h.y >> c.sy) & c.mb);
    const u32 mv = ((r.h.w >> c.sm) & c.ma) | ((r.h.z >> c.sy) & c.mb);
    const float sc0 = (float)(sv & 0xffu), sc1 = (float)((sv >> 8) & 0xffu);
    const float m0 = (float)(mv & 0xffu), m1 = (float)((mv >> 8) & 0xffu);
    const u32 q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    int a0[NC], a1[NC], b0[NC], b1[NC];
#pragma unroll
    for (int t = 0; t < NC; ++t) a0[t] = a1[t] = b0[t] = b1[t] = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const u32 lo = q[k] & 0x0f0f0f0fu, hn = (q[k] >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int t = 0; t < NC; ++t) {
            a0[t] = dot4(lo, x[t].q[k], a0[t]);
            b0[t] = dot4(lo, x[t].q2[k], b0[t]);
            a1[t] = dot4(hn, x[t].q[8 + k], a1[t]);
            b1[t] = dot4(hn, x[t].q2[8 + k], b1[t]);
        }
    }
    const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
#pragma unroll
    for (int t = 0; t < NC; ++t) {
        const float g0 = (float)(__mul24(a0[t], 254) + b0[t]) * (x[t].d[0] * FEIN);
        const float g1 = (float)(__mul24(a1[t], 254) + b1[t]) * (x[t].d[1] * FEIN);
        o[t] = d * (sc0 * g0 + sc1 * g1) - dmin * (m0 * x[t].s[0] + m1 * x[t].s[1]);
    }
}

// Q6_K, 210-byte blocks (quant.py:140-159, mmvq.py:421-482): unit u = 4b + 2h + j takes
// l = 16j .. 16j+15 of half h: ql[64h + l], ql[64h + 32 + l], qh[32h + l]; runs k = 0..3 are the
// values 128h + 32k + l with the int8 scales sc[8h + 2k + j].
template <>
struct Fmt<NMQ_Q6_K> {
    static constexpr int BV = 256, BB = 210;
    static constexpr bool STRIDED = true, HAS_MIN = false;
    struct Raw {
        u32x4 la, lb, qh;
        u32x2 sc;
        u32 d;
    };
    __device__ static void load(const u8* row, int u, int /*row_units*/, Raw& r) {
        const u8* blk = row + (u >> 2) * BB;
        const int h = (u >> 1) & 1, j = u & 1;
        r.la = ld4(blk + 64 * h + 16 * j);
        r.lb = ld4(blk + 64 * h + 32 + 16 * j);
        r.qh = ld4(blk + 128 + 32 * h + 16 * j);
        r.sc = ld2(blk + 192 + 8 * h);
        r.d = ld16(blk + 208);
    }
    __device__ static void decode(const Raw& r, int u, const u64* /*tab*/, WUnit& o) {
        const u32 la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
        const u32 lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
        const u32 qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o.w[0 + k] = sub32x4((la[k] & 0x0f0f0f0fu) | ((qh[k] & 0x03030303u) << 4));
            o.w[4 + k] = sub32x4((lb[k] & 0x0f0f0f0fu) | (((qh[k] >> 2) & 0x03030303u) << 4));
            o.w[8 + k] = sub32x4(((la[k] >> 4) & 0x0f0f0f0fu) | (((qh[k] >> 4) & 0x03030303u) << 4));
            o.w[12 + k] = sub32x4(((lb[k] >> 4) & 0x0f0f0f0fu) | (((qh[k] >> 6) & 0x03030303u) << 4));
        }
        const int j = u & 1;
        const float d = h2f(r.d);
        // scale bytes sc[8h + 2k + j]: k = 0,1 in the low dword, k = 2,3 in the high one
        const u32 sh = 8u * j;
        o.ws[0] = d * (float)(int8_t)bfe(r.sc.x, sh, 8);
        o.ws[1] = d * (float)(int8_t)bfe(r.sc.x, sh + 16, 8);
        o.ws[2] = d * (float)(int8_t)bfe(r.sc.y, sh, 8);
        o.ws[3] = d * (float)(int8_t)bfe(r.sc.y, sh + 16, 8);
        o.wm[0] = o.wm[1] = 0.f;
    }
};

// Q6_K unit (one token) on the raw 6-bit codes c (0..63, signed bytes as they are; value c - 32), one
// 16-value group g at a time: with S1' = sum c xq and S2' = sum c xq2 over the group,
//   254 sum (c - 32) xq + sum (c - 32) xq2 = 254 S1' + S2' - 32 (254 X1 + X2),
// X1, X2 the group's input sums.  The xq2 chain starts at the group's input constant -32 (254 X1 + X2)
// (Q6kLane, formed once per input slice), one 24-bit multiply-add joins the stages (|S1'| <= 16*63*127),
// the integer (|.| < 2^24, exact in fp32) is weighted by the int8 sub-block scale times xd / 254, and the
// block scale d multiplies the unit's sum.  Every kernel forms each group's term with this expression, so
// the one-token and few-token kernels agree bit for bit.
struct Q6kLane {
    int k[4];    // xq2 chain start per 16-value group
    float e[4];  // xd / 254 per group
};

__device__ __forceinline__ int q6k_group_const(u32 q0, u32 q1, u32 q2, u32 q3, u32 r0, u32 r1, u32 r2, u32 r3) {
    int x1 = dot4(0x01010101u, q0, 0), x2 = dot4(0x01010101u, r0, 0);
    x1 = dot4(0x01010101u, q1, x1); x2 = dot4(0x01010101u, r1, x2);
    x1 = dot4(0x01010101u, q2, x1); x2 = dot4(0x01010101u, r2, x2);
    x1 = dot4(0x01010101u, q3, x1); x2 = dot4(0x01010101u, r3, x2);
    return -32 * (254 * x1 + x2);
}

__device__ __forceinline__ Q6kLane q6k_lane(const XSlice& x) {
    Q6kLane c;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        c.k[g] = q6k_group_const(x.q[4 * g], x.q[4 * g + 1], x.q[4 * g + 2], x.q[4 * g + 3], x.q2[4 * g],
                                 x.q2[4 * g + 1], x.q2[4 * g + 2], x.q2[4 * g + 3]);
        c.e[g] = x.d[g] * FEIN;
    }
    return c;
}

// Group g's term: the chains from the raw codes and the group constant, joined and scaled.
template <int G>
__device__ __forceinline__ float q6k_group(const u32 (&lo)[4], const u32 (&qh)[4], const u32 (&xa)[4],
                                           const u32 (&xc)[4], int k0, float sc_e, float acc) {
    int a = 0, b = k0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u32 c = q6k_codes<G>(lo[k], qh[k]);
        a = dot4(c, xa[k], a);
        b = dot4(c, xc[k], b);
    }
    return fmaf((float)(__mul24(a, 254) + b), sc_e, acc);
}

__device__ __forceinline__ float q6k_dot1(const Fmt<NMQ_Q6_K>::Raw& r, const XSlice& x, int u, const Q6kLane& c) {
    const u32 la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
    const u32 lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
    const u32 qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    const u32 sh = 8u * (u32)(u & 1);
    float sc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) sc[g] = (float)(int8_t)bfe(g < 2 ? r.sc.x : r.sc.y, sh + 16u * (u32)(g & 1), 8);
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const u32 xa[4] = {x.q[4 * g], x.q[4 * g + 1], x.q[4 * g + 2], x.q[4 * g + 3]};
        const u32 xc[4] = {x.q2[4 * g], x.q2[4 * g + 1], x.q2[4 * g + 2], x.q2[4 * g + 3]};
        const float se = sc[g] * c.e[g];
        acc = g == 0 ? q6k_group<0>(la, qh, xa, xc, c.k[0], se, acc)
            : g == 1 ? q6k_group<1>(lb, qh, xa, xc, c.k[1], se, acc)
            : g == 2 ? q6k_group<2>(la, qh, xa, xc, c.k[2], se, acc) : q6k_group<3>(lb, qh, xa, xc, c.k[3], se, acc);
    }
    return acc * h2f(r.d);
}

// Q8_0, 34-byte blocks (quant.py:46-50, cudakern.py:307-313): unit u = blocks 2u and 2u+1 (68
// bytes).  The second block is absent when the row has an odd number of blocks and u is the last.
template <>
struct Fmt<NMQ_Q8_0> {
    static constexpr int BV = 32, BB = 34;
    static constexpr bool STRIDED = false, HAS_MIN = false;
    struct Raw {
        u32 v[17];
    };
    __device__ static void load(const u8* row, int u, int nblk, Raw& r) {
        const u8* p = row + 68 * u;
        const u32x4 a = ld4(p), b = ld4(p + 16);
        r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
        r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
        // Block 1 is past the row end when the row has an odd number of blocks and u is its last
        // unit: then block 0 is read a second time (a valid address, no branch around the loads)
        // and the words are cleared.
        const bool two = 2 * u + 1 < nblk;
        const u8* p1 = two ? p + 32 : p;
        const u32 v8 = ld1(p1), lo16 = ld16(p + 32);
        const u32x4 c = ld4(p1 + 4), e = ld4(p1 + 20);
        r.v[8] = two ? v8 : lo16;  // qs[30], qs[31] of block 0 (and d of block 1)
        r.v[9] = two ? c.x : 0u; r.v[10] = two ? c.y : 0u; r.v[11] = two ? c.z : 0u; r.v[12] = two ? c.w : 0u;
        r.v[13] = two ? e.x : 0u; r.v[14] = two ? e.y : 0u; r.v[15] = two ? e.z : 0u; r.v[16] = two ? e.w : 0u;
    }
    __device__ static void decode(const Raw& r, int /*u*/, const u64* /*tab*/, WUnit& o) {
#pragma unroll
        for (int k = 0; k < 8; ++k) o.w[k] = __builtin_amdgcn_alignbyte(r.v[k + 1], r.v[k], 2);
#pragma unroll
        for (int k = 0; k < 8; ++k) o.w[8 + k] = r.v[9 + k];
        o.ws[0] = o.ws[1] = h2f(r.v[0]);
        o.ws[2] = o.ws[3] = h2f(r.v[8] >> 16);
        o.wm[0] = o.wm[1] = 0.f;
    }
};

// Q4_0, 18-byte blocks (quant.py:60-64, cudakern.py:315-321): fp16 d, then qs[16] whose low
// nibbles are values 0..15 and high nibbles values 16..31; value = d * (nibble - 8).  Unit u = blocks
// 2u and 2u+1 (36 bytes); the second is absent when the row has an odd number of blocks and u is the
// last (then block 0 is read again, its copy's weights set to 0 and its factor to 0).
template <>
struct Fmt<NMQ_Q4_0> {
    static constexpr int BV = 32, BB = 18;
    static constexpr bool STRIDED = false, HAS_MIN = false;
    struct Raw {
        u32x4 q0, q1;
        u32 d0, d1;
    };
    __device__ static void load(const u8* row, int u, int nblk, Raw& r) {
        const u8* p = row + 36 * u;
        const bool two = 2 * u + 1 < nblk;
        const u8* p1 = two ? p + 18 : p;
        r.q0 = ld4(p + 2);
        r.d0 = ld16(p);
        const u32x4 c = ld4(p1 + 2);
        const u32 d1 = ld16(p1);
        r.q1 = two ? c : u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};  // nibbles 8: weight 0
        r.d1 = two ? d1 : 0u;
    }
    __device__ static void decode(const Raw& r, int /*u*/, const u64* /*tab*/, WUnit& o) {
        const u32 a[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
        const u32 b[4] = {r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o.w[k] = sub8x4(a[k] & 0x0f0f0f0fu);
            o.w[4 + k] = sub8x4((a[k] >> 4) & 0x0f0f0f0fu);
            o.w[8 + k] = sub8x4(b[k] & 0x0f0f0f0fu);
            o.w[12 + k] = sub8x4((b[k] >> 4) & 0x0f0f0f0fu);
        }
        o.ws[0] = o.ws[1] = h2f(r.d0);
        o.ws[2] = o.ws[3] = h2f(r.d1);
        o.wm[0] = o.wm[1] = 0.f;
    }
};

// TQ2_0, 66-byte blocks (quant.py:417-421, cudakern.py:432-439): unit u = 4b + 2n + j takes qs
// bytes 32n + 16j .. +15; run l holds the 2-bit codes at shift 2l (values 128n + 32l + 16j + m).
template <>
struct Fmt<NMQ_TQ2_0> {
    static constexpr int BV = 256, BB = 66;
    static constexpr bool STRIDED = true, HAS_MIN = false;
    struct Raw {
        u32x4 q;
        u32 d;
    };
    __device__ static void load(const u8* row, int u, int /*row_units*/, Raw& r) {
        const u8* blk = row + (u >> 2) * BB;
        r.q = ld4(blk + 16 * (u & 3));
        r.d = ld16(blk + 64);
    }
    __device__ static void decode(const Raw& r, int /*u*/, const u64* /*tab*/, WUnit& o) {
        const u32 q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int l = 0; l < 4; ++l)
#pragma unroll
            for (int k = 0; k < 4; ++k) o.w[4 * l + k] = sub1x4((q[k] >> (2 * l)) & 0x03030303u);
        const float d = h2f(r.d);
        o.ws[0] = o.ws[1] = o.ws[2] = o.ws[3] = d;
        o.wm[0] = o.wm[1] = 0.f;
    }
};

// IQ2_XXS, 66-byte blocks (quant.py:235-245, cudakern.py:187-195): unit u = sub-blocks 2i, 2i+1
// (i = u % 4) of block u / 4; each sub-block is {u32 aux0: 4 grid indices, u32 aux1: 4 x 7 sign
// bits + 4-bit scale ls}.  tab[0..255] = grid (LDS), tab[256..383] = byte masks of the 128 sign
// patterns with the parity bit as bit 7.
template <>
struct Fmt<NMQ_IQ2_XXS> {
    static constexpr int BV = 256, BB = 66;
    static constexpr bool STRIDED = false, HAS_MIN = false;
    struct Raw {
        u32x4 q;
        u32 d;
    };
    __device__ static void load(const u8* row, int u, int /*row_units*/, Raw& r) {
        const u8* blk = row + (u >> 2) * BB;
        r.q = ld4(blk + 2 + 16 * (u & 3));
        r.d = ld16(blk);
    }
    __device__ static void decode(const Raw& r, int /*u*/, const u64* tab, WUnit& o) {
        const float d = h2f(r.d);
        const u32 aux0[2] = {r.q.x, r.q.z}, aux1[2] = {r.q.y, r.q.w};
#pragma unroll
        for (int z = 0; z < 2; ++z) {
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const u64 g = tab[bfe(aux0[z], 8 * l, 8)];
                const u64 m = tab[256 + bfe(aux1[z], 7 * l, 7)];
                const u32 glo = (u32)g, ghi = (u32)(g >> 32), mlo = (u32)m, mhi = (u32)(m >> 32);
                o.w[8 * z + 2 * l] = (glo ^ mlo) + (mlo & 0x01010101u);
                o.w[8 * z + 2 * l + 1] = (ghi ^ mhi) + (mhi & 0x01010101u);
            }
            const float db = d * (0.125f + 0.25f * (float)(aux1[z] >> 28));
            o.ws[2 * z] = o.ws[2 * z + 1] = db;
        }
        o.wm[0] = o.wm[1] = 0.f;
    }
};

// IQ2_XXS tables for LDS: the grid and the 128 sign masks (bit j of the 8-bit sign pattern ->
// byte j = 0xff).  Filled by the first threads of a workgroup.
__device__ const u64 IQ2XXS_GRID[256] = {
#include "iq2xxs_grid.inc"
};

__device__ __forceinline__ u64 iq2_sign_mask(u32 s7) {
    const u32 s = s7 | ((u32)(__builtin_popcount(s7) & 1) << 7);
    u64 m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if ((s >> j) & 1u) m |= (u64)0xff << (8 * j);
    return m;
}

}  // namespace nmq
