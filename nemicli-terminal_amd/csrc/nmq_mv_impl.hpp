// The general mat-vec kernel of every format: y[m][c][r] = W_m[r,:] . x_c for NC tokens.
//
// Work split (wave64 on gfx950):
//   - a workgroup of W waves (W = 1, 2 or 4) owns `groups` consecutive row groups of W*P*RW rows;
//   - inside a wave, P = 64/T teams of T lanes each take RW rows; the T lanes of a team stride over
//     the row's 64-value units (T = 64 for long rows, 32 or 16 for short ones so that few lanes
//     idle), then add their partial sums with xor shuffles;
//   - the two-stage input of all NC tokens is staged once per workgroup into LDS (per tile of KT
//     values; one tile unless the row is too long for the LDS budget), in 16-byte chunks permuted
//     with an XOR pattern so that the lanes' 16-byte reads of their slices hit distinct banks;
//   - each unit of weights is read once from HBM (global_load_dwordx4) and decoded once for all NC
//     tokens; the int8 products use v_dot4_i32_i8, fp32 only for the per-16/32-value combine.
// Expert gather: blockIdx.y = instance m; its weights start at w + ids[m]*per_expert (or at the
// address table entry ids[m] when per_expert < 0) and it reads the input row m / x_group.
#pragma once

#include <stdlib.h>

#include "nmq_device.hpp"
#include "nmq_tune.hpp"

namespace nmq {

struct MvParams {
    const u8* w;
    const int64_t* ids;  // nullptr: one matrix
    int64_t per_expert;  // bytes between experts; < 0: w is a table of int64 addresses
    int64_t row_bytes;
    const int8_t* xq;
    const int8_t* xq2;
    const float* xd;
    const float* xs;
    float* y;
    int n_out, n_in;
    int x_group;   // instance m reads input rows from (m / x_group)
    int kt;        // values per tile (multiple of 64; 256 for 256-value blocks)
    int ktp;       // kt rounded up to 128 (bytes of one xq region in LDS)
    int n_tiles;
    int groups;    // row groups per workgroup
    int nblk;      // blocks per row
    int nt;        // threads per workgroup, set by the launcher (the built-in block size is read from the
                   // launch's hidden arguments by a dependent scalar and vector load at kernel entry)
    const u8* w2;  // experts: a second expert tensor (same format and shape) for instances n_ids.. 2 n_ids-1
    int n_ids;     // experts: entries of ids (instances per expert tensor)
    // One token over up to four matrices of one format and row length whose rows are concatenated
    // (segments): rows [seg_end[i-1], seg_end[i]) belong to matrix i (seg_end[-1] = 0; entries past
    // the last matrix are INT_MAX), read from seg_w[i] and written to seg_y[i].  n_seg = 0: one matrix.
    int n_seg;
    int seg_end[3];
    const u8* seg_w[4];
    float* seg_y[4];
    // One-token kernels: the input given as values (row m / x_group of n_in values each) instead of
    // xq, xq2, xd, xs; the staging forms the two-stage input from them (x_mode: NMQ_X_*, xv2 the second
    // operand of NMQ_X_SILU_MUL_BF16).  xv = nullptr: the two-stage arrays.
    const void* xv;
    const void* xv2;
    int x_mode;
};

// Weights and input row of instance m (blockIdx.y).  One matrix: w, input row 0.  Experts: instance m
// reads expert ids[m'] of tensor w (m' = m) or, with a second tensor, of w2 (m' = m - n_ids for
// m >= n_ids), at ids[m'] * per_expert bytes or at the address table entry ids[m']; its input row is
// m' / x_group.
// The expert id and the table entry are moved into scalar registers (readfirstlane: they are uniform
// per workgroup): left in vector registers, the weight addresses of every kernel would depend on a
// vector load on one path, and where the paths meet the compiler would wait for every outstanding
// read of the wave (the input reads issued ahead of the weight reads included) before any weight read.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const u32 lo = __builtin_amdgcn_readfirstlane((u32)v);
    const u32 hi = __builtin_amdgcn_readfirstlane((u32)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ const u8* instance_weights(const MvParams& p, int m, int64_t& xrow) {
    if (!p.ids) {
        xrow = 0;
        return p.w;
    }
    const bool second = p.w2 != nullptr && m >= p.n_ids;
    const int mm = second ? m - p.n_ids : m;
    const int64_t e = uniform64(gp<int64_t>(p.ids)[mm]);
    xrow = mm / p.x_group;
    const u8* base = second ? p.w2 : p.w;
    return p.per_expert >= 0 ? base + e * p.per_expert : (const u8*)uniform64(gp<int64_t>(base)[e]);
}

// Row addressing of the one-token kernels: one matrix (rows back to back from w, outputs from y) or
// segments.  Copied out of the kernel arguments at entry: the helpers below take it by reference, and
// a reference to the argument block itself would make the compiler copy the whole block to scratch.
struct RowMap {
    const u8* w[4];
    float* y[4];
    int64_t row_bytes;
    int n_out, nblk, n_seg;
    int end[3];
    __device__ __forceinline__ int seg(int r) const { return (r >= end[0]) + (r >= end[1]) + (r >= end[2]); }
    __device__ __forceinline__ int start(int i) const {
        return i == 0 ? 0 : (i == 1 ? end[0] : (i == 2 ? end[1] : end[2]));
    }
    __device__ __forceinline__ const u8* row(int r) const {
        if (n_seg == 0) return w[0] + (int64_t)r * row_bytes;
        const int i = seg(r);
        const u8* b = i == 0 ? w[0] : (i == 1 ? w[1] : (i == 2 ? w[2] : w[3]));
        return b + (int64_t)(r - start(i)) * row_bytes;
    }
    __device__ __forceinline__ float* out(int r) const {
        if (n_seg == 0) return y[0] + r;
        const int i = seg(r);
        float* o = i == 0 ? y[0] : (i == 1 ? y[1] : (i == 2 ? y[2] : y[3]));
        return o + (r - start(i));
    }
};

// EXT = false: the kernel variant without segments (the compiler drops their addressing).
template <bool EXT>
__device__ __forceinline__ RowMap row_map(const MvParams& p, const u8* wbase, float* y) {
    RowMap m;
    m.row_bytes = p.row_bytes;
    m.n_out = p.n_out;
    m.nblk = p.nblk;
    m.n_seg = EXT ? p.n_seg : 0;
    if (m.n_seg == 0) {
        m.w[0] = m.w[1] = m.w[2] = m.w[3] = wbase;
        m.y[0] = m.y[1] = m.y[2] = m.y[3] = y;
        m.end[0] = m.end[1] = m.end[2] = 0x7fffffff;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m.w[i] = p.seg_w[i];
            m.y[i] = p.seg_y[i];
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) m.end[i] = p.seg_end[i];
    }
    return m;
}

// Every kernel argument (and the launch shape) into the first batch of scalar loads at kernel entry:
// left alone, the compiler fetches some of them behind branches, one dependent round trip each.
// The asm statement is empty; it only makes the values live in scalar registers at that point.
template <bool EXT = false>
__device__ __forceinline__ void args_early(const MvParams& p) {
    asm volatile("" ::"s"(p.w), "s"(p.ids), "s"(p.per_expert), "s"(p.row_bytes), "s"(p.xq), "s"(p.xq2),
                 "s"(p.xd), "s"(p.xs), "s"(p.y), "s"(p.n_out), "s"(p.n_in), "s"(p.x_group), "s"(p.kt),
                 "s"(p.ktp), "s"(p.n_tiles), "s"(p.groups), "s"(p.nblk), "s"(p.nt), "s"(p.w2), "s"(p.n_ids),
                 "s"(gridDim.x));
    if constexpr (EXT) asm volatile("" ::"s"(p.n_seg), "s"(p.xv), "s"(p.xv2), "s"(p.x_mode));
}

// 16-byte chunk permutations of the LDS input (bijective inside every aligned group of 8 chunks).
template <bool STRIDED>
__device__ __forceinline__ int swz(int ch) {
    return STRIDED ? (ch ^ (((ch >> 3) & 3) << 1)) : (ch ^ ((ch >> 3) & 7));
}

template <bool STRIDED>
__device__ __forceinline__ void stage_tile(u8* lds, const int8_t* xq, const int8_t* xq2, const float* xd,
                                           const float* xs, int n_in, int nc, int k0, int kt, int ktp, int nt) {
    const int tid = threadIdx.x;
    const int tok = (ktp * 9) / 4;
    for (int c = 0; c < nc; ++c) {
        u8* base = lds + c * tok;
        const int8_t* q = xq + (int64_t)c * n_in + k0;
        const int8_t* q2 = xq2 + (int64_t)c * n_in + k0;
        for (int ch = tid; ch < ktp / 16; ch += nt) {
            u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
            if (ch * 16 < kt) {
                a = *gp<u32x4>(q + 16 * ch);
                b = *gp<u32x4>(q2 + 16 * ch);
            }
            const int ph = swz<STRIDED>(ch);
            *(u32x4*)(base + 16 * ph) = a;
            *(u32x4*)(base + ktp + 16 * ph) = b;
        }
        float* d = (float*)(base + 2 * ktp);
        float* s = d + ktp / 32;
        const int64_t g0 = ((int64_t)c * n_in + k0) / 32;
        for (int i = tid; i < ktp / 32; i += nt) {
            const bool ok = i < kt / 32;
            d[i] = ok ? gp<float>(xd)[g0 + i] : 0.f;
            s[i] = ok ? gp<float>(xs)[g0 + i] : 0.f;
        }
    }
}

template <bool STRIDED>
__device__ __forceinline__ void read_slice(const u8* base, int ktp, int u, XSlice& x) {
    const u8* q = base;
    const u8* q2 = base + ktp;
    const float* d = (const float*)(base + 2 * ktp);
    const float* s = d + ktp / 32;
    if (!STRIDED) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int ph = swz<false>(4 * u + k);
            const u32x4 a = *(const u32x4*)(q + 16 * ph);
            const u32x4 b = *(const u32x4*)(q2 + 16 * ph);
            x.q[4 * k] = a.x; x.q[4 * k + 1] = a.y; x.q[4 * k + 2] = a.z; x.q[4 * k + 3] = a.w;
            x.q2[4 * k] = b.x; x.q2[4 * k + 1] = b.y; x.q2[4 * k + 2] = b.z; x.q2[4 * k + 3] = b.w;
        }
        const float2 dd = *(const float2*)(d + 2 * u);
        const float2 ss = *(const float2*)(s + 2 * u);
        x.d[0] = dd.x; x.d[1] = dd.y; x.d[2] = 0.f; x.d[3] = 0.f;
        x.s[0] = ss.x; x.s[1] = ss.y;
    } else {
        const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int ph = swz<true>(16 * b + 8 * h + 2 * k + j);
            const u32x4 a = *(const u32x4*)(q + 16 * ph);
            const u32x4 c = *(const u32x4*)(q2 + 16 * ph);
            x.q[4 * k] = a.x; x.q[4 * k + 1] = a.y; x.q[4 * k + 2] = a.z; x.q[4 * k + 3] = a.w;
            x.q2[4 * k] = c.x; x.q2[4 * k + 1] = c.y; x.q2[4 * k + 2] = c.z; x.q2[4 * k + 3] = c.w;
        }
        const float4 dd = *(const float4*)(d + 8 * b + 4 * h);
        x.d[0] = dd.x; x.d[1] = dd.y; x.d[2] = dd.z; x.d[3] = dd.w;
        x.s[0] = x.s[1] = 0.f;
    }
}

// Reads issued by hand (inline assembly): the compiler's wait insertion does not see them, so its own
// waits can only wait longer than needed, and the code that issues them places its own waits
// (vm_wait<N>: until at most N reads of the wave are outstanding, the registers tied to the wait so
// that nothing reads them before).  Used where the compiler would otherwise wait for every read of
// the wave (buffers rotating through a loop, staging stores ahead of weight reads).
__device__ __forceinline__ u32x4 gload16(const void* ptr) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr));
    return v;
}
__device__ __forceinline__ u32x2 gload8(const void* ptr) {
    u32x2 v;
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(v) : "v"(ptr));
    return v;
}
__device__ __forceinline__ float gload4f(const void* ptr) {
    float v;
    asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(ptr));
    return v;
}

// One token, whole row, in rounds of one 16-byte chunk of xq and of xq2 and one (xd, xs) pair per
// thread.  Every read of a round is issued (threads past the row re-read its start), so a kernel can
// issue round 0 before its weight reads and wait for it alone; the stores apply stage_tile's layout.
struct XRound {
    u32x4 a, b;
    float d, s;
};

__device__ __forceinline__ void stage1_load(XRound& r, int rnd, const int8_t* xq, const int8_t* xq2, const float* xd,
                                            const float* xs, int n_in, int nt) {
    const int i = rnd * nt + (int)threadIdx.x;
    const int ch = 16 * i < n_in ? i : 0;
    r.a = *gp<u32x4>(xq + 16 * ch);
    r.b = *gp<u32x4>(xq2 + 16 * ch);
    const int g = i < n_in / 32 ? i : 0;
    r.d = gp<float>(xd)[g];
    r.s = gp<float>(xs)[g];
}

// stage1_load with the reads issued by hand; xround_wait<N>() waits for them with N later reads out.
__device__ __forceinline__ void stage1_load_hand(XRound& r, int rnd, const int8_t* xq, const int8_t* xq2,
                                                 const float* xd, const float* xs, int n_in, int nt) {
    const int i = rnd * nt + (int)threadIdx.x;
    const int ch = 16 * i < n_in ? i : 0;
    r.a = gload16(xq + 16 * ch);
    r.b = gload16(xq2 + 16 * ch);
    const int g = i < n_in / 32 ? i : 0;
    r.d = gload4f(xd + g);
    r.s = gload4f(xs + g);
}

template <int N>
__device__ __forceinline__ void xround_wait(XRound& r) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(r.a), "+v"(r.b), "+v"(r.d), "+v"(r.s) : "n"(N));
}

template <bool STRIDED>
__device__ __forceinline__ void stage1_store(const XRound& r, int rnd, u8* lds, int n_in, int ktp, int nt) {
    const int i = rnd * nt + (int)threadIdx.x;
    if (i < ktp / 16) {
        const bool ok = 16 * i < n_in;
        const int ph = swz<STRIDED>(i);
        *(u32x4*)(lds + 16 * ph) = ok ? r.a : u32x4{0u, 0u, 0u, 0u};
        *(u32x4*)(lds + ktp + 16 * ph) = ok ? r.b : u32x4{0u, 0u, 0u, 0u};
    }
    if (i < ktp / 32) {
        const bool ok = i < n_in / 32;
        float* d = (float*)(lds + 2 * ktp);
        d[i] = ok ? r.d : 0.f;
        d[ktp / 32 + i] = ok ? r.s : 0.f;
    }
}

// IQ2_XXS tables in LDS (grid[256], then sign masks[128]), split like the input staging: tab_load()
// reads this thread's grid entry (always a valid address), tab_store() writes the tables.
template <int F>
__device__ __forceinline__ u64 tab_load() {
    return F == NMQ_IQ2_XXS ? IQ2XXS_GRID[min((int)threadIdx.x, 255)] : 0ull;
}

template <int F>
__device__ __forceinline__ void tab_store(u64* tab, u64 gv, int nt) {
    if (F != NMQ_IQ2_XXS) return;
    if (nt >= 256) {
        if (threadIdx.x < 256) tab[threadIdx.x] = gv;
    } else {
        for (int i = threadIdx.x; i < 256; i += nt) tab[i] = IQ2XXS_GRID[i];
    }
    for (int i = threadIdx.x; i < 128; i += nt) tab[256 + i] = iq2_sign_mask((u32)i);
}

// ---- input staging from values ---------------------------------------------------------------
// A workgroup forms the token's two-stage input itself, with the arithmetic of quant_q8_kernel (the
// same results bit for bit), straight into stage1_store's LDS layout.  Four values per lane: a
// 32-value group spans 8 aligned lanes.  For value j = 4l + e of a group, the partners of the
// butterfly levels j ^ 16, ^ 8, ^ 4, ^ 2, ^ 1 are element e of lanes l ^ 4, ^ 2, ^ 1 and then elements
// e ^ 2, e ^ 1 of the lane itself, so max and sum make the additions of the 32-lane butterfly.
struct VRound {
    float v[4];
    float u[4];  // second operand (NMQ_X_SILU_MUL_BF16)
};

__device__ __forceinline__ void stagev_load(VRound& r, int rnd, const void* x, const void* x2, int mode, int n_in,
                                            int nt) {
    const int j = rnd * nt + (int)threadIdx.x;  // values 4j .. 4j + 3
    const int o = 4 * j < n_in ? 4 * j : 0;     // past the row: re-read its start (discarded)
    if (mode == NMQ_X_BF16) {
        const u32x2 b = *gp<u32x2>((const u16*)x + o);
        r.v[0] = __uint_as_float(b.x << 16);
        r.v[1] = __uint_as_float(b.x & 0xffff0000u);
        r.v[2] = __uint_as_float(b.y << 16);
        r.v[3] = __uint_as_float(b.y & 0xffff0000u);
    } else {
        const u32x4 a = *gp<u32x4>((const float*)x + o);
        r.v[0] = __uint_as_float(a.x); r.v[1] = __uint_as_float(a.y);
        r.v[2] = __uint_as_float(a.z); r.v[3] = __uint_as_float(a.w);
    }
    if (mode == NMQ_X_SILU_MUL_BF16) {
        const u32x4 c = *gp<u32x4>((const float*)x2 + o);
        r.u[0] = __uint_as_float(c.x); r.u[1] = __uint_as_float(c.y);
        r.u[2] = __uint_as_float(c.z); r.u[3] = __uint_as_float(c.w);
    }
}

// The two stages of a lane's four values v in a group of scale d (0: an all-zero group):
// q = rint(v / d), q2 = rint((v - q d) / (d FEIN)) clamped to +-127, every quotient the IEEE one.  For
// d >= 2^-100 the product t = v * rcp(d) (v_rcp_f32: 1 ulp) lies within 128 * 1.5 * 2^-23 of the exact
// quotient and the IEEE quotient within 128 * 2^-24, so where t is more than 2^-14 from the half-integer
// between its neighbours both round to the same integer (the test below may see the unrounded product;
// the difference, half an ulp of t, is inside the slack).  Only a wave with a lane next to such a
// half-integer, or with a scale below 2^-100, divides (one scalar branch per stage).
__device__ __forceinline__ void quant4(const float (&v)[4], float d, int (&q)[4], int (&q2)[4]) {
    const bool small = d > 0.0f && !(d >= 0x1p-100f);
    const float rd = __builtin_amdgcn_rcpf(d);
    float t[4];
    bool near = small;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        t[e] = v[e] * rd;
        near |= fabsf(t[e] - floorf(t[e]) - 0.5f) <= 0x1p-14f;
    }
    if (__builtin_amdgcn_ballot_w64(near) != 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = v[e] / d;
    }
    const float b = d * FEIN, rb = __builtin_amdgcn_rcpf(b);
    float r[4], t2[4];
    bool near2 = small;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        q[e] = d > 0.0f ? (int)rintf(t[e]) : 0;
        r[e] = fmaf(-(float)q[e], d, v[e]);
        t2[e] = r[e] * rb;
        near2 |= fabsf(t2[e] - floorf(t2[e]) - 0.5f) <= 0x1p-14f;
    }
    if (__builtin_amdgcn_ballot_w64(near2) != 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) t2[e] = r[e] / b;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int k = (int)rintf(t2[e]);
        q2[e] = d > 0.0f ? (k < -127 ? -127 : (k > 127 ? 127 : k)) : 0;
    }
}

template <bool STRIDED>
__device__ __forceinline__ void stagev_store(const VRound& r, int rnd, u8* lds, int mode, int n_in, int ktp, int nt) {
    const int j = rnd * nt + (int)threadIdx.x;
    const int idx = 4 * j;
    if (idx >= ktp) return;  // whole groups of 8 lanes (ktp % 32 == 0)
    const bool in = idx < n_in;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float t = r.v[e];
        if (mode == NMQ_X_F32_BF16) t = round_bf16(t);
        else if (mode == NMQ_X_SILU_MUL_BF16) t = silu_mul_bf16(t, r.u[e]);
        v[e] = in ? t : 0.f;
    }
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = fmaxf(m, swz_xor4(m));
    m = fmaxf(m, dpp_f<0x4E>(m));  // quad_perm 2,3,0,1: lane ^ 2
    m = fmaxf(m, dpp_f<0xB1>(m));  // quad_perm 1,0,3,2: lane ^ 1
    const float d = m / 127.0f;
    int q[4], q2[4];
    quant4(v, d, q, q2);
    u32 pq = 0u, pq2 = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        pq |= ((u32)q[e] & 0xffu) << (8 * e);
        pq2 |= ((u32)q2[e] & 0xffu) << (8 * e);
    }
    float a[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = v[e] + swz_xor4(v[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = a[e] + dpp_f<0x4E>(a[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = a[e] + dpp_f<0xB1>(a[e]);
    const float sum = (a[0] + a[2]) + (a[1] + a[3]);
    u8* qb = lds + 16 * swz<STRIDED>(idx >> 4) + (idx & 15);
    *(u32*)qb = pq;
    *(u32*)(qb + ktp) = pq2;
    if ((threadIdx.x & 7) == 0) {
        float* dd = (float*)(lds + 2 * ktp);
        dd[idx >> 5] = d;
        dd[ktp / 32 + (idx >> 5)] = sum;
    }
}

// Input staging of the one-token kernels around their first weight reads.  One round (the input fits
// one chunk per thread): its reads and the table entry go out first, the weight reads (issue()) next,
// and the stores wait only for the older input reads.  Several rounds: everything is staged before
// the weight reads, so that no input read can still be pending where the two paths meet (a pending
// read there makes the compiler wait for every outstanding read, the weights included).
// MAXR: rounds of the two-stage input a thread may hold in registers while the weight reads go out
// (longer inputs are staged completely before them).
template <int F, bool EXT, int MAXR, typename Issue>
__device__ __forceinline__ void stage1_around(u8* lds, u64* tab, const MvParams& p, int64_t xrow, Issue issue) {
    using FM = Fmt<F>;
    const int nt = p.nt;
    if (EXT && p.xv) {
        const int esz = p.x_mode == NMQ_X_BF16 ? 2 : 4;
        const void* xv = (const u8*)p.xv + xrow * p.n_in * esz;
        const void* xv2 = p.xv2 ? (const u8*)p.xv2 + xrow * p.n_in * 4 : p.xv;
        const int rounds = (p.ktp / 4 + nt - 1) / nt;
        if (rounds <= 2) {  // the value reads first, the weight reads next, then the quantisation
            // Both rounds unconditionally (reads past the row are clamped to its start, stores past it
            // skipped): with a branch per round the compiler waits for each round's reads before the next.
            VRound r[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) stagev_load(r[k], k, xv, xv2, p.x_mode, p.n_in, nt);
            const u64 gv = tab_load<F>();
            __builtin_amdgcn_sched_barrier(0);
            issue();
            __builtin_amdgcn_sched_barrier(0);
            tab_store<F>(tab, gv, nt);
#pragma unroll
            for (int k = 0; k < 2; ++k) stagev_store<FM::STRIDED>(r[k], k, lds, p.x_mode, p.n_in, p.ktp, nt);
        } else {
            for (int k = 0; k < rounds; ++k) {
                VRound r;
                stagev_load(r, k, xv, xv2, p.x_mode, p.n_in, nt);
                stagev_store<FM::STRIDED>(r, k, lds, p.x_mode, p.n_in, p.ktp, nt);
            }
            tab_store<F>(tab, tab_load<F>(), nt);
            __builtin_amdgcn_sched_barrier(0);
            issue();
        }
        lds_barrier();
        return;
    }
    const int8_t* xq = p.xq + xrow * p.n_in;
    const int8_t* xq2 = p.xq2 + xrow * p.n_in;
    const float* xd = p.xd + xrow * (p.n_in / 32);
    const float* xs = p.xs + xrow * (p.n_in / 32);
    const int rounds = (p.ktp / 16 + nt - 1) / nt;
    if (rounds <= MAXR) {
        // All MAXR rounds unconditionally (reads past the row are clamped to its start, stores past it
        // skipped): with a branch per round the compiler waits for each round's reads before the next.
        XRound r[MAXR];
#pragma unroll
        for (int k = 0; k < MAXR; ++k) stage1_load(r[k], k, xq, xq2, xd, xs, p.n_in, nt);
        const u64 gv = tab_load<F>();
        __builtin_amdgcn_sched_barrier(0);  // keep the input reads ahead of the weight reads
        issue();
        __builtin_amdgcn_sched_barrier(0);
        tab_store<F>(tab, gv, nt);
#pragma unroll
        for (int k = 0; k < MAXR; ++k) stage1_store<FM::STRIDED>(r[k], k, lds, p.n_in, p.ktp, nt);
    } else {
        for (int k = 0; k < rounds; ++k) {
            XRound r;
            stage1_load(r, k, xq, xq2, xd, xs, p.n_in, nt);
            stage1_store<FM::STRIDED>(r, k, lds, p.n_in, p.ktp, nt);
        }
        tab_store<F>(tab, tab_load<F>(), nt);
        __builtin_amdgcn_sched_barrier(0);
        issue();
    }
    lds_barrier();
}

// Input staging around hand-issued weight reads (Q4kStepAsm): two-stage input, one round (the row fits
// one 16-byte chunk per thread; the launcher checks), straight-line code.  The input reads are issued
// by hand before issue()'s HW weight reads and waited for with exactly those left outstanding.  No
// branch may join between a hand-issued read and its wait: where paths join, the compiler may copy a
// register whose read is still outstanding (it takes the value as present once the instruction issued).
// The same for fp32 values (NMQ_X_F32, NMQ_X_F32_BF16: both read 16 bytes per lane and round), at most
// two rounds of four values per thread (the launcher checks); the quantisation follows the wait.
// IQ2_XXS: the thread's grid entry is read by hand with the input and stored after the same wait
// (the launcher gives such launches at least 256 threads).
template <int F>
__device__ __forceinline__ u32x2 tab_load_hand() {
    if constexpr (F == NMQ_IQ2_XXS) return gload8(&IQ2XXS_GRID[min((int)threadIdx.x, 255)]);
    else return u32x2{0u, 0u};
}

template <int F>
__device__ __forceinline__ void tab_store_hand(u64* tab, u32x2 gv, int nt) {
    if constexpr (F == NMQ_IQ2_XXS) {
        if (threadIdx.x < 256) tab[threadIdx.x] = (u64)gv.x | ((u64)gv.y << 32);
        for (int i = threadIdx.x; i < 128; i += nt) tab[256 + i] = iq2_sign_mask((u32)i);
    }
}

template <int F, int HW, typename Issue>
__device__ __forceinline__ void stagev_hand(u8* lds, u64* tab, const MvParams& p, int64_t xrow, Issue issue) {
    using FM = Fmt<F>;
    const float* xv = (const float*)p.xv + xrow * p.n_in;
    const int nt = p.nt;
    const int j0 = (int)threadIdx.x, j1 = nt + (int)threadIdx.x;
    u32x4 a0 = gload16(xv + (4 * j0 < p.n_in ? 4 * j0 : 0));  // past the row: its start (discarded)
    u32x4 a1 = gload16(xv + (4 * j1 < p.n_in ? 4 * j1 : 0));
    u32x2 gv = tab_load_hand<F>();
    __builtin_amdgcn_sched_barrier(0);
    issue();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%3)" : "+v"(a0), "+v"(a1), "+v"(gv) : "n"(HW));
    tab_store_hand<F>(tab, gv, nt);
    VRound r0, r1;
    r0.v[0] = __uint_as_float(a0.x); r0.v[1] = __uint_as_float(a0.y);
    r0.v[2] = __uint_as_float(a0.z); r0.v[3] = __uint_as_float(a0.w);
    r1.v[0] = __uint_as_float(a1.x); r1.v[1] = __uint_as_float(a1.y);
    r1.v[2] = __uint_as_float(a1.z); r1.v[3] = __uint_as_float(a1.w);
    stagev_store<FM::STRIDED>(r0, 0, lds, p.x_mode, p.n_in, p.ktp, nt);
    stagev_store<FM::STRIDED>(r1, 1, lds, p.x_mode, p.n_in, p.ktp, nt);
    lds_barrier();
}

template <int F, int HW, typename Issue>
__device__ __forceinline__ void stage1_hand(u8* lds, u64* tab, const MvParams& p, int64_t xrow, Issue issue) {
    using FM = Fmt<F>;
    XRound r;
    stage1_load_hand(r, 0, p.xq + xrow * p.n_in, p.xq2 + xrow * p.n_in, p.xd + xrow * (p.n_in / 32),
                     p.xs + xrow * (p.n_in / 32), p.n_in, p.nt);
    u32x2 gv = tab_load_hand<F>();
    __builtin_amdgcn_sched_barrier(0);
    issue();
    __builtin_amdgcn_sched_barrier(0);
    xround_wait<HW>(r);
    asm volatile("" : "+v"(gv));
    tab_store_hand<F>(tab, gv, p.nt);
    stage1_store<FM::STRIDED>(r, 0, lds, p.n_in, p.ktp, p.nt);
    lds_barrier();
}

template <int F>
__device__ __forceinline__ void fill_tables(u64* tab, int nt) {
    if (F == NMQ_IQ2_XXS) {
        for (int i = threadIdx.x; i < 384; i += nt)
            tab[i] = i < 256 ? IQ2XXS_GRID[i] : iq2_sign_mask((u32)(i - 256));
    }
}

template <int F, int NC, int T, int RW>
__global__ __launch_bounds__(256) void mv_kernel(MvParams p) {
    args_early(p);
    using FM = Fmt<F>;
    constexpr bool S = FM::STRIDED;
    constexpr int TW = T > 64 ? T / 64 : 1;  // waves per team
    constexpr int P = T < 64 ? 64 / T : 1;   // teams per wave
    constexpr int TL = T < 64 ? T : 64;      // lanes of a team inside one wave
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    __shared__ float red[T > 64 ? 4 * RW * NC : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, W = p.nt >> 6;
    const int team = T >= 64 ? wave / TW : wave * P + lane / T;
    const int lt = T >= 64 ? (wave % TW) * 64 + lane : lane % T;
    const int teams = T >= 64 ? W / TW : W * P;
    const int m = blockIdx.y;

    int64_t xrow;
    const u8* wbase = instance_weights(p, m, xrow);
    const int8_t* xq = p.xq + xrow * p.n_in;
    const int8_t* xq2 = p.xq2 + xrow * p.n_in;
    const float* xd = p.xd + xrow * (p.n_in / 32);
    const float* xs = p.xs + xrow * (p.n_in / 32);
    float* y = p.y + (int64_t)m * NC * p.n_out;

    fill_tables<F>(tab, p.nt);
    const int tok = (p.ktp * 9) / 4;
    const int rows_iter = teams * RW;
    const int row_wg = blockIdx.x * p.groups * rows_iter;

    for (int g = 0; g < p.groups; ++g) {
        const int r0 = row_wg + g * rows_iter + team * RW;
        float acc[RW][NC];
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[rr][c] = 0.f;
        const u8* rowp[RW];
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) rowp[rr] = wbase + (int64_t)min(r0 + rr, p.n_out - 1) * p.row_bytes;

        for (int tile = 0; tile < p.n_tiles; ++tile) {
            const int k0 = tile * p.kt;
            const int kt = min(p.kt, p.n_in - k0);
            const int U = (kt + 63) >> 6;
            const int u0 = k0 >> 6;
            const int nit = (U + T - 1) / T;
            // the first unit's weights of all RW rows are requested before the input is staged
            typename FM::Raw raw[RW];
            if (lt < U) {
#pragma unroll
                for (int rr = 0; rr < RW; ++rr) FM::load(rowp[rr], u0 + lt, p.nblk, raw[rr]);
            }
            if (p.n_tiles > 1 || g == 0) {
                __syncthreads();
                stage_tile<S>(lds, xq, xq2, xd, xs, p.n_in, NC, k0, kt, p.ktp, p.nt);
                __syncthreads();
            }
            for (int it = 0; it < nit; ++it) {
                const int u = lt + it * T;
                if (u < U) {
                    if (it > 0) {
#pragma unroll
                        for (int rr = 0; rr < RW; ++rr) FM::load(rowp[rr], u0 + u, p.nblk, raw[rr]);
                    }
                    WUnit wu[RW];
#pragma unroll
                    for (int rr = 0; rr < RW; ++rr) FM::decode(raw[rr], u0 + u, tab, wu[rr]);
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        XSlice x;
                        read_slice<S>(lds + c * tok, p.ktp, u, x);
#pragma unroll
                        for (int rr = 0; rr < RW; ++rr) acc[rr][c] += unit_dot<S, FM::HAS_MIN>(wu[rr], x);
                    }
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float v = acc[rr][c];
#pragma unroll
                for (int o = TL / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
                acc[rr][c] = v;
            }
        if (T > 64) {
            // teams span TW waves: lane 0 of every wave posts its sums, the team's first wave adds them
            if (lane == 0) {
#pragma unroll
                for (int rr = 0; rr < RW; ++rr)
#pragma unroll
                    for (int c = 0; c < NC; ++c) red[(wave * RW + rr) * NC + c] = acc[rr][c];
            }
            __syncthreads();
            if (wave % TW == 0 && lane < RW * NC) {
                const int rr = lane / NC, c = lane % NC;
                float v = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < TW; ++w2) v += red[((wave + w2) * RW + rr) * NC + c];
                const int row = r0 + rr;
                if (row < p.n_out) gpw<float>(y)[(int64_t)c * p.n_out + row] = v;
            }
            __syncthreads();
        } else if (lt == 0) {
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                const int row = r0 + rr;
                if (row < p.n_out) {
#pragma unroll
                    for (int c = 0; c < NC; ++c) gpw<float>(y)[(int64_t)c * p.n_out + row] = acc[rr][c];
                }
            }
        }
    }
}

// ---- one token: x slice in registers, rows streamed with one step of prefetch ------------------
// For NC = 1 a lane's units of the row (u = lt + it*T) are the same for every row, so its slice of
// the input is read once into registers.  The input is staged once per workgroup in LDS (one copy
// per CU rather than one per wave from L2).  Waves are persistent: wave gw of nw handles row steps
// gw, gw + nw, ... (a step = P teams x RW rows) and requests the next step's weights before it
// computes the current one, so HBM traffic and VALU work overlap.

// Sum over the T lanes of a team (T = 16, 32 or 64): DPP within rows of 16, then xor shuffles.
template <int T>
__device__ __forceinline__ float team_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // xor 1
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // xor 2
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));  // 8-lane mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));  // 16-lane mirror
    // across rows without LDS (gfx950 lane swaps): the two results of permlane16_swap(v, v) hold, in every
    // lane, its own value and that of lane ^ 16 (permlane32_swap: lane ^ 32), so their sum is what
    // v + shfl_xor(v, 16 / 32) gives, bit for bit (a + b = b + a)
    if (T >= 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if (T >= 64) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

// team_sum<64> of N values, level by level so that the N chains interleave (no wait states between a
// DPP add and the one that reads its result); each result equals team_sum<64> of that value bit for bit.
template <int N>
__device__ __forceinline__ void team_sum64_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0xB1, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x4E, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x141, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[i]), 0x140, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

template <int F, int T, int RW, int NITM>
struct Mv1Step {
    using FM = Fmt<F>;
    typename FM::Raw raw[RW][NITM];
    // Rows at or past n_out are replaced by row fb + rr (a row this wave has just read, so the
    // surplus loads of the last steps hit cache lines nearby instead of all waves' one last row).
    __device__ __forceinline__ void load(const RowMap& rm, int r0, int lt, int U, int fb) {
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {
            const int r = r0 + rr < rm.n_out ? r0 + rr : min(fb + rr, rm.n_out - 1);
            const u8* rp = rm.row(r);
#pragma unroll
            for (int it = 0; it < NITM; ++it) FM::load(rp, min(lt + it * T, U - 1), rm.nblk, raw[rr][it]);
        }
    }
};

// One step of Q4_K weight reads of the one-token kernel, issued by hand (gload16): with buffers
// rotating through the loop, the compiler's wait insertion waits for every outstanding read at the
// loop head (all of a wave's prefetched steps); wait<N>() waits for this step with N later reads out.
// With one row per wave (T = 64) the row address is uniform: the reads take it in scalar registers
// and a lane-constant 32-bit offset (global_load with a scalar base), no 64-bit address arithmetic per
// step.
__device__ __forceinline__ u32x4 gload16s(const u8* base, u32 off) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
    return v;
}
__device__ __forceinline__ u32x4 gload16s_16(const u8* base, u32 off) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:16" : "=v"(v) : "v"(off), "s"(base));
    return v;
}

template <int NITM>
struct Q4kStepAsm {
    Fmt<NMQ_Q4_K>::Raw raw[NITM];
    template <int T>
    __device__ __forceinline__ void load(const RowMap& rm, int r, int lt, int U, int fb) {
        const int rs = r < rm.n_out ? r : min(fb, rm.n_out - 1);
        if constexpr (T == 64) {
            const u8* rp = (const u8*)uniform64((int64_t)rm.row(rs));
#pragma unroll
            for (int it = 0; it < NITM; ++it) {
                const int u = min(lt + it * T, U - 1);
                const u32 oh = (u32)((u >> 2) * Fmt<NMQ_Q4_K>::BB), oa = oh + 16u + 32u * (u32)(u & 3);
                raw[it].h = gload16s(rp, oh);
                raw[it].a = gload16s(rp, oa);
                raw[it].b = gload16s_16(rp, oa);
            }
        } else {
            const u8* rp = rm.row(rs);
#pragma unroll
            for (int it = 0; it < NITM; ++it) {
                const int u = min(lt + it * T, U - 1);
                const u8* blk = rp + (u >> 2) * Fmt<NMQ_Q4_K>::BB + 32 * (u & 3);
                raw[it].h = gload16(rp + (u >> 2) * Fmt<NMQ_Q4_K>::BB);
                raw[it].a = gload16(blk + 16);
                raw[it].b = gload16(blk + 32);
            }
        }
    }
    template <int N>
    __device__ __forceinline__ void wait() {
#pragma unroll
        for (int it = 0; it < NITM; ++it) {
            if (it == 0)
                asm volatile("s_waitcnt vmcnt(%3)" : "+v"(raw[it].h), "+v"(raw[it].a), "+v"(raw[it].b) : "n"(N));
            else
                asm volatile("" : "+v"(raw[it].h), "+v"(raw[it].a), "+v"(raw[it].b));
        }
    }
};

__device__ __forceinline__ u32 gload2u(const u8* ptr) {
    u32 v;
    asm volatile("global_load_ushort %0, %1, off" : "=v"(v) : "v"(ptr));
    return v;
}
__device__ __forceinline__ u32 gload2us(const u8* base, u32 off) {
    u32 v;
    asm volatile("global_load_ushort %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
    return v;
}

// The same for the formats whose unit is 16 code bytes and the block's fp16 scale (TQ2_0: codes at
// 16 (u & 3), scale at 64; IQ2_XXS: scale at 0, codes at 2 + 16 (u & 3)): two reads per unit.
template <int F, int NITM>
struct QdStepAsm {
    static_assert(F == NMQ_TQ2_0 || F == NMQ_IQ2_XXS, "16 code bytes + fp16 scale per unit");
    static constexpr int QO = F == NMQ_TQ2_0 ? 0 : 2, DO = F == NMQ_TQ2_0 ? 64 : 0;
    typename Fmt<F>::Raw raw[NITM];
    template <int T>
    __device__ __forceinline__ void load(const RowMap& rm, int r, int lt, int U, int fb) {
        const int rs = r < rm.n_out ? r : min(fb, rm.n_out - 1);
        if constexpr (T == 64) {
            const u8* rp = (const u8*)uniform64((int64_t)rm.row(rs));
#pragma unroll
            for (int it = 0; it < NITM; ++it) {
                const int u = min(lt + it * T, U - 1);
                const u32 ob = (u32)((u >> 2) * Fmt<F>::BB);
                raw[it].q = gload16s(rp, ob + (u32)(QO + 16 * (u & 3)));
                raw[it].d = gload2us(rp, ob + (u32)DO);
            }
        } else {
            const u8* rp = rm.row(rs);
#pragma unroll
            for (int it = 0; it < NITM; ++it) {
                const int u = min(lt + it * T, U - 1);
                const u8* blk = rp + (u >> 2) * Fmt<F>::BB;
                raw[it].q = gload16(blk + QO + 16 * (u & 3));
                raw[it].d = gload2u(blk + DO);
            }
        }
    }
    template <int N>
    __device__ __forceinline__ void wait() {
#pragma unroll
        for (int it = 0; it < NITM; ++it) {
            if (it == 0)
                asm volatile("s_waitcnt vmcnt(%2)" : "+v"(raw[it].q), "+v"(raw[it].d) : "n"(N));
            else
                asm volatile("" : "+v"(raw[it].q), "+v"(raw[it].d));
        }
    }
};

__device__ __forceinline__ u32x2 gload8s(const u8* base, u32 off) {
    u32x2 v;
    asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
    return v;
}
template <int OFF>
__device__ __forceinline__ u32x4 gload16so(const u8* base, u32 off) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(v) : "v"(off), "s"(base), "n"(OFF));
    return v;
}

// Q6_K unit reads by hand for kernels with one row per wave (T = 64): five reads per unit from the row's
// address in scalar registers and lane-constant offsets (Fmt<Q6_K>::load's layout: ql at 64h + 16j and
// +32, qh at 128 + 32h + 16j, the scales at 192 + 8h, d at 208 of block u / 4).
template <int NITM>
struct Q6kStepAsm {
    Fmt<NMQ_Q6_K>::Raw raw[NITM];
    template <int T>
    __device__ __forceinline__ void load(const RowMap& rm, int r, int lt, int U, int fb) {
        static_assert(T == 64, "one row per wave");
        const int rs = r < rm.n_out ? r : min(fb, rm.n_out - 1);
        const u8* rp = (const u8*)uniform64((int64_t)rm.row(rs));
#pragma unroll
        for (int it = 0; it < NITM; ++it) {
            const int u = min(lt + it * T, U - 1), h = (u >> 1) & 1, j = u & 1;
            const u32 ob = (u32)((u >> 2) * Fmt<NMQ_Q6_K>::BB), ol = ob + (u32)(64 * h + 16 * j);
            raw[it].la = gload16s(rp, ol);
            raw[it].lb = gload16so<32>(rp, ol);
            raw[it].qh = gload16s(rp, ob + (u32)(128 + 32 * h + 16 * j));
            raw[it].sc = gload8s(rp, ob + (u32)(192 + 8 * h));
            raw[it].d = gload2us(rp, ob + 208u);
        }
    }
    template <int N>
    __device__ __forceinline__ void wait() {
#pragma unroll
        for (int it = 0; it < NITM; ++it) {
            if (it == 0)
                asm volatile("s_waitcnt vmcnt(%5)"
                             : "+v"(raw[it].la), "+v"(raw[it].lb), "+v"(raw[it].qh), "+v"(raw[it].sc), "+v"(raw[it].d)
                             : "n"(N));
            else
                asm volatile("" : "+v"(raw[it].la), "+v"(raw[it].lb), "+v"(raw[it].qh), "+v"(raw[it].sc), "+v"(raw[it].d));
        }
    }
};

// Hand-issued step buffers per format (HandStep<F, NITM>::NL reads per unit).
template <int F, int NITM>
struct HandStep : QdStepAsm<F, NITM> {
    static constexpr int NL = 2;
};
template <int NITM>
struct HandStep<NMQ_Q4_K, NITM> : Q4kStepAsm<NITM> {
    static constexpr int NL = 3;
};
template <int NITM>
struct HandStep<NMQ_Q6_K, NITM> : Q6kStepAsm<NITM> {  // one row per wave only (the K-split kernel)
    static constexpr int NL = 5;
};
constexpr bool hand_format(int f) { return f == NMQ_Q4_K || f == NMQ_TQ2_0 || f == NMQ_IQ2_XXS; }
// formats whose reads the K-split kernel issues by hand
constexpr bool mvk_hand(int f) { return f == NMQ_Q4_K || f == NMQ_TQ2_0 || f == NMQ_Q6_K; }

// Per-lane constants of the one-token path (units of a lane are fixed: u = lt + it*T).
// TQ2_0 on the raw 2-bit codes c (value c - 1).  Run r of a unit (16 values, one xd) holds its codes at bit
// offset 2r of the unit's four code dwords, so q & (3 << 2r) is the run's codes times 4^r as bytes; run 3
// is shifted right by 2 first, (q >> 2) & 0x30303030 = 16 c, so that every byte stays <= 32 and the signed
// dot4 is exact.  With the run's scale f (1, 4, 16, 16), S1' = sum f c xq and S2' = sum f c xq2:
//   f (254 sum (c - 1) xq + sum (c - 1) xq2) = 254 S1' + S2' - f (254 X1 + X2),
// X1, X2 the run's input sums.  The xq2 chain starts at -f (254 X1 + X2) (a lane constant, formed once from
// the lane's input slice), one 24-bit multiply-add joins the stages, an exact arithmetic shift removes f, and
// the run adds (that integer, |.| < 2^20: exact in fp32) times xd / 254; the block scale d multiplies the
// unit's sum.  About half the VALU instructions of unpacking every code to a signed byte.
struct Tq2Lane {
    int k[4];    // xq2 chain start per run
    float e[4];  // xd / 254 per run
};

__device__ __forceinline__ Tq2Lane tq2_lane(const XSlice& x) {
    Tq2Lane c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int x1 = 0, x2 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x1 = dot4(0x01010101u, x.q[4 * r + k], x1);
            x2 = dot4(0x01010101u, x.q2[4 * r + k], x2);
        }
        const int f = r == 0 ? 1 : (r == 1 ? 4 : 16);
        c.k[r] = -f * (254 * x1 + x2);
        c.e[r] = x.d[r] * FEIN;
    }
    return c;
}

__device__ __forceinline__ float tq2_dot1(const Fmt<NMQ_TQ2_0>::Raw& raw, const XSlice& x, const Tq2Lane& c) {
    const u32 q[4] = {raw.q.x, raw.q.y, raw.q.z, raw.q.w};
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int a = 0, b = c.k[r];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32 w = r == 3 ? ((q[k] >> 2) & 0x30303030u) : (q[k] & (0x03030303u << (2 * r)));
            a = dot4(w, x.q[4 * r + k], a);
            b = dot4(w, x.q2[4 * r + k], b);
        }
        const int t = (__mul24(a, 254) + b) >> (r == 0 ? 0 : (r == 1 ? 2 : 4));  // |a| <= 16*32*127: 24-bit
        acc = fmaf((float)t, c.e[r], acc);
    }
    return acc * h2f(raw.d);
}

struct LaneConst {
    Q4kLane q4k[4];  // Q4_K: the unit's scale/min selection
    Tq2Lane tq2[4];  // TQ2_0 (kernels that hold their input slices): the unit's input constants
    Q6kLane q6k[4];  // Q6_K (likewise)
};

template <int F, int T, int NITM>
__device__ __forceinline__ LaneConst lane_const(int lt) {
    LaneConst c{};
#pragma unroll
    for (int it = 0; it < NITM && it < 4; ++it) c.q4k[it] = q4k_lane(lt + it * T);
    return c;
}

// Kernels that keep the lane's input slices in registers for all their rows: also the per-slice constants.
template <int F, int T, int NITM>
__device__ __forceinline__ LaneConst lane_const(int lt, const XSlice (&x)[NITM]) {
    LaneConst c = lane_const<F, T, NITM>(lt);
    if constexpr (F == NMQ_TQ2_0) {
#pragma unroll
        for (int it = 0; it < NITM && it < 4; ++it) c.tq2[it] = tq2_lane(x[it]);
    }
    if constexpr (F == NMQ_Q6_K) {
#pragma unroll
        for (int it = 0; it < NITM && it < 4; ++it) c.q6k[it] = q6k_lane(x[it]);
    }
    return c;
}

// HELD: the slice constants of lane_const(lt, x) are present; otherwise TQ2_0 and Q6_K form them from the
// slice on the spot (the same integers: both give the same bits).
template <int F, bool HELD = false>
__device__ __forceinline__ float unit_dot1(const typename Fmt<F>::Raw& raw, int u, const u64* tab, const XSlice& x,
                                           const LaneConst& lc, int it) {
    using FM = Fmt<F>;
    if constexpr (F == NMQ_Q4_K) {
        return q4k_dot1(raw, x, lc.q4k[it]);
    } else if constexpr (F == NMQ_Q6_K) {
        return HELD ? q6k_dot1(raw, x, u, lc.q6k[it]) : q6k_dot1(raw, x, u, q6k_lane(x));
    } else if constexpr (F == NMQ_TQ2_0) {
        return HELD ? tq2_dot1(raw, x, lc.tq2[it]) : tq2_dot1(raw, x, tq2_lane(x));
    } else {
        WUnit wu;
        FM::decode(raw, u, tab, wu);
        return unit_dot<FM::STRIDED, FM::HAS_MIN>(wu, x);
    }
}

// The team's RW row sums of one step (every lane of the team holds them after the team reduction).
template <int F, int T, int RW, int NITM>
__device__ __forceinline__ void mv1_dots(const Mv1Step<F, T, RW, NITM>& st, const XSlice (&x)[NITM], int lt, int U,
                                         const u64* tab, const LaneConst& lc, float (&acc)[RW]) {
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        acc[rr] = 0.f;
#pragma unroll
        for (int it = 0; it < NITM; ++it) {
            const int u = lt + it * T;
            const float v = unit_dot1<F, true>(st.raw[rr][it], min(u, U - 1), tab, x[it], lc, it);
            acc[rr] += u < U ? v : 0.f;
        }
    }
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) acc[rr] = team_sum<T>(acc[rr]);
}

template <int F, int T, int RW, int NITM>
__device__ __forceinline__ void mv1_compute(const Mv1Step<F, T, RW, NITM>& st, const XSlice (&x)[NITM], int r0,
                                            const RowMap& rm, int lt, int U, const u64* tab,
                                            const LaneConst& lc) {
    float acc[RW];
    mv1_dots<F, T, RW, NITM>(st, x, lt, U, tab, lc, acc);
    if (lt == 0) {
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
            if (r0 + rr < rm.n_out) *gpw<float>(rm.out(r0 + rr)) = acc[rr];
    }
}

// EXT: the variant that also takes segments and value input (the plain one keeps the shorter code).
// HR (Q4_K, TQ2_0, IQ2_XXS; 1: two-stage input, 2: fp32 values): the weight reads are issued by hand (Q4kStepAsm, the compiler waits for all of a wave's
// outstanding reads at the head of its own loop) and the row results are held in registers (lane k of a
// team: the team's k-th row), written when the team holds T of them (then every outstanding access is
// waited for) and after the last row, so that the pipelined loop issues reads only.
template <int F, int T, int RW, int NITM, int NBUF, bool EXT, int HR = 0>
__global__ __launch_bounds__(512) void mv1_kernel(MvParams p) {
    static_assert(HR == 0 || (hand_format(F) && RW == 1 && (HR == 1 || EXT)), "HR: hand formats, one row per team");
    // HR = 1: the launcher guarantees two-stage input staged in one round; HR = 2: fp32 values (x_mode
    // NMQ_X_F32 or NMQ_X_F32_BF16) in at most two rounds
    args_early<EXT>(p);
    using FM = Fmt<F>;
    constexpr int P = 64 / T;
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = p.nt >> 6;
    const int team = lane / T, lt = lane % T;
    const int m = blockIdx.y;
    int64_t xrow;
    const u8* wbase = instance_weights(p, m, xrow);
    const RowMap rm = row_map<EXT>(p, wbase, p.y + (int64_t)m * p.n_out);
    const int U = (p.n_in + 63) >> 6;
    const int gw = blockIdx.x * W + wave, nw = gridDim.x * W;
    constexpr int SR = P * RW;  // rows per step
    const int off = team * RW;

    // Loads are issued unconditionally (rows and units clamped to valid addresses, surplus results
    // discarded), so the compiler can wait for exactly the oldest step and keep the others in flight.
    // NBUF step buffers rotate: while one step is computed, the next NBUF - 1 are in flight (the first
    // NBUF - 1 go out while the input is staged).
    Mv1Step<F, T, RW, NITM> buf[NBUF];
    using HS = HandStep<hand_format(F) ? F : NMQ_Q4_K, NITM>;
    HS hb[NBUF];  // HR: the step buffers of the hand-issued reads
    const int stride = nw * SR;
    int base = gw * SR;
    if constexpr (HR) {
        auto issue = [&] {
#pragma unroll
            for (int i = 0; i < NBUF - 1; ++i) hb[i].template load<T>(rm, base + i * stride + off, lt, U, base + off);
        };
        if constexpr (HR == 1) stage1_hand<F, HS::NL * NITM * (NBUF - 1)>(lds, tab, p, xrow, issue);
        else stagev_hand<F, HS::NL * NITM * (NBUF - 1)>(lds, tab, p, xrow, issue);
    } else {
        stage1_around<F, EXT, 1>(lds, tab, p, xrow, [&] {
#pragma unroll
            for (int i = 0; i < NBUF - 1; ++i) buf[i].load(rm, base + i * stride + off, lt, U, base + off);
        });
    }
    XSlice x[NITM];
#pragma unroll
    for (int it = 0; it < NITM; ++it) {
        const int u = lt + it * T;
        if (u < U) read_slice<FM::STRIDED>(lds, p.ktp, u, x[it]);
    }

    const LaneConst lc = lane_const<F, T, NITM>(lt, x);
    if constexpr (HR) {
        float res = 0.f;
        int k = 0, first = base;
        bool more = true;
        while (more) {
#pragma unroll
            for (int i = 0; i < NBUF; ++i) {
                if (base >= p.n_out) {  // wave-uniform
                    more = false;
                    break;
                }
                hb[(i + NBUF - 1) % NBUF].template load<T>(rm, base + (NBUF - 1) * stride + off, lt, U, base + off);
                hb[i].template wait<HS::NL * NITM * (NBUF - 1)>();  // this step's reads; the later steps stay out
                float acc = 0.f;
#pragma unroll
                for (int it = 0; it < NITM; ++it) {
                    const int u = lt + it * T;
                    const float v = unit_dot1<F, true>(hb[i].raw[it], min(u, U - 1), tab, x[it], lc, it);
                    acc += u < U ? v : 0.f;
                }
                acc = team_sum<T>(acc);
                res = lt == k ? acc : res;
                base += stride;
                if (++k == T) {
                    const int r = first + lt * stride + off;
                    if (r < rm.n_out) *gpw<float>(rm.out(r)) = res;
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    k = 0;
                    first = base;
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the surplus reads of the last steps
        const int r = first + lt * stride + off;
        if (lt < k && r < rm.n_out) *gpw<float>(rm.out(r)) = res;
        return;
    }
    for (;;) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            if (base >= p.n_out) return;  // wave-uniform
            buf[(i + NBUF - 1) % NBUF].load(rm, base + (NBUF - 1) * stride + off, lt, U, base + off);
            mv1_compute<F, T, RW, NITM>(buf[i], x, base + off, rm, lt, U, tab, lc);
            base += stride;
        }
    }
}

// Where a launch writes a two-stage input (xq, xq2: one byte per value; xd, xs: one float per 32 values),
// and of which activation (NMQ_ACT_*: silu or gelu, rounded to bf16 or not; the MoE kernel: silu, bf16).
struct QuantOut {
    int8_t* xq;
    int8_t* xq2;
    float* xd;
    float* xs;
    int act;
};

// ---- gate and up of a dense FFN with the activation, one token (mvp_kernel) -----------------------------
// Rows of the gate (tensor w) and up (tensor w2) projections in groups of 32: workgroup b takes groups b,
// b + gridDim.x, ...  Waves 0..W/2-1 compute the groups' gate rows, W/2..W-1 their up rows, RPW rows per
// group each, one row per step with the one-token kernel's hand-issued reads (64 lanes, one unit per lane:
// rows of up to 4096 values) and NBUF - 1 steps in flight, across groups too.  A row's sum is the
// persistent kernel's (acc = 0 + the unit's product, team_sum<64>), so every sum equals that row of the
// gathered launch bit for bit.  The sums go to LDS as each group ends; no wave waits for another until
// the last step.  Then (every read complete, one barrier) wave w takes groups w, w + W, ...: lanes 0..31
// form a = act(g) * u (o.act: silu or gelu, rounded to bf16 or not; the expressions of the activation
// launches) and write its two-stage input (quant32).  The group loop body is
// straight-line code of RPW steps, RPW a multiple of NBUF, so the step buffers sit in the same registers
// at every iteration.
constexpr int MVP_MAXG = 16;  // groups per workgroup

template <int F, int HR, int RPW>
__global__ __launch_bounds__(4096 / RPW) void mvp_kernel(MvParams p, QuantOut o) {
    static_assert(hand_format(F) && (HR == 1 || HR == 2), "hand-read formats; two-stage (1) or fp32 (2) input");
    args_early<true>(p);
    using FM = Fmt<F>;
    using HS = HandStep<F, 1>;
    constexpr int T = 64, NBUF = 4, W = 64 / RPW;  // W waves: 32 rows of each projection per group
    static_assert(RPW % NBUF == 0, "the step buffers rotate through whole groups");
    constexpr int HW = HS::NL * (NBUF - 1);
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    __shared__ float res[MVP_MAXG][64];  // per group: the gate sums, then the up sums
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool up = wave >= W / 2;
    const int wj = up ? wave - W / 2 : wave;
    const RowMap rm = row_map<false>(p, up ? p.w2 : p.w, p.y);
    const int U = (p.n_in + 63) >> 6;
    const int nb = gridDim.x, G = p.n_out >> 5;
    const int ng = (G - (int)blockIdx.x + nb - 1) / nb;  // this workgroup's groups (the launcher: 1..MVP_MAXG)
    const int fb = (int)blockIdx.x * 32;                // a row of this workgroup (surplus reads go there)
    // step q: row 32 (b + (q / RPW) nb) + RPW wj + q % RPW; past the last group the row is >= n_out and
    // the read goes to row fb instead
    auto row_of = [&](int q) { return ((int)blockIdx.x + (q / RPW) * nb) * 32 + wj * RPW + q % RPW; };
    HS hb[NBUF];
    auto issue = [&] {
#pragma unroll
        for (int i = 0; i < NBUF - 1; ++i) hb[i].template load<T>(rm, row_of(i), lane, U, fb);
    };
    if constexpr (HR == 1) stage1_hand<F, HW>(lds, tab, p, 0, issue);
    else stagev_hand<F, HW>(lds, tab, p, 0, issue);
    XSlice x[1];
    read_slice<FM::STRIDED>(lds, p.ktp, min(lane, U - 1), x[0]);
    const LaneConst lc = lane_const<F, T, 1>(lane, x);
    float mine = 0.f;  // lane k: the k-th row of the wave's current group
    for (int gi = 0; gi < ng; ++gi) {
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const int i = k % NBUF;
            hb[(i + NBUF - 1) % NBUF].template load<T>(rm, row_of(gi * RPW + k + NBUF - 1), lane, U, fb);
            hb[i].template wait<HW>();  // this step's reads; the later steps stay out
            float acc = 0.f;
            const float v = unit_dot1<F, true>(hb[i].raw[0], min(lane, U - 1), tab, x[0], lc, 0);
            acc += lane < U ? v : 0.f;
            acc = team_sum<T>(acc);
            mine = lane == k ? acc : mine;
        }
        if (lane < RPW) res[gi][(up ? 32 : 0) + wj * RPW + lane] = mine;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the surplus reads of the last steps
    lds_barrier();
    for (int gi = wave; gi < ng; gi += W) {
        if (lane < 32) {
            const int64_t at = ((int64_t)blockIdx.x + (int64_t)gi * nb) * 32 + lane;
            float v = act_value(res[gi][lane], (o.act & NMQ_ACT_GELU) != 0) * res[gi][32 + lane];
            if (o.act & NMQ_ACT_BF16) v = round_bf16(v);
            quant32_store(v, at, o.xq, o.xq2, o.xd, o.xs);
        }
    }
}

// ---- 2..4 tokens (speculative verification), Q4_K ----------------------------------------------------
// The one-token kernel with hand-issued reads for NC tokens: all inputs staged in LDS (one round each,
// read by hand ahead of the first weight steps), all slices held in registers, every weight unit
// decoded once for all (q4k_dotn); a row's NC results stay in registers like the one-token loop's and
// are written to y + t n_out.
template <int T, int NC>
__global__ __launch_bounds__(256) void mvt_kernel(MvParams p) {
    args_early<false>(p);
    constexpr int NITM = 1, NBUF = 3;
    using FM = Fmt<NMQ_Q4_K>;
    using HS = HandStep<NMQ_Q4_K, NITM>;
    constexpr int P = 64 / T;
    constexpr int HW = HS::NL * NITM * (NBUF - 1);
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = p.nt >> 6;
    const int team = lane / T, lt = lane % T;
    const RowMap rm = row_map<false>(p, p.w, p.y);
    const int U = (p.n_in + 63) >> 6;
    const int gw = blockIdx.x * W + wave, nw = gridDim.x * W;
    const int off = team;
    const int stride = nw * P;
    int base = gw * P;
    const int tok = p.ktp * 9 / 4;  // LDS bytes per token
    HS hb[NBUF];
    {
        XRound r[NC];
        const int64_t g = p.n_in / 32;
#pragma unroll
        for (int t = 0; t < NC; ++t)
            stage1_load_hand(r[t], 0, p.xq + t * p.n_in, p.xq2 + t * p.n_in, p.xd + t * g, p.xs + t * g, p.n_in, p.nt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NBUF - 1; ++i) hb[i].template load<T>(rm, base + i * stride + off, lt, U, base + off);
        __builtin_amdgcn_sched_barrier(0);
        xround_wait<HW>(r[0]);
#pragma unroll
        for (int t = 1; t < NC; ++t) asm volatile("" : "+v"(r[t].a), "+v"(r[t].b), "+v"(r[t].d), "+v"(r[t].s));
#pragma unroll
        for (int t = 0; t < NC; ++t) stage1_store<FM::STRIDED>(r[t], 0, lds + t * tok, p.n_in, p.ktp, p.nt);
        lds_barrier();
    }
    XSlice x[NC];
    const int u = min(lt, U - 1);
#pragma unroll
    for (int t = 0; t < NC; ++t) read_slice<FM::STRIDED>(lds + t * tok, p.ktp, u, x[t]);
    const LaneConst lc = lane_const<NMQ_Q4_K, T, NITM>(lt);
    float res[NC];
#pragma unroll
    for (int t = 0; t < NC; ++t) res[t] = 0.f;
    int k = 0, first = base;
    bool more = true;
    while (more) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            if (base >= p.n_out) {  // wave-uniform
                more = false;
                break;
            }
            hb[(i + NBUF - 1) % NBUF].template load<T>(rm, base + (NBUF - 1) * stride + off, lt, U, base + off);
            hb[i].template wait<HW>();
            float v[NC];
            q4k_dotn<NC>(hb[i].raw[0], x, lc.q4k[0], v);
#pragma unroll
            for (int t = 0; t < NC; ++t) {
                const float a = team_sum<T>(0.f + (lt < U ? v[t] : 0.f));
                res[t] = lt == k ? a : res[t];
            }
            base += stride;
            if (++k == T) {
                const int r = first + lt * stride + off;
                if (r < p.n_out) {
#pragma unroll
                    for (int t = 0; t < NC; ++t) gpw<float>(p.y)[(int64_t)t * p.n_out + r] = res[t];
                }
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                k = 0;
                first = base;
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the surplus reads of the last steps
    const int r = first + lt * stride + off;
    if (lt < k && r < p.n_out) {
#pragma unroll
        for (int t = 0; t < NC; ++t) gpw<float>(p.y)[(int64_t)t * p.n_out + r] = res[t];
    }
}

template <int NC>
inline void (*pick_mvt(int T))(MvParams) {
    return T == 16 ? mvt_kernel<16, NC> : (T == 32 ? mvt_kernel<32, NC> : mvt_kernel<64, NC>);
}

// ---- one token, long rows (more than 128 units of 64 values) ---------------------------------------
// A wave owns whole rows (RW at a time, T = 64 lanes, NIT units per lane): all of a row group's weights
// are requested at once; the input is staged once per workgroup in LDS and each unit's slice is read
// from there as it is used (holding NIT slices in registers would not fit beside the weights).
// PIPE = false: one row group per wave (the launch has at least as many waves as groups).  PIPE: waves
// with several row groups request the next group's weights before computing the current one.
// Q6_K unit against the input staged in LDS (stage_tile layout), one 16-value group at a time:
// q6k_dot1 with the group's 2 x 16 input bytes and its xd read just before use.  (Unsigned codes with a
// per-group offset -32 (sum xq + sum xq2 / 254) formed once per workgroup took 14 % fewer VALU
// instructions but an extra LDS pass and barrier: 14.2 against 13.8 us for 4096x14336, not kept.)
// q6k_dot1 with the unit's input read from the staged LDS copy and its group constants formed on the spot
// (the same integers and fp32 operations: results equal q6k_dot1's bit for bit).
__device__ __forceinline__ float q6k_dot1_lds(const Fmt<NMQ_Q6_K>::Raw& r, const u8* base, int ktp, int u) {
    const u32 la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
    const u32 lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
    const u32 qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    const u32 sh = 8u * (u32)(u & 1);
    const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
    const float4 xd = *(const float4*)((const float*)(base + 2 * ktp) + 8 * b + 4 * h);
    const float xdg[4] = {xd.x, xd.y, xd.z, xd.w};
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int ph = swz<true>(16 * b + 8 * h + 2 * g + j);
        const u32x4 a = *(const u32x4*)(base + 16 * ph);
        const u32x4 c = *(const u32x4*)(base + ktp + 16 * ph);
        const u32 xa[4] = {a.x, a.y, a.z, a.w};
        const u32 xc[4] = {c.x, c.y, c.z, c.w};
        const int k0 = q6k_group_const(a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w);
        const float se = (float)(int8_t)bfe(g < 2 ? r.sc.x : r.sc.y, sh + 16u * (u32)(g & 1), 8) * (xdg[g] * FEIN);
        acc = g == 0 ? q6k_group<0>(la, qh, xa, xc, k0, se, acc)
            : g == 1 ? q6k_group<1>(lb, qh, xa, xc, k0, se, acc)
            : g == 2 ? q6k_group<2>(la, qh, xa, xc, k0, se, acc) : q6k_group<3>(lb, qh, xa, xc, k0, se, acc);
    }
    return acc * h2f(r.d);
}

template <int F, int RW, int NIT>
__device__ __forceinline__ void mvl_compute(const Mv1Step<F, 64, RW, NIT>& st, const u8* lds, int ktp, int r0,
                                            const RowMap& rm, int lane, int U, const u64* tab,
                                            const LaneConst& lc) {
    using FM = Fmt<F>;
    float acc[RW];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) acc[rr] = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int u = lane + it * 64;
        const int uc = min(u, U - 1);
        // each 64-unit slice summed over the wave, the slices added in order from zero: the K-split
        // kernel's order, so value input (staged here) and the two-stage input give the same bits
        if constexpr (F == NMQ_Q6_K) {
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                const float v = q6k_dot1_lds(st.raw[rr][it], lds, ktp, uc);
                acc[rr] += team_sum<64>(u < U ? v : 0.f);
            }
        } else {
            XSlice x;
            read_slice<FM::STRIDED>(lds, ktp, uc, x);
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                const float v = unit_dot1<F>(st.raw[rr][it], uc, tab, x, lc, it);
                acc[rr] += team_sum<64>(u < U ? v : 0.f);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // one input slice live at a time
    }
    if (lane == 0) {
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
            if (r0 + rr < rm.n_out) *gpw<float>(rm.out(r0 + rr)) = acc[rr];
    }
}

template <int F, int RW, int NIT, bool PIPE, bool EXT>
__global__ __launch_bounds__(PIPE ? 512 : 1024) void mvl_kernel(MvParams p) {
    args_early<EXT>(p);
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = p.nt >> 6;
    const int m = blockIdx.y;
    int64_t xrow;
    const u8* wbase = instance_weights(p, m, xrow);
    const RowMap rm = row_map<EXT>(p, wbase, p.y + (int64_t)m * p.n_out);
    const int U = (p.n_in + 63) >> 6;
    const int stride = gridDim.x * W * RW;
    int base = (blockIdx.x * W + wave) * RW;
    Mv1Step<F, 64, RW, NIT> a;
    stage1_around<F, EXT, 4>(lds, tab, p, xrow, [&] { a.load(rm, base, lane, U, base); });
    const LaneConst lc = lane_const<F, 64, NIT>(lane);
    if constexpr (!PIPE) {
        // the launch gives every wave at most one row group (grid x W >= groups)
        if (base < p.n_out) mvl_compute<F, RW, NIT>(a, lds, p.ktp, base, rm, lane, U, tab, lc);
    } else {
        Mv1Step<F, 64, RW, NIT> b;
        for (;;) {
            b.load(rm, base + stride, lane, U, base);
            mvl_compute<F, RW, NIT>(a, lds, p.ktp, base, rm, lane, U, tab, lc);
            base += stride;
            if (base >= p.n_out) return;
            a.load(rm, base + stride, lane, U, base);
            mvl_compute<F, RW, NIT>(b, lds, p.ktp, base, rm, lane, U, tab, lc);
            base += stride;
            if (base >= p.n_out) return;
        }
    }
}

// ---- one token, one chunk per wave -------------------------------------------------------------
// Each wave owns one chunk of P*RW rows: it requests all of the chunk's weights while the input is
// staged (the HBM latency overlaps the staging), then computes the rows in order as their data
// arrives.  Used when the matrix fits in the resident waves of one launch (then every
// weight byte of the matvec is in flight at once, the shape a streaming read needs at this size).
template <int F, int T, int RW, bool EXT>
__device__ __forceinline__ void mvc_body(const MvParams& p) {
    using FM = Fmt<F>;
    constexpr int P = 64 / T;
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    // the wave index is uniform across the wave: readfirstlane lets the row addressing run on SALU
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = p.nt >> 6;
    const int team = lane / T, lt = lane % T;
    const int m = blockIdx.y;
    int64_t xrow;
    const u8* wbase = instance_weights(p, m, xrow);
    const RowMap rm = row_map<EXT>(p, wbase, p.y + (int64_t)m * p.n_out);
    const int U = (p.n_in + 63) >> 6;
    const int r0 = ((blockIdx.x * W + wave) * P + team) * RW;
    Mv1Step<F, T, RW, 1> a;
    stage1_around<F, EXT, 1>(lds, tab, p, xrow, [&] { a.load(rm, r0, lt, U, r0); });
    XSlice x[1];
    read_slice<FM::STRIDED>(lds, p.ktp, min(lt, U - 1), x[0]);
    const LaneConst lc = lane_const<F, T, 1>(lt, x);
    mv1_compute<F, T, RW, 1>(a, x, r0, rm, lt, U, tab, lc);
}

template <int F, int T, int RW, bool EXT>
__global__ __launch_bounds__(RW >= 8 ? 512 : 1024) void mvc_kernel(MvParams p) {
    args_early<EXT>(p);
    mvc_body<F, T, RW, EXT>(p);
}

// The down projection of an expert layer with the weighted combine in the same workgroup (MoE, one
// token per blockIdx.y): workgroup (x, t) computes rows [x*R, (x+1)*R) of all k slots of token t -- slot j
// (instance t*k + j, expert ids[t*k + j]) on waves j*WS .. j*WS + WS - 1, each wave one chunk of P*RW rows
// like the chunk kernel -- keeps the k*R sums in LDS and then forms
//   out[t][r] = sum_j w[t*k + j] * y_j[r]   (fp32 fused multiply-adds in slot order),
// bit for bit the plain gathered launch followed by nmq_moe_combine, with no global intermediate and no
// ordering between workgroups.  The k slots' inputs are consecutive rows of values (x_group = 1), staged
// as one row of k*n_in values: slot j's unit u is unit j*U + u of that row.
struct Combine {
    const float* w;  // L*k slot weights
    float* out;      // L x n_out
    int k;           // slots per token
    int ws;          // waves per slot
};

template <int F, int T, int RW>
__global__ __launch_bounds__(1024) void moe_down_kernel(MvParams p, Combine c) {
    args_early<true>(p);
    using FM = Fmt<F>;
    constexpr int P = 64 / T;
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = lane / T, lt = lane % T;
    const int t = blockIdx.y, j = wave / c.ws, wj = wave % c.ws;
    const int R = c.ws * P * RW;  // rows per workgroup
    int64_t xrow;
    const u8* wbase = instance_weights(p, t * c.k + j, xrow);
    const RowMap rm = row_map<false>(p, wbase, p.y);
    const int U = (p.n_in + 63) >> 6;
    const int lr = (wj * P + team) * RW;  // the team's first row in the block
    const int r0 = blockIdx.x * R + lr;
    // the token's slot weights, read now so that the combine at the end does not wait for memory
    __shared__ float wt[16];
    const float wv = (int)threadIdx.x < c.k ? gp<float>(c.w)[(int64_t)t * c.k + threadIdx.x] : 0.f;
    Mv1Step<F, T, RW, 1> a;
    MvParams q = p;  // the token's k input rows as one row of k*n_in values
    q.n_in = p.n_in * c.k;
    stage1_around<F, true, 1>(lds, tab, q, t, [&] { a.load(rm, r0, lt, U, r0); });
    XSlice x[1];
    read_slice<FM::STRIDED>(lds, p.ktp, j * U + min(lt, U - 1), x[0]);
    const LaneConst lc = lane_const<F, T, 1>(lt, x);
    float acc[RW];
    mv1_dots<F, T, RW, 1>(a, x, lt, U, tab, lc, acc);
    float* res = (float*)(lds + p.ktp * 9 / 4);  // k x R sums
    if (lt == 0) {
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) res[j * R + lr + rr] = acc[rr];
    }
    if ((int)threadIdx.x < c.k) wt[threadIdx.x] = wv;
    lds_barrier();
    for (int r = (int)threadIdx.x; r < R; r += p.nt) {
        const int row = blockIdx.x * R + r;
        if (row >= p.n_out) break;
        float sum = 0.f;
        for (int s = 0; s < c.k; ++s) sum = fmaf(wt[s], res[s * R + r], sum);
        gpw<float>(c.out)[(int64_t)t * p.n_out + row] = sum;
    }
}

// The gate and up projections of an expert layer with the gated activation in the same workgroup (MoE):
// workgroup (x, s) computes rows [32x, 32x + 32) of slot s's gate projection (instance s: expert ids[s] of
// tensor w) on waves 0 .. WH - 1 and of its up projection (instance n_ids + s, tensor w2) on waves
// WH .. 2WH - 1, each wave P*RW rows with the chunk kernel's unit products and team sums (so every sum
// equals that row of the gathered launch bit for bit), keeps the 64 sums in LDS, and then writes the
// two-stage input of a[s][r] = silu_mul_bf16(g[r], u[r]) for its 32 rows -- one group of the down
// projection's input.  The gate and up outputs never leave the workgroup and the activation needs no
// launch of its own.  Slot s reads input row s / x_group (the token).
// Workgroup (group g, slot s) of the gate|up kernel; the rows of a projection on WH = 32 / (P*RW) waves (the
// workgroup has 2*WH).  res: 64 floats of LDS.  Wave 0 writes the group's two-stage input.
template <int F, int T, int RW>
__device__ __forceinline__ void moe_gu_body(const MvParams& p, const QuantOut& o, int g, int s, u8* lds, u64* tab,
                                            float* res) {
    using FM = Fmt<F>;
    constexpr int P = 64 / T;
    constexpr int WH = 32 / (P * RW);  // waves per projection
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = lane / T, lt = lane % T;
    const bool up = wave >= WH;
    const int lr = ((up ? wave - WH : wave) * P + team) * RW;  // the team's first row in the group
    const int r0 = g * 32 + lr;
    int64_t xrow;
    const u8* wbase = instance_weights(p, up ? p.n_ids + s : s, xrow);
    const RowMap rm = row_map<false>(p, wbase, p.y);
    const int U = (p.n_in + 63) >> 6;
    Mv1Step<F, T, RW, 1> a;
    stage1_around<F, true, 1>(lds, tab, p, xrow, [&] { a.load(rm, r0, lt, U, r0); });
    XSlice x[1];
    read_slice<FM::STRIDED>(lds, p.ktp, min(lt, U - 1), x[0]);
    const LaneConst lc = lane_const<F, T, 1>(lt, x);
    float acc[RW];
    mv1_dots<F, T, RW, 1>(a, x, lt, U, tab, lc, acc);
    if (lt == 0) {
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) res[(up ? 32 : 0) + lr + rr] = acc[rr];
    }
    lds_barrier();
    if (wave == 0 && lane < 32) {
        const float v = silu_mul_bf16(res[lane], res[32 + lane]);
        quant32_store(v, (int64_t)s * p.n_out + g * 32 + lane, o.xq, o.xq2, o.xd, o.xs);
    }
}

template <int F, int T, int RW>
__global__ __launch_bounds__(1024) void moe_gu_kernel(MvParams p, QuantOut o) {
    args_early<true>(p);
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    __shared__ float res[64];  // gate sums, then up sums
    moe_gu_body<F, T, RW>(p, o, blockIdx.x, blockIdx.y, lds, tab, res);
}

// ---- host side --------------------------------------------------------------------------------

struct DeviceInfo {
    int cus;
    int lds_max;      // bytes of dynamic LDS one workgroup may use (<= 64 KB)
    int lds_max_big;  // bytes of LDS one workgroup may use in total (160 KB on gfx950)
};
DeviceInfo device_info();

typedef void (*MvKernel)(MvParams);

template <int F, int NC, int RW>
inline MvKernel pick_t(int T) {
    switch (T) {
        case 16: return mv_kernel<F, NC, 16, RW>;
        case 32: return mv_kernel<F, NC, 32, RW>;
        case 64: return mv_kernel<F, NC, 64, RW>;
        case 128: return mv_kernel<F, NC, 128, RW>;
        default: return mv_kernel<F, NC, 256, RW>;
    }
}

template <int F, int NC>
inline MvKernel pick_rw(int rw, int T) {
    if (NC <= 2) {
        switch (rw) {
            case 1: return pick_t<F, NC, 1>(T);
            case 2: return pick_t<F, NC, 2>(T);
            default: return pick_t<F, NC, 4>(T);
        }
    }
    return rw == 1 ? pick_t<F, NC, 1>(T) : pick_t<F, NC, 2>(T);
}

template <int F>
inline MvKernel pick_kernel(int nc, int rw, int T) {
    switch (nc) {
        case 1: return pick_rw<F, 1>(rw, T);
        case 2: return pick_rw<F, 2>(rw, T);
        case 3: return pick_rw<F, 3>(rw, T);
        case 4: return pick_rw<F, 4>(rw, T);
        case 5: return pick_rw<F, 5>(rw, T);
        case 6: return pick_rw<F, 6>(rw, T);
        case 7: return pick_rw<F, 7>(rw, T);
        default: return pick_rw<F, 8>(rw, T);
    }
}

// Launch shape for one call (exposed for the tuning tests): team width T (lanes per row), rows per
// team RW, waves per workgroup W, row groups per workgroup and the K tile.
struct MvShape {
    int T, rw, W, groups, kt, ktp, n_tiles, grid_x;
    size_t lds;
};

template <int F>
inline MvShape plan_mv(int n_out, int n_in, int nc, int n_mats, const DeviceInfo& di) {
    using FM = Fmt<F>;
    MvShape s{};
    // K tile: the whole row when the input of all tokens fits the LDS budget
    const int budget = nc == 1 ? 40 * 1024 : di.lds_max;
    const int step = FM::BV == 256 ? 256 : 64;
    int kt = (int)((int64_t)budget * 4 / 9 / nc) / 128 * 128 / step * step;
    if (kt < step) kt = step;
    if (kt >= n_in) kt = n_in;
    s.kt = kt;
    s.ktp = (kt + 127) / 128 * 128;
    s.n_tiles = (n_in + kt - 1) / kt;
    const int U = (kt + 63) / 64;  // units per row in a tile
    s.T = U <= 16 ? 16 : U <= 32 ? 32 : U <= 64 ? 64 : U <= 128 ? 128 : 256;
    // rows per team: as many as keep >= 8 (RW=4) or >= 4 (RW=2) waves per CU busy
    const int64_t rows = (int64_t)n_out * n_mats;
    auto waves = [&](int rw) { return (rows + rw - 1) / rw * s.T / 64; };
    const int rw_max = nc <= 2 ? 4 : 2;
    s.rw = 1;
    if (rw_max >= 4 && waves(4) >= 8 * di.cus) s.rw = 4;
    else if (waves(2) >= 4 * di.cus) s.rw = 2;
    const int TW = s.T > 64 ? s.T / 64 : 1;
    const int P = s.T < 64 ? 64 / s.T : 1;
    int W = 4;
    // fewer waves per workgroup for small problems, so that more workgroups spread over the CUs
    while (W > TW && (int64_t)(n_out + (W / TW) * P * s.rw - 1) / ((W / TW) * P * s.rw) * n_mats < 2 * di.cus) W /= 2;
    if (W < TW) W = TW;
    s.W = W;
    const int rows_iter = (W / TW) * P * s.rw;
    const int iters = (n_out + rows_iter - 1) / rows_iter;
    int groups = 1;
    if (s.n_tiles == 1 && (int64_t)iters * n_mats > 16 * di.cus) groups = (int)((int64_t)iters * n_mats / (8 * di.cus));
    s.groups = groups < 1 ? 1 : (groups > 64 ? 64 : groups);
    s.grid_x = (iters + s.groups - 1) / s.groups;
    s.lds = (size_t)nc * ((size_t)s.ktp * 9 / 4);
    return s;
}

template <int F, int T, int RW>
inline MvKernel pick_mv1_nit(int nitm, int nbuf) {
    switch (nitm) {
        case 1: return nbuf == 4 ? mv1_kernel<F, T, RW, 1, 4, false> : mv1_kernel<F, T, RW, 1, 3, false>;
        case 2: return nbuf == 4 ? mv1_kernel<F, T, RW, 2, 4, false> : mv1_kernel<F, T, RW, 2, 3, false>;
        default: return mv1_kernel<F, T, RW, 4, 3, false>;
    }
}
template <int F, int T>
inline MvKernel pick_mv1_rw(int rw, int nitm, int nbuf) {
    return rw == 1 ? pick_mv1_nit<F, T, 1>(nitm, nbuf) : pick_mv1_nit<F, T, 2>(nitm, nbuf);
}
// ext: segments or value input, one row per team and 3 buffers (the default shape) only
template <int F, int T>
inline MvKernel pick_mv1_ext(int nitm) {
    return nitm == 1 ? mv1_kernel<F, T, 1, 1, 3, true> : (nitm == 2 ? mv1_kernel<F, T, 1, 2, 3, true>
                                                                     : mv1_kernel<F, T, 1, 4, 3, true>);
}
// hr: the Q4_K variant with hand-issued weight reads and register-held results (one row per team,
// 3 buffers)
template <int F, int T, bool EXT, int HR>
inline MvKernel pick_mv1_hr(int nitm, int nbuf) {
    if constexpr (!hand_format(F)) return nullptr;
    else if (nitm == 1) return nbuf == 4 ? mv1_kernel<F, T, 1, 1, 4, EXT, HR> : mv1_kernel<F, T, 1, 1, 3, EXT, HR>;
    else return mv1_kernel<F, T, 1, 2, 3, EXT, HR>;
}
template <int F, bool EXT, int HR>
inline MvKernel pick_mv1_hr_t(int T, int nitm, int nbuf) {
    return T == 16 ? pick_mv1_hr<F, 16, EXT, HR>(nitm, nbuf)
                   : (T == 32 ? pick_mv1_hr<F, 32, EXT, HR>(nitm, nbuf) : pick_mv1_hr<F, 64, EXT, HR>(nitm, nbuf));
}
template <int F>
inline MvKernel pick_mv1(int T, int rw, int nitm, int nbuf, bool ext, int hr = 0) {
    if (hr == 2) return pick_mv1_hr_t<F, true, 2>(T, nitm, nbuf);
    if (hr == 1) return ext ? pick_mv1_hr_t<F, true, 1>(T, nitm, nbuf) : pick_mv1_hr_t<F, false, 1>(T, nitm, nbuf);
    if (ext) return T == 16 ? pick_mv1_ext<F, 16>(nitm) : (T == 32 ? pick_mv1_ext<F, 32>(nitm) : pick_mv1_ext<F, 64>(nitm));
    switch (T) {
        case 16: return pick_mv1_rw<F, 16>(rw, nitm, nbuf);
        case 32: return pick_mv1_rw<F, 32>(rw, nitm, nbuf);
        default: return pick_mv1_rw<F, 64>(rw, nitm, nbuf);
    }
}

}  // namespace nmq
#include "nmq_mfma.hpp"
#include "nmq_mmh.hpp"
namespace nmq {

struct Mv1Shape {
    bool ok;
    int T, rw, nitm, nbuf, W, grid_x, ktp;
    size_t lds;
};

inline Mv1Shape plan_mv1(int n_out, int n_in, int n_mats, const DeviceInfo& di, bool values = false) {
    Mv1Shape s{};
    if (!tune(TUNE_MV1, 1)) return s;
    const int U = (n_in + 63) / 64;
    s.T = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
    const int tf = tune(TUNE_MV1_T, 0);
    if (tf == 16 || tf == 32 || tf == 64) s.T = tf;
    const int nit = (U + s.T - 1) / s.T;
    if (nit > tune(TUNE_MV1_MAXNIT, 2)) return s;
    s.nitm = nit <= 1 ? 1 : (nit <= 2 ? 2 : 4);
    s.rw = tune(TUNE_MV1_RW, 1);
    s.rw = s.rw == 2 ? 2 : 1;
    s.nbuf = tune(TUNE_MV1_NBUF, 3) == 4 && s.nitm * s.rw <= 2 ? 4 : 3;
    const int P = 64 / s.T;
    const int64_t steps = ((int64_t)n_out + P * s.rw - 1) / (P * s.rw);  // per instance
    // Two-stage input: 8 resident waves per CU in 4-wave workgroups (two per CU).  Measured on MI355X against
    // 16 waves per CU in 8-wave workgroups: Q4_K 14336x4096 8.37 -> 7.43 us, TQ2_0 12288x4096 6.21 -> 5.82,
    // Q6_K 14336x4096 13.37 -> 11.60, Q8_0 14336x4096 16.25 -> 14.02, gate|up in one launch 13.39 -> 13.10;
    // more step buffers per wave, or 4 to 6 waves per CU, were not faster overall.  Value input: 16 waves per
    // CU in 8-wave workgroups (the hand-issued staging of 4096 fp32 values needs 512 threads; at 8 waves per
    // CU the gate|up launch of the Llama-3-8B layer was faster alone but the layer 1.4 us slower).
    const int wpc = tune(TUNE_MV1_WPC, values ? 16 : 8);
    int64_t waves = (int64_t)wpc * di.cus / n_mats;
    if (waves < 1) waves = 1;
    if (waves > steps) waves = steps;
    int wmax = tune(TUNE_MV1_W, values ? 8 : 4);
    wmax = wmax < 1 ? 1 : (wmax > 8 ? 8 : wmax);  // launch bound: 512 threads
    s.W = (int)(waves < wmax ? waves : wmax);
    s.grid_x = (int)((waves + s.W - 1) / s.W);
    s.ktp = (n_in + 127) / 128 * 128;
    s.lds = (size_t)s.ktp * 9 / 4;
    s.ok = s.lds <= (size_t)di.lds_max;
    return s;
}

// Long rows at one token: T = 64 lanes per row, NIT = 3 or 4 units per lane (129..256 units = up to
// 16384 values); one row per wave while the rows fit the resident waves (NMQ_MVL_WPC = 16 per CU),
// otherwise the pipelined variant.  The input (2.25 bytes per value) must fit the workgroup's LDS.
struct MvlShape {
    bool ok;
    int nit, W, grid_x, ktp;
    bool pipe;
    size_t lds;
};

inline MvlShape plan_mvl(int n_out, int n_in, int n_mats, const DeviceInfo& di) {
    MvlShape s{};
    const int U = (n_in + 63) / 64;
    if (U <= 128 || U > 256 || !tune(TUNE_MVL, 1)) return s;
    s.nit = U <= 192 ? 3 : 4;
    int64_t waves_max = (int64_t)tune(TUNE_MVL_WPC, 16) * di.cus / n_mats;
    if (waves_max < 1) waves_max = 1;
    const int64_t groups = n_out;  // RW = 1
    s.pipe = groups > waves_max;
    int64_t waves = groups < waves_max ? groups : waves_max;
    if (waves < 1) waves = 1;
    const int wcap = s.pipe ? 8 : 16;  // launch bounds: 512 / 1024 threads
    int wmax = tune(TUNE_MVL_W, s.pipe ? 8 : 4);  // measured on MI355X: 4-wave workgroups (several
                                                       // per CU) beat one 16-wave workgroup per CU
    wmax = wmax < 1 ? 1 : (wmax > wcap ? wcap : wmax);
    s.W = (int)(waves < wmax ? waves : wmax);
    s.grid_x = (int)((waves + s.W - 1) / s.W);
    s.ktp = (n_in + 127) / 128 * 128;
    s.lds = (size_t)s.ktp * 9 / 4;
    s.ok = s.lds <= (size_t)di.lds_max;
    return s;
}

// ---- one token, long rows split along K over the waves of a workgroup ------------------------------------
// The input slice of unit u straight from global memory, in the register layout read_slice forms from LDS
// (contiguous formats: values 64u .. 64u+63; strided formats: the 16-value runs 128h + 32k + 16j of block b).
template <bool STRIDED>
__device__ __forceinline__ void load_slice(const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int u,
                                           XSlice& x) {
    if (!STRIDED) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 a = *gp<u32x4>(xq + 64 * u + 16 * k);
            const u32x4 b = *gp<u32x4>(xq2 + 64 * u + 16 * k);
            x.q[4 * k] = a.x; x.q[4 * k + 1] = a.y; x.q[4 * k + 2] = a.z; x.q[4 * k + 3] = a.w;
            x.q2[4 * k] = b.x; x.q2[4 * k + 1] = b.y; x.q2[4 * k + 2] = b.z; x.q2[4 * k + 3] = b.w;
        }
        const u32x2 dd = *gp<u32x2>(xd + 2 * u);
        const u32x2 ss = *gp<u32x2>(xs + 2 * u);
        x.d[0] = __uint_as_float(dd.x); x.d[1] = __uint_as_float(dd.y); x.d[2] = 0.f; x.d[3] = 0.f;
        x.s[0] = __uint_as_float(ss.x); x.s[1] = __uint_as_float(ss.y);
    } else {
        const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
        const int v0 = 256 * b + 128 * h + 16 * j;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 a = *gp<u32x4>(xq + v0 + 32 * k);
            const u32x4 c = *gp<u32x4>(xq2 + v0 + 32 * k);
            x.q[4 * k] = a.x; x.q[4 * k + 1] = a.y; x.q[4 * k + 2] = a.z; x.q[4 * k + 3] = a.w;
            x.q2[4 * k] = c.x; x.q2[4 * k + 1] = c.y; x.q2[4 * k + 2] = c.z; x.q2[4 * k + 3] = c.w;
        }
        const u32x4 dd = *gp<u32x4>(xd + 8 * b + 4 * h);
        x.d[0] = __uint_as_float(dd.x); x.d[1] = __uint_as_float(dd.y);
        x.d[2] = __uint_as_float(dd.z); x.d[3] = __uint_as_float(dd.w);
        x.s[0] = x.s[1] = 0.f;
    }
}

// load_slice with the reads issued by hand (gload16/gload8): wait<N>() waits for them with N later reads
// out, then unpack() forms the slice.
template <bool STRIDED>
struct SliceAsm {
    u32x4 a[4], c[4], dd;
    u32x2 d2, s2;
    __device__ __forceinline__ void load(const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int u) {
        if (!STRIDED) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[k] = gload16(xq + 64 * u + 16 * k);
                c[k] = gload16(xq2 + 64 * u + 16 * k);
            }
            d2 = gload8(xd + 2 * u);
            s2 = gload8(xs + 2 * u);
        } else {
            const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
            const int v0 = 256 * b + 128 * h + 16 * j;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[k] = gload16(xq + v0 + 32 * k);
                c[k] = gload16(xq2 + v0 + 32 * k);
            }
            dd = gload16(xd + 8 * b + 4 * h);
        }
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
        if (!STRIDED)
            asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(c[0]), "+v"(c[1]), "+v"(c[2]),
                         "+v"(c[3]), "+v"(d2), "+v"(s2));
        else
            asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(c[0]), "+v"(c[1]), "+v"(c[2]),
                         "+v"(c[3]), "+v"(dd));
    }
    __device__ __forceinline__ void unpack(XSlice& x) const {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x.q[4 * k] = a[k].x; x.q[4 * k + 1] = a[k].y; x.q[4 * k + 2] = a[k].z; x.q[4 * k + 3] = a[k].w;
            x.q2[4 * k] = c[k].x; x.q2[4 * k + 1] = c[k].y; x.q2[4 * k + 2] = c[k].z; x.q2[4 * k + 3] = c[k].w;
        }
        if (!STRIDED) {
            x.d[0] = __uint_as_float(d2.x); x.d[1] = __uint_as_float(d2.y); x.d[2] = 0.f; x.d[3] = 0.f;
            x.s[0] = __uint_as_float(s2.x); x.s[1] = __uint_as_float(s2.y);
        } else {
            x.d[0] = __uint_as_float(dd.x); x.d[1] = __uint_as_float(dd.y);
            x.d[2] = __uint_as_float(dd.z); x.d[3] = __uint_as_float(dd.w);
            x.s[0] = x.s[1] = 0.f;
        }
    }
};

// Rows of 65..256 units (one token, two-stage input): a workgroup of KS = ceil(U / 64) waves walks the rows
// blockIdx.x, blockIdx.x + G, ... (G = gridDim.x); wave w takes units 64w .. 64w+63 of every row, one per lane,
// with that unit's input slice read straight from global memory into registers once (no LDS staging) and the
// weight reads of the next NBUF - 1 rows in flight.  Each step's wave sum (team_sum over the 64 lanes) is kept
// in register lane k for the wave's k-th row; every 64 rows and at the end the KS partial sums of each row
// meet in LDS and are added in slice order starting from zero, ((0 + p_0) + p_1) + ..., which is how the
// few-token long-row kernel forms each token's sum.
// EXT: rows of several matrices scheduled as one (segments, nmq_mv_multi), each output as a launch of its
// matrix alone gives it.
template <int F, int KS, int NBUF, bool EXT, bool HR = false>
__global__ __launch_bounds__(256) void mvk_kernel(MvParams p) {
    args_early<EXT>(p);
    using FM = Fmt<F>;
    static_assert(F != NMQ_IQ2_XXS, "the grid table is staged by the LDS kernels only");
    static_assert(!HR || (mvk_hand(F) && !EXT), "hand-issued reads: Q4_K, TQ2_0, Q6_K, without segments");
    __shared__ float part[KS][64];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const RowMap rm = row_map<EXT>(p, p.w, p.y);
    const int U = (p.n_in + 63) >> 6;
    const int u = 64 * w + lane, uc = min(u, U - 1);
    const int G = gridDim.x;
    XSlice x[1];
    if constexpr (!HR) load_slice<FM::STRIDED>(p.xq, p.xq2, p.xd, p.xs, uc, x[0]);
    const u64* tab = nullptr;
    float res = 0.f;
    int r = blockIdx.x;
    int k = 0, first = r;
    // the KS partial sums of the batch's k rows, added in slice order from zero (a macro rather than a
    // lambda: a lambda capturing the row map by reference made the compiler keep the map in scratch)
#define NMQ_MVK_FLUSH()                                                           \
    do {                                                                          \
        part[w][lane] = res;                                                      \
        lds_barrier();                                                            \
        if (threadIdx.x < (unsigned)k) {                                          \
            float sum = 0.f;                                                      \
            _Pragma("unroll") for (int q = 0; q < KS; ++q) sum += part[q][threadIdx.x]; \
            *gpw<float>(rm.out(first + (int)threadIdx.x * G)) = sum;             \
        }                                                                         \
        lds_barrier();                                                            \
        k = 0;                                                                    \
        first = r;                                                                \
    } while (0)
    if constexpr (HR) {
        // The reads of every step are issued by hand (with buffers rotating through the loop the compiler
        // waits for all outstanding reads at its head) and each step waits for its own reads only.  The code
        // from a read to its wait is straight-line: the loop leaves by a branch taken before any read of the
        // step is issued, and every flush and the exit first wait for all outstanding reads.
        // The input slice is read by hand too, ahead of the first weight steps, and waited for with them out.
        using HS = HandStep<F, 1>;
        constexpr int HW = HS::NL * (NBUF - 1);
        HS hb[NBUF];
        {
            SliceAsm<FM::STRIDED> sl;
            sl.load(p.xq, p.xq2, p.xd, p.xs, uc);
#pragma unroll
            for (int i = 0; i < NBUF - 1; ++i) hb[i].template load<64>(rm, r + i * G, u, U, r);
            sl.template wait<HW>();
            sl.unpack(x[0]);
        }
        const LaneConst lc = lane_const<F, 64, 1>(u, x);
        bool more = true;
        while (more) {
#pragma unroll
            for (int i = 0; i < NBUF; ++i) {
                if (r >= p.n_out) {  // workgroup-uniform
                    more = false;
                    break;
                }
                hb[(i + NBUF - 1) % NBUF].template load<64>(rm, r + (NBUF - 1) * G, u, U, r);
                hb[i].template wait<HW>();
                const float v = unit_dot1<F, true>(hb[i].raw[0], uc, tab, x[0], lc, 0);
                const float ws = team_sum<64>(u < U ? v : 0.f);
                res = lane == k ? ws : res;
                r += G;
                if (++k == 64) {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    NMQ_MVK_FLUSH();
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the surplus reads of the last steps
        if (k > 0) NMQ_MVK_FLUSH();
        return;
    }
    Mv1Step<F, 64, 1, 1> buf[NBUF];
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i) buf[i].load(rm, r + i * G, u, U, r);
    const LaneConst lc = lane_const<F, 64, 1>(u, x);
    for (;;) {
#pragma unroll
        for (int i = 0; i < NBUF; ++i) {
            const bool more = r < p.n_out;  // workgroup-uniform
            if (more) {
                buf[(i + NBUF - 1) % NBUF].load(rm, r + (NBUF - 1) * G, u, U, r);
                const float v = unit_dot1<F, true>(buf[i].raw[0][0], uc, tab, x[0], lc, 0);
                const float ws = team_sum<64>(u < U ? v : 0.f);
                res = lane == k ? ws : res;
                ++k;
                r += G;
            }
            if (k == 64 || (!more && k > 0)) NMQ_MVK_FLUSH();  // a batch of rows
            if (!more) return;
        }
    }
#undef NMQ_MVK_FLUSH
}

template <int F, bool EXT, bool HR, int NBUF = 3>
inline MvKernel pick_mvk_e(int ks) {
    return ks == 2 ? mvk_kernel<F, 2, NBUF, EXT, HR>
                   : (ks == 3 ? mvk_kernel<F, 3, NBUF, EXT, HR> : mvk_kernel<F, 4, NBUF, EXT, HR>);
}
// Hand-issued reads only without segments: the first GPU run of the segment variant with them
// (nmq_mv_multi over long Q6_K rows) faulted, and its cause is not known; the segment variant keeps the
// compiler-scheduled reads.
template <int F>
inline MvKernel pick_mvk(int ks, bool ext, bool hr) {
    if constexpr (F == NMQ_IQ2_XXS) return nullptr;
    else if constexpr (mvk_hand(F))
        return ext ? pick_mvk_e<F, true, false>(ks)
                   : (hr ? (tune(TUNE_MVK_NBUF, 3) == 4 ? pick_mvk_e<F, false, true, 4>(ks) : pick_mvk_e<F, false, true>(ks))
                         : pick_mvk_e<F, false, false>(ks));
    else return ext ? pick_mvk_e<F, true, false>(ks) : pick_mvk_e<F, false, false>(ks);
}

// ---- 2..4 tokens, long rows (Q6_K: the layer's down projection) ---------------------------------------
// LDS bytes per token of the few-token long-row kernel: xq and xq2 (ktp each, stage1_store's strided
// layout), xd / 254 per 32-value group (ktp / 32 floats), the xq2 chain start -32 (254 X1 + X2) of every
// 16-value group (ktp / 16 ints, the four of a unit together).
__host__ __device__ constexpr int q6k_tok_bytes(int ktp) { return 2 * ktp + ktp / 8 + ktp / 4; }

// One token's staging round in that layout.  The thread holding chunk i (values 16i .. 16i + 15, one
// Q6_K group: i = 16b + 8h + 2g + j for group g of unit u = 4b + 2h + j) forms its group constant from
// the registers it is about to store, so the constants cost no LDS pass of their own.
__device__ __forceinline__ void stage_q6k_store(const XRound& r, u8* lds, int n_in, int ktp) {
    const int i = threadIdx.x;
    if (i < ktp / 16) {
        const bool ok = 16 * i < n_in;
        const u32x4 a = ok ? r.a : u32x4{0u, 0u, 0u, 0u}, b = ok ? r.b : u32x4{0u, 0u, 0u, 0u};
        const int ph = swz<true>(i);
        *(u32x4*)(lds + 16 * ph) = a;
        *(u32x4*)(lds + ktp + 16 * ph) = b;
        const int u = ((i >> 4) << 2) | (((i >> 3) & 1) << 1) | (i & 1);
        ((int*)(lds + 2 * ktp + ktp / 8))[4 * u + ((i >> 1) & 3)] =
            q6k_group_const(a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w);
    }
    if (i < ktp / 32) ((float*)(lds + 2 * ktp))[i] = i < n_in / 32 ? r.d * FEIN : 0.f;
}

// Q6_K unit u for NC tokens staged by stage_q6k_store: the 64 codes and the four scales decoded once,
// each token's groups formed with q6k_dot1's integers and fp32 operations in its order, so v[t] equals
// q6k_dot1 on token t bit for bit.
template <int NC>
__device__ __forceinline__ void q6k_dotn_lds(const Fmt<NMQ_Q6_K>::Raw& r, const u8* lds, int tok, int ktp, int u,
                                             float (&v)[NC]) {
    const u32 la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
    const u32 lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
    const u32 qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    u32 c[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        c[0][k] = q6k_codes<0>(la[k], qh[k]);
        c[1][k] = q6k_codes<1>(lb[k], qh[k]);
        c[2][k] = q6k_codes<2>(la[k], qh[k]);
        c[3][k] = q6k_codes<3>(lb[k], qh[k]);
    }
    const u32 sh = 8u * (u32)(u & 1);
    float sc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) sc[g] = (float)(int8_t)bfe(g < 2 ? r.sc.x : r.sc.y, sh + 16u * (u32)(g & 1), 8);
    const float d = h2f(r.d);
    const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
#pragma unroll
    for (int t = 0; t < NC; ++t) {
        const u8* base = lds + t * tok;
        const float4 xd = *(const float4*)((const float*)(base + 2 * ktp) + 8 * b + 4 * h);
        const u32x4 kc = *(const u32x4*)((const int*)(base + 2 * ktp + ktp / 8) + 4 * u);
        const float e[4] = {xd.x, xd.y, xd.z, xd.w};
        const int k0[4] = {(int)kc.x, (int)kc.y, (int)kc.z, (int)kc.w};
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int ph = swz<true>(16 * b + 8 * h + 2 * g + j);
            const u32x4 xa = *(const u32x4*)(base + 16 * ph);
            const u32x4 xc = *(const u32x4*)(base + ktp + 16 * ph);
            int s1 = dot4(c[g][0], xa.x, 0), s2 = dot4(c[g][0], xc.x, k0[g]);
            s1 = dot4(c[g][1], xa.y, s1); s2 = dot4(c[g][1], xc.y, s2);
            s1 = dot4(c[g][2], xa.z, s1); s2 = dot4(c[g][2], xc.z, s2);
            s1 = dot4(c[g][3], xa.w, s1); s2 = dot4(c[g][3], xc.w, s2);
            acc = fmaf((float)(__mul24(s1, 254) + s2), sc[g] * e[g], acc);
        }
        v[t] = acc * d;
    }
}

// The long-row kernel for NC tokens: one row per wave in 16-wave workgroups (one per CU with the NC
// staged inputs, 34 KB each for 14336 values), all of the row's weights requested at once, every token's
// input staged in LDS (one round each, read before the weight reads, stored after them), each unit's
// codes decoded once for all tokens, and each token's sum formed exactly as the one-token K-split kernel
// forms it (q6k_dot1's terms per unit, team_sum per 64-unit slice, slices added in order from zero):
// every output equals the one-token launch on that token bit for bit.
template <int NC, int NIT>
__global__ __launch_bounds__(1024) void mvlt_kernel(MvParams p) {
    args_early<false>(p);
    constexpr int F = NMQ_Q6_K;
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = p.nt >> 6;
    const RowMap rm = row_map<false>(p, p.w, p.y);
    const int U = (p.n_in + 63) >> 6;
    const int row = blockIdx.x * W + wave;
    const int tok = q6k_tok_bytes(p.ktp);
    Mv1Step<F, 64, 1, NIT> a;
    {
        XRound r[NC];
        const int64_t g = p.n_in / 32;
#pragma unroll
        for (int t = 0; t < NC; ++t)
            stage1_load(r[t], 0, p.xq + t * p.n_in, p.xq2 + t * p.n_in, p.xd + t * g, p.xs + t * g, p.n_in, p.nt);
        __builtin_amdgcn_sched_barrier(0);  // the input reads ahead of the weight reads
        a.load(rm, row, lane, U, row);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NC; ++t) stage_q6k_store(r[t], lds + t * tok, p.n_in, p.ktp);
        lds_barrier();
    }
    if (row >= p.n_out) return;  // wave-uniform, after the workgroup's last barrier
    float acc[NC];
#pragma unroll
    for (int t = 0; t < NC; ++t) acc[t] = 0.f;
    // each 64-unit slice's sum over the wave first, then the slices in order from zero: the order of the
    // one-token K-split kernel (mvk_kernel), so every token's output equals the one-token launch
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int u = lane + it * 64;
        const int uc = min(u, U - 1);
        float v[NC];
        q6k_dotn_lds<NC>(a.raw[0][it], lds, tok, p.ktp, uc, v);
#pragma unroll
        for (int t = 0; t < NC; ++t) v[t] = u < U ? v[t] : 0.f;
        team_sum64_n<NC>(v);
#pragma unroll
        for (int t = 0; t < NC; ++t) acc[t] += v[t];
        __builtin_amdgcn_sched_barrier(0);  // one unit's codes live at a time
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < NC; ++t) gpw<float>(p.y)[(int64_t)t * p.n_out + row] = acc[t];
    }
}

template <int F, bool EXT>
inline MvKernel pick_mvl_e(int nit, bool pipe) {
    if (nit == 3) return pipe ? mvl_kernel<F, 1, 3, true, EXT> : mvl_kernel<F, 1, 3, false, EXT>;
    return pipe ? mvl_kernel<F, 1, 4, true, EXT> : mvl_kernel<F, 1, 4, false, EXT>;
}
template <int F>
inline MvKernel pick_mvl(int nit, bool pipe, bool ext) {
    return ext ? pick_mvl_e<F, true>(nit, pipe) : pick_mvl_e<F, false>(nit, pipe);
}

template <int F, int T, bool EXT>
inline MvKernel pick_mvc_rw(int rw) {
    switch (rw) {
        case 1: return mvc_kernel<F, T, 1, EXT>;
        case 2: return mvc_kernel<F, T, 2, EXT>;
        case 4: return mvc_kernel<F, T, 4, EXT>;
        default: return mvc_kernel<F, T, 8, EXT>;
    }
}
template <int F, bool EXT>
inline MvKernel pick_mvc_e(int T, int rw) {
    switch (T) {
        case 16: return pick_mvc_rw<F, 16, EXT>(rw);
        case 32: return pick_mvc_rw<F, 32, EXT>(rw);
        default: return pick_mvc_rw<F, 64, EXT>(rw);
    }
}
template <int F>
inline MvKernel pick_mvc(int T, int rw, bool ext) {
    return ext ? pick_mvc_e<F, true>(T, rw) : pick_mvc_e<F, false>(T, rw);
}

// Chunk mode (mvc_kernel) for one token.  The rows are spread evenly over about one workgroup per
// CU (per instance for expert batches): rows per workgroup R = ceil(rows / WGs), then the smallest
// rows-per-team RW with R <= P*RW*16 (at most 16 waves, 8 when RW = 8), so every CU streams the
// same number of rows and all of them are in flight at once.
// values: the launch forms the input from values in its staging (more rounds the fewer threads a
// workgroup has), else it reads the two-stage input.
inline Mv1Shape plan_mvc(int n_out, int n_in, int n_mats, const DeviceInfo& di, bool values = true,
                          bool four_rows = false, bool wide_tab = false) {
    Mv1Shape s{};
    const int U = (n_in + 63) / 64;
    s.T = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
    if (U > s.T) return s;  // one unit per lane only
    const int P = 64 / s.T;
    // two-stage input, formats without the four-row teams (Q8_0, Q4_0, Q6_K), at least 16 rows per CU: 4
    // workgroups per CU (measured on MI355X, one token: 4096x4096 Q8_0 6.15 -> 5.66 us, Q4_0 5.16 -> 4.54,
    // Q6_K 5.90 -> 5.14; 6144x4096 Q8_0 8.24 -> 7.30; but 1024x4096 Q8_0 2.92 -> 3.86, so not below 16 rows
    // per CU; IQ2_XXS 4096x4096 4.22 against 4.40)
    const bool quad = !values && !four_rows && !wide_tab && (int64_t)n_out * n_mats >= (int64_t)16 * di.cus;
    const int wg_per_cu = tune(TUNE_MVC_WGPC, quad ? 4 : 1);
    int64_t wgs = (int64_t)di.cus * wg_per_cu / n_mats;
    if (wgs < 1) wgs = 1;
    const int64_t R = ((int64_t)n_out + wgs - 1) / wgs;  // rows per workgroup
    int rw = tune(TUNE_MVC_RW, 0);
    if (rw <= 0 && !values && four_rows) {
        rw = 4;  // two-stage input, Q4_K / TQ2_0: 4 rows per team, fewer waves per workgroup (measured on
                 // MI355X: Q4_K 4096x4096 4.1 against 4.7 us, TQ2_0 4.2 against 4.4 us; Q8_0 and IQ2_XXS
                 // were slower)
    } else if (rw <= 0) {
        rw = 1;
        while (rw < 8 && R > (int64_t)P * rw * 16) rw *= 2;
    }
    rw = rw <= 1 ? 1 : (rw <= 2 ? 2 : (rw <= 4 ? 4 : 8));  // the instantiated widths
    const int wmax = rw >= 8 ? 8 : 16;
    int64_t W = (R + P * rw - 1) / (P * rw);
    if (W > wmax) W = wmax;
    if (W < 1) W = 1;
    s.rw = rw;
    s.W = (int)W;
    const int64_t rows_wg = (int64_t)P * rw * W;
    s.grid_x = (int)((n_out + rows_wg - 1) / rows_wg);
    s.ktp = (n_in + 127) / 128 * 128;
    s.lds = (size_t)s.ktp * 9 / 4;
    s.ok = s.lds <= (size_t)di.lds_max;
    return s;
}

inline int seg_start_host(const MvParams& p, int i) { return i == 0 ? 0 : p.seg_end[i - 1]; }

// One launch of NC <= NMQ_MAX_COLS tokens (n_mats instances along blockIdx.y).
template <int F>
int launch_mv(MvParams p, int nc, int n_mats, hipStream_t stream) {
    using FM = Fmt<F>;
    const DeviceInfo di = device_info();
    p.nblk = p.n_in / FM::BV;
    p.row_bytes = (int64_t)p.nblk * FM::BB;
    // 2..16 tokens of one matrix: the matrix cores (see nmq_mfma.hpp); more than 8 tokens that cannot
    // go there in one launch run as two launches of at most 8
    if (nc > 8) {
        // where the dense-read kernel takes 8 tokens, two launches of it beat one matrix-core launch of
        // both groups (14336x4096 at 16 tokens: Q4_0 52.1 -> 22.9 us, Q8_0 60.6 -> 33.2, Q4_K 24.9 -> 20.5,
        // TQ2_0 19.5 -> 16.1, IQ2_XXS 27.4 -> 24.7)
        const MvmShape sm = plan_mvm<F>(p.n_out, p.n_in, nc, di.cus, di.lds_max_big);
        const bool dense8 = p.ids == nullptr && (plan_mvd<F>(p.n_out, p.n_in, 8, di.cus, di.lds_max_big, p.w).ok ||
                                                 (tune(TUNE_MVD_LONG, 1) == 1 &&
                                                  plan_mvd_long<F>(p.n_out, p.n_in, 8, di.cus, di.lds_max_big, p.w,
                                                                   p.row_bytes).ok));
        if (!(sm.ok && p.ids == nullptr) || dense8) {
            int e = launch_mv<F>(p, 8, n_mats, stream);
            if (e) return e;
            MvParams q = p;
            q.xq += (int64_t)8 * p.n_in;
            q.xq2 += (int64_t)8 * p.n_in;
            q.xd += (int64_t)8 * (p.n_in / 32);
            q.xs += (int64_t)8 * (p.n_in / 32);
            q.y += (int64_t)8 * p.n_out;
            return launch_mv<F>(q, nc - 8, n_mats, stream);
        }
    }
    // The dense-read matrix-core kernel: from 2 tokens, Q4_K from 5 (MVD_MIN; at 4 tokens it beats the
    // few-token loop below, 14336x4096 10.6 against 12.9 us, but 2..4 tokens keep outputs equal to
    // one-token launches bit for bit)
    {
        if (nc >= 2 && p.ids == nullptr) {
            const MvdShape sd = plan_mvd<F>(p.n_out, p.n_in, nc, di.cus, di.lds_max_big, p.w);
            if (sd.ok) {
                MvmParams q{};
                q.w = p.w; q.xq = p.xq; q.xq2 = p.xq2; q.xd = p.xd; q.xs = p.xs; q.y = p.y;
                q.n_out = p.n_out; q.n_in = p.n_in; q.nc = nc;
                q.row_bytes = p.row_bytes;
                q.nblk = p.n_in / 256;
                return launch_mvd<F>(sd, q, stream);
            }
        }
    }
    if constexpr (F == NMQ_Q4_K) {
        // 2..NMQ_MVT_MAX (default 4) tokens of one matrix: the one-token kernel's loop for all of them
        // (one unit per lane: rows of up to 4096 values; the NC input slices take about 65 + 34 NC VGPRs
        // (133 for 2 tokens, 174 for 3, 227 for 4), so 4-wave workgroups at 12 waves per CU for 2 tokens,
        // 8 for 3 and 4)
        if (nc >= 2 && nc <= tune(TUNE_MVT_MAX, 4) && nc <= 4 && p.ids == nullptr && p.xv == nullptr &&
            p.n_seg == 0) {
            const int U = (p.n_in + 63) / 64;
            const int T = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
            const int P = 64 / T;
            const int ktp = (p.n_in + 127) / 128 * 128;
            const size_t lds = (size_t)nc * ktp * 9 / 4;
            const int W = 4;
            const int64_t steps = ((int64_t)p.n_out + P - 1) / P;
            int64_t waves = (int64_t)tune(TUNE_MVT_WPC, nc == 2 ? 12 : 8) * di.cus;
            if (waves > steps) waves = steps;
            if (U <= 64 && ktp / 16 <= 64 * W && lds <= (size_t)di.lds_max) {
                p.ktp = ktp;
                p.nt = 64 * W;
                MvKernel k = nc == 2 ? pick_mvt<2>(T) : (nc == 3 ? pick_mvt<3>(T) : pick_mvt<4>(T));
                hipLaunchKernelGGL(k, dim3((unsigned)((waves + W - 1) / W)), dim3(p.nt), lds, stream, p);
                return (int)hipGetLastError();
            }
        }
    }
    if constexpr (F == NMQ_Q6_K) {
        // 2..4 tokens of one matrix with long rows (129..256 units): the long-row loop for all of them
        if (nc >= 2 && nc <= tune(TUNE_MVLT_MAX, 4) && nc <= 4 && p.ids == nullptr && p.xv == nullptr &&
            p.n_seg == 0) {
            const int U = (p.n_in + 63) / 64;
            const int ktp = (p.n_in + 127) / 128 * 128;
            const size_t lds = (size_t)nc * q6k_tok_bytes(ktp);
            const int W = 16;
            if (U > 128 && U <= 256 && ktp / 16 <= 64 * W && lds + 4096 <= (size_t)di.lds_max_big) {
                p.ktp = ktp;
                p.nt = 64 * W;
                const bool n3 = U <= 192;  // units per lane: 3 or 4
                MvKernel k = nc == 2 ? (n3 ? mvlt_kernel<2, 3> : mvlt_kernel<2, 4>)
                           : nc == 3 ? (n3 ? mvlt_kernel<3, 3> : mvlt_kernel<3, 4>)
                                     : (n3 ? mvlt_kernel<4, 3> : mvlt_kernel<4, 4>);
                hipLaunchKernelGGL(k, dim3((unsigned)((p.n_out + W - 1) / W)), dim3(p.nt), lds, stream, p);
                return (int)hipGetLastError();
            }
        }
    }
    // Rows beyond the dense kernel's 4096 values, 2..8 tokens of one matrix (Q6_K: from 5, after the
    // few-token long-row kernel above): K ranges of 4096 values (the last one shorter), one dense launch
    // each, in range order on the stream, each adding its sums to y (the first writes it), so the
    // result does not depend on timing.  The rows and the ranges must start on 16-byte boundaries.
    if (nc >= 2 && nc <= 8 && p.ids == nullptr && p.xv == nullptr && p.n_seg == 0 && p.n_in > 4096 &&
        tune(TUNE_MVD_LONG, 1) == 1) {
        const MvdShape sl = plan_mvd_long<F>(p.n_out, p.n_in, nc, di.cus, di.lds_max_big, p.w, p.row_bytes);
        if (sl.ok) {
            MvmParams q{};
            q.w = p.w; q.xq = p.xq; q.xq2 = p.xq2; q.xd = p.xd; q.xs = p.xs; q.y = p.y;
            q.n_out = p.n_out; q.n_in = p.n_in; q.nc = nc;
            q.row_bytes = p.row_bytes;
            q.nblk = p.n_in / 256;
            return launch_mvd_long<F>(sl, q, stream);
        }
    }
    if (nc >= 2 && nc <= 8 && p.ids == nullptr && p.xv == nullptr && p.n_seg == 0 && p.n_in > 4096 &&
        p.n_in <= 8 * 4096 && p.row_bytes % 16 == 0 && tune(TUNE_MVD_LONG, 1) != 0) {
        constexpr int R = 4096;
        const int nr = (p.n_in + R - 1) / R;
        MvdShape sh[8];
        bool ok = true;
        for (int j = 0; j < nr && ok; ++j) {
            const int k0 = j * R, len = p.n_in - k0 < R ? p.n_in - k0 : R;
            const int64_t off = (int64_t)(k0 / 256) * Mfma<F>::BB;
            sh[j] = plan_mvd<F>(p.n_out, len, nc, di.cus, di.lds_max_big, p.w + off, 2);
            ok = sh[j].ok && off % 16 == 0;
        }
        if (ok) {
            for (int j = 0; j < nr; ++j) {
                const int k0 = j * R, len = p.n_in - k0 < R ? p.n_in - k0 : R;
                MvmParams q{};
                q.w = p.w + (int64_t)(k0 / 256) * Mfma<F>::BB;
                q.xq = p.xq + k0; q.xq2 = p.xq2 + k0; q.xd = p.xd + k0 / 32; q.xs = p.xs + k0 / 32; q.y = p.y;
                q.n_out = p.n_out; q.n_in = len; q.nc = nc;
                q.row_bytes = p.row_bytes;
                q.nblk = len / 256;
                q.x_stride = p.n_in;
                q.acc_y = j > 0;
                const int e = launch_mvd<F>(sh[j], q, stream);
                if (e) return e;
            }
            return 0;
        }
    }
    if (nc >= 2 && p.ids == nullptr) {
        const MvmShape sm = plan_mvm<F>(p.n_out, p.n_in, nc, di.cus, di.lds_max_big);
        if (sm.ok) {
            MvmParams q{};
            q.w = p.w; q.xq = p.xq; q.xq2 = p.xq2; q.xd = p.xd; q.xs = p.xs; q.y = p.y;
            q.n_out = p.n_out; q.n_in = p.n_in; q.nc = nc;
            q.row_bytes = p.row_bytes;
            q.nblk = p.n_in / 256;
            return launch_mvm<F>(sm, q, stream);
        }
    }
    // One token: chunk mode while the rows per CU are few (every weight in flight at once), the
    // persistent prefetching kernel for larger matrices (measured on MI355X: chunk mode is faster up
    // to 4096 rows of 4096 values, the persistent kernel from 12288 rows).
    const bool ext = p.n_seg > 0 || p.xv != nullptr;  // the kernel variant with segments / value input
    const int64_t rows_per_cu = ((int64_t)p.n_out * n_mats + di.cus - 1) / di.cus;
    // rows per CU up to which chunk mode runs: 24 for one matrix, 64 for gathered experts (MoE layer at
    // one token, both expert launches in chunk mode: 17.9 against 18.5 us; at 4 tokens both stay above)
    const int mvc_max = tune(TUNE_MVC_ROWS, n_mats > 1 ? 64 : 24);
    const int mode = tune(TUNE_MV1_MODE, rows_per_cu > mvc_max ? 2 : 1);
    if (nc == 1 && mode == 1) {
        const Mv1Shape sc = plan_mvc(p.n_out, p.n_in, n_mats, di, p.xv != nullptr, F == NMQ_Q4_K || F == NMQ_TQ2_0,
                                     F == NMQ_IQ2_XXS);
        if (sc.ok) {
            p.ktp = sc.ktp;
            MvKernel k = pick_mvc<F>(sc.T, sc.rw, ext);
            p.nt = 64 * sc.W;
            hipLaunchKernelGGL(k, dim3((unsigned)sc.grid_x, (unsigned)n_mats), dim3(p.nt), sc.lds, stream, p);
            return (int)hipGetLastError();
        }
    }
    if constexpr (F != NMQ_IQ2_XXS) {
        // one token over rows of 129..256 units from the two-stage input: the K-split kernel (the long-row
        // kernel below stays for value input, experts and IQ2_XXS)
        const int U = (p.n_in + 63) / 64;
        if (nc == 1 && U > 128 && U <= 256 && p.ids == nullptr && p.xv == nullptr && tune(TUNE_MVK, 1) != 0) {
            const int ks = (U + 63) / 64;
            // Hand-issued reads (no segments, Q4_K / TQ2_0 / Q6_K): whole workgroups of about 4 waves per CU
            // (Q6_K 4096x14336, KS = 4: one workgroup per CU 11.2 us, against 12.7 at 8 waves per CU, 13.4 at
            // 3 and 16.0 at 5, where the workgroups do not divide evenly over the CUs, and 17.3 at 2); the
            // compiler-scheduled reads: 8 waves per CU (12.9 us).
            const bool hr = mvk_hand(F) && p.n_seg == 0 && tune(TUNE_MVK_HR, 1) != 0;
            const int wpc = tune(TUNE_MVK_WPC, 0);
            int64_t g = wpc > 0 ? (int64_t)wpc * di.cus / ks
                                : (hr ? (int64_t)di.cus * (ks >= 4 ? 1 : 4 / ks) : (int64_t)8 * di.cus / ks);
            if (g < 1) g = 1;
            if (g > p.n_out) g = p.n_out;
            p.nt = 64 * ks;
            hipLaunchKernelGGL(pick_mvk<F>(ks, p.n_seg > 0, hr), dim3((unsigned)g), dim3(p.nt), 0, stream, p);
            return (int)hipGetLastError();
        }
    }
    if (nc == 1) {
        const MvlShape sl = plan_mvl(p.n_out, p.n_in, n_mats, di);
        if (sl.ok) {
            p.ktp = sl.ktp;
            MvKernel k = pick_mvl<F>(sl.nit, sl.pipe, ext);
            p.nt = 64 * sl.W;
            hipLaunchKernelGGL(k, dim3((unsigned)sl.grid_x, (unsigned)n_mats), dim3(p.nt), sl.lds, stream, p);
            return (int)hipGetLastError();
        }
    }
    if (nc == 1 && mode != 0) {
        const Mv1Shape s1 = plan_mv1(p.n_out, p.n_in, n_mats, di, p.xv != nullptr);
        if (s1.ok) {
            p.ktp = s1.ktp;
            // Q4_K, TQ2_0, IQ2_XXS (with at least 256 threads: the grid table) with the two-stage input
            // staged in one round, or fp32 values in at most two: hand-issued reads (NMQ_MV1_HR=0 for the
            // compiler-scheduled loop)
            int hr = 0;
            if (hand_format(F) && s1.rw == 1 && (s1.nbuf == 3 || s1.nitm == 1) && s1.nitm <= 2 &&
                (F != NMQ_IQ2_XXS || s1.W >= 4) &&
                tune(TUNE_MV1_HR, 1) != 0) {
                if (p.xv == nullptr) hr = s1.ktp / 16 <= 64 * s1.W ? 1 : 0;
                else if (p.x_mode == NMQ_X_F32 || p.x_mode == NMQ_X_F32_BF16) hr = s1.ktp / 4 <= 2 * 64 * s1.W ? 2 : 0;
            }
            MvKernel k = pick_mv1<F>(s1.T, s1.rw, s1.nitm, s1.nbuf, ext, hr);
            p.nt = 64 * s1.W;
            hipLaunchKernelGGL(k, dim3((unsigned)s1.grid_x, (unsigned)n_mats), dim3(p.nt), s1.lds, stream, p);
            return (int)hipGetLastError();
        }
    }
    if (p.n_seg > 0) {  // the general kernel reads one matrix: one launch per segment
        for (int i = 0; i < p.n_seg; ++i) {
            MvParams q = p;
            q.n_seg = 0;
            q.w = p.seg_w[i];
            q.y = p.seg_y[i];
            q.n_out = (i + 1 < p.n_seg ? p.seg_end[i] : p.n_out) - seg_start_host(p, i);
            const int e = launch_mv<F>(q, nc, n_mats, stream);
            if (e) return e;
        }
        return 0;
    }
    if (p.xv) return NMQ_ERR_SHAPE;  // values are staged by the one-token kernels only
    const MvShape s = plan_mv<F>(p.n_out, p.n_in, nc, n_mats, di);
    p.kt = s.kt;
    p.ktp = s.ktp;
    p.n_tiles = s.n_tiles;
    p.groups = s.groups;
    MvKernel k = pick_kernel<F>(nc, s.rw, s.T);
    p.nt = 64 * s.W;
    hipLaunchKernelGGL(k, dim3((unsigned)s.grid_x, (unsigned)n_mats), dim3(p.nt), s.lds, stream, p);
    return (int)hipGetLastError();
}


// ---- the expert down projection with the weighted combine (moe_down_kernel) --------------------------
typedef void (*MoeDownKernel)(MvParams, Combine);

template <int F, int T>
inline MoeDownKernel pick_moe_down_rw(int rw) {
    switch (rw) {
        case 1: return moe_down_kernel<F, T, 1>;
        case 2: return moe_down_kernel<F, T, 2>;
        default: return moe_down_kernel<F, T, 4>;
    }
}

struct MoeDownShape {
    bool ok;
    int T, rw, ws, W, R, grid_x, ktp;
    size_t lds;
};

// Waves per slot WS (W = k*WS <= 16) and rows per team RW: about 256 workgroups per launch when the rows
// allow it (R = WS*P*RW rows per workgroup), one unit per lane (rows of up to T*64 values).
inline MoeDownShape plan_moe_down(int n_out, int n_in, int L, int k, const DeviceInfo& di) {
    MoeDownShape s{};
    const int U = (n_in + 63) / 64;
    s.T = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
    if (U > s.T || k < 1 || k > 16) return s;
    const int P = 64 / s.T;
    s.ws = 16 / k >= 2 ? 2 : 1;
    if (s.ws > 16 / k) return s;
    s.W = k * s.ws;
    int64_t R = ((int64_t)n_out * L + di.cus - 1) / di.cus;  // rows per workgroup for ~one per CU
    s.rw = 1;
    while (s.rw < 4 && R > (int64_t)s.ws * P * s.rw) s.rw *= 2;
    s.R = s.ws * P * s.rw;
    s.grid_x = (n_out + s.R - 1) / s.R;
    s.ktp = (n_in * k + 127) / 128 * 128;
    s.lds = (size_t)s.ktp * 9 / 4 + (size_t)k * s.R * 4;
    s.ok = s.lds <= (size_t)di.lds_max && n_in % 64 == 0;
    return s;
}

// One launch (value input, x_group = 1).  NMQ_ERR_SHAPE when the kernel does not take the shape.
template <int F>
int launch_moe_down(MvParams p, Combine c, int L, hipStream_t stream) {
    using FM = Fmt<F>;
    const DeviceInfo di = device_info();
    const MoeDownShape sh = plan_moe_down(p.n_out, p.n_in, L, c.k, di);
    if (!sh.ok) return NMQ_ERR_SHAPE;
    p.nblk = p.n_in / FM::BV;
    p.row_bytes = (int64_t)p.nblk * FM::BB;
    p.ktp = sh.ktp;
    p.nt = 64 * sh.W;
    c.ws = sh.ws;
    const MoeDownKernel kern = sh.T == 16 ? pick_moe_down_rw<F, 16>(sh.rw)
                             : sh.T == 32 ? pick_moe_down_rw<F, 32>(sh.rw) : pick_moe_down_rw<F, 64>(sh.rw);
    hipLaunchKernelGGL(kern, dim3((unsigned)sh.grid_x, (unsigned)L), dim3(p.nt), sh.lds, stream, p, c);
    return (int)hipGetLastError();
}


// ---- gate and up projections with the gated activation (moe_gu_kernel) ----------------------------------
typedef void (*MoeGuKernel)(MvParams, QuantOut);

// One launch over the p.n_ids slots (value input).  T lanes per row with one unit each (rows of up to
// 4096 values) and RW rows per team: 32 rows of a projection take 32 / (P*RW) waves, so a workgroup has
// 2 to 16.  While the workgroups fit one per CU, the smaller RW (more waves per workgroup); with more, the
// larger (more workgroups resident per CU, one's weight reads overlapping another's compute).
// NMQ_ERR_SHAPE for longer rows or n_out not a multiple of 32 (a group of the output is one workgroup's).
template <int F>
int launch_moe_gu(MvParams p, QuantOut o, hipStream_t stream) {
    using FM = Fmt<F>;
    const DeviceInfo di = device_info();
    const int U = (p.n_in + 63) / 64;
    const int T = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
    if (U > T || p.n_out % 32 || p.n_ids < 1 || p.n_ids > 65535) return NMQ_ERR_SHAPE;
    const int P = 64 / T;
    const int64_t wgs = (int64_t)(p.n_out / 32) * p.n_ids;
    const int lo = T == 64 ? 4 : 2;
    int rw = tune(TUNE_MOE_GU_RW, wgs <= di.cus ? lo : 2 * lo);
    rw = rw <= lo ? lo : 2 * lo;
    p.nblk = p.n_in / FM::BV;
    p.row_bytes = (int64_t)p.nblk * FM::BB;
    p.ktp = (p.n_in + 127) / 128 * 128;
    p.nt = 64 * (2 * 32 / (P * rw));
    const size_t lds = (size_t)p.ktp * 9 / 4;
    if (lds > (size_t)di.lds_max || p.ktp / 4 > 2 * p.nt) return NMQ_ERR_SHAPE;
    const bool big = rw > lo;
    const MoeGuKernel k = T == 16 ? (big ? moe_gu_kernel<F, 16, 4> : moe_gu_kernel<F, 16, 2>)
                        : T == 32 ? (big ? moe_gu_kernel<F, 32, 4> : moe_gu_kernel<F, 32, 2>)
                                  : (big ? moe_gu_kernel<F, 64, 8> : moe_gu_kernel<F, 64, 4>);
    hipLaunchKernelGGL(k, dim3((unsigned)(p.n_out / 32), (unsigned)p.n_ids), dim3(p.nt), lds, stream, p, o);
    return (int)hipGetLastError();
}


// ---- gate|up with the activation of a dense FFN (mvp_kernel) --------------------------------------------
typedef void (*MvpKernel)(MvParams, QuantOut);

// One launch: p.w gate, p.w2 up (n_out x n_in each), fp32 input values (NMQ_X_F32 / NMQ_X_F32_BF16; the
// kernel also takes the two-stage input, HR = 1, which no entry point passes yet).  NMQ_ERR_SHAPE where
// the kernel does not apply: other formats or input modes, rows of more than 4096 values, n_out not a
// multiple of 32.  16 waves of 4 rows per group (NMQ_MVP_RPW = 4) or 8 of 8; workgroups: the fewest groups
// per workgroup that the CUs allow, spread evenly (NMQ_MVP_WGS overrides).  Measured on MI355X, Llama-3-8B
// gate|up 14336x4096 Q4_K: 14.3 us at 16 waves and 2 groups per workgroup (224 workgroups), 14.7 at 256
// workgroups (1 or 2 groups), 18.4 at 448 (one each), 15.3 with 8 waves; the gathered launch alone takes
// 14.4-14.5 us and with the activation launch after it 16.8-17.3.
template <int F>
int launch_mvp(MvParams p, QuantOut o, hipStream_t stream) {
    if constexpr (!hand_format(F)) {
        return NMQ_ERR_SHAPE;
    } else {
        using FM = Fmt<F>;
        const DeviceInfo di = device_info();
        const int U = (p.n_in + 63) / 64;
        if (U > 64 || p.n_out % 32 || p.n_out < 32) return NMQ_ERR_SHAPE;
        if (!p.xv || (p.x_mode != NMQ_X_F32 && p.x_mode != NMQ_X_F32_BF16)) return NMQ_ERR_SHAPE;
        const int rpw = tune(TUNE_MVP_RPW, 4) == 8 ? 8 : 4;
        p.nt = 64 * (64 / rpw);
        p.nblk = p.n_in / FM::BV;
        p.row_bytes = (int64_t)p.nblk * FM::BB;
        p.ktp = (p.n_in + 127) / 128 * 128;
        const size_t lds = (size_t)p.ktp * 9 / 4;
        if (lds > (size_t)di.lds_max || p.ktp / 4 > 2 * p.nt) return NMQ_ERR_SHAPE;
        const int G = p.n_out / 32;
        const int per = (G + di.cus - 1) / di.cus;  // groups per workgroup
        int nb = tune(TUNE_MVP_WGS, (G + per - 1) / per);
        nb = nb < 1 ? 1 : (nb > G ? G : nb);
        if ((G + nb - 1) / nb > MVP_MAXG) nb = (G + MVP_MAXG - 1) / MVP_MAXG;
        const MvpKernel k = rpw == 8 ? mvp_kernel<F, 2, 8> : mvp_kernel<F, 2, 4>;
        hipLaunchKernelGGL(k, dim3((unsigned)nb), dim3(p.nt), lds, stream, p, o);
        return (int)hipGetLastError();
    }
}

}  // namespace nmq
