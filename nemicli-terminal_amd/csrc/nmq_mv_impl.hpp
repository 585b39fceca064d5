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

#include "nmq_device.hpp"

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
};

// 16-byte chunk permutations of the LDS input (bijective inside every aligned group of 8 chunks).
template <bool STRIDED>
__device__ __forceinline__ int swz(int ch) {
    return STRIDED ? (ch ^ (((ch >> 3) & 3) << 1)) : (ch ^ ((ch >> 3) & 7));
}

template <bool STRIDED>
__device__ __forceinline__ void stage_tile(u8* lds, const int8_t* xq, const int8_t* xq2, const float* xd,
                                           const float* xs, int n_in, int nc, int k0, int kt, int ktp) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int tok = (ktp * 9) / 4;
    for (int c = 0; c < nc; ++c) {
        u8* base = lds + c * tok;
        const int8_t* q = xq + (int64_t)c * n_in + k0;
        const int8_t* q2 = xq2 + (int64_t)c * n_in + k0;
        for (int ch = tid; ch < ktp / 16; ch += nt) {
            u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
            if (ch * 16 < kt) {
                a = *(const u32x4*)(q + 16 * ch);
                b = *(const u32x4*)(q2 + 16 * ch);
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
            d[i] = ok ? xd[g0 + i] : 0.f;
            s[i] = ok ? xs[g0 + i] : 0.f;
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

template <int F>
__device__ __forceinline__ void fill_tables(u64* tab) {
    if (F == NMQ_IQ2_XXS) {
        for (int i = threadIdx.x; i < 384; i += blockDim.x)
            tab[i] = i < 256 ? IQ2XXS_GRID[i] : iq2_sign_mask((u32)(i - 256));
    }
}

template <int F, int NC, int T, int RW>
__global__ __launch_bounds__(256) void mv_kernel(MvParams p) {
    using FM = Fmt<F>;
    constexpr bool S = FM::STRIDED;
    constexpr int P = 64 / T;
    extern __shared__ __attribute__((aligned(16))) u8 lds[];
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, W = blockDim.x >> 6;
    const int team = lane / T, lt = lane % T;
    const int m = blockIdx.y;

    const u8* wbase = p.w;
    int64_t xrow = 0;
    if (p.ids) {
        const int64_t e = p.ids[m];
        wbase = p.per_expert >= 0 ? p.w + e * p.per_expert : (const u8*)(((const int64_t*)p.w)[e]);
        xrow = m / p.x_group;
    }
    const int8_t* xq = p.xq + xrow * p.n_in;
    const int8_t* xq2 = p.xq2 + xrow * p.n_in;
    const float* xd = p.xd + xrow * (p.n_in / 32);
    const float* xs = p.xs + xrow * (p.n_in / 32);
    float* y = p.y + (int64_t)m * NC * p.n_out;

    fill_tables<F>(tab);
    const int tok = (p.ktp * 9) / 4;
    const int rows_iter = W * P * RW;
    const int row_wg = blockIdx.x * p.groups * rows_iter;

    for (int g = 0; g < p.groups; ++g) {
        const int r0 = row_wg + g * rows_iter + (wave * P + team) * RW;
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
            if (p.n_tiles > 1 || g == 0) {
                __syncthreads();
                stage_tile<S>(lds, xq, xq2, xd, xs, p.n_in, NC, k0, kt, p.ktp);
                __syncthreads();
            }
            const int U = (kt + 63) >> 6;
            const int u0 = k0 >> 6;
            for (int u = lt; u < U; u += T) {
                WUnit wu[RW];
#pragma unroll
                for (int rr = 0; rr < RW; ++rr) {
                    typename FM::Raw raw;
                    FM::load(rowp[rr], u0 + u, p.nblk, raw);
                    FM::decode(raw, u0 + u, tab, wu[rr]);
                }
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    XSlice x;
                    read_slice<S>(lds + c * tok, p.ktp, u, x);
#pragma unroll
                    for (int rr = 0; rr < RW; ++rr) acc[rr][c] += unit_dot<S, FM::HAS_MIN>(wu[rr], x);
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float v = acc[rr][c];
#pragma unroll
                for (int o = T / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
                acc[rr][c] = v;
            }
        if (lt == 0) {
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                const int row = r0 + rr;
                if (row < p.n_out) {
#pragma unroll
                    for (int c = 0; c < NC; ++c) y[(int64_t)c * p.n_out + row] = acc[rr][c];
                }
            }
        }
    }
}

// ---- host side --------------------------------------------------------------------------------

struct DeviceInfo {
    int cus;
    int lds_max;  // bytes of dynamic LDS one workgroup may use
};
DeviceInfo device_info();

typedef void (*MvKernel)(MvParams);

template <int F, int NC, int RW>
inline MvKernel pick_t(int T) {
    switch (T) {
        case 16: return mv_kernel<F, NC, 16, RW>;
        case 32: return mv_kernel<F, NC, 32, RW>;
        default: return mv_kernel<F, NC, 64, RW>;
    }
}

template <int F>
inline MvKernel pick_kernel(int nc, int T) {
    switch (nc) {
        case 1: return pick_t<F, 1, 1>(T);
        case 2: return pick_t<F, 2, 2>(T);
        case 3: return pick_t<F, 3, 2>(T);
        case 4: return pick_t<F, 4, 2>(T);
        case 5: return pick_t<F, 5, 2>(T);
        case 6: return pick_t<F, 6, 2>(T);
        case 7: return pick_t<F, 7, 2>(T);
        default: return pick_t<F, 8, 2>(T);
    }
}

// One launch of NC <= NMQ_MAX_COLS tokens (n_mats instances along blockIdx.y).
template <int F>
int launch_mv(MvParams p, int nc, int n_mats, hipStream_t stream) {
    using FM = Fmt<F>;
    const DeviceInfo di = device_info();
    const int rw = nc == 1 ? 1 : 2;
    const int units = (p.n_in + 63) / 64;
    const int T = units >= 48 ? 64 : (units >= 24 ? 32 : 16);
    const int P = 64 / T;
    // K tile: the whole row when the input of all tokens fits the LDS budget
    const int budget = nc == 1 ? 40 * 1024 : di.lds_max;
    const int step = FM::BV == 256 ? 256 : 64;
    int kt = (int)((int64_t)budget * 4 / 9 / nc) / 128 * 128 / step * step;
    if (kt < step) kt = step;
    if (kt >= p.n_in) kt = p.n_in;
    p.kt = kt;
    p.ktp = (kt + 127) / 128 * 128;
    p.n_tiles = (p.n_in + kt - 1) / kt;
    p.nblk = p.n_in / FM::BV;
    p.row_bytes = (int64_t)p.nblk * FM::BB;
    int W = 4;
    while (W > 1 && (p.n_out + W * P * rw - 1) / (W * P * rw) * n_mats < 2 * di.cus) W /= 2;
    const int rows_iter = W * P * rw;
    const int iters = (p.n_out + rows_iter - 1) / rows_iter;
    int groups = 1;
    if (p.n_tiles == 1) {
        const int target = 4 * di.cus;
        groups = iters * n_mats / target;
        groups = groups < 1 ? 1 : (groups > 64 ? 64 : groups);
    }
    p.groups = groups;
    const dim3 grid((unsigned)((iters + groups - 1) / groups), (unsigned)n_mats);
    const size_t lds = (size_t)nc * ((size_t)p.ktp * 9 / 4);
    MvKernel k = pick_kernel<F>(nc, T);
    hipLaunchKernelGGL(k, grid, dim3(64 * W), lds, stream, p);
    return (int)hipGetLastError();
}

}  // namespace nmq
