// C ABI of libnmq (include/nmq.h): argument checks, launch selection, and the small kernels that
// are not mat-vecs (two-stage activation, integer-sum diagnostic, unpack to bf16).
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "nmq_mv_impl.hpp"

namespace nmq {

// ---- device properties (per device, cached) ---------------------------------------------------

static std::mutex g_info_mu;
static DeviceInfo g_info[64];
static bool g_info_ok[64];

DeviceInfo device_info() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DeviceInfo{256, 60 * 1024, 64 * 1024};
    std::lock_guard<std::mutex> lk(g_info_mu);
    if (!g_info_ok[dev]) {
        int cus = 256, lds = 64 * 1024;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
        if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 64 * 1024;
        // static LDS of the kernels (IQ2 tables) comes on top of the dynamic part
        const int small = (lds > 64 * 1024 ? 64 * 1024 : lds) - 4096;
        g_info[dev] = DeviceInfo{cus, small, lds};
        g_info_ok[dev] = true;
    }
    return g_info[dev];
}

// ---- two-stage int8 activation (reference mmvq.py:59-83) ----------------------------------------
// One lane per value, 32 lanes (half a wave) per group.  max|x| and the sum use the xor butterfly
// over offsets 16, 8, 4, 2, 1 (never crossing the 32-lane half), in the order of mmvq.py:42-46
// (half_max / half_sum_xor: one swizzle and four DPP rotations per reduction).
// d = max / 127 and the quotients are IEEE divisions (the library is built without fast-math);
// the residual x - q*d is one fused multiply-add (the CPU oracle does the same).
// Input modes: 0 bf16; 1 fp32; 2 fp32 rounded to bf16 first (what the reference's cudakern entry
// points do to their input, cudakern.py:764); 3 silu(g) * u in fp32 (g = x, u second operand), then
// rounded to bf16 (the gated activation of a MoE expert fed to the down projection as bf16).
template <int MODE>
__global__ __launch_bounds__(256) void quant_q8_kernel(const void* __restrict__ x, const float* __restrict__ u2,
                                                        int8_t* __restrict__ xq, int8_t* __restrict__ xq2,
                                                        float* __restrict__ xd, float* __restrict__ xs, int64_t n) {
    // every argument in the first batch of scalar loads (the compiler would otherwise fetch some of
    // them behind the branches below, one dependent round trip each)
    asm volatile("" ::"s"(x), "s"(u2), "s"(xq), "s"(xq2), "s"(xd), "s"(xs), "s"(n));
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // launched with 256 threads
    if ((i & ~(int64_t)31) >= n) return;  // whole 32-lane groups only (n % 32 == 0)
    float v;
    if constexpr (MODE == 0) {
        v = __uint_as_float((u32)((const u16*)x)[i] << 16);
    } else if constexpr (MODE == 3) {
        const float g = ((const float*)x)[i];
        v = silu_mul_bf16(g, u2[i]);
    } else {
        v = ((const float*)x)[i];
        if constexpr (MODE == 2) v = round_bf16(v);
    }
    quant32_store(v, i, xq, xq2, xd, xs);
}

// ---- fused producers of the two-stage input (one token) ----------------------------------------
// RMS norm of one row (reference mmvq.py:102-120, norm_q8): v = h + rs * r (r given: also written to
// hout), inv = 1 / sqrt(sum(v^2) / n + eps), xn = v * inv * w, and the two-stage input of xn.  One
// workgroup of 1024 threads; value i belongs to thread i % 1024 in both passes, so the second pass
// quantises one value per lane.  NV > 0 (rows of at most 1024 NV values): h, r and w are requested
// together in one round of loads and held in registers across the reduction; NV = 0 (longer rows):
// the second pass reads them again.  v and xn are rounded after every operation (no contraction),
// so they are reproducible from h, r, rs, w and inv; only the sum of squares depends on the order.
template <int NV>
__global__ __launch_bounds__(1024) void norm_q8_kernel(const float* __restrict__ h, const float* __restrict__ r,
                                                       float rs, float* __restrict__ hout, const float* __restrict__ w,
                                                       float eps, float* __restrict__ xn, int8_t* __restrict__ xq,
                                                       int8_t* __restrict__ xq2, float* __restrict__ xd,
                                                       float* __restrict__ xs, int n) {
    asm volatile("" ::"s"(h), "s"(r), "s"(rs), "s"(hout), "s"(w), "s"(eps), "s"(xn), "s"(xq), "s"(xq2), "s"(xd),
                 "s"(xs), "s"(n));
    __shared__ float red[16];
    const int t = threadIdx.x;
    float ss = 0.f;
    constexpr int NR = NV > 0 ? NV : 1;
    float v[NR], wv[NR];
    if constexpr (NV > 0) {
        float rv[NR];
#pragma unroll
        for (int k = 0; k < NV; ++k) {  // clamped indexes: every load is issued unconditionally
            const int ic = min(t + 1024 * k, n - 1);
            v[k] = h[ic];
            wv[k] = w[ic];
        }
        if (r) {
#pragma unroll
            for (int k = 0; k < NV; ++k) rv[k] = r[min(t + 1024 * k, n - 1)];
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                v[k] = __fadd_rn(v[k], __fmul_rn(rs, rv[k]));
                if (t + 1024 * k < n) hout[t + 1024 * k] = v[k];
            }
        }
#pragma unroll
        for (int k = 0; k < NV; ++k)
            if (t + 1024 * k < n) ss = fmaf(v[k], v[k], ss);
    } else {
        for (int i = t; i < n; i += 1024) {
            float x = h[i];
            if (r) {
                x = __fadd_rn(x, __fmul_rn(rs, r[i]));
                hout[i] = x;
            }
            ss = fmaf(x, x, ss);
        }
    }
    ss = team_sum<64>(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) tot += red[k];
    const float inv = 1.0f / sqrtf(tot / (float)n + eps);
    // n % 32 == 0: each 32-lane half of a wave is wholly inside or wholly past the row
    if constexpr (NV > 0) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int i = t + 1024 * k;
            if (i < n) {
                const float o = __fmul_rn(__fmul_rn(v[k], inv), wv[k]);
                xn[i] = o;
                quant32_store(o, i, xq, xq2, xd, xs);
            }
        }
    } else {
        for (int i = t; i < n; i += 1024) {
            const float x = r ? __fadd_rn(h[i], __fmul_rn(rs, r[i])) : h[i];  // recomputed, the same rounding
            const float o = __fmul_rn(__fmul_rn(x, inv), w[i]);
            xn[i] = o;
            quant32_store(o, i, xq, xq2, xd, xs);
        }
    }
}

// a = act(g) * u (u == nullptr: act(g)), act = silu (GELU 0) or the tanh form of gelu (GELU 1), fp32,
// and the two-stage input of a (reference mmvq.py:122-133, akt_q8).
template <int GELU>
__global__ __launch_bounds__(256) void akt_q8_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ a, int8_t* __restrict__ xq,
                                                     int8_t* __restrict__ xq2, float* __restrict__ xd,
                                                     float* __restrict__ xs, int64_t n) {
    asm volatile("" ::"s"(g), "s"(u), "s"(a), "s"(xq), "s"(xq2), "s"(xd), "s"(xs), "s"(n));
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // launched with 256 threads
    if ((i & ~(int64_t)31) >= n) return;
    float v = act_value(g[i], GELU != 0);
    if (u) v *= u[i];
    a[i] = v;
    quant32_store(v, i, xq, xq2, xd, xs);
}

// ---- two-stage fp16 input of the several-token matrix-core kernels (reference mmvq.py:617-641) ---
// One workgroup of 1024 threads per token row: m = max|x| over the row, xs = 2^(e - 8) for m = f 2^e
// (f in [0.5, 1); e >= -100, m == 0 gives e = 0), v = x / xs (exact: a power of two), xh = fp16(v)
// and xl = fp16(v - xh), both rounded to nearest even (v - xh is exact in fp32).  |xh| <= 256 and
// xh + xl is v to about 2^-22 relative.  x: fp32 (F32 = 1) or bf16; 8 values per thread and round.
// xh and xl are written in the matrix cores' operand order (mmh_kernel reads one contiguous 1 KB
// fragment per 16 tokens and 32 values): value k of token t at
//   ((t / 16 * (n / 32) + k / 32) * 64 + (k % 32) / 8 * 16 + t % 16) * 8 + k % 8,
// and xsum[(t / 16 * (n / 32) + k / 32) * 16 + t % 16] = the sum of xh + xl over the 32 values of
// sub-block k / 32: each thread adds its 8 values in order (fp32), then the 4 threads of the
// sub-block add pairwise (xor 1, then xor 2).  Rows past ncols up to the next multiple of 16
// (blockIdx.x >= ncols) are written as zeros.
template <int F32>
__device__ __forceinline__ void load8(const void* x, int64_t i, float (&v)[8]) {
    if constexpr (F32) {
        const u32x4 a = *gp<u32x4>((const float*)x + i), b = *gp<u32x4>((const float*)x + i + 4);
        const u32 w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
    } else {
        const u32x4 a = *gp<u32x4>((const u16*)x + i);
        const u32 w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    }
}

// 8 values of the row (fp32 / bf16 input) at v: xh, xl in operand order, their sub-block sum.
__device__ __forceinline__ void mm_input_store(const float (&v)[8], float inv, int i, int t, int64_t gbase,
                                               int tid, u16* __restrict__ xh, u16* __restrict__ xl,
                                               float* __restrict__ xsum) {
    u32 hi[4], lo[4];
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        u32 h2b = 0, l2b = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float a = v[2 * j + k] * inv;
            const _Float16 h = (_Float16)a;
            const _Float16 l = (_Float16)(a - (float)h);
            sum += (float)h + (float)l;
            h2b |= (u32)__builtin_bit_cast(u16, h) << (16 * k);
            l2b |= (u32)__builtin_bit_cast(u16, l) << (16 * k);
        }
        hi[j] = h2b;
        lo[j] = l2b;
    }
    // the 4 threads of a sub-block are 4 consecutive lanes (all active: n % 32 == 0)
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    const int64_t o = ((gbase + (i >> 5)) * 64 + ((i & 31) >> 3) * 16 + (t & 15)) * 8;
    *gpw<u32x4>(xh + o) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    *gpw<u32x4>(xl + o) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    if ((tid & 3) == 0) gpw<float>(xsum)[(gbase + (i >> 5)) * 16 + (t & 15)] = sum;
}

// 1024 threads per row; NR > 0: rows of at most 8192 NR values, read once and held in registers
// across the reduction; NR = 0: longer rows, read twice.
template <int F32, int NR>
__global__ __launch_bounds__(1024) void mm_input_kernel(const void* __restrict__ x, u16* __restrict__ xh,
                                                        u16* __restrict__ xl, float* __restrict__ xsum,
                                                        float* __restrict__ xs, int n, int ncols) {
    asm volatile("" ::"s"(x), "s"(xh), "s"(xl), "s"(xsum), "s"(xs), "s"(n), "s"(ncols));
    __shared__ float part[16];
    const int t = blockIdx.x;
    const bool real = t < ncols;  // workgroup-uniform
    const int64_t row = (int64_t)t * n;
    const int tid = threadIdx.x;
    constexpr int R = NR > 0 ? NR : 1;
    float v[R][8];
    float m = 0.f;
    if constexpr (NR > 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int i = 8 * tid + 8192 * r;
            if (real && i < n) {
                load8<F32>(x, row + i, v[r]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[r][j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[r][j]));
        }
    } else if (real) {
        for (int i = 8 * tid; i < n; i += 8192) {
            load8<F32>(x, row + i, v[0]);
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[0][j]));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) part[tid >> 6] = m;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) m = fmaxf(m, part[k]);
    int e = 0;
    frexpf(m, &e);
    if (e < -100) e = -100;
    const float inv = ldexpf(1.0f, 8 - e);
    if (real && tid == 0) xs[t] = ldexpf(1.0f, e - 8);
    const int64_t gbase = (int64_t)(t >> 4) * (n >> 5);  // first step of this token's group
    if constexpr (NR > 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int i = 8 * tid + 8192 * r;
            if (i < n) mm_input_store(v[r], inv, i, t, gbase, tid, xh, xl, xsum);
        }
    } else {
        for (int i = 8 * tid; i < n; i += 8192) {
            if (real) {
                load8<F32>(x, row + i, v[0]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[0][j] = 0.f;
            }
            mm_input_store(v[0], inv, i, t, gbase, tid, xh, xl, xsum);
        }
    }
}

// ---- weighted combine of expert outputs (reference models/moe.py:275-277, 319-320) --------------
// out[t][e] = sum_j w[t*k + j] * y[t*k + j][e], j = 0..k-1 in this order (a fixed order).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y, const float* __restrict__ w,
                                                           int L, int k, int E, float* __restrict__ out) {
    asm volatile("" ::"s"(y), "s"(w), "s"(L), "s"(k), "s"(E), "s"(out));
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)L * E) return;
    const int t = (int)(i / E), e = (int)(i % E);
    float acc = 0.f;
    if (k <= 16) {  // every read issued before the first sum (one memory round trip, not k)
        float wv[16], yv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int jj = j < k ? j : 0;
            wv[j] = gp<float>(w)[(int64_t)t * k + jj];
            yv[j] = gp<float>(y)[((int64_t)t * k + jj) * E + e];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (j < k) acc = fmaf(wv[j], yv[j], acc);
    } else {
        for (int j = 0; j < k; ++j)
            acc = fmaf(gp<float>(w)[(int64_t)t * k + j], gp<float>(y)[((int64_t)t * k + j) * E + e], acc);
    }
    gpw<float>(out)[i] = acc;
}

// ---- diagnostic: per-16 integer sums, through the same unit decoders as mv_kernel ---------------
template <int F>
__global__ __launch_bounds__(256) void block_sums_kernel(const u8* __restrict__ w, const int8_t* __restrict__ xq,
                                                          const int8_t* __restrict__ xq2, int32_t* __restrict__ s1,
                                                          int32_t* __restrict__ s2, int n_out, int n_in) {
    using FM = Fmt<F>;
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    fill_tables<F>(tab, 256);
    __syncthreads();
    const int units = (n_in + 63) / 64, nblk = n_in / FM::BV;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // launched with 256 threads
    if (idx >= (int64_t)n_out * units) return;
    const int row = (int)(idx / units), u = (int)(idx % units);
    typename FM::Raw raw;
    WUnit wu;
    FM::load(w + (int64_t)row * nblk * FM::BB, u, nblk, raw);
    FM::decode(raw, u, tab, wu);
    XSlice x;
    int g[4];
    const int G = n_in / 16;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int pos;
        if (FM::STRIDED) {
            const int b = u >> 2, h = (u >> 1) & 1, j = u & 1;
            pos = 256 * b + 128 * h + 32 * k + 16 * j;
        } else {
            pos = 64 * u + 16 * k;
        }
        g[k] = pos / 16;
        const bool ok = pos < n_in;
        const u32x4 a = ok ? *(const u32x4*)(xq + pos) : u32x4{0u, 0u, 0u, 0u};
        const u32x4 b = ok ? *(const u32x4*)(xq2 + pos) : u32x4{0u, 0u, 0u, 0u};
        x.q[4 * k] = a.x; x.q[4 * k + 1] = a.y; x.q[4 * k + 2] = a.z; x.q[4 * k + 3] = a.w;
        x.q2[4 * k] = b.x; x.q2[4 * k + 1] = b.y; x.q2[4 * k + 2] = b.z; x.q2[4 * k + 3] = b.w;
    }
    int a1[4], a2[4];
    unit_sums(wu.w, x, a1, a2);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (g[k] < G) {
            s1[(int64_t)row * G + g[k]] = a1[k];
            s2[(int64_t)row * G + g[k]] = a2[k];
        }
}

// ---- unpack to bf16 (exact quant.py fp32 value, then round to nearest even) --------------------
__device__ __forceinline__ u16 f2bf(float f) {
    const u32 u = __float_as_uint(f);
    return (u16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <int F>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const u8* __restrict__ w, u16* __restrict__ out,
                                                            int64_t n_blocks) {
#pragma clang fp contract(off)
    using FM = Fmt<F>;
    __shared__ u64 tab[F == NMQ_IQ2_XXS ? 384 : 1];
    fill_tables<F>(tab, 256);
    __syncthreads();
    // a "row" of one block; Q4_0 / Q8_0 units span two blocks, so their rows are two blocks (last may be one)
    constexpr int BPU = FM::BV == 32 ? 2 : 1;  // blocks per row handled here
    constexpr int UPR = FM::BV == 32 ? 1 : 4;  // units per row
    const int64_t rows = (n_blocks + BPU - 1) / BPU;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // launched with 256 threads
    if (idx >= rows * UPR) return;
    const int64_t row = idx / UPR;
    const int u = (int)(idx % UPR);
    const int nblk = (int)((n_blocks - row * BPU) < BPU ? (n_blocks - row * BPU) : BPU);
    typename FM::Raw raw;
    WUnit wu;
    FM::load(w + row * BPU * FM::BB, u, nblk, raw);
    FM::decode(raw, u, tab, wu);
    u16* o = out + row * BPU * FM::BV;
    const int nvals = nblk * FM::BV;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        int pos;
        if (FM::STRIDED) {
            const int h = (u >> 1) & 1, j = u & 1;
            pos = 128 * h + 32 * r + 16 * j;
        } else {
            pos = 64 * u + 16 * r;
        }
        if (pos >= nvals) continue;
        const float sc = wu.ws[r];
        const float mn = FM::HAS_MIN ? wu.wm[r >> 1] : 0.f;
        u32 pk[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32 v = wu.w[4 * r + k];
            float f[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float q = (float)(int8_t)(v >> (8 * e));
                f[e] = FM::HAS_MIN ? (sc * q - mn) : sc * q;
            }
            pk[2 * k] = (u32)f2bf(f[0]) | ((u32)f2bf(f[1]) << 16);
            pk[2 * k + 1] = (u32)f2bf(f[2]) | ((u32)f2bf(f[3]) << 16);
        }
        u32x4* dst = (u32x4*)(o + pos);
        dst[0] = u32x4{pk[0], pk[1], pk[2], pk[3]};
        dst[1] = u32x4{pk[4], pk[5], pk[6], pk[7]};
    }
}

// ---- per-format launch tables -----------------------------------------------------------------
template <int F>
int launch_mv(MvParams p, int nc, int n_mats, hipStream_t stream);
extern template int launch_mv<NMQ_Q4_0>(MvParams, int, int, hipStream_t);
extern template int launch_mv<NMQ_Q8_0>(MvParams, int, int, hipStream_t);
extern template int launch_mv<NMQ_Q4_K>(MvParams, int, int, hipStream_t);
extern template int launch_mv<NMQ_Q6_K>(MvParams, int, int, hipStream_t);
extern template int launch_mv<NMQ_IQ2_XXS>(MvParams, int, int, hipStream_t);
extern template int launch_mv<NMQ_TQ2_0>(MvParams, int, int, hipStream_t);

template <int F>
int launch_moe_down(MvParams p, Combine c, int L, hipStream_t stream);
extern template int launch_moe_down<NMQ_Q4_0>(MvParams, Combine, int, hipStream_t);
extern template int launch_moe_down<NMQ_Q8_0>(MvParams, Combine, int, hipStream_t);
extern template int launch_moe_down<NMQ_Q4_K>(MvParams, Combine, int, hipStream_t);
extern template int launch_moe_down<NMQ_Q6_K>(MvParams, Combine, int, hipStream_t);
extern template int launch_moe_down<NMQ_IQ2_XXS>(MvParams, Combine, int, hipStream_t);
extern template int launch_moe_down<NMQ_TQ2_0>(MvParams, Combine, int, hipStream_t);

static int launch_moe_down_any(int fmt, const MvParams& p, const Combine& c, int L, hipStream_t s) {
    switch (fmt) {
        case NMQ_Q4_0: return launch_moe_down<NMQ_Q4_0>(p, c, L, s);
        case NMQ_Q8_0: return launch_moe_down<NMQ_Q8_0>(p, c, L, s);
        case NMQ_Q4_K: return launch_moe_down<NMQ_Q4_K>(p, c, L, s);
        case NMQ_Q6_K: return launch_moe_down<NMQ_Q6_K>(p, c, L, s);
        case NMQ_IQ2_XXS: return launch_moe_down<NMQ_IQ2_XXS>(p, c, L, s);
        case NMQ_TQ2_0: return launch_moe_down<NMQ_TQ2_0>(p, c, L, s);
        default: return NMQ_ERR_FORMAT;
    }
}

template <int F>
int launch_moe_gu(MvParams p, QuantOut o, hipStream_t stream);
extern template int launch_moe_gu<NMQ_Q4_0>(MvParams, QuantOut, hipStream_t);
extern template int launch_moe_gu<NMQ_Q8_0>(MvParams, QuantOut, hipStream_t);
extern template int launch_moe_gu<NMQ_Q4_K>(MvParams, QuantOut, hipStream_t);
extern template int launch_moe_gu<NMQ_Q6_K>(MvParams, QuantOut, hipStream_t);
extern template int launch_moe_gu<NMQ_IQ2_XXS>(MvParams, QuantOut, hipStream_t);
extern template int launch_moe_gu<NMQ_TQ2_0>(MvParams, QuantOut, hipStream_t);

static int launch_moe_gu_any(int fmt, const MvParams& p, const QuantOut& o, hipStream_t s) {
    switch (fmt) {
        case NMQ_Q4_0: return launch_moe_gu<NMQ_Q4_0>(p, o, s);
        case NMQ_Q8_0: return launch_moe_gu<NMQ_Q8_0>(p, o, s);
        case NMQ_Q4_K: return launch_moe_gu<NMQ_Q4_K>(p, o, s);
        case NMQ_Q6_K: return launch_moe_gu<NMQ_Q6_K>(p, o, s);
        case NMQ_IQ2_XXS: return launch_moe_gu<NMQ_IQ2_XXS>(p, o, s);
        case NMQ_TQ2_0: return launch_moe_gu<NMQ_TQ2_0>(p, o, s);
        default: return NMQ_ERR_FORMAT;
    }
}

template <int F>
int launch_mvp(MvParams p, QuantOut o, hipStream_t stream);
extern template int launch_mvp<NMQ_Q4_0>(MvParams, QuantOut, hipStream_t);
extern template int launch_mvp<NMQ_Q8_0>(MvParams, QuantOut, hipStream_t);
extern template int launch_mvp<NMQ_Q4_K>(MvParams, QuantOut, hipStream_t);
extern template int launch_mvp<NMQ_Q6_K>(MvParams, QuantOut, hipStream_t);
extern template int launch_mvp<NMQ_IQ2_XXS>(MvParams, QuantOut, hipStream_t);
extern template int launch_mvp<NMQ_TQ2_0>(MvParams, QuantOut, hipStream_t);

static int launch_mvp_any(int fmt, const MvParams& p, const QuantOut& o, hipStream_t s) {
    switch (fmt) {
        case NMQ_Q4_0: return launch_mvp<NMQ_Q4_0>(p, o, s);
        case NMQ_Q8_0: return launch_mvp<NMQ_Q8_0>(p, o, s);
        case NMQ_Q4_K: return launch_mvp<NMQ_Q4_K>(p, o, s);
        case NMQ_Q6_K: return launch_mvp<NMQ_Q6_K>(p, o, s);
        case NMQ_IQ2_XXS: return launch_mvp<NMQ_IQ2_XXS>(p, o, s);
        case NMQ_TQ2_0: return launch_mvp<NMQ_TQ2_0>(p, o, s);
        default: return NMQ_ERR_FORMAT;
    }
}

template <int F>
int launch_mmh(MmhParams p, hipStream_t stream);
extern template int launch_mmh<NMQ_Q4_K>(MmhParams, hipStream_t);
extern template int launch_mmh<NMQ_Q6_K>(MmhParams, hipStream_t);

static int launch_any(int fmt, const MvParams& p, int nc, int n_mats, hipStream_t s) {
    switch (fmt) {
        case NMQ_Q4_0: return launch_mv<NMQ_Q4_0>(p, nc, n_mats, s);
        case NMQ_Q8_0: return launch_mv<NMQ_Q8_0>(p, nc, n_mats, s);
        case NMQ_Q4_K: return launch_mv<NMQ_Q4_K>(p, nc, n_mats, s);
        case NMQ_Q6_K: return launch_mv<NMQ_Q6_K>(p, nc, n_mats, s);
        case NMQ_IQ2_XXS: return launch_mv<NMQ_IQ2_XXS>(p, nc, n_mats, s);
        case NMQ_TQ2_0: return launch_mv<NMQ_TQ2_0>(p, nc, n_mats, s);
        default: return NMQ_ERR_FORMAT;
    }
}

template <template <int> class K, typename... A>
static int launch_fmt_kernel(int fmt, dim3 grid, hipStream_t s, A... a) {
    switch (fmt) {
        case NMQ_Q4_0: hipLaunchKernelGGL(K<NMQ_Q4_0>::fn, grid, dim3(256), 0, s, a...); break;
        case NMQ_Q8_0: hipLaunchKernelGGL(K<NMQ_Q8_0>::fn, grid, dim3(256), 0, s, a...); break;
        case NMQ_Q4_K: hipLaunchKernelGGL(K<NMQ_Q4_K>::fn, grid, dim3(256), 0, s, a...); break;
        case NMQ_Q6_K: hipLaunchKernelGGL(K<NMQ_Q6_K>::fn, grid, dim3(256), 0, s, a...); break;
        case NMQ_IQ2_XXS: hipLaunchKernelGGL(K<NMQ_IQ2_XXS>::fn, grid, dim3(256), 0, s, a...); break;
        case NMQ_TQ2_0: hipLaunchKernelGGL(K<NMQ_TQ2_0>::fn, grid, dim3(256), 0, s, a...); break;
        default: return NMQ_ERR_FORMAT;
    }
    return (int)hipGetLastError();
}
template <int F>
struct SumsK {
    static constexpr auto fn = block_sums_kernel<F>;
};
template <int F>
struct DeqK {
    static constexpr auto fn = dequant_bf16_kernel<F>;
};

// ---- pure streaming read (diagnostic) ----------------------------------------------------------------
// Reads n16 16-byte words with a grid-stride loop, U loads in flight per thread, and folds them into one
// value per thread; a lane stores only if its fold equals a constant no real input produces in practice, so
// the reads cannot be dropped and the kernel writes (almost) nothing.  It is the reference point for what
// one launch of a given size reads from HBM.
template <int U>
__global__ __launch_bounds__(1024) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16, u32* sink,
                                                           int nt) {
    const int64_t stride = (int64_t)gridDim.x * nt;
    int64_t i = (int64_t)blockIdx.x * nt + threadIdx.x;
    u32 acc = 0;
    for (; i + (int64_t)(U - 1) * stride < n16; i += (int64_t)U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = src[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace nmq

using namespace nmq;

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

extern "C" {

int nmq_abi_version(void) { return 2; }

const char* nmq_strerror(int code) {
    switch (code) {
        case NMQ_OK: return "ok";
        case NMQ_ERR_FORMAT: return "nmq: unsupported block format";
        case NMQ_ERR_SHAPE: return "nmq: bad shape (n_in must be a multiple of the block size; sizes in range)";
        case NMQ_ERR_ARG: return "nmq: bad argument (NULL or misaligned pointer, bad count)";
        case NMQ_ERR_DEVICE: return "nmq: no usable gfx950 device";
        default: return code > 0 ? hipGetErrorString((hipError_t)code) : "nmq: unknown error";
    }
}

int nmq_set_tuning(const char* name, int value) {
    static std::mutex mu;
    const int k = tune_index(name);
    if (k < 0) return NMQ_ERR_ARG;
    std::lock_guard<std::mutex> g(mu);
    if (!g_tune_ready.load(std::memory_order_acquire)) tune_reset_all();
    g_tune[k].store(value == NMQ_TUNE_DEFAULT ? TUNE_UNSET : value, std::memory_order_relaxed);
    return NMQ_OK;
}

int nmq_get_tuning(const char* name, int* value) {
    const int k = tune_index(name);
    if (k < 0 || !value) return NMQ_ERR_ARG;
    const int v = g_tune_ready.load(std::memory_order_acquire) ? g_tune[k].load(std::memory_order_relaxed)
                                                               : TUNE_UNSET;
    *value = v == TUNE_UNSET ? NMQ_TUNE_DEFAULT : v;
    return NMQ_OK;
}

int nmq_format_info(int fmt, int* block_values, int* block_bytes) {
    int bv, bb;
    switch (fmt) {
        case NMQ_Q4_0: bv = 32; bb = 18; break;
        case NMQ_Q8_0: bv = 32; bb = 34; break;
        case NMQ_Q4_K: bv = 256; bb = 144; break;
        case NMQ_Q6_K: bv = 256; bb = 210; break;
        case NMQ_IQ2_XXS: bv = 256; bb = 66; break;
        case NMQ_TQ2_0: bv = 256; bb = 66; break;
        default: return NMQ_ERR_FORMAT;
    }
    if (block_values) *block_values = bv;
    if (block_bytes) *block_bytes = bb;
    return NMQ_OK;
}

int nmq_device_arch(char* buf, int len) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (!buf || len <= 0) return NMQ_ERR_ARG;
    buf[0] = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return NMQ_ERR_DEVICE;
    snprintf(buf, (size_t)len, "%s", prop.gcnArchName);
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? NMQ_OK : NMQ_ERR_DEVICE;
}

int nmq_quant_q8(const void* x, int x_is_f32, int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n,
                 void* stream) {
    if (!x || !xq || !xq2 || !xd || !xs) return NMQ_ERR_ARG;
    if (x_is_f32 < 0 || x_is_f32 > 2) return NMQ_ERR_ARG;
    if (n <= 0 || n % 32) return NMQ_ERR_SHAPE;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    const dim3 g((unsigned)blocks), b(256);
    const hipStream_t s = (hipStream_t)stream;
    if (x_is_f32 == 0) hipLaunchKernelGGL(quant_q8_kernel<0>, g, b, 0, s, x, nullptr, xq, xq2, xd, xs, n);
    else if (x_is_f32 == 1) hipLaunchKernelGGL(quant_q8_kernel<1>, g, b, 0, s, x, nullptr, xq, xq2, xd, xs, n);
    else hipLaunchKernelGGL(quant_q8_kernel<2>, g, b, 0, s, x, nullptr, xq, xq2, xd, xs, n);
    return (int)hipGetLastError();
}

int nmq_silu_mul_quant(const float* g, const float* u, int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n,
                       void* stream) {
    if (!g || !u || !xq || !xq2 || !xd || !xs) return NMQ_ERR_ARG;
    if (!aligned(g, 4) || !aligned(u, 4)) return NMQ_ERR_ARG;
    if (n <= 0 || n % 32) return NMQ_ERR_SHAPE;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    hipLaunchKernelGGL(quant_q8_kernel<3>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, g, u, xq, xq2,
                       xd, xs, n);
    return (int)hipGetLastError();
}

int nmq_norm_q8(const float* h, const float* r, float rs, float* hout, const float* w, float eps, float* xn,
                int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n, void* stream) {
    if (!h || !w || !xn || !xq || !xq2 || !xd || !xs || (r && !hout)) return NMQ_ERR_ARG;
    if (!aligned(h, 4) || !aligned(w, 4) || !aligned(xn, 4) || (r && (!aligned(r, 4) || !aligned(hout, 4))))
        return NMQ_ERR_ARG;
    if (n <= 0 || n % 32 || n > NMQ_NORM_MAX) return NMQ_ERR_SHAPE;
    if (r) {  // the second pass recomputes v from h and r, so hout must not overlap either
        const uintptr_t o0 = (uintptr_t)hout, o1 = o0 + (uintptr_t)n * 4;
        for (const float* in : {h, r})
            if ((uintptr_t)in < o1 && o0 < (uintptr_t)in + (uintptr_t)n * 4) return NMQ_ERR_ARG;
    }
    void (*k)(const float*, const float*, float, float*, const float*, float, float*, int8_t*, int8_t*, float*,
              float*, int) = n <= 1024   ? norm_q8_kernel<1>
                             : n <= 2048 ? norm_q8_kernel<2>
                             : n <= 4096 ? norm_q8_kernel<4>
                             : n <= 8192 ? norm_q8_kernel<8>
                             : n <= 16384 ? norm_q8_kernel<16> : norm_q8_kernel<0>;
    hipLaunchKernelGGL(k, dim3(1), dim3(1024), 0, (hipStream_t)stream, h, r, rs, hout, w, eps, xn, xq, xq2, xd, xs,
                       (int)n);
    return (int)hipGetLastError();
}

int nmq_akt_q8(const float* g, const float* u, int gelu, float* a, int8_t* xq, int8_t* xq2, float* xd, float* xs,
               int64_t n, void* stream) {
    if (!g || !a || !xq || !xq2 || !xd || !xs) return NMQ_ERR_ARG;
    if (!aligned(g, 4) || !aligned(a, 4) || (u && !aligned(u, 4)) || (gelu != 0 && gelu != 1)) return NMQ_ERR_ARG;
    if (n <= 0 || n % 32) return NMQ_ERR_SHAPE;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    const dim3 gr((unsigned)blocks), b(256);
    const hipStream_t s = (hipStream_t)stream;
    if (gelu) hipLaunchKernelGGL(akt_q8_kernel<1>, gr, b, 0, s, g, u, a, xq, xq2, xd, xs, n);
    else hipLaunchKernelGGL(akt_q8_kernel<0>, gr, b, 0, s, g, u, a, xq, xq2, xd, xs, n);
    return (int)hipGetLastError();
}

int nmq_moe_combine(const float* y, const float* w, int L, int k, int E, float* out, void* stream) {
    if (!y || !w || !out || !aligned(y, 4) || !aligned(w, 4) || !aligned(out, 4)) return NMQ_ERR_ARG;
    if (L < 1 || k < 1 || E < 1 || (int64_t)L * k > 65535) return NMQ_ERR_SHAPE;
    const int64_t blocks = ((int64_t)L * E + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, y, w, L, k, E,
                       out);
    return (int)hipGetLastError();
}

static int check_w(int fmt, const void* w, const float* y, int n_out, int n_in) {
    int bv, bb;
    if (nmq_format_info(fmt, &bv, &bb)) return NMQ_ERR_FORMAT;
    if (!w || !y || !aligned(y, 4)) return NMQ_ERR_ARG;
    if (n_out < 1 || n_in < bv || n_in % bv || n_in > (1 << 20)) return NMQ_ERR_SHAPE;
    // Q4_K reads its 16-byte block header and quant groups with aligned 16-byte loads
    if (fmt == NMQ_Q4_K && !aligned(w, 16)) return NMQ_ERR_ARG;
    if (!aligned(w, 2)) return NMQ_ERR_ARG;
    return NMQ_OK;
}

static int check_mv(int fmt, const void* w, const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs,
                    const float* y, int n_out, int n_in) {
    const int e = check_w(fmt, w, y, n_out, n_in);
    if (e) return e;
    if (!xq || !xq2 || !xd || !xs) return NMQ_ERR_ARG;
    if (!aligned(xq, 16) || !aligned(xq2, 16) || !aligned(xd, 4) || !aligned(xs, 4)) return NMQ_ERR_ARG;
    return NMQ_OK;
}

// Input given as values: the one-token kernels stage it (rows of at most NMQ_X_MAX_N_IN values).
static int check_values(const void* x, int x_mode, const void* x2, int n_in) {
    if (!x || x_mode < NMQ_X_BF16 || x_mode > NMQ_X_SILU_MUL_BF16) return NMQ_ERR_ARG;
    if (!aligned(x, x_mode == NMQ_X_BF16 ? 8 : 16)) return NMQ_ERR_ARG;
    if (x_mode == NMQ_X_SILU_MUL_BF16 && (!x2 || !aligned(x2, 16))) return NMQ_ERR_ARG;
    if (n_in % 32 || n_in > NMQ_X_MAX_N_IN) return NMQ_ERR_SHAPE;
    return NMQ_OK;
}

int nmq_mv(int fmt, const void* w, const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, float* y,
           int n_out, int n_in, int ncols, void* stream) {
    int e = check_mv(fmt, w, xq, xq2, xd, xs, y, n_out, n_in);
    if (e) return e;
    if (ncols < 1) return NMQ_ERR_ARG;
    for (int c0 = 0; c0 < ncols; c0 += 2 * NMQ_MAX_COLS) {
        // up to 16 tokens per call of the launcher (one launch on the matrix cores, or two of 8)
        const int nc = ncols - c0 < 2 * NMQ_MAX_COLS ? ncols - c0 : 2 * NMQ_MAX_COLS;
        MvParams p{};
        p.w = (const u8*)w;
        p.ids = nullptr;
        p.per_expert = 0;
        p.xq = xq + (int64_t)c0 * n_in;
        p.xq2 = xq2 + (int64_t)c0 * n_in;
        p.xd = xd + (int64_t)c0 * (n_in / 32);
        p.xs = xs + (int64_t)c0 * (n_in / 32);
        p.y = y + (int64_t)c0 * n_out;
        p.n_out = n_out;
        p.n_in = n_in;
        p.x_group = 1;
        e = launch_any(fmt, p, nc, 1, (hipStream_t)stream);
        if (e) return e;
    }
    return NMQ_OK;
}

int nmq_mm_input(const void* x, int x_is_f32, uint16_t* xh, uint16_t* xl, float* xsum, float* xs, int n_in,
                 int ncols, void* stream) {
    if (!x || !xh || !xl || !xsum || !xs || x_is_f32 < 0 || x_is_f32 > 1) return NMQ_ERR_ARG;
    if (!aligned(x, 16) || !aligned(xh, 16) || !aligned(xl, 16) || !aligned(xsum, 4) || !aligned(xs, 4))
        return NMQ_ERR_ARG;
    if (n_in < 32 || n_in % 32 || n_in > (1 << 20) || ncols < 1) return NMQ_ERR_SHAPE;
    const dim3 g((unsigned)((ncols + 15) / 16 * 16)), b(1024);
    const hipStream_t s = (hipStream_t)stream;
    const int nr = n_in <= 8192 ? 1 : n_in <= 16384 ? 2 : 0;
    void (*k)(const void*, u16*, u16*, float*, float*, int, int) =
        x_is_f32 ? (nr == 1 ? mm_input_kernel<1, 1> : nr == 2 ? mm_input_kernel<1, 2> : mm_input_kernel<1, 0>)
                 : (nr == 1 ? mm_input_kernel<0, 1> : nr == 2 ? mm_input_kernel<0, 2> : mm_input_kernel<0, 0>);
    hipLaunchKernelGGL(k, g, b, 0, s, x, (u16*)xh, (u16*)xl, xsum, xs, n_in, ncols);
    return (int)hipGetLastError();
}

int nmq_mm(int fmt, const void* w, const uint16_t* xh, const uint16_t* xl, const float* xsum, const float* xs,
           float* y, int n_out, int n_in, int ncols, void* stream) {
    if (fmt != NMQ_Q4_K && fmt != NMQ_Q6_K) return NMQ_ERR_FORMAT;
    int e = check_w(fmt, w, y, n_out, n_in);
    if (e) return e;
    if (!xh || !xl || !xsum || !xs || !aligned(xh, 16) || !aligned(xl, 16) || !aligned(xsum, 4) || !aligned(xs, 4))
        return NMQ_ERR_ARG;
    if (ncols < 1) return NMQ_ERR_ARG;
    for (int c0 = 0; c0 < ncols; c0 += MMH_MAX_COLS) {
        MmhParams p{};
        p.w = (const u8*)w;
        p.xh = (const u16*)xh + (int64_t)c0 * n_in;
        p.xl = (const u16*)xl + (int64_t)c0 * n_in;
        p.xsum = xsum + (int64_t)c0 * (n_in / 32);
        p.xs = xs + c0;
        p.y = y + (int64_t)c0 * n_out;
        p.n_out = n_out;
        p.n_in = n_in;
        p.nc = ncols - c0 < MMH_MAX_COLS ? ncols - c0 : MMH_MAX_COLS;
        e = fmt == NMQ_Q4_K ? launch_mmh<NMQ_Q4_K>(p, (hipStream_t)stream)
                            : launch_mmh<NMQ_Q6_K>(p, (hipStream_t)stream);
        if (e) return e;
    }
    return NMQ_OK;
}

// One token over 1..NMQ_MAX_MATS matrices (segments), input as the two-stage arrays or as values.
static int mv_segments(int fmt, int n_mats, const void* const* ws, const int* n_outs, float* const* ys,
                       const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, const void* xv,
                       const void* xv2, int x_mode, int n_in, void* stream) {
    if (n_mats < 1 || n_mats > NMQ_MAX_MATS || !ws || !n_outs || !ys) return NMQ_ERR_ARG;
    int64_t total = 0;
    for (int i = 0; i < n_mats; ++i) {
        const int e = xv ? check_w(fmt, ws[i], ys[i], n_outs[i], n_in)
                         : check_mv(fmt, ws[i], xq, xq2, xd, xs, ys[i], n_outs[i], n_in);
        if (e) return e;
        total += n_outs[i];
    }
    if (xv) {
        const int e = check_values(xv, x_mode, xv2, n_in);
        if (e) return e;
    }
    if (total > (1 << 30)) return NMQ_ERR_SHAPE;
    MvParams p{};
    p.w = (const u8*)ws[0];
    p.y = ys[0];
    p.xq = xq;
    p.xq2 = xq2;
    p.xd = xd;
    p.xs = xs;
    p.xv = xv;
    p.xv2 = xv2;
    p.x_mode = x_mode;
    p.n_out = (int)total;
    p.n_in = n_in;
    p.x_group = 1;
    p.n_seg = n_mats == 1 ? 0 : n_mats;
    int end = 0;
    for (int i = 0; i < 4; ++i) {
        const bool used = i < n_mats;
        p.seg_w[i] = (const u8*)(used ? ws[i] : ws[0]);
        p.seg_y[i] = used ? ys[i] : ys[0];
        if (used) end += n_outs[i];
        if (i < 3) p.seg_end[i] = i + 1 < n_mats ? end : 0x7fffffff;
    }
    return launch_any(fmt, p, 1, 1, (hipStream_t)stream);
}

int nmq_mv_multi(int fmt, int n_mats, const void* const* ws, const int* n_outs, float* const* ys,
                 const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int n_in, void* stream) {
    return mv_segments(fmt, n_mats, ws, n_outs, ys, xq, xq2, xd, xs, nullptr, nullptr, 0, n_in, stream);
}

int nmq_mv_x(int fmt, int n_mats, const void* const* ws, const int* n_outs, float* const* ys, const void* x,
             int x_mode, const void* x2, int n_in, void* stream) {
    if (!x) return NMQ_ERR_ARG;
    return mv_segments(fmt, n_mats, ws, n_outs, ys, nullptr, nullptr, nullptr, nullptr, x, x2, x_mode, n_in, stream);
}

static int check_experts(int fmt, const void* w, int n_ids, int64_t per_expert, int x_group, int n_out, int n_in) {
    if (n_ids < 1 || n_ids > 65535 || x_group < 1) return NMQ_ERR_ARG;
    if (per_expert >= 0) {
        int bv, bb;
        nmq_format_info(fmt, &bv, &bb);
        if (per_expert < (int64_t)n_out * (n_in / bv) * bb) return NMQ_ERR_SHAPE;
        if (fmt == NMQ_Q4_K && per_expert % 16) return NMQ_ERR_ARG;
        if (per_expert % 2) return NMQ_ERR_ARG;
    } else if (!aligned(w, 8)) {
        return NMQ_ERR_ARG;
    }
    return NMQ_OK;
}

int nmq_mv_experts(int fmt, const void* w, const int64_t* ids, int n_ids, int64_t per_expert, const int8_t* xq,
                   const int8_t* xq2, const float* xd, const float* xs, int x_group, float* y, int n_out, int n_in,
                   void* stream) {
    int e = check_mv(fmt, w, xq, xq2, xd, xs, y, n_out, n_in);
    if (e) return e;
    if (!ids) return NMQ_ERR_ARG;
    e = check_experts(fmt, w, n_ids, per_expert, x_group, n_out, n_in);
    if (e) return e;
    MvParams p{};
    p.w = (const u8*)w;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xq = xq;
    p.xq2 = xq2;
    p.xd = xd;
    p.xs = xs;
    p.y = y;
    p.n_out = n_out;
    p.n_in = n_in;
    p.x_group = x_group;
    p.n_ids = n_ids;
    return launch_any(fmt, p, 1, n_ids, (hipStream_t)stream);
}

int nmq_mv_experts2(int fmt, const void* w_a, const void* w_b, const int64_t* ids, int n_ids, int64_t per_expert,
                    const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int x_group, float* y,
                    int n_out, int n_in, void* stream) {
    int e = check_mv(fmt, w_a, xq, xq2, xd, xs, y, n_out, n_in);
    if (e) return e;
    e = check_mv(fmt, w_b, xq, xq2, xd, xs, y, n_out, n_in);
    if (e) return e;
    if (!ids || n_ids > 32767) return NMQ_ERR_ARG;
    e = check_experts(fmt, w_a, n_ids, per_expert, x_group, n_out, n_in);
    if (e) return e;
    e = check_experts(fmt, w_b, n_ids, per_expert, x_group, n_out, n_in);
    if (e) return e;
    MvParams p{};
    p.w = (const u8*)w_a;
    p.w2 = (const u8*)w_b;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xq = xq;
    p.xq2 = xq2;
    p.xd = xd;
    p.xs = xs;
    p.y = y;
    p.n_out = n_out;
    p.n_in = n_in;
    p.x_group = x_group;
    p.n_ids = n_ids;
    return launch_any(fmt, p, 1, 2 * n_ids, (hipStream_t)stream);
}

int nmq_mv_experts_x(int fmt, const void* w_a, const void* w_b, const int64_t* ids, int n_ids, int64_t per_expert,
                     const void* x, int x_mode, const void* x2, int x_group, float* y, int n_out, int n_in,
                     void* stream) {
    int e = check_w(fmt, w_a, y, n_out, n_in);
    if (e) return e;
    if (w_b && (e = check_w(fmt, w_b, y, n_out, n_in))) return e;
    if ((e = check_values(x, x_mode, x2, n_in))) return e;
    if (!ids || n_ids > (w_b ? 32767 : 65535)) return NMQ_ERR_ARG;
    if ((e = check_experts(fmt, w_a, n_ids, per_expert, x_group, n_out, n_in))) return e;
    if (w_b && (e = check_experts(fmt, w_b, n_ids, per_expert, x_group, n_out, n_in))) return e;
    MvParams p{};
    p.w = (const u8*)w_a;
    p.w2 = (const u8*)w_b;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xv = x;
    p.xv2 = x2;
    p.x_mode = x_mode;
    p.y = y;
    p.n_out = n_out;
    p.n_in = n_in;
    p.x_group = x_group;
    p.n_ids = n_ids;
    return launch_any(fmt, p, 1, w_b ? 2 * n_ids : n_ids, (hipStream_t)stream);
}

}  // extern "C"

extern "C" {

int nmq_mv_gate_up_act(int fmt, const void* w_gate, const void* w_up, const void* x, int x_mode, int act,
                       int8_t* xq, int8_t* xq2, float* xd, float* xs, int n_out, int n_in, void* stream) {
    int e = check_mv(fmt, w_gate, xq, xq2, xd, xs, xd, n_out, n_in);
    if (e) return e;
    if ((e = check_w(fmt, w_up, xd, n_out, n_in))) return e;
    if (x_mode == NMQ_X_SILU_MUL_BF16) return NMQ_ERR_ARG;
    if ((e = check_values(x, x_mode, nullptr, n_in))) return e;
    if (act & ~(NMQ_ACT_GELU | NMQ_ACT_BF16)) return NMQ_ERR_ARG;
    MvParams p{};
    p.w = (const u8*)w_gate;
    p.w2 = (const u8*)w_up;
    p.xv = x;
    p.x_mode = x_mode;
    p.n_out = n_out;
    p.n_in = n_in;
    return launch_mvp_any(fmt, p, QuantOut{xq, xq2, xd, xs, act}, (hipStream_t)stream);
}

}  // extern "C"

// ---- expert down projection fused with the weighted combine ---------------------------------------------
// One launch of moe_down_kernel where it takes the shape (no workspace).  Otherwise the slots go through the
// plain gathered launch into a workspace of L*k x n_out fp32 and moe_combine_kernel sums them.
static int64_t moe_work_bytes(int L, int k, int n_out, int n_in) {
    return plan_moe_down(n_out, n_in, L, k, device_info()).ok ? 0 : (int64_t)L * k * n_out * 4;
}

static int moe_check_slots(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert,
                           const float* wts, int n_out, int n_in) {
    if (!ids || !wts || !aligned(wts, 4) || L < 1 || k < 1 || (int64_t)L * k > 65535) return NMQ_ERR_ARG;
    return check_experts(fmt, w, L * k, per_expert, 1, n_out, n_in);
}

static int moe_check(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const void* x,
                     int x_mode, const void* x2, const float* wts, float* out, int n_out, int n_in) {
    int e = check_w(fmt, w, out, n_out, n_in);
    if (e) return e;
    if ((e = check_values(x, x_mode, x2, n_in))) return e;
    return moe_check_slots(fmt, w, ids, L, k, per_expert, wts, n_out, n_in);
}

// Device memory of nmq_moe_down_static: the slot results of the two-launch form (one copy per GPU the
// library runs on, held until the process ends).  Host code never passes `scratch` itself to a kernel (on
// the host it names a stand-in, not the device address): the address comes from hipGetSymbolAddress, taken
// once per device with that device current.  Every element a call reads was written by the same call, so
// nothing needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[NMQ_MOE_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_at[64];

static int scratch_address(void** at) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return NMQ_ERR_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_at[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return NMQ_ERR_DEVICE;
        g_scratch_at[dev] = ptr;
    }
    *at = g_scratch_at[dev];
    return NMQ_OK;
}

// The checked call on a workspace of at least moe_work_bytes(...) bytes at `work`; p holds the weights, the
// expert table and the input (values or the two-stage input), whose slot rows are consecutive (x_group 1).
static int moe_launch(int fmt, MvParams p, int L, int k, const float* wts, float* out, float* work, hipStream_t s) {
    p.x_group = 1;
    p.n_ids = L * k;
    const Combine c{wts, out, k, 0};
    const int e = launch_moe_down_any(fmt, p, c, L, s);
    if (e != NMQ_ERR_SHAPE) return e;
    p.y = work;
    const int e2 = launch_any(fmt, p, 1, L * k, s);
    if (e2) return e2;
    const int64_t blocks = ((int64_t)L * p.n_out + 255) / 256;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (const float*)work, wts, L, k,
                       p.n_out, out);
    return (int)hipGetLastError();
}

static MvParams moe_values(const void* w, const int64_t* ids, int64_t per_expert, const void* x, int x_mode,
                           const void* x2, int n_out, int n_in) {
    MvParams p{};
    p.w = (const u8*)w;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xv = x;
    p.xv2 = x2;
    p.x_mode = x_mode;
    p.n_out = n_out;
    p.n_in = n_in;
    return p;
}

extern "C" {

int nmq_moe_down_work_bytes(int fmt, int L, int k, int n_out, int n_in, int64_t* bytes) {
    int bv, bb;
    if (!bytes || L < 1 || k < 1 || n_out < 1 || n_in < 1) return NMQ_ERR_ARG;
    if (nmq_format_info(fmt, &bv, &bb)) return NMQ_ERR_FORMAT;
    *bytes = moe_work_bytes(L, k, n_out, n_in);
    return NMQ_OK;
}

int nmq_moe_down(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const void* x,
                 int x_mode, const void* x2, const float* wts, float* out, int n_out, int n_in, void* work,
                 int64_t work_bytes, void* stream) {
    const int e = moe_check(fmt, w, ids, L, k, per_expert, x, x_mode, x2, wts, out, n_out, n_in);
    if (e) return e;
    const int64_t need = moe_work_bytes(L, k, n_out, n_in);
    if (need > 0 && (!work || !aligned(work, 256))) return NMQ_ERR_ARG;
    if (work_bytes < need) return NMQ_ERR_SHAPE;
    return moe_launch(fmt, moe_values(w, ids, per_expert, x, x_mode, x2, n_out, n_in), L, k, wts, out,
                      (float*)work, (hipStream_t)stream);
}

int nmq_moe_down_q8(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const int8_t* xq,
                    const int8_t* xq2, const float* xd, const float* xs, const float* wts, float* out, int n_out,
                    int n_in, void* work, int64_t work_bytes, void* stream) {
    int e = check_mv(fmt, w, xq, xq2, xd, xs, out, n_out, n_in);
    if (e) return e;
    if ((e = moe_check_slots(fmt, w, ids, L, k, per_expert, wts, n_out, n_in))) return e;
    const int64_t need = moe_work_bytes(L, k, n_out, n_in);
    if (need > 0 && (!work || !aligned(work, 256))) return NMQ_ERR_ARG;
    if (work_bytes < need) return NMQ_ERR_SHAPE;
    MvParams p{};
    p.w = (const u8*)w;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xq = xq;
    p.xq2 = xq2;
    p.xd = xd;
    p.xs = xs;
    p.n_out = n_out;
    p.n_in = n_in;
    return moe_launch(fmt, p, L, k, wts, out, (float*)work, (hipStream_t)stream);
}

int nmq_moe_gate_up(int fmt, const void* w_gate, const void* w_up, const int64_t* ids, int L, int k,
                    int64_t per_expert, const void* x, int x_mode, int8_t* xq, int8_t* xq2, float* xd, float* xs,
                    int n_out, int n_in, void* stream) {
    int e = check_mv(fmt, w_gate, xq, xq2, xd, xs, xd, n_out, n_in);
    if (e) return e;
    if ((e = check_w(fmt, w_up, xd, n_out, n_in))) return e;
    if (x_mode == NMQ_X_SILU_MUL_BF16) return NMQ_ERR_ARG;
    if ((e = check_values(x, x_mode, nullptr, n_in))) return e;
    if (!ids || L < 1 || k < 1 || (int64_t)L * k > 32767) return NMQ_ERR_ARG;
    if (n_out % 32) return NMQ_ERR_SHAPE;
    if ((e = check_experts(fmt, w_gate, L * k, per_expert, k, n_out, n_in))) return e;
    if ((e = check_experts(fmt, w_up, L * k, per_expert, k, n_out, n_in))) return e;
    MvParams p{};
    p.w = (const u8*)w_gate;
    p.w2 = (const u8*)w_up;
    p.ids = ids;
    p.per_expert = per_expert;
    p.xv = x;
    p.x_mode = x_mode;
    p.n_out = n_out;
    p.n_in = n_in;
    p.x_group = k;
    p.n_ids = L * k;
    return launch_moe_gu_any(fmt, p, QuantOut{xq, xq2, xd, xs}, (hipStream_t)stream);
}

// ---- the expert layer (gate|up, activation, down, weighted combine) ------------------------------------------
// Workspace of nmq_moe_layer, in 256-byte aligned pieces: the two-stage activation (L*k*FF values), the down
// launch's workspace where it needs one, the fp32 gate|up results of the form for many tokens.
struct MoeLayerWork {
    int64_t xq, xq2, xd, xs, down, gu, total;
};

static int64_t up256(int64_t v) { return (v + 255) / 256 * 256; }

static MoeLayerWork moe_layer_work(int L, int k, int E, int FF) {
    MoeLayerWork w{};
    const int64_t n = (int64_t)L * k * FF;
    w.xq = 0;
    w.xq2 = w.xq + up256(n);
    w.xd = w.xq2 + up256(n);
    w.xs = w.xd + up256(n / 32 * 4);
    w.down = w.xs + up256(n / 32 * 4);
    w.gu = w.down + up256(moe_work_bytes(L, k, E, FF));
    w.total = w.gu + up256(2 * n * 4);
    return w;
}

int nmq_moe_layer_work_bytes(int L, int k, int E, int FF, int64_t* bytes) {
    if (!bytes || L < 1 || k < 1 || E < 1 || FF < 1 || (int64_t)L * k > 32767) return NMQ_ERR_ARG;
    *bytes = moe_layer_work(L, k, E, FF).total;
    return NMQ_OK;
}

int nmq_moe_layer(int fmt_gu, const void* w_gate, const void* w_up, int64_t per_gu, int fmt_down, const void* w_down,
                  int64_t per_down, const int64_t* ids, const float* wts, int L, int k, const void* x, int x_mode,
                  float* out, int E, int FF, void* work, int64_t work_bytes, void* stream) {
    int e = check_w(fmt_gu, w_gate, out, FF, E);
    if (e) return e;
    if ((e = check_w(fmt_gu, w_up, out, FF, E))) return e;
    if ((e = check_w(fmt_down, w_down, out, E, FF))) return e;
    if (x_mode == NMQ_X_SILU_MUL_BF16) return NMQ_ERR_ARG;
    if ((e = check_values(x, x_mode, nullptr, E))) return e;
    if (FF % 32 || FF > NMQ_X_MAX_N_IN) return NMQ_ERR_SHAPE;
    if ((int64_t)L * k > 32767) return NMQ_ERR_ARG;
    if ((e = moe_check_slots(fmt_down, w_down, ids, L, k, per_down, wts, E, FF))) return e;
    if ((e = check_experts(fmt_gu, w_gate, L * k, per_gu, k, FF, E))) return e;
    if ((e = check_experts(fmt_gu, w_up, L * k, per_gu, k, FF, E))) return e;
    const MoeLayerWork lw = moe_layer_work(L, k, E, FF);
    if (!work || !aligned(work, 256)) return NMQ_ERR_ARG;
    if (work_bytes < lw.total) return NMQ_ERR_SHAPE;
    u8* wb = (u8*)work;
    const hipStream_t s = (hipStream_t)stream;
    MvParams pg{};
    pg.w = (const u8*)w_gate;
    pg.w2 = (const u8*)w_up;
    pg.ids = ids;
    pg.per_expert = per_gu;
    pg.xv = x;
    pg.x_mode = x_mode;
    pg.n_out = FF;
    pg.n_in = E;
    pg.x_group = k;
    pg.n_ids = L * k;
    const QuantOut o{(int8_t*)(wb + lw.xq), (int8_t*)(wb + lw.xq2), (float*)(wb + lw.xd), (float*)(wb + lw.xs)};
    MvParams pd{};
    pd.w = (const u8*)w_down;
    pd.ids = ids;
    pd.per_expert = per_down;
    pd.xq = o.xq;
    pd.xq2 = o.xq2;
    pd.xd = o.xd;
    pd.xs = o.xs;
    pd.n_out = E;
    pd.n_in = FF;
    // gate|up with the activation, then the down launch on its two-stage input, while the gate|up
    // workgroups fit one per CU (measured on MI355X, 128 experts top-8: one token 13.6 us against 15.0 for
    // the form below, four tokens 31.6 against 27.5)
    if ((int64_t)(FF / 32) * L * k <= tune(TUNE_MOE_GU_WGS, device_info().cus)) {
        e = launch_moe_gu_any(fmt_gu, pg, o, s);
        if (e == NMQ_OK) return moe_launch(fmt_down, pd, L, k, wts, out, (float*)(wb + lw.down), s);
        if (e != NMQ_ERR_SHAPE) return e;
    }
    // gate and up into fp32 (the gathered launch), the down launch forming the activation in its staging
    float* gu = (float*)(wb + lw.gu);
    pg.y = gu;
    if ((e = launch_any(fmt_gu, pg, 1, 2 * L * k, s))) return e;
    const int64_t n = (int64_t)L * k * FF;
    return moe_launch(fmt_down, moe_values(w_down, ids, per_down, gu, NMQ_X_SILU_MUL_BF16, gu + n, E, FF), L, k, wts,
                      out, (float*)(wb + lw.down), s);
}

int nmq_moe_down_static(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const void* x,
                        int x_mode, const void* x2, const float* wts, float* out, int n_out, int n_in, void* stream) {
    int e = moe_check(fmt, w, ids, L, k, per_expert, x, x_mode, x2, wts, out, n_out, n_in);
    if (e) return e;
    const int64_t need = moe_work_bytes(L, k, n_out, n_in);
    if (need > NMQ_MOE_SCRATCH_BYTES) return NMQ_ERR_SHAPE;
    void* work = nullptr;
    if ((e = scratch_address(&work))) return e;
    return moe_launch(fmt, moe_values(w, ids, per_expert, x, x_mode, x2, n_out, n_in), L, k, wts, out,
                      (float*)work, (hipStream_t)stream);
}

int nmq_block_sums(int fmt, const void* w, const int8_t* xq, const int8_t* xq2, int32_t* s1, int32_t* s2, int n_out,
                   int n_in, void* stream) {
    int bv, bb;
    if (nmq_format_info(fmt, &bv, &bb)) return NMQ_ERR_FORMAT;
    if (!w || !xq || !xq2 || !s1 || !s2 || !aligned(xq, 16) || !aligned(xq2, 16) || !aligned(w, 16))
        return NMQ_ERR_ARG;
    if (n_out < 1 || n_in < bv || n_in % bv || n_in > (1 << 20)) return NMQ_ERR_SHAPE;
    const int64_t threads = (int64_t)n_out * ((n_in + 63) / 64);
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    return launch_fmt_kernel<SumsK>(fmt, dim3((unsigned)blocks), (hipStream_t)stream, (const u8*)w, xq, xq2, s1, s2,
                                    n_out, n_in);
}

int nmq_stream_read(const void* src, int64_t n_bytes, uint32_t* sink, int waves_per_cu, int wg_waves, int unroll,
                    void* stream) {
    if (!src || !sink || !aligned(src, 16) || n_bytes % 16) return NMQ_ERR_ARG;
    if (n_bytes <= 0 || waves_per_cu < 1 || waves_per_cu > 32 || wg_waves < 1 || wg_waves > 16 ||
        waves_per_cu % wg_waves)
        return NMQ_ERR_SHAPE;
    const DeviceInfo di = device_info();
    const int nt = 64 * wg_waves;
    const unsigned grid = (unsigned)((int64_t)di.cus * waves_per_cu / wg_waves);
    const hipStream_t s = (hipStream_t)stream;
    switch (unroll) {
        case 1: hipLaunchKernelGGL(stream_read_kernel<1>, dim3(grid), dim3(nt), 0, s, (const u32x4*)src, n_bytes / 16, sink, nt); break;
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(grid), dim3(nt), 0, s, (const u32x4*)src, n_bytes / 16, sink, nt); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(nt), 0, s, (const u32x4*)src, n_bytes / 16, sink, nt); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(nt), 0, s, (const u32x4*)src, n_bytes / 16, sink, nt); break;
        default: return NMQ_ERR_ARG;
    }
    return (int)hipGetLastError();
}

int nmq_dequant_bf16(int fmt, const void* w, uint16_t* out, int64_t n_blocks, void* stream) {
    int bv, bb;
    if (nmq_format_info(fmt, &bv, &bb)) return NMQ_ERR_FORMAT;
    if (!w || !out || !aligned(out, 16) || !aligned(w, fmt == NMQ_Q4_K ? 16 : 2)) return NMQ_ERR_ARG;
    if (n_blocks < 1) return NMQ_ERR_SHAPE;
    const int64_t threads = bv == 32 ? (n_blocks + 1) / 2 : n_blocks * 4;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffff) return NMQ_ERR_SHAPE;
    return launch_fmt_kernel<DeqK>(fmt, dim3((unsigned)blocks), (hipStream_t)stream, (const u8*)w, (u16*)out,
                                   n_blocks);
}

}  // extern "C"
