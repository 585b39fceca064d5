/*
 * CPU baseline for bench.py -- TEST INFRASTRUCTURE ONLY (timed beside the GPU path, never shipped).
 *
 * Restates the reference's CPU path for one linear layer:
 *   - Q4_K / Q6_K / Q8_0 go through models/common.py:190 `Linear(self.get(name))`: the matrix is
 *     dequantised once at load time and each call is F.linear, an fp32 GEMV (common.py:526-527).
 *     or_gemv_f32 below is that GEMV (fp32 accumulation, OpenMP over rows).
 *   - TQ2_0 / IQ2_XXS go through the PackedLinear fallback (common.py:414-428), which dequantises a
 *     chunk of rows and multiplies it on every call: or_deq_gemv_f32.
 * Built with vectorisation and FMA allowed (this file is a baseline, not a parity oracle).
 */
#include <stdint.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_dequant(int fmt, const uint8_t* raw, int64_t n_blocks, float* out);
int or_format_info(int fmt, int* block_values, int* block_bytes);

static float dot_f32(const float* a, const float* b, int n) {
    float s[16] = {0};
    int k = 0;
    for (; k + 16 <= n; k += 16)
        for (int j = 0; j < 16; ++j) s[j] += a[k + j] * b[k + j];
    float t = 0.0f;
    for (; k < n; ++k) t += a[k] * b[k];
    for (int j = 0; j < 16; ++j) t += s[j];
    return t;
}

/* y[r] = sum_k w[r][k] x[k], rows split over `threads` OpenMP threads. */
void or_gemv_f32(const float* w, int n_out, int n_in, const float* x, float* y, int threads) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
    for (int r = 0; r < n_out; ++r) y[r] = dot_f32(w + (int64_t)r * n_in, x, n_in);
}

/* Dequantise-per-call GEMV: each thread dequantises its rows block by block and multiplies. */
int or_deq_gemv_f32(int fmt, const uint8_t* raw, int n_out, int n_in, const float* x, float* y, int threads) {
    int bv, bb;
    if (or_format_info(fmt, &bv, &bb) || n_in % bv) return -1;
    const int nb = n_in / bv;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
    for (int r = 0; r < n_out; ++r) {
        float row[16384];
        float acc = 0.0f;
        for (int k0 = 0; k0 < nb; k0 += 16384 / bv) {
            const int cnt = nb - k0 < 16384 / bv ? nb - k0 : 16384 / bv;
            or_dequant(fmt, raw + ((int64_t)r * nb + k0) * bb, cnt, row);
            acc += dot_f32(row, x + (int64_t)k0 * bv, cnt * bv);
        }
        y[r] = acc;
    }
    return 0;
}
