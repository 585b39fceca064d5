/*
 * nmq.h -- C ABI of the MI355X (gfx950) GGUF quantized mat-vec library (libnmq.so).
 *
 * Plain pointers and sizes only.  Every device pointer is a HIP device address (a torch tensor's
 * data_ptr() on ROCm).  `stream` is a hipStream_t passed as void* (torch.cuda.current_stream()
 * .cuda_stream); NULL means the null stream.  No entry point allocates, frees or synchronises:
 * launches are asynchronous on `stream` and may be captured in a HIP graph.
 *
 * Return value: 0 on success; a negative NMQ_ERR_* for a rejected argument (nothing launched); a
 * positive hipError_t if the launch itself failed.  nmq_strerror() names either kind.
 *
 * Format ids are the GGML type ids (reference ggufengine/gguf.py:64-78).
 */
#ifndef NMQ_H
#define NMQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NMQ_Q4_0 2     /* 32 values, 18 bytes: fp16 d, qs[16] (lo nibbles 0..15, hi 16..31), d*(q-8) */
#define NMQ_Q8_0 8     /* 32 values, 34 bytes: fp16 d, int8 qs[32]                             */
#define NMQ_Q4_K 12    /* 256 values, 144 bytes: fp16 d, dmin, scales[12], qs[128]              */
#define NMQ_Q6_K 14    /* 256 values, 210 bytes: ql[128], qh[64], int8 sc[16], fp16 d           */
#define NMQ_IQ2_XXS 16 /* 256 values, 66 bytes: fp16 d, 8 x {u32 grid idx, u32 signs+scale}     */
#define NMQ_TQ2_0 35   /* 256 values, 66 bytes: qs[64] (2-bit codes), fp16 d                    */

#define NMQ_OK 0
#define NMQ_ERR_FORMAT (-1) /* unknown or unsupported format id                                  */
#define NMQ_ERR_SHAPE (-2)  /* n_in not a multiple of the block size, sizes <= 0 or too large      */
#define NMQ_ERR_ARG (-3)    /* NULL pointer where one is required, bad count                       */
#define NMQ_ERR_DEVICE (-4) /* no usable device / not a gfx950 device                             */

/* Tokens handled by one launch of the dot4 mat-vec kernels (the matrix-core kernel takes up to twice
 * as many); nmq_mv loops over larger counts. */
#define NMQ_MAX_COLS 8

/* ABI version of this header, bumped on incompatible changes (2: nmq_quant_q8 mode 2, the fused
 * expert entry points). */
int nmq_abi_version(void);

/* Text for a return code of any entry point (static storage). */
const char* nmq_strerror(int code);

/*
 * Launch-plan overrides for timing runs and tests (no counterpart in the reference, whose kernels
 * take their launch shape from constants in mmvq.py:25-37 and cudakern.py:31-54).  name: a knob of
 * the launch planner without or with the "NMQ_" prefix (MV1, MV1_MODE, MV1_HR, MV1_WPC, MV1_W,
 * MV1_RW, MV1_NBUF, MV1_MAXNIT, MVL, MVL_WPC, MVL_W, MVC_WGPC, MVC_RW, MVC_ROWS, MVT_MAX, MVT_WPC,
 * MVLT_MAX, MVM, MVM_TPW, MVM_KS, MMH_T, MMH_G, MVK, MVK_WPC, MVK_HR, MVK_NBUF, MVD, MVD_MIN, MVD_TPW,
 * MVD_KS, MVD_WGPC, MVD_LONG, MVD_UNEQ, MV1_T, MOE_GU_RW, MOE_GU_WGS, MVP_RPW, MVP_WGS); value
 * NMQ_TUNE_DEFAULT restores the measured default.
 * Process-wide, read by every later launch; the environment is never consulted.  NMQ_ERR_ARG for an
 * unknown name.  nmq_get_tuning writes the override or NMQ_TUNE_DEFAULT.
 */
#define NMQ_TUNE_DEFAULT (-2147483647 - 1)
int nmq_set_tuning(const char* name, int value);
int nmq_get_tuning(const char* name, int* value);

/* Values and bytes per block of a format; returns NMQ_OK or NMQ_ERR_FORMAT.
 * Replaces the table lookups GGML_TYPES[...] (gguf.py:64-78), mmvq.FORMATE (mmvq.py:25) and
 * cudakern.FORMATE (cudakern.py:42-49) for the five formats of this library. */
int nmq_format_info(int fmt, int* block_values, int* block_bytes);

/* Name of the current device's architecture (e.g. "gfx950") into buf; NMQ_OK or NMQ_ERR_DEVICE.
 * Replaces the availability probe behind mmvq.verfuegbar / cudakern.verfuegbar
 * (mmvq.py:792-810, cudakern.py:717-739): the kernels exist only for gfx950. */
int nmq_device_arch(char* buf, int len);

/*
 * Two-stage int8 activation ("Eingang").  Replaces the `quant_q8` launch of mmvq.Eingang
 * (mmvq.py:62-83, 825-843).  x: n values, n % 32 == 0; several token rows may be passed back to
 * back.  x_is_f32: 0 bf16; 1 fp32; 2 fp32 rounded to bf16 first (nearest even), the input the
 * reference's cudakern entry points form (cudakern.py:764).  Per 32 values g:
 *   xd[g] = max|x| / 127, xq = rint(x / xd), xq2 = clamp(rint((x - xq*xd) / (xd/254)), +-127),
 *   xs[g] = sum of the 32 values.
 */
int nmq_quant_q8(const void* x, int x_is_f32, int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n,
                 void* stream);

/*
 * The gated activation of an expert MLP, made the down projection's two-stage input in one launch:
 * a = bf16(silu(g) * u) (silu(g) = g / (1 + exp(-g)), fp32, then rounded to bf16 nearest even),
 * then the two-stage quantisation of nmq_quant_q8.  g, u: fp32[n], n % 32 == 0.  Replaces the
 * `silu(gate) * up` of Experten._gu (models/moe.py:252-255) followed by cudakern.mv's bf16 cast and
 * the input quantisation of the down call (the reference's fused one-token path does the same in
 * mmvq.akt_q8, mmvq.py:959-966).
 */
int nmq_silu_mul_quant(const float* g, const float* u, int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n,
                       void* stream);

/* Largest row nmq_norm_q8 takes (one workgroup per row). */
#define NMQ_NORM_MAX 65536

/*
 * RMS norm of one row fused with its two-stage input.  With r: v = h + rs*r, written to hout
 * (hout must not overlap h or r); without r (NULL): v = h and hout is not used.  Then
 *   inv = 1 / sqrt(sum(v^2) / n + eps),  xn = (v * inv) * w,
 * and (xq, xq2, xd, xs) = the two-stage input of xn, as nmq_quant_q8 forms it from fp32.  Every fp32
 * operation is rounded on its own (no fused multiply-add) except the sum of squares.  h, r, w, hout,
 * xn: fp32[n]; n % 32 == 0, n <= NMQ_NORM_MAX.  One workgroup.
 * Replaces the norm_q8 kernel and wrapper of mmvq (mmvq.py:102-120, 951-961).
 */
int nmq_norm_q8(const float* h, const float* r, float rs, float* hout, const float* w, float eps, float* xn,
                int8_t* xq, int8_t* xq2, float* xd, float* xs, int64_t n, void* stream);

/*
 * a = act(g) * u (u NULL: a = act(g)), act(x) = x / (1 + exp(-x)) (gelu == 0) or
 * 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))) (gelu == 1), fp32, written to a, and the
 * two-stage input of a.  g, u, a: fp32[n], n % 32 == 0.
 * Replaces the akt_q8 kernel and wrapper of mmvq (mmvq.py:122-133, 964-971).
 */
int nmq_akt_q8(const float* g, const float* u, int gelu, float* a, int8_t* xq, int8_t* xq2, float* xd, float* xs,
               int64_t n, void* stream);

/*
 * y[c][r] = W[r,:] . x_c for c < ncols tokens (any ncols >= 1; launches of up to 2 * NMQ_MAX_COLS
 * tokens on the matrix cores, NMQ_MAX_COLS on the dot4 kernels; 9..16 tokens as two launches of up to 8
 * where the dense-read matrix-core kernel takes the shape; rows beyond 4096 values that do not split
 * into equal aligned K ranges: one launch per range, each adding to y in range order).  2..4 tokens of
 * Q4_K with rows of up
 * to 4096 values, or of Q6_K with rows of 8K..16K values: every token's output equals the ncols = 1 call
 * on that token bit for bit.
 * w: n_out rows of n_in values in GGUF block format, rows back to back.  Token c's two-stage input
 * lies at xq + c*n_in, xq2 + c*n_in, xd + c*n_in/32, xs + c*n_in/32 (the layout of an Eingang of
 * ncols rows).  y: fp32, token-major (ncols x n_out).
 * Replaces the mvq_<fmt>_<nc> launches of mmvq.mv (mmvq.py:341-489, 852-865) and the mv/mm
 * kernels of cudakern for one matrix (cudakern.py:482-555, 756-790).
 * n_in % block_values == 0 (Q8_0: 32, others 256), 1 <= n_out, n_in <= 1<<20.
 */
int nmq_mv(int fmt, const void* w, const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs,
           float* y, int n_out, int n_in, int ncols, void* stream);

/*
 * Two-stage fp16 input of nmq_mm for ncols token rows of n_in values (x: fp32 if x_is_f32 else bf16,
 * rows back to back): per row xs = 2^(e - 8) where max|x| = f * 2^e, f in [0.5, 1) (e >= -100),
 * v = x / xs (exact), xh = fp16(v), xl = fp16(v - xh), rounded to nearest even (xh + xl is v to
 * about 2^-22), and per 32 values the fp32 sum of xh + xl.  xs: ncols fp32.  xh, xl: ceil(ncols/16)*16
 * rows of n_in fp16 each (16-byte aligned), xsum: ceil(ncols/16)*16 rows of n_in/32 fp32, in the
 * matrix cores' operand order:
 *   xh, xl: value k of token t at ((t/16 * (n_in/32) + k/32) * 64 + (k%32)/8 * 16 + t%16) * 8 + k%8
 *   xsum:   sub-block s of token t at (t/16 * (n_in/32) + s) * 16 + t%16
 * (the rows past ncols are written as zeros; the sign of a zero in xh, xl is not specified).
 * n_in % 32 == 0, n_in <= 1<<20.
 * Replaces the mmq_eingang launch of mmvq._mmq_eingang (mmvq.py:617-641, 882-899), which keeps one
 * fp16 stage scaled by max|x| / 256.
 */
int nmq_mm_input(const void* x, int x_is_f32, uint16_t* xh, uint16_t* xl, float* xsum, float* xs, int n_in,
                 int ncols, void* stream);

/*
 * Several tokens on the fp16 matrix cores (Q4_K and Q6_K; other formats NMQ_ERR_FORMAT):
 *   y[c][r] = xs[c] * sum_k w[r][k] * (xh + xl)[c][k]
 * with w the exact dequantised weights: per 256-value block, d times the integer products q*sc
 * (Q4_K; Q6_K as (8h + l)*sc with q - 32 = 8h + l, every part exact in fp16) summed with the input on
 * the matrix cores (exact products, fp32 sums), minus dmin * sum_s mn_s * xsum_s (Q4_K, an fp32
 * matrix product).  xh, xl, xsum, xs from nmq_mm_input for the same ncols and n_in.  Up to 64 tokens
 * per launch; larger ncols loop.  y: fp32, token-major (ncols x n_out).
 * Replaces the mmq_<fmt>_<nt> launches of mmvq.mm (mmvq.py:536-724, 902-920), which round the
 * weights and the input to fp16; y written directly instead of split-K atomic adds into zeros.
 * n_in % 256 == 0, 1 <= n_out, n_in <= 1<<20; w 16-byte aligned for Q4_K.
 */
int nmq_mm(int fmt, const void* w, const uint16_t* xh, const uint16_t* xl, const float* xsum, const float* xs,
           float* y, int n_out, int n_in, int ncols, void* stream);

/* Most matrices one nmq_mv_multi call takes. */
#define NMQ_MAX_MATS 4

/*
 * Several matrices of one format and row length applied to one token's input in one launch:
 *   y_i[r] = W_i[r,:] . x   for i < n_mats, r < n_outs[i],
 * ws[i]: matrix i's rows (GGUF block format, rows back to back), ys[i]: its fp32 outputs; ws, n_outs
 * and ys are host arrays of n_mats (1..NMQ_MAX_MATS) entries.  The input as for nmq_mv (one token).
 * The rows of all matrices are scheduled as one matrix, so small matrices share the launch and its
 * fixed cost.  Replaces consecutive mmvq.mv / PackedLinear calls on one shared Eingang (q, k, v and
 * gate, up inside mmvq.eingang_teilen, models/baukasten.py:140-143, 259-260); each output equals what
 * nmq_mv gives for that matrix alone.
 */
int nmq_mv_multi(int fmt, int n_mats, const void* const* ws, const int* n_outs, float* const* ys,
                 const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int n_in, void* stream);

/*
 * Input given as values instead of an Eingang (nmq_mv_x, nmq_mv_experts_x): each launch forms the
 * two-stage input itself, bit for bit what nmq_quant_q8 (or nmq_silu_mul_quant) writes, and saves
 * that launch.  x_mode:
 */
#define NMQ_X_BF16 0          /* bf16 values                                                     */
#define NMQ_X_F32 1           /* fp32 values                                                     */
#define NMQ_X_F32_BF16 2      /* fp32 values rounded to bf16 first (the cudakern input convention)*/
#define NMQ_X_SILU_MUL_BF16 3 /* bf16(silu(x) * x2), x and x2 fp32 (the down input of an expert)  */
#define NMQ_X_MAX_N_IN 16384  /* longest row (values) of a launch with value input                */

/*
 * nmq_mv_multi with the token given as values: x (n_in values, mode x_mode; x2 the second operand of
 * NMQ_X_SILU_MUL_BF16, else NULL), 16-byte aligned (8 for bf16).  n_in % 32 == 0, n_in <=
 * NMQ_X_MAX_N_IN.  Replaces the quant_q8 launch of mmvq.Eingang plus the mat-vec launch(es) of
 * mmvq.mv on a tensor (mmvq.py:852-865) with one launch.
 */
int nmq_mv_x(int fmt, int n_mats, const void* const* ws, const int* n_outs, float* const* ys, const void* x,
             int x_mode, const void* x2, int n_in, void* stream);

/*
 * Expert-id-gathered mat-vec with the input given as values: y[j] = A_{ids[j]} x_(j / x_group) for
 * j < n_ids, and with a second tensor w_b (else NULL) also y[n_ids + j] = B_{ids[j]} x_(j / x_group)
 * (n_ids <= 32767 then).  x: rows of n_in values (mode x_mode; x2 likewise for NMQ_X_SILU_MUL_BF16).
 * Otherwise as nmq_mv_experts / nmq_mv_experts2.  Replaces the input quantisation plus the gathered
 * launch(es) of cudakern.mv with ids (cudakern.py:756-774) and, with NMQ_X_SILU_MUL_BF16, the
 * silu(gate) * up of Experten (models/moe.py:252-255) in front of the down call.
 */
int nmq_mv_experts_x(int fmt, const void* w_a, const void* w_b, const int64_t* ids, int n_ids, int64_t per_expert,
                     const void* x, int x_mode, const void* x2, int x_group, float* y, int n_out, int n_in,
                     void* stream);

/*
 * Expert-id-gathered mat-vec (MoE): for j < n_ids,
 *   y[j][r] = W_{ids[j]}[r,:] . x_(j / x_group)
 * Weights of expert e start at w + e*per_expert (per_expert >= 0, bytes), or, with per_expert < 0,
 * at the address ((const int64_t*)w)[e] (a device table of expert addresses: VRAM slots or mapped
 * pinned host memory).  ids: int64 on the device (read by the kernel, so a captured graph follows
 * new ids without a host sync).  x_group = n_ids: one input shared by all experts (gate/up of one
 * token); x_group = 1: every expert has its own input row (down); x_group = k: rows of k slots per
 * token.  y: fp32 (n_ids x n_out).
 * Replaces cudakern.mv with ids / adressen (cudakern.py:482-505, 756-774) as called by
 * PackedExperts.matvec / matvec_je (models/common.py:462-475).
 */
int nmq_mv_experts(int fmt, const void* w, const int64_t* ids, int n_ids, int64_t per_expert,
                   const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int x_group,
                   float* y, int n_out, int n_in, void* stream);

/*
 * Two expert tensors of the same format and shape (gate and up) on the same ids and inputs in one
 * launch: y[j] = A_{ids[j]} x_(j / x_group) and y[n_ids + j] = B_{ids[j]} x_(j / x_group) for
 * j < n_ids (n_ids <= 32767); w_a, w_b, per_expert as in nmq_mv_experts.  y: fp32 (2 n_ids x n_out).
 * Replaces the gate and up calls of Experten (models/moe.py:270-274, PackedExperts.matvec), two
 * launches of the gathered kernel, with one.
 */
int nmq_mv_experts2(int fmt, const void* w_a, const void* w_b, const int64_t* ids, int n_ids, int64_t per_expert,
                    const int8_t* xq, const int8_t* xq2, const float* xd, const float* xs, int x_group,
                    float* y, int n_out, int n_in, void* stream);

/*
 * Weighted combine of expert outputs: out[t][e] = sum_{j<k} w[t*k + j] * y[t*k + j][e], the slots j
 * added in order (fp32 fused multiply-adds).  y: fp32 (L*k x E), w: fp32 (L x k), out: fp32 (L x E).
 * Replaces the `(y * w).sum(...)` combine of Experten.__call__ (models/moe.py:275-277, 319-320).
 */
int nmq_moe_combine(const float* y, const float* w, int L, int k, int E, float* out, void* stream);

/*
 * The down projection of an expert layer fused with the weighted combine:
 *   out[t][r] = sum_{j<k} wts[t*k + j] * (W_{ids[t*k + j]}[r,:] . x_(t*k + j)),   t < L, r < n_out,
 * each slot's product exactly as nmq_mv_experts_x forms it (x_group = 1: slot t*k + j reads input row
 * t*k + j of x, mode x_mode, x2 for NMQ_X_SILU_MUL_BF16), the slots summed in order j = 0..k-1 with fp32
 * fused multiply-adds (bit for bit nmq_moe_combine on those products).  ids: L*k int64 on the device;
 * wts: L*k fp32; out: fp32 L x n_out; w, per_expert as in nmq_mv_experts; n_in <= NMQ_X_MAX_N_IN.
 * Rows of up to 4096 values and k <= 16: one launch, each workgroup computing a block of rows for all k
 * slots of one token and summing them in LDS (no workspace: nmq_moe_down_work_bytes reports 0).  Other
 * shapes: the gathered launch writes the L*k slot results into `work` (nmq_moe_down_work_bytes bytes,
 * 256-byte aligned) and a second launch sums them; calls that overlap in time must not share it.
 * NMQ_ERR_SHAPE when work_bytes is too small.
 * Replaces the down call of Experten.__call__ plus its weighted combine (models/moe.py:264-277, 319-320;
 * cudakern.mv with ids, cudakern.py:756-774).
 */
int nmq_moe_down_work_bytes(int fmt, int L, int k, int n_out, int n_in, int64_t* bytes);
int nmq_moe_down(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const void* x,
                 int x_mode, const void* x2, const float* wts, float* out, int n_out, int n_in, void* work,
                 int64_t work_bytes, void* stream);

/*
 * The gate and up projections of a dense FFN with the activation, one token:
 *   a[r] = act(W_gate[r,:] . x) * (W_up[r,:] . x),   r < n_out,
 * act: NMQ_ACT_SILU or NMQ_ACT_GELU as nmq_akt_q8 forms them, | NMQ_ACT_BF16 to round a to bf16 (as
 * nmq_silu_mul_quant does for silu); each product exactly as nmq_mv_x forms it from the same x and x_mode
 * (NMQ_X_F32 or NMQ_X_F32_BF16).  Writes the two-stage input of a (n_out values) to xq, xq2 (16-byte
 * aligned), xd, xs: bit for bit nmq_mv_x on both matrices followed by nmq_akt_q8 (or nmq_silu_mul_quant),
 * in one launch and without the fp32 outputs.  Q4_K, TQ2_0 and IQ2_XXS, rows of at most 4096 values,
 * n_out % 32 == 0; NMQ_ERR_SHAPE otherwise (the caller then takes the two launches).
 * Replaces the gate and up calls of the FFN and the activation between them and the down call (the
 * reference's one-token step: mmvq mv on gate and up, then akt_q8, mmvq.py:122-133, 964-971).
 */
#define NMQ_ACT_SILU 0
#define NMQ_ACT_GELU 1
#define NMQ_ACT_BF16 2
int nmq_mv_gate_up_act(int fmt, const void* w_gate, const void* w_up, const void* x, int x_mode, int act,
                       int8_t* xq, int8_t* xq2, float* xd, float* xs, int n_out, int n_in, void* stream);

/*
 * The gate and up projections of an expert layer with the gated activation in the same launch: for slot
 * s = t*k + j (t < L) and row r < n_out,
 *   g = W_gate_{ids[s]}[r,:] . x_t,   u = W_up_{ids[s]}[r,:] . x_t,   a[s][r] = bf16(silu(g) * u),
 * g and u exactly as nmq_mv_experts_x forms them (x_group = k; x_mode NMQ_X_BF16, NMQ_X_F32 or
 * NMQ_X_F32_BF16), silu(g) * u as nmq_silu_mul_quant forms it, and writes the two-stage input of a
 * (L*k x n_out values, slot-major) to xq, xq2 (16-byte aligned), xd, xs -- bit for bit what
 * nmq_mv_experts_x followed by nmq_silu_mul_quant writes.  Each workgroup computes 32 rows of both
 * projections of one slot and quantises them as one group, so g and u are never written.  Requires
 * n_out % 32 == 0 and rows of at most 4096 values (NMQ_ERR_SHAPE otherwise); L*k <= 32767.
 * Replaces the gate and up calls of Experten.__call__ and the activation between them and the down call
 * (models/moe.py:270-276 and 278-285: the gate and up matvecs, then Experten._gu, 252-255).
 */
int nmq_moe_gate_up(int fmt, const void* w_gate, const void* w_up, const int64_t* ids, int L, int k,
                    int64_t per_expert, const void* x, int x_mode, int8_t* xq, int8_t* xq2, float* xd, float* xs,
                    int n_out, int n_in, void* stream);

/*
 * nmq_moe_down on the two-stage input (slot s = t*k + j reads row s of xq, xq2, xd, xs: what
 * nmq_moe_gate_up writes), each slot's product exactly as nmq_mv_experts forms it with x_group = 1;
 * workspace, combine and errors as nmq_moe_down (nmq_moe_down_work_bytes sizes `work` for both).
 * Replaces the down call of Experten.__call__ plus its weighted combine (models/moe.py:276-277, 284-285).
 */
int nmq_moe_down_q8(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const int8_t* xq,
                    const int8_t* xq2, const float* xd, const float* xs, const float* wts, float* out, int n_out,
                    int n_in, void* work, int64_t work_bytes, void* stream);

/*
 * The whole expert layer of an MoE block: for token t < L with slots s = t*k + j (expert ids[s], weight
 * wts[s]),
 *   a_s = bf16(silu(W_gate_{ids[s]} . x_t) * (W_up_{ids[s]} . x_t)),   out[t] = sum_j wts[s] * (W_down_{ids[s]} . a_s),
 * bit for bit nmq_moe_gate_up followed by nmq_moe_down_q8 (and so nmq_mv_experts_x, nmq_silu_mul_quant,
 * nmq_mv_experts and nmq_moe_combine).  Gate and up: fmt_gu, FF x E, experts per_gu bytes apart (or address
 * tables, per_gu < 0); down: fmt_down, E x FF, per_down; x: L x E values (NMQ_X_BF16, NMQ_X_F32 or
 * NMQ_X_F32_BF16); out: fp32 L x E; FF % 32 == 0; L*k <= 32767.
 * work: nmq_moe_layer_work_bytes(L, k, E, FF) bytes, 256-byte aligned (no clearing needed); calls that
 * overlap in time must not share it.  Two launches: nmq_moe_gate_up + nmq_moe_down_q8 while the gate|up
 * workgroups ((FF / 32) * L * k) fit one per CU and the rows fit that kernel (E <= 4096), else the gathered
 * gate|up launch into fp32 (in `work`) followed by nmq_moe_down forming the activation in its staging.
 * Replaces Experten.__call__ (models/moe.py:264-277).
 */
int nmq_moe_layer_work_bytes(int L, int k, int E, int FF, int64_t* bytes);
int nmq_moe_layer(int fmt_gu, const void* w_gate, const void* w_up, int64_t per_gu, int fmt_down, const void* w_down,
                  int64_t per_down, const int64_t* ids, const float* wts, int L, int k, const void* x, int x_mode,
                  float* out, int E, int FF, void* work, int64_t work_bytes, void* stream);

/*
 * nmq_moe_down without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid allocation); no counterpart in the reference.
 * The two-launch form keeps its slot results in a device array inside the library, one per GPU, of
 * NMQ_MOE_SCRATCH_BYTES bytes (held until the process ends): shapes whose L*k x n_out fp32 results do not
 * fit are refused with NMQ_ERR_SHAPE.  It allocates nothing.  Calls that overlap in time on one GPU share
 * that array and race; nothing needs clearing between calls (a call reads only what it wrote).
 * Otherwise identical to nmq_moe_down (results bit for bit equal).
 */
#define NMQ_MOE_SCRATCH_BYTES (8 << 20)
int nmq_moe_down_static(int fmt, const void* w, const int64_t* ids, int L, int k, int64_t per_expert, const void* x,
                        int x_mode, const void* x2, const float* wts, float* out, int n_out, int n_in, void* stream);

/*
 * Diagnostic: the int32 sums the mat-vec kernels form, per 16 weights, for one token:
 *   s1[r][g] = sum_{j<16} w_int(r, 16g+j) * xq[16g+j],  s2 likewise with xq2,
 * where w_int is the format's integer weight (Q4_K nibble, Q6_K q-32, Q8_0 qs, TQ2_0 code-1,
 * IQ2_XXS +-grid byte).  s1, s2: int32 (n_out x n_in/16).  Uses the same device decoders as
 * nmq_mv; exists so the integer part can be checked bit-exactly.  No counterpart in the reference
 * (its kernels keep these sums in registers, mmvq.py:385-396).
 */
int nmq_block_sums(int fmt, const void* w, const int8_t* xq, const int8_t* xq2, int32_t* s1, int32_t* s2,
                   int n_out, int n_in, void* stream);

/*
 * Unpack n_blocks blocks to bf16 values (uint16 bit patterns), the exact fp32 dequantisation of
 * quant.py rounded to bf16.  Replaces mmvq.entpacken / aus_<fmt> (mmvq.py:496-534, 923-931) and
 * the unpack step of the PackedLinear fallback (models/common.py:414-428).
 */
int nmq_dequant_bf16(int fmt, const void* w, uint16_t* out, int64_t n_blocks, void* stream);

/*
 * Diagnostic: a pure streaming read of n_bytes at src (16-byte aligned, n_bytes % 16 == 0) with 16-byte
 * loads, `unroll` (1, 2, 4, 8) in flight per thread, waves_per_cu (1..32) resident waves per CU in
 * workgroups of wg_waves (1..16, dividing waves_per_cu) waves; writes at most one word to sink.  The
 * reference point for what one launch of that size can read from HBM (the mat-vec kernels read the same
 * weight bytes plus their input).  No counterpart in the reference.
 */
int nmq_stream_read(const void* src, int64_t n_bytes, uint32_t* sink, int waves_per_cu, int wg_waves, int unroll,
                    void* stream);

/* ---- host-side encoders (CPU, no device involved) -----------------------------------------------
 * Write n values (n % block_values == 0) of fp32 weights into GGUF blocks at out
 * (n / block_values * block_bytes bytes).  Return the number of bytes written, or a negative
 * NMQ_ERR_*.  The reference ships no quantiser for Q4_K, Q6_K or IQ2_XXS; these are this library's
 * own (the mat-vec is checked against the dequantisation of the same bytes, so the encoder only
 * decides how realistic the weights are).  threads <= 0: all cores.
 */
int64_t nmq_encode(int fmt, const float* w, int64_t n, uint8_t* out, int threads);

#ifdef __cplusplus
}
#endif

#endif /* NMQ_H */
