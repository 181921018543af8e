/*
 * myelin_hip.h -- C ABI of libmyelin_hip.so, the MI355X (gfx950) kernels of
 * myelin's fused-time spiking-neuron path.
 *
 * Conventions
 *   - Plain pointers to device memory, int64 sizes, fp32 scalars; no torch
 *     or HIP types.  `myelin_stream_t` is layout-compatible with hipStream_t
 *     (pass torch.cuda.current_stream().cuda_stream).
 *   - Every call is asynchronous on `stream`, allocates nothing, holds no
 *     global mutable state, and may be called from any host thread (the
 *     autograd engine runs backward on its own device thread).
 *   - Return value: 0 on success, MYELIN_EINVAL for a rejected argument,
 *     MYELIN_EHIP for a HIP launch error.  myelin_last_error() returns the
 *     message of the calling thread's last failure.
 *   - Time-major layout: a [T, B, N] tensor is passed as T rows of BN = B*N
 *     contiguous floats.  Chunk-start checkpoints are [ceil(T/chunk), BN]:
 *     row k holds the state *before* step k*chunk (row 0 = initial state).
 *
 * Citations are file:line in djsaunde/myelin (src/myelin/...).
 */
#ifndef MYELIN_HIP_H
#define MYELIN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *myelin_stream_t;

#define MYELIN_OK 0
#define MYELIN_EINVAL 1
#define MYELIN_EHIP 2

/* spike rules */
#define MYELIN_RULE_THRESHOLD 0 /* s = m' >= th            (neurons.py:112,124) */
#define MYELIN_RULE_SURROGATE 1 /* s = slope*(m' - th) >= 0 (surrogates.py:108) */
/* Rules that evaluate the surrogate primitive sigma(c), c = slope*(m' - th),
 * op by op in fp32 as myelin's torch backend does (surrogates.py:29-75) and
 * emit the spike value its autograd graph carries; the membrane then resets
 * as m = m'*(1 - s) + reset*s and ALIF adapts as a = a*rho + s
 * (functional.py:140-143,183-186).  Add the surrogate id (0-5).
 *   MYELIN_RULE_STRAIGHT_THROUGH + id: s = (H(c) + sigma(c)) - sigma(c),
 *     H(c) = c >= 0 (hard_surrogate_spike, surrogates.py:105-111); equal
 *     to 0 or within a few ulp of 1.
 *   MYELIN_RULE_SMOOTH + id: s = sigma(c) (hard_forward=False,
 *     functional.py:141,184).
 * Dense spikes only (packed output rejects them). */
#define MYELIN_RULE_STRAIGHT_THROUGH 16
#define MYELIN_RULE_SMOOTH 32

/* surrogate ids, same numbering as triton/lif.py:356-370 */
#define MYELIN_SG_SIGMOID 0
#define MYELIN_SG_FAST_SIGMOID 1
#define MYELIN_SG_ATAN 2
#define MYELIN_SG_TRIANGULAR 3
#define MYELIN_SG_SUPERSPIKE 4
#define MYELIN_SG_MULTI_GAUSSIAN 5
/* hard threshold, zero spike derivative: the adjoint of the plain
 * lif_unroll / alif_unroll through the membrane path only (their spikes
 * carry no gradient, functional.py:21-78) */
#define MYELIN_SG_NONE 6
/* Backward surrogate codes for a forward run with MYELIN_RULE_STRAIGHT_THROUGH
 * (resp. MYELIN_RULE_SMOOTH) + id: MYELIN_SG_AUTOGRAD (resp.
 * MYELIN_SG_AUTOGRAD_SMOOTH) + id.  The recompute reproduces that forward
 * and the adjoint is evaluated in the operation order and fp32 rounding of
 * torch autograd through surrogate_lif_unroll / surrogate_alif_unroll
 * (functional.py:115-189): per step, dL/ds = ((dL/ds_t + dL/da' +
 * dL/dm'' * reset) - dL/dm'' * m'), then the primitive's own backward
 * formulas (quotient rule for fast_sigmoid / superspike, sigmoid_backward,
 * atan's 1/(1+p^2), clamp mask, erf's 2/sqrt(pi)*exp(-z^2)).  Chunk 16 only
 * (chunk 8 rejects both codes with MYELIN_EINVAL).
 * The other codes (0-6) use the closed-form derivative sigma'(c) of
 * surrogates.py:78-102, as the reference's Triton kernels do
 * (triton/lif.py:225-249) with exact 0/1 spikes. */
#define MYELIN_SG_AUTOGRAD 16
#define MYELIN_SG_AUTOGRAD_SMOOTH 32

/* GEMM input precision (accumulation is always fp32) */
#define MYELIN_PREC_F32 0
#define MYELIN_PREC_BF16 1 /* inputs rounded to bf16 (nearest even) */

/* element type codes for pack / unpack */
#define MYELIN_DT_F32 0
#define MYELIN_DT_F16 1
#define MYELIN_DT_BF16 2
#define MYELIN_DT_U8 3 /* bool, uint8, int8 */
#define MYELIN_DT_I32 4
#define MYELIN_DT_I64 5
#define MYELIN_DT_F64 6
#define MYELIN_DT_BITS 7 /* packed spike bits: int32 words, bit i of word w = column 32w + i */
#define MYELIN_DT_BF16X3 8 /* three bf16 planes [3, ...] (hi, mid, lo) whose float sum is exact */

const char *myelin_last_error(void);
int myelin_abi_version(void);

/*
 * Fused-time LIF forward over T steps in one launch, state in registers.
 *   m' = m*decay + x_t ; s_t = rule(m', threshold) ; m = s_t ? reset : m'
 * spikes   [T, BN] fp32 0/1, or NULL when `packed` is given
 * packed   [T, B, ceil(N/32)] int32 words (bit i = neuron 32w+i), or NULL
 * ckpt_m   [ceil(T/chunk), BN] chunk-start membranes, or NULL
 * Replaces: _lif_forward_kernel + lif_forward (triton/lif.py:16-95),
 *   _surrogate_lif_forward_kernel + surrogate_lif_forward (triton/lif.py:195-222,
 *   373-405), _lif_forward_packed_spikes_kernel + lif_forward_packed_spikes
 *   (triton/lif.py:98-192); semantics of functional.py:21-45,115-146.
 */
int myelin_lif_fwd_f32(const float *x, const float *m0, float *m_final,
                       float *spikes, int32_t *packed, float *ckpt_m,
                       int64_t T, int64_t B, int64_t N, float decay,
                       float threshold, float reset, float slope, int rule,
                       int64_t chunk, myelin_stream_t stream);

/*
 * Fused-time ALIF forward.
 *   m' = m*decay + x ; th = threshold + beta*a ; s = rule(m', th)
 *   m = s ? reset : m' ; a = a*rho + s
 * Replaces: generated_alif_forward (triton/generated.py:1159-1189, whose
 *   step body is dsl.py:1064-1089) and the forward of surrogate_alif_unroll
 *   (functional.py:149-189); semantics of neurons.py:117-128.
 */
int myelin_alif_fwd_f32(const float *x, const float *m0, const float *a0,
                        float *m_final, float *a_final, float *spikes,
                        int32_t *packed, float *ckpt_m, float *ckpt_a,
                        int64_t T, int64_t B, int64_t N, float decay,
                        float rho, float threshold, float beta, float reset,
                        float slope, int rule, int64_t chunk,
                        myelin_stream_t stream);

/*
 * Reverse-time surrogate backward with chunked recompute: each chunk is
 * re-run forward from its checkpoint (x re-read once), staged in
 * registers, then walked backward.  grad_spikes / grad_m_final may be NULL.
 * chunk must be 8 or 16 (the value the forward used for ckpt_m).
 * surrogate_id MYELIN_SG_NONE recomputes with the threshold rule and
 * propagates only through the membrane (grad_spikes is then ignored).
 * Replaces: _surrogate_lif_backward_kernel + surrogate_lif_backward
 *   (triton/lif.py:252-288,408-475) together with the recompute Function
 *   (autograd.py:232-312).
 */
int myelin_lif_bwd_f32(const float *x, const float *ckpt_m,
                       const float *grad_spikes, const float *grad_m_final,
                       float *grad_x, float *grad_m0, int64_t T, int64_t BN,
                       float decay, float threshold, float reset, float slope,
                       int surrogate_id, int64_t chunk, myelin_stream_t stream);

/*
 * Two-state (membrane, adaptation) adjoint of surrogate_alif_unroll
 * (functional.py:149-189).  The reference has no fused kernel for it
 * (kernels.py:368-372 raise); this replaces its torch-autograd route.
 */
int myelin_alif_bwd_f32(const float *x, const float *ckpt_m,
                        const float *ckpt_a, const float *grad_spikes,
                        const float *grad_m_final, const float *grad_a_final,
                        float *grad_x, float *grad_m0, float *grad_a0,
                        int64_t T, int64_t BN, float decay, float rho,
                        float threshold, float beta, float reset, float slope,
                        int surrogate_id, int64_t chunk,
                        myelin_stream_t stream);

/*
 * Pack nonzero elements of a [rows, n] tensor into [rows, ceil(n/32)] int32
 * words, LSB first, padding bits zero.
 * Replaces: _pack_spikes_kernel + pack_spikes_triton (triton/packing.py:20-41,
 *   100-130); semantics of pack_spikes (packing.py:45-71).
 */
int myelin_pack(const void *src, int dtype, int32_t *words, int64_t rows,
                int64_t n, myelin_stream_t stream);

/*
 * Unpack words to 0/1 elements of `dtype` ([rows, n]).
 * Replaces: _unpack_spikes_kernel (triton/packing.py:44-66); semantics of
 *   unpack_spikes (packing.py:74-81).
 */
int myelin_unpack(const int32_t *words, void *dst, int dtype, int64_t rows,
                  int64_t n, myelin_stream_t stream);

/*
 * Spike counts reduced over the last (packed) dim and over every leading dim
 * whose bit is set in `reduce_mask`.  lead_shape (host memory, ndim_lead <= 8
 * entries) is the shape of the leading dims; out has the shape of the kept
 * leading dims (a scalar when all are reduced), int64.
 * Replaces: _packed_spike_row_counts_kernel + packed_spike_counts_triton
 *   (triton/packing.py:69-91,160-225); semantics of packed_spike_counts
 *   (packing.py:110-142).
 */
int myelin_packed_counts(const int32_t *words, int ndim_lead,
                         const int64_t *lead_shape, uint32_t reduce_mask,
                         int64_t n, int64_t *out, myelin_stream_t stream);

/*
 * Per-neuron counts over a block of leading rows that are NOT packed:
 * words viewed as [R, K, ceil(n/32)]; out[k, j] = sum_r bit j of row (r, k),
 * int64 [K, n].
 * Replaces: the unpack-and-sum branches of packed_spike_count
 *   (packing.py:97-107,209-216).
 */
int myelin_packed_counts_keep_last(const int32_t *words, int64_t R, int64_t K,
                                   int64_t n, int64_t *out,
                                   myelin_stream_t stream);

/*
 * rate[i] = (float)count[i] / (float)denominator, IEEE division.
 * Replaces: counts.to(dtype) / denominator in packed_spike_rate
 *   (packing.py:145-162) for float32 (dtype F32) and float64 (dtype F64).
 */
int myelin_counts_to_rate(const int64_t *counts, void *out, int dtype,
                          int64_t numel, int64_t denominator,
                          myelin_stream_t stream);

/*
 * C[M,N] = (accumulate ? C : 0) + A(m,k) B(k,n) (+ bias[n]) on MFMA tiles,
 * fp32 out; bias may be NULL.
 *   A(m,k) = trans_a ? A[k*lda + m] : A[m*lda + k]
 *   B(k,n) = trans_b ? B[n*ldb + k] : B[k*ldb + n]
 * precision MYELIN_PREC_F32 or MYELIN_PREC_BF16.  Outputs of at least
 * 128 x 128 with 16-byte-aligned operands (lda, ldb multiples of 4) run on
 * 128 x 128 tiles, others on 64 x 64 tiles; both sum each output element in
 * the same fixed k order (deterministic, no atomics).  When the output has
 * few tiles and K is long, K is split across workgroups: partial tiles go
 * to `workspace` (workspace_elems floats; 0 or NULL disables splitting;
 * myelin_gemm_workspace_elems gives the size that allows every split) and
 * are added in split order.
 * Replaces: the per-step matmuls of LinearSynapse / the stream functions
 *   (modules.py:129-133, autograd.py:477-556) and the Triton backward GEMMs
 *   _linear_surrogate_lif_backward_inputs_kernel / _weight_kernel
 *   (triton/lif.py:1136-1228).
 */
int myelin_gemm_f32(const float *A, const float *B, const float *bias, float *C,
                    int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                    int64_t ldc, int trans_a, int trans_b, int accumulate,
                    int precision, float *workspace, int64_t workspace_elems,
                    myelin_stream_t stream);

/*
 * myelin_gemm_f32 with operand types: a_dtype = b_dtype = MYELIN_DT_F32, or
 * MYELIN_DT_BF16 (bf16 values in memory, precision MYELIN_PREC_BF16 only;
 * k-contiguous operand rows 16-byte aligned, mn-contiguous ones 8-byte
 * aligned).  bf16 operands run on 128 x 128 tiles, or 256 x 128 tiles for
 * long K with both operands k-contiguous; operands both k-contiguous or
 * both mn-contiguous with 16-byte rows (and K a multiple of 64 for the
 * former) are staged by direct global -> LDS loads.  Every bf16 engine sums
 * each output element in the same k order, so without a K split the result
 * depends neither on M nor on the engine.  bf16 operands give bit-identical
 * results to fp32 operands holding the same values, at half the bytes.
 * a_dtype = MYELIN_DT_BITS with b_dtype = MYELIN_DT_F32: A is packed spike
 * bits in myelin_pack's format (lda counts int32 words: A(m,k) is bit k of
 * row m, or with trans_a bit m of row k), expanded to 0/1 on load on
 * 64 x 64 tiles -- bit-identical to the unpacked float32 A on those tiles.
 * Replaces: as myelin_gemm_f32.
 */
int myelin_gemm(const void *A, int a_dtype, const void *B, int b_dtype,
                const float *bias, float *C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, int trans_a,
                int trans_b, int accumulate, int precision, float *workspace,
                int64_t workspace_elems, myelin_stream_t stream);

/*
 * Workspace (floats) with which myelin_gemm_f32 can use its full K split
 * for an M x N x K product at `precision`; 0 when it would not split.
 * No counterpart in the reference (its Triton GEMMs accumulate with fp32
 * atomics instead of split-K partials).
 */
int64_t myelin_gemm_workspace_elems(int64_t M, int64_t N, int64_t K,
                                    int precision);

/*
 * C (+)= sum over p < parts (1..8) of op(A) op(B_p) (+ bias), B_p = B +
 * p*b_part, all bf16 operands (alignment as myelin_gemm's bf16 operands,
 * for every part) on the bf16 MFMA engines; each part's k range is summed
 * in turn into the same fp32 accumulators, from the last part to the first
 * (for the planes of myelin_split_bf16x3, smallest first: only the largest
 * plane's products round against the full-size sum).  With A exactly
 * representable in bf16 (spikes) and B_p the three planes of
 * myelin_split_bf16x3, every product is exact and the result is an fp32
 * GEMM of the unsplit B to fp32 summation accuracy, at bf16 MFMA rate.
 * Workspace as myelin_gemm_workspace_elems(M, N, K, MYELIN_PREC_BF16).
 * Replaces: as myelin_gemm_f32 (the fp32 synapse GEMMs when the layer input
 *   is spikes).
 */
int myelin_gemm_parts(const uint16_t *A, const uint16_t *B, int parts,
                      int64_t b_part, const float *bias, float *C, int64_t M,
                      int64_t N, int64_t K, int64_t lda, int64_t ldb,
                      int64_t ldc, int trans_a, int trans_b, int accumulate,
                      float *workspace, int64_t workspace_elems,
                      myelin_stream_t stream);

/*
 * myelin_gemm / myelin_gemm_parts followed by an independent column sum
 * cs_out[n] = sum_r cs_in[r, n] over [cs_rows, cs_cols] (as
 * myelin_col_sum_f32 with accumulate = 0, same bits): its workgroups join
 * the GEMM's split-K reduce launch when K is split, else it runs as a
 * launch of its own after the GEMM -- the weight and bias gradients of a
 * layer in one launch fewer.  cs_in must not be written by the GEMM nor
 * cs_out read by it.  cs_cols = 0 attaches nothing.
 * Replaces: grad_weight and grad_bias of the Functions' backward
 *   (autograd.py:553-556,712-715) and
 *   _linear_surrogate_lif_backward_weight_kernel /
 *   _linear_surrogate_lif_backward_bias_kernel (triton/lif.py:1136-1258).
 */
int myelin_gemm_col_sum(const void *A, int a_dtype, const void *B,
                        int b_dtype, const float *bias, float *C, int64_t M,
                        int64_t N, int64_t K, int64_t lda, int64_t ldb,
                        int64_t ldc, int trans_a, int trans_b, int accumulate,
                        int precision, float *workspace,
                        int64_t workspace_elems, const float *cs_in,
                        float *cs_out, int64_t cs_rows, int64_t cs_cols,
                        myelin_stream_t stream);
int myelin_gemm_parts_col_sum(const uint16_t *A, const uint16_t *B, int parts,
                              int64_t b_part, const float *bias, float *C,
                              int64_t M, int64_t N, int64_t K, int64_t lda,
                              int64_t ldb, int64_t ldc, int trans_a,
                              int trans_b, int accumulate, float *workspace,
                              int64_t workspace_elems, const float *cs_in,
                              float *cs_out, int64_t cs_rows, int64_t cs_cols,
                              myelin_stream_t stream);

/* floats of device scratch myelin_gemm_noalloc holds per GPU (64 MiB) */
#define MYELIN_NOALLOC_SCRATCH_ELEMS (16LL * 1024 * 1024)

/*
 * myelin_gemm with no workspace argument and no allocation of any kind: the
 * K split's partial tiles go to a static device array of
 * MYELIN_NOALLOC_SCRATCH_ELEMS floats that each GPU holds until the process
 * ends.  Same kernels, split and result as myelin_gemm called with a
 * workspace of myelin_gemm_workspace_elems(M, N, K, precision) floats.
 * Returns MYELIN_EINVAL when that workspace size exceeds the array.  The
 * first call on a device looks up the array's device address there (a
 * host-side query).  All calls on one GPU share its array: calls that
 * overlap in time on one GPU (two streams or two host threads at once)
 * race on it.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.
 */
int myelin_gemm_noalloc(const void *A, int a_dtype, const void *B, int b_dtype,
                        const float *bias, float *C, int64_t M, int64_t N,
                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                        int trans_a, int trans_b, int accumulate,
                        int precision, myelin_stream_t stream);


/*
 * Streamed synapse fused ahead of the LIF update, over steps
 * [t_begin, t_end) of x [T, B, F] with W [F, N] (+ bias [N]):
 *   I_t = x_t @ W + bias ; m' = m*decay + I_t ; s = rule(m') ; m = s ? reset : m'
 * m0 NULL means a zero initial membrane (the reference's linear paths start
 * at 0, autograd.py:470-474).  Optional outputs (NULL to skip):
 *   spikes [T,B,N] fp32 and packed [T,B,ceil(N/32)] at absolute t;
 *   pre [t_end-t_begin,B,N] pre-reset membranes at relative t;
 *   rates [B,N] = spike count / T;  ckpt rows every ckpt_every steps from
 *   t_begin (row 0 = m0);  m_final [B,N].
 * Replaces: _linear_surrogate_lif_forward_kernel, the checkpoint / packed /
 *   rate forward kernels and their launchers (triton/lif.py:554-1133), and
 *   the recompute-chunk kernel (triton/lif.py:1746-1810).
 */
int myelin_linear_lif_fwd(const float *x, const float *w, const float *bias,
                          const float *m0, float *m_final, float *spikes,
                          float *pre, int32_t *packed, float *rates,
                          float *ckpt, int64_t T, int64_t B, int64_t F,
                          int64_t N, int64_t t_begin, int64_t t_end,
                          int64_t ckpt_every, float decay, float threshold,
                          float reset, float slope, int rule, int precision,
                          myelin_stream_t stream);

/*
 * myelin_linear_lif_fwd for the bf16 synapse from bf16 operands in memory:
 * x [T, B, F] and the transposed weight wt [N, F] (both bf16, 16-byte
 * aligned rows, F % 8 == 0), on 128 x 128 tiles.  Bit-identical to
 * myelin_linear_lif_fwd(precision = MYELIN_PREC_BF16) on the same values.
 * Replaces: as myelin_linear_lif_fwd.
 */
int myelin_linear_lif_fwd_bf16(const uint16_t *x, const uint16_t *wt,
                               const float *bias, const float *m0,
                               float *m_final, float *spikes, float *pre,
                               int32_t *packed, float *rates, float *ckpt,
                               int64_t T, int64_t B, int64_t F, int64_t N,
                               int64_t t_begin, int64_t t_end,
                               int64_t ckpt_every, float decay,
                               float threshold, float reset, float slope,
                               int rule, myelin_stream_t stream);

/*
 * bf16 operand copies (round to nearest even, as the bf16 GEMMs round fp32
 * operands): dst[i] = bf16(src[i]) (both 16-byte aligned), and the
 * transposed copy dst[c*rows + r] = bf16(src[r*cols + c]).  No counterpart
 * in the reference (its tl.dot consumes fp32 operands).
 */
int myelin_cast_bf16(const float *src, uint16_t *dst, int64_t n,
                     myelin_stream_t stream);
int myelin_transpose_bf16(const float *src, uint16_t *dst, int64_t rows,
                          int64_t cols, myelin_stream_t stream);

/*
 * myelin_cast_bf16(x, xb, n) and myelin_transpose_bf16(w, wt, rows, cols)
 * in one launch (same bits): the bf16 synapse's two operand copies.  No
 * counterpart in the reference.
 */
int myelin_cast_transpose_bf16(const float *x, uint16_t *xb, int64_t n,
                               const float *w, uint16_t *wt, int64_t rows,
                               int64_t cols, myelin_stream_t stream);

/*
 * myelin_cast_bf16 that also sets *inexact = 1 (never clears it) when some
 * element is not a bf16 value the MFMA multiplies exactly (its rounding
 * changes it, or it is a nonzero denormal).  No counterpart in the
 * reference.
 */
int myelin_cast_bf16_checked(const float *src, uint16_t *dst, int64_t n,
                             int *inexact, myelin_stream_t stream);

/*
 * Splits src [rows, cols] fp32 into three bf16 planes hi, mid, lo with
 * float(hi) + float(mid) + float(lo) == src exactly (hi = bf16(v), mid =
 * bf16(v - hi), lo = v - hi - mid; exact for |v| >= 2^-110, non-finite v
 * in hi alone).  Plane p starts at dst + p*rows*cols and is [rows, cols],
 * or with `transpose` [cols, rows].  No counterpart in the reference.
 */
int myelin_split_bf16x3(const float *src, uint16_t *dst, int64_t rows,
                        int64_t cols, int transpose, myelin_stream_t stream);

/*
 * Reverse recurrence over C steps of a saved pre-reset trace [C, BN]:
 *   d = slope*sigma'(slope*(pre - thr)); gp = gm*((1-s) + (reset-pre)*d)
 *   + g_spike*d; G[j] = gp; gm = gp*decay   (grad_m is in/out)
 * g_spike = grad_spikes[j] (may be NULL) plus grad_rates/T_total (may be
 * NULL).  gbias_acc [BN] (may be NULL) accumulates sum_j gp.  grad_m NULL
 * makes the launch a whole reverse pass: gm starts at zero and is not
 * returned, and gbias_acc receives sum_j gp (written, not accumulated),
 * so the caller needs no zero-filled buffers.  G is written
 * as g_dtype MYELIN_DT_F32, or MYELIN_DT_BF16 (round to nearest even, the
 * rounding the bf16 GEMMs apply) when only bf16 GEMMs read it, or
 * MYELIN_DT_BF16X3: three bf16 planes [3, C, BN] as myelin_split_bf16x3
 * writes them, for myelin_gemm_parts.
 * Replaces: the reverse loops of the torch stream / checkpoint / rate
 *   Functions (autograd.py:540-556,694-715,857-883) and
 *   _linear_surrogate_lif_checkpoint_backward_chunk_packed_spikes_kernel
 *   (triton/lif.py:1934-2067).
 */
int myelin_linear_pre_bwd(const float *pre, const float *grad_spikes,
                          const float *grad_rates, float *grad_m, void *G,
                          int g_dtype, float *gbias_acc, int64_t C, int64_t BN,
                          int64_t T_total, float decay, float threshold,
                          float reset, float slope, int surrogate_id, int rule,
                          myelin_stream_t stream);

/*
 * myelin_linear_pre_bwd for the hidden layer [C, B, N] of a two-layer
 * network, with its spike gradient formed in the kernel from the readout's
 * G_o = grad_out [C, B, O] and weight w_out [N, O] (row-major, as the
 * readout's weight [in, out]): g_spike[j, b, n] = sum_o grad_out[j, b, o]
 * * w_out[n, o], the product myelin_gemm_f32(grad_out, w_out^T) computes
 * (fused multiply-adds in o order from zero), so G equals that GEMM's dS
 * fed to myelin_linear_pre_bwd, without dS in memory.  No rate gradient.
 * Needs 1 <= O <= 32, N a multiple of 256, C x O within the kernel's
 * 64 KB of staged grad_out rows (C <= 512 at O = 32, <= 819 at O = 20)
 * and g_dtype MYELIN_DT_F32 or MYELIN_DT_BF16X3; else MYELIN_EINVAL.
 * Replaces: the readout's grad_inputs[t] = grad_pre_reset @ weight.t()
 *   (autograd.py:877-878) feeding the hidden layer's reverse loop
 *   (autograd.py:694-715).
 */
int myelin_linear_pre_bwd_readout(const float *pre, const float *grad_out,
                                  const float *w_out, int O, float *grad_m,
                                  void *G, int g_dtype, float *gbias_acc,
                                  int64_t C, int64_t B, int64_t N, float decay,
                                  float threshold, float reset, float slope,
                                  int surrogate_id, int rule,
                                  myelin_stream_t stream);

/*
 * out[n] = (accumulate ? out[n] : 0) + sum_r in[r, n], fixed order per
 * column.  Replaces: _linear_surrogate_lif_backward_bias_kernel
 *   (triton/lif.py:1231-1258) without its atomics.
 */
int myelin_col_sum_f32(const float *in, float *out, int64_t rows, int64_t cols,
                       int accumulate, myelin_stream_t stream);

/*
 * The LIF recurrence of myelin_linear_lif_fwd over precomputed currents
 * [t_end - t_begin, B, N] (x_t @ W + bias from myelin_gemm_f32), for steps
 * [t_begin, t_end).  Long horizons run as several calls with the membrane
 * (m0 -> m_final, may alias) and spike counts (`counts`, [B, N] in/out,
 * may be NULL) carried across calls.  pre rows are t - pre_origin;
 * checkpoint rows count from ck_origin (row k = state before step
 * ck_origin + k*ckpt_every); spikes / packed use absolute t; rates =
 * counts / T at the end of the call.  Used when the fused kernel would leave
 * the chip under-filled: narrow layers (10/20-neuron readouts) and few
 * batch x neuron tiles with long horizons.
 * Replaces: the recurrence half of _linear_surrogate_lif_checkpoint_rate_
 *   forward_kernel / _linear_surrogate_lif_forward_kernel
 *   (triton/lif.py:554-612,823-889).
 */
int myelin_lif_currents_fwd(const float *currents, const float *m0,
                            float *m_final, float *spikes, float *pre,
                            int32_t *packed, float *rates, float *counts,
                            float *ckpt, int64_t T, int64_t B, int64_t N,
                            int64_t t_begin, int64_t t_end, int64_t pre_origin,
                            int64_t ck_origin, int64_t ckpt_every, float decay,
                            float threshold, float reset, float slope, int rule,
                            myelin_stream_t stream);

/*
 * A narrow layer (N <= 32 neurons) over a packed-spike input, the synapse
 * currents and the LIF recurrence in one launch: words [T, B, ceil(F/32)]
 * (bit k % 32 of word k / 32 is input k; bits past F are ignored), w [F, N]
 * fp32, bias [N] or NULL, for steps [t_begin, t_end).  precision 1 rounds w
 * to bf16; precision 0 takes fp32 w exactly (the three-plane bf16 split,
 * exact products, fp32 sums).  Outputs as myelin_lif_currents_fwd: pre
 * rows are t - t_begin, spikes use absolute t, rates = count / T (only
 * with the whole range [0, T)); any output may be NULL.  One workgroup per
 * batch row: for batches that fill the chip (the 10-neuron readout at
 * B = 256) it replaces the currents GEMM, its split-K reduce and the
 * recurrence launch, with the same sums bit for bit.  W^T and a chunk of
 * bit rows are staged in LDS: myelin_narrow_bits_fits (host only) returns
 * 1 when an (F, N, precision) layer fits, and the entry rejects one that
 * does not.
 * Replaces: the rate readout's forward in _linear_surrogate_lif_checkpoint_
 *   rate_forward_kernel (triton/lif.py:823-889) for a spiking input.
 */
int myelin_narrow_bits_fits(int64_t F, int64_t N, int precision);
int myelin_linear_lif_fwd_narrow_bits(const int32_t *words, const float *w,
                                      const float *bias, const float *m0,
                                      float *m_final, float *spikes, float *pre,
                                      float *rates, int64_t T, int64_t B,
                                      int64_t F, int64_t N, int64_t t_begin,
                                      int64_t t_end, float decay,
                                      float threshold, float reset, float slope,
                                      int rule, int precision,
                                      myelin_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MYELIN_HIP_H */
