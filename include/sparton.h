/*
 * sparton.h -- C ABI of libsparton_hip.so, the MI355X (gfx950) implementation of
 * the SpartonHead forward and backward.
 *
 * Math (every entry point below computes exactly this):
 *   x[b,s,v]   = (sum_d H[b,s,d] * W[v,d] + bias[v]) * mask[b,s]
 *   M[b,v]     = max(0, max_s x[b,s,v])
 *   I[b,v]     = lowest s with x[b,s,v] == M[b,v] if M[b,v] > 0, else 0
 *   reps[b,v]  = log1p(M[b,v])
 *   g'[b,v]    = G[b,v] * exp(-reps[b,v]) * mask[b, I[b,v]]  if reps[b,v] > 0, else 0
 *   dbias[v]   = sum_b g'[b,v]
 *   dW[v,:]    = sum_b g'[b,v] * H[b, I[b,v], :]
 *   dH[b,s,:]  = sum_{v : I[b,v] == s} g'[b,v] * W[v,:]
 *
 * Conventions:
 *   - Every pointer is a device pointer owned by the caller; no entry point allocates,
 *     frees or synchronises. Work is enqueued on `stream` (a hipStream_t, passed as
 *     void* so this header does not need the HIP headers; NULL = the null stream).
 *   - Tensors are dense row-major with unit inner stride and 16-byte aligned bases:
 *     H [B,S,D], W [V,D], bias [V], mask [B,S], reps/grad [B,V], argmax [B,V] int32,
 *     d_hidden [B,S,D], d_weight [V,D], d_bias [V] (fp32 or `dtype`, see sparton_bwd).
 *   - `dtype` (enum sparton_dtype) is the element type of H, W, bias, reps and grad.
 *   - D must be a multiple of 8 (16-bit dtypes) or 4 (fp32).
 *   - Return value: 0 on success, < 0 for an invalid argument (nothing is launched),
 *     > 0 is the hipError_t of a failed launch. sparton_strerror() names each code.
 *   - Calls are reentrant. The only mutable global state is the per-device address of
 *     the static scratch of sparton_fwd_noalloc, resolved once per device under a lock.
 */
#ifndef SPARTON_H
#define SPARTON_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum sparton_dtype {
  SPARTON_F32 = 0,
  SPARTON_BF16 = 1,
  SPARTON_F16 = 2,
};

/*
 * Flag OR'ed into the forward's `dtype` with SPARTON_F32 only (sparton_fwd,
 * sparton_fwd_noalloc, sparton_fwd_profile; any other use is SPARTON_EINVAL): torch's
 * 'high' float32 matmul precision, which the reference sets when it is imported
 * (src/sparton/sparton_kernel.py:14, torch.set_float32_matmul_precision('high')). Each
 * fp32 operand is taken as the sum of two bf16 values (hi = bf16(x), lo = bf16(x - hi)) and
 * each product as hi*hi + hi*lo + lo*hi on bf16 MFMAs with fp32 accumulation, within
 * 3 * 2^-16 relative of the exact product. It applies to the small-batch kernel
 * (B*S <= 128); larger batches are computed in fp32 exactly either way.
 */
#define SPARTON_F32_SPLIT 0x100

/* Element type of the attention mask. Any nonzero value takes part in the
 * multiply; a tokenizer mask is int64 0/1. */
enum sparton_mask_dtype {
  SPARTON_MASK_I64 = 0,
  SPARTON_MASK_I32 = 1,
  SPARTON_MASK_U8 = 2, /* torch.bool / uint8 */
  SPARTON_MASK_F32 = 3,
  SPARTON_MASK_BF16 = 4,
  SPARTON_MASK_F16 = 5,
};

enum sparton_status {
  SPARTON_OK = 0,
  SPARTON_EINVAL = -1,       /* null pointer, bad shape or bad enum value */
  SPARTON_EALIGN = -2,       /* a base pointer is not 16-byte aligned */
  SPARTON_EUNSUPPORTED = -3, /* shape outside the supported range (see sparton_limits) */
  SPARTON_EWORKSPACE = -4,   /* workspace missing or smaller than sparton_{fwd,bwd}_workspace_bytes */
  SPARTON_ESCRATCH = -5,     /* sparton_fwd_noalloc: sizes need more than its static scratch */
};

/*
 * Bytes of device scratch sparton_fwd needs for these sizes (256-byte aligned
 * sections: the per-row block plan and the partial results of batch rows whose
 * positions span several row tiles). No counterpart in the reference: its forward
 * materializes a [B,S,C] logits tile per vocab tile instead (sparton_kernel.py:245-247).
 */
size_t sparton_fwd_workspace_bytes(int64_t B, int64_t S, int64_t D, int64_t V, int dtype);

/*
 * Forward: reps[B,V] (in `dtype`) and argmax I[B,V] (int32).
 * `argmax` may be NULL: the inference-only variant then skips the index store.
 * `reps_f32` may be NULL; if given, it receives reps[B,V] unrounded in fp32, which a
 * training caller keeps for the backward instead of the rounded `reps`.
 * `bias` may be NULL (use_bias=False). `workspace` (256-byte aligned, at least
 * sparton_fwd_workspace_bytes) is overwritten; S <= 16384.
 *
 * Replaces the reference's forward path: fused_sparton_fwd_with_indices
 * (src/sparton/sparton_kernel.py:226-253), its V-tile GEMM (:204-210) and the
 * reduce kernel reduce_seq_max_log1p_relu_kernel_with_indices (:85-168); called where
 * the custom op sparton::fused_sparton_fwd calls it (:651). With argmax == NULL it
 * replaces the no-index variant fused_sparton_fwd (:372-394, kernel :262-334).
 * The [B,S,V] logits are never written to memory.
 */
int sparton_fwd(const void* hidden, const void* weight, const void* bias,
                const void* mask, int mask_dtype, void* reps, int32_t* argmax,
                float* reps_f32, int64_t B, int64_t S, int64_t D, int64_t V,
                int dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * sparton_fwd without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The same kernels and results as sparton_fwd; the workspace
 * is a static device array of sparton_fwd_noalloc_max_workspace() bytes (32 MiB), one per
 * GPU, held until the process ends. Sizes whose sparton_fwd_workspace_bytes() exceeds it
 * return SPARTON_ESCRATCH and launch nothing (at V = 30522 that allows about 68 row tiles of
 * 256 packed positions, e.g. B = 64, S = 256). Calls that overlap on one GPU share that
 * array and race: the caller serialises them. Allocates, frees and synchronises nothing.
 */
int sparton_fwd_noalloc(const void* hidden, const void* weight, const void* bias,
                        const void* mask, int mask_dtype, void* reps, int32_t* argmax,
                        float* reps_f32, int64_t B, int64_t S, int64_t D, int64_t V,
                        int dtype, void* stream);

/* Size in bytes of sparton_fwd_noalloc's static scratch. */
size_t sparton_fwd_noalloc_max_workspace(void);

/*
 * Profiling variant of sparton_fwd: the same work and results; *main_ms receives the
 * device time of the main (MFMA) kernel alone, from HIP events recorded on `stream`
 * just before and after its launch (summed over the row chunks of very large batches).
 * Blocks the host until that kernel has finished. No counterpart in the reference: it
 * serves measurement (the kernel's roofline), not the operator path.
 */
int sparton_fwd_profile(const void* hidden, const void* weight, const void* bias,
                        const void* mask, int mask_dtype, void* reps, int32_t* argmax,
                        float* reps_f32, int64_t B, int64_t S, int64_t D, int64_t V,
                        int dtype, void* workspace, size_t workspace_bytes, void* stream,
                        float* main_ms);

/*
 * Bytes of device scratch sparton_bwd needs for these sizes (256-byte aligned
 * sections: per-chunk histograms, segment offsets and the bucketed entry list).
 * No counterpart in the reference: its backward needs no scratch because it
 * accumulates with atomics into zero-filled outputs (sparton_kernel.py:676-678).
 */
size_t sparton_bwd_workspace_bytes(int64_t B, int64_t S, int64_t D, int64_t V);

/*
 * Backward: d_hidden, d_weight, d_bias from grad_reps [B,V] (`dtype`).
 * `reps` is the forward's reps in `reps_dtype` (enum sparton_dtype): the rounded
 * `dtype` output, as the reference saves it, or the fp32 `reps_f32` output (any other
 * `reps_dtype` is SPARTON_EINVAL).
 * `grad_dtype` is SPARTON_F32 (the reference's fp32 gradients) or `dtype` (the
 * gradients rounded once to the parameters' dtype, as autograd would cast them).
 * Every element of each non-NULL output is written (no zero-fill needed); a NULL
 * output is skipped. `mask` is read to apply mask[b, I[b,v]] (1 for a 0/1 mask).
 * Deterministic: no atomics on floating-point data; every output row is summed in
 * a fixed order (dW and dbias over b ascending, dH over v ascending).
 *
 * Replaces fused_sparton_bwd_with_bias (src/sparton/sparton_kernel.py:567-597), the
 * kernel fused_sparton_bwd_kernel_with_bias (:473-565) and the zeros_like of the
 * outputs (:676-678); called where the custom op sparton::fused_sparton_bwd calls it
 * (:680). Unlike the reference it also runs when bias is absent (d_bias == NULL).
 */
int sparton_bwd(const void* grad_reps, const void* reps, int reps_dtype,
                const int32_t* argmax, const void* mask, int mask_dtype, const void* hidden,
                const void* weight, void* d_hidden, void* d_weight, void* d_bias,
                int grad_dtype, void* workspace, size_t workspace_bytes, int64_t B,
                int64_t S, int64_t D, int64_t V, int dtype, void* stream);

/*
 * The MLM transform before the head (its output is the head's hidden input):
 *     y = LayerNorm(gelu(x W^T + dense_bias)) * ln_weight + ln_bias, per row of D,
 * gelu in the exact erf form -- BERT's cls.predictions.transform and RoBERTa's
 * lm_head dense/gelu/layer_norm, which the reference calls before the head
 * (training/model.py:14-40, :56-58). The two D x D GEMMs are plain library GEMMs that
 * the caller runs; these entry points are the fused work around them, on M rows
 * of D elements (D % 4 == 0, D <= 3072). `dtype` (enum sparton_dtype) is the type of
 * z, y, dy and dz; dense_bias, ln_weight, ln_bias, mean and rstd are fp32.
 */

/* Bytes of device scratch sparton_transform_bwd needs (column partial sums). */
size_t sparton_transform_workspace_bytes(int64_t M, int64_t D);

/*
 * Forward epilogue: z = x W^T [M,D] (from the GEMM) -> y [M,D], and each row's mean and
 * 1/sqrt(var + eps) of gelu(z + dense_bias) for the backward.
 */
int sparton_transform_fwd(const void* z, const float* dense_bias, const float* ln_weight,
                          const float* ln_bias, float eps, void* y, float* mean, float* rstd,
                          int64_t M, int64_t D, int dtype, void* stream);

/*
 * Backward epilogue: dy [M,D] -> dz [M,D], the gradient at z (the caller's GEMMs then give
 * dx = dz W and dW = dz^T x), and the fp32 column sums d_ln_weight = sum dy * xhat,
 * d_ln_bias = sum dy, d_dense_bias = sum dz (each may be NULL). Deterministic: every sum
 * runs in a fixed order.
 */
int sparton_transform_bwd(const void* dy, const void* z, const float* dense_bias,
                          const float* ln_weight, const float* mean, const float* rstd, void* dz,
                          float* d_ln_weight, float* d_ln_bias, float* d_dense_bias,
                          void* workspace, size_t workspace_bytes, int64_t M, int64_t D,
                          int dtype, void* stream);

/*
 * Weight gradient of the transform's dense layer, dW = dz^T x, as a batched GEMM over C row
 * chunks (the caller runs the GEMM): sparton_transform_dz_chunks writes dzt [C, D, M/C] with
 * dzt[c][i][l] = dz[c (M/C) + l][i] (bf16/fp16; M % C == 0, (M/C) % 64 == 0, D % 64 == 0,
 * 16-byte aligned), the K-contiguous left operands of part[c] = dzt[c] x[c (M/C) : (c+1) (M/C), :] (fp32 [C, D, D]); then
 * sparton_transform_chunk_sum writes out[k] = sum_c part[c][k] in chunk order, in dtype
 * (n % 4 == 0, 16-byte aligned). The reference gets dW from autograd of nn.Linear
 * (training/model.py:14-40); these two calls and one batched GEMM replace that one GEMM.
 */
int sparton_transform_dz_chunks(const void* dz, void* dzt, int64_t M, int64_t D, int64_t C,
                                int dtype, void* stream);
int sparton_transform_chunk_sum(const float* part, void* out, int64_t C, int64_t n, int dtype,
                                void* stream);

/*
 * The SPLADE training loss on the head's reps (reference training/train.py:73-88, combined in
 * compute_loss at :164-197). q [Bq,V] are query reps, d [Bd,V] document reps (row-major, the
 * reps dtype; d may be NULL with Bd = 0). With S = q d^T / temperature:
 *   CE = mean_i (logsumexp_j S[i,j] - S[i,i])   info_nce_loss, labels arange(Bq) (:73-77)
 *   L1(x) = mean_b sum_v |x[b,v]|               l1_regularization (:80-82)
 *   FL(x) = mean_v (sum_b x[b,v])^2             flops_regularization (:85-87)
 *   total = w_ce CE + w_l1 (L1(q) + L1(d)) + w_flops (FL(q) + FL(d))   (:196-197)
 * Limits: Bq >= 1, Bd >= 0, Bq <= Bd when Bd > 0 (the labels index d's rows), temperature
 * > 0 and finite when Bd > 0; sizes whose scores or offsets pass the kernels' int range return
 * SPARTON_EUNSUPPORTED. Up to 64 rows per side run slice-staged kernels, larger batches
 * tiled GEMM kernels on the matrix cores (16-bit reps on the 16-bit MFMA, whose products are
 * exact in fp32; fp32 reps on the fp32 MFMA); the workspace size follows. Accumulated in fp32
 * whatever the reps dtype.
 */
size_t sparton_loss_workspace_bytes(int64_t Bq, int64_t Bd, int64_t V);

/*
 * out[6] (device fp32) = (total, CE, L1(q), L1(d), FL(q), FL(d)); probs [Bq,Bd] (device
 * fp32, unused when Bd = 0) = (softmax(S) - I) / (Bq temperature), kept for the backward.
 */
int sparton_loss_fwd(const void* q, const void* d, int64_t Bq, int64_t Bd, int64_t V,
                     float temperature, float w_ce, float w_l1, float w_flops, float* out,
                     float* probs, void* workspace, size_t workspace_bytes, int dtype,
                     void* stream);

/*
 * grad_q [Bq,V] and grad_d [Bd,V] (reps dtype) from grad_out[6] (device fp32), the upstream
 * gradients of the six outputs of sparton_loss_fwd, and its probs. Deterministic.
 */
int sparton_loss_bwd(const void* q, const void* d, const float* probs, const float* grad_out,
                     int64_t Bq, int64_t Bd, int64_t V, float w_ce, float w_l1, float w_flops,
                     void* grad_q, void* grad_d, int dtype, void* stream);

/*
 * The same backward with the six upstream gradients given separately: grad_terms is a host
 * array of six device pointers to fp32 scalars, in sparton_loss_fwd's output order, each
 * possibly NULL for a zero gradient. It serves callers that hand the six terms out as
 * separate tensors (a training loop that backpropagates `total` alone passes one pointer)
 * and so never have to assemble a six-element gradient. No counterpart in the reference,
 * whose loss is plain torch (training/train.py:178-197).
 */
int sparton_loss_bwd_terms(const void* q, const void* d, const float* probs,
                           const float* const* grad_terms, int64_t Bq, int64_t Bd, int64_t V,
                           float w_ce, float w_l1, float w_flops, void* grad_q, void* grad_d,
                           int dtype, void* stream);

/*
 * Measurement probe, no counterpart in the reference: `grid` workgroups (one per CU) of 4
 * waves each run `iters` rounds of 16 independent v_mfma_f32_32x32x16_{bf16,f16} on random
 * register operands (dtype SPARTON_BF16 or SPARTON_F16). clk[2*w] receives workgroup w's
 * shader-clock cycles and clk[2*w+1] its 100 MHz real-time ticks over the loop; out[256*w+t]
 * a sink value. It measures the MFMA rate all CUs sustain together on data-like operands
 * (the GPU is power-limited under such a load), the ceiling the forward's main kernel runs
 * against. `out` and `clk` are device pointers.
 */
int sparton_mfma_probe(int dtype, int grid, int iters, float* out, long long* clk, void* stream);

/* Static, thread-safe description of a status code. */
const char* sparton_strerror(int code);

/* Supported ranges: writes max S and max B of the backward (each 2^31 - 1 since ABI 8;
 * B * S and B * V must also stay below 2^31). */
void sparton_limits(int64_t* max_bwd_seq, int64_t* max_bwd_batch);

/* ABI version of this header (bumped on any signature change or new argument value;
 * 10: SPARTON_F32_SPLIT). */
int sparton_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SPARTON_H */
