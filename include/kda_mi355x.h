/*
 * kda_mi355x.h — C ABI of the MI355X (gfx950) Kimi Delta Attention operator library
 * (libkda_mi355x.so).
 *
 * Every entry point takes raw device pointers plus explicit sizes, launches on the
 * given HIP stream, never synchronises, never allocates, and returns KDA_OK (0) or a
 * nonzero status; kda_last_error() then describes the failure (thread-local).  All
 * tensors are dense and contiguous in the layouts written next to each argument.
 * "bf16" is IEEE bfloat16 stored as 16-bit words; "f32" is float.
 *
 * Layout conventions (the reference's own, nanochat/mixers/kda.py:23-35,246-266):
 *   q, k, gate   [B, T, H, K]      v, output [B, T, H, V]      beta_logits [B, T, H]
 *   state        [N, H, V, K] f32 ("V-first"; N = B, or the number of packed sequences)
 *   A_log [H] f32, dt_bias [H*K] f32
 * With cu_seqlens (device int32, num_seqs+1 entries, B must be 1) the T axis holds
 * num_seqs packed sequences and the recurrent state resets at each boundary.
 */
#ifndef KDA_MI355X_H
#define KDA_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_OK 0
#define KDA_ERR_INVALID 1   /* bad shape, size, pointer or flag */
#define KDA_ERR_LAUNCH 2    /* a HIP launch or runtime call failed */
#define KDA_ERR_TIMEOUT 3   /* a bounded in-kernel wait gave up (kda_chunk_backward_status) */

/* Gate parameterisations. */
#define KDA_GATE_K3 0        /* g = lb*sigmoid(exp(A_log[h])*(raw+dt_bias[h,k])); gate is bf16 raw logits */
#define KDA_GATE_LOGDECAY 1  /* gate is the activated f32 log decay g (<= 0) */

/* Shape / option descriptor shared by the chunked forward and backward. */
typedef struct kda_chunk_problem {
  int32_t batch;       /* B */
  int32_t seq_len;     /* T (total packed length when cu_seqlens != NULL) */
  int32_t heads;       /* H */
  int32_t key_dim;     /* K in [1, 256]: 64 and 128 run the chunked kernels, other sizes the
                          token-serial ones (as the reference's generic lane, chunk.cu:135-213) */
  int32_t value_dim;   /* V in [1, 4096] (chunked kernels when K and V are 64 or 128) */
  int32_t num_seqs;    /* B without cu_seqlens; number of packed sequences with it */
  const int32_t* cu_seqlens; /* device pointer or NULL */
  int32_t gate_mode;   /* KDA_GATE_K3 or KDA_GATE_LOGDECAY */
  float lower_bound;   /* K3 lower bound lb (< 0) */
  float scale;         /* query scale (resolved by the caller, normally K^-0.5) */
  int32_t grad_row_stride; /* backward only: elements between consecutive tokens' rows of
                              dq, dk and dv (a multiple of 8, at least H * max(K, V)); 0 for
                              dense [.., H, K] / [.., H, V] gradients.  Lets the three land
                              interleaved in one [B, T, 3 H K] buffer.  (No reference
                              counterpart: the reference returns three tensors.) */
  int32_t beta_row_stride; /* elements between consecutive tokens' rows of beta_logits
                              (forward) and of dbeta_logits (backward); 0 for dense [.., H].
                              Lets both be column slices of a wider per-token row. */
  int32_t beta_grad_pad;   /* backward only: number of elements after each token's H
                              dbeta_logits values that the backward sets to zero (padding
                              columns of such a row); 0 normally */
  int32_t norm_gate_row_stride; /* norm-gate forwards only: elements between consecutive
                              tokens' rows of norm_gate; 0 for dense [.., H, V].  (These
                              three have no reference counterpart: they let the training
                              mixer pass slices of its packed projection output.) */
} kda_chunk_problem;

/* Last error message of the calling thread ("" when none). */
const char* kda_last_error(void);

/* Library version string. */
const char* kda_version(void);

/*
 * Bytes of the residual workspace the chunked forward fills and the chunked backward
 * reads back (chunk table, per-chunk WY factors, state and delta histories).
 * Replaces the output-storage "sidecar" of nanochat/mixers/cuda_kda/chunk_wy_forward.cu:1613-1652.
 */
size_t kda_chunk_workspace_bytes(const kda_chunk_problem* p);

/* Bytes of scratch the chunked backward needs in addition to the workspace. */
size_t kda_chunk_backward_scratch_bytes(const kda_chunk_problem* p);

/*
 * Chunked (C = 64) WY forward.  Replaces torch.ops.nanochat_kda.chunk_forward
 * (nanochat/mixers/cuda_kda/chunk.cu:1665-1756, schema chunk.cu:2118-2121).
 *   gate: bf16 raw gate logits (K3) or f32 log decay (LOGDECAY), [B,T,H,K]
 *   A_log, dt_bias: used for K3 only (may be NULL for LOGDECAY)
 *   initial_state: f32 [N,H,V,K] or NULL (zeros); never written
 *   output: bf16 [B,T,H,V];  final_state: f32 [N,H,V,K] or NULL
 *   workspace: kda_chunk_workspace_bytes(p) bytes, 256-byte aligned
 * Deterministic: identical inputs give bitwise identical outputs.
 */
int kda_chunk_forward(const kda_chunk_problem* p,
                      const void* q, const void* k, const void* v, const void* gate,
                      const void* beta_logits, const float* A_log, const float* dt_bias,
                      const float* initial_state, void* output, float* final_state,
                      void* workspace, hipStream_t stream);

/*
 * kda_chunk_forward with the mixer's output RMSNorm * weight * sigmoid(gate) fused into the
 * output kernel's epilogue (a producer/consumer fusion: the norm takes o from registers instead
 * of a second kernel reading it back from HBM).  No single counterpart in
 * the reference: it replaces the pair chunk_forward (chunk.cu:1380-1757) followed by
 * torch.ops.nanochat_kda.rmsnorm_gate_forward (rmsnorm_gate.cu:31-71) on its output, as
 * composed in kda.py:761-770.  All arguments of kda_chunk_forward keep their meaning (output
 * still receives o, which the norm backward reads), plus
 *   norm_gate bf16 [B,T,H,V], norm_weight f32 [V], epsilon >= 0,
 *   norm_output bf16 [B,T,H,V] = rms_norm(bf16(o), weight, eps) * sigmoid(norm_gate),
 *   inverse_rms f32 [B*T*H] (what kda_rmsnorm_gate_backward takes).
 * key_dim and value_dim must be 64 or 128 (other sizes: kda_chunk_forward, then
 * kda_rmsnorm_gate_forward).
 */
int kda_chunk_forward_norm_gate(const kda_chunk_problem* p,
                                const void* q, const void* k, const void* v, const void* gate,
                                const void* beta_logits, const float* A_log, const float* dt_bias,
                                const float* initial_state, void* output, float* final_state,
                                void* workspace, const void* norm_gate, const float* norm_weight,
                                float epsilon, void* norm_output, float* inverse_rms,
                                hipStream_t stream);

/*
 * kda_chunk_forward_norm_gate with the mixer's short convolution + SiLU of q, k and v
 * computed by the chunk forward's first kernel.  Replaces the reference's sequence
 * causal_convolution_forward (x3) -> chunk_forward -> rmsnorm_gate_forward
 * (nanochat/mixers/kda.py:744-770; causal_convolution_forward.cu:42-238) on the stateless
 * training path: no convolution or recurrent state in or out, no cu_seqlens.
 *   conv_x      bf16 rows of conv_ld elements, one per token ([B*T][conv_ld]); columns
 *               [0, HK), [HK, 2HK), [2HK, 3HK) hold the pre-convolution q, k, v projections
 *               (HK = heads * key_dim); conv_ld % 8 == 0, 16-byte aligned
 *   conv_weight bf16 [3 HK][conv_width], conv_width in [1, 4], the same channel order
 *   q, k, v     outputs: bf16 [B,T,H,K] post-SiLU activations (what kda_chunk_backward and
 *               kda_causal_conv_backward take); bit-identical to kda_causal_conv_forward's
 * key_dim == value_dim, 64 or 128.  The other arguments as in kda_chunk_forward_norm_gate.
 */
int kda_chunk_forward_conv_norm_gate(const kda_chunk_problem* p, const void* conv_x,
                                     int64_t conv_ld, const void* conv_weight, int32_t conv_width,
                                     void* q, void* k, void* v, const void* gate,
                                     const void* beta_logits, const float* A_log,
                                     const float* dt_bias, void* output, void* workspace,
                                     const void* norm_gate, const float* norm_weight,
                                     float epsilon, void* norm_output, float* inverse_rms,
                                     hipStream_t stream);

/*
 * Exact chunked backward.  Replaces torch.ops.nanochat_kda.chunk_backward
 * (nanochat/mixers/cuda_kda/chunk.cu:1758-2113, schema chunk.cu:2122-2129).
 *   workspace: as filled by kda_chunk_forward on the same inputs
 *   grad_output bf16 [B,T,H,V]; grad_final_state f32 [N,H,V,K] or NULL
 *   dq, dk: bf16 [B,T,H,K]; dv: bf16 [B,T,H,V]
 *   dgate: bf16 [B,T,H,K] (K3: d raw_gate) or f32 (LOGDECAY: dL/dg)
 *   dbeta_logits: bf16 [B,T,H]
 *   dA_log f32 [H], ddt_bias f32 [H*K]: K3 only (may be NULL for LOGDECAY)
 *   dinitial_state f32 [N,H,V,K] or NULL
 *   scratch: kda_chunk_backward_scratch_bytes(p) bytes, 256-byte aligned
 * Parameter gradients are reduced in a fixed order (no atomics).
 */
int kda_chunk_backward(const kda_chunk_problem* p,
                       const void* q, const void* k, const void* v, const void* gate,
                       const void* beta_logits, const float* A_log, const float* dt_bias,
                       const float* initial_state, const void* workspace,
                       const void* grad_output, const float* grad_final_state,
                       void* dq, void* dk, void* dv, void* dgate, void* dbeta_logits,
                       float* dA_log, float* ddt_bias, float* dinitial_state,
                       void* scratch, hipStream_t stream);

/*
 * Failure report of the last kda_chunk_backward on `scratch` (the same problem and scratch
 * buffer).  The fused backward launch runs the reverse scan and the per-chunk VJP tiles in
 * one grid; a tile waits, with a bound, for the scan to finish its chunk.  A wait that gives
 * up makes the tile overwrite all of its gradients with NaN (and dA_log / ddt_bias become NaN)
 * and leaves a flag in the scratch, which this call reads: it synchronises `stream` and
 * returns KDA_ERR_TIMEOUT (with kda_last_error() saying so) when the flag is set, else KDA_OK.
 * The next kda_chunk_backward on the scratch clears the flag.  Counterpart: the reference
 * reports launch failures through C10_CUDA_KERNEL_LAUNCH_CHECK (chunk.cu:1731); its kernels
 * have no in-kernel waits.
 */
int kda_chunk_backward_status(const kda_chunk_problem* p, const void* scratch, hipStream_t stream);

/*
 * Sets the bound of every in-kernel wait of later kda_chunk_backward launches, in ticks of
 * the 100 MHz wall clock (process-wide; negative restores the 2 s default).  For tests of
 * the failure path: a bound of 0 makes every wait that is not already satisfied give up at
 * once, and every kernel still exits normally.  No counterpart in the reference.
 */
int kda_debug_set_wait_limit(int64_t ticks);

/*
 * kda_chunk_backward without the scratch argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The scratch is a file-scope device array
 * of kda_chunk_backward_noalloc_max_scratch_bytes() bytes (128 MiB), held by every device
 * the library runs on until the process ends; a problem whose
 * kda_chunk_backward_scratch_bytes exceeds it is rejected (KDA_ERR_INVALID).  Every call on
 * one device shares that array: calls that overlap on one device (different streams or
 * threads) race.  All other arguments and results are those of kda_chunk_backward.
 */
int kda_chunk_backward_noalloc(const kda_chunk_problem* p,
                               const void* q, const void* k, const void* v, const void* gate,
                               const void* beta_logits, const float* A_log, const float* dt_bias,
                               const float* initial_state, const void* workspace,
                               const void* grad_output, const float* grad_final_state,
                               void* dq, void* dk, void* dv, void* dgate, void* dbeta_logits,
                               float* dA_log, float* ddt_bias, float* dinitial_state,
                               hipStream_t stream);
size_t kda_chunk_backward_noalloc_max_scratch_bytes(void);

/*
 * Runs one kernel of the chunked forward or backward on buffers that a full
 * kda_chunk_forward / kda_chunk_backward call with the same arguments has prepared, so a
 * benchmark can time that kernel alone.  No counterpart in the reference (it exists for
 * measurement only).  Forward stages: KDA_STAGE_PREP, KDA_STAGE_FWD_INTRA,
 * KDA_STAGE_FWD_SCAN, KDA_STAGE_FWD_OUTPUT; backward stages: KDA_STAGE_BWD_SCAN, KDA_STAGE_BWD_DENSE,
 * KDA_STAGE_BWD_DECAY, KDA_STAGE_BWD_PARAMS.  Arguments are those of the full calls.
 */
#define KDA_STAGE_PREP 0
#define KDA_STAGE_FWD_INTRA 1
#define KDA_STAGE_FWD_SCAN 2
#define KDA_STAGE_FWD_OUTPUT 3
#define KDA_STAGE_BWD_SCAN 10
#define KDA_STAGE_BWD_DENSE 11
#define KDA_STAGE_BWD_DECAY 12
#define KDA_STAGE_BWD_PARAMS 13
#define KDA_STAGE_BWD_VJP 14 /* dense and decay tiles together, as the full backward launches them */
int kda_chunk_forward_stage(int32_t stage, const kda_chunk_problem* p, const void* q,
                            const void* k, const void* v, const void* gate,
                            const void* beta_logits, const float* A_log, const float* dt_bias,
                            const float* initial_state, void* output, float* final_state,
                            void* workspace, hipStream_t stream);
int kda_chunk_backward_stage(int32_t stage, const kda_chunk_problem* p, const void* q,
                             const void* k, const void* v, const void* gate,
                             const void* beta_logits, const float* A_log, const float* dt_bias,
                             const float* initial_state, const void* workspace,
                             const void* grad_output, const float* grad_final_state, void* dq,
                             void* dk, void* dv, void* dgate, void* dbeta_logits, float* dA_log,
                             float* ddt_bias, float* dinitial_state, void* scratch,
                             hipStream_t stream);

/*
 * Single-token recurrent step (T == 1).  Replaces torch.ops.nanochat_kda.recurrent_decode
 * (nanochat/mixers/cuda_kda/recurrent_decode.cu:24-181, schema :186-189).
 *   q, k, gate [B,1,H,K] bf16 (gate K3 raw logits), v [B,1,H,V] bf16, beta_logits [B,1,H] bf16
 *   initial_state f32 [B,H,V,K] or NULL; output bf16 [B,1,H,V]; final_state f32 [B,H,V,K]
 *   or NULL.  final_state may alias initial_state (in-place update).  key_dim in [1, 256]
 *   (64 and 128 on the vector kernel, other sizes one step of the token-serial kernel).
 */
int kda_recurrent_decode(int32_t batch, int32_t heads, int32_t key_dim, int32_t value_dim,
                         int32_t gate_mode, float lower_bound, float scale,
                         const void* q, const void* k, const void* v, const void* gate,
                         const void* beta_logits, const float* A_log, const float* dt_bias,
                         const float* initial_state, void* output, float* final_state,
                         hipStream_t stream);

/*
 * Depthwise causal convolution + SiLU.  Replaces torch.ops.nanochat_kda.causal_convolution_forward
 * (nanochat/mixers/cuda_kda/causal_convolution_forward.cu:149-238, schema :241-244).
 *   x [B,T,C] bf16, weight [C,W] bf16, initial_state [B,C,W] bf16 or NULL,
 *   output [B,T,C] bf16, final_state [B,C,W] bf16 or NULL.  The state holds the W most
 *   recent inputs including the current token.  C % 8 == 0, 1 <= W <= 8.
 */
int kda_causal_conv_forward(int32_t batch, int32_t seq_len, int32_t channels, int32_t width,
                            const void* x, const void* weight, const void* initial_state,
                            void* output, void* final_state, hipStream_t stream);

/* Bytes of scratch kda_causal_conv_backward needs (weight-gradient partials). */
size_t kda_causal_conv_backward_scratch_bytes(int32_t batch, int32_t seq_len, int32_t channels,
                                              int32_t width);

/*
 * Backward of kda_causal_conv_forward.  Replaces torch.ops.nanochat_kda.causal_convolution_backward
 * (nanochat/mixers/cuda_kda/causal_convolution_backward.cu:74-453, schema :455-460).
 *   grad_output [B,T,C] bf16, grad_final_state [B,C,W] bf16 or NULL
 *   dx [B,T,C] bf16, dweight [C,W] bf16, dinitial_state [B,C,W] bf16 or NULL
 * The weight gradient is reduced over (B, T) in a fixed order.
 */
int kda_causal_conv_backward(int32_t batch, int32_t seq_len, int32_t channels, int32_t width,
                             const void* x, const void* weight, const void* initial_state,
                             const void* grad_output, const void* grad_final_state,
                             void* dx, void* dweight, void* dinitial_state,
                             void* scratch, hipStream_t stream);

/*
 * kda_causal_conv_backward with row strides (elements per token) for x and dx, each a
 * multiple of 8 of at least C: x may be a column slice of a wider row (the projection GEMM's
 * output) and dx may land in a slice of a wider gradient row.  No counterpart in the
 * reference (its op takes dense tensors); kda_causal_conv_backward is this with both strides C.
 */
int kda_causal_conv_backward_strided(int32_t batch, int32_t seq_len, int32_t channels, int32_t width,
                                     const void* x, int64_t x_row_stride, const void* weight,
                                     const void* initial_state, const void* grad_output,
                                     const void* grad_final_state, void* dx, int64_t dx_row_stride,
                                     void* dweight, void* dinitial_state, void* scratch,
                                     hipStream_t stream);

/*
 * Fused RMSNorm(x) * weight * sigmoid(gate) over rows of D in [1, 1024] (16-byte vector
 * kernels for D = 64 and 128, one wave per row otherwise).  Replaces
 * torch.ops.nanochat_kda.rmsnorm_gate_forward (nanochat/mixers/cuda_kda/rmsnorm_gate.cu:31-71,
 * schema :278-280).  x, gate, output [rows, D] bf16; weight [D] f32; inv_rms [rows] f32.
 */
int kda_rmsnorm_gate_forward(int64_t rows, int32_t dim, const void* x, const void* gate,
                             const float* weight, float eps, void* output, float* inv_rms,
                             hipStream_t stream);

/* Bytes of scratch kda_rmsnorm_gate_backward needs (weight-gradient partials). */
size_t kda_rmsnorm_gate_backward_scratch_bytes(int64_t rows, int32_t dim);

/*
 * Backward of the fused RMSNorm*gate.  Replaces torch.ops.nanochat_kda.rmsnorm_gate_backward
 * (nanochat/mixers/cuda_kda/rmsnorm_gate.cu:73-184, schema :281-284).
 *   dx, dgate [rows, D] bf16; dweight [D] f32 (fixed-order reduction).
 */
int kda_rmsnorm_gate_backward(int64_t rows, int32_t dim, const void* x, const void* gate,
                              const float* weight, const float* inv_rms, const void* grad_output,
                              float eps, void* dx, void* dgate, float* dweight, void* scratch,
                              hipStream_t stream);

/*
 * kda_rmsnorm_gate_backward with gate and dgate as column slices of wider per-token rows:
 * row r of x / grad_output / dx is (token r / heads, head r % heads); that row's gate is read
 * at token * gate_row_stride + head * dim and its dgate written at
 * token * dgate_row_stride + head * dim (strides multiples of 8, at least heads * dim).
 * heads = 1 and both strides = dim is kda_rmsnorm_gate_backward.  (No reference counterpart:
 * it lets the training mixer read the output gate from, and write its gradient into, the
 * packed projection rows.)
 */
int kda_rmsnorm_gate_backward_strided(int64_t rows, int32_t dim, int32_t heads, const void* x,
                                      const void* gate, int64_t gate_row_stride, const float* weight,
                                      const float* inv_rms, const void* grad_output, float eps, void* dx,
                                      void* dgate, int64_t dgate_row_stride, float* dweight, void* scratch,
                                      hipStream_t stream);

/*
 * Trainer support: soft-capped cross entropy over bf16 logits [rows, stride] (columns
 * >= vocab are vocabulary padding).  Replaces the eager f32 chain of nanochat/gpt.py:600-608
 * (logits.float(), softcap * tanh(logits / softcap), F.cross_entropy(ignore_index=-1)),
 * which the reference fuses with torch.compile (scripts/base_train.py:267).
 *   loss_rows[r] = lse_r - z[r, t_r] (0 where t_r == ignore_index), lse_rows[r] = log sum_j exp z[r, j]
 * The mean is sum(loss_rows) / count(t != ignore_index), formed by the caller.
 */
int kda_softcap_cross_entropy_forward(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                                      const void* logits, const int64_t* targets,
                                      int64_t ignore_index, float* loss_rows, float* lse_rows,
                                      hipStream_t stream);

/*
 * Backward of the above: grad_logits [rows, stride] bf16 =
 *   grad_scale[0] * (softmax(z) - onehot(t)) * (1 - (z / softcap)^2), zero in ignored rows
 * and padding columns.  grad_scale is a device scalar (dL/dmean / non-ignored count).
 */
int kda_softcap_cross_entropy_backward(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                                       const void* logits, const int64_t* targets,
                                       int64_t ignore_index, const float* lse_rows,
                                       const float* grad_scale, void* grad_logits,
                                       hipStream_t stream);

/*
 * Forward and backward of the above in one pass (one read of the logits instead of two),
 * for rows whose columns are all vocabulary: vocab == stride, a multiple of 4096, at most
 * 32768 (kda_softcap_cross_entropy_fused_supported; other shapes use the two calls above).
 * Writes loss_rows and lse_rows as the forward does and grad_logits as the backward would
 * for the device scalar grad_scale (the expected dL/dmean / non-ignored count, as written by
 * kda_softcap_cross_entropy_count).  Same semantics as nanochat/gpt.py:600-608 plus its
 * autograd backward; no counterpart entry point in the reference (its cross entropy runs
 * under torch.compile).
 */
int kda_softcap_cross_entropy_fused_supported(int32_t vocab, int64_t stride);
int kda_softcap_cross_entropy_fused(int64_t rows, int32_t vocab, int64_t stride, float softcap,
                                    const void* logits, const int64_t* targets, int64_t ignore_index,
                                    const float* grad_scale, float* loss_rows, float* lse_rows,
                                    void* grad_logits, hipStream_t stream);

/*
 * count[0] = number of targets != ignore_index, grad_scale[0] = expected_grad / count[0]
 * (device scalars; one workgroup, fixed order): the scale the fused call above assumes when
 * the mean loss will be back-propagated with gradient expected_grad.  Trainer support, no
 * counterpart in the reference.
 */
int kda_softcap_cross_entropy_count(int64_t rows, const int64_t* targets, int64_t ignore_index,
                                    float expected_grad, float* count, float* grad_scale,
                                    hipStream_t stream);

/*
 * data[0..n) (bf16, n a multiple of 8) *= actual[0] / expected, unless actual[0] == expected,
 * in which case nothing is read or written: the backward of the fused cross entropy when the
 * upstream gradient (a device scalar) is not the one its forward assumed.  No host
 * synchronisation.  Trainer support, no counterpart in the reference.
 */
int kda_bf16_rescale_if_changed(int64_t n, void* data, const float* actual, float expected,
                                hipStream_t stream);

/*
 * Mean of loss_rows [rows] over the rows whose target differs from ignore_index, and that
 * row count (both f32 scalars on the device; loss is NaN when every row is ignored).  The
 * reduction F.cross_entropy(reduction="mean") applies in nanochat/gpt.py:600-608, in one
 * workgroup with a fixed summation order.
 */
int kda_softcap_cross_entropy_mean(int64_t rows, const float* loss_rows, const int64_t* targets,
                                   int64_t ignore_index, float* loss, float* count,
                                   hipStream_t stream);

/* Bytes of scratch kda_weight_grad needs for an (M, N, K) problem (0: none). */
size_t kda_weight_grad_scratch_bytes(int64_t M, int32_t N, int32_t K);

/*
 * Trainer support: weight gradient of a linear layer, dweight[N, K] f32 = dy[M, N]^T x[M, K]
 * (bf16, row-major with leading dimensions ldd, ldx).  Replaces the weight-gradient GEMM
 * autograd runs for nanochat's Linear (nanochat/gpt.py:52-57).  Split-contraction partials
 * are summed in a fixed order (deterministic); dweight is overwritten.
 */
int kda_weight_grad(int64_t M, int32_t N, int32_t K, const void* dy, int64_t ldd, const void* x,
                    int64_t ldx, float* dweight, void* scratch, hipStream_t stream);

/*
 * Trainer support: fused elementwise glue of the decoder (reference nanochat/gpt.py,
 * fused there by torch.compile).  bf16 tensors of n elements (n % 8 == 0, 16-byte aligned).
 *   resid_mix: y = a x + b x0 with device scalars a, b (the per-layer resid / x0 lambdas,
 *     gpt.py:585-587); backward dx = a g, dx0 = b g and the scalar gradients sum g x, sum g x0
 *     (fixed-order reduction through `scratch`, kda_resid_mix_backward_scratch_bytes(n)
 *     bytes) written to da[slot], db[slot] of nslots-entry vectors that are zero elsewhere
 *     (a, b point at lambda[slot] of the lambda vectors).
 *   relu2: y = relu(x)^2 (the MLP activation, gpt.py:151-156); backward dx = 2 relu(x) g.
 */
size_t kda_resid_mix_backward_scratch_bytes(int64_t n);
int kda_resid_mix_forward(int64_t n, const float* a, const float* b, const void* x, const void* x0,
                          void* y, hipStream_t stream);
int kda_resid_mix_backward(int64_t n, const float* a, const float* b, const void* x, const void* x0,
                           const void* grad, void* dx, void* dx0, float* da, float* db, int32_t slot,
                           int32_t nslots, void* scratch, hipStream_t stream);
int kda_relu2_forward(int64_t n, const void* x, void* y, hipStream_t stream);
/* rms_norm (no weight; the decoder's norm(), gpt.py:46-48) over bf16 rows of dim = 128 J
 * (J in {1,2,3,4,6,8}): y = x / sqrt(mean(x^2) + eps), rinv [rows] f32 = 1/rms;
 * backward dx = rinv (g - y mean(g y)). */
int kda_rms_norm_forward(int64_t rows, int32_t dim, float eps, const void* x, void* y, float* rinv,
                         hipStream_t stream);
int kda_rms_norm_backward(int64_t rows, int32_t dim, const void* x, const float* rinv,
                          const void* grad, void* dx, hipStream_t stream);
/* The residual add or mix fused into the norm that follows it (gpt.py:585-587 and :200-205):
 * sum = bf16(a x + b x2) (a, b device scalars; NULL means 1, i.e. sum = x + x2) is stored and
 * normalised as kda_rms_norm_forward does (y, rinv of the rounded sum). */
int kda_mix_rms_norm_forward(int64_t rows, int32_t dim, float eps, const float* a, const float* b,
                             const void* x, const void* x2, void* sum, void* y, float* rinv,
                             hipStream_t stream);
/* kda_rms_norm_backward plus grad_add, the gradient reaching x by another path (a residual
 * branch), added before the one rounding; grad_add NULL is kda_rms_norm_backward. */
int kda_rms_norm_backward_add(int64_t rows, int32_t dim, const void* x, const float* rinv,
                              const void* grad, const void* grad_add, void* dx, hipStream_t stream);
int kda_relu2_backward(int64_t n, const void* x, const void* grad, void* dx, hipStream_t stream);
/*
 * Gradient of the token-embedding lookup (the backward of nn.Embedding for the decoder's
 * wte, nanochat/gpt.py:559): grad_weight [vocab, dim] bf16 = sum over tokens t with
 * idx[t] == v of grad_output[t] (f32 sums in token order, one bf16 rounding; rows no token
 * hits are zero).  dim a multiple of 8, at most 512; idx values outside [0, vocab) are
 * ignored.  No sort, atomics or memory-set operations (HIP-graph safe).
 */
int kda_embedding_backward(int64_t n_tokens, int32_t vocab, int32_t dim, const int64_t* idx,
                           const void* grad_output, void* grad_weight, hipStream_t stream);

/*
 * Measurement only (no counterpart in the reference): launches `workgroups` workgroups of
 * four waves; each wave runs `iters` rounds of 8 x 16,384 FLOP of bf16 MFMAs in independent
 * chains with no memory traffic (shape 0: v_mfma_f32_16x16x32_bf16, 8 chains; shape 1:
 * v_mfma_f32_32x32x16_bf16, 4 chains) and *flop receives the launch's FLOP count.  sink:
 * >= workgroups + 2 floats; sink[0] and sink[1] receive workgroup 0's shader-clock cycles and
 * 100 MHz wall-clock ticks over its loop.  bench.py times it between HIP events to obtain the
 * bf16 MFMA rate the device sustains.
 */
int kda_mfma_probe(int32_t shape, int32_t workgroups, int32_t iters, float* sink, double* flop, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KDA_MI355X_H */
