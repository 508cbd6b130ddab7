/*
 * forge_hip.h -- C ABI of libforge_hip.so, the MI355X (gfx950) backend for
 * ForgeLM's autoregressive token loop.
 *
 * Every function returns an int status (FH_OK = 0, negative = error class) and
 * never throws across the boundary.  On failure fh_last_error() returns a
 * thread-local message.  Pointers are plain host pointers unless a parameter
 * name ends in _dev.  All calls on one context must be serialised by the
 * caller (the C# side keeps a lock, as the reference CudaBackend does with
 * lock(_gate), src/LLM.Core/Tensor/Cuda/CudaBackend.cs:36).
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   fh_context_*            CudaBackend ctor / Dispose / DeviceName / DeviceMemoryBytes
 *                           (src/LLM.Core/Tensor/Cuda/CudaBackend.cs:114-215, 1067-1093;
 *                           banner in src/LLM.Cli/Program.cs:132-145)
 *   fh_session_create       GptModel ctor shape (src/LLM.Core/Model/GptModel.cs:38-99,
 *                           ModelConfig.cs:8-25)
 *   fh_session_init_random  GptModel ctor random init from new Random(seed)
 *                           (GptModel.cs:38-99, Tensor.FillNormal Tensor.cs:79-91)
 *   fh_session_load_weights Checkpoint.LoadCore's ReadTensor into Parameters, registry
 *                           order (src/LLM.Core/Checkpoint/Checkpoint.cs:222-227)
 *   fh_session_read_param   EnsureHostCurrent on one parameter (ITensorBackend.cs:193)
 *   fh_forward_last         GptModel.ForwardLast (GptModel.cs:202-209)
 *   fh_generate             Sampler.Generate (src/LLM.Core/Inference/Sampler.cs:78-109)
 *                           incl. ApplyRepetitionControls (:111-165) and Sample (:29-69)
 *   fh_sample_logits        Sampler.ApplyRepetitionControls + Sampler.Sample on
 *                           caller-provided device logits (Sampler.cs:29-69, 111-165)
 */
#ifndef FORGE_HIP_H
#define FORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define FH_OK 0
#define FH_ERR_INVALID (-1)     /* bad argument: ArgumentException in the reference */
#define FH_ERR_RANGE (-2)       /* out of range: ArgumentOutOfRangeException */
#define FH_ERR_HIP (-3)         /* HIP runtime failure */
#define FH_ERR_OOM (-4)         /* device allocation failed */
#define FH_ERR_STATE (-5)       /* call out of order (e.g. generate before weights) */
#define FH_ERR_UNSUPPORTED (-6) /* shape or option this build does not run */
#define FH_ERR_DATA (-7)        /* malformed or corrupted file: InvalidDataException */

/* weight / activation storage type of a session */
#define FH_DTYPE_F32 0
#define FH_DTYPE_BF16 1

typedef struct fh_context fh_context;
typedef struct fh_session fh_session;

/* Model shape, ModelConfig(VocabSize, ContextLength, DModel, NLayers, NHeads).
 * max_batch: sequences decoded together by one session (all share the prompt
 * length).  dtype: FH_DTYPE_F32 or FH_DTYPE_BF16 (weights and GEMM operands;
 * accumulation and the residual stream stay fp32). */
typedef struct fh_model_desc {
  int32_t vocab_size;
  int32_t context_length;
  int32_t d_model;
  int32_t n_layers;
  int32_t n_heads;
  int32_t max_batch;
  int32_t dtype;
  int32_t reserved;
} fh_model_desc;

/* Sampler.Generate options.  temperature <= 0 selects Greedy (no RNG draw);
 * top_k <= 0 or >= V disables filtering; eos_id < 0 means no EOS;
 * repetition_penalty == 1 and no_repeat_ngram == 0 skip ApplyRepetitionControls. */
typedef struct fh_sampling {
  float temperature;
  int32_t top_k;
  float repetition_penalty;
  int32_t no_repeat_ngram;
  int32_t eos_id;
  int32_t reserved;
} fh_sampling;

/* errors */
int fh_last_error(char* buf, size_t n);
const char* fh_version(void);

/* The first n NextDouble() values of new System.Random(seed) (the legacy seeded
 * generator): the uniforms Sampler.Sample draws (Sampler.cs:61) when the CLI
 * seeds its Random (src/LLM.Cli/Program.cs:664).  Host-only. */
int fh_random_doubles(int32_t seed, int n, double* out);

/* context = one device + one stream */
int fh_context_create(int device, fh_context** out);
int fh_context_destroy(fh_context* ctx);
int fh_context_info(fh_context* ctx, char* name, size_t name_len, uint64_t* total_mem_bytes,
                    int32_t* compute_units);
/* Memory figures for the banner and for callers that budget device memory: the
 * device's free bytes (hipMemGetInfo) and the device bytes this context holds as
 * fh_sample_logits' scratch (0 until its first call).  Either pointer may be NULL.
 * (The CUDA backend's counterpart is its arena accounting, CudaBackend.cs:397-543.) */
int fh_context_memory(fh_context* ctx, uint64_t* free_bytes, uint64_t* sampler_scratch_bytes);

/* Device buffers for op-level callers: the residency half of the tensor contract
 * (CudaBackend's arena rent/return and Read/Write, CudaBackend.cs:397-543;
 * InvalidateDeviceCache = write, EnsureHostCurrent = read, ITensorBackend.cs:166-193).
 * Writes and reads are synchronous with respect to the context's stream. */
int fh_buffer_alloc(fh_context* ctx, size_t bytes, void** out_dev);
int fh_buffer_free(fh_context* ctx, void* dev);
int fh_buffer_write(fh_context* ctx, void* dst_dev, const void* src, size_t bytes);
int fh_buffer_read(fh_context* ctx, void* dst, const void* src_dev, size_t bytes);
/* ITensorBackend.Copy(src, dst) on device buffers (ITensorBackend.cs:86): one copy
 * kernel on the context stream, synchronous.  Both pointers 16-byte aligned.  When
 * ms_out is not NULL it receives the kernel's duration from HIP events (the
 * bandwidth calibration of the benchmark's traffic counters). */
int fh_buffer_copy(fh_context* ctx, void* dst_dev, const void* src_dev, size_t bytes, float* ms_out);
/* The sum of a device buffer's 32-bit words mod 2^64 (an integrity check of an
 * upload; no reference counterpart), synchronous.  src 16-byte aligned, bytes a
 * multiple of 4.  When ms_out is not NULL it receives the duration of the pass
 * that reads the buffer (one read of every byte: the device's read bandwidth,
 * reported next to the decode kernel's roofline). */
int fh_buffer_checksum(fh_context* ctx, const void* src_dev, size_t bytes, uint64_t* sum_out, float* ms_out);

/* ITensorBackend.MatMulNN(a, b, y, M, K, N, accumulate) (ITensorBackend.cs:22) on
 * device buffers: y[M][N] = a[M][K] @ b[K][N], or += when accumulate != 0.  a and
 * y fp32; b fp32 or bf16 (dtype).  The product runs on the MFMA GEMM the token
 * loop uses for more than 4 rows (bf16: a rounded to bf16, fp32 accumulation).
 * Synchronous. */
int fh_matmul_nn(fh_context* ctx, const void* a_dev, const void* b_dev, void* y_dev, int M, int K, int N,
                 int dtype, int accumulate);

/* session = weights + KV cache + token history + scratch for max_batch sequences */
int fh_session_create(fh_context* ctx, const fh_model_desc* desc, fh_session** out);
int fh_session_destroy(fh_session* s);
int64_t fh_param_count(const fh_model_desc* desc);
/* Number of registry tensors, and the name/size of tensor i (registry order). */
int fh_param_info(const fh_model_desc* desc, int index, char* name, size_t name_len, int64_t* numel);
int fh_session_init_random(fh_session* s, int32_t seed);
/* The same initial weights into a host array of n floats (registry order): the GptModel
 * constructor's init from new Random(seed) (GptModel.cs:38-99), without a device. */
int fh_init_weights(const fh_model_desc* desc, int32_t seed, float* out, int64_t n);
/* tensors[i] points at registry tensor i (fp32, host); n must equal the registry size. */
int fh_session_load_weights(fh_session* s, const float* const* tensors, int n);
/* Copies the device copy of registry tensor `index` back as fp32 (bf16 sessions widen). */
int fh_session_read_param(fh_session* s, int index, float* out, int64_t numel);

/* FORGEMODEL1 checkpoints (Checkpoint.Load / LoadCore, src/LLM.Core/Checkpoint/Checkpoint.cs:116-250).
 * fh_checkpoint_info validates the header the way LoadCore does (magic, header length,
 * architecture, model name, training header, ModelConfig, registry names, payload size)
 * and, with verify != 0, the SHA-256 trailer too; it fills desc's five model fields and
 * the model name.  fh_session_load_checkpoint reads and verifies the whole file and
 * uploads the weights into a session of the same configuration (the optimizer moments
 * are checksummed and dropped).  Data errors return FH_ERR_DATA with LoadCore's message. */
int fh_checkpoint_info(const char* path, fh_model_desc* desc, char* name, size_t name_len, int verify);
int fh_session_load_checkpoint(fh_session* s, const char* path);
/* SHA-256 (FIPS 180-4) of n bytes, the checkpoint trailer's hash. */
int fh_sha256(const void* data, size_t n, uint8_t* out32);

/* GptModel.ForwardLast for `batch` windows of equal length T (ids[b*T + t]):
 * logits_out[b*V + v] is the last row's logits.  Full recompute, no state kept. */
int fh_forward_last(fh_session* s, const int32_t* ids, int batch, int T, float* logits_out);

/* Sampler.Generate for `batch` sequences that share prompt_len.
 *   prompts[b*prompt_len + t]  prompt ids
 *   uniforms[b*max_new + n]    the NextDouble of step n (read only when temperature > 0;
 *                              may be NULL for greedy)
 *   out_ids[b*max_new + n]     generated ids; out_counts[b] = tokens yielded
 *                              (fewer than max_new only when eos_id was yielded)
 *   logits_dump                optional [batch][max_new][V] raw ForwardLast logits
 * Only the sampled ids cross back to the host (plus the optional dump). */
int fh_generate(fh_session* s, const int32_t* prompts, int batch, int prompt_len, int max_new,
                const fh_sampling* opts, const double* uniforms, int32_t* out_ids,
                int32_t* out_counts, float* logits_dump);

/* Sampler.Generate as a stream (Sampler.cs:78-109 yields one id per step): the same
 * generation as fh_generate, run a chunk of steps at a time so ids reach the host
 * (and a tokenizer's decoder) while the loop continues.  fh_generate_begin validates
 * and uploads like fh_generate and enqueues nothing; each fh_generate_next enqueues up
 * to `steps` more steps, waits for them, copies out_ids [batch][max_new] and out_counts
 * as fh_generate does for the steps done so far, and sets *produced to the steps done.
 * Sampled generations take the uniforms either all at begin ([batch][max_new]) or, when
 * begin's uniforms are null, per call ([batch][steps], one NextDouble per step, so a
 * caller that stops after eos has drawn exactly the reference's count).  The stream ends
 * after max_new steps; fh_generate, fh_forward_last or a new begin on the session end it
 * earlier.  The ids equal fh_generate's for any chunking. */
int fh_generate_begin(fh_session* s, const int32_t* prompts, int batch, int prompt_len, int max_new,
                      const fh_sampling* opts, const double* uniforms);
int fh_generate_next(fh_session* s, int steps, const double* uniforms, int32_t* out_ids, int32_t* out_counts,
                     int32_t* produced);

/* Timing of the last fh_generate, from HIP events on the session stream:
 * prefill_ms (first forward, incl. embedding of the prompt) and decode_ms
 * (all later steps), plus how many decode steps ran without a re-prefill. */
int fh_last_timing(fh_session* s, double* prefill_ms, double* decode_ms, int32_t* cached_steps,
                   int32_t* reprefill_steps);

/* Which kernels ran the cached decode steps of the last fh_generate /
 * fh_generate_begin (0 when it had none): a diagnostic for tests, like the
 * reference CUDA backend's test-only call counters (FusedAttentionCallCount and
 * the others, src/LLM.Core/Tensor/Cuda/CudaBackend.cs:257-270). */
#define FH_ROUTE_FUSED_STEP 1       /* the persistent batch-1 decode kernel */
#define FH_ROUTE_FUSED_EPILOGUES 2  /* split-K reductions fused with the KV store and LayerNorms */
#define FH_ROUTE_ATTN_IN_PROJ 4     /* + attention chunks combined in attn.proj's operand load */
#define FH_ROUTE_UNFUSED 8          /* one kernel per op */
#define FH_ROUTE_FUSED_SAMPLER 16   /* the persistent kernel also drew the sampled ids (top-k sampling) */
#define FH_ROUTE_RETRIED 32         /* ... and met an exact top-k tie, so the generation re-ran per step */
#define FH_ROUTE_FALLBACK 64        /* a fused launch gave up (a hand-off wait past its spin limit, or its
                                       blocks not covering the XCD slots): fh_generate re-ran the generation
                                       on the generic kernels, whose ids it returned */
int fh_last_route(fh_session* s, int32_t* route);

/* Diagnostics of the persistent decode kernel (no reference counterpart): with
 * FORGE_HIP_TRACE=1 set when the session is created, each fused launch records
 * wall-clock timestamps (100 MHz) of one step (layer 1 of its sixth token, and the
 * head of that token) in every block: 64 per block, block-major, n >= 256 * 64.
 * Entries 0-31 are the control wave's marks, 32-63 data wave 0's; entry 12 is the
 * block's XCD.  forge_hip.trace prints the per-hand-off timeline from them. */
int fh_debug_fused_trace(fh_session* s, unsigned long long* out, int n);

/* Sampler.ApplyRepetitionControls + Sampler.Sample on one logit row already on
 * the device: logits_dev [V] (not modified), history [n_hist] host ids, u01 the
 * NextDouble for this draw.  Returns the id in *out_id. */
int fh_sample_logits(fh_context* ctx, const float* logits_dev, int V, const int32_t* history,
                     int n_hist, const fh_sampling* opts, double u01, int32_t* out_id);

/* fh_sample_logits without any device allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, checks and result as fh_sample_logits, but
 * the scratch (the work row, the uploaded history, the uniform and the result) is
 * one fixed array in device memory that each device holds until the process ends
 * (about 392 KB), so V may be at most FH_NOALLOC_MAX_VOCAB and n_hist at most
 * FH_NOALLOC_MAX_HISTORY (FH_ERR_RANGE otherwise).  Every call on one device shares
 * that array; the library serialises calls on one device (a per-device lock held for
 * the whole call, which returns after the stream has finished), so overlapping calls
 * from several threads or contexts take turns.  Device ids must be below 64. */
#define FH_NOALLOC_MAX_VOCAB 65536
#define FH_NOALLOC_MAX_HISTORY 32768
int fh_sample_logits_noalloc(fh_context* ctx, const float* logits_dev, int V, const int32_t* history, int n_hist,
                             const fh_sampling* opts, double u01, int32_t* out_id);

/* ---- op-level ITensorBackend on device buffers ---------------------------------
 * One entry point per ITensorBackend method (src/LLM.Core/Tensor/ITensorBackend.cs);
 * every tensor argument is a device pointer to row-major fp32 of the documented
 * shape, sizes are explicit.  Work is ordered on the context's stream and returns
 * without waiting, except where a host value comes back (the cross-entropy loss,
 * fh_op_end_loss_accumulation, the sums of squares) or a host index array is
 * uploaded (it is copied before the call returns).  `accumulate` means += into y.
 * The host mirror keeps the residency contract (InvalidateDeviceCache /
 * EnsureHostCurrent, ITensorBackend.cs:166-193) over these pointers. */

/* MatMulNN / BatchedMatMulNN (ITensorBackend.cs:22, 35): per slot s < slots,
 * y[s] (+)= a[s] @ b[s]; a [slots*M, K], b [slots*K, N], y [slots*M, N]. */
int fh_op_matmul_nn(fh_context* ctx, const void* a, const void* b, void* y, int slots, int M, int K, int N,
                    int accumulate);
/* MatMulNT / BatchedMatMulNT (:24, 37): y[s] (+)= a[s] @ b[s]^T; b [slots*N, K]. */
int fh_op_matmul_nt(fh_context* ctx, const void* a, const void* b, void* y, int slots, int M, int K, int N,
                    int accumulate);
/* MatMulTN / BatchedMatMulTN (:26, 39): y[s] (+)= a[s]^T @ b[s]; a [slots*K, M]. */
int fh_op_matmul_tn(fh_context* ctx, const void* a, const void* b, void* y, int slots, int M, int K, int N,
                    int accumulate);
/* PackHeads (:49): dst[(q*H+h)*T+t, e] = src[q*T+t, col_base+h*hd+e]; src rows are
 * src_cols wide.  UnpackHeads (:55) is the inverse into dst rows dst_cols wide. */
int fh_op_pack_heads(fh_context* ctx, const void* src, int src_cols, void* dst, int batch, int T, int n_heads,
                     int head_dim, int col_base);
int fh_op_unpack_heads(fh_context* ctx, const void* src, void* dst, int dst_cols, int batch, int T, int n_heads,
                       int head_dim, int col_base);
/* AddBias (:80) y[r,:] += bias; SumRows (:82) dbias += column sums of dy (accumulates). */
int fh_op_add_bias(fh_context* ctx, void* y, const void* bias, int rows, int cols);
int fh_op_sum_rows(fh_context* ctx, const void* dy, void* dbias, int rows, int cols);
/* AddInPlace (:84), Copy (:86), Scale (:94), Zero (:200) over n floats. */
int fh_op_add_in_place(fh_context* ctx, void* dst, const void* src, int64_t n);
int fh_op_copy(fh_context* ctx, const void* src, void* dst, int64_t n);
int fh_op_scale(fh_context* ctx, void* x, int64_t n, float factor);
int fh_op_zero(fh_context* ctx, void* x, int64_t n);
/* CopyBlock (:92): rows x cols block from (src_row, src_col) of src to (dst_row,
 * dst_col) of dst; the rest of dst is kept. */
int fh_op_copy_block(fh_context* ctx, const void* src, int src_cols, void* dst, int dst_cols, int src_row,
                     int src_col, int dst_row, int dst_col, int rows, int cols);
/* Transpose (:96): out [cols, rows] = x [rows, cols]^T. */
int fh_op_transpose(fh_context* ctx, const void* x, void* out, int rows, int cols);
/* LayerNormForward (:103): out, and mean / rstd [rows]; LayerNormBackward (:106): dx
 * overwritten, dw and db accumulate. */
int fh_op_layernorm_forward(fh_context* ctx, const void* x, const void* w, const void* b, void* out, void* mean,
                            void* rstd, int rows, int cols, float eps);
int fh_op_layernorm_backward(fh_context* ctx, const void* dout, const void* x, const void* w, const void* mean,
                             const void* rstd, void* dx, void* dw, void* db, int rows, int cols);
/* SoftmaxForward (:112) in place; ScaledCausalSoftmaxForward (:117): scale, causal mask
 * (row r is query r % T of a packed [T,T] block) and softmax, in place. */
int fh_op_softmax_forward(fh_context* ctx, void* x, int rows, int cols);
int fh_op_scaled_causal_softmax_forward(fh_context* ctx, void* scores, int rows, int T, float scale);
/* SoftmaxBackward (:114) with scale 1; ScaledSoftmaxBackward (:125) with the scale. */
int fh_op_softmax_backward(fh_context* ctx, const void* dout, const void* softmax_out, void* dx, int rows, int cols,
                           float scale);
/* GeluForward / GeluBackward (:134-135) over n floats. */
int fh_op_gelu_forward(fh_context* ctx, const void* x, void* out, int64_t n);
int fh_op_gelu_backward(fh_context* ctx, const void* dout, const void* x, void* dx, int64_t n);
/* EmbeddingForward (:139): out[t,:] = table[indices[t],:]; EmbeddingBackward (:141):
 * dtable[indices[t],:] += dout[t,:].  indices is a host array of n ids, each checked
 * against the table's rows (FH_ERR_RANGE). */
int fh_op_embedding_forward(fh_context* ctx, const void* table, int table_rows, const int32_t* indices, int n,
                            void* out, int D);
int fh_op_embedding_backward(fh_context* ctx, const void* dout, const int32_t* indices, int n, void* dtable,
                             int table_rows, int D);
/* CausalMask (:145) over len floats of packed [T,T] blocks. */
int fh_op_causal_mask(fh_context* ctx, void* scores, int64_t len, int T);
/* CrossEntropyForward (:154): probs (may alias logits) and the mean loss over the
 * non-ignored targets (host array of T) in *loss; while a loss accumulation is active
 * the loss stays on the device and *loss is 0.  BeginLossAccumulation /
 * EndLossAccumulation (:159-161): the mean over every non-ignored target since begin;
 * out-of-order calls return FH_ERR_STATE with the reference's messages.
 * CrossEntropyBackward (:164): dlogits (may alias probs) = (probs - onehot) / count. */
int fh_op_cross_entropy_forward(fh_context* ctx, const void* logits, const int32_t* targets, void* probs, int T,
                                int V, int ignore_index, float* loss);
int fh_op_begin_loss_accumulation(fh_context* ctx);
int fh_op_end_loss_accumulation(fh_context* ctx, float* mean_loss);
int fh_op_cross_entropy_backward(fh_context* ctx, const void* probs, const int32_t* targets, void* dlogits, int T,
                                 int V, int ignore_index);
/* SumSquares (:214) and GlobalSumSquares (:227): sum of x^2 in double, one readback. */
int fh_op_sum_squares(fh_context* ctx, const void* x, int64_t n, double* out);
int fh_op_global_sum_squares(fh_context* ctx, const void* const* xs, const int64_t* ns, int count, double* out);
/* AdamWStep (:241): moments and weights of n elements; step is 1-based; weight decay
 * applies when weight_decay != 0 and is_matrix (the tensor's rank is above 1). */
int fh_op_adamw_step(fh_context* ctx, void* w, const void* g, void* m, void* v, int64_t n, float lr, float beta1,
                     float beta2, float eps, float weight_decay, int step, int is_matrix);

#ifdef __cplusplus
}
#endif
#endif /* FORGE_HIP_H */
