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

/* Sampler.ApplyRepetitionControls + Sampler.Sample on one logit row already on
 * the device: logits_dev [V] (not modified), history [n_hist] host ids, u01 the
 * NextDouble for this draw.  Returns the id in *out_id. */
int fh_sample_logits(fh_context* ctx, const float* logits_dev, int V, const int32_t* history,
                     int n_hist, const fh_sampling* opts, double u01, int32_t* out_id);

#ifdef __cplusplus
}
#endif
#endif /* FORGE_HIP_H */
