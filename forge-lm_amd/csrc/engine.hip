// engine.hip -- session engine and C ABI of libforge_hip.so (include/forge_hip.h).
//
// A session owns, in device memory:
//   * the parameters in registry order (GptModel.cs:38-99), each 256-byte
//     aligned; matrices in the session dtype, vectors always fp32;
//   * the KV cache, K and V each [L][B][H][ctx][hd] (contiguous 256-byte rows
//     per head and position, so decode attention streams one head at a time);
//   * the token history [B][prompt_len + max_new], the step counter, sampler
//     scratch and activations for B*ctx rows.
// The token loop (Sampler.Generate, src/LLM.Core/Inference/Sampler.cs:78-109)
// runs on the stream with no host round trip per token: each step's kernels
// read the step counter from device memory, the sampler appends the sampled id
// to the device history and advances the counter.  The host only decides,
// from the lengths alone, which steps are cached decode steps and which are
// re-prefills after the window slid (Sampler.cs:93-94 restarts positions at 0,
// so no cache survives a slide).  Each kind of step is captured once into a
// HIP graph and replayed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/forge_hip.h"
#include "decode_fast.hpp"
#include "kernels.hpp"

namespace fh {
void init_registry_random(int seed, int n_layers, const std::vector<int64_t>& offsets,
                          const std::vector<int64_t>& sizes, const std::vector<int>& kinds, float* w);
void random_doubles(int seed, int n, double* out);
struct CkptHeader {
  int vocab = 0, ctx = 0, d = 0, layers = 0, heads = 0;
  std::string name, arch;
  std::vector<std::string> names;
  bool has_training = false, has_moments = false;
};
std::string read_checkpoint(const char* path, CkptHeader* hdr,
                            std::string (*registry)(const CkptHeader&, std::vector<std::string>*, int64_t*),
                            std::vector<float>* weights, bool header_only, bool* data_error);
void sha256(const void* data, size_t n, uint8_t out[32]);
}

using namespace fh;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_err;

// gen_collect's answer when a persistent sampled launch reported a case for the
// per-step sampler (not returned across the C ABI: fh_generate repeats the generation)
constexpr int kRetryPerStep = -100;
constexpr int kRetryGeneric = -101;  // a fused launch failed: fh_generate re-runs on the generic kernels
constexpr int kResumePerStep = -102;  // a stream's in-kernel sampler met a tie: resume on the per-step sampler

static int set_err(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

namespace fh {
// the same thread-local message, for the op entry points (ops.hip)
int set_error(int code, const char* msg) {
  g_err = msg;
  return code;
}
struct OpsState;
void ops_state_free(OpsState* o);
}  // namespace fh

#define HIP_TRY(expr)                                                                                   \
  do {                                                                                                  \
    hipError_t e_ = (expr);                                                                             \
    if (e_ != hipSuccess)                                                                               \
      return set_err(e_ == hipErrorOutOfMemory ? FH_ERR_OOM : FH_ERR_HIP, "%s failed: %s (%s:%d)", #expr, \
                     hipGetErrorString(e_), __FILE__, __LINE__);                                        \
  } while (0)

#define FH_TRY(expr)        \
  do {                      \
    int r_ = (expr);        \
    if (r_ != FH_OK) return r_; \
  } while (0)

// ---------------------------------------------------------------------------
// registry
// ---------------------------------------------------------------------------
namespace {

struct Slot {
  std::string name;
  int64_t numel;
  bool matrix;  // stored in the session dtype
  int init_kind;  // 0 zero, 1 ones, 2 N(0,0.02), 3 N(0,0.02/sqrt(2L))
};

std::vector<Slot> make_registry(const fh_model_desc& d) {
  const int64_t D = d.d_model;
  std::vector<Slot> r;
  r.push_back({"tok_emb", (int64_t)d.vocab_size * D, true, 2});
  r.push_back({"pos_emb", (int64_t)d.context_length * D, true, 2});
  for (int i = 0; i < d.n_layers; i++) {
    std::string p = "blocks." + std::to_string(i) + ".";
    r.push_back({p + "ln1.w", D, false, 1});
    r.push_back({p + "ln1.b", D, false, 0});
    r.push_back({p + "attn.qkv.w", D * 3 * D, true, 2});
    r.push_back({p + "attn.qkv.b", 3 * D, false, 0});
    r.push_back({p + "attn.proj.w", D * D, true, 3});
    r.push_back({p + "attn.proj.b", D, false, 0});
    r.push_back({p + "ln2.w", D, false, 1});
    r.push_back({p + "ln2.b", D, false, 0});
    r.push_back({p + "mlp.fc.w", D * 4 * D, true, 2});
    r.push_back({p + "mlp.fc.b", 4 * D, false, 0});
    r.push_back({p + "mlp.proj.w", 4 * D * D, true, 3});
    r.push_back({p + "mlp.proj.b", D, false, 0});
  }
  r.push_back({"ln_f.w", D, false, 1});
  r.push_back({"ln_f.b", D, false, 0});
  return r;
}

int validate_desc(const fh_model_desc* d) {
  if (!d) return set_err(FH_ERR_INVALID, "model descriptor is null");
  if (d->vocab_size <= 0) return set_err(FH_ERR_INVALID, "VocabSize must be positive.");
  if (d->context_length <= 0) return set_err(FH_ERR_INVALID, "ContextLength must be positive.");
  if (d->d_model <= 0) return set_err(FH_ERR_INVALID, "DModel must be positive.");
  if (d->n_layers <= 0) return set_err(FH_ERR_INVALID, "NLayers must be positive.");
  if (d->n_heads <= 0) return set_err(FH_ERR_INVALID, "NHeads must be positive.");
  if (d->d_model % d->n_heads != 0)
    return set_err(FH_ERR_INVALID, "DModel (%d) must be divisible by NHeads (%d).", d->d_model, d->n_heads);
  if (d->max_batch <= 0) return set_err(FH_ERR_INVALID, "max_batch must be positive.");
  if (d->dtype != FH_DTYPE_F32 && d->dtype != FH_DTYPE_BF16) return set_err(FH_ERR_INVALID, "unknown dtype %d", d->dtype);
  if (d->d_model % 8 != 0 || d->d_model > 1024)
    return set_err(FH_ERR_UNSUPPORTED, "this build runs DModel in multiples of 8 up to 1024 (got %d)", d->d_model);
  if (d->d_model / d->n_heads > 128) return set_err(FH_ERR_UNSUPPORTED, "head_dim above 128 is not supported");
  if (d->vocab_size > 65536) return set_err(FH_ERR_UNSUPPORTED, "vocabularies above 65536 are not supported");
  return FH_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
struct fh_context {
  int device = 0;
  hipStream_t stream = nullptr;
  hipDeviceProp_t props{};
  // scratch for fh_sample_logits
  float* s_work = nullptr;
  int* s_ints = nullptr;  // tokens | step | done | out | count
  int s_V = 0, s_hist = 0;
  double* s_u = nullptr;
  int sessions = 0;              // live sessions on this context
  bool destroy_pending = false;  // fh_context_destroy ran while sessions were alive
  fh::OpsState* ops = nullptr;   // state of the op-level entry points (ops.hip)
};

namespace fh {
hipStream_t context_stream(fh_context* c) { return c->stream; }
int context_device(fh_context* c) { return c->device; }
OpsState*& context_ops(fh_context* c) { return c->ops; }
}  // namespace fh

// ---------------------------------------------------------------------------
// session
// ---------------------------------------------------------------------------
struct GraphKey {
  int kind = -1, B = 0, P = 0, max_new = 0, top_k = 0, ngram = 0, eos = 0;
  float temperature = 0.f, penalty = 0.f;
  const void* dump = nullptr;
  const void* uniforms = nullptr;
  uint64_t gen = 0;
  bool fused = false;  // captured with the fused decode step
  bool operator==(const GraphKey& o) const {
    return kind == o.kind && B == o.B && P == o.P && max_new == o.max_new && top_k == o.top_k && ngram == o.ngram &&
           eos == o.eos && temperature == o.temperature && penalty == o.penalty && dump == o.dump &&
           uniforms == o.uniforms && gen == o.gen && fused == o.fused;
  }
};

struct CachedGraph {
  GraphKey key;
  hipGraphExec_t exec = nullptr;
  int route = 0;  // FH_ROUTE_* bits of the decode step the graph holds
};

namespace {
struct StepPlan {
  int P = 0, max_new = 0, tok_stride = 0;
  const fh_sampling* opts = nullptr;
  bool with_sample = true;
};

// a generation between fh_generate_begin and its last fh_generate_next (or inside fh_generate)
struct GenState {
  bool active = false;
  int B = 0, P = 0, max_new = 0;
  int next = 0;         // first step not yet enqueued (step 0 is the prompt's forward)
  int n_dec = 0, n_re = 0;
  bool persistent = false, dump = false, sampled = false;
  bool persist_sampled = false;  // the persistent launches also draw (sampled kernel)
  bool deferred = false;  // sampled, uniforms supplied per fh_generate_next call
  bool one_shot = false;  // inside fh_generate (not a stream of fh_generate_next calls)
  fh_sampling opts{};
  StepPlan plan;        // plan.opts points at opts
};
}  // namespace

struct fh_session {
  fh_context* ctx = nullptr;
  fh_model_desc d{};
  std::vector<Slot> reg;
  std::vector<size_t> off;  // byte offsets in wbuf
  char* wbuf = nullptr;
  size_t wbytes = 0;
  // per layer, the four matrices transposed to [N][K] (session dtype) for the MFMA GEMM
  char* wtbuf = nullptr;
  std::vector<size_t> wtoff;  // byte offset in wtbuf per registry slot (matrices of blocks only)
  bool loaded = false;
  int esize = 4;  // bytes per matrix element
  // KV cache
  void* kc = nullptr;
  void* vc = nullptr;
  size_t kv_layer = 0;  // elements per layer (B*H*ctx*hd)
  // activations (rows = B*ctx)
  float *x = nullptr, *x2 = nullptr, *xn = nullptr, *qkv = nullptr, *o = nullptr, *h = nullptr;
  float *part = nullptr, *apart = nullptr, *logits = nullptr, *work = nullptr;
  size_t part_floats = 0;
  // bf16 sessions: arrival counters of the window mlp.proj with K split in two
  // (one per 256 x 256 tile, zero between launches; o holds the first halves' sums)
  int* gsplit = nullptr;
  int gsplit_cap = 0;
  int* step = nullptr;
  int* done = nullptr;
  int* out_counts = nullptr;
  // per-call buffers (grow on demand)
  int* tokens = nullptr;
  size_t tokens_cap = 0;
  int* out_ids = nullptr;
  size_t out_cap = 0;
  double* uniforms = nullptr;
  size_t uni_cap = 0;
  // pinned host staging of a generation's results: ids [B * max_new], counts [B],
  // then the fused kernel's and the split-K GEMM's error words (one stream sync)
  int32_t* hstage = nullptr;
  size_t hstage_cap = 0;
  float* dump = nullptr;
  size_t dump_cap = 0;
  uint64_t buf_gen = 1;
  // fast decode path state
  FastDecode fast;
  bool fast_allowed = true;  // FORGE_HIP_FUSED_DECODE=0 at session creation selects the generic kernels
  bool bf16_act = true;      // FORGE_HIP_BF16_ACT=0 keeps a bf16 session's window GEMMs on fp32 operands
  bool last_tail = true;     // FORGE_HIP_LAST_LAYER_TAIL=0 runs a window's last layer on every row
  bool counted = false;      // holds a reference on its context
  bool no_sampled_fused = false;  // set while fh_generate repeats a generation on the per-step path
  bool use_fast() const { return fast.enabled && fast_allowed; }
  // generation in progress
  GenState gen;
  // graphs
  CachedGraph g_decode, g_reprefill;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  double t_prefill = 0, t_decode = 0;
  int n_cached = 0, n_reprefill = 0;
  int route = 0;  // FH_ROUTE_* bits of the decode steps enqueued since the last generate began

  template <typename T>
  const T* w(size_t i) const {
    return reinterpret_cast<const T*>(wbuf + off[i]);
  }
  template <typename T>
  const T* wt(size_t i) const {
    return reinterpret_cast<const T*>(wtbuf + wtoff[i]);
  }
  const float* v(size_t i) const { return reinterpret_cast<const float*>(wbuf + off[i]); }
  size_t idx_tok() const { return 0; }
  size_t idx_pos() const { return 1; }
  size_t idx_blk(int l, int k) const { return 2 + (size_t)l * 12 + k; }  // k: 0 ln1w .. 11 mpb
  size_t idx_lnf() const { return 2 + (size_t)d.n_layers * 12; }
  int B() const { return d.max_batch; }
  int hd() const { return d.d_model / d.n_heads; }
};

namespace {

template <typename T>
int dev_alloc(T** p, size_t count) {
  if (count == 0) count = 1;
  void* q = nullptr;
  hipError_t e = hipMalloc(&q, count * sizeof(T));
  if (e != hipSuccess)
    return set_err(e == hipErrorOutOfMemory ? FH_ERR_OOM : FH_ERR_HIP, "hipMalloc(%zu bytes): %s", count * sizeof(T),
                   hipGetErrorString(e));
  *p = static_cast<T*>(q);
  return FH_OK;
}

template <typename T>
void dev_free(T*& p) {
  if (p) (void)hipFree((void*)p);
  p = nullptr;
}

template <typename T>
int ensure(T** p, size_t* cap, size_t need, uint64_t* gen) {
  if (need <= *cap && *p) return FH_OK;
  dev_free(*p);
  *cap = 0;
  FH_TRY(dev_alloc(p, need));
  *cap = need;
  ++*gen;
  return FH_OK;
}

void drop_graph(CachedGraph& g) {
  if (g.exec) (void)hipGraphExecDestroy(g.exec);
  g.exec = nullptr;
  g.key = GraphKey{};
}

int check_launch(hipError_t e, const char* what) {
  if (e == hipSuccess) return FH_OK;
  if (e == hipErrorInvalidValue) return set_err(FH_ERR_INVALID, "%s: operand shapes rejected by the kernel wrapper", what);
  return set_err(FH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define LAUNCH(expr) FH_TRY(check_launch((expr), #expr))

// y = epi(x @ W + b) (+ res) for registry matrix `slot`: split-K GEMV for up to
// 4 rows, the MFMA GEMM on the transposed copy above that.
template <typename WT>
int linear(fh_session* s, const float* x, int M, int K, size_t slot, int N, const float* b, int epi, const float* res,
           float* y) {
  hipStream_t st = s->ctx->stream;
  if (M <= 4) {
    int S = 0;
    int splits = std::max(1, std::min(64, K / 16));
    LAUNCH(launch_gemv_splitk<WT>(st, x, M, K, s->w<WT>(slot), N, s->part, splits, &S));
    LAUNCH(launch_splitk_epilogue(st, s->part, S, M, N, b, epi, res, y));
  } else if (K % 32 == 0) {
    LAUNCH(launch_gemm_mfma<WT>(st, x, M, K, s->wt<WT>(slot), N, b, epi, res, y, s->part, s->part_floats,
                                s->ctx->props.multiProcessorCount));
  } else {  // tiny models (K not a multiple of 32): the plain tiled GEMM
    LAUNCH(launch_gemm<WT>(st, x, M, K, s->w<WT>(slot), N, b, epi, res, y));
  }
  return FH_OK;
}

// x @ W for registry matrix `slot` into split-K partials s->part (no bias or
// epilogue); *S receives the split count for the fused epilogue that sums them.
template <typename WT>
int linear_parts(fh_session* s, const float* x, int M, int K, size_t slot, int N, int* S) {
  hipStream_t st = s->ctx->stream;
  if (M <= 4) {
    const int splits = std::max(1, std::min(64, K / 16));
    LAUNCH(launch_gemv_splitk<WT>(st, x, M, K, s->w<WT>(slot), N, s->part, splits, S));
  } else {
    LAUNCH(launch_gemm_mfma_split<WT>(st, x, M, K, s->wt<WT>(slot), N, s->part, s->part_floats,
                                      s->ctx->props.multiProcessorCount, S));
  }
  return FH_OK;
}

// Whether a decode step folds the split-K reductions into the kernels after them
// (qkv + KV store, proj + LN2, mproj + the next LayerNorm, LN_f included).
bool decode_fused_epilogues(const fh_session* s) {
  const int D = s->d.d_model;
  return D <= 1024 && (s->B() <= 4 || D % 32 == 0);
}

// Tied head for B rows: logits = xn @ tok_emb^T.  tok_emb [V][d] is already
// the transposed operand the MFMA GEMM reads, so more than 4 rows go there.
template <typename WT>
int head(fh_session* s, int B) {
  hipStream_t st = s->ctx->stream;
  const int D = s->d.d_model, V = s->d.vocab_size;
  if (B > 4 && D % 32 == 0) {
    LAUNCH(launch_gemm_mfma<WT>(st, s->xn, B, D, s->w<WT>(s->idx_tok()), V, nullptr, EPI_NONE, nullptr, s->logits,
                                s->part, s->part_floats, s->ctx->props.multiProcessorCount));
  } else {
    LAUNCH(launch_head<WT>(st, s->xn, B, D, s->w<WT>(s->idx_tok()), V, s->logits));
  }
  return FH_OK;
}

// Where the layers leave the last window row of each sequence (the head's input):
// row r0 + b * stride of x; x == nullptr: LN_f of those rows is already in xn.
struct LastRows {
  const float* x;
  int stride, r0;
};

// After a window forward only the K/V caches and the last row of each sequence
// are read (GptModel.ForwardLast takes the last row of the full forward,
// src/LLM.Core/Models/GptModel.cs:202-209), so the last layer stops after its qkv
// projection and KV store (which fill the caches for every row) and runs the rest
// on the B last rows only, as a batched decode step does: the attention of the
// query at window position T - 1 over keys 0 .. T - 1, attn.proj, LN2, mlp.fc and
// mlp.proj.  The attention, attn.proj, LN2 and MLP of the other B (T - 1) rows
// (9 d^2 + 2 d t FLOP per row) are work whose result nothing reads.
// FORGE_HIP_LAST_LAYER_TAIL=0 at session creation runs the layer on every row.
bool last_rows_tail(const fh_session* s, int T) { return s->last_tail && T >= 3; }

// q: layer l's q rows (row r at q + r * q_ld); x: the layer's input rows.  Uses h
// (M * 4D floats, free once the last qkv projection ran) for the B-row operands:
// q [B][3D] (q columns only, the attention's qkv layout), x, x2, GELU [B][4D], y.
template <typename WT, typename QT>
int enqueue_last_rows(fh_session* s, int T, RowSrc src, int l, const QT* q, int q_ld, LastRows* last) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model, H = s->d.n_heads, C = s->d.context_length;
  const size_t BD = (size_t)B * D;
  WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
  WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
  float* q1 = s->h;
  float* x1 = q1 + 3 * BD;
  float* x21 = x1 + BD;
  float* f1 = x21 + BD;
  float* y1 = f1 + 4 * BD;
  LAUNCH(launch_gather_rows<QT>(st, q, q_ld, T - 1, T, B, D, q1, 3 * D));
  LAUNCH(launch_gather_rows<float>(st, s->x, D, T - 1, T, B, D, x1, D));
  const RowSrc qsrc{src.tokens, src.step, src.tok_stride, src.tok_off + T - 1, T - 1, 0};
  if (D == 64 * H)
    LAUNCH(launch_attn_decode_wide<WT>(st, qsrc, q1, B, D, H, C, kc, vc, s->apart, s->o));
  else
    LAUNCH(launch_attn_decode<WT>(st, qsrc, q1, B, D, H, C, kc, vc, s->apart, 64, s->o));
  if (decode_fused_epilogues(s)) {
    // as in batched decode: the split-K sums of attn.proj and mlp.proj fused with
    // the LayerNorm after them (LN2, LN_f), so xn holds the head's input on return
    int S = 0;
    const size_t lf = s->idx_lnf();
    FH_TRY(linear_parts<WT>(s, s->o, B, D, s->idx_blk(l, 4), D, &S));
    LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 5)), x1, x21, s->v(s->idx_blk(l, 6)),
                              s->v(s->idx_blk(l, 7)), s->xn, 1e-5f));
    FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr, f1));
    FH_TRY(linear_parts<WT>(s, f1, B, 4 * D, s->idx_blk(l, 10), D, &S));
    LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 11)), x21, y1, s->v(lf), s->v(lf + 1), s->xn,
                              1e-5f));
    *last = LastRows{nullptr, 0, 0};
    return FH_OK;
  }
  FH_TRY(linear<WT>(s, s->o, B, D, s->idx_blk(l, 4), D, s->v(s->idx_blk(l, 5)), EPI_NONE, x1, x21));
  LAUNCH(launch_layernorm(st, x21, B, B, 0, 0, s->v(s->idx_blk(l, 6)), s->v(s->idx_blk(l, 7)), s->xn, D, 1e-5f));
  FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr, f1));
  FH_TRY(linear<WT>(s, f1, B, 4 * D, s->idx_blk(l, 10), D, s->v(s->idx_blk(l, 11)), EPI_RESIDUAL, x21, y1));
  *last = LastRows{y1, 1, 0};
  return FH_OK;
}

// bf16 sessions over many rows: the GEMM operands (LayerNorm, attention and GELU
// outputs) are written in bf16, rounded as the fp32-operand GEMM rounds them, into
// the same buffers (xn, o, h hold M*D, M*D, M*4D floats, twice the bf16 bytes).
// The QKV GEMM writes q in bf16 (as the attention kernel rounds it) and K, V
// straight into the bf16 caches.  The last layer ends on the last rows
// (enqueue_last_rows).
int enqueue_layers_window_bf16(fh_session* s, int T, RowSrc src, LastRows* last) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model, H = s->d.n_heads, C = s->d.context_length, M = B * T, L = s->d.n_layers;
  bf16_t* xnh = reinterpret_cast<bf16_t*>(s->xn);
  bf16_t* oh = reinterpret_cast<bf16_t*>(s->o);
  bf16_t* hh = reinterpret_cast<bf16_t*>(s->h);
  bf16_t* qh = reinterpret_cast<bf16_t*>(s->qkv);  // q [M][D] in bf16 (the fp32 qkv rows are not written)
  const bool tail = last_rows_tail(s, T);
  for (int l = 0; l < L; l++) {
    bf16_t* kc = reinterpret_cast<bf16_t*>(s->kc) + (size_t)l * s->kv_layer;
    bf16_t* vc = reinterpret_cast<bf16_t*>(s->vc) + (size_t)l * s->kv_layer;
    LAUNCH(launch_layernorm_bf16(st, s->x, M, s->v(s->idx_blk(l, 0)), s->v(s->idx_blk(l, 1)), xnh, D, 1e-5f));
    LAUNCH(launch_gemm_bf16_qkv(st, xnh, M, D, s->wt<bf16_t>(s->idx_blk(l, 2)), s->v(s->idx_blk(l, 3)), src, T, H, C,
                                qh, kc, vc));
    if (tail && l + 1 == L) return enqueue_last_rows<bf16_t, bf16_t>(s, T, src, l, qh, D, last);
    LAUNCH(launch_attn_prefill_mfma_q16(st, qh, B, T, D, H, C, kc, vc, oh));
    LAUNCH(launch_gemm_bf16(st, oh, M, D, s->wt<bf16_t>(s->idx_blk(l, 4)), D, s->v(s->idx_blk(l, 5)), EPI_NONE, s->x,
                            s->x2, nullptr));
    LAUNCH(launch_layernorm_bf16(st, s->x2, M, s->v(s->idx_blk(l, 6)), s->v(s->idx_blk(l, 7)), xnh, D, 1e-5f));
    LAUNCH(launch_gemm_bf16(st, xnh, M, D, s->wt<bf16_t>(s->idx_blk(l, 8)), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU,
                            nullptr, nullptr, hh));
    // mlp.proj: o (the attention output, consumed by attn.proj) holds the sums of
    // the first K halves when the product is split
    LAUNCH(launch_gemm_bf16_split(st, hh, M, 4 * D, s->wt<bf16_t>(s->idx_blk(l, 10)), D, s->v(s->idx_blk(l, 11)),
                                  s->x2, s->x, s->o, (size_t)B * C * D, s->gsplit, s->gsplit_cap));
  }
  return FH_OK;
}

template <typename WT>
int enqueue_layers_window(fh_session* s, int T, RowSrc src, LastRows* last) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model, H = s->d.n_heads, C = s->d.context_length, M = B * T;
  *last = LastRows{s->x, T, T - 1};
  if constexpr (sizeof(WT) == 2) {
    if (s->bf16_act && M >= 256 && D % 64 == 0 && D == 64 * H)
      return enqueue_layers_window_bf16(s, T, src, last);
  }
  if (M > 4 && D % 32 == 0 && D <= 1024 && (size_t)M * 3 * D <= s->part_floats) {
    // short windows: the split-K reductions also store K/V and apply LN2 and the
    // next layer's LN1, as in batched decode (the last mlp.proj keeps its residual
    // epilogue: LN_f runs on the last rows only)
    const int L = s->d.n_layers;
    const bool tail = last_rows_tail(s, T);
    LAUNCH(launch_layernorm(st, s->x, M, M, 0, 0, s->v(s->idx_blk(0, 0)), s->v(s->idx_blk(0, 1)), s->xn, D, 1e-5f));
    for (int l = 0; l < L; l++) {
      WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
      WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
      int S = 0;
      FH_TRY(linear_parts<WT>(s, s->xn, M, D, s->idx_blk(l, 2), 3 * D, &S));
      LAUNCH(launch_epilogue_qkv<WT>(st, s->part, S, M, D, s->v(s->idx_blk(l, 3)), s->qkv, src, T, H, C, kc, vc));
      if (tail && l + 1 == L) return enqueue_last_rows<WT, float>(s, T, src, l, s->qkv, 3 * D, last);
      if (D == 64 * H)
        LAUNCH((launch_attn_prefill_mfma<WT, float>(st, s->qkv, B, T, D, H, C, kc, vc, s->o)));
      else
        LAUNCH(launch_attn_prefill<WT>(st, s->qkv, B, T, D, H, C, kc, vc, s->o));
      FH_TRY(linear_parts<WT>(s, s->o, M, D, s->idx_blk(l, 4), D, &S));
      LAUNCH(launch_epilogue_ln(st, s->part, S, M, D, s->v(s->idx_blk(l, 5)), s->x, s->x2, s->v(s->idx_blk(l, 6)),
                                s->v(s->idx_blk(l, 7)), s->xn, 1e-5f));
      FH_TRY(linear<WT>(s, s->xn, M, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr,
                        s->h));
      if (l + 1 < L) {
        FH_TRY(linear_parts<WT>(s, s->h, M, 4 * D, s->idx_blk(l, 10), D, &S));
        LAUNCH(launch_epilogue_ln(st, s->part, S, M, D, s->v(s->idx_blk(l, 11)), s->x2, s->x,
                                  s->v(s->idx_blk(l + 1, 0)), s->v(s->idx_blk(l + 1, 1)), s->xn, 1e-5f));
      } else {
        FH_TRY(linear<WT>(s, s->h, M, 4 * D, s->idx_blk(l, 10), D, s->v(s->idx_blk(l, 11)), EPI_RESIDUAL, s->x2,
                          s->x));
      }
    }
    return FH_OK;
  }
  const bool tail = last_rows_tail(s, T);
  for (int l = 0; l < s->d.n_layers; l++) {
    WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
    WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
    LAUNCH(launch_layernorm(st, s->x, M, M, 0, 0, s->v(s->idx_blk(l, 0)), s->v(s->idx_blk(l, 1)), s->xn, D, 1e-5f));
    FH_TRY(linear<WT>(s, s->xn, M, D, s->idx_blk(l, 2), 3 * D, s->v(s->idx_blk(l, 3)), EPI_NONE, nullptr,
                      s->qkv));
    LAUNCH(launch_kv_store<WT>(st, src, s->qkv, B, T, D, H, C, kc, vc));
    if (tail && l + 1 == s->d.n_layers) return enqueue_last_rows<WT, float>(s, T, src, l, s->qkv, 3 * D, last);
    if (D == 64 * H)
      LAUNCH((launch_attn_prefill_mfma<WT, float>(st, s->qkv, B, T, D, H, C, kc, vc, s->o)));
    else
      LAUNCH(launch_attn_prefill<WT>(st, s->qkv, B, T, D, H, C, kc, vc, s->o));
    FH_TRY(linear<WT>(s, s->o, M, D, s->idx_blk(l, 4), D, s->v(s->idx_blk(l, 5)), EPI_NONE, s->x, s->x2));
    LAUNCH(launch_layernorm(st, s->x2, M, M, 0, 0, s->v(s->idx_blk(l, 6)), s->v(s->idx_blk(l, 7)), s->xn, D, 1e-5f));
    FH_TRY(linear<WT>(s, s->xn, M, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr,
                      s->h));
    FH_TRY(linear<WT>(s, s->h, M, 4 * D, s->idx_blk(l, 10), D, s->v(s->idx_blk(l, 11)), EPI_RESIDUAL, s->x2,
                      s->x));
  }
  return FH_OK;
}

template <typename WT>
int enqueue_layers_decode(fh_session* s, RowSrc src) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model, H = s->d.n_heads, C = s->d.context_length;
  if (decode_fused_epilogues(s)) {
    // each split-K reduction also does the work of the kernel after it; the last
    // mproj reduction applies LN_f, so xn holds the head's input on return
    const int L = s->d.n_layers;
    s->route |= FH_ROUTE_FUSED_EPILOGUES;
    LAUNCH(launch_layernorm(st, s->x, B, B, 0, 0, s->v(s->idx_blk(0, 0)), s->v(s->idx_blk(0, 1)), s->xn, D, 1e-5f));
    if (B > 4 && D == 64 * H && C <= 4 * kAttnDecodeChunk) {
      s->route |= FH_ROUTE_ATTN_IN_PROJ;
      // the qkv reduction and KV store are folded into the attention and the
      // attention combine into the attn.proj GEMM's operand load (8 launches per
      // layer); folding the mlp.fc reduction into mlp.proj's
      // operand load was measured slower (each mlp.proj block re-reads 8 partials
      // of its A chunk: 19 MB per layer)
      const int cus = s->ctx->props.multiProcessorCount;
      // fp32 batches of up to 32 rows: mlp.fc on the skinny GEMM, its bias and GELU
      // in the same launch (8.2 us against 6.1 + 4.4 for the split-K GEMM and its
      // reduction at C4).  qkv and mlp.proj stay split-K: their partials are summed by
      // kernels that run anyway (the attention, the LayerNorm epilogue), and the
      // skinny GEMM's 16-column strips re-read the 32 rows of x twice as often as
      // the split GEMM's 128-column tiles (7.9 against 6.7-7.1 us)
      const bool skinny = std::is_same<WT, float>::value && gemm_skinny_fits(B, D, 4 * D);
      for (int l = 0; l < L; l++) {
        WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
        WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
        int S = 0;
        LAUNCH(launch_gemm_mfma_split<WT>(st, s->xn, B, D, s->wt<WT>(s->idx_blk(l, 2)), 3 * D, s->part,
                                          s->part_floats, cus, &S));
        // the attention sums the qkv partials itself and stores the new K/V rows
        const QkvParts qp{s->part, S, B, s->v(s->idx_blk(l, 3))};
        LAUNCH(launch_attn_decode_wide<WT>(st, src, nullptr, B, D, H, C, kc, vc, s->apart, s->o, false, &qp));
        AOperand ao{};
        ao.kind = AOP_ATTN;
        ao.apart = s->apart;
        ao.src = src;
        ao.H = H;
        ao.ctx = C;
        ao.chunk = kAttnDecodeChunk;
        ao.maxc = (C + kAttnDecodeChunk - 1) / kAttnDecodeChunk;
        LAUNCH(launch_gemm_mfma_split<WT>(st, s->apart, B, D, s->wt<WT>(s->idx_blk(l, 4)), D, s->part,
                                          s->part_floats, cus, &S, &ao));
        LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 5)), s->x, s->x2, s->v(s->idx_blk(l, 6)),
                                  s->v(s->idx_blk(l, 7)), s->xn, 1e-5f));
        if (skinny)
          LAUNCH(launch_gemm_skinny(st, s->xn, B, D, reinterpret_cast<const float*>(s->wt<WT>(s->idx_blk(l, 8))),
                                    4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, s->h, nullptr));
        else
          FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr,
                            s->h));
        LAUNCH(launch_gemm_mfma_split<WT>(st, s->h, B, 4 * D, s->wt<WT>(s->idx_blk(l, 10)), D, s->part,
                                          s->part_floats, cus, &S));
        const size_t ln = l + 1 < L ? s->idx_blk(l + 1, 0) : s->idx_lnf();
        LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 11)), s->x2, s->x, s->v(ln),
                                  s->v(ln + 1), s->xn, 1e-5f));
      }
      return FH_OK;
    }
    for (int l = 0; l < L; l++) {
      WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
      WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
      int S = 0;
      FH_TRY(linear_parts<WT>(s, s->xn, B, D, s->idx_blk(l, 2), 3 * D, &S));
      LAUNCH(launch_epilogue_qkv<WT>(st, s->part, S, B, D, s->v(s->idx_blk(l, 3)), s->qkv, src, 1, H, C, kc, vc));
      if (D == 64 * H)
        LAUNCH(launch_attn_decode_wide<WT>(st, src, s->qkv, B, D, H, C, kc, vc, s->apart, s->o));
      else
        LAUNCH(launch_attn_decode<WT>(st, src, s->qkv, B, D, H, C, kc, vc, s->apart, 64, s->o));
      FH_TRY(linear_parts<WT>(s, s->o, B, D, s->idx_blk(l, 4), D, &S));
      LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 5)), s->x, s->x2, s->v(s->idx_blk(l, 6)),
                                s->v(s->idx_blk(l, 7)), s->xn, 1e-5f));
      FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr,
                        s->h));
      FH_TRY(linear_parts<WT>(s, s->h, B, 4 * D, s->idx_blk(l, 10), D, &S));
      const size_t ln = l + 1 < L ? s->idx_blk(l + 1, 0) : s->idx_lnf();
      LAUNCH(launch_epilogue_ln(st, s->part, S, B, D, s->v(s->idx_blk(l, 11)), s->x2, s->x, s->v(ln), s->v(ln + 1),
                                s->xn, 1e-5f));
    }
    return FH_OK;
  }
  s->route |= FH_ROUTE_UNFUSED;
  for (int l = 0; l < s->d.n_layers; l++) {
    WT* kc = reinterpret_cast<WT*>(s->kc) + (size_t)l * s->kv_layer;
    WT* vc = reinterpret_cast<WT*>(s->vc) + (size_t)l * s->kv_layer;
    LAUNCH(launch_layernorm(st, s->x, B, B, 0, 0, s->v(s->idx_blk(l, 0)), s->v(s->idx_blk(l, 1)), s->xn, D, 1e-5f));
    FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 2), 3 * D, s->v(s->idx_blk(l, 3)), EPI_NONE, nullptr,
                      s->qkv));
    LAUNCH(launch_kv_store<WT>(st, src, s->qkv, B, 1, D, H, C, kc, vc));
    if (D == 64 * H)
      LAUNCH(launch_attn_decode_wide<WT>(st, src, s->qkv, B, D, H, C, kc, vc, s->apart, s->o));
    else
      LAUNCH(launch_attn_decode<WT>(st, src, s->qkv, B, D, H, C, kc, vc, s->apart, 64, s->o));
    FH_TRY(linear<WT>(s, s->o, B, D, s->idx_blk(l, 4), D, s->v(s->idx_blk(l, 5)), EPI_NONE, s->x, s->x2));
    LAUNCH(launch_layernorm(st, s->x2, B, B, 0, 0, s->v(s->idx_blk(l, 6)), s->v(s->idx_blk(l, 7)), s->xn, D, 1e-5f));
    FH_TRY(linear<WT>(s, s->xn, B, D, s->idx_blk(l, 8), 4 * D, s->v(s->idx_blk(l, 9)), EPI_GELU, nullptr,
                      s->h));
    FH_TRY(linear<WT>(s, s->h, B, 4 * D, s->idx_blk(l, 10), D, s->v(s->idx_blk(l, 11)), EPI_RESIDUAL, s->x2,
                      s->x));
  }
  return FH_OK;
}


SampleArgs make_sample_args(fh_session* s, const StepPlan& p) {
  SampleArgs a{};
  a.logits = s->logits;
  a.work = s->work;
  a.tokens = s->tokens;
  a.step = s->step;
  a.done = s->done;
  a.out_ids = s->out_ids;
  a.out_counts = s->out_counts;
  a.uniforms = s->uniforms;
  a.dump = s->dump;
  a.B = s->B();
  a.V = s->d.vocab_size;
  a.tok_stride = p.tok_stride;
  a.prompt_len = p.P;
  a.ctx = s->d.context_length;
  a.max_new = p.max_new;
  a.temperature = p.opts->temperature;
  a.penalty = p.opts->repetition_penalty;
  a.top_k = p.opts->top_k;
  a.ngram = p.opts->no_repeat_ngram;
  a.eos = p.opts->eos_id;
  return a;
}

// One forward over a window of T rows per sequence (prefill / re-prefill),
// then the head on the last row and (optionally) the sampler.
template <typename WT>
int enqueue_window_step(fh_session* s, int T, const StepPlan& p) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model;
  RowSrc src{s->tokens, s->step, p.tok_stride, p.P - T, 0, 0};
  LAUNCH(launch_embed<WT>(st, src, B, T, s->w<WT>(s->idx_tok()), s->w<WT>(s->idx_pos()), D, s->d.vocab_size,
                          s->d.context_length, s->x));
  LastRows last{};
  FH_TRY(enqueue_layers_window<WT>(s, T, src, &last));
  const size_t lf = s->idx_lnf();
  if (last.x)
    LAUNCH(launch_layernorm(st, last.x, B, 1, last.stride, last.r0, s->v(lf), s->v(lf + 1), s->xn, D, 1e-5f));
  FH_TRY(head<WT>(s, B));
  if (p.with_sample) LAUNCH(launch_sample(st, make_sample_args(s, p)));
  return FH_OK;
}

// The fused kernel's greedy mode: no repetition controls, no logits dump.
bool fused_greedy(const fh_session* s, const fh_sampling* o) {
  return s->use_fast() && !(o->temperature > 0.f) && o->repetition_penalty == 1.f && o->no_repeat_ngram == 0 &&
         s->dump == nullptr;
}

FastDecode::Step fused_step(fh_session* s, const StepPlan& p, int greedy, int nsteps, bool sampled = false,
                            int window_end = 0) {
  FastDecode::Step fs{};
  fs.src = RowSrc{s->tokens, s->step, p.tok_stride, p.P - 1, p.P - 1, 1};
  fs.tok_emb = s->v(s->idx_tok());
  fs.pos_emb = s->v(s->idx_pos());
  fs.kcache = reinterpret_cast<float*>(s->kc);
  fs.vcache = reinterpret_cast<float*>(s->vc);
  fs.logits = s->logits;
  fs.out_ids = s->out_ids;
  fs.out_counts = s->out_counts;
  fs.max_new = p.max_new;
  fs.eos = p.opts->eos_id;
  fs.greedy = greedy;
  fs.nsteps = nsteps;
  fs.tokens = s->tokens;
  fs.step = s->step;
  if (sampled) {
    fs.sampled = 1;
    fs.uniforms = s->uniforms;
    fs.temperature = p.opts->temperature;
    fs.penalty = p.opts->repetition_penalty;
    fs.top_k = p.opts->top_k;
    fs.ngram = p.opts->no_repeat_ngram;
    fs.window_end = window_end;
  }
  return fs;
}

// One cached decode step: the token sampled last step at position P-1+n.
template <typename WT>
int enqueue_decode_step(fh_session* s, const StepPlan& p) {
  hipStream_t st = s->ctx->stream;
  const int B = s->B(), D = s->d.d_model;
  RowSrc src{s->tokens, s->step, p.tok_stride, p.P - 1, p.P - 1, 1};
  if (s->use_fast()) {
    // greedy without repetition controls or a logits dump: the argmax runs
    // inside the decode kernel and no sampler launch follows
    const bool greedy = fused_greedy(s, p.opts);
    s->route |= FH_ROUTE_FUSED_STEP;
    int rc = s->fast.enqueue(st, fused_step(s, p, greedy ? 1 : 0, 1));
    if (rc != FH_OK) return set_err(rc, "fused decode step launch failed: %s", hipGetErrorString(hipGetLastError()));
    if (greedy) return FH_OK;
  } else {
    LAUNCH(launch_embed<WT>(st, src, B, 1, s->w<WT>(s->idx_tok()), s->w<WT>(s->idx_pos()), D, s->d.vocab_size,
                            s->d.context_length, s->x));
    FH_TRY(enqueue_layers_decode<WT>(s, src));
    const size_t lf = s->idx_lnf();
    if (!decode_fused_epilogues(s))
      LAUNCH(launch_layernorm(st, s->x, B, 1, 1, 0, s->v(lf), s->v(lf + 1), s->xn, D, 1e-5f));
    FH_TRY(head<WT>(s, B));
  }
  LAUNCH(launch_sample(st, make_sample_args(s, p)));
  return FH_OK;
}

int enqueue_window(fh_session* s, int T, const StepPlan& p) {
  return s->d.dtype == FH_DTYPE_BF16 ? enqueue_window_step<bf16_t>(s, T, p) : enqueue_window_step<float>(s, T, p);
}
int enqueue_decode(fh_session* s, const StepPlan& p) {
  return s->d.dtype == FH_DTYPE_BF16 ? enqueue_decode_step<bf16_t>(s, p) : enqueue_decode_step<float>(s, p);
}

// Captures `enqueue` into `g` unless the cached graph already matches `key`.
template <class F>
int capture(fh_session* s, CachedGraph& g, const GraphKey& key, F&& enqueue) {
  if (g.exec && g.key == key) return FH_OK;
  drop_graph(g);
  hipStream_t st = s->ctx->stream;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  s->route = 0;
  int rc = enqueue();
  g.route = s->route;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(st, &graph);
  if (rc != FH_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  if (e != hipSuccess) return set_err(FH_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) {
    g.exec = nullptr;
    return set_err(FH_ERR_HIP, "graph instantiate failed: %s", hipGetErrorString(e));
  }
  g.key = key;
  return FH_OK;
}

__global__ void k_fill_int(int* p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

int reset_step_state(fh_session* s) {
  hipStream_t st = s->ctx->stream;
  hipLaunchKernelGGL(k_fill_int, dim3(1), dim3(64), 0, st, s->step, 1, 0);
  hipLaunchKernelGGL(k_fill_int, dim3(1), dim3(64), 0, st, s->done, 1, 0);
  hipLaunchKernelGGL(k_fill_int, dim3((s->B() + 255) / 256), dim3(256), 0, st, s->out_counts, s->B(), -1);
  HIP_TRY(hipGetLastError());
  return FH_OK;
}

int upload_weights(fh_session* s, const float* const* tensors) {
  // Matrices go to the session dtype; vectors stay fp32 (rounded through bf16
  // in bf16 sessions so every parameter carries bf16 precision).
  const bool bf = s->d.dtype == FH_DTYPE_BF16;
  std::vector<char> host;
  for (size_t i = 0; i < s->reg.size(); i++) {
    const Slot& sl = s->reg[i];
    const float* src = tensors[i];
    if (!src) return set_err(FH_ERR_INVALID, "tensor %zu (%s) is null", i, sl.name.c_str());
    size_t bytes;
    const void* p;
    if (bf && sl.matrix) {
      host.resize(sl.numel * 2);
      bf16_t* h = reinterpret_cast<bf16_t*>(host.data());
      for (int64_t j = 0; j < sl.numel; j++) h[j] = f32_to_bf16(src[j]);
      bytes = sl.numel * 2;
      p = host.data();
    } else if (bf) {
      host.resize(sl.numel * 4);
      float* h = reinterpret_cast<float*>(host.data());
      for (int64_t j = 0; j < sl.numel; j++) h[j] = bf16_to_f32(f32_to_bf16(src[j]));
      bytes = sl.numel * 4;
      p = host.data();
    } else {
      bytes = sl.numel * 4;
      p = src;
    }
    HIP_TRY(hipMemcpy(s->wbuf + s->off[i], p, bytes, hipMemcpyHostToDevice));
  }
  // [K][N] -> [N][K] copies of every block matrix for the MFMA GEMM
  {
    const int64_t D = s->d.d_model;
    for (int l = 0; l < s->d.n_layers; l++)
      for (int k : {2, 4, 8, 10}) {
        const size_t i = s->idx_blk(l, k);
        const int K = (int)(k == 10 ? 4 * D : D);
        const int N = (int)(s->reg[i].numel / K);
        hipError_t e = bf ? launch_transpose<bf16_t>(s->ctx->stream, s->w<bf16_t>(i), K, N,
                                                     reinterpret_cast<bf16_t*>(s->wtbuf + s->wtoff[i]))
                          : launch_transpose<float>(s->ctx->stream, s->w<float>(i), K, N,
                                                    reinterpret_cast<float*>(s->wtbuf + s->wtoff[i]));
        HIP_TRY(e);
      }
    HIP_TRY(hipStreamSynchronize(s->ctx->stream));
  }
  s->loaded = true;
  drop_graph(s->g_decode);
  drop_graph(s->g_reprefill);
  if (!s->fast.enabled) return FH_OK;
  std::vector<const float*> ptrs;
  for (size_t i = 0; i < s->reg.size(); i++) ptrs.push_back(s->v(i));
  const int rc = s->fast.build(s->ctx->stream, ptrs.data());
  if (rc != FH_OK) return set_err(rc, "building the fused decode tiles failed");
  return FH_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int fh_last_error(char* buf, size_t n) {
  if (!buf || n == 0) return FH_ERR_INVALID;
  snprintf(buf, n, "%s", g_err.c_str());
  return FH_OK;
}

const char* fh_version(void) { return "forge_hip 0.1 gfx950"; }

int fh_random_doubles(int32_t seed, int n, double* out) {
  if (n < 0 || (n > 0 && !out)) return set_err(FH_ERR_INVALID, "bad output buffer");
  random_doubles(seed, n, out);
  return FH_OK;
}

static int scratch_init(int device);

int fh_context_create(int device, fh_context** out) {
  if (!out) return set_err(FH_ERR_INVALID, "out is null");
  *out = nullptr;
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return set_err(FH_ERR_RANGE, "device %d not present (%d devices)", device, n);
  auto c = std::make_unique<fh_context>();
  c->device = device;
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(hipGetDeviceProperties(&c->props, device));
  FH_TRY(scratch_init(device));  // the no-allocation sampler's scratch address on this device
  HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  *out = c.release();
  return FH_OK;
}

static void context_free(fh_context* c) {
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  dev_free(c->s_work);
  dev_free(c->s_ints);
  dev_free(c->s_u);
  ops_state_free(c->ops);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

// Sessions keep their context alive: destroying a context that still has
// sessions defers the release to the last fh_session_destroy.
int fh_context_destroy(fh_context* c) {
  if (!c) return FH_OK;
  if (c->sessions > 0) {
    c->destroy_pending = true;
    return FH_OK;
  }
  context_free(c);
  return FH_OK;
}

int fh_context_info(fh_context* c, char* name, size_t name_len, uint64_t* total_mem, int32_t* cus) {
  if (!c) return set_err(FH_ERR_INVALID, "context is null");
  if (name && name_len) {
    if (c->props.name[0])
      snprintf(name, name_len, "%s (%s)", c->props.name, c->props.gcnArchName);
    else
      snprintf(name, name_len, "%s", c->props.gcnArchName);
  }
  if (total_mem) *total_mem = c->props.totalGlobalMem;
  if (cus) *cus = c->props.multiProcessorCount;
  return FH_OK;
}

int fh_context_memory(fh_context* c, uint64_t* free_bytes, uint64_t* sampler_scratch_bytes) {
  if (!c) return set_err(FH_ERR_INVALID, "context is null");
  if (free_bytes) {
    HIP_TRY(hipSetDevice(c->device));
    size_t fr = 0, tot = 0;
    HIP_TRY(hipMemGetInfo(&fr, &tot));
    *free_bytes = fr;
  }
  if (sampler_scratch_bytes)
    *sampler_scratch_bytes = (uint64_t)(c->s_work ? (size_t)c->s_V * sizeof(float) : 0) +
                             (c->s_ints ? (size_t)c->s_hist * sizeof(int) : 0) + (c->s_u ? sizeof(double) : 0);
  return FH_OK;
}

int fh_buffer_alloc(fh_context* c, size_t bytes, void** out_dev) {
  if (!c || !out_dev) return set_err(FH_ERR_INVALID, "null argument");
  *out_dev = nullptr;
  HIP_TRY(hipSetDevice(c->device));
  char* p = nullptr;
  FH_TRY(dev_alloc(&p, bytes));
  *out_dev = p;
  return FH_OK;
}

int fh_buffer_free(fh_context* c, void* dev) {
  if (!c) return set_err(FH_ERR_INVALID, "context is null");
  if (!dev) return FH_OK;
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipStreamSynchronize(c->stream));
  HIP_TRY(hipFree(dev));
  return FH_OK;
}

int fh_buffer_write(fh_context* c, void* dst_dev, const void* src, size_t bytes) {
  if (!c || !dst_dev || (!src && bytes)) return set_err(FH_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return FH_OK;
}

int fh_buffer_read(fh_context* c, void* dst, const void* src_dev, size_t bytes) {
  if (!c || !src_dev || (!dst && bytes)) return set_err(FH_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return FH_OK;
}

int fh_buffer_copy(fh_context* c, void* dst_dev, const void* src_dev, size_t bytes, float* ms_out) {
  if (!c || !dst_dev || !src_dev) return set_err(FH_ERR_INVALID, "null argument");
  if (((uintptr_t)dst_dev | (uintptr_t)src_dev) % 16)
    return set_err(FH_ERR_INVALID, "device buffers must be 16-byte aligned");
  HIP_TRY(hipSetDevice(c->device));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (ms_out) {
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    HIP_TRY(hipEventRecord(e0, c->stream));
  }
  hipError_t e = launch_copy(c->stream, dst_dev, src_dev, bytes);
  if (e == hipSuccess && ms_out) e = hipEventRecord(e1, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess && ms_out) e = hipEventElapsedTime(ms_out, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  HIP_TRY(e);
  return FH_OK;
}

int fh_buffer_checksum(fh_context* c, const void* src_dev, size_t bytes, uint64_t* sum_out, float* ms_out) {
  if (!c || !src_dev || !sum_out) return set_err(FH_ERR_INVALID, "null argument");
  if ((uintptr_t)src_dev % 16) return set_err(FH_ERR_INVALID, "the device buffer must be 16-byte aligned");
  if (bytes % 4) return set_err(FH_ERR_INVALID, "bytes (%zu) must be a multiple of 4", bytes);
  HIP_TRY(hipSetDevice(c->device));
  // eight blocks per CU (a whole number of passes over most buffers), at most one per 4 KB
  const int nparts = (int)std::max<size_t>(1, std::min<size_t>({(size_t)kChecksumParts,
                                                                 (size_t)c->props.multiProcessorCount * 8,
                                                                 (bytes + 4095) / 4096}));
  unsigned long long* dbuf = nullptr;
  FH_TRY(dev_alloc(&dbuf, (size_t)nparts + 1));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipSuccess;
  if (ms_out) {
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventRecord(e0, c->stream);
  }
  if (e == hipSuccess) e = launch_checksum(c->stream, src_dev, bytes, dbuf + 1, nparts, dbuf, e1);
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&h, dbuf, sizeof h, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess && ms_out) e = hipEventElapsedTime(ms_out, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  dev_free(dbuf);
  HIP_TRY(e);
  *sum_out = h;
  return FH_OK;
}

int fh_matmul_nn(fh_context* c, const void* a_dev, const void* b_dev, void* y_dev, int M, int K, int N, int dtype,
                 int accumulate) {
  if (!c || !a_dev || !b_dev || !y_dev) return set_err(FH_ERR_INVALID, "null argument");
  if (M <= 0 || K <= 0 || N <= 0) return set_err(FH_ERR_INVALID, "M, K and N must be positive");
  if (dtype != FH_DTYPE_F32 && dtype != FH_DTYPE_BF16) return set_err(FH_ERR_INVALID, "unknown dtype %d", dtype);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->stream;
  const float* a = static_cast<const float*>(a_dev);
  float* y = static_cast<float*>(y_dev);
  const float* res = accumulate ? y : nullptr;  // each output element is read, then written, by one lane
  const bool bf = dtype == FH_DTYPE_BF16;
  hipError_t e = hipSuccess;
  if (K % 32 == 0) {
    // the GEMM takes the weights transposed, plus room for split-K partials (or,
    // for bf16 with many rows, for a rounded to bf16: the window path's kernel)
    const bool big = bf && M >= 256 && K % 64 == 0;
    const size_t esz = bf ? 2 : 4, part_floats = big ? 0 : (size_t)8 * M * N;
    // an accumulating bf16 product may split K in two: first halves' sums and tile counters
    const size_t ws_floats = big && res ? (size_t)M * N : 0;
    const int ncnt = big && res ? ((M + 255) / 256) * ((N + 255) / 256) : 0;
    char* tmp = nullptr;
    const size_t wbytes = (size_t)N * K * esz + (big ? (size_t)M * K * 2 : part_floats * 4);
    // the tile counters are followed by the split's error word
    HIP_TRY(hipMalloc(&tmp, (wbytes + 255) / 256 * 256 + ws_floats * 4 + (size_t)(ncnt + 1) * 4));
    float* part = reinterpret_cast<float*>(tmp + (size_t)N * K * esz);
    float* ws = reinterpret_cast<float*>(tmp + (wbytes + 255) / 256 * 256);
    int* cnt = reinterpret_cast<int*>(ws + ws_floats);
    if (big) {
      bf16_t* wt = reinterpret_cast<bf16_t*>(tmp);
      bf16_t* ah = wt + (size_t)N * K;
      e = launch_transpose<bf16_t>(st, static_cast<const bf16_t*>(b_dev), K, N, wt);
      if (e == hipSuccess) e = launch_round_bf16(st, a, (size_t)M * K, ah);
      if (e == hipSuccess && res) e = hipMemsetAsync(cnt, 0, (size_t)(ncnt + 1) * 4, st);
      if (e == hipSuccess)
        e = res ? launch_gemm_bf16_split(st, ah, M, K, wt, N, nullptr, res, y, ws, ws_floats, cnt, ncnt)
                : launch_gemm_bf16(st, ah, M, K, wt, N, nullptr, EPI_NONE, res, y, nullptr);
    } else if (bf) {
      e = launch_transpose<bf16_t>(st, static_cast<const bf16_t*>(b_dev), K, N, reinterpret_cast<bf16_t*>(tmp));
      if (e == hipSuccess)
        e = launch_gemm_mfma<bf16_t>(st, a, M, K, reinterpret_cast<const bf16_t*>(tmp), N, nullptr, EPI_NONE, res, y,
                                     part, part_floats, c->props.multiProcessorCount);
    } else {
      e = launch_transpose<float>(st, static_cast<const float*>(b_dev), K, N, reinterpret_cast<float*>(tmp));
      if (e == hipSuccess)
        e = launch_gemm_mfma<float>(st, a, M, K, reinterpret_cast<const float*>(tmp), N, nullptr, EPI_NONE, res, y,
                                    part, part_floats, c->props.multiProcessorCount);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    int split_err = 0;
    if (e == hipSuccess && big && res) e = hipMemcpy(&split_err, cnt + ncnt, sizeof(int), hipMemcpyDeviceToHost);
    (void)hipFree(tmp);
    if (e == hipSuccess && split_err)
      return set_err(FH_ERR_HIP, "split-K GEMM: a tile's two K halves did not meet (%s; y is not valid)",
                     (split_err & 1) ? "the wait for the first half exceeded its bound"
                                     : "the halves ran on different XCDs");
  } else {
    e = bf ? launch_gemm<bf16_t>(st, a, M, K, static_cast<const bf16_t*>(b_dev), N, nullptr, EPI_NONE, res, y)
           : launch_gemm<float>(st, a, M, K, static_cast<const float*>(b_dev), N, nullptr, EPI_NONE, res, y);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
  }
  HIP_TRY(e);
  return FH_OK;
}

int64_t fh_param_count(const fh_model_desc* d) {
  if (validate_desc(d) != FH_OK) return -1;
  int64_t n = 0;
  for (auto& s : make_registry(*d)) n += s.numel;
  return n;
}

int fh_param_info(const fh_model_desc* d, int index, char* name, size_t name_len, int64_t* numel) {
  FH_TRY(validate_desc(d));
  auto reg = make_registry(*d);
  if (index < 0 || index >= (int)reg.size())
    return set_err(FH_ERR_RANGE, "parameter index %d outside [0,%zu)", index, reg.size());
  if (name && name_len) snprintf(name, name_len, "%s", reg[index].name.c_str());
  if (numel) *numel = reg[index].numel;
  return (int)reg.size();
}

int fh_session_destroy(fh_session* s);

int fh_session_create(fh_context* c, const fh_model_desc* desc, fh_session** out) {
  if (!c || !out) return set_err(FH_ERR_INVALID, "null argument");
  *out = nullptr;
  FH_TRY(validate_desc(desc));
  HIP_TRY(hipSetDevice(c->device));
  auto s = std::make_unique<fh_session>();
  s->ctx = c;
  s->d = *desc;
  s->reg = make_registry(*desc);
  s->esize = desc->dtype == FH_DTYPE_BF16 ? 2 : 4;
  size_t o = 0;
  for (auto& sl : s->reg) {
    s->off.push_back(o);
    o += ((size_t)sl.numel * (sl.matrix ? s->esize : 4) + 255) / 256 * 256;
  }
  s->wbytes = o;
  // transposed copies of the blocks' matrices (tok_emb / pos_emb are not needed)
  size_t ot = 0;
  s->wtoff.assign(s->reg.size(), 0);
  for (size_t i = 2; i < s->reg.size(); i++)
    if (s->reg[i].matrix) {
      s->wtoff[i] = ot;
      ot += ((size_t)s->reg[i].numel * s->esize + 255) / 256 * 256;
    }
  const size_t wtbytes = ot;
  fh_session* sp = s.get();
  auto fail = [&](int rc) {
    fh_session_destroy(s.release());
    return rc;
  };
  int rc;
  if ((rc = dev_alloc(&sp->wbuf, sp->wbytes)) != FH_OK) return fail(rc);
  if ((rc = dev_alloc(&sp->wtbuf, wtbytes)) != FH_OK) return fail(rc);
  const int B = desc->max_batch, D = desc->d_model, C = desc->context_length, V = desc->vocab_size;
  const int H = desc->n_heads, hd = D / H;
  sp->kv_layer = (size_t)B * H * C * hd;
  const size_t kvb = sp->kv_layer * desc->n_layers * sp->esize;
  char* kc = nullptr;
  char* vc = nullptr;
  if ((rc = dev_alloc(&kc, kvb)) != FH_OK) return fail(rc);
  sp->kc = kc;
  if ((rc = dev_alloc(&vc, kvb)) != FH_OK) return fail(rc);
  sp->vc = vc;
  const size_t rows = (size_t)B * C;
  const int maxc = (C + 63) / 64;
  // split-K partials: the GEMV path (up to 64 splits of 4 rows), the MFMA GEMM's
  // small-M split (up to 8 splits of 64 rows of the widest layer), and at least
  // one unsplit product of every decode row (the batched decode's split GEMMs need
  // B x 3D; the split count shrinks to what fits)
  sp->part_floats = std::max({(size_t)64 * 4 * 4 * D, (size_t)8 * 64 * 4 * D, (size_t)B * 4 * D});
  if ((rc = dev_alloc(&sp->x, rows * D)) || (rc = dev_alloc(&sp->x2, rows * D)) || (rc = dev_alloc(&sp->xn, rows * D)) ||
      (rc = dev_alloc(&sp->qkv, rows * 3 * D)) || (rc = dev_alloc(&sp->o, rows * D)) ||
      (rc = dev_alloc(&sp->h, rows * 4 * D)) || (rc = dev_alloc(&sp->part, sp->part_floats)) ||
      (rc = dev_alloc(&sp->apart, (size_t)B * H * maxc * (hd + 2))) || (rc = dev_alloc(&sp->logits, (size_t)B * V)) ||
      (rc = dev_alloc(&sp->work, (size_t)B * V)) || (rc = dev_alloc(&sp->step, 1)) || (rc = dev_alloc(&sp->done, 1)) ||
      (rc = dev_alloc(&sp->out_counts, B)))
    return fail(rc);
  if (sp->esize == 2) {
    // one counter per tile, then the split's error word
    sp->gsplit_cap = (int)((rows + 255) / 256) * ((D + 255) / 256);
    if ((rc = dev_alloc(&sp->gsplit, sp->gsplit_cap + 1)) != FH_OK) return fail(rc);
    const hipError_t he = hipMemset(sp->gsplit, 0, (size_t)(sp->gsplit_cap + 1) * sizeof(int));
    if (he != hipSuccess) return fail(set_err(FH_ERR_HIP, "hipMemset: %s", hipGetErrorString(he)));
  }
  for (auto& e : sp->ev) {
    hipError_t he = hipEventCreate(&e);
    if (he != hipSuccess) return fail(set_err(FH_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(he)));
  }
  const char* fused_env = getenv("FORGE_HIP_FUSED_DECODE");
  sp->fast_allowed = !(fused_env && fused_env[0] == '0');
  const char* act_env = getenv("FORGE_HIP_BF16_ACT");
  sp->bf16_act = !(act_env && act_env[0] == '0');
  const char* tail_env = getenv("FORGE_HIP_LAST_LAYER_TAIL");
  sp->last_tail = !(tail_env && tail_env[0] == '0');
  if (sp->fast_allowed && (rc = sp->fast.init(*desc, c->props.multiProcessorCount)) != FH_OK)
    return fail(set_err(rc, "allocating the fused decode state failed"));
  c->sessions++;
  sp->counted = true;
  *out = s.release();
  return FH_OK;
}

int fh_session_destroy(fh_session* s) {
  if (!s) return FH_OK;
  (void)hipSetDevice(s->ctx->device);
  (void)hipStreamSynchronize(s->ctx->stream);
  drop_graph(s->g_decode);
  drop_graph(s->g_reprefill);
  s->fast.release();
  for (auto& e : s->ev)
    if (e) (void)hipEventDestroy(e);
  dev_free(s->wbuf);
  dev_free(s->wtbuf);
  char* kc = static_cast<char*>(s->kc);
  char* vc = static_cast<char*>(s->vc);
  dev_free(kc);
  dev_free(vc);
  dev_free(s->x); dev_free(s->x2); dev_free(s->xn); dev_free(s->qkv); dev_free(s->o); dev_free(s->h);
  dev_free(s->part); dev_free(s->apart); dev_free(s->logits); dev_free(s->work);
  dev_free(s->step); dev_free(s->done); dev_free(s->out_counts); dev_free(s->gsplit);
  if (s->hstage) (void)hipHostFree(s->hstage);
  s->hstage = nullptr;
  dev_free(s->tokens); dev_free(s->out_ids); dev_free(s->uniforms); dev_free(s->dump);
  fh_context* c = s->ctx;
  const bool counted = s->counted;
  delete s;
  if (counted && --c->sessions == 0 && c->destroy_pending) context_free(c);
  return FH_OK;
}

int fh_init_weights(const fh_model_desc* desc, int32_t seed, float* out, int64_t n) {
  FH_TRY(validate_desc(desc));
  if (!out) return set_err(FH_ERR_INVALID, "null output");
  auto reg = make_registry(*desc);
  std::vector<int64_t> offs, sizes;
  std::vector<int> kinds;
  int64_t tot = 0;
  for (auto& sl : reg) {
    offs.push_back(tot);
    sizes.push_back(sl.numel);
    kinds.push_back(sl.init_kind);
    tot += sl.numel;
  }
  if (n != tot) return set_err(FH_ERR_INVALID, "the registry holds %lld floats, not %lld", (long long)tot, (long long)n);
  init_registry_random(seed, desc->n_layers, offs, sizes, kinds, out);
  return FH_OK;
}

int fh_session_init_random(fh_session* s, int32_t seed) {
  if (!s) return set_err(FH_ERR_INVALID, "session is null");
  std::vector<int64_t> offs, sizes;
  std::vector<int> kinds;
  int64_t tot = 0;
  for (auto& sl : s->reg) {
    offs.push_back(tot);
    sizes.push_back(sl.numel);
    kinds.push_back(sl.init_kind);
    tot += sl.numel;
  }
  std::vector<float> w((size_t)tot);
  init_registry_random(seed, s->d.n_layers, offs, sizes, kinds, w.data());
  std::vector<const float*> ptrs;
  for (auto o : offs) ptrs.push_back(w.data() + o);
  HIP_TRY(hipSetDevice(s->ctx->device));
  return upload_weights(s, ptrs.data());
}

// ---------------------------------------------------------------------------
// FORGEMODEL1 checkpoints (Checkpoint.Load, src/LLM.Core/Checkpoint/Checkpoint.cs:116-250)
// ---------------------------------------------------------------------------
extern "C++" {
namespace {

// the registry a checkpoint's header describes (ModelConfig's checks first)
std::string ckpt_registry(const CkptHeader& h, std::vector<std::string>* names, int64_t* nparams) {
  fh_model_desc d{h.vocab, h.ctx, h.d, h.layers, h.heads, 1, FH_DTYPE_F32, 0};
  if (d.vocab_size <= 0) return "VocabSize must be positive.";
  if (d.context_length <= 0) return "ContextLength must be positive.";
  if (d.d_model <= 0) return "DModel must be positive.";
  if (d.n_layers <= 0) return "NLayers must be positive.";
  if (d.n_heads <= 0) return "NHeads must be positive.";
  if (d.d_model % d.n_heads != 0)
    return "DModel (" + std::to_string(d.d_model) + ") must be divisible by NHeads (" + std::to_string(d.n_heads) +
           ").";
  *nparams = 0;
  for (auto& sl : make_registry(d)) {
    names->push_back(sl.name);
    *nparams += sl.numel;
  }
  return "";
}

}  // namespace
}  // extern "C++"

int fh_checkpoint_info(const char* path, fh_model_desc* desc, char* name, size_t name_len, int verify) {
  if (!path || !desc) return set_err(FH_ERR_INVALID, "null argument");
  CkptHeader h;
  bool data_error = true;
  const std::string e = read_checkpoint(path, &h, ckpt_registry, nullptr, verify == 0, &data_error);
  if (!e.empty()) return set_err(data_error ? FH_ERR_DATA : FH_ERR_INVALID, "%s", e.c_str());
  desc->vocab_size = h.vocab;
  desc->context_length = h.ctx;
  desc->d_model = h.d;
  desc->n_layers = h.layers;
  desc->n_heads = h.heads;
  if (name && name_len) snprintf(name, name_len, "%s", h.name.c_str());
  return FH_OK;
}

int fh_session_load_checkpoint(fh_session* s, const char* path) {
  if (!s || !path) return set_err(FH_ERR_INVALID, "null argument");
  CkptHeader h;
  bool data_error = true;
  std::vector<float> w;
  const std::string e = read_checkpoint(path, &h, ckpt_registry, &w, false, &data_error);
  if (!e.empty()) return set_err(data_error ? FH_ERR_DATA : FH_ERR_INVALID, "%s", e.c_str());
  const fh_model_desc& d = s->d;
  if (h.vocab != d.vocab_size || h.ctx != d.context_length || h.d != d.d_model || h.layers != d.n_layers ||
      h.heads != d.n_heads)
    return set_err(FH_ERR_INVALID,
                   "checkpoint model (V %d, ctx %d, d %d, L %d, H %d) does not match the session's "
                   "(V %d, ctx %d, d %d, L %d, H %d)",
                   h.vocab, h.ctx, h.d, h.layers, h.heads, d.vocab_size, d.context_length, d.d_model, d.n_layers,
                   d.n_heads);
  std::vector<const float*> ptrs;
  int64_t off = 0;
  for (auto& sl : s->reg) {
    ptrs.push_back(w.data() + off);
    off += sl.numel;
  }
  HIP_TRY(hipSetDevice(s->ctx->device));
  return upload_weights(s, ptrs.data());
}

int fh_sha256(const void* data, size_t n, uint8_t* out32) {
  if ((!data && n) || !out32) return set_err(FH_ERR_INVALID, "null argument");
  sha256(data, n, out32);
  return FH_OK;
}

int fh_session_load_weights(fh_session* s, const float* const* tensors, int n) {
  if (!s || !tensors) return set_err(FH_ERR_INVALID, "null argument");
  if (n != (int)s->reg.size())
    return set_err(FH_ERR_INVALID, "expected %zu registry tensors, got %d", s->reg.size(), n);
  HIP_TRY(hipSetDevice(s->ctx->device));
  return upload_weights(s, tensors);
}

int fh_session_read_param(fh_session* s, int index, float* out, int64_t numel) {
  if (!s || !out) return set_err(FH_ERR_INVALID, "null argument");
  if (index < 0 || index >= (int)s->reg.size()) return set_err(FH_ERR_RANGE, "parameter index %d out of range", index);
  const Slot& sl = s->reg[index];
  if (numel != sl.numel) return set_err(FH_ERR_INVALID, "%s has %lld elements, not %lld", sl.name.c_str(),
                                        (long long)sl.numel, (long long)numel);
  HIP_TRY(hipSetDevice(s->ctx->device));
  HIP_TRY(hipStreamSynchronize(s->ctx->stream));
  if (sl.matrix && s->esize == 2) {
    std::vector<bf16_t> h(sl.numel);
    HIP_TRY(hipMemcpy(h.data(), s->wbuf + s->off[index], sl.numel * 2, hipMemcpyDeviceToHost));
    for (int64_t j = 0; j < sl.numel; j++) out[j] = bf16_to_f32(h[j]);
  } else {
    HIP_TRY(hipMemcpy(out, s->wbuf + s->off[index], sl.numel * 4, hipMemcpyDeviceToHost));
  }
  return FH_OK;
}

static int validate_ids(const fh_session* s, const int32_t* ids, size_t n) {
  for (size_t i = 0; i < n; i++)
    if ((uint32_t)ids[i] >= (uint32_t)s->d.vocab_size)
      return set_err(FH_ERR_INVALID, "Token id %d out of range [0,%d).", ids[i], s->d.vocab_size);
  return FH_OK;
}

// After the stream has finished: the error word of the bf16 window path's split-K
// GEMM (mlp.proj), cleared for the next call.  Non-zero means a tile's two halves
// did not meet and its output is NaN.
static int check_split_error(fh_session* s) {
  if (!s->gsplit) return FH_OK;
  int word = 0;
  HIP_TRY(hipMemcpy(&word, s->gsplit + s->gsplit_cap, sizeof(int), hipMemcpyDeviceToHost));
  if (word == 0) return FH_OK;
  const int zero = 0;
  HIP_TRY(hipMemcpy(s->gsplit + s->gsplit_cap, &zero, sizeof(int), hipMemcpyHostToDevice));
  return set_err(FH_ERR_HIP, "split-K GEMM: a tile's two K halves did not meet (%s; results discarded)",
                 (word & 1) ? "the wait for the first half exceeded its bound" : "the halves ran on different XCDs");
}

int fh_forward_last(fh_session* s, const int32_t* ids, int batch, int T, float* logits_out) {
  if (!s || !ids || !logits_out) return set_err(FH_ERR_INVALID, "null argument");
  if (!s->loaded) return set_err(FH_ERR_STATE, "weights are not loaded");
  if (batch != s->B()) return set_err(FH_ERR_INVALID, "batch %d must equal the session's max_batch %d", batch, s->B());
  if (T <= 0) return set_err(FH_ERR_INVALID, "Need at least one token.");
  if (T > s->d.context_length)
    return set_err(FH_ERR_INVALID, "Sequence length %d exceeds ContextLength %d.", T, s->d.context_length);
  FH_TRY(validate_ids(s, ids, (size_t)batch * T));
  HIP_TRY(hipSetDevice(s->ctx->device));
  hipStream_t st = s->ctx->stream;
  FH_TRY(ensure(&s->tokens, &s->tokens_cap, (size_t)batch * T, &s->buf_gen));
  HIP_TRY(hipMemcpyAsync(s->tokens, ids, sizeof(int32_t) * batch * T, hipMemcpyHostToDevice, st));
  s->gen.active = false;  // the forward reuses the token buffer and step state of a generation
  FH_TRY(reset_step_state(s));
  fh_sampling greedy{0.f, 0, 1.f, 0, -1, 0};
  StepPlan p;
  p.P = T;
  p.max_new = 1;
  p.tok_stride = T;
  p.opts = &greedy;
  p.with_sample = false;
  FH_TRY(enqueue_window(s, T, p));
  HIP_TRY(hipMemcpyAsync(logits_out, s->logits, sizeof(float) * batch * s->d.vocab_size, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return check_split_error(s);
}

// Captures the per-step graphs the generation in s->gen needs (the decode step
// unless the persistent kernel runs the cached steps, and the re-prefill once the
// window slides) and sets the session's route.
static int gen_capture(fh_session* s) {
  GenState& g = s->gen;
  const int C = s->d.context_length;
  const fh_sampling* opts = &g.opts;
  // dump/uniform pointers are baked into the graphs
  float* saved_dump = s->dump;
  double* saved_u = s->uniforms;
  if (!g.dump) s->dump = nullptr;
  if (!g.sampled) s->uniforms = nullptr;
  GraphKey key;
  key.B = g.B;
  key.P = g.P;
  key.max_new = g.max_new;
  key.top_k = opts->top_k;
  key.ngram = opts->no_repeat_ngram;
  key.eos = opts->eos_id;
  key.temperature = opts->temperature;
  key.penalty = opts->repetition_penalty;
  key.dump = s->dump;
  key.uniforms = s->uniforms;
  key.gen = s->buf_gen;
  key.fused = s->use_fast();
  int rc = FH_OK;
  if (g.n_dec > 0 && !g.persistent) {
    GraphKey k = key;
    k.kind = 0;
    rc = capture(s, s->g_decode, k, [&] { return enqueue_decode(s, g.plan); });
  }
  if (rc == FH_OK && g.n_re > 0) {
    GraphKey k = key;
    k.kind = 1;
    rc = capture(s, s->g_reprefill, k, [&] { return enqueue_window(s, C, g.plan); });
  }
  s->dump = saved_dump;
  s->uniforms = saved_u;
  if (rc != FH_OK) return rc;
  s->route = g.persistent ? (FH_ROUTE_FUSED_STEP | (g.persist_sampled ? FH_ROUTE_FUSED_SAMPLER : 0))
                          : (g.n_dec > 0 ? s->g_decode.route : 0);
  return FH_OK;
}

// Validation (Sampler.cs:82-89, 169-175), buffers, prompt upload and the step
// graphs of a generation; nothing is enqueued yet.  The state lives in s->gen.
static int gen_setup(fh_session* s, const int32_t* prompts, int batch, int P, int max_new, const fh_sampling* opts,
                     const double* uniforms, bool dump, bool deferred_uniforms = false, bool one_shot = false) {
  s->gen.active = false;
  if (!s->loaded) return set_err(FH_ERR_STATE, "weights are not loaded");
  if (P <= 0) return set_err(FH_ERR_INVALID, "Need at least one prompt token.");
  if (max_new < 0) return set_err(FH_ERR_RANGE, "maxNewTokens must be >= 0");
  if (opts->eos_id >= s->d.vocab_size)
    return set_err(FH_ERR_RANGE, "EOS token must be inside the model vocabulary.");
  if (!std::isfinite(opts->repetition_penalty) || opts->repetition_penalty < 1.f)
    return set_err(FH_ERR_RANGE, "Repetition penalty must be finite and >= 1.");
  if (opts->no_repeat_ngram < 0) return set_err(FH_ERR_RANGE, "No-repeat n-gram size must be >= 0.");
  if (!std::isfinite(opts->temperature)) return set_err(FH_ERR_INVALID, "Temperature must be finite.");
  if (batch != s->B()) return set_err(FH_ERR_INVALID, "batch %d must equal the session's max_batch %d", batch, s->B());
  if (opts->temperature > 0.f && !uniforms && !deferred_uniforms)
    return set_err(FH_ERR_INVALID, "sampling with temperature > 0 needs one uniform per step");
  FH_TRY(validate_ids(s, prompts, (size_t)batch * P));
  GenState& g = s->gen;
  g = GenState{};
  g.B = batch;
  g.P = P;
  g.max_new = max_new;
  g.opts = *opts;
  g.one_shot = one_shot;
  if (max_new == 0) {
    g.active = true;
    return FH_OK;
  }
  HIP_TRY(hipSetDevice(s->ctx->device));
  hipStream_t st = s->ctx->stream;
  const int B = batch, V = s->d.vocab_size, C = s->d.context_length;
  const int stride = P + max_new;
  FH_TRY(ensure(&s->tokens, &s->tokens_cap, (size_t)B * stride, &s->buf_gen));
  FH_TRY(ensure(&s->out_ids, &s->out_cap, (size_t)B * max_new, &s->buf_gen));
  const bool sampled = opts->temperature > 0.f;
  if (sampled) FH_TRY(ensure(&s->uniforms, &s->uni_cap, (size_t)B * max_new, &s->buf_gen));
  if (dump) FH_TRY(ensure(&s->dump, &s->dump_cap, (size_t)B * max_new * V, &s->buf_gen));
  for (int b = 0; b < B; b++)
    HIP_TRY(hipMemcpyAsync(s->tokens + (size_t)b * stride, prompts + (size_t)b * P, sizeof(int32_t) * P,
                           hipMemcpyHostToDevice, st));
  if (uniforms)
    HIP_TRY(hipMemcpyAsync(s->uniforms, uniforms, sizeof(double) * B * max_new, hipMemcpyHostToDevice, st));
  FH_TRY(reset_step_state(s));
  g.dump = dump;
  g.sampled = sampled;
  g.deferred = sampled && !uniforms;
  g.plan.P = P;
  g.plan.max_new = max_new;
  g.plan.tok_stride = stride;
  g.plan.opts = &g.opts;
  int rc = FH_OK;
  // which of steps 1..max_new-1 are cached decode steps (window fits) vs re-prefills
  for (int n = 1; n < max_new; n++) (P + n > C ? g.n_re : g.n_dec)++;
  if (s->use_fast() && g.n_dec > 0 && s->fast.before_launches(g.n_dec) != FH_OK)
    rc = set_err(FH_ERR_HIP, "resetting the fused decode state failed");
  // greedy on the fused kernel: launches run whole runs of cached steps (the
  // argmax of a step feeds the next inside the kernel); otherwise one graph per step
  {
    float* saved_dump = s->dump;  // fused_greedy reads the dump pointer the graphs would bake in
    if (!dump) s->dump = nullptr;
    g.persistent = g.n_dec > 0 && fused_greedy(s, opts);
    s->dump = saved_dump;
  }
  // sampled with top-k: the persistent launches draw in-kernel too (a stream's
  // launch covers the steps of one fh_generate_next call, whose uniforms are on
  // the device by then)
  if (!g.persistent && !s->no_sampled_fused && g.n_dec > 0 && s->use_fast() && sampled && !dump &&
      s->fast.sampler_fits(opts->top_k, P + g.n_dec)) {
    g.persistent = true;
    g.persist_sampled = true;
  }
  if (rc == FH_OK) rc = gen_capture(s);
  if (rc != FH_OK) return rc;
  g.active = true;
  return FH_OK;
}

// Enqueues steps gen.next .. upto-1: step 0 is the prompt's window forward,
// then the cached steps (one fused launch per run of them in greedy mode), then
// the re-prefill steps once the window slides.
static int gen_advance(fh_session* s, int upto) {
  GenState& g = s->gen;
  hipStream_t st = s->ctx->stream;
  const int C = s->d.context_length;
  upto = std::min(upto, g.max_new);
  float* saved_dump = s->dump;
  double* saved_u = s->uniforms;
  if (!g.dump) s->dump = nullptr;
  if (!g.sampled) s->uniforms = nullptr;
  int rc = FH_OK;
  if (g.next == 0 && upto > 0) {
    rc = enqueue_window(s, std::min(g.P, C), g.plan);
    g.next = 1;
  }
  while (rc == FH_OK && g.next < upto) {
    const int n = g.next;
    if (g.persistent && g.P + n <= C) {
      const int run = std::min(upto, 1 + g.n_dec) - n;  // cached steps are 1 .. n_dec
      rc = s->fast.enqueue(st, fused_step(s, g.plan, 1, run, g.persist_sampled, g.P + n + run - 1));
      if (rc != FH_OK) rc = set_err(rc, "fused decode launch failed: %s", hipGetErrorString(hipGetLastError()));
      g.next += run;
    } else {
      hipError_t e = hipGraphLaunch(g.P + n > C ? s->g_reprefill.exec : s->g_decode.exec, st);
      if (e != hipSuccess) rc = set_err(FH_ERR_HIP, "hipGraphLaunch: %s", hipGetErrorString(e));
      g.next++;
    }
  }
  s->dump = saved_dump;
  s->uniforms = saved_u;
  return rc;
}

// Copies the ids (and logits) produced so far and checks the fused kernel's
// hand-off status and the split-K GEMM's error word: every copy is queued on the
// stream into pinned host memory, then one synchronization.
static int gen_collect(fh_session* s, int32_t* out_ids, int32_t* out_counts, float* logits_dump) {
  GenState& g = s->gen;
  hipStream_t st = s->ctx->stream;
  const int B = g.B, V = s->d.vocab_size;
  const size_t nid = (size_t)B * g.max_new, need = nid + B + 2;
  if (need > s->hstage_cap) {
    if (s->hstage) (void)hipHostFree(s->hstage);
    s->hstage = nullptr;
    s->hstage_cap = 0;
    HIP_TRY(hipHostMalloc((void**)&s->hstage, need * sizeof(int32_t), hipHostMallocDefault));
    s->hstage_cap = need;
  }
  int32_t* h_ids = s->hstage;
  int32_t* h_counts = s->hstage + nid;
  int32_t* h_err = h_counts + B;  // [0] fused kernel, [1] split-K GEMM
  const bool fused = s->use_fast() && g.n_dec > 0;
  h_err[0] = h_err[1] = 0;
  HIP_TRY(hipMemcpyAsync(h_ids, s->out_ids, sizeof(int32_t) * nid, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(h_counts, s->out_counts, sizeof(int32_t) * B, hipMemcpyDeviceToHost, st));
  if (fused) HIP_TRY(hipMemcpyAsync(h_err, s->fast.error_word(), sizeof(int32_t), hipMemcpyDeviceToHost, st));
  if (s->gsplit)
    HIP_TRY(hipMemcpyAsync(h_err + 1, s->gsplit + s->gsplit_cap, sizeof(int32_t), hipMemcpyDeviceToHost, st));
  if (logits_dump)
    HIP_TRY(hipMemcpyAsync(logits_dump, s->dump, sizeof(float) * B * g.max_new * V, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  std::memcpy(out_ids, h_ids, sizeof(int32_t) * nid);
  std::memcpy(out_counts, h_counts, sizeof(int32_t) * B);
  if (h_err[1] != 0 && check_split_error(s) != FH_OK) {
    g.active = false;
    return FH_ERR_HIP;
  }
  const unsigned wait_code = (unsigned)h_err[0];
  if (fused && wait_code != 0) {
    s->fast.reset();
    const unsigned what = (wait_code >> 24) & 0x7f;
    if (what == 13 && g.persist_sampled) {
      // an exact top-k tie (or a non-finite logit): fh_generate repeats the
      // generation per step; a stream resumes on the per-step sampler
      if (g.one_shot) {
        g.active = false;
        return kRetryPerStep;
      }
      return kResumePerStep;
    }
    g.active = false;
    if (what == 11)
      return set_err(FH_ERR_HIP, "fused decode step: a token id outside [0, VocabSize) (results discarded)");
    if (what == 12)
      set_err(FH_ERR_HIP,
              "fused decode step: two blocks of one launch ran on the same XCD slot (block %u; the "
              "dispatcher no longer deals blocks round-robin over the XCDs; results discarded)",
              wait_code & 0xffff);
    else
      set_err(FH_ERR_HIP,
              "fused decode step: a hand-off wait exceeded its spin limit (wait %u, layer %u, block %u; "
              "results discarded)",
              what, (wait_code >> 16) & 0xff, wait_code & 0xffff);
    // fh_generate repeats the generation on the generic kernels; a stream
    // (fh_generate_next) has handed out earlier chunks and reports the error
    return g.one_shot ? kRetryGeneric : FH_ERR_HIP;
  }
  // a sequence without EOS so far has produced every step enqueued
  for (int b = 0; b < B; b++)
    if (out_counts[b] < 0) out_counts[b] = g.next;
  return FH_OK;
}

static int generate_once(fh_session* s, const int32_t* prompts, int batch, int P, int max_new,
                         const fh_sampling* opts, const double* uniforms, int32_t* out_ids, int32_t* out_counts,
                         float* logits_dump) {
  FH_TRY(gen_setup(s, prompts, batch, P, max_new, opts, uniforms, logits_dump != nullptr, false, true));
  for (int b = 0; b < batch; b++) out_counts[b] = 0;
  if (max_new == 0) return FH_OK;
  hipStream_t st = s->ctx->stream;
  (void)hipEventRecord(s->ev[0], st);
  int rc = gen_advance(s, 1);
  (void)hipEventRecord(s->ev[1], st);
  if (rc == FH_OK) rc = gen_advance(s, max_new);
  (void)hipEventRecord(s->ev[2], st);
  if (rc != FH_OK) {
    s->gen.active = false;
    (void)hipStreamSynchronize(st);
    return rc;
  }
  FH_TRY(gen_collect(s, out_ids, out_counts, logits_dump));
  s->gen.active = false;
  float ms0 = 0, ms1 = 0;
  (void)hipEventElapsedTime(&ms0, s->ev[0], s->ev[1]);
  (void)hipEventElapsedTime(&ms1, s->ev[1], s->ev[2]);
  s->t_prefill = ms0;
  s->t_decode = ms1;
  s->n_cached = s->gen.n_dec;
  s->n_reprefill = s->gen.n_re;
  return FH_OK;
}

int fh_generate(fh_session* s, const int32_t* prompts, int batch, int P, int max_new, const fh_sampling* opts,
                const double* uniforms, int32_t* out_ids, int32_t* out_counts, float* logits_dump) {
  if (!s || !prompts || !opts || !out_ids || !out_counts) return set_err(FH_ERR_INVALID, "null argument");
  int rc = generate_once(s, prompts, batch, P, max_new, opts, uniforms, out_ids, out_counts, logits_dump);
  if (rc == kRetryPerStep) {
    // the in-kernel sampler met a case it leaves to the per-step sampler (an exact
    // tie at a top-k threshold, a non-finite logit): the same generation again,
    // every step drawn by the per-step sampler kernel
    s->no_sampled_fused = true;
    rc = generate_once(s, prompts, batch, P, max_new, opts, uniforms, out_ids, out_counts, logits_dump);
    s->no_sampled_fused = false;
    if (rc == FH_OK) s->route |= FH_ROUTE_RETRIED;
  }
  if (rc == kRetryGeneric) {
    // a fused launch gave up (a hand-off wait past its spin limit, or its blocks
    // not covering the XCD slots): the same generation again on the generic
    // kernels, which need no co-resident blocks
    const bool saved = s->fast_allowed;
    s->fast_allowed = false;
    rc = generate_once(s, prompts, batch, P, max_new, opts, uniforms, out_ids, out_counts, logits_dump);
    s->fast_allowed = saved;
    if (rc == FH_OK) s->route |= FH_ROUTE_FALLBACK;
  }
  return rc;
}

int fh_generate_begin(fh_session* s, const int32_t* prompts, int batch, int P, int max_new, const fh_sampling* opts,
                      const double* uniforms) {
  if (!s || !prompts || !opts) return set_err(FH_ERR_INVALID, "null argument");
  return gen_setup(s, prompts, batch, P, max_new, opts, uniforms, false, true);
}

int fh_generate_next(fh_session* s, int steps, const double* uniforms, int32_t* out_ids, int32_t* out_counts,
                     int32_t* produced) {
  if (!s || !out_ids || !out_counts || !produced) return set_err(FH_ERR_INVALID, "null argument");
  if (!s->gen.active) return set_err(FH_ERR_STATE, "no generation in progress (fh_generate_begin first)");
  if (steps < 1) return set_err(FH_ERR_INVALID, "steps must be positive");
  GenState& g = s->gen;
  if (g.max_new == 0) {
    for (int b = 0; b < g.B; b++) out_counts[b] = 0;
    *produced = 0;
    return FH_OK;
  }
  HIP_TRY(hipSetDevice(s->ctx->device));
  const int n = std::min(steps, g.max_new - g.next);
  if (g.deferred) {
    // this call's uniforms, [batch][steps], for steps next .. next+n-1
    if (!uniforms) return set_err(FH_ERR_INVALID, "sampling with temperature > 0 needs one uniform per step");
    for (int b = 0; b < g.B; b++)
      HIP_TRY(hipMemcpyAsync(s->uniforms + (size_t)b * g.max_new + g.next, uniforms + (size_t)b * steps,
                             sizeof(double) * n, hipMemcpyHostToDevice, s->ctx->stream));
  }
  int rc = gen_advance(s, g.next + steps);
  if (rc != FH_OK) {
    g.active = false;
    (void)hipStreamSynchronize(s->ctx->stream);
    return rc;
  }
  rc = gen_collect(s, out_ids, out_counts, nullptr);
  if (rc == kResumePerStep) {
    // The in-kernel sampler met an exact tie at a top-k threshold (or a
    // non-finite logit) in this call's steps.  Every earlier step it drew equals
    // the per-step sampler's draw, so the stream goes on from a re-run of steps
    // 0 .. next-1 on the per-step path (the uniforms of every step so far are on
    // the device); ids already handed out are reproduced.
    const int upto = g.next;
    g.persistent = g.persist_sampled = false;
    FH_TRY(reset_step_state(s));
    if ((rc = gen_capture(s)) != FH_OK) {
      g.active = false;
      return rc;
    }
    g.next = 0;
    rc = gen_advance(s, upto);
    if (rc == FH_OK) rc = gen_collect(s, out_ids, out_counts, nullptr);
    s->route |= FH_ROUTE_RETRIED;
  }
  if (rc != FH_OK) {
    g.active = false;
    return rc;
  }
  *produced = g.next;
  if (g.next >= g.max_new) g.active = false;
  return FH_OK;
}

// Per-block timestamps (256 x 64) of one traced step of the last fused decode
// launch when the session was created with FORGE_HIP_TRACE=1.
int fh_debug_fused_trace(fh_session* s, unsigned long long* out, int n) {
  if (!s || !out || n < 0) return set_err(FH_ERR_INVALID, "bad argument");
  if (!s->fast.trace) return set_err(FH_ERR_STATE, "tracing is off (set FORGE_HIP_TRACE=1 before creating the session)");
  HIP_TRY(hipStreamSynchronize(s->ctx->stream));
  HIP_TRY(hipMemcpy(out, s->fast.trace, sizeof(unsigned long long) * std::min(n, 256 * 64), hipMemcpyDeviceToHost));
  return FH_OK;
}

int fh_last_route(fh_session* s, int32_t* route) {
  if (!s || !route) return set_err(FH_ERR_INVALID, "null argument");
  *route = s->route;
  return FH_OK;
}

int fh_last_timing(fh_session* s, double* prefill_ms, double* decode_ms, int32_t* cached, int32_t* reprefill) {
  if (!s) return set_err(FH_ERR_INVALID, "session is null");
  if (prefill_ms) *prefill_ms = s->t_prefill;
  if (decode_ms) *decode_ms = s->t_decode;
  if (cached) *cached = s->n_cached;
  if (reprefill) *reprefill = s->n_reprefill;
  return FH_OK;
}

// Sampler.ApplyRepetitionControls + Sampler.Sample of one device logit row with the
// caller's scratch: work [V] floats, ints [n_hist + 5] (history, step, done, out,
// count), u [1].  Synchronous; the id comes back through *out_id.
static int sample_row(fh_context* c, const float* logits_dev, int V, const int32_t* history, int n_hist,
                      const fh_sampling* opts, double u01, int32_t* out_id, float* work, int* ints, double* u) {
  hipStream_t st = c->stream;
  int* tokens = ints;
  int* misc = ints + n_hist + 1;  // step, done, out, count: cleared for every call
  if (n_hist > 0) HIP_TRY(hipMemcpyAsync(tokens, history, sizeof(int32_t) * n_hist, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(u, &u01, sizeof(double), hipMemcpyHostToDevice, st));
  const int init[4] = {0, 0, 0, -1};
  HIP_TRY(hipMemcpyAsync(misc, init, sizeof init, hipMemcpyHostToDevice, st));
  SampleArgs a{};
  a.logits = logits_dev;
  a.work = work;
  a.tokens = tokens;
  a.step = misc;
  a.done = misc + 1;
  a.out_ids = misc + 2;
  a.out_counts = misc + 3;
  a.uniforms = u;
  a.dump = nullptr;
  a.B = 1;
  a.V = V;
  a.tok_stride = n_hist + 1;
  a.prompt_len = n_hist;
  a.ctx = n_hist > 0 ? n_hist : 1;
  a.max_new = 1;
  a.temperature = opts->temperature;
  a.penalty = opts->repetition_penalty;
  a.top_k = opts->top_k;
  a.ngram = opts->no_repeat_ngram;
  a.eos = -1;
  if (n_hist == 0) {
    // an empty history never triggers the controls (T = 0 < ngram - 1 only for ngram > 1)
    a.ctx = 1;
    a.prompt_len = 0;
  }
  hipError_t e = launch_sample(st, a);
  if (e != hipSuccess) return check_launch(e, "launch_sample");
  int32_t r = 0;
  HIP_TRY(hipMemcpyAsync(&r, misc + 2, sizeof(int32_t), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  *out_id = r;
  return FH_OK;
}

static int check_sample_args(fh_context* c, const float* logits_dev, int V, const int32_t* history, int n_hist,
                             const fh_sampling* opts, int32_t* out_id) {
  if (!c || !logits_dev || !opts || !out_id || (n_hist > 0 && !history))
    return set_err(FH_ERR_INVALID, "null argument");
  if (V <= 0 || V > 65536) return set_err(FH_ERR_UNSUPPORTED, "V must be in [1, 65536]");
  if (n_hist < 0) return set_err(FH_ERR_INVALID, "n_hist must be >= 0");
  if (!std::isfinite(opts->temperature)) return set_err(FH_ERR_INVALID, "Temperature must be finite.");
  if (!std::isfinite(opts->repetition_penalty) || opts->repetition_penalty < 1.f)
    return set_err(FH_ERR_RANGE, "Repetition penalty must be finite and >= 1.");
  if (opts->no_repeat_ngram < 0) return set_err(FH_ERR_RANGE, "No-repeat n-gram size must be >= 0.");
  return FH_OK;
}

int fh_sample_logits(fh_context* c, const float* logits_dev, int V, const int32_t* history, int n_hist,
                     const fh_sampling* opts, double u01, int32_t* out_id) {
  FH_TRY(check_sample_args(c, logits_dev, V, history, n_hist, opts, out_id));
  HIP_TRY(hipSetDevice(c->device));
  if (V > c->s_V) {
    dev_free(c->s_work);
    FH_TRY(dev_alloc(&c->s_work, V));
    c->s_V = V;
  }
  const int need = n_hist + 1 + 4;
  if (need > c->s_hist) {
    dev_free(c->s_ints);
    FH_TRY(dev_alloc(&c->s_ints, need));
    c->s_hist = need;
  }
  if (!c->s_u) FH_TRY(dev_alloc(&c->s_u, 1));
  return sample_row(c, logits_dev, V, history, n_hist, opts, u01, out_id, c->s_work, c->s_ints, c->s_u);
}

// ---------------------------------------------------------------------------
// fh_sample_logits_noalloc: the same draw on a fixed scratch array in device
// memory, for callers that must not allocate.  Layout of `scratch`: the work row
// (FH_NOALLOC_MAX_VOCAB floats), then the uniform (one double), then the ints
// (history of up to FH_NOALLOC_MAX_HISTORY ids, step, done, out, count).  Each
// device holds its own copy until the process ends; host code reaches it only
// through the per-device address from hipGetSymbolAddress (g_scratch_dev).
// ---------------------------------------------------------------------------
constexpr size_t kScratchWork = (size_t)FH_NOALLOC_MAX_VOCAB * sizeof(float);
constexpr size_t kScratchU = kScratchWork;
constexpr size_t kScratchInts = kScratchU + 256;
constexpr size_t kScratchBytes = kScratchInts + ((size_t)FH_NOALLOC_MAX_HISTORY + 5) * sizeof(int);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static std::vector<unsigned char*> g_scratch_dev;  // per device id: the device address of `scratch`
// one lock per device id, held for a whole fh_sample_logits_noalloc call: calls on
// one device from several threads or contexts take turns on the shared array
constexpr int kScratchLocks = 64;
static std::mutex g_scratch_call_mu[kScratchLocks];

// Resolves `scratch`'s address on the current device (once per device); called by
// fh_context_create with the context's device current.
static int scratch_init(int device) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if ((size_t)device < g_scratch_dev.size() && g_scratch_dev[device]) return FH_OK;
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return set_err(FH_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
  if ((size_t)device >= g_scratch_dev.size()) g_scratch_dev.resize(device + 1, nullptr);
  g_scratch_dev[device] = static_cast<unsigned char*>(ptr);
  return FH_OK;
}

int fh_sample_logits_noalloc(fh_context* c, const float* logits_dev, int V, const int32_t* history, int n_hist,
                             const fh_sampling* opts, double u01, int32_t* out_id) {
  FH_TRY(check_sample_args(c, logits_dev, V, history, n_hist, opts, out_id));
  if (V > FH_NOALLOC_MAX_VOCAB)
    return set_err(FH_ERR_RANGE, "V (%d) exceeds the no-allocation scratch (%d)", V, FH_NOALLOC_MAX_VOCAB);
  if (n_hist > FH_NOALLOC_MAX_HISTORY)
    return set_err(FH_ERR_RANGE, "history of %d ids exceeds the no-allocation scratch (%d)", n_hist,
                   FH_NOALLOC_MAX_HISTORY);
  unsigned char* base = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if ((size_t)c->device < g_scratch_dev.size()) base = g_scratch_dev[c->device];
  }
  if (!base) return set_err(FH_ERR_STATE, "no scratch address for device %d", c->device);
  if (c->device >= kScratchLocks) return set_err(FH_ERR_RANGE, "device id %d >= %d", c->device, kScratchLocks);
  HIP_TRY(hipSetDevice(c->device));
  // sample_row returns once the stream has finished, so the array is free again
  std::lock_guard<std::mutex> g(g_scratch_call_mu[c->device]);
  return sample_row(c, logits_dev, V, history, n_hist, opts, u01, out_id, reinterpret_cast<float*>(base),
                    reinterpret_cast<int*>(base + kScratchInts), reinterpret_cast<double*>(base + kScratchU));
}

}  // extern "C"
