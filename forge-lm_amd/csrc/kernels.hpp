// kernels.hpp -- launch wrappers for the generic gfx950 kernels (kernels.hip).
// Vectors (LayerNorm weights, biases) are fp32 in every session; matrices are
// fp32 or bf16 (WT).  Every wrapper checks on the host that its operands fit what the kernel and
// its grid assume before launching, and returns a hipError_t.
#pragma once

#include "common.hpp"

namespace fh {

enum Epilogue : int { EPI_NONE = 0, EPI_GELU = 1, EPI_RESIDUAL = 2, EPI_QKV = 3 };

// x[r,:] = tok_emb[id(r)] + pos_emb[pos(r)] for rows r = b*T + t.
template <typename WT>
hipError_t launch_embed(hipStream_t st, RowSrc src, int B, int T, const WT* tok, const WT* pos, int d, int V,
                        int ctx, float* x);

// out[r,:] = LN(in[r_in,:]) with r_in = r_in0 + (r / rows_per_seq) * seq_stride + (r % rows_per_seq).
hipError_t launch_layernorm(hipStream_t st, const float* in, int rows, int rows_per_seq, int seq_stride,
                            int r_in0, const float* w, const float* b, float* out, int d, float eps);

// The same for every row of in (rows_per_seq = rows), rounded to bf16 into out.
hipError_t launch_layernorm_bf16(hipStream_t st, const float* in, int rows, const float* w, const float* b,
                                 bf16_t* out, int d, float eps);

// Split-K GEMV for M <= 4 rows: part[s][m][n] = sum_{k in chunk s} x[m,k] W[k,n].
template <typename WT>
hipError_t launch_gemv_splitk(hipStream_t st, const float* x, int M, int K, const WT* W, int N, float* part,
                              int splits, int* used_splits);

// y[m,n] = epi(sum_s part[s][m][n] + bias[n]) (+ res[m,n]).
hipError_t launch_splitk_epilogue(hipStream_t st, const float* part, int splits, int M, int N, const float* bias,
                                  int epi, const float* res, float* y);

// The split-K reduction fused with the LayerNorm that follows (N <= 1024): y = sum_s
// part[s] + bias (+ res), out = LN(y) per row; equal to launch_splitk_epilogue then
// launch_layernorm.
hipError_t launch_epilogue_ln(hipStream_t st, const float* part, int splits, int M, int N, const float* bias,
                              const float* res, float* y, const float* w, const float* b, float* out, float eps);

// The split-K reduction of a qkv projection fused with the KV store: qkv = sum_s
// part[s] + bias, and the K, V columns into the caches at pos(row) (as launch_kv_store).
template <typename KT>
hipError_t launch_epilogue_qkv(hipStream_t st, const float* part, int splits, int M, int d, const float* bias,
                               float* qkv, RowSrc src, int T, int H, int ctx, KT* kcache, KT* vcache);

// Tiled GEMM for any M: y[m,n] = epi(sum_k a[m,k] W[k,n] + bias[n]) (+ res[m,n]).
template <typename WT>
hipError_t launch_gemm(hipStream_t st, const float* a, int M, int K, const WT* W, int N, const float* bias, int epi,
                       const float* res, float* y);

// dst[r, c] = src[row0 + r * rstride, c] (leading dimensions src_ld, dst_ld) in fp32,
// for r < rows, c < d.
template <typename IT>
hipError_t launch_gather_rows(hipStream_t st, const IT* src, int src_ld, int row0, int rstride, int rows, int d,
                              float* dst, int dst_ld);

// K/V columns of qkv [B*T, 3d] into the cache [B][H][ctx][hd] at positions pos(row).
template <typename KT>
hipError_t launch_kv_store(hipStream_t st, RowSrc src, const float* qkv, int B, int T, int d, int H, int ctx,
                           KT* kcache, KT* vcache);

// Causal attention of every window row (prefill): o[r, h*hd:] for r = b*T + t over keys 0..t.
template <typename KT>
hipError_t launch_attn_prefill(hipStream_t st, const float* qkv, int B, int T, int d, int H, int ctx,
                               const KT* kcache, const KT* vcache, float* o);

// The same on MFMA tiles (attn_mfma.hip), for head_dim 64: bf16 caches multiply in bf16
// (q and the softmax weights rounded to bf16), fp32 caches in fp32.  o is fp32, or
// bf16 (rounded) for a bf16 session's large-M GEMM.
template <typename KT, typename OT>
hipError_t launch_attn_prefill_mfma(hipStream_t st, const float* qkv, int B, int T, int d, int H, int ctx,
                                    const KT* kcache, const KT* vcache, OT* o);

// The same with q already in bf16, q [B*T][d] (from launch_gemm_bf16_qkv).
hipError_t launch_attn_prefill_mfma_q16(hipStream_t st, const bf16_t* q, int B, int T, int d, int H, int ctx,
                                        const bf16_t* kcache, const bf16_t* vcache, bf16_t* o);

// Decode attention of one row per sequence over keys 0..pos (pos from src), split over
// chunks of `chunk` keys, then combined.  part must hold B*H*max_chunks*(hd+2) floats.
template <typename KT>
hipError_t launch_attn_decode(hipStream_t st, RowSrc src, const float* qkv, int B, int d, int H, int ctx,
                              const KT* kcache, const KT* vcache, float* part, int chunk, float* o);

// Combines the chunk partials part[(b*H + h)*maxc + c][hd + 2] (o, max, sum) of
// the keys 0..pos (pos from src) into o[b, h*hd:].
hipError_t launch_attn_decode_combine(hipStream_t st, RowSrc src, int B, int d, int H, int ctx, const float* part,
                                      int chunk, int maxc, float* o);

// The same decode attention for head_dim 64 (attn_decode.hip): 256-key chunks,
// one 1 KB request per 4 K or V rows.  part must hold B*H*ceil(ctx/256)*66 floats.
// Without `combine` only the chunk partials are written (the consumer combines).
// With qp, q comes from the qkv projection's split-K partials (summed with the
// bias as k_epilogue_qkv does; qkv is not read) and the new K/V row of each
// sequence is written into the caches by the block that attends over it.
constexpr int kAttnDecodeChunk = 256;
struct QkvParts {
  const float* part;  // [S][M][3d]
  int S, M;
  const float* bias;  // [3d] or null
};
template <typename KT>
hipError_t launch_attn_decode_wide(hipStream_t st, RowSrc src, const float* qkv, int B, int d, int H, int ctx,
                                   const KT* kcache, const KT* vcache, float* part, float* o, bool combine = true,
                                   const QkvParts* qp = nullptr);

// Tied head for B rows: logits[b, v] = dot(xn[b,:], E[v,:]).
template <typename WT>
hipError_t launch_head(hipStream_t st, const float* xn, int B, int d, const WT* E, int V, float* logits);

// MFMA GEMM (gemm_mfma.hip): y = epi(a[M,K] @ W + bias) (+ res) with W given
// transposed as Wt[N][K]; K a multiple of 32.  Small M splits K over up to
// part_floats of partials (then sums them with launch_splitk_epilogue).
template <typename WT>
hipError_t launch_gemm_mfma(hipStream_t st, const float* a, int M, int K, const WT* Wt, int N, const float* bias,
                            int epi, const float* res, float* y, float* part, size_t part_floats, int cus);

// bf16 GEMM for large M (gemm_bf16.hip): y = epi(a[M,K] @ W + bias) (+ res) with a
// in bf16 and W given transposed as Wt[N][K] bf16; K a multiple of 64.  Exactly one
// of y (fp32) and yh (bf16, rounded) is the output.
hipError_t launch_gemm_bf16(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                            const float* bias, int epi, const float* res, float* y, bf16_t* yh);

// The residual form of launch_gemm_bf16 (y = a @ W + bias + res, fp32 y) with
// the sum over K split in two halves on separate blocks when the product has too
// few 256 x 256 tiles to fill the CUs (mlp.proj: N 1024, K 4096): the half that
// finishes first leaves its partial sums in ws (M*N floats), the other adds them
// (fp32 addition commutes, so the bits do not depend on which half is first).
// cnt holds cnt_cap + 1 ints: one per tile, zero before the call and zero after
// it, then an error word that stays zero unless a tile's halves failed to meet
// (bit 0: the second half's bounded wait for the first gave up; bit 1: the halves
// ran on different XCDs); such a tile's y is NaN, and the caller reads the word
// once the stream has finished.  Calls sharing ws or cnt must not overlap.
// Shapes the split does not suit run as launch_gemm_bf16.
hipError_t launch_gemm_bf16_split(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                                  const float* bias, const float* res, float* y, float* ws, size_t ws_floats,
                                  int* cnt, int cnt_cap);

// Outputs of the bf16 GEMM's epilogues (one set is used per launch).
struct GemmBf16Out {
  const float* res;  // residual added to y, or null
  float* y;          // fp32 output [M][N]
  bf16_t* yh;        // bf16 output [M][N]
  bf16_t* q;         // EPI_QKV: q [M][D]; K and V into the caches [B][H][ctx][64] at pos(row)
  bf16_t* kc;
  bf16_t* vc;
  RowSrc src;
  int T, H, ctx;
  float* ws;  // K split in two: the first half's partial sums [M][N] (launch_gemm_bf16_split)
  int* cnt;   // and one arrival counter per 256 x 256 tile, zero between launches
  int* err;   // and the split's error word (see launch_gemm_bf16_split)
};

// The QKV projection of a window with the cache store fused (replaces the fp32
// qkv row + launch_kv_store): y = a @ Wqkv + b over M = B*T rows, q columns
// rounded to bf16 into q [M][D], K and V columns into kcache / vcache at the
// row's position (rows past ctx are dropped), D = 64 H.
hipError_t launch_gemm_bf16_qkv(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, const float* bias,
                                RowSrc src, int T, int H, int ctx, bf16_t* q, bf16_t* kcache, bf16_t* vcache);

// Where a split-K GEMM's A operand [M][K] comes from.  AOP_ATTN: decode
// attention's chunk partials apart[(b*H + h)*maxc + c][hd + 2] of row b combined
// as k_attn_decode_combine does (keys 0..pos, pos from src): the A values equal
// what the combine kernel would have written, without that launch.
enum AOpKind : int { AOP_PLAIN = 0, AOP_ATTN = 2 };
struct AOperand {
  int kind;
  const float* apart;
  RowSrc src;
  int H, ctx, chunk, maxc;
};

// The same GEMM writing only the split-K partials part[S][M][N] (S >= 1, returned
// in *splits) for a fused epilogue to reduce; A is `a` or, with aop, built from
// the producer's partials (AOP_ATTN: at most 4 chunks, ctx <= 1024).
template <typename WT>
hipError_t launch_gemm_mfma_split(hipStream_t st, const float* a, int M, int K, const WT* Wt, int N, float* part,
                                  size_t part_floats, int cus, int* splits, const AOperand* aop = nullptr);

// Decode GEMMs of at most 32 fp32 rows (gemm_skinny.hip): 16 output columns per
// block over a 768-deep K range, S = K / 768 blocks per column strip.  EPI_GELU
// (S == 1): y = gelu(x @ W + bias) [M][N]; EPI_NONE: y = part[S][M][N] of x @ W
// (no bias).  gemm_skinny_fits says whether a shape qualifies.
bool gemm_skinny_fits(int M, int K, int N);
hipError_t launch_gemm_skinny(hipStream_t st, const float* x, int M, int K, const float* Wt, int N,
                              const float* bias, int epi, float* y, int* splits);

// Wt[n][k] = W[k][n].
template <typename WT>
hipError_t launch_transpose(hipStream_t st, const WT* W, int K, int N, WT* Wt);

// out[i] = in[i] rounded to bf16 (nearest-even), i < n.
hipError_t launch_round_bf16(hipStream_t st, const float* in, size_t n, bf16_t* out);

// dst[0..bytes) = src[0..bytes) on the device (both 16-byte aligned).
hipError_t launch_copy(hipStream_t st, void* dst, const void* src, size_t bytes);
// Sum of the 32-bit words of src (bytes % 4 == 0, 16-byte aligned) mod 2^64 into
// *out (device); part holds nparts (<= kChecksumParts) per-block partials;
// read_done (optional) is recorded after the pass that reads src.
constexpr int kChecksumParts = 4096;
hipError_t launch_checksum(hipStream_t st, const void* src, size_t bytes, unsigned long long* part, int nparts,
                           unsigned long long* out, hipEvent_t read_done);

struct SampleArgs {
  const float* logits;  // [B][V] raw ForwardLast logits
  float* work;          // [B][V] scratch
  int* tokens;          // [B][tok_stride] prompt + generated ids
  int* step;            // device step counter (advanced by the last block)
  int* done;            // block arrival counter (zeroed before first use; self-resetting)
  int* out_ids;         // [B][max_new]
  int* out_counts;      // [B]
  const double* uniforms;  // [B][max_new] or null
  float* dump;          // [B][max_new][V] or null
  int B, V, tok_stride, prompt_len, ctx, max_new;
  float temperature, penalty;
  int top_k, ngram, eos;
};
hipError_t launch_sample(hipStream_t st, const SampleArgs& a);

}  // namespace fh
