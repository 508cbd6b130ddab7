// kernels.hip -- generic gfx950 kernels of the ForgeLM token loop.
//
// These run every model shape (any d divisible by 8, any head count with
// head_dim <= 128, any batch) and are the path for prefill, re-prefill after a
// window slide, and batched decode.  The batch-1 fp32 decode step has a fused
// fast path in decode_fast.hip.
//
// Reference semantics (paths relative to the reference checkout):
//   embedding + positions  GptModel.cs:217-218, CpuBackend.cs:527-531
//   LayerNorm              CpuBackend.cs:377-398 (biased variance, eps 1e-5)
//   Linear                 Layers.cs:29-37 (x @ W[in,out] + b)
//   attention              Layers.cs:191-229, ITensorBackend.cs:117-122
//   GELU                   CpuBackend.cs:510-514
//   tied head              Layers.cs:80-86 (x @ tok_emb^T)
//   sampler                Sampler.cs:14-69, 111-165
#include "kernels.hpp"

#include <math.h>

namespace fh {

namespace {

template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; i++) s += red[i];
  return s;
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; i++) s = fmaxf(s, red[i]);
  return s;
}

template <typename WT, int VEC>
__device__ __forceinline__ void load_vec(const WT* p, float* out);

template <>
__device__ __forceinline__ void load_vec<float, 4>(const float* p, float* out) {
  float4 v = *reinterpret_cast<const float4*>(p);
  out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}

template <>
__device__ __forceinline__ void load_vec<bf16_t, 8>(const bf16_t* p, float* out) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// embedding
// ---------------------------------------------------------------------------
template <typename WT>
__global__ __launch_bounds__(256) void k_embed(RowSrc src, int T, const WT* __restrict__ tok,
                                               const WT* __restrict__ pos, int d, int V, int ctx,
                                               float* __restrict__ x) {
  const int r = blockIdx.x, b = r / T, t = r % T;
  const int n = *src.step;
  int id = src.tokens[(size_t)b * src.tok_stride + src.tok_off + n + t];
  int p = src.pos_off + src.pos_mul * n + t;
  if ((unsigned)id >= (unsigned)V) id = 0;  // ids are validated on the host; never index out of range
  if ((unsigned)p >= (unsigned)ctx) p = 0;
  for (int c = threadIdx.x; c < d; c += blockDim.x)
    x[(size_t)r * d + c] = to_f32(tok[(size_t)id * d + c]) + to_f32(pos[(size_t)p * d + c]);
}

// ---------------------------------------------------------------------------
// LayerNorm, one 256-thread block per row
// ---------------------------------------------------------------------------
template <typename OT>
__global__ __launch_bounds__(256) void k_layernorm(const float* __restrict__ in, int rows_per_seq,
                                                   int seq_stride, int r_in0, const float* __restrict__ w,
                                                   const float* __restrict__ b, OT* __restrict__ out, int d,
                                                   float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const int rin = r_in0 + (r / rows_per_seq) * seq_stride + (r % rows_per_seq);
  const float* xr = in + (size_t)rin * d;
  float s = 0.f;
  for (int c = threadIdx.x; c < d; c += 256) s += xr[c];
  const float mu = block_sum<256>(s, red) / (float)d;
  float v = 0.f;
  for (int c = threadIdx.x; c < d; c += 256) {
    float dd = xr[c] - mu;
    v += dd * dd;
  }
  const float var = block_sum<256>(v, red);
  const float rs = 1.f / sqrtf(var / (float)d + eps);
  for (int c = threadIdx.x; c < d; c += 256) out[(size_t)r * d + c] = from_f32<OT>((xr[c] - mu) * rs * w[c] + b[c]);
}

// The same for d a multiple of 256, one wave per row, rounded to bf16: the row
// stays in registers (VPL float4 per lane, coalesced 1 KB loads), mean and
// variance are wave sums, the output goes out as 8-byte bf16 quads.  w and b are
// requested with the row (a load issued after the first output store would wait
// for it: loads and stores share one completion counter).
template <int VPL>
__global__ __launch_bounds__(256) void k_layernorm_rows_bf16(const float* __restrict__ in, int rows,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ b, bf16_t* __restrict__ out,
                                                             float eps) {
  constexpr int d = 256 * VPL;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float4* xr = reinterpret_cast<const float4*>(in + (size_t)r * d);
  float4 x[VPL], wv[VPL], bv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; i++) x[i] = xr[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < VPL; i++) {
    wv[i] = reinterpret_cast<const float4*>(w)[i * 64 + lane];
    bv[i] = reinterpret_cast<const float4*>(b)[i * 64 + lane];
  }
  __builtin_amdgcn_sched_barrier(0);  // the loads stay here, ahead of the reductions
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; i++) s += (x[i].x + x[i].y) + (x[i].z + x[i].w);
  const float mu = wave_sum_dpp(s) / (float)d;
  float v = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; i++) {
    x[i] = make_float4(x[i].x - mu, x[i].y - mu, x[i].z - mu, x[i].w - mu);
    v += (x[i].x * x[i].x + x[i].y * x[i].y) + (x[i].z * x[i].z + x[i].w * x[i].w);
  }
  const float rs = 1.f / sqrtf(wave_sum_dpp(v) / (float)d + eps);
  uint2* orow = reinterpret_cast<uint2*>(out + (size_t)r * d);
#pragma unroll
  for (int i = 0; i < VPL; i++) {
    const uint32_t lo = (uint32_t)bf16_rn(x[i].x * rs * wv[i].x + bv[i].x) |
                        ((uint32_t)bf16_rn(x[i].y * rs * wv[i].y + bv[i].y) << 16);
    const uint32_t hi = (uint32_t)bf16_rn(x[i].z * rs * wv[i].z + bv[i].z) |
                        ((uint32_t)bf16_rn(x[i].w * rs * wv[i].w + bv[i].w) << 16);
    orow[i * 64 + lane] = make_uint2(lo, hi);
  }
}

// Split-K reduction (k_splitk_epilogue's sum, bias, residual) fused with the
// LayerNorm that follows: one 1024-thread block per row (a thread per column)
// writes the row to y, exactly as k_splitk_epilogue would, and its LayerNorm to
// out, with k_layernorm's formula over block sums.  N <= 1024.
__global__ __launch_bounds__(1024) void k_epilogue_ln(const float* __restrict__ part, int S, int M, int N,
                                                      const float* __restrict__ bias, const float* __restrict__ res,
                                                      float* __restrict__ y, const float* __restrict__ w,
                                                      const float* __restrict__ b, float* __restrict__ out,
                                                      float eps) {
  __shared__ float red[16];
  const int r = blockIdx.x, c = threadIdx.x;
  const bool on = c < N;
  // one column per thread, up to 32 of its partials in flight together through a
  // bounded resource (skipped ones, past S or N, read as zeros); the partials add
  // in order, and the zeros after the last one change nothing.  Each partial is
  // read once: the loads carry the non-temporal hint (C4: 870 -> 863 us per step).
  const int pbytes = (int)((size_t)S * M * N * 4);
  const __amdgpu_buffer_rsrc_t rp =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(part), (short)0, pbytes, 0x00020000);
  const size_t idx = (size_t)r * N + c;
  // the column's bias, residual and LayerNorm weights are requested with the
  // partials: issued later, each would cost a round trip of its own (the last ones
  // behind the store of y: loads and stores share one completion counter)
  float bc = 0.f, rc = 0.f, wc = 0.f, lbc = 0.f;
  if (on) {
    if (bias) bc = bias[c];
    if (res) rc = res[idx];
    wc = w[c];
    lbc = b[c];
  }
  float v = 0.f;
  for (int i0 = 0; i0 < S; i0 += 32) {
    float t[32];
#pragma unroll
    for (int ii = 0; ii < 32; ii++) {
      const int off = (on && i0 + ii < S) ? (int)((((size_t)(i0 + ii) * M + r) * N + c) * 4) : pbytes;
      t[ii] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, 2));
    }
#pragma unroll
    for (int ii = 0; ii < 32; ii++) v += t[ii];
  }
  if (on) {
    if (bias) v += bc;
    if (res) v += rc;
    y[idx] = v;
  } else {
    v = 0.f;
  }
  const float mu = block_sum<1024>(v, red) / (float)N;
  const float dd = on ? v - mu : 0.f;
  const float rs = 1.f / sqrtf(block_sum<1024>(dd * dd, red) / (float)N + eps);
  if (on) out[idx] = dd * rs * wc + lbc;
}

// Split-K reduction of a qkv projection (sum + bias into qkv) fused with the KV
// store: the K and V columns also go to the caches at the row's position, as
// k_kv_store writes them.
template <typename KT>
__global__ __launch_bounds__(256) void k_epilogue_qkv(const float* __restrict__ part, int S, int M, int d,
                                                      const float* __restrict__ bias, float* __restrict__ qkv,
                                                      RowSrc src, int T, int H, int ctx, KT* __restrict__ kc,
                                                      KT* __restrict__ vc) {
  const int N = 3 * d;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)M * N) return;
  const int col = (int)(idx % N), r = (int)(idx / N);
  // the bias and the step counter are requested with the partials (a load issued
  // after the store of qkv would wait for it)
  const float bc = bias ? bias[col] : 0.f;
  const int step = *src.step;
  float a = 0.f;
#pragma unroll 8
  for (int i = 0; i < S; i++) a += part[(size_t)i * M * N + idx];
  if (bias) a += bc;
  qkv[idx] = a;
  if (col < d) return;
  const int pos = src.pos_off + src.pos_mul * step + r % T;
  if ((unsigned)pos >= (unsigned)ctx) return;
  const int hd = d / H, c = col < 2 * d ? col - d : col - 2 * d, h = c / hd, e = c % hd;
  const size_t dst = (((size_t)(r / T) * H + h) * ctx + pos) * hd + e;
  if (col < 2 * d)
    kc[dst] = from_f32<KT>(a);
  else
    vc[dst] = from_f32<KT>(a);
}

// ---------------------------------------------------------------------------
// split-K GEMV (M <= 4): each block owns a 64*VEC column tile and one K chunk;
// each of its 4 waves walks every 4th row of the chunk with 16-byte loads.
// ---------------------------------------------------------------------------
template <typename WT, int MR>
__global__ __launch_bounds__(256) void k_gemv_splitk(const float* __restrict__ x, int M, int K,
                                                     const WT* __restrict__ W, int N, int kchunk,
                                                     float* __restrict__ part) {
  constexpr int VEC = 16 / sizeof(WT);
  constexpr int TILE = 64 * VEC;
  __shared__ float red[4][MR][TILE];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = blockIdx.x * TILE + lane * VEC;
  const int s = blockIdx.y;
  const int k0 = s * kchunk, k1 = min(K, k0 + kchunk);
  float acc[MR][VEC];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int j = 0; j < VEC; j++) acc[m][j] = 0.f;
  if (c0 < N) {
#pragma unroll 4
    for (int k = k0 + wv; k < k1; k += 4) {
      float wvv[VEC];
      load_vec<WT, VEC>(W + (size_t)k * N + c0, wvv);
#pragma unroll
      for (int m = 0; m < MR; m++) {
        // rows past M (never stored) read row M - 1: no branch around the load
        const float xm = x[(size_t)min(m, M - 1) * K + k];
#pragma unroll
        for (int j = 0; j < VEC; j++) acc[m][j] += xm * wvv[j];
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int j = 0; j < VEC; j++) red[wv][m][lane * VEC + j] = acc[m][j];
  __syncthreads();
  for (int idx = threadIdx.x; idx < MR * TILE; idx += 256) {
    const int m = idx / TILE, cc = idx % TILE;
    const int col = blockIdx.x * TILE + cc;
    if (m < M && col < N)
      part[((size_t)s * M + m) * N + col] = red[0][m][cc] + red[1][m][cc] + red[2][m][cc] + red[3][m][cc];
  }
}

__global__ __launch_bounds__(256) void k_splitk_epilogue(const float* __restrict__ part, int S, int M, int N,
                                                         const float* __restrict__ bias, int epi,
                                                         const float* __restrict__ res, float* __restrict__ y) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)M * N) return;
  const int n = (int)(idx % N);
  // the bias and residual are requested with the partials (one round trip, not three)
  const float bn = bias ? bias[n] : 0.f, rn = res ? res[idx] : 0.f;
  float s = 0.f;
  // partials summed in order; the unrolled loads of a batch are independent and go out together
#pragma unroll 8
  for (int i = 0; i < S; i++) s += part[(size_t)i * M * N + idx];
  if (bias) s += bn;
  if (epi == EPI_GELU) s = gelu_tanh(s);
  if (res) s += rn;
  y[idx] = s;
}

// ---------------------------------------------------------------------------
// tiled GEMM (any M): 64x64 tile, 256 threads x 4x4 outputs, K steps of 16
// ---------------------------------------------------------------------------
template <typename WT>
__global__ __launch_bounds__(256) void k_gemm_tiled(const float* __restrict__ A, int M, int K,
                                                    const WT* __restrict__ W, int N, const float* __restrict__ bias,
                                                    int epi, const float* __restrict__ res, float* __restrict__ Y) {
  __shared__ float As[16][68];
  __shared__ float Bs[16][68];
  const int tid = threadIdx.x;
  const int tm = blockIdx.y * 64, tn = blockIdx.x * 64;
  const int tx = tid % 16, ty = tid / 16;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = tid; i < 1024; i += 256) {
      const int r = i / 16, kk = i % 16;
      As[kk][r] = (tm + r < M && k0 + kk < K) ? A[(size_t)(tm + r) * K + k0 + kk] : 0.f;
    }
    for (int i = tid; i < 1024; i += 256) {
      const int kk = i / 64, c = i % 64;
      Bs[kk][c] = (k0 + kk < K && tn + c < N) ? to_f32(W[(size_t)(k0 + kk) * N + tn + c]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float a[4], bb[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) bb[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] += a[i] * bb[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = tm + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = tn + tx * 4 + j;
      if (n >= N) continue;
      float s = acc[i][j] + (bias ? bias[n] : 0.f);
      if (epi == EPI_GELU) s = gelu_tanh(s);
      if (res) s += res[(size_t)m * N + n];
      Y[(size_t)m * N + n] = s;
    }
  }
}

// dst[r, c] = src[row0 + r * rstride, c] in fp32: one block per row.
template <typename IT>
__global__ __launch_bounds__(256) void k_gather_rows(const IT* __restrict__ src, int src_ld, int row0, int rstride,
                                                     int d, float* __restrict__ dst, int dst_ld) {
  const int r = blockIdx.x;
  const IT* s = src + (size_t)(row0 + (size_t)r * rstride) * src_ld;
  float* o = dst + (size_t)r * dst_ld;
  for (int c = threadIdx.x; c < d; c += 256) o[c] = to_f32<IT>(s[c]);
}

// ---------------------------------------------------------------------------
// KV cache store and attention
// ---------------------------------------------------------------------------
template <typename KT>
__global__ __launch_bounds__(256) void k_kv_store(RowSrc src, const float* __restrict__ qkv, int T, int d, int H,
                                                  int ctx, KT* __restrict__ kc, KT* __restrict__ vc) {
  const int r = blockIdx.x, b = r / T, t = r % T;
  const int n = *src.step;
  const int pos = src.pos_off + src.pos_mul * n + t;
  if ((unsigned)pos >= (unsigned)ctx) return;
  const int hd = d / H;
  for (int c = threadIdx.x; c < d; c += 256) {
    const int h = c / hd, e = c % hd;
    const size_t dst = (((size_t)b * H + h) * ctx + pos) * hd + e;
    kc[dst] = from_f32<KT>(qkv[(size_t)r * 3 * d + d + c]);
    vc[dst] = from_f32<KT>(qkv[(size_t)r * 3 * d + 2 * d + c]);
  }
}

// Online-softmax attention of one query over keys [j0, j1) of one head, one
// wave; lane e accumulates output dims e and e+64.  Returns the running
// (max, sum) and the unnormalised output.
template <typename KT>
__device__ __forceinline__ void attend_range(const float* qs, const KT* __restrict__ K, const KT* __restrict__ Vv,
                                             int hd, int j0, int j1, float scale, float& m, float& l, float& acc0,
                                             float& acc1) {
  const int lane = threadIdx.x & 63;
  for (int jb = j0; jb < j1; jb += 64) {
    const int j = jb + lane;
    float s = -INFINITY;
    if (j < j1) {
      const KT* kr = K + (size_t)j * hd;
      float dot = 0.f;
      for (int e = 0; e < hd; e++) dot += qs[e] * to_f32(kr[e]);
      s = dot * scale;
    }
    const float cm = wave_max(s);
    const float nm = fmaxf(m, cm);
    const float corr = (m == -INFINITY) ? 0.f : expf(m - nm);
    const float p = (j < j1) ? expf(s - nm) : 0.f;
    l = l * corr + wave_sum(p);
    acc0 *= corr;
    acc1 *= corr;
    const int cnt = min(64, j1 - jb);
    for (int jj = 0; jj < cnt; jj++) {
      const float pj = __shfl(p, jj, 64);
      const KT* vr = Vv + (size_t)(jb + jj) * hd;
      if (lane < hd) acc0 += pj * to_f32(vr[lane]);
      if (lane + 64 < hd) acc1 += pj * to_f32(vr[lane + 64]);
    }
    m = nm;
  }
}

template <typename KT>
__global__ __launch_bounds__(64) void k_attn_prefill(const float* __restrict__ qkv, int T, int d, int H, int ctx,
                                                     const KT* __restrict__ kc, const KT* __restrict__ vc,
                                                     float* __restrict__ o) {
  __shared__ float qs[128];
  const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int hd = d / H;
  const float scale = 1.f / sqrtf((float)hd);
  const float* q = qkv + (size_t)(b * T + t) * 3 * d + h * hd;
  for (int e = lane; e < hd; e += 64) qs[e] = q[e];
  __syncthreads();
  const KT* K = kc + ((size_t)b * H + h) * ctx * hd;
  const KT* Vv = vc + ((size_t)b * H + h) * ctx * hd;
  float m = -INFINITY, l = 0.f, a0 = 0.f, a1 = 0.f;
  attend_range(qs, K, Vv, hd, 0, t + 1, scale, m, l, a0, a1);
  float* orow = o + (size_t)(b * T + t) * d + h * hd;
  const float inv = 1.f / l;
  if (lane < hd) orow[lane] = a0 * inv;
  if (lane + 64 < hd) orow[lane + 64] = a1 * inv;
}

template <typename KT>
__global__ __launch_bounds__(64) void k_attn_decode_part(RowSrc src, const float* __restrict__ qkv, int d, int H,
                                                         int ctx, const KT* __restrict__ kc,
                                                         const KT* __restrict__ vc, float* __restrict__ part,
                                                         int chunk, int maxc) {
  __shared__ float qs[128];
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int hd = d / H;
  const int n = *src.step;
  const int nkeys = min(ctx, src.pos_off + src.pos_mul * n + 1);
  const int j0 = c * chunk, j1 = min(nkeys, j0 + chunk);
  if (j0 >= j1) return;
  const float scale = 1.f / sqrtf((float)hd);
  const float* q = qkv + (size_t)b * 3 * d + h * hd;
  for (int e = lane; e < hd; e += 64) qs[e] = q[e];
  __syncthreads();
  const KT* K = kc + ((size_t)b * H + h) * ctx * hd;
  const KT* Vv = vc + ((size_t)b * H + h) * ctx * hd;
  float m = -INFINITY, l = 0.f, a0 = 0.f, a1 = 0.f;
  attend_range(qs, K, Vv, hd, j0, j1, scale, m, l, a0, a1);
  float* P = part + (((size_t)b * H + h) * maxc + c) * (hd + 2);
  if (lane < hd) P[lane] = a0;
  if (lane + 64 < hd) P[lane + 64] = a1;
  if (lane == 0) {
    P[hd] = m;
    P[hd + 1] = l;
  }
}

__global__ __launch_bounds__(64) void k_attn_decode_combine(RowSrc src, int d, int H, int ctx,
                                                            const float* __restrict__ part, int chunk, int maxc,
                                                            float* __restrict__ o) {
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int hd = d / H;
  const int n = *src.step;
  const int nkeys = min(ctx, src.pos_off + src.pos_mul * n + 1);
  const int nch = (nkeys + chunk - 1) / chunk;
  const float* P0 = part + ((size_t)b * H + h) * maxc * (hd + 2);
  float M = -INFINITY;
  for (int c = 0; c < nch; c++) M = fmaxf(M, P0[(size_t)c * (hd + 2) + hd]);
  float L = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c = 0; c < nch; c++) {
    const float* P = P0 + (size_t)c * (hd + 2);
    const float f = expf(P[hd] - M);
    L += P[hd + 1] * f;
    if (lane < hd) a0 += P[lane] * f;
    if (lane + 64 < hd) a1 += P[lane + 64] * f;
  }
  const float inv = 1.f / L;
  float* orow = o + (size_t)b * d + h * hd;
  if (lane < hd) orow[lane] = a0 * inv;
  if (lane + 64 < hd) orow[lane + 64] = a1 * inv;
}

// ---------------------------------------------------------------------------
// tied head: logits[b, v] = dot(xn[b], E[v]); one wave per vocab row, 4 rows of
// x at a time staged in LDS
// ---------------------------------------------------------------------------
template <typename WT>
__global__ __launch_bounds__(256) void k_head(const float* __restrict__ xn, int B, int d, const WT* __restrict__ E,
                                              int V, float* __restrict__ logits) {
  constexpr int VEC = 16 / sizeof(WT);
  __shared__ float xs[4][1024];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int b0 = 0; b0 < B; b0 += 4) {
    for (int i = threadIdx.x; i < 4 * d; i += 256) {
      const int bb = i / d, k = i % d;
      xs[bb][k] = (b0 + bb < B) ? xn[(size_t)(b0 + bb) * d + k] : 0.f;
    }
    __syncthreads();
    for (int v = blockIdx.x * 4 + w; v < V; v += gridDim.x * 4) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int k = lane * VEC; k < d; k += 64 * VEC) {
        float e[VEC];
        load_vec<WT, VEC>(E + (size_t)v * d + k, e);
#pragma unroll
        for (int bb = 0; bb < 4; bb++)
#pragma unroll
          for (int j = 0; j < VEC; j++) acc[bb] += xs[bb][k + j] * e[j];
      }
#pragma unroll
      for (int bb = 0; bb < 4; bb++) {
        const float s = wave_sum(acc[bb]);
        if (lane == 0 && b0 + bb < B) logits[(size_t)(b0 + bb) * V + v] = s;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// sampler: one 1024-thread block per sequence (Sampler.cs:29-69, 111-165)
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)

namespace {

constexpr int kST = 1024;        // sampler block size
constexpr int kMaxVocab = 65536; // LDS bitmaps hold V bits
constexpr int kSurvCap = 4096;   // top-k survivors summed in index order
constexpr int kRowV = 16;        // logits per thread in the register sampler (V <= kST * kRowV)

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0;  // -0 and +0 compare equal, as in Array.Sort
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

struct SampleSmem {
  uint32_t seen[kMaxVocab / 32];
  uint32_t ban[kMaxVocab / 32];
  int hist[256];
  int surv[kSurvCap];
  int scan[kST];
  float redf[kST / 64];
  int redi[kST / 64];
  int misc[4];
};

__device__ int block_argmax(const float* __restrict__ v, int V, SampleSmem& sm) {
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < V; i += kST) argmax_merge(best, bi, v[i], i);
  wave_argmax(best, bi);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) {
    sm.redf[w] = best;
    sm.redi[w] = bi;
  }
  __syncthreads();
  float bv = sm.redf[0];
  int ii = sm.redi[0];
  for (int i = 1; i < kST / 64; i++) argmax_merge(bv, ii, sm.redf[i], sm.redi[i]);
  __syncthreads();
  if (ii == 0x7fffffff) ii = 0;  // all NaN: Greedy keeps index 0
  return ii;
}

__device__ bool block_any(bool p, SampleSmem& sm) {
  __syncthreads();
  if (threadIdx.x == 0) sm.misc[0] = 0;
  __syncthreads();
  if (p) sm.misc[0] = 1;
  __syncthreads();
  const bool r = sm.misc[0] != 0;
  __syncthreads();
  return r;
}

// k-th largest value (duplicates counted) of v[0..V): sorted ascending, index V-k.
__device__ float kth_largest(const float* __restrict__ v, int V, int k, SampleSmem& sm) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kST) sm.hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += kST) {
      const uint32_t key = order_key(v[i]);
      if ((key & mask) == prefix) atomicAdd(&sm.hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const int c0 = sm.hist[4 * lane], c1 = sm.hist[4 * lane + 1], c2 = sm.hist[4 * lane + 2],
                c3 = sm.hist[4 * lane + 3];
      const int own = c0 + c1 + c2 + c3;
      int suf = own;  // count in bins >= 4*lane
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_down(suf, o, 64);
        if (lane + o < 64) suf += t;
      }
      const int above = suf - own;  // bins >= 4*lane+4
      if (above < remaining && remaining <= suf) {
        int cum = above, dg = 4 * lane + 3;
        const int cs[4] = {c0, c1, c2, c3};
        for (int q = 3; q >= 0; q--) {
          if (cum + cs[q] >= remaining) {
            dg = 4 * lane + q;
            break;
          }
          cum += cs[q];
        }
        sm.misc[1] = dg;
        sm.misc[2] = remaining - cum;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sm.misc[1] << shift;
    mask |= 255u << shift;
    remaining = sm.misc[2];
    __syncthreads();
  }
  return key_to_float(prefix);
}

// Exclusive scan of one int per thread (thread order); returns the total.
__device__ int block_exclusive_scan(int v, int& excl, SampleSmem& sm) {
  sm.scan[threadIdx.x] = v;
  __syncthreads();
  for (int o = 1; o < kST; o <<= 1) {
    const int t = (threadIdx.x >= (unsigned)o) ? sm.scan[threadIdx.x - o] : 0;
    __syncthreads();
    sm.scan[threadIdx.x] += t;
    __syncthreads();
  }
  excl = sm.scan[threadIdx.x] - v;
  const int total = sm.scan[kST - 1];
  __syncthreads();
  return total;
}

}  // namespace

// ---- register sampler for V <= kST * kRowV (the configurations' 16384) -------------
// The same steps and arithmetic as k_sample, with thread t holding logits
// 16t .. 16t+15 in registers (index order = thread order, then register order):
// bans and penalties are applied from LDS bitmaps, reductions are wave DPP /
// shuffle steps plus one LDS exchange of the 16 wave results, the top-k threshold
// is a two-bits-per-pass radix select over register keys, and the top-k survivors'
// sequential sum and CDF walk run on one wave (expf in parallel, the fold in index
// order through readlane).  The all-vocabulary path keeps k_sample's per-thread
// partial sums folded in thread order.

// x lies in the candidate window [lo, max] (lo finite; -inf and NaN never do)
__device__ __forceinline__ bool dlt_ok(float x, float lo) { return x >= lo; }

// integer wave sum through DPP row shifts and a row broadcast, result in every lane
__device__ __forceinline__ int wave_sum_int_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row half mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row broadcast 15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row broadcast 31
  return __builtin_amdgcn_readlane(v, 63);
}

struct SampleRowSmem {
  uint32_t seen[kST * kRowV / 32];
  uint32_t ban[kST * kRowV / 32];
  float redf[2][kST / 64];
  int redi[2][kST / 64];
  int cntp[2][kST / 64][2];
  int wscan[kST / 64];
  uint32_t ckey[1024];
  int ladder[8][kST / 64];
  int surv[kSurvCap];
  float survv[kSurvCap];
  float part[kST];
  int misc[4];
};

// block max of one value per thread (all threads get it); slot alternates between calls
__device__ __forceinline__ float row_block_max(float v, SampleRowSmem& sm, int slot) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) sm.redf[slot][threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sm.redf[slot][0];
#pragma unroll
  for (int i = 1; i < kST / 64; i++) r = fmaxf(r, sm.redf[slot][i]);
  return r;
}

__device__ __forceinline__ int row_block_argmax(const float (&x)[kRowV], int V, SampleRowSmem& sm, int slot) {
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < kRowV; j++) {
    const int i = threadIdx.x * kRowV + j;
    if (i < V) argmax_merge(best, bi, x[j], i);
  }
  wave_argmax(best, bi);
  if ((threadIdx.x & 63) == 0) {
    sm.redf[slot][threadIdx.x >> 6] = best;
    sm.redi[slot][threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  float bv = sm.redf[slot][0];
  int ii = sm.redi[slot][0];
#pragma unroll
  for (int i = 1; i < kST / 64; i++) argmax_merge(bv, ii, sm.redf[slot][i], sm.redi[slot][i]);
  if (ii == 0x7fffffff) ii = 0;  // all NaN: Greedy keeps index 0
  return ii;
}

__global__ __launch_bounds__(kST) void k_sample_row(SampleArgs a) {
  __shared__ SampleRowSmem sm;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, V = a.V;
  const int n = *a.step;
  const float* lg = a.logits + (size_t)b * V;
  const int total = a.prompt_len + n;
  const int T = min(total, a.ctx);
  const int* hist = a.tokens + (size_t)b * a.tok_stride + (total - T);
  if (a.dump && n < a.max_new)
    for (int i = tid; i < V; i += kST) a.dump[((size_t)b * a.max_new + n) * V + i] = lg[i];
  float x[kRowV];
  if ((V & 3) == 0 && (reinterpret_cast<uintptr_t>(lg) & 15) == 0) {
    // 16-byte loads; groups past V load the last group and drop it (no branch around the loads)
#pragma unroll
    for (int q = 0; q < kRowV / 4; q++) {
      const int i = tid * kRowV + 4 * q;
      const float4 v = *reinterpret_cast<const float4*>(lg + min(i, V - 4));
      x[4 * q] = v.x;
      x[4 * q + 1] = v.y;
      x[4 * q + 2] = v.z;
      x[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kRowV; j++) x[j] = lg[min(tid * kRowV + j, V - 1)];
  }
#pragma unroll
  for (int j = 0; j < kRowV; j++)
    if (tid * kRowV + j >= V) x[j] = -INFINITY;
  const bool controls = (a.penalty != 1.f) || (a.ngram > 0);
  const bool sampling = a.temperature > 0.f;
  int result = 0;
  if (!controls && !sampling) {
    result = row_block_argmax(x, V, sm, 0);
  } else {
    if (a.penalty != 1.f) {  // Sampler.cs:117-127: each distinct id of the window once
      for (int i = tid; i < kST * kRowV / 32; i += kST) sm.seen[i] = 0;
      __syncthreads();
      for (int i = tid; i < T; i += kST) {
        const int t = hist[i];
        if ((unsigned)t < (unsigned)V) atomicOr(&sm.seen[t >> 5], 1u << (t & 31));
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kRowV; j++) {
        const int i = tid * kRowV + j;
        if ((sm.seen[i >> 5] >> (i & 31)) & 1u) x[j] = x[j] < 0.f ? x[j] * a.penalty : x[j] / a.penalty;
      }
    }
    if (a.ngram > 0 && T >= a.ngram - 1) {  // Sampler.cs:129-164
      for (int i = tid; i < kST * kRowV / 32; i += kST) sm.ban[i] = 0;
      __syncthreads();
      const int ng = a.ngram;
      if (ng == 1) {
        for (int i = tid; i < T; i += kST) {
          const int t = hist[i];
          if ((unsigned)t < (unsigned)V) atomicOr(&sm.ban[t >> 5], 1u << (t & 31));
        }
      } else {
        const int pre = ng - 1, suf = T - pre;
        for (int s0 = tid; s0 + ng <= T; s0 += kST) {
          bool match = true;
          for (int j = 0; j < pre; j++)
            if (hist[s0 + j] != hist[suf + j]) {
              match = false;
              break;
            }
          const int t = hist[s0 + pre];
          if (match && (unsigned)t < (unsigned)V) atomicOr(&sm.ban[t >> 5], 1u << (t & 31));
        }
      }
      __syncthreads();
      // all banned (or -inf): Sampler.cs:156-164 keeps the post-penalty logits
      int avail = 0;
#pragma unroll
      for (int j = 0; j < kRowV; j++) {
        const int i = tid * kRowV + j;
        if (i < V && !((sm.ban[i >> 5] >> (i & 31)) & 1u) && !(x[j] == -INFINITY)) avail = 1;
      }
      avail = __syncthreads_or(avail);
      if (avail) {
#pragma unroll
        for (int j = 0; j < kRowV; j++) {
          const int i = tid * kRowV + j;
          if ((sm.ban[i >> 5] >> (i & 31)) & 1u) x[j] = -INFINITY;
        }
      }
    }
    if (!sampling) {
      result = row_block_argmax(x, V, sm, 1);
    } else {
#pragma unroll
      for (int j = 0; j < kRowV; j++) x[j] = x[j] / a.temperature;
      const bool filt = a.top_k > 0 && a.top_k < V;
      float thr = -INFINITY;
      if (filt) {
        // k-th largest (duplicates counted) by a radix select on order keys,
        // two bits a pass; absent entries hold key 0, below every real key
        uint32_t key[kRowV];
#pragma unroll
        for (int j = 0; j < kRowV; j++) key[j] = (tid * kRowV + j < V) ? order_key(x[j]) : 0u;
        uint32_t prefix = 0;
        int rem = a.top_k;
        int nin = kST * kRowV;  // slots whose key matches the prefix (absent slots included)
        // the k-th largest key's digit among counts c1..c3 (digit 0 takes the rest)
        auto choose = [&](int t1, int t2, int t3) -> uint32_t {
          if (t3 >= rem) return nin = t3, 3u;
          rem -= t3;
          if (t2 >= rem) return nin = t2, 2u;
          rem -= t2;
          if (t1 >= rem) return nin = t1, 1u;
          rem -= t1;
          nin = nin - t1 - t2 - t3;
          return 0u;
        };
        int sh = 30;
        // Candidate window: with M the largest value, the first t of a ladder
        // for which [M - t, M] holds at least k values contains the k-th largest;
        // when it holds at most 1024 they are gathered for the wave-0 passes and
        // the block-wide passes are skipped (the selection stays exact).
        float lo = -INFINITY;
        {
          float lm = -INFINITY;
#pragma unroll
          for (int j = 0; j < kRowV; j++) lm = fmaxf(lm, x[j]);
          const float M = row_block_max(lm, sm, 1);
          if (M > -INFINITY && M < INFINITY) {
            int cl[8];
#pragma unroll
            for (int q = 0; q < 8; q++) cl[q] = 0;
            // window q is x >= M - 2^q / 8; the same lower bound gathers it below
            // (NaN and absent -inf entries are in no window)
#pragma unroll
            for (int j = 0; j < kRowV; j++) {
#pragma unroll
              for (int q = 0; q < 8; q++) cl[q] += dlt_ok(x[j], M - (float)(1 << q) * 0.125f) ? 1 : 0;
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
              cl[q] = wave_sum_int_dpp(cl[q]);
              if (lane == 0) sm.ladder[q][wv] = cl[q];
            }
            __syncthreads();
            int pick = -1;
            for (int q = 0; q < 8 && pick < 0; q++) {
              int tot = 0;
              for (int w2 = 0; w2 < kST / 64; w2++) tot += sm.ladder[q][w2];
              if (tot >= a.top_k) pick = tot <= 1024 ? q : 8;
            }
            if (pick >= 0 && pick < 8) lo = M - (float)(1 << pick) * 0.125f;
          }
        }
        if (lo > -INFINITY) {
          // gather the window's keys; the prefix starts empty and the wave passes do every bit
          int cnt = 0;
#pragma unroll
          for (int j = 0; j < kRowV; j++) cnt += (dlt_ok(x[j], lo)) ? 1 : 0;
          int incl = cnt;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
          }
          if (lane == 63) sm.wscan[wv] = incl;
          __syncthreads();
          int off = incl - cnt;
          nin = 0;
          for (int w2 = 0; w2 < kST / 64; w2++) {
            if (w2 < wv) off += sm.wscan[w2];
            nin += sm.wscan[w2];
          }
#pragma unroll
          for (int j = 0; j < kRowV; j++)
            if (dlt_ok(x[j], lo)) sm.ckey[off++] = key[j];
          __syncthreads();
        }
        // block-wide passes while many keys still match the prefix
        for (; lo == -INFINITY && sh >= 0 && nin > 1024; sh -= 2) {
          const uint32_t hm = sh == 30 ? 0u : (0xffffffffu << (sh + 2));
          // counts of digits 1 and 2 packed in 16-bit fields, digit 3 apart (a wave
          // counts at most 1024 and the block at most 16384 of each)
          int c12 = 0, c3 = 0;
#pragma unroll
          for (int j = 0; j < kRowV; j++) {
            const uint32_t d = (key[j] >> sh) & 3u;
            const bool in = (key[j] & hm) == prefix;
            c12 += (in && d == 1u) ? 1 : ((in && d == 2u) ? 0x10000 : 0);
            c3 += (in && d == 3u) ? 1 : 0;
          }
          c12 = wave_sum_int_dpp(c12);
          c3 = wave_sum_int_dpp(c3);
          const int slot = (sh >> 1) & 1;  // rewritten two passes later, after the next barrier
          if (lane == 0) {
            sm.cntp[slot][wv][0] = c12;
            sm.cntp[slot][wv][1] = c3;
          }
          __syncthreads();
          int t12 = 0, t3 = 0;
#pragma unroll
          for (int w2 = 0; w2 < kST / 64; w2++) {
            t12 += sm.cntp[slot][w2][0];
            t3 += sm.cntp[slot][w2][1];
          }
          const int t1 = t12 & 0xffff, t2 = (int)((uint32_t)t12 >> 16);
          prefix |= choose(t1, t2, t3) << sh;
        }
        if (sh >= 0 && lo == -INFINITY) {
          // at most 1024 keys match: gather them into LDS (any order) and finish
          // the remaining passes on wave 0 alone, without block barriers
          const uint32_t hm = sh == 30 ? 0u : (0xffffffffu << (sh + 2));
          int cnt = 0;
#pragma unroll
          for (int j = 0; j < kRowV; j++) cnt += (key[j] & hm) == prefix ? 1 : 0;
          int incl = cnt;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
          }
          if (lane == 63) sm.wscan[wv] = incl;
          __syncthreads();
          int off = incl - cnt;
          for (int w2 = 0; w2 < wv; w2++) off += sm.wscan[w2];
#pragma unroll
          for (int j = 0; j < kRowV; j++)
            if ((key[j] & hm) == prefix) sm.ckey[off++] = key[j];
          __syncthreads();
        }
        if (sh >= 0) {
          if (wv == 0) {
            constexpr int E = 1024 / 64;
            const int ne = (nin + 63) >> 6;  // filled key groups (uniform)
            uint32_t ck[E];
            bool ok[E];
            uint32_t kand = 0xffffffffu, kor = 0u;
#pragma unroll
            for (int e = 0; e < E; e++) {
              ok[e] = lane + 64 * e < nin;
              ck[e] = sm.ckey[min(lane + 64 * e, 1023)];
              if (ok[e]) {
                kand &= ck[e];
                kor |= ck[e];
              }
            }
            // bits every gathered key shares (below the prefix already fixed) are
            // the k-th largest's too: take them and start at the first digit that differs
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
              kand &= (uint32_t)__shfl_xor((int)kand, o, 64);
              kor |= (uint32_t)__shfl_xor((int)kor, o, 64);
            }
            const uint32_t diff = kand ^ kor;
            const uint32_t low = sh >= 30 ? 0xffffffffu : ((1u << (sh + 2)) - 1u);  // bits not yet fixed
            if (nin > 0) {
              const int top = diff & low ? 31 - __builtin_clz(diff & low) : -1;  // highest differing bit
              const int shd = top < 0 ? -2 : (top & ~1);                         // its 2-bit digit
              const uint32_t fixed = top < 0 ? low : (low & ~((1u << (shd + 2)) - 1u));
              prefix |= kand & fixed;
              sh = min(sh, shd);
            }
            for (; sh >= 0; sh -= 2) {
              const uint32_t hm2 = sh == 30 ? 0u : (0xffffffffu << (sh + 2));  // no 32-bit shift
              int c12 = 0, c3 = 0;
#pragma unroll
              for (int e = 0; e < E; e++) {
                if (e >= ne) break;
                const uint32_t d = (ck[e] >> sh) & 3u;
                const bool in = ok[e] && (ck[e] & hm2) == prefix;
                c12 += (in && d == 1u) ? 1 : ((in && d == 2u) ? 0x10000 : 0);
                c3 += (in && d == 3u) ? 1 : 0;
              }
              c12 = wave_sum_int_dpp(c12);
              c3 = wave_sum_int_dpp(c3);
              prefix |= choose(c12 & 0xffff, (int)((uint32_t)c12 >> 16), c3) << sh;
            }
            if (lane == 0) sm.misc[1] = (int)prefix;
          }
          __syncthreads();
          prefix = (uint32_t)sm.misc[1];
        }
        thr = key_to_float(prefix);
      }
      float p[kRowV];
      float lmx = -INFINITY;
#pragma unroll
      for (int j = 0; j < kRowV; j++) {
        p[j] = (tid * kRowV + j >= V || (filt && x[j] < thr)) ? -INFINITY : x[j];
        lmx = fmaxf(lmx, p[j]);
      }
      const float mx = row_block_max(lmx, sm, 0);
      const double u01 = a.uniforms ? a.uniforms[(size_t)b * a.max_new + n] : 0.0;
      int nsurv = 0;
      if (filt) {
        // survivors (x >= thr) in index order: per-thread counts, wave scan, wave offsets
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kRowV; j++) cnt += (tid * kRowV + j < V && x[j] >= thr) ? 1 : 0;
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int t = __shfl_up(incl, o, 64);
          if (lane >= o) incl += t;
        }
        if (lane == 63) sm.wscan[wv] = incl;
        __syncthreads();
        int before = 0;
        for (int w2 = 0; w2 < kST / 64; w2++) {
          const int c = sm.wscan[w2];
          if (w2 < wv) before += c;
          nsurv += c;
        }
        if (nsurv <= kSurvCap) {
          int off = before + incl - cnt;
#pragma unroll
          for (int j = 0; j < kRowV; j++)
            if (tid * kRowV + j < V && x[j] >= thr) {
              sm.surv[off] = tid * kRowV + j;
              sm.survv[off] = x[j];
              off++;
            }
        }
        __syncthreads();
      }
      if (filt && nsurv <= kSurvCap) {
        // exact reference order: the sum and the CDF walk over the survivors in
        // index order; wave 0 computes the exps in parallel and folds them in order
        if (wv == 0) {
          float sum = 0.f;
          for (int c0 = 0; c0 < nsurv; c0 += 64) {
            const float e = (c0 + lane < nsurv) ? expf(sm.survv[c0 + lane] - mx) : 0.f;
            const int m = min(64, nsurv - c0);
            for (int q = 0; q < m; q++) sum = sum + __shfl(e, q, 64);
          }
          const float u = (float)u01 * sum;
          float acc = 0.f;
          int r = V - 1;
          bool found = false;
          for (int c0 = 0; c0 < nsurv && !found; c0 += 64) {
            const float e = (c0 + lane < nsurv) ? expf(sm.survv[c0 + lane] - mx) : 0.f;
            const int m = min(64, nsurv - c0);
            for (int q = 0; q < m; q++) {
              acc = acc + __shfl(e, q, 64);
              if (u < acc) {
                r = sm.surv[c0 + q];
                found = true;
                break;
              }
            }
          }
          if (lane == 0) sm.misc[3] = r;
        }
        __syncthreads();
        result = sm.misc[3];
      } else {
        // all-vocabulary CDF: per-thread sequential partial sums combined in
        // thread order (rounding may differ from one sequential pass)
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < kRowV; j++)
          if (tid * kRowV + j < V) ls = ls + expf(p[j] - mx);
        sm.part[tid] = ls;
        __syncthreads();
        if (wv == 0) {
          // the same thread-order fold, one partial per readlane, keeping each
          // thread's exclusive prefix
          float run = 0.f;
          for (int c0 = 0; c0 < kST; c0 += 64) {
            const int v = __float_as_int(sm.part[c0 + lane]);
            float pre = 0.f;
#pragma unroll
            for (int q = 0; q < 64; q++) {
              pre = lane == q ? run : pre;
              run = run + __int_as_float(__builtin_amdgcn_readlane(v, q));
            }
            sm.part[c0 + lane] = pre;
          }
          if (lane == 0) {
            sm.misc[0] = __float_as_int(run);
            sm.misc[3] = 0x7fffffff;
          }
        }
        __syncthreads();
        const float u = (float)u01 * __int_as_float(sm.misc[0]);
        float acc = sm.part[tid];
        int cand = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < kRowV; j++) {
          if (tid * kRowV + j < V && cand == 0x7fffffff) {
            acc = acc + expf(p[j] - mx);
            if (u < acc) cand = tid * kRowV + j;
          }
        }
        if (cand != 0x7fffffff) atomicMin(&sm.misc[3], cand);
        __syncthreads();
        result = sm.misc[3] == 0x7fffffff ? V - 1 : sm.misc[3];
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (a.prompt_len + n < a.tok_stride) a.tokens[(size_t)b * a.tok_stride + a.prompt_len + n] = result;
    if (n < a.max_new) a.out_ids[(size_t)b * a.max_new + n] = result;
    if (a.out_counts[b] < 0 && a.eos >= 0 && result == a.eos) a.out_counts[b] = n + 1;
    __threadfence();
    const int prev = atomicAdd(a.done, 1);
    if (prev == a.B - 1) {  // last block: every block has read the step already
      *a.done = 0;
      *a.step = n + 1;
      __threadfence();
    }
  }
}

__global__ __launch_bounds__(kST) void k_sample(SampleArgs a) {
  __shared__ SampleSmem sm;
  const int b = blockIdx.x, tid = threadIdx.x, V = a.V;
  const int n = *a.step;
  const float* lg = a.logits + (size_t)b * V;
  float* w = a.work + (size_t)b * V;
  const int total = a.prompt_len + n;
  const int T = min(total, a.ctx);
  const int* hist = a.tokens + (size_t)b * a.tok_stride + (total - T);
  if (a.dump && n < a.max_new)
    for (int i = tid; i < V; i += kST) a.dump[((size_t)b * a.max_new + n) * V + i] = lg[i];
  const bool controls = (a.penalty != 1.f) || (a.ngram > 0);
  const bool sampling = a.temperature > 0.f;
  int result = 0;
  if (!controls && !sampling) {
    result = block_argmax(lg, V, sm);
  } else {
    for (int i = tid; i < V; i += kST) w[i] = lg[i];
    __syncthreads();
    if (a.penalty != 1.f) {  // Sampler.cs:117-127, each distinct id once
      for (int i = tid; i < kMaxVocab / 32; i += kST) sm.seen[i] = 0;
      __syncthreads();
      for (int i = tid; i < T; i += kST) {
        const int t = hist[i];
        if ((unsigned)t >= (unsigned)V) continue;
        const uint32_t bit = 1u << (t & 31);
        const uint32_t old = atomicOr(&sm.seen[t >> 5], bit);
        if (!(old & bit)) w[t] = w[t] < 0.f ? w[t] * a.penalty : w[t] / a.penalty;
      }
      __syncthreads();
    }
    if (a.ngram > 0 && T >= a.ngram - 1) {  // Sampler.cs:129-164
      for (int i = tid; i < kMaxVocab / 32; i += kST) sm.ban[i] = 0;
      __syncthreads();
      const int ng = a.ngram;
      if (ng == 1) {
        for (int i = tid; i < T; i += kST) {
          const int t = hist[i];
          if ((unsigned)t < (unsigned)V) atomicOr(&sm.ban[t >> 5], 1u << (t & 31));
        }
      } else {
        const int pre = ng - 1, suf = T - pre;
        for (int s0 = tid; s0 + ng <= T; s0 += kST) {
          bool match = true;
          for (int j = 0; j < pre; j++)
            if (hist[s0 + j] != hist[suf + j]) {
              match = false;
              break;
            }
          const int t = hist[s0 + pre];
          if (match && (unsigned)t < (unsigned)V) atomicOr(&sm.ban[t >> 5], 1u << (t & 31));
        }
      }
      __syncthreads();
      bool avail = false;
      for (int i = tid; i < V; i += kST) {
        const bool banned = (sm.ban[i >> 5] >> (i & 31)) & 1u;
        if (!banned && !(w[i] == -INFINITY)) avail = true;
      }
      if (block_any(avail, sm)) {
        for (int i = tid; i < V; i += kST)
          if ((sm.ban[i >> 5] >> (i & 31)) & 1u) w[i] = -INFINITY;
      }
      __syncthreads();
    }
    if (!sampling) {
      result = block_argmax(w, V, sm);
    } else {
      for (int i = tid; i < V; i += kST) w[i] = w[i] / a.temperature;
      __syncthreads();
      const bool filt = a.top_k > 0 && a.top_k < V;
      float thr = -INFINITY;
      if (filt) thr = kth_largest(w, V, a.top_k, sm);
      float mx = -INFINITY;
      for (int i = tid; i < V; i += kST) {
        const float p = (filt && w[i] < thr) ? -INFINITY : w[i];
        mx = fmaxf(mx, p);
      }
      mx = block_max<kST>(mx, sm.redf);
      const double u01 = a.uniforms ? a.uniforms[(size_t)b * a.max_new + n] : 0.0;
      // contiguous per-thread ranges keep index order for the scans below
      const int per = (V + kST - 1) / kST;
      const int i0 = min(V, tid * per), i1 = min(V, i0 + per);
      int nsurv = 0;
      if (filt) {
        int cnt = 0;
        for (int i = i0; i < i1; i++) cnt += (w[i] >= thr);
        int off;
        nsurv = block_exclusive_scan(cnt, off, sm);
        if (nsurv <= kSurvCap) {
          for (int i = i0; i < i1; i++)
            if (w[i] >= thr) sm.surv[off++] = i;
        }
        __syncthreads();
      }
      if (filt && nsurv <= kSurvCap) {
        // exact reference order: sum and CDF walk over survivors in index order
        if (tid == 0) {
          float sum = 0.f;
          for (int s = 0; s < nsurv; s++) sum = sum + expf(w[sm.surv[s]] - mx);
          const float u = (float)u01 * sum;
          float acc = 0.f;
          int r = V - 1;
          for (int s = 0; s < nsurv; s++) {
            acc = acc + expf(w[sm.surv[s]] - mx);
            if (u < acc) {
              r = sm.surv[s];
              break;
            }
          }
          sm.misc[3] = r;
        }
        __syncthreads();
        result = sm.misc[3];
      } else {
        // all-vocabulary CDF: per-thread sequential partial sums combined in
        // thread order (rounding may differ from one sequential pass)
        float ls = 0.f;
        for (int i = i0; i < i1; i++) {
          const float p = (filt && w[i] < thr) ? -INFINITY : w[i];
          ls = ls + expf(p - mx);
        }
        sm.redf[0] = 0.f;
        __syncthreads();
        float* fs = reinterpret_cast<float*>(sm.scan);
        fs[tid] = ls;
        __syncthreads();
        if (tid == 0) {
          float run = 0.f;
          for (int t = 0; t < kST; t++) {
            const float v = fs[t];
            fs[t] = run;
            run = run + v;
          }
          sm.redf[0] = run;
        }
        __syncthreads();
        const float sum = sm.redf[0];
        const float u = (float)u01 * sum;
        float acc = fs[tid];
        int cand = 0x7fffffff;
        for (int i = i0; i < i1; i++) {
          const float p = (filt && w[i] < thr) ? -INFINITY : w[i];
          acc = acc + expf(p - mx);
          if (u < acc) {
            cand = i;
            break;
          }
        }
        __syncthreads();
        if (tid == 0) sm.misc[3] = 0x7fffffff;
        __syncthreads();
        if (cand != 0x7fffffff) atomicMin(&sm.misc[3], cand);
        __syncthreads();
        result = sm.misc[3] == 0x7fffffff ? V - 1 : sm.misc[3];
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (a.prompt_len + n < a.tok_stride) a.tokens[(size_t)b * a.tok_stride + a.prompt_len + n] = result;
    if (n < a.max_new) a.out_ids[(size_t)b * a.max_new + n] = result;
    if (a.out_counts[b] < 0 && a.eos >= 0 && result == a.eos) a.out_counts[b] = n + 1;
    __threadfence();
    const int prev = atomicAdd(a.done, 1);
    if (prev == a.B - 1) {  // last block: every block has read the step already
      *a.done = 0;
      *a.step = n + 1;
      __threadfence();
    }
  }
}

#pragma clang fp contract(on)

// Plain device copy: 16-byte vector loads and stores over a grid-stride loop,
// then the byte tail.  Also the calibration kernel for HBM traffic counters.
__global__ void k_copy_bytes(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16,
                             const unsigned char* __restrict__ src_tail, unsigned char* __restrict__ dst_tail,
                             int tail) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
  if (blockIdx.x == 0 && (int)threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

// Sum of the 32-bit words of a buffer (mod 2^64): per-block partials.  Block b
// reads one contiguous chunk of the buffer (consecutive 4 KB per pass, eight
// 16-byte loads in flight per thread), so the kernel streams the buffer at the
// device's read bandwidth; integer addition makes the order immaterial.
__global__ __launch_bounds__(256) void k_checksum_part(const uint4* __restrict__ src, size_t n16,
                                                       const unsigned* __restrict__ tail, int ntail,
                                                       unsigned long long* __restrict__ part) {
  __shared__ unsigned long long red[256];
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = (size_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
  unsigned long long s = 0;
  size_t i = b0 + threadIdx.x;
  for (; i + 7 * 256 < b1; i += 8 * 256) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = src[i + u * 256];
#pragma unroll
    for (int u = 0; u < 8; u++) s += (unsigned long long)v[u].x + v[u].y + v[u].z + v[u].w;
  }
  for (; i < b1; i += 256) {
    const uint4 a = src[i];
    s += (unsigned long long)a.x + a.y + a.z + a.w;
  }
  if (blockIdx.x == 0 && (int)threadIdx.x < ntail) s += tail[threadIdx.x];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void k_checksum_final(const unsigned long long* __restrict__ part, int n,
                                                        unsigned long long* __restrict__ out) {
  __shared__ unsigned long long red[256];
  unsigned long long s = 0;
  for (int i = threadIdx.x; i < n; i += 256) s += part[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = red[0];
}

// out[i] = bf16(in[i]), nearest-even, over a grid-stride loop
__global__ void k_round_bf16(const float* __restrict__ in, bf16_t* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = bf16_rn(in[i]);
}

// ---------------------------------------------------------------------------
// launch wrappers
// ---------------------------------------------------------------------------
#define FH_CHECK_ARG(c) \
  do {                  \
    if (!(c)) return hipErrorInvalidValue; \
  } while (0)

template <typename WT>
hipError_t launch_embed(hipStream_t st, RowSrc src, int B, int T, const WT* tok, const WT* pos, int d, int V,
                              int ctx, float* x) {
  FH_CHECK_ARG(B > 0 && T > 0 && d > 0 && V > 0 && ctx > 0 && tok && pos && x && src.tokens && src.step);
  hipLaunchKernelGGL(k_embed<WT>, dim3(B * T), dim3(256), 0, st, src, T, tok, pos, d, V, ctx, x);
  return hipGetLastError();
}

hipError_t launch_layernorm(hipStream_t st, const float* in, int rows, int rows_per_seq, int seq_stride, int r_in0,
                            const float* w, const float* b, float* out, int d, float eps) {
  FH_CHECK_ARG(rows > 0 && rows_per_seq > 0 && d > 0 && in && w && b && out);
  hipLaunchKernelGGL(k_layernorm<float>, dim3(rows), dim3(256), 0, st, in, rows_per_seq, seq_stride, r_in0, w, b, out,
                     d, eps);
  return hipGetLastError();
}

hipError_t launch_layernorm_bf16(hipStream_t st, const float* in, int rows, const float* w, const float* b,
                                 bf16_t* out, int d, float eps) {
  FH_CHECK_ARG(rows > 0 && d > 0 && in && w && b && out);
  const dim3 g((rows + 3) / 4);
  if (d == 1024)
    hipLaunchKernelGGL(k_layernorm_rows_bf16<4>, g, dim3(256), 0, st, in, rows, w, b, out, eps);
  else if (d == 768)
    hipLaunchKernelGGL(k_layernorm_rows_bf16<3>, g, dim3(256), 0, st, in, rows, w, b, out, eps);
  else if (d == 512)
    hipLaunchKernelGGL(k_layernorm_rows_bf16<2>, g, dim3(256), 0, st, in, rows, w, b, out, eps);
  else if (d == 256)
    hipLaunchKernelGGL(k_layernorm_rows_bf16<1>, g, dim3(256), 0, st, in, rows, w, b, out, eps);
  else
    hipLaunchKernelGGL(k_layernorm<bf16_t>, dim3(rows), dim3(256), 0, st, in, rows, 0, 0, w, b, out, d, eps);
  return hipGetLastError();
}

template <typename WT>
hipError_t launch_gemv_splitk(hipStream_t st, const float* x, int M, int K, const WT* W, int N, float* part,
                              int splits, int* used_splits) {
  constexpr int VEC = 16 / sizeof(WT);
  constexpr int TILE = 64 * VEC;
  FH_CHECK_ARG(M >= 1 && M <= 4 && K > 0 && N > 0 && N % VEC == 0 && splits >= 1 && x && W && part);
  const int kchunk = (K + splits - 1) / splits;
  const int S = (K + kchunk - 1) / kchunk;
  *used_splits = S;
  dim3 grid((N + TILE - 1) / TILE, S);
  if (M == 1)
    hipLaunchKernelGGL((k_gemv_splitk<WT, 1>), grid, dim3(256), 0, st, x, M, K, W, N, kchunk, part);
  else if (M == 2)
    hipLaunchKernelGGL((k_gemv_splitk<WT, 2>), grid, dim3(256), 0, st, x, M, K, W, N, kchunk, part);
  else
    hipLaunchKernelGGL((k_gemv_splitk<WT, 4>), grid, dim3(256), 0, st, x, M, K, W, N, kchunk, part);
  return hipGetLastError();
}

hipError_t launch_splitk_epilogue(hipStream_t st, const float* part, int splits, int M, int N, const float* bias,
                                  int epi, const float* res, float* y) {
  FH_CHECK_ARG(splits >= 1 && M > 0 && N > 0 && part && y);
  const size_t tot = (size_t)M * N;
  hipLaunchKernelGGL(k_splitk_epilogue, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, part, splits, M, N,
                     bias, epi, res, y);
  return hipGetLastError();
}

template <typename WT>
hipError_t launch_gemm(hipStream_t st, const float* a, int M, int K, const WT* W, int N, const float* bias, int epi,
                       const float* res, float* y) {
  FH_CHECK_ARG(M > 0 && K > 0 && N > 0 && a && W && y);
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  hipLaunchKernelGGL(k_gemm_tiled<WT>, grid, dim3(256), 0, st, a, M, K, W, N, bias, epi, res, y);
  return hipGetLastError();
}

template <typename IT>
hipError_t launch_gather_rows(hipStream_t st, const IT* src, int src_ld, int row0, int rstride, int rows, int d,
                              float* dst, int dst_ld) {
  FH_CHECK_ARG(rows > 0 && d > 0 && src_ld >= d && dst_ld >= d && row0 >= 0 && rstride >= 0 && src && dst);
  hipLaunchKernelGGL(k_gather_rows<IT>, dim3(rows), dim3(256), 0, st, src, src_ld, row0, rstride, d, dst, dst_ld);
  return hipGetLastError();
}

template <typename KT>
hipError_t launch_kv_store(hipStream_t st, RowSrc src, const float* qkv, int B, int T, int d, int H, int ctx,
                           KT* kcache, KT* vcache) {
  FH_CHECK_ARG(B > 0 && T > 0 && d > 0 && H > 0 && d % H == 0 && ctx > 0 && qkv && kcache && vcache);
  hipLaunchKernelGGL(k_kv_store<KT>, dim3(B * T), dim3(256), 0, st, src, qkv, T, d, H, ctx, kcache, vcache);
  return hipGetLastError();
}

template <typename KT>
hipError_t launch_attn_prefill(hipStream_t st, const float* qkv, int B, int T, int d, int H, int ctx,
                               const KT* kcache, const KT* vcache, float* o) {
  FH_CHECK_ARG(B > 0 && T > 0 && T <= ctx && H > 0 && d % H == 0 && d / H <= 128 && qkv && kcache && vcache && o);
  hipLaunchKernelGGL(k_attn_prefill<KT>, dim3(T, H, B), dim3(64), 0, st, qkv, T, d, H, ctx, kcache, vcache, o);
  return hipGetLastError();
}

template <typename KT>
hipError_t launch_attn_decode(hipStream_t st, RowSrc src, const float* qkv, int B, int d, int H, int ctx,
                              const KT* kcache, const KT* vcache, float* part, int chunk, float* o) {
  FH_CHECK_ARG(B > 0 && H > 0 && d % H == 0 && d / H <= 128 && chunk > 0 && qkv && kcache && vcache && part && o);
  const int maxc = (ctx + chunk - 1) / chunk;
  hipLaunchKernelGGL(k_attn_decode_part<KT>, dim3(maxc, H, B), dim3(64), 0, st, src, qkv, d, H, ctx, kcache, vcache,
                     part, chunk, maxc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_decode_combine, dim3(H, B), dim3(64), 0, st, src, d, H, ctx, part, chunk, maxc, o);
  return hipGetLastError();
}

hipError_t launch_attn_decode_combine(hipStream_t st, RowSrc src, int B, int d, int H, int ctx, const float* part,
                                      int chunk, int maxc, float* o) {
  FH_CHECK_ARG(B > 0 && H > 0 && d % H == 0 && d / H <= 128 && chunk > 0 && maxc > 0 && part && o);
  hipLaunchKernelGGL(k_attn_decode_combine, dim3(H, B), dim3(64), 0, st, src, d, H, ctx, part, chunk, maxc, o);
  return hipGetLastError();
}

template <typename WT>
hipError_t launch_head(hipStream_t st, const float* xn, int B, int d, const WT* E, int V, float* logits) {
  constexpr int VEC = 16 / sizeof(WT);
  FH_CHECK_ARG(B > 0 && d > 0 && d <= 1024 && d % VEC == 0 && V > 0 && xn && E && logits);
  const int blocks = min(1024, (V + 3) / 4);
  hipLaunchKernelGGL(k_head<WT>, dim3(blocks), dim3(256), 0, st, xn, B, d, E, V, logits);
  return hipGetLastError();
}

hipError_t launch_epilogue_ln(hipStream_t st, const float* part, int splits, int M, int N, const float* bias,
                              const float* res, float* y, const float* w, const float* b, float* out, float eps) {
  FH_CHECK_ARG(splits >= 1 && M > 0 && N > 0 && N <= 1024 && part && y && w && b && out &&
               (size_t)splits * M * N * 4 < 0x7fffffffu);
  hipLaunchKernelGGL(k_epilogue_ln, dim3(M), dim3(1024), 0, st, part, splits, M, N, bias, res, y, w, b, out, eps);
  return hipGetLastError();
}

template <typename KT>
hipError_t launch_epilogue_qkv(hipStream_t st, const float* part, int splits, int M, int d, const float* bias,
                               float* qkv, RowSrc src, int T, int H, int ctx, KT* kcache, KT* vcache) {
  FH_CHECK_ARG(splits >= 1 && M > 0 && d > 0 && H > 0 && d % H == 0 && T > 0 && M % T == 0 && ctx > 0 && part &&
               qkv && kcache && vcache && src.step);
  const size_t tot = (size_t)M * 3 * d;
  hipLaunchKernelGGL(k_epilogue_qkv<KT>, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, part, splits, M, d,
                     bias, qkv, src, T, H, ctx, kcache, vcache);
  return hipGetLastError();
}
template hipError_t launch_epilogue_qkv<float>(hipStream_t, const float*, int, int, int, const float*, float*, RowSrc,
                                               int, int, int, float*, float*);
template hipError_t launch_epilogue_qkv<bf16_t>(hipStream_t, const float*, int, int, int, const float*, float*,
                                                RowSrc, int, int, int, bf16_t*, bf16_t*);

hipError_t launch_round_bf16(hipStream_t st, const float* in, size_t n, bf16_t* out) {
  FH_CHECK_ARG(in && out);
  if (n == 0) return hipSuccess;
  const size_t want = (n + 255) / 256;
  const unsigned blocks = (unsigned)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(k_round_bf16, dim3(blocks), dim3(256), 0, st, in, out, n);
  return hipGetLastError();
}

hipError_t launch_copy(hipStream_t st, void* dst, const void* src, size_t bytes) {
  FH_CHECK_ARG(dst && src && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0);
  if (bytes == 0) return hipSuccess;
  const size_t n16 = bytes / 16;
  const int tail = (int)(bytes % 16);
  const size_t want = (n16 + 255) / 256;
  const unsigned blocks = (unsigned)(want < 8192 ? (want ? want : 1) : 8192);
  hipLaunchKernelGGL(k_copy_bytes, dim3(blocks), dim3(256), 0, st, static_cast<const uint4*>(src),
                     static_cast<uint4*>(dst), n16, static_cast<const unsigned char*>(src) + n16 * 16,
                     static_cast<unsigned char*>(dst) + n16 * 16, tail);
  return hipGetLastError();
}

hipError_t launch_checksum(hipStream_t st, const void* src, size_t bytes, unsigned long long* part, int nparts,
                           unsigned long long* out, hipEvent_t read_done) {
  FH_CHECK_ARG(src && part && out && nparts >= 1 && nparts <= kChecksumParts && ((uintptr_t)src % 16) == 0 &&
               bytes % 4 == 0);
  const size_t n16 = bytes / 16;
  const int ntail = (int)((bytes % 16) / 4);
  hipLaunchKernelGGL(k_checksum_part, dim3(nparts), dim3(256), 0, st, static_cast<const uint4*>(src), n16,
                     reinterpret_cast<const unsigned*>(static_cast<const char*>(src) + n16 * 16), ntail, part);
  if (read_done) (void)hipEventRecord(read_done, st);
  hipLaunchKernelGGL(k_checksum_final, dim3(1), dim3(256), 0, st, part, nparts, out);
  return hipGetLastError();
}

hipError_t launch_sample(hipStream_t st, const SampleArgs& a) {
  FH_CHECK_ARG(a.B > 0 && a.V > 0 && a.V <= kMaxVocab && a.logits && a.work && a.tokens && a.step && a.done &&
               a.out_ids && a.out_counts && a.max_new > 0);
  FH_CHECK_ARG(!(a.temperature > 0.f) || a.uniforms);
  if (a.V <= kST * kRowV)
    hipLaunchKernelGGL(k_sample_row, dim3(a.B), dim3(kST), 0, st, a);
  else
    hipLaunchKernelGGL(k_sample, dim3(a.B), dim3(kST), 0, st, a);
  return hipGetLastError();
}

template hipError_t launch_embed<float>(hipStream_t, RowSrc, int, int, const float*, const float*, int, int,
                                              int, float*);
template hipError_t launch_embed<bf16_t>(hipStream_t, RowSrc, int, int, const bf16_t*, const bf16_t*, int,
                                               int, int, float*);
template hipError_t launch_gemv_splitk<float>(hipStream_t, const float*, int, int, const float*, int, float*, int,
                                              int*);
template hipError_t launch_gemv_splitk<bf16_t>(hipStream_t, const float*, int, int, const bf16_t*, int, float*, int,
                                               int*);
template hipError_t launch_gemm<float>(hipStream_t, const float*, int, int, const float*, int, const float*, int,
                                       const float*, float*);
template hipError_t launch_gemm<bf16_t>(hipStream_t, const float*, int, int, const bf16_t*, int, const float*, int,
                                        const float*, float*);
template hipError_t launch_gather_rows<float>(hipStream_t, const float*, int, int, int, int, int, float*, int);
template hipError_t launch_gather_rows<bf16_t>(hipStream_t, const bf16_t*, int, int, int, int, int, float*, int);
template hipError_t launch_kv_store<float>(hipStream_t, RowSrc, const float*, int, int, int, int, int, float*,
                                           float*);
template hipError_t launch_kv_store<bf16_t>(hipStream_t, RowSrc, const float*, int, int, int, int, int, bf16_t*,
                                            bf16_t*);
template hipError_t launch_attn_prefill<float>(hipStream_t, const float*, int, int, int, int, int, const float*,
                                               const float*, float*);
template hipError_t launch_attn_prefill<bf16_t>(hipStream_t, const float*, int, int, int, int, int, const bf16_t*,
                                                const bf16_t*, float*);
template hipError_t launch_attn_decode<float>(hipStream_t, RowSrc, const float*, int, int, int, int, const float*,
                                              const float*, float*, int, float*);
template hipError_t launch_attn_decode<bf16_t>(hipStream_t, RowSrc, const float*, int, int, int, int, const bf16_t*,
                                               const bf16_t*, float*, int, float*);
template hipError_t launch_head<float>(hipStream_t, const float*, int, int, const float*, int, float*);
template hipError_t launch_head<bf16_t>(hipStream_t, const float*, int, int, const bf16_t*, int, float*);

}  // namespace fh
