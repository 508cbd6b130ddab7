// ops.hip -- the op-level ITensorBackend contract on device buffers.
//
// ITensorBackend (src/LLM.Core/Tensor/ITensorBackend.cs:18-266) is the
// reference's per-op plug-in seam: row-major fp32 tensors, explicit shapes,
// `accumulate` meaning +=, host index arrays uploaded per call.  These entry
// points implement every method of it (forward, backward, optimizer and the
// reductions) on device pointers, ordered on the context's stream; only the
// calls that return host values (the cross-entropy loss, the loss
// accumulation's end, the sums of squares) wait for the device.  The residency
// contract (InvalidateDeviceCache / EnsureHostCurrent) lives in the host
// mirror, which owns the device copies of its tensors.
//
// The kernels are the straightforward HBM-bound forms: grid-stride elementwise
// loops, one block per row for the row reductions, column sums in fixed
// row-chunk order, a 64x64 LDS-tiled FMA kernel for the (batched) matmuls with
// the large plain NN product on the MFMA GEMM.  Results follow CpuBackend
// within the reference's own GPU-contract tolerances (GpuBackendTests.cs:23-24:
// 1e-4 forward, 1e-2 backward); the gathers, copies, masks and the embedding
// scatter-add (which adds each index's rows in ascending position, as the CPU
// loop does) are exact.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "common.hpp"
#include "../../include/forge_hip.h"
#include "kernels.hpp"

namespace fh {

int set_error(int code, const char* msg);
hipStream_t context_stream(fh_context* c);
int context_device(fh_context* c);
struct OpsState;
OpsState*& context_ops(fh_context* c);

namespace {

constexpr int kT = 256;

__device__ __forceinline__ float ops_block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float ops_block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + kT - 1) / kT, 65536); }

// ---- matmuls: y[s] (+)= op(a[s]) @ op(b[s]), 64x64 tiles, k steps of 16 ------------
// MODE 0 NN (a [M,K], b [K,N]), 1 NT (b [N,K]), 2 TN (a [K,M]).
template <int MODE>
__global__ __launch_bounds__(256) void k_matmul(const float* __restrict__ a, const float* __restrict__ b,
                                                float* __restrict__ y, int M, int K, int N, int acc) {
  __shared__ float As[16][65];
  __shared__ float Bs[16][65];
  const int s = blockIdx.z;
  a += (size_t)s * M * K;
  b += (size_t)s * K * N;
  y += (size_t)s * M * N;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float c[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 1024; i += 256) {
      // A tile [16 k][64 m], B tile [16 k][64 n]
      int kk, mm;
      if (MODE == 2) {
        kk = i / 64, mm = i % 64;  // a[k][m]: m contiguous
      } else {
        mm = i / 16, kk = i % 16;  // a[m][k]: k contiguous
      }
      const int gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < M && gk < K) ? (MODE == 2 ? a[(size_t)gk * M + gm] : a[(size_t)gm * K + gk]) : 0.f;
      int kb, nn;
      if (MODE == 1) {
        nn = i / 16, kb = i % 16;  // b[n][k]
      } else {
        kb = i / 64, nn = i % 64;  // b[k][n]
      }
      const int gn = n0 + nn, gk2 = k0 + kb;
      Bs[kb][nn] = (gn < N && gk2 < K) ? (MODE == 1 ? b[(size_t)gn * K + gk2] : b[(size_t)gk2 * N + gn]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) av[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) c[i][j] = fmaf(av[i], bv[j], c[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + ty + 16 * i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + tx + 16 * j;
      if (n >= N) continue;
      float& o = y[(size_t)m * N + n];
      o = acc ? o + c[i][j] : c[i][j];
    }
  }
}

// ---- head packing (PackHeads / UnpackHeads, CpuBackend.cs:225-262) ----------------
__global__ void k_pack_heads(const float* __restrict__ src, int src_cols, float* __restrict__ dst, int batch, int T,
                             int H, int hd, int col_base, int unpack) {
  const size_t n = (size_t)batch * H * T * hd;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int e = (int)(i % hd);
    const size_t row = i / hd;  // slot-packed row (q*H + h)*T + t
    const int t = (int)(row % T), h = (int)((row / T) % H), q = (int)(row / ((size_t)T * H));
    const size_t wide = (size_t)(q * T + t) * src_cols + col_base + h * hd + e;
    if (unpack)
      dst[wide] = src[i];
    else
      dst[i] = src[wide];
  }
}

// ---- elementwise and row kernels -----------------------------------------------------
__global__ void k_add_bias(float* __restrict__ y, const float* __restrict__ bias, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = y[i] + bias[i % cols];
}

__global__ void k_add_in_place(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = dst[i] + src[i];
}

__global__ void k_scale(float* __restrict__ x, size_t n, float f) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    x[i] = x[i] * f;
}

__global__ void k_copy_block(const float* __restrict__ src, int src_cols, float* __restrict__ dst, int dst_cols,
                             int src_row, int src_col, int dst_row, int dst_col, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / cols), c = (int)(i % cols);
    dst[(size_t)(dst_row + r) * dst_cols + dst_col + c] = src[(size_t)(src_row + r) * src_cols + src_col + c];
  }
}

__global__ __launch_bounds__(256) void k_transpose_f32(const float* __restrict__ x, float* __restrict__ out, int rows,
                                                       int cols) {
  __shared__ float tile[32][33];
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8)
    if (r0 + i < rows && c0 + tx < cols) tile[i][tx] = x[(size_t)(r0 + i) * cols + c0 + tx];
  __syncthreads();
  for (int i = ty; i < 32; i += 8)
    if (c0 + i < cols && r0 + tx < rows) out[(size_t)(c0 + i) * rows + r0 + tx] = tile[tx][i];
}

// Column sums over a chunk of rows: sums[chunk][c] = sum of rows in the chunk, in
// row order.  With one chunk the kernel adds straight into dst (dst[c] + rows in
// order, the CPU's sequence); otherwise k_sum_chunks adds the chunks in order.
constexpr int kRowChunk = 256;
// KIND 0: plain column sums of y (SumRows).  KIND 1: LayerNorm's dW and dB
// (sums of dOut * xhat and of dOut) into dst and dst2.
template <int KIND>
__global__ void k_col_sums(const float* __restrict__ y, const float* __restrict__ x, const float* __restrict__ mean,
                           const float* __restrict__ rstd, int rows, int cols, float* __restrict__ dst,
                           float* __restrict__ dst2, float* __restrict__ part, int chunks) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const int r0 = blockIdx.y * kRowChunk, r1 = min(rows, r0 + kRowChunk);
  float s = chunks == 1 ? dst[c] : 0.f;
  float s2 = (KIND == 1 && chunks == 1) ? dst2[c] : 0.f;
  for (int r = r0; r < r1; r++) {
    const float d = y[(size_t)r * cols + c];
    if (KIND == 1) {
      const float xhat = (x[(size_t)r * cols + c] - mean[r]) * rstd[r];
      s = s + d * xhat;
      s2 = s2 + d;
    } else {
      s = s + d;
    }
  }
  if (chunks == 1) {
    dst[c] = s;
    if (KIND == 1) dst2[c] = s2;
  } else {
    part[(size_t)blockIdx.y * cols + c] = s;
    if (KIND == 1) part[((size_t)chunks + blockIdx.y) * cols + c] = s2;
  }
}

__global__ void k_sum_chunks(const float* __restrict__ part, int chunks, int cols, float* __restrict__ dst) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int k = 0; k < chunks; k++) s = s + part[(size_t)k * cols + c];
  dst[c] = dst[c] + s;
}

// ---- LayerNorm (CpuBackend.cs:377-430), one block per row ------------------------------
__global__ __launch_bounds__(256) void k_ln_forward(const float* __restrict__ x, const float* __restrict__ w,
                                                    const float* __restrict__ b, float* __restrict__ out,
                                                    float* __restrict__ mean, float* __restrict__ rstd, int cols,
                                                    float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* xr = x + (size_t)r * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) s += xr[c];
  const float mu = ops_block_sum(s, red) / (float)cols;
  float v = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float dd = xr[c] - mu;
    v += dd * dd;
  }
  const float rs = 1.f / sqrtf(ops_block_sum(v, red) / (float)cols + eps);
  if (threadIdx.x == 0) {
    mean[r] = mu;
    rstd[r] = rs;
  }
  for (int c = threadIdx.x; c < cols; c += 256) out[(size_t)r * cols + c] = (xr[c] - mu) * rs * w[c] + b[c];
}

__global__ __launch_bounds__(256) void k_ln_backward_dx(const float* __restrict__ dout, const float* __restrict__ x,
                                                        const float* __restrict__ w, const float* __restrict__ mean,
                                                        const float* __restrict__ rstd, float* __restrict__ dx,
                                                        int cols) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* dr = dout + (size_t)r * cols;
  const float* xr = x + (size_t)r * cols;
  const float mu = mean[r], rs = rstd[r];
  float s1 = 0.f, s2 = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float xhat = (xr[c] - mu) * rs, dxhat = dr[c] * w[c];
    s1 += dxhat;
    s2 += dxhat * xhat;
  }
  const float inv_n = 1.f / (float)cols;
  const float m1 = ops_block_sum(s1, red) * inv_n;
  const float m2 = ops_block_sum(s2, red) * inv_n;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float xhat = (xr[c] - mu) * rs, dxhat = dr[c] * w[c];
    dx[(size_t)r * cols + c] = rs * (dxhat - m1 - xhat * m2);
  }
}

// ---- softmax (CpuBackend.cs:446-473; ITensorBackend.cs:117-130) ----------------------
// In place; with causal != 0 row r is query r % T of a packed [T,T] block: its
// keys past the query become -inf after the scale (Scale, CausalMask, Softmax).
__global__ __launch_bounds__(256) void k_softmax_rows(float* __restrict__ x, int cols, float scale, int causal) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  float* row = x + (size_t)r * cols;
  const int lim = causal ? r % cols : cols - 1;  // last unmasked column
  float mx = -INFINITY;
  for (int c = threadIdx.x; c <= lim; c += 256) mx = fmaxf(mx, row[c] * scale);
  mx = ops_block_max(mx, red);
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float e = c <= lim ? expf(row[c] * scale - mx) : 0.f;
    row[c] = e;
    s += e;
  }
  const float inv = 1.f / ops_block_sum(s, red);
  for (int c = threadIdx.x; c < cols; c += 256) row[c] = row[c] * inv;
}

__global__ __launch_bounds__(256) void k_softmax_backward(const float* __restrict__ dout, const float* __restrict__ sm,
                                                          float* __restrict__ dx, int cols, float scale) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* dr = dout + (size_t)r * cols;
  const float* sr = sm + (size_t)r * cols;
  float d = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) d += dr[c] * sr[c];
  const float dot = ops_block_sum(d, red);
  for (int c = threadIdx.x; c < cols; c += 256) dx[(size_t)r * cols + c] = sr[c] * (dr[c] - dot) * scale;
}

// ---- GELU (CpuBackend.cs:477-514) ------------------------------------------------------
__device__ __forceinline__ float gelu_c() { return 0.7978845238685608f; }  // MathF.Sqrt(2f / MathF.PI)

__global__ void k_gelu_forward(const float* __restrict__ x, float* __restrict__ out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = gelu_tanh(x[i]);
}

__global__ void k_gelu_backward(const float* __restrict__ dout, const float* __restrict__ x, float* __restrict__ dx,
                                size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    const float u = gelu_c() * (v + 0.044715f * v * v * v);
    const float t = tanhf(u);
    const float du = gelu_c() * (1.f + 3.f * 0.044715f * v * v);
    dx[i] = dout[i] * 0.5f * (1.f + t + v * (1.f - t * t) * du);
  }
}

// ---- embedding (CpuBackend.cs:518-543) ----------------------------------------------------
__global__ void k_embedding_forward(const float* __restrict__ table, const int* __restrict__ idx,
                                    float* __restrict__ out, int D) {
  const int t = blockIdx.x;
  const float* src = table + (size_t)idx[t] * D;
  for (int c = threadIdx.x; c < D; c += blockDim.x) out[(size_t)t * D + c] = src[c];
}

// dTable[id] += dOut[t] for the positions t of each distinct id, ascending:
// uniq[u] is the id, pos[start[u] .. start[u+1]) its positions in order.
__global__ void k_embedding_backward(const float* __restrict__ dout, const int* __restrict__ uniq,
                                     const int* __restrict__ start, const int* __restrict__ pos,
                                     float* __restrict__ dtable, int D) {
  const int u = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= D) return;
  float* row = dtable + (size_t)uniq[u] * D;
  float s = row[c];
  for (int k = start[u]; k < start[u + 1]; k++) s = s + dout[(size_t)pos[k] * D + c];
  row[c] = s;
}

// ---- causal mask (CpuBackend.cs:551-557) ----------------------------------------------------
__global__ void k_causal_mask(float* __restrict__ s, size_t n, int T) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(i % T), q = (int)((i / T) % T);
    if (j > q) s[i] = -INFINITY;
  }
}

// ---- cross-entropy (CpuBackend.cs:594-644) --------------------------------------------------
// One block per position: probs (may alias logits) and the position's negative
// log-likelihood (0 when ignored).
__global__ __launch_bounds__(256) void k_ce_forward(const float* logits, const int* __restrict__ targets, float* probs,
                                                    int V, int ignore, float* __restrict__ nll) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* lr = logits + (size_t)t * V;
  float* pr = probs + (size_t)t * V;
  const int tg = targets[t];
  const bool ignored = tg == ignore;
  const float tl = ignored ? 0.f : lr[tg];
  float mx = -INFINITY;
  for (int v = threadIdx.x; v < V; v += 256) mx = fmaxf(mx, lr[v]);
  mx = ops_block_max(mx, red);  // every read of the row is done before the first write
  float s = 0.f;
  for (int v = threadIdx.x; v < V; v += 256) {
    const float e = expf(lr[v] - mx);
    pr[v] = e;
    s += e;
  }
  const float sum = ops_block_sum(s, red);
  const float inv = 1.f / sum;
  for (int v = threadIdx.x; v < V; v += 256) pr[v] = pr[v] * inv;
  if (threadIdx.x == 0) nll[t] = ignored ? 0.f : logf(sum) + mx - tl;
}

// acc (double, device) += sum of the T per-position terms, in position order
__global__ void k_ce_accumulate(const float* __restrict__ nll, int T, double* __restrict__ acc) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float s = 0.f;
  for (int t = 0; t < T; t++) s = s + nll[t];
  acc[0] += (double)s;
}

__global__ void k_ce_backward(const float* probs, const int* __restrict__ targets, float* dl, int V, int ignore,
                              float scale, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / V), v = (int)(i % V);
    const int tg = targets[t];
    float g = 0.f;
    if (tg != ignore) {
      g = probs[i] * scale;
      if (v == tg) g = g - scale;
    }
    dl[i] = g;
  }
}

// ---- sums of squares and AdamW (ITensorBackend.cs:214-265) ---------------------------------
// per-block double partials of sum x^2; the final pass adds the partials in order
__global__ __launch_bounds__(256) void k_sumsq_partials(const float* __restrict__ x, size_t n,
                                                        double* __restrict__ part) {
  __shared__ double red[256];
  double s = 0;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    s += (double)x[i] * x[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ void k_sum_doubles(const double* __restrict__ part, int n, double* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  double s = 0;
  for (int i = 0; i < n; i++) s += part[i];
  out[0] = s;
}

__global__ void k_adamw(float* __restrict__ w, const float* __restrict__ g, float* __restrict__ m,
                        float* __restrict__ v, size_t n, float lr, float b1, float b2, float eps, float wd, float bc1,
                        float bc2, int decay) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float gi = g[i];
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    float wi = w[i];
    if (decay) wi = wi - lr * wd * wi;
    const float mh = mi / bc1, vh = vi / bc2;
    w[i] = wi - lr * mh / (sqrtf(vh) + eps);
  }
}

}  // namespace

// Per-context state of the op entry points: device scratch for uploaded index
// arrays and reduction partials, and the loss accumulation.
struct OpsState {
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  double* acc = nullptr;  // device loss accumulator + a result slot
  bool accumulating = false;
  long long accumulated_targets = 0;
};

void ops_state_free(OpsState* o) {
  if (!o) return;
  if (o->scratch) (void)hipFree(o->scratch);
  if (o->acc) (void)hipFree(o->acc);
  delete o;
}

}  // namespace fh

using namespace fh;

namespace {

int set_err(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_error(code, buf);
}

#define HIP_TRY(expr)                                                                                         \
  do {                                                                                                        \
    hipError_t e_ = (expr);                                                                                   \
    if (e_ != hipSuccess)                                                                                     \
      return set_err(e_ == hipErrorOutOfMemory ? FH_ERR_OOM : FH_ERR_HIP, "%s failed: %s", #expr,            \
                     hipGetErrorString(e_));                                                                  \
  } while (0)

#define FH_TRY(expr)            \
  do {                          \
    int r_ = (expr);            \
    if (r_ != FH_OK) return r_; \
  } while (0)

int ops_begin(fh_context* c, OpsState** out) {
  if (!c) return set_err(FH_ERR_INVALID, "null context");
  HIP_TRY(hipSetDevice(context_device(c)));
  OpsState*& o = context_ops(c);
  if (!o) {
    o = new OpsState();
    if (hipMalloc(&o->acc, 2 * sizeof(double)) != hipSuccess) {
      delete o;
      o = nullptr;
      return set_err(FH_ERR_OOM, "allocating the loss accumulator failed");
    }
  }
  *out = o;
  return FH_OK;
}

// device scratch of at least `bytes` (the previous contents are not kept)
int ops_scratch(fh_context* c, OpsState* o, size_t bytes, void** p) {
  if (bytes > o->scratch_bytes) {
    HIP_TRY(hipStreamSynchronize(context_stream(c)));  // earlier kernels may still read the old scratch
    if (o->scratch) (void)hipFree(o->scratch);
    o->scratch = nullptr;
    o->scratch_bytes = 0;
    const size_t nb = std::max<size_t>(bytes, 1 << 16);
    if (hipMalloc(&o->scratch, nb) != hipSuccess) return set_err(FH_ERR_OOM, "allocating %zu bytes of scratch", nb);
    o->scratch_bytes = nb;
  }
  *p = o->scratch;
  return FH_OK;
}

int op_launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_err(FH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return FH_OK;
}

#define OPS_PROLOGUE(c)    \
  OpsState* ops_ = nullptr; \
  FH_TRY(ops_begin((c), &ops_));                \
  hipStream_t st_ = context_stream(c);          \
  (void)ops_;                                   \
  (void)st_

#define OPS_ARG(cond, ...) \
  if (!(cond)) return set_err(FH_ERR_INVALID, __VA_ARGS__)

int upload_ints(fh_context* c, OpsState* o, const int32_t* host, size_t n, int** dev) {
  void* p = nullptr;
  FH_TRY(ops_scratch(c, o, n * sizeof(int32_t), &p));
  // synchronous: the caller's array may go away as soon as the entry point returns
  HIP_TRY(hipMemcpyAsync(p, host, n * sizeof(int32_t), hipMemcpyHostToDevice, context_stream(c)));
  HIP_TRY(hipStreamSynchronize(context_stream(c)));
  *dev = static_cast<int*>(p);
  return FH_OK;
}

int matmul_common(fh_context* c, int mode, const void* a, const void* b, void* y, int slots, int M, int K, int N,
                  int acc) {
  OPS_PROLOGUE(c);
  OPS_ARG(a && b && y, "null buffer");
  OPS_ARG(slots > 0 && slots <= 65535 && M > 0 && K > 0 && N > 0, "slots (at most 65535), M, K and N must be positive");
  if (mode == 0 && slots == 1 && K % 32 == 0 && (size_t)M * K * N >= ((size_t)1 << 24))
    return fh_matmul_nn(c, a, b, y, M, K, N, FH_DTYPE_F32, acc);  // the MFMA GEMM
  dim3 grid((N + 63) / 64, (M + 63) / 64, slots);
  const float* fa = static_cast<const float*>(a);
  const float* fb = static_cast<const float*>(b);
  float* fy = static_cast<float*>(y);
  if (mode == 0)
    hipLaunchKernelGGL(k_matmul<0>, grid, dim3(256), 0, st_, fa, fb, fy, M, K, N, acc);
  else if (mode == 1)
    hipLaunchKernelGGL(k_matmul<1>, grid, dim3(256), 0, st_, fa, fb, fy, M, K, N, acc);
  else
    hipLaunchKernelGGL(k_matmul<2>, grid, dim3(256), 0, st_, fa, fb, fy, M, K, N, acc);
  return op_launched("matmul");
}

int softmax_common(fh_context* c, void* x, int rows, int cols, float scale, int causal) {
  OPS_PROLOGUE(c);
  OPS_ARG(x, "null buffer");
  OPS_ARG(rows > 0 && cols > 0, "rows and cols must be positive");
  hipLaunchKernelGGL(k_softmax_rows, dim3(rows), dim3(256), 0, st_, static_cast<float*>(x), cols, scale, causal);
  return op_launched("softmax");
}

int sumsq_partials(hipStream_t st, const float* x, size_t n, double* part, int* blocks) {
  const int nb = (int)std::min<size_t>(256, std::max<size_t>(1, (n + 255) / 256));
  hipLaunchKernelGGL(k_sumsq_partials, dim3(nb), dim3(256), 0, st, x, n, part);
  *blocks = nb;
  return op_launched("sum of squares");
}

}  // namespace

extern "C" {

int fh_op_matmul_nn(fh_context* c, const void* a, const void* b, void* y, int slots, int M, int K, int N, int acc) {
  return matmul_common(c, 0, a, b, y, slots, M, K, N, acc);
}
int fh_op_matmul_nt(fh_context* c, const void* a, const void* b, void* y, int slots, int M, int K, int N, int acc) {
  return matmul_common(c, 1, a, b, y, slots, M, K, N, acc);
}
int fh_op_matmul_tn(fh_context* c, const void* a, const void* b, void* y, int slots, int M, int K, int N, int acc) {
  return matmul_common(c, 2, a, b, y, slots, M, K, N, acc);
}

int fh_op_pack_heads(fh_context* c, const void* src, int src_cols, void* dst, int batch, int T, int n_heads,
                     int head_dim, int col_base) {
  OPS_PROLOGUE(c);
  OPS_ARG(src && dst, "null buffer");
  OPS_ARG(batch > 0 && T > 0 && n_heads > 0 && head_dim > 0 && col_base >= 0 &&
              col_base + n_heads * head_dim <= src_cols,
          "head slices outside the source rows");
  const size_t n = (size_t)batch * n_heads * T * head_dim;
  hipLaunchKernelGGL(k_pack_heads, dim3(grid_for(n)), dim3(kT), 0, st_, static_cast<const float*>(src), src_cols,
                     static_cast<float*>(dst), batch, T, n_heads, head_dim, col_base, 0);
  return op_launched("pack heads");
}

int fh_op_unpack_heads(fh_context* c, const void* src, void* dst, int dst_cols, int batch, int T, int n_heads,
                       int head_dim, int col_base) {
  OPS_PROLOGUE(c);
  OPS_ARG(src && dst, "null buffer");
  OPS_ARG(batch > 0 && T > 0 && n_heads > 0 && head_dim > 0 && col_base >= 0 &&
              col_base + n_heads * head_dim <= dst_cols,
          "head slices outside the destination rows");
  const size_t n = (size_t)batch * n_heads * T * head_dim;
  hipLaunchKernelGGL(k_pack_heads, dim3(grid_for(n)), dim3(kT), 0, st_, static_cast<const float*>(src), dst_cols,
                     static_cast<float*>(dst), batch, T, n_heads, head_dim, col_base, 1);
  return op_launched("unpack heads");
}

int fh_op_add_bias(fh_context* c, void* y, const void* bias, int rows, int cols) {
  OPS_PROLOGUE(c);
  OPS_ARG(y && bias && rows > 0 && cols > 0, "bad arguments");
  const size_t n = (size_t)rows * cols;
  hipLaunchKernelGGL(k_add_bias, dim3(grid_for(n)), dim3(kT), 0, st_, static_cast<float*>(y),
                     static_cast<const float*>(bias), rows, cols);
  return op_launched("add bias");
}

int fh_op_sum_rows(fh_context* c, const void* dy, void* dbias, int rows, int cols) {
  OPS_PROLOGUE(c);
  OPS_ARG(dy && dbias && rows > 0 && cols > 0, "bad arguments");
  const int chunks = (rows + kRowChunk - 1) / kRowChunk;
  float* part = nullptr;
  if (chunks > 1) {
    void* p = nullptr;
    FH_TRY(ops_scratch(c, ops_, (size_t)chunks * cols * sizeof(float), &p));
    part = static_cast<float*>(p);
  }
  hipLaunchKernelGGL(k_col_sums<0>, dim3((cols + 255) / 256, chunks), dim3(256), 0, st_,
                     static_cast<const float*>(dy), nullptr, nullptr, nullptr, rows, cols, static_cast<float*>(dbias),
                     nullptr, part, chunks);
  if (chunks > 1)
    hipLaunchKernelGGL(k_sum_chunks, dim3((cols + 255) / 256), dim3(256), 0, st_, part, chunks, cols,
                       static_cast<float*>(dbias));
  return op_launched("sum rows");
}

int fh_op_add_in_place(fh_context* c, void* dst, const void* src, int64_t n) {
  OPS_PROLOGUE(c);
  OPS_ARG(dst && src && n > 0, "bad arguments");
  hipLaunchKernelGGL(k_add_in_place, dim3(grid_for((size_t)n)), dim3(kT), 0, st_, static_cast<float*>(dst),
                     static_cast<const float*>(src), (size_t)n);
  return op_launched("add in place");
}

int fh_op_copy(fh_context* c, const void* src, void* dst, int64_t n) {
  OPS_PROLOGUE(c);
  OPS_ARG(dst && src && n >= 0, "bad arguments");
  if (n > 0) HIP_TRY(hipMemcpyAsync(dst, src, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice, st_));
  return FH_OK;
}

int fh_op_copy_block(fh_context* c, const void* src, int src_cols, void* dst, int dst_cols, int src_row, int src_col,
                     int dst_row, int dst_col, int rows, int cols) {
  OPS_PROLOGUE(c);
  OPS_ARG(src && dst && rows >= 0 && cols >= 0 && src_row >= 0 && src_col >= 0 && dst_row >= 0 && dst_col >= 0 &&
              src_col + cols <= src_cols && dst_col + cols <= dst_cols,
          "block outside the source or destination rows");
  const size_t n = (size_t)rows * cols;
  if (n == 0) return FH_OK;
  hipLaunchKernelGGL(k_copy_block, dim3(grid_for(n)), dim3(kT), 0, st_, static_cast<const float*>(src), src_cols,
                     static_cast<float*>(dst), dst_cols, src_row, src_col, dst_row, dst_col, rows, cols);
  return op_launched("copy block");
}

int fh_op_scale(fh_context* c, void* x, int64_t n, float factor) {
  OPS_PROLOGUE(c);
  OPS_ARG(x && n > 0, "bad arguments");
  hipLaunchKernelGGL(k_scale, dim3(grid_for((size_t)n)), dim3(kT), 0, st_, static_cast<float*>(x), (size_t)n, factor);
  return op_launched("scale");
}

int fh_op_transpose(fh_context* c, const void* x, void* out, int rows, int cols) {
  OPS_PROLOGUE(c);
  OPS_ARG(x && out && rows > 0 && cols > 0, "bad arguments");
  hipLaunchKernelGGL(k_transpose_f32, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, st_,
                     static_cast<const float*>(x), static_cast<float*>(out), rows, cols);
  return op_launched("transpose");
}

int fh_op_layernorm_forward(fh_context* c, const void* x, const void* w, const void* b, void* out, void* mean,
                            void* rstd, int rows, int cols, float eps) {
  OPS_PROLOGUE(c);
  OPS_ARG(x && w && b && out && mean && rstd && rows > 0 && cols > 0, "bad arguments");
  hipLaunchKernelGGL(k_ln_forward, dim3(rows), dim3(256), 0, st_, static_cast<const float*>(x),
                     static_cast<const float*>(w), static_cast<const float*>(b), static_cast<float*>(out),
                     static_cast<float*>(mean), static_cast<float*>(rstd), cols, eps);
  return op_launched("layernorm forward");
}

int fh_op_layernorm_backward(fh_context* c, const void* dout, const void* x, const void* w, const void* mean,
                             const void* rstd, void* dx, void* dw, void* db, int rows, int cols) {
  OPS_PROLOGUE(c);
  OPS_ARG(dout && x && w && mean && rstd && dx && dw && db && rows > 0 && cols > 0, "bad arguments");
  const float *fd = static_cast<const float*>(dout), *fx = static_cast<const float*>(x);
  const float *fm = static_cast<const float*>(mean), *fr = static_cast<const float*>(rstd);
  hipLaunchKernelGGL(k_ln_backward_dx, dim3(rows), dim3(256), 0, st_, fd, fx, static_cast<const float*>(w), fm, fr,
                     static_cast<float*>(dx), cols);
  const int chunks = (rows + kRowChunk - 1) / kRowChunk;
  float* part = nullptr;
  if (chunks > 1) {
    void* p = nullptr;
    FH_TRY(ops_scratch(c, ops_, (size_t)2 * chunks * cols * sizeof(float), &p));
    part = static_cast<float*>(p);
  }
  hipLaunchKernelGGL(k_col_sums<1>, dim3((cols + 255) / 256, chunks), dim3(256), 0, st_, fd, fx, fm, fr, rows, cols,
                     static_cast<float*>(dw), static_cast<float*>(db), part, chunks);
  if (chunks > 1) {
    hipLaunchKernelGGL(k_sum_chunks, dim3((cols + 255) / 256), dim3(256), 0, st_, part, chunks, cols,
                       static_cast<float*>(dw));
    hipLaunchKernelGGL(k_sum_chunks, dim3((cols + 255) / 256), dim3(256), 0, st_, part + (size_t)chunks * cols, chunks,
                       cols, static_cast<float*>(db));
  }
  return op_launched("layernorm backward");
}

int fh_op_softmax_forward(fh_context* c, void* x, int rows, int cols) { return softmax_common(c, x, rows, cols, 1.f, 0); }

int fh_op_scaled_causal_softmax_forward(fh_context* c, void* scores, int rows, int T, float scale) {
  return softmax_common(c, scores, rows, T, scale, 1);
}

int fh_op_softmax_backward(fh_context* c, const void* dout, const void* sm, void* dx, int rows, int cols, float scale) {
  OPS_PROLOGUE(c);
  OPS_ARG(dout && sm && dx && rows > 0 && cols > 0, "bad arguments");
  hipLaunchKernelGGL(k_softmax_backward, dim3(rows), dim3(256), 0, st_, static_cast<const float*>(dout),
                     static_cast<const float*>(sm), static_cast<float*>(dx), cols, scale);
  return op_launched("softmax backward");
}

int fh_op_gelu_forward(fh_context* c, const void* x, void* out, int64_t n) {
  OPS_PROLOGUE(c);
  OPS_ARG(x && out && n > 0, "bad arguments");
  hipLaunchKernelGGL(k_gelu_forward, dim3(grid_for((size_t)n)), dim3(kT), 0, st_, static_cast<const float*>(x),
                     static_cast<float*>(out), (size_t)n);
  return op_launched("gelu forward");
}

int fh_op_gelu_backward(fh_context* c, const void* dout, const void* x, void* dx, int64_t n) {
  OPS_PROLOGUE(c);
  OPS_ARG(dout && x && dx && n > 0, "bad arguments");
  hipLaunchKernelGGL(k_gelu_backward, dim3(grid_for((size_t)n)), dim3(kT), 0, st_, static_cast<const float*>(dout),
                     static_cast<const float*>(x), static_cast<float*>(dx), (size_t)n);
  return op_launched("gelu backward");
}

int fh_op_embedding_forward(fh_context* c, const void* table, int table_rows, const int32_t* indices, int n, void* out,
                            int D) {
  OPS_PROLOGUE(c);
  OPS_ARG(table && out && (indices || n == 0) && n >= 0 && D > 0 && table_rows > 0, "bad arguments");
  for (int t = 0; t < n; t++)
    if (indices[t] < 0 || indices[t] >= table_rows)
      return set_err(FH_ERR_RANGE, "index %d at position %d outside the table's %d rows", indices[t], t, table_rows);
  if (n == 0) return FH_OK;
  int* di = nullptr;
  FH_TRY(upload_ints(c, ops_, indices, (size_t)n, &di));
  hipLaunchKernelGGL(k_embedding_forward, dim3(n), dim3(256), 0, st_, static_cast<const float*>(table), di,
                     static_cast<float*>(out), D);
  return op_launched("embedding forward");
}

int fh_op_embedding_backward(fh_context* c, const void* dout, const int32_t* indices, int n, void* dtable,
                             int table_rows, int D) {
  OPS_PROLOGUE(c);
  OPS_ARG(dout && dtable && (indices || n == 0) && n >= 0 && D > 0 && table_rows > 0, "bad arguments");
  for (int t = 0; t < n; t++)
    if (indices[t] < 0 || indices[t] >= table_rows)
      return set_err(FH_ERR_RANGE, "index %d at position %d outside the table's %d rows", indices[t], t, table_rows);
  if (n == 0) return FH_OK;
  // group the positions by id, ascending within each id
  std::vector<int> order(n);
  for (int t = 0; t < n; t++) order[t] = t;
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return indices[x] < indices[y]; });
  std::vector<int> host;  // uniq[U] | start[U+1] | pos[n]
  std::vector<int> uniq, start;
  for (int k = 0; k < n; k++)
    if (k == 0 || indices[order[k]] != indices[order[k - 1]]) {
      uniq.push_back(indices[order[k]]);
      start.push_back(k);
    }
  start.push_back(n);
  const int U = (int)uniq.size();
  host.insert(host.end(), uniq.begin(), uniq.end());
  host.insert(host.end(), start.begin(), start.end());
  host.insert(host.end(), order.begin(), order.end());
  int* dev = nullptr;
  FH_TRY(upload_ints(c, ops_, host.data(), host.size(), &dev));
  hipLaunchKernelGGL(k_embedding_backward, dim3((D + 255) / 256, U), dim3(256), 0, st_,
                     static_cast<const float*>(dout), dev, dev + U, dev + 2 * U + 1, static_cast<float*>(dtable), D);
  return op_launched("embedding backward");
}

int fh_op_causal_mask(fh_context* c, void* scores, int64_t len, int T) {
  OPS_PROLOGUE(c);
  OPS_ARG(scores && T > 0 && len > 0 && len % ((int64_t)T * T) == 0, "scores must hold whole [T,T] blocks");
  hipLaunchKernelGGL(k_causal_mask, dim3(grid_for((size_t)len)), dim3(kT), 0, st_, static_cast<float*>(scores),
                     (size_t)len, T);
  return op_launched("causal mask");
}

int fh_op_cross_entropy_forward(fh_context* c, const void* logits, const int32_t* targets, void* probs, int T, int V,
                                int ignore_index, float* loss) {
  OPS_PROLOGUE(c);
  OPS_ARG(logits && probs && targets && loss && T > 0 && V > 0, "bad arguments");
  int count = 0;
  for (int t = 0; t < T; t++) {
    if (targets[t] == ignore_index) continue;
    if (targets[t] < 0 || targets[t] >= V)
      return set_err(FH_ERR_RANGE, "target %d at position %d outside [0,%d)", targets[t], t, V);
    count++;
  }
  void* p = nullptr;
  FH_TRY(ops_scratch(c, ops_, (size_t)T * (sizeof(int32_t) + sizeof(float)), &p));
  int* dt = static_cast<int*>(p);
  float* nll = reinterpret_cast<float*>(dt + T);
  HIP_TRY(hipMemcpyAsync(dt, targets, (size_t)T * sizeof(int32_t), hipMemcpyHostToDevice, st_));
  HIP_TRY(hipStreamSynchronize(st_));
  hipLaunchKernelGGL(k_ce_forward, dim3(T), dim3(256), 0, st_, static_cast<const float*>(logits), dt,
                     static_cast<float*>(probs), V, ignore_index, nll);
  FH_TRY(op_launched("cross-entropy forward"));
  if (ops_->accumulating) {
    // the loss stays on the device until the accumulation ends (ITensorBackend.cs:154-161)
    hipLaunchKernelGGL(k_ce_accumulate, dim3(1), dim3(64), 0, st_, nll, T, ops_->acc);
    ops_->accumulated_targets += count;
    *loss = 0.f;
    return op_launched("loss accumulation");
  }
  std::vector<float> per(T);
  HIP_TRY(hipMemcpyAsync(per.data(), nll, (size_t)T * sizeof(float), hipMemcpyDeviceToHost, st_));
  HIP_TRY(hipStreamSynchronize(st_));
  double total = 0;
  for (int t = 0; t < T; t++)
    if (targets[t] != ignore_index) total += per[t];
  *loss = count == 0 ? 0.f : (float)(total / count);
  return FH_OK;
}

int fh_op_begin_loss_accumulation(fh_context* c) {
  OPS_PROLOGUE(c);
  if (ops_->accumulating) return set_err(FH_ERR_STATE, "Loss accumulation is already active.");
  HIP_TRY(hipMemsetAsync(ops_->acc, 0, sizeof(double), st_));
  ops_->accumulating = true;
  ops_->accumulated_targets = 0;
  return FH_OK;
}

int fh_op_end_loss_accumulation(fh_context* c, float* mean_loss) {
  OPS_PROLOGUE(c);
  OPS_ARG(mean_loss, "null result pointer");
  if (!ops_->accumulating) return set_err(FH_ERR_STATE, "Loss accumulation is not active.");
  double s = 0;
  HIP_TRY(hipMemcpyAsync(&s, ops_->acc, sizeof(double), hipMemcpyDeviceToHost, st_));
  HIP_TRY(hipStreamSynchronize(st_));
  ops_->accumulating = false;
  *mean_loss = ops_->accumulated_targets == 0 ? 0.f : (float)(s / (double)ops_->accumulated_targets);
  return FH_OK;
}

int fh_op_cross_entropy_backward(fh_context* c, const void* probs, const int32_t* targets, void* dlogits, int T, int V,
                                 int ignore_index) {
  OPS_PROLOGUE(c);
  OPS_ARG(probs && dlogits && targets && T > 0 && V > 0, "bad arguments");
  int count = 0;
  for (int t = 0; t < T; t++) {
    if (targets[t] == ignore_index) continue;
    if (targets[t] < 0 || targets[t] >= V)
      return set_err(FH_ERR_RANGE, "target %d at position %d outside [0,%d)", targets[t], t, V);
    count++;
  }
  const size_t n = (size_t)T * V;
  if (count == 0) {
    HIP_TRY(hipMemsetAsync(dlogits, 0, n * sizeof(float), st_));
    return FH_OK;
  }
  int* dt = nullptr;
  FH_TRY(upload_ints(c, ops_, targets, (size_t)T, &dt));
  hipLaunchKernelGGL(k_ce_backward, dim3(grid_for(n)), dim3(kT), 0, st_, static_cast<const float*>(probs), dt,
                     static_cast<float*>(dlogits), V, ignore_index, 1.f / (float)count, n);
  return op_launched("cross-entropy backward");
}

int fh_op_zero(fh_context* c, void* x, int64_t n) {
  OPS_PROLOGUE(c);
  OPS_ARG(x && n >= 0, "bad arguments");
  if (n > 0) HIP_TRY(hipMemsetAsync(x, 0, (size_t)n * sizeof(float), st_));
  return FH_OK;
}

int fh_op_sum_squares(fh_context* c, const void* x, int64_t n, double* out) {
  const void* xs[1] = {x};
  const int64_t ns[1] = {n};
  return fh_op_global_sum_squares(c, xs, ns, 1, out);
}

int fh_op_global_sum_squares(fh_context* c, const void* const* xs, const int64_t* ns, int count, double* out) {
  OPS_PROLOGUE(c);
  OPS_ARG(out && count >= 0 && (count == 0 || (xs && ns)), "bad arguments");
  *out = 0;
  if (count == 0) return FH_OK;
  for (int i = 0; i < count; i++) OPS_ARG(xs[i] && ns[i] >= 0, "bad tensor %d", i);
  void* p = nullptr;
  FH_TRY(ops_scratch(c, ops_, ((size_t)count * 256 + 1) * sizeof(double), &p));
  double* part = static_cast<double*>(p);
  int off = 0;
  for (int i = 0; i < count; i++) {
    if (ns[i] == 0) continue;
    int nb = 0;
    FH_TRY(sumsq_partials(st_, static_cast<const float*>(xs[i]), (size_t)ns[i], part + off, &nb));
    off += nb;
  }
  double* res = part + (size_t)count * 256;
  hipLaunchKernelGGL(k_sum_doubles, dim3(1), dim3(64), 0, st_, part, off, res);
  FH_TRY(op_launched("sum of squares"));
  HIP_TRY(hipMemcpyAsync(out, res, sizeof(double), hipMemcpyDeviceToHost, st_));
  HIP_TRY(hipStreamSynchronize(st_));
  return FH_OK;
}

int fh_op_adamw_step(fh_context* c, void* w, const void* g, void* m, void* v, int64_t n, float lr, float beta1,
                     float beta2, float eps, float weight_decay, int step, int is_matrix) {
  OPS_PROLOGUE(c);
  OPS_ARG(w && g && m && v && n > 0 && step >= 1, "bad arguments");
  const float bc1 = 1.f - powf(beta1, (float)step);
  const float bc2 = 1.f - powf(beta2, (float)step);
  const int decay = weight_decay != 0.f && is_matrix;
  hipLaunchKernelGGL(k_adamw, dim3(grid_for((size_t)n)), dim3(kT), 0, st_, static_cast<float*>(w),
                     static_cast<const float*>(g), static_cast<float*>(m), static_cast<float*>(v), (size_t)n, lr,
                     beta1, beta2, eps, weight_decay, bc1, bc2, decay);
  return op_launched("adamw step");
}

}  // extern "C"
