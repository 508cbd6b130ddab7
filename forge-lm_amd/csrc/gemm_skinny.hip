// gemm_skinny.hip -- the decode GEMMs of a batch of up to 32 rows, fp32.
//
// Linear.Forward (src/LLM.Core/Layers/Layers.cs:29-37) for the M <= 32 decode
// rows of a batched session: y = epi(x @ W + b).  At this M every weight is used
// by 32 rows only, so the product streams W once (HBM-bound) and the question is
// how many CUs stream it and how many launches the layer costs.  A block owns 16
// output columns and the whole of its K range (768 per block: S = K / 768 blocks
// share a column strip when K is larger); its four waves take a quarter of that
// range each on v_mfma_f32_16x16x4_f32 (two 16-row tiles per wave, the weight
// operand shared), and the four partial tiles are added through LDS in wave
// order.  With one block per strip (S = 1) the bias and GELU are applied in the
// block (mlp.fc: no partial sums and no reduction launch); otherwise the block
// writes its strip's sums as split S of part[S][M][N] for the kernel after it.
//
// Operand layout of v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16]; the result's element r in lane l is D[4 (l / 16) + r][l % 16].
// The k index of the hardware step is permuted: lane (j, q) of step (t, e) holds
// k = k0 + 16 t + 4 q + e, so each lane's operands for four steps are one 16-byte
// load of A (a row) and one of W^T (a column), and every k of the range is used
// exactly once (the sum is over the same terms in another order).
#include "kernels.hpp"

namespace fh {

namespace {

constexpr int SK_COLS = 16;        // output columns per block
constexpr int SK_KW = 192;         // k per wave
constexpr int SK_KB = 4 * SK_KW;   // k per block
constexpr int SK_T = SK_KW / 16;   // 16-k steps per wave

typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_skinny(const float* __restrict__ x, int M, int K,
                                                     const float* __restrict__ Wt, int N,
                                                     const float* __restrict__ bias, float* __restrict__ y) {
  __shared__ float red[4][32][SK_COLS + 1];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * SK_COLS, split = blockIdx.y;
  const int k0 = split * SK_KB + w * SK_KW;
  const int j = lane & 15, q = lane >> 4;
  // bounded resources: A rows past M read as zeros (their sums are never stored);
  // the block's 16 rows of W^T, read once per step: non-temporal hint (C4 835 ->
  // 828 us per step)
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), (short)0, M * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(Wt + (size_t)n0 * K), (short)0, SK_COLS * K * 4, 0x00020000);
  f32x4_t a0[SK_T], a1[SK_T], b[SK_T];
#pragma unroll
  for (int t = 0; t < SK_T; t++) {
    const int k = k0 + 16 * t + 4 * q;
    b[t] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rb, (j * K + k) * 4, 0, 2));
    a0[t] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, (j * K + k) * 4, 0, 0));
    a1[t] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, ((16 + j) * K + k) * 4, 0, 0));
  }
  // every load is in flight before the first product: the scheduler would
  // otherwise place each load just before its use and wait for it there, one
  // memory latency per step
  __builtin_amdgcn_sched_barrier(0);
  f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < SK_T; t++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[t][e], b[t][e], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[t][e], b[t][e], c1, 0, 0, 0);
    }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    red[w][4 * q + r][j] = c0[r];
    red[w][16 + 4 * q + r][j] = c1[r];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int o = tid + 256 * h, row = o >> 4, col = o & 15;
    if (row < M) {
      float v = ((red[0][row][col] + red[1][row][col]) + red[2][row][col]) + red[3][row][col];
      if constexpr (EPI == EPI_GELU) {
        v = gelu_tanh(v + bias[n0 + col]);
        y[(size_t)row * N + n0 + col] = v;
      } else {
        y[((size_t)split * M + row) * N + n0 + col] = v;
      }
    }
  }
}

}  // namespace

bool gemm_skinny_fits(int M, int K, int N) {
  return M >= 1 && M <= 32 && K % SK_KB == 0 && N % SK_COLS == 0 && (size_t)32 * K * 4 <= 0x7fffffffu &&
         (size_t)SK_COLS * K * 4 <= 0x7fffffffu;
}

hipError_t launch_gemm_skinny(hipStream_t st, const float* x, int M, int K, const float* Wt, int N,
                              const float* bias, int epi, float* y, int* splits) {
  if (!x || !Wt || !y || !gemm_skinny_fits(M, K, N)) return hipErrorInvalidValue;
  const int S = K / SK_KB;
  if (epi == EPI_GELU) {
    if (S != 1 || !bias) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_skinny<EPI_GELU>), dim3(N / SK_COLS, 1), dim3(256), 0, st, x, M, K, Wt, N, bias, y);
  } else {
    if (epi != EPI_NONE) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_skinny<EPI_NONE>), dim3(N / SK_COLS, S), dim3(256), 0, st, x, M, K, Wt, N, nullptr,
                       y);
  }
  if (splits) *splits = S;
  return hipGetLastError();
}

}  // namespace fh
