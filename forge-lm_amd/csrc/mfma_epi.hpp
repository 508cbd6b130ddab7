// mfma_epi.hpp -- epilogue of the MFMA GEMMs: y = epi(acc + bias) (+ res) for
// one 32x32 accumulator tile, through bounded buffer resources.
//
// The resources start at the block's first row and end at the last row that
// exists, so rows past M load zeros and their stores are dropped by the
// hardware; columns past N are masked by the caller.  All residual loads of a
// tile are issued before its first store, so a tile costs one memory round trip
// rather than one per element.
#pragma once

#include "kernels.hpp"

namespace fh {

typedef float mfma_f32x16_t __attribute__((ext_vector_type(16)));

// MFMA 32x32 accumulator layout: lane l holds column l % 32 and, in element r,
// row (r / 4) * 8 + (l / 32) * 4 + r % 4.
__device__ __forceinline__ int mfma_acc_row(int lane, int r) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, size_t row0, int rows, int N, int esz) {
  return __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(base) + row0 * (size_t)N * esz), (short)0, rows * N * esz,
      0x00020000);
}

// GELU for an output rounded to bf16 (relative step 2^-8): 0.5 v (1 + tanh u) =
// v / (1 + 2^(-2 u log2 e)) on the hardware exp2 and reciprocal, with
// -2 u log2 e = v (K0 + K1 v^2) (C = MathF.Sqrt(2f / MathF.PI), 0.044715 and
// log2 e folded into two constants: 5 VALU operations and 2 transcendentals per
// element, where the epilogue of a bf16-out GEMM tile is VALU-bound), a few fp32
// ulps from the tanhf form, far below the rounding that follows
__device__ __forceinline__ float gelu_for_bf16(float v) {
  constexpr float K0 = (float)(-2.0 * 0.7978845238685608 * 1.4426950408889634);
  constexpr float K1 = (float)(-2.0 * 0.7978845238685608 * 1.4426950408889634 * 0.044715);
  const float q = v * __builtin_fmaf(v * v, K1, K0);
  return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(q));
}

// rows trow0 + mfma_acc_row(lane, r) (relative to the resources' first row) of column col;
// SAUX is the fp32 stores' cache policy (2: non-temporal, for split-K partial sums,
// which are read once by the kernel after: C4 859 -> 850-853 us per step)
template <int EPI, bool RES, bool OUT_BF16, int SAUX = 0>
__device__ __forceinline__ void mfma_store_tile(const mfma_f32x16_t& acc, int lane, int trow0, int col, int N,
                                                float bcol, __amdgpu_buffer_rsrc_t rres,
                                                __amdgpu_buffer_rsrc_t ry) {
  float rv[16];
  if constexpr (RES) {
#pragma unroll
    for (int r = 0; r < 16; r++)
      rv[r] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rres, ((trow0 + mfma_acc_row(lane, r)) * N + col) * 4, 0, 0));
  }
#pragma unroll
  for (int r = 0; r < 16; r++) {
    float s = acc[r] + bcol;
    if constexpr (EPI == EPI_GELU) s = OUT_BF16 ? gelu_for_bf16(s) : gelu_tanh(s);
    if constexpr (RES) s += rv[r];
    const int e = (trow0 + mfma_acc_row(lane, r)) * N + col;
    if constexpr (OUT_BF16)
      __builtin_amdgcn_raw_buffer_store_b16(bf16_rn(s), ry, e * 2, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, s), ry, e * 4, 0, SAUX);
  }
}

}  // namespace fh
