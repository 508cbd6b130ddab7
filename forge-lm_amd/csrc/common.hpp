// common.hpp -- device helpers shared by every gfx950 kernel of libforge_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fh {

constexpr int kWave = 64;  // CDNA wavefront width

typedef uint16_t bf16_t;  // raw bfloat16 bits

__device__ __host__ __forceinline__ float bf16_to_f32(bf16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __host__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// The same rounding on the device: one v_cvt_pk_bf16_f32 (round to nearest even,
// the bits of f32_to_bf16 for every value that is not a NaN).
__device__ __forceinline__ bf16_t bf16_rn(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<bf16_t>(bf16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return bf16_rn(v); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Wave sum through DPP row operations (quad permutes, half-row and row mirrors,
// row broadcasts 15 and 31); the total ends in lane 63 and is broadcast with
// readlane.  Much cheaper than the ds_bpermute shuffles of wave_sum.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  const int ninf = __builtin_bit_cast(int, -INFINITY);
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(ninf, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false)));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Value of lane `src` (wave-uniform) in every lane.
__device__ __forceinline__ float lane_bcast(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// (value, index) argmax with the reference's tie rule: larger value wins, equal
// values keep the smaller index (Sampler.Greedy scans with a strict '>').
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, kWave);
    int oi = __shfl_xor(i, o, kWave);
    argmax_merge(v, i, ov, oi);
  }
}

// tanh-approximation GELU with the reference constants
// (src/LLM.Core/Tensor/CpuBackend.cs:25-26, 510-514): 0.5*v*(1+tanh(C*(v+0.044715*v^3))).
__device__ __forceinline__ float gelu_tanh(float v) {
  // MathF.Sqrt(2f / MathF.PI) evaluated in fp32 = 0x3f4c4229 (one ulp below
  // the fp32 rounding of sqrt(2/pi) itself).
  const float C = 0.7978845238685608f;
  float u = C * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.f + tanhf(u));
}

// Where the token id and position of row t of a window come from, given the
// device step counter n (tokens generated so far in this fh_generate call):
//   id  = tokens[b*tok_stride + tok_off + n + t]
//   pos = pos_off + pos_mul*n + t
// A prefill window of T rows uses tok_off = P - T, pos_off = 0, pos_mul = 0; a
// cached decode row uses tok_off = P - 1, pos_off = P - 1, pos_mul = 1.
struct RowSrc {
  const int* tokens;
  const int* step;
  int tok_stride;
  int tok_off;
  int pos_off;
  int pos_mul;
};

}  // namespace fh
