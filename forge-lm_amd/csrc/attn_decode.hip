// attn_decode.hip -- decode attention of a batch of sequences (one new query
// row per sequence) over the KV cache, head_dim 64 (gfx950).
//
// MultiHeadAttention.Forward on the cached window (src/LLM.Core/Layers/Layers.cs:191-229):
// for each sequence b and head h, s_j = q.k_j * (1/sqrt(64)) over keys 0..pos,
// softmax, o = sum_j p_j v_j.  A block takes 256 keys of one (b, h): each of
// its 4 waves reads 64 K and 64 V rows with one 1 KB load per 4 rows (lane l:
// dims 4*(l % 16) .. +3 of row 4i + l / 16), so every request is a contiguous
// 1 KB; the block's partial (o[64], max, sum) is combined with the other
// chunks' by k_attn_decode_combine, or by the attn.proj GEMM as it loads its
// operand.  In batched decode the kernel also takes q from the qkv projection's
// split-K partials and the block over the new position stores its K/V rows
// before reading the cache.  Memory bound: 2 * nkeys * 256 bytes per (b, h).
#include "kernels.hpp"

#include <math.h>

namespace fh {

namespace {

constexpr int KW = 64;        // keys per wave
constexpr int CHUNK = 4 * KW;  // keys per block
static_assert(CHUNK == kAttnDecodeChunk, "chunk size shared with the GEMM's attention operand");

__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// 4 consecutive elements of a row through a bounded buffer resource (reads past
// the bound return zeros).  The K/V rows are read once per step, so the loads carry
// the non-temporal hint (NT) and leave the L2 to the partial sums and weights the
// step's other kernels read (C4: 886 -> 869 us per step; the same hint on the decode
// GEMMs' weight loads measured 12 us slower).
template <typename KT>
__device__ __forceinline__ float4 load4(__amdgpu_buffer_rsrc_t r, int elem_off);
template <>
__device__ __forceinline__ float4 load4<float>(__amdgpu_buffer_rsrc_t r, int elem_off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, elem_off * 4, 0, 2);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
template <>
__device__ __forceinline__ float4 load4<bf16_t>(__amdgpu_buffer_rsrc_t r, int elem_off) {
  const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, elem_off * 2, 0, 2);
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xffff0000u));
}

template <typename KT, bool FROM_PARTS>
__global__ __launch_bounds__(256) void k_attn_decode_wide(RowSrc src, const float* __restrict__ qkv, int d, int H,
                                                          int ctx, KT* __restrict__ kc, KT* __restrict__ vc,
                                                          float* __restrict__ part, int maxc, QkvParts qp) {
  __shared__ float wm[4], wl[4];
  __shared__ __align__(16) float wo[4][64];
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, d4 = 4 * (lane & 15);
  const int n = *src.step;
  const int nkeys = min(ctx, src.pos_off + src.pos_mul * n + 1);
  if (c * CHUNK >= nkeys) return;  // the whole block: no chunk of keys here
  const size_t head = ((size_t)b * H + h) * ctx * 64;
  float4 qr;
  if constexpr (FROM_PARTS) {
    // the qkv projection's split-K partials summed here (k_epilogue_qkv's order:
    // 0 + partials + bias); the block whose chunk holds the new position first
    // writes the new K and V rows into the caches, which its loads below then read
    const size_t N3 = (size_t)3 * d, MN = (size_t)qp.M * N3;
    const float* p0 = qp.part + (size_t)b * N3;
    // the bias is requested with the partials (one round trip, not two)
    const float4 bb =
        qp.bias ? *reinterpret_cast<const float4*>(qp.bias + h * 64 + d4) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
    for (int i = 0; i < qp.S; i++) {
      const float4 v = *reinterpret_cast<const float4*>(p0 + i * MN + h * 64 + d4);
      a.x += v.x;
      a.y += v.y;
      a.z += v.z;
      a.w += v.w;
    }
    if (qp.bias) {
      a.x += bb.x;
      a.y += bb.y;
      a.z += bb.z;
      a.w += bb.w;
    }
    qr = a;
    const int pos = src.pos_off + src.pos_mul * n;
    if ((unsigned)pos < (unsigned)ctx && c == pos / CHUNK) {
      if (tid < 128) {
        const int col = (tid < 64 ? d : 2 * d) + h * 64 + (tid & 63);
        const float bcol = qp.bias ? qp.bias[col] : 0.f;  // requested with the partials
        float v = 0.f;
#pragma unroll 8
        for (int i = 0; i < qp.S; i++) v += p0[i * MN + col];
        if (qp.bias) v += bcol;
        (tid < 64 ? kc : vc)[head + (size_t)pos * 64 + (tid & 63)] = from_f32<KT>(v);
      }
      __syncthreads();  // the new rows are stored before any wave reads them
    }
  } else {
    qr = *reinterpret_cast<const float4*>(qkv + (size_t)b * 3 * d + h * 64 + d4);
  }
  // q scaled by 1/sqrt(64) = 2^-3: exact, so q'.k = (q.k) / 8 bit for bit
  const float4 q4 = make_float4(qr.x * 0.125f, qr.y * 0.125f, qr.z * 0.125f, qr.w * 0.125f);
  const int j0 = c * CHUNK + w * KW;  // this wave's first key
  // a wave past the last key fetches nothing (an empty buffer resource reads zeros)
  const int bytes = j0 < nkeys ? ctx * 64 * (int)sizeof(KT) : 0;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(kc + head), (short)0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(vc + head), (short)0, bytes, 0x00020000);
  float4 kr[KW / 4], vr[KW / 4];
#pragma unroll
  for (int i = 0; i < KW / 4; i++) kr[i] = load4<KT>(rk, (j0 + 4 * i + g) * 64 + d4);
#pragma unroll
  for (int i = 0; i < KW / 4; i++) vr[i] = load4<KT>(rv, (j0 + 4 * i + g) * 64 + d4);
  float sc[KW / 4];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < KW / 4; i++) {
    const int j = j0 + 4 * i + g;
    const float s = row16_sum(q4.x * kr[i].x + q4.y * kr[i].y + q4.z * kr[i].z + q4.w * kr[i].w);
    sc[i] = j < nkeys ? s : -INFINITY;
    m = fmaxf(m, sc[i]);
  }
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  if (m != -INFINITY) {
#pragma unroll
    for (int i = 0; i < KW / 4; i++) {
      const int j = j0 + 4 * i + g;
      const float p = j < nkeys ? __expf(sc[i] - m) : 0.f;
      // rows past the last key may hold anything (even NaN): never multiplied
      const float4 v = j < nkeys ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      l += p;
      o.x += p * v.x;
      o.y += p * v.y;
      o.z += p * v.z;
      o.w += p * v.w;
    }
  }
  // the four key rows of the wave (lanes l, l^16, l^32, l^48)
#pragma unroll
  for (int s = 16; s <= 32; s *= 2) {
    l += __shfl_xor(l, s, 64);
    o.x += __shfl_xor(o.x, s, 64);
    o.y += __shfl_xor(o.y, s, 64);
    o.z += __shfl_xor(o.z, s, 64);
    o.w += __shfl_xor(o.w, s, 64);
  }
  if (lane == 0) {
    wm[w] = m;
    wl[w] = l;
  }
  if (g == 0) *reinterpret_cast<float4*>(&wo[w][d4]) = o;
  __syncthreads();
  if (w == 0) {
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) M = fmaxf(M, wm[i]);
    float L = 0.f, a = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float f = wm[i] == -INFINITY ? 0.f : __expf(wm[i] - M);
      L += wl[i] * f;
      a += wo[i][lane] * f;
    }
    float* P = part + (((size_t)b * H + h) * maxc + c) * 66;
    P[lane] = a;
    if (lane == 0) {
      P[64] = M;
      P[65] = L;
    }
  }
}

}  // namespace

template <typename KT>
hipError_t launch_attn_decode_wide(hipStream_t st, RowSrc src, const float* qkv, int B, int d, int H, int ctx,
                                   const KT* kcache, const KT* vcache, float* part, float* o, bool combine,
                                   const QkvParts* qp) {
  if (B <= 0 || H <= 0 || d != 64 * H || ctx <= 0 || (size_t)ctx * 64 * sizeof(KT) > 0x7fffffffu ||
      !(qkv || qp) || !kcache || !vcache || !part || !o)
    return hipErrorInvalidValue;
  if (qp && (!qp->part || qp->S < 1 || qp->M != B || (size_t)qp->S * B * 3 * d * 4 > 0x7fffffffu))
    return hipErrorInvalidValue;
  const int maxc = (ctx + CHUNK - 1) / CHUNK;
  KT* kc = const_cast<KT*>(kcache);
  KT* vc = const_cast<KT*>(vcache);
  if (qp)
    hipLaunchKernelGGL((k_attn_decode_wide<KT, true>), dim3(maxc, H, B), dim3(256), 0, st, src, qkv, d, H, ctx, kc, vc,
                       part, maxc, *qp);
  else
    hipLaunchKernelGGL((k_attn_decode_wide<KT, false>), dim3(maxc, H, B), dim3(256), 0, st, src, qkv, d, H, ctx, kc,
                       vc, part, maxc, QkvParts{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !combine) return e;
  return launch_attn_decode_combine(st, src, B, d, H, ctx, part, CHUNK, maxc, o);
}

template hipError_t launch_attn_decode_wide<float>(hipStream_t, RowSrc, const float*, int, int, int, int,
                                                   const float*, const float*, float*, float*, bool, const QkvParts*);
template hipError_t launch_attn_decode_wide<bf16_t>(hipStream_t, RowSrc, const float*, int, int, int, int,
                                                    const bf16_t*, const bf16_t*, float*, float*, bool, const QkvParts*);

}  // namespace fh
