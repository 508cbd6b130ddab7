// gemm_mfma.hip -- LDS-staged MFMA GEMM for gfx950: prefill and batched decode.
//
// Linear.Forward (src/LLM.Core/Layers/Layers.cs:29-37): y = x @ W + b for M
// rows.  W comes pre-transposed as Wt[N][K] (k contiguous, built once per
// session), so both MFMA operands are k-contiguous in global memory and in
// LDS.  A block computes a BM x 128 tile of y; each of its 4 waves owns a
// 32-column strip and BM/32 MFMA 32x32 accumulators.  K advances 32 per stage
// through a double-buffered LDS pair: the next stage's global loads are in
// registers while the current stage's MFMAs run.
//
//   bf16 sessions: v_mfma_f32_32x32x16_bf16; activations are rounded to bf16
//                  on their way into LDS, accumulation is fp32.
//   fp32 sessions: v_mfma_f32_32x32x2_f32 on exact fp32 operands; within a
//                  32-wide k stage the LDS rows hold the even k first, then the
//                  odd k, so each half-wave reads its k values as float4s.
//
// With S > 1 (blockIdx.z) each block covers K/S of the reduction and writes a
// partial; launch_splitk_epilogue then sums the partials in order, adds the
// bias (if any) and applies GELU / the residual.  With S == 1 the epilogue is
// fused.
#include "kernels.hpp"
#include "mfma_epi.hpp"

namespace fh {

namespace {

constexpr int BN = 128;  // columns per block (4 waves x 32)
constexpr int BK = 32;   // k per stage

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <typename WT>
struct Tr;

// ---- bf16: LDS rows of BK bf16 (+8 pad), fragments of 8 k per lane ----
template <>
struct Tr<bf16_t> {
  static constexpr int LDK = BK + 8;  // bf16 per LDS row
  typedef bf16_t elem;
};

// ---- fp32: LDS rows of BK floats (+4 pad), even k then odd k ----
template <>
struct Tr<float> {
  static constexpr int LDK = BK + 4;
  typedef float elem;
};

// Four consecutive A values A[m][k..k+3] built from decode attention's chunk
// partials (AOperand): rows past M repeat the last row (their products are
// dropped).  The chunk loop runs to a fixed count on clamped addresses, so every
// load of a stage issues at once; chunks past the real count are skipped.
constexpr int kAttnChunksMax = 4;
__device__ __forceinline__ float4 load_attn_a4(const AOperand& ao, int m, int k, int M, int K) {
  // k_attn_decode_combine for sequence r, head k / hd, dims e .. e+3
  const int r = min(m, M - 1);
  {
    const int hd = K / ao.H, h = k / hd, e = k % hd;
    const int n = *ao.src.step;
    const int nkeys = min(ao.ctx, ao.src.pos_off + ao.src.pos_mul * n + 1);
    const int nch = (nkeys + ao.chunk - 1) / ao.chunk;
    const float* P0 = ao.apart + ((size_t)r * ao.H + h) * ao.maxc * (hd + 2);
    float mc[kAttnChunksMax], lc[kAttnChunksMax], pc[kAttnChunksMax][4];
#pragma unroll
    for (int c = 0; c < kAttnChunksMax; c++) {
      const float* P = P0 + (size_t)min(c, nch - 1) * (hd + 2);
      mc[c] = P[hd];
      lc[c] = P[hd + 1];
#pragma unroll
      for (int j = 0; j < 4; j++) pc[c][j] = P[e + j];
    }
    float Mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < kAttnChunksMax; c++)
      if (c < nch) Mx = fmaxf(Mx, mc[c]);
    float L = 0.f, a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int c = 0; c < kAttnChunksMax; c++)
      if (c < nch) {
        const float f = expf(mc[c] - Mx);
        L += lc[c] * f;
        a0 += pc[c][0] * f;
        a1 += pc[c][1] * f;
        a2 += pc[c][2] * f;
        a3 += pc[c][3] * f;
      }
    const float inv = 1.f / L;
    return make_float4(a0 * inv, a1 * inv, a2 * inv, a3 * inv);
  }
}

// NSR == 0: K streams through a double-buffered LDS pair, one stage ahead.
// NSR > 0 (short K chunks of split-K decode GEMMs, at most NSR stages): every
// stage's loads are issued at once into NSR register sets and LDS buffers, so
// the block pays one memory latency instead of one per stage.
template <typename WT, int BM, int EPI, bool RES, int NSR, int AOP = AOP_PLAIN>
__global__ __launch_bounds__(256) void k_gemm_mfma(const float* __restrict__ A, int M, int K,
                                                  const WT* __restrict__ Wt, int N, int kchunk,
                                                  const float* __restrict__ bias,
                                                  const float* __restrict__ res, float* __restrict__ Y,
                                                  float* __restrict__ part, AOperand ao) {
  using E = typename Tr<WT>::elem;
  constexpr int LDK = Tr<WT>::LDK;
  constexpr int MT = BM / 32;  // MFMA tiles along M per wave
  constexpr int NBUF = NSR > 0 ? NSR : 2;
  constexpr int NREG = NSR > 0 ? NSR : 1;
  __shared__ __align__(16) E As[NBUF][BM][LDK];
  __shared__ __align__(16) E Bs[NBUF][BN][LDK];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int kb = blockIdx.z * kchunk, ke = min(K, kb + kchunk);
  const int nst = (ke - kb) / BK;

  // global -> register staging: A as float4 (BM*BK/4 per stage), W as 16 B
  constexpr int AV = BM * BK / 4 / 256;  // float4 of A per thread per stage
  constexpr int WB = BN * BK * (int)sizeof(WT) / 16 / 256;  // 16-byte pieces of W per thread per stage
  static_assert(AV >= 1 && WB >= 1, "tile too small for 256 threads");
  float4 ra[NREG][AV];
  uint4 rw[NREG][WB];
  // bounded buffer resources over this block's rows of A and Wt: rows past M
  // (N) read as zeros, with no branch around the loads (a branch would make the
  // compiler wait for each load before the next one)
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(A + (size_t)m0 * K), (short)0, min(BM, M - m0) * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<WT*>(Wt + (size_t)n0 * K), (short)0, min(BN, N - n0) * K * (int)sizeof(WT), 0x00020000);
  auto gload = [&](float4 (&a)[AV], uint4 (&wv)[WB], int k0) {
#pragma unroll
    for (int i = 0; i < AV; i++) {
      const int idx = tid + 256 * i, row = idx / (BK / 4), kq = idx % (BK / 4);
      if constexpr (AOP != AOP_PLAIN) {
        a[i] = load_attn_a4(ao, m0 + row, k0 + 4 * kq, M, K);
      } else {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsa, (row * K + k0 + 4 * kq) * 4, 0, 0);
        a[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
      }
    }
    constexpr int PER_ROW = BK * (int)sizeof(WT) / 16;  // 16-byte pieces per W row and stage
    // the non-resident decode product (M <= 32 rows, W streamed stage by stage: the
    // tied head over tok_emb) reads W once per step: non-temporal hint (C4 849.5 ->
    // 841.5 us per step; on the resident split-K decode products it measured slower)
    constexpr int WAUX = (BM == 32 && NSR == 0) ? 2 : 0;
#pragma unroll
    for (int i = 0; i < WB; i++) {
      const int idx = tid + 256 * i, row = idx / PER_ROW, q = idx % PER_ROW;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsw, (row * K + k0) * (int)sizeof(WT) + 16 * q, 0, WAUX);
      wv[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  auto sstore = [&](int b, const float4 (&a)[AV], const uint4 (&wv)[WB]) {
#pragma unroll
    for (int i = 0; i < AV; i++) {
      const int idx = tid + 256 * i, row = idx / (BK / 4), kq = idx % (BK / 4);
      if constexpr (sizeof(WT) == 2) {
        const uint32_t lo = (uint32_t)bf16_rn(a[i].x) | ((uint32_t)bf16_rn(a[i].y) << 16);
        const uint32_t hi = (uint32_t)bf16_rn(a[i].z) | ((uint32_t)bf16_rn(a[i].w) << 16);
        *reinterpret_cast<uint2*>(&As[b][row][4 * kq]) = make_uint2(lo, hi);
      } else {
        // k = 4kq .. 4kq+3: even k to positions 2kq, 2kq+1; odd k to BK/2 + 2kq, +1
        *reinterpret_cast<float2*>(&As[b][row][2 * kq]) = make_float2(a[i].x, a[i].z);
        *reinterpret_cast<float2*>(&As[b][row][BK / 2 + 2 * kq]) = make_float2(a[i].y, a[i].w);
      }
    }
    constexpr int PER_ROW = BK * (int)sizeof(WT) / 16;
#pragma unroll
    for (int i = 0; i < WB; i++) {
      const int idx = tid + 256 * i, row = idx / PER_ROW, q = idx % PER_ROW;
      if constexpr (sizeof(WT) == 2) {
        *reinterpret_cast<uint4*>(&Bs[b][row][8 * q]) = wv[i];
      } else {
        const float4 v = make_float4(__uint_as_float(wv[i].x), __uint_as_float(wv[i].y), __uint_as_float(wv[i].z),
                                     __uint_as_float(wv[i].w));
        *reinterpret_cast<float2*>(&Bs[b][row][2 * q]) = make_float2(v.x, v.z);
        *reinterpret_cast<float2*>(&Bs[b][row][BK / 2 + 2 * q]) = make_float2(v.y, v.w);
      }
    }
  };

  f32x16_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[t][r] = 0.f;

  const int fr = lane & 31, fh = lane >> 5;  // fragment row / column and k half
  auto compute = [&](int b) {
    if constexpr (sizeof(WT) == 2) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; kk++) {
        const bf16x8_t bf = *reinterpret_cast<const bf16x8_t*>(&Bs[b][w * 32 + fr][kk * 16 + 8 * fh]);
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(&As[b][t * 32 + fr][kk * 16 + 8 * fh]);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc[t], 0, 0, 0);
        }
      }
    } else {
      // k step s covers k = 2s (lanes 0..31) and 2s + 1 (lanes 32..63)
#pragma unroll
      for (int q = 0; q < BK / 8; q++) {
        const float4 bq = *reinterpret_cast<const float4*>(&Bs[b][w * 32 + fr][fh * (BK / 2) + 4 * q]);
        float4 aq[MT];
#pragma unroll
        for (int t = 0; t < MT; t++)
          aq[t] = *reinterpret_cast<const float4*>(&As[b][t * 32 + fr][fh * (BK / 2) + 4 * q]);
#pragma unroll
        for (int t = 0; t < MT; t++) {
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[t].x, bq.x, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[t].y, bq.y, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[t].z, bq.z, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(aq[t].w, bq.w, acc[t], 0, 0, 0);
        }
      }
    }
  };

  if constexpr (NSR > 0) {
    // stages past the chunk re-read its last stage (never multiplied): no branches around the loads
#pragma unroll
    for (int s2 = 0; s2 < NSR; s2++) gload(ra[s2], rw[s2], kb + min(s2, nst - 1) * BK);
#pragma unroll
    for (int s2 = 0; s2 < NSR; s2++) sstore(s2, ra[s2], rw[s2]);
    __syncthreads();
#pragma unroll
    for (int s2 = 0; s2 < NSR; s2++)
      if (s2 < nst) compute(s2);
  } else {
    if (nst > 0) {
      gload(ra[0], rw[0], kb);
      sstore(0, ra[0], rw[0]);
    }
    __syncthreads();
    for (int st = 0; st < nst; st++) {
      const int b = st & 1;
      if (st + 1 < nst) gload(ra[0], rw[0], kb + (st + 1) * BK);
      compute(b);
      if (st + 1 < nst) sstore(b ^ 1, ra[0], rw[0]);
      __syncthreads();
    }
  }

  const int col = n0 + w * 32 + fr;
  if (col >= N) return;
  const int nrows = min(BM, M - m0);
  if (part) {
    // split-K partial of this block's K chunk: raw sums, no bias or epilogue (stored
    // with the non-temporal hint: read once, by the reduction or the attention)
    const __amdgpu_buffer_rsrc_t rp = rows_rsrc(part, (size_t)blockIdx.z * M + m0, nrows, N, 4);
#pragma unroll
    for (int t = 0; t < MT; t++) mfma_store_tile<EPI_NONE, false, false, 2>(acc[t], lane, t * 32, col, N, 0.f, rp, rp);
    return;
  }
  const float bcol = bias ? bias[col] : 0.f;
  const __amdgpu_buffer_rsrc_t ry = rows_rsrc(Y, m0, nrows, N, 4);
  const __amdgpu_buffer_rsrc_t rres = RES ? rows_rsrc(res, m0, nrows, N, 4) : ry;  // unused without RES
#pragma unroll
  for (int t = 0; t < MT; t++) mfma_store_tile<EPI, RES, false>(acc[t], lane, t * 32, col, N, bcol, rres, ry);
}

// Wt[n][k] = W[k][n] (one-time weight transpose at session load), 32x32 LDS tiles
template <typename WT>
__global__ __launch_bounds__(256) void k_transpose(const WT* __restrict__ W, int K, int N, WT* __restrict__ Wt) {
  __shared__ WT tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8)
    if (k0 + i < K && n0 + tx < N) tile[i][tx] = W[(size_t)(k0 + i) * N + n0 + tx];
  __syncthreads();
  for (int i = ty; i < 32; i += 8)
    if (n0 + i < N && k0 + tx < K) Wt[(size_t)(n0 + i) * K + k0 + tx] = tile[tx][i];
}

}  // namespace

template <typename WT>
hipError_t launch_transpose(hipStream_t st, const WT* W, int K, int N, WT* Wt) {
  if (!W || !Wt || K <= 0 || N <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_transpose<WT>, dim3((N + 31) / 32, (K + 31) / 32), dim3(256), 0, st, W, K, N, Wt);
  return hipGetLastError();
}

// the epilogue (GELU or not, residual or not) is a template parameter of the kernel
template <typename WT, int BM, int NSR>
static hipError_t launch_epi(hipStream_t st, dim3 grid, const float* a, int M, int K, const WT* Wt, int N, int kchunk,
                             const float* bias, int epi, const float* res, float* y, float* part) {
  const bool gelu = epi == EPI_GELU;
  const AOperand ao{};
  if (part || (!gelu && !res))
    hipLaunchKernelGGL((k_gemm_mfma<WT, BM, EPI_NONE, false, NSR>), grid, dim3(256), 0, st, a, M, K, Wt, N, kchunk,
                       bias, res, y, part, ao);
  else if (!gelu)
    hipLaunchKernelGGL((k_gemm_mfma<WT, BM, EPI_NONE, true, NSR>), grid, dim3(256), 0, st, a, M, K, Wt, N, kchunk,
                       bias, res, y, part, ao);
  else if (!res)
    hipLaunchKernelGGL((k_gemm_mfma<WT, BM, EPI_GELU, false, NSR>), grid, dim3(256), 0, st, a, M, K, Wt, N, kchunk,
                       bias, res, y, part, ao);
  else
    hipLaunchKernelGGL((k_gemm_mfma<WT, BM, EPI_GELU, true, NSR>), grid, dim3(256), 0, st, a, M, K, Wt, N, kchunk,
                       bias, res, y, part, ao);
  return hipGetLastError();
}

template <typename WT>
hipError_t launch_gemm_mfma(hipStream_t st, const float* a, int M, int K, const WT* Wt, int N, const float* bias,
                            int epi, const float* res, float* y, float* part, size_t part_floats, int cus) {
  if (!a || !Wt || !y || M <= 0 || N <= 0 || K <= 0 || K % BK != 0) return hipErrorInvalidValue;
  // byte offsets inside a block's rows of A and Wt are 32-bit
  if ((size_t)128 * K * 4 > 0x7fffffffu) return hipErrorInvalidValue;
  const int gn = (N + BN - 1) / BN;
  const int bm = M > 64 ? 128 : (M > 32 ? 64 : 32);
  const int gm = (M + bm - 1) / bm;
  // split K until the grid covers the CUs about twice (partials must fit)
  int S = 1;
  const int target = 2 * (cus > 0 ? cus : 256);
  while (gn * gm * S * 2 <= target && (K / BK) % (S * 2) == 0 && (size_t)S * 2 * M * N <= part_floats && part)
    S *= 2;
  const int kchunk = K / S;
  dim3 grid(gn, gm, S);
  float* pp = S > 1 ? part : nullptr;
  // chunks of at most 3 stages (split-K decode GEMMs) load all their stages at once
  const bool resident = kchunk <= 3 * BK;
  hipError_t e;
  if (bm == 128)
    e = launch_epi<WT, 128, 0>(st, grid, a, M, K, Wt, N, kchunk, bias, epi, res, y, pp);
  else if (bm == 64)
    e = resident ? launch_epi<WT, 64, 3>(st, grid, a, M, K, Wt, N, kchunk, bias, epi, res, y, pp)
                 : launch_epi<WT, 64, 0>(st, grid, a, M, K, Wt, N, kchunk, bias, epi, res, y, pp);
  else
    e = resident ? launch_epi<WT, 32, 3>(st, grid, a, M, K, Wt, N, kchunk, bias, epi, res, y, pp)
                 : launch_epi<WT, 32, 0>(st, grid, a, M, K, Wt, N, kchunk, bias, epi, res, y, pp);
  if (e != hipSuccess || S == 1) return e;
  return launch_splitk_epilogue(st, part, S, M, N, bias, epi, res, y);
}

template <typename WT, int BM, int NSR, int AOP>
static hipError_t launch_parts(hipStream_t st, dim3 grid, const float* a, int M, int K, const WT* Wt, int N,
                               int kchunk, float* part, const AOperand& ao) {
  hipLaunchKernelGGL((k_gemm_mfma<WT, BM, EPI_NONE, false, NSR, AOP>), grid, dim3(256), 0, st, a, M, K, Wt, N, kchunk,
                     nullptr, nullptr, part, part, ao);
  return hipGetLastError();
}

template <typename WT, int AOP>
static hipError_t launch_parts_bm(hipStream_t st, dim3 grid, int bm, bool resident, const float* a, int M, int K,
                                  const WT* Wt, int N, int kchunk, float* part, const AOperand& ao) {
  if (bm == 128) return launch_parts<WT, 128, 0, AOP>(st, grid, a, M, K, Wt, N, kchunk, part, ao);
  if (bm == 64)
    return resident ? launch_parts<WT, 64, 3, AOP>(st, grid, a, M, K, Wt, N, kchunk, part, ao)
                    : launch_parts<WT, 64, 0, AOP>(st, grid, a, M, K, Wt, N, kchunk, part, ao);
  return resident ? launch_parts<WT, 32, 3, AOP>(st, grid, a, M, K, Wt, N, kchunk, part, ao)
                  : launch_parts<WT, 32, 0, AOP>(st, grid, a, M, K, Wt, N, kchunk, part, ao);
}

template <typename WT>
hipError_t launch_gemm_mfma_split(hipStream_t st, const float* a, int M, int K, const WT* Wt, int N, float* part,
                                  size_t part_floats, int cus, int* splits, const AOperand* aop) {
  if (!Wt || !part || !splits || M <= 0 || N <= 0 || K <= 0 || K % BK != 0 || (size_t)M * N > part_floats)
    return hipErrorInvalidValue;
  if ((size_t)128 * K * 4 > 0x7fffffffu) return hipErrorInvalidValue;
  const int kind = aop ? aop->kind : AOP_PLAIN;
  if (kind == AOP_PLAIN && !a) return hipErrorInvalidValue;
  if (kind == AOP_ATTN && (!aop->apart || aop->H <= 0 || K % aop->H != 0 || (K / aop->H) % 4 != 0 ||
                           aop->chunk <= 0 || aop->maxc <= 0 || aop->maxc > kAttnChunksMax || !aop->src.step ||
                           (size_t)aop->maxc * aop->chunk < (size_t)aop->ctx))
    return hipErrorInvalidValue;
  const int gn = (N + BN - 1) / BN;
  const int bm = M > 64 ? 128 : (M > 32 ? 64 : 32);
  const int gm = (M + bm - 1) / bm;
  int S = 1;
  const int target = 2 * (cus > 0 ? cus : 256);
  while (gn * gm * S * 2 <= target && (K / BK) % (S * 2) == 0 && (size_t)S * 2 * M * N <= part_floats) S *= 2;
  // attn.proj of batched decode (N = d: 6 column tiles at d 768) takes any divisor
  // of its stage count up to 32 partials (the epilogue's loads in flight): 24 splits
  // on 144 blocks instead of 8 on 48 (C4 495.7 -> 489.1 ms per generate on one box;
  // the same rule for every split GEMM was slower)
  if (kind == AOP_ATTN)
    for (int s = std::min(32, K / BK); s > S; s--)
      if ((K / BK) % s == 0 && gn * gm * s <= target && (size_t)s * M * N <= part_floats) {
        S = s;
        break;
      }
  *splits = S;
  const int kchunk = K / S;
  dim3 grid(gn, gm, S);
  const bool resident = kchunk <= 3 * BK;
  const AOperand none{};
  if (kind == AOP_ATTN)
    return launch_parts_bm<WT, AOP_ATTN>(st, grid, bm, resident, a, M, K, Wt, N, kchunk, part, *aop);
  return launch_parts_bm<WT, AOP_PLAIN>(st, grid, bm, resident, a, M, K, Wt, N, kchunk, part, none);
}

template hipError_t launch_gemm_mfma_split<float>(hipStream_t, const float*, int, int, const float*, int, float*,
                                                  size_t, int, int*, const AOperand*);
template hipError_t launch_gemm_mfma_split<bf16_t>(hipStream_t, const float*, int, int, const bf16_t*, int, float*,
                                                   size_t, int, int*, const AOperand*);
template hipError_t launch_transpose<float>(hipStream_t, const float*, int, int, float*);
template hipError_t launch_transpose<bf16_t>(hipStream_t, const bf16_t*, int, int, bf16_t*);
template hipError_t launch_gemm_mfma<float>(hipStream_t, const float*, int, int, const float*, int, const float*, int,
                                            const float*, float*, float*, size_t, int);
template hipError_t launch_gemm_mfma<bf16_t>(hipStream_t, const float*, int, int, const bf16_t*, int, const float*,
                                             int, const float*, float*, float*, size_t, int);

}  // namespace fh
