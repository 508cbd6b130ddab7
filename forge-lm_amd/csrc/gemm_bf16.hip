// gemm_bf16.hip -- large-M bf16 GEMM for prefill in bf16 sessions (gfx950).
//
// Linear.Forward (src/LLM.Core/Layers/Layers.cs:29-37) over a whole window:
// y = epi(a @ W + b) (+ res) with a [M][K] already in bf16 (the LayerNorm,
// attention and GELU kernels that produce a write it rounded, as the reference
// comparison's bf16 activations are) and W transposed as Wt[N][K] bf16.  Both
// operands are k-contiguous in HBM and in LDS.
//
// A block computes a BM x 128 tile of y (BM 256 or 128) with 4 waves in a 2 x 2
// arrangement, each wave a (BM/2) x 64 sub-tile of (BM/64) x 2 MFMA 32x32x16
// accumulators: per 16-k step a wave reads BM/64 + 2 fragments from LDS for
// 2 * BM/64 MFMAs, which keeps LDS reads under the CU's LDS bandwidth at full
// MFMA rate.  K advances 32 per stage through a double-buffered LDS pair; the
// 16-byte global loads (bounded buffer loads: rows past M or N read as zeros)
// of stage s + 2 are in flight in a second register set while stage s is
// multiplied, which covers the ~800-cycle load latency measured under this
// kernel's load.  Two blocks fit a CU (48 KB of LDS each at BM 256), so one
// block's barrier and LDS waits hide behind the other's MFMAs.
//
// The blocks are dispatched to the 8 XCDs in turn; the tile order gives each
// XCD a contiguous run of row-major tiles, so the A rows a run shares are
// fetched into one L2.
#include "kernels.hpp"
#include "mfma_epi.hpp"

namespace fh {

namespace {

constexpr int TN = 128;       // columns per block
constexpr int TK = 32;        // k per stage
constexpr int LDK = TK;       // bf16 per LDS row: 64 B, four 16-byte chunks
constexpr int SROW = 64 + 8;  // bf16 per row of a wave's output staging (64 columns + pad)

// LDS position of 16-byte chunk c of tile row r: chunks are XOR-swizzled by
// bits 2-3 of the row, so a 16-lane group reading chunk c of 16 consecutive rows
// (a fragment read) and one writing the 4 chunks of 4 consecutive rows (a
// staging store) both touch each of the 64 banks once
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 2) & 3); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int BM, int EPI, bool RES, bool OUT_BF16>
__global__ __launch_bounds__(256, 2) void k_gemm_bf16(const bf16_t* __restrict__ A, int M, int K,
                                                     const bf16_t* __restrict__ Wt, int N,
                                                     const float* __restrict__ bias, GemmBf16Out o, int gm,
                                                     int gn) {
  constexpr int MT = BM / 64;                 // 32-row accumulator tiles per wave
  constexpr int NT = 2;                       // 32-column accumulator tiles per wave
  constexpr int AP = BM * TK / 8 / 256;       // 16-byte A pieces per thread and stage
  constexpr int BP = TN * TK / 8 / 256;       // 16-byte W pieces per thread and stage
  static_assert(AP >= 1 && BP >= 1, "tile too small for 256 threads");
  // operand tiles; after the last stage the same LDS stages the bf16 outputs
  constexpr int SMEM_OPS = 2 * (BM + TN) * LDK * 2, SMEM_STG = 4 * 64 * SROW * 2;
  constexpr int SMEM = SMEM_OPS > SMEM_STG ? SMEM_OPS : SMEM_STG;
  __shared__ __align__(16) char smem[SMEM];
  typedef bf16_t ATile[BM][LDK];
  typedef bf16_t BTile[TN][LDK];
  ATile* As = reinterpret_cast<ATile*>(smem);
  BTile* Bs = reinterpret_cast<BTile*>(smem + 2 * BM * LDK * 2);

  // tile of this block: XCD x = bid % 8 takes tiles [x * T/8, (x+1) * T/8) when 8 divides T
  const int ntiles = gm * gn, bid = blockIdx.x;
  const int t = (ntiles % 8 == 0) ? (bid % 8) * (ntiles / 8) + bid / 8 : bid;
  const int m0 = (t / gn) * BM, n0 = (t % gn) * TN;

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w & 1, wn = w >> 1;
  const int fr = lane & 31, fh = lane >> 5;   // fragment row and k half

  // bounded resources over this block's rows: loads past row M (N) return zeros
  const int arows = min(BM, M - m0), brows = min(TN, N - n0);
  const __amdgpu_buffer_rsrc_t ra_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(A + (size_t)m0 * K), (short)0, arows * K * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(Wt + (size_t)n0 * K), (short)0, brows * K * 2, 0x00020000);
  // piece i of this thread: row (tid / 4) + 64 i, 16 bytes at k offset 8 * (tid % 4)
  const int prow = tid >> 2, pq = tid & 3;
  // two register sets: the loads for stage s + 2 are issued while stage s is
  // multiplied, so each load has two stages of MFMAs to arrive
  uint4 ra0[AP], rb0[BP], ra1[AP], rb1[BP];
  auto gload = [&](uint4 (&ra)[AP], uint4 (&rb)[BP], int k0) {
#pragma unroll
    for (int i = 0; i < AP; i++) ra[i] = load16(ra_rs, ((prow + 64 * i) * K + k0 + 8 * pq) * 2);
#pragma unroll
    for (int i = 0; i < BP; i++) rb[i] = load16(rb_rs, ((prow + 64 * i) * K + k0 + 8 * pq) * 2);
  };
  auto sstore = [&](int b, const uint4 (&ra)[AP], const uint4 (&rb)[BP]) {
#pragma unroll
    for (int i = 0; i < AP; i++) *reinterpret_cast<uint4*>(&As[b][prow + 64 * i][8 * swz(prow, pq)]) = ra[i];
#pragma unroll
    for (int i = 0; i < BP; i++) *reinterpret_cast<uint4*>(&Bs[b][prow + 64 * i][8 * swz(prow, pq)]) = rb[i];
  };

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  auto compute = [&](int b) {
#pragma unroll
    for (int kk = 0; kk < TK / 16; kk++) {
      bf16x8_t bf[NT];
#pragma unroll
      for (int j = 0; j < NT; j++)
        bf[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[b][wn * 64 + j * 32 + fr][8 * swz(fr, 2 * kk + fh)]);
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const bf16x8_t af =
            *reinterpret_cast<const bf16x8_t*>(&As[b][wm * (BM / 2) + i * 32 + fr][8 * swz(fr, 2 * kk + fh)]);
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // stages alternate LDS buffers 0 and 1 and register sets 0 and 1; the stage
  // count is even (K % 64 == 0).  Loads past the last stage re-read it (their
  // values are stored into a buffer nobody reads again), which keeps the loop
  // free of branches around loads.
  const int nst = K / TK;
  gload(ra0, rb0, 0);
  gload(ra1, rb1, TK);
  sstore(0, ra0, rb0);
  __syncthreads();
  for (int st = 0; st < nst; st += 2) {
    gload(ra0, rb0, min(st + 2, nst - 1) * TK);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs, not after them
    compute(0);
    sstore(1, ra1, rb1);
    __syncthreads();
    gload(ra1, rb1, min(st + 3, nst - 1) * TK);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    sstore(0, ra0, rb0);
    __syncthreads();
  }

  if constexpr (OUT_BF16) {
    // bf16 outputs leave through LDS: each wave writes 64 rows x 64 columns of
    // its sub-tile at a time (bias and GELU applied, rounded), then reads them
    // back as 16-byte row pieces (8 columns) for 16-byte global stores.  The
    // staging is wave-private: LDS ops of one wave complete in order.
    bf16_t* stg = reinterpret_cast<bf16_t*>(smem) + w * 64 * SROW;
    float bcol[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int col = n0 + wn * 64 + j * 32 + fr;
      bcol[j] = (bias && col < N) ? bias[col] : 0.f;
    }
    const int cc = lane & 7;                       // 8-column piece of a staged row
    const int col8 = n0 + wn * 64 + cc * 8;        // its first column
    int part = 0, hcol = 0, pos0 = 0, D = 0;
    if constexpr (EPI == EPI_QKV) {
      D = N / 3;
      part = (n0 + wn * 64) / D;                   // the 64 columns lie in one of q, K, V (64 | D)
      hcol = col8 - part * D;                      // h * 64 + e
      pos0 = o.src.pos_off + o.src.pos_mul * *o.src.step;
    }
#pragma unroll
    for (int half = 0; half < MT / 2; half++) {
#pragma unroll
      for (int ii = 0; ii < 2; ii++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            float v = acc[2 * half + ii][j][r] + bcol[j];
            if constexpr (EPI == EPI_GELU) v = gelu_for_bf16(v);
            stg[(ii * 32 + mfma_acc_row(lane, r)) * SROW + j * 32 + fr] = bf16_rn(v);
          }
#pragma unroll
      for (int it = 0; it < 8; it++) {
        const int rr = it * 8 + (lane >> 3);
        const uint4 val = *reinterpret_cast<const uint4*>(&stg[rr * SROW + cc * 8]);
        const int row = m0 + wm * (BM / 2) + half * 64 + rr;
        if (row >= M || col8 >= N) continue;
        if constexpr (EPI == EPI_QKV) {
          if (part == 0) {
            *reinterpret_cast<uint4*>(o.q + (size_t)row * D + hcol) = val;
          } else {
            const int b = row / o.T, pos = pos0 + (row - b * o.T);
            bf16_t* cache = part == 1 ? o.kc : o.vc;
            if ((unsigned)pos < (unsigned)o.ctx)
              *reinterpret_cast<uint4*>(cache + (((size_t)b * o.H + (hcol >> 6)) * o.ctx + pos) * 64 + (hcol & 63)) =
                  val;
          }
        } else {
          *reinterpret_cast<uint4*>(o.yh + (size_t)row * N + col8) = val;
        }
      }
    }
    return;
  }
  const int nrows = min(BM, M - m0);
  const __amdgpu_buffer_rsrc_t ry = rows_rsrc(o.y, m0, nrows, N, 4);
  const __amdgpu_buffer_rsrc_t rres = RES ? rows_rsrc(o.res, m0, nrows, N, 4) : ry;  // unused without RES
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int col = n0 + wn * 64 + j * 32 + fr;
    if (col < N) {
      const float bcol = bias ? bias[col] : 0.f;
#pragma unroll
      for (int i = 0; i < MT; i++)
        mfma_store_tile<EPI, RES, false>(acc[i][j], lane, wm * (BM / 2) + i * 32, col, N, bcol, rres, ry);
    }
  }
}

}  // namespace

template <int BM, int EPI, bool RES, bool OUT_BF16>
static hipError_t launch_tiles(hipStream_t st, int gm, int gn, const bf16_t* a, int M, int K, const bf16_t* Wt,
                               int N, const float* bias, const GemmBf16Out& o) {
  hipLaunchKernelGGL((k_gemm_bf16<BM, EPI, RES, OUT_BF16>), dim3(gm * gn), dim3(256), 0, st, a, M, K, Wt, N, bias, o,
                     gm, gn);
  return hipGetLastError();
}

template <int BM>
static hipError_t launch_bm(hipStream_t st, int gm, int gn, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                            const float* bias, int epi, const GemmBf16Out& o) {
  const bool gelu = epi == EPI_GELU, res = o.res != nullptr;
  if (epi == EPI_QKV) return launch_tiles<BM, EPI_QKV, false, true>(st, gm, gn, a, M, K, Wt, N, bias, o);
  if (!gelu && !res && o.y) return launch_tiles<BM, EPI_NONE, false, false>(st, gm, gn, a, M, K, Wt, N, bias, o);
  if (!gelu && res && o.y) return launch_tiles<BM, EPI_NONE, true, false>(st, gm, gn, a, M, K, Wt, N, bias, o);
  if (gelu && !res && o.yh) return launch_tiles<BM, EPI_GELU, false, true>(st, gm, gn, a, M, K, Wt, N, bias, o);
  if (gelu && !res && o.y) return launch_tiles<BM, EPI_GELU, false, false>(st, gm, gn, a, M, K, Wt, N, bias, o);
  return hipErrorInvalidValue;  // an epilogue combination no caller uses
}

static hipError_t launch_any(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                             const float* bias, int epi, const GemmBf16Out& o) {
  // bf16 outputs leave as 16-byte pieces of 8 columns
  if (!a || !Wt || M <= 0 || N <= 0 || K <= 0 || K % (2 * TK) != 0 || ((o.yh || o.q) && N % 8 != 0))
    return hipErrorInvalidValue;
  // byte offsets inside a block's rows (operands and outputs) are 32-bit
  if ((size_t)256 * K * 2 > 0x7fffffffu || (size_t)256 * N * 4 > 0x7fffffffu) return hipErrorInvalidValue;
  const int gn = (N + TN - 1) / TN;
  // 256-row tiles while they give two tiles per CU (two blocks fit a CU); 128 below
  // that (attn.proj and mlp.proj at N 1024: 512 tiles of 128 rows instead of 256
  // of 256, measured 2 % faster on the whole C5 forward)
  const int gm256 = (M + 255) / 256, gm128 = (M + 127) / 128;
  if (gm256 * gn >= 512) return launch_bm<256>(st, gm256, gn, a, M, K, Wt, N, bias, epi, o);
  return launch_bm<128>(st, gm128, gn, a, M, K, Wt, N, bias, epi, o);
}

hipError_t launch_gemm_bf16(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                            const float* bias, int epi, const float* res, float* y, bf16_t* yh) {
  if ((!y) == (!yh) || epi == EPI_QKV) return hipErrorInvalidValue;
  GemmBf16Out o{};
  o.res = res;
  o.y = y;
  o.yh = yh;
  return launch_any(st, a, M, K, Wt, N, bias, epi, o);
}

hipError_t launch_gemm_bf16_qkv(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, const float* bias,
                                RowSrc src, int T, int H, int ctx, bf16_t* q, bf16_t* kcache, bf16_t* vcache) {
  const int D = 64 * H;
  if (!q || !kcache || !vcache || !src.step || T <= 0 || H <= 0 || ctx <= 0 || M % T != 0) return hipErrorInvalidValue;
  GemmBf16Out o{};
  o.q = q;
  o.kc = kcache;
  o.vc = vcache;
  o.src = src;
  o.T = T;
  o.H = H;
  o.ctx = ctx;
  return launch_any(st, a, M, K, Wt, 3 * D, bias, EPI_QKV, o);
}

}  // namespace fh
