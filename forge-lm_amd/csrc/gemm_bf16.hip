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
#include <type_traits>

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

// ---- 8-wave ping-pong kernel for windows of many rows -------------------------
//
// A block of 8 waves computes BM x 256 tiles (BM 256 or 128), one CU each,
// looping over the tiles of its XCD's run.  The waves form two groups of four
// (each SIMD holds one wave of each): group g owns rows [g BM/2, (g+1) BM/2) of
// the tile, wave q of a group columns [64 q, 64 q + 64).  The groups alternate
// between two phases separated by barriers: while one multiplies a 32-k step
// from fragments already in its registers (16 MFMAs, nothing else), the other
// reads its fragments of the next step from LDS and issues direct-to-LDS loads
// of the operands two steps ahead, so each SIMD's matrix unit always has one
// wave feeding it.  K steps rotate through four LDS stages (A rows, then W rows,
// 64-byte rows with the chunks XOR-swizzled as above).  The products are formed
// as (W a^T) tiles, W fragment first: a lane then holds 4 consecutive columns of
// one row, so the epilogue stores 16-byte (fp32) or 8-byte (bf16) pieces.  The
// accumulation order per output equals k_gemm_bf16's (16-k MFMA steps in k
// order), so both kernels give the same bits.
constexpr int PBN = 256;  // columns per tile
constexpr int PNB = 4;    // LDS stages

// The lane index as a value the compiler cannot move out of a loop: the
// epilogue's per-lane addresses are then formed where they are used instead of
// being held in registers through the whole tile loop.
__device__ __forceinline__ int opaque_lane() {
  int l;
  asm volatile("v_and_b32 %0, 63, %1" : "=v"(l) : "v"((int)threadIdx.x));
  return l;
}

// a barrier nothing is scheduled across; VM >= 0 first waits until at most VM of
// this wave's vector memory operations are in flight
template <int VM>
__device__ __forceinline__ void pp_sync() {
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (VM == 3) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
  if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// SPLIT (BM 256, fp32 y with the residual): items are (tile, K half) pairs, both
// halves of a tile in one XCD's run; the first half to finish stores its raw sums
// in o.ws and marks the tile's counter ready, the second waits for the mark, adds
// them and runs the epilogue, then clears the counter for the next launch.  The
// sums pass through the XCD's L2 (plain stores, loads that miss the CU's L1), so
// both halves must run on one XCD: workgroups reach the XCDs round-robin by index
// (continuing from the previous dispatch, so blocks b and b + 8 share one), the
// two halves of a tile are such a pair, each adds its hardware XCD to the tile's
// counter, and a second half that finds the first on another XCD writes NaN
// instead of sums it might not see.  Either failure (that, or a ready mark that
// does not come within the wait's bound) also sets the error word o.err, which
// the host reads after the stream has finished.  Whichever half touches a
// tile's counter last returns it to zero: normally the second half once it has
// seen the mark; after the second half gave up (SPLIT_GAVEUP), the first half
// when it sets the mark, so no stale mark survives into the next launch.
constexpr int SPLIT_READY = 0x10000, SPLIT_GAVEUP = 0x20000;
// The even item's share of K, in sixteenths: 7 / 16 lets most first halves store
// their sums while the second halves still multiply (C5 4.68 against 4.71 ms per
// window for 8 / 16 on one box; 6 / 16 4.76)
constexpr int SPLIT_FIRST16 = 7;

__device__ __forceinline__ int hw_xcc() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return (int)(v & 0xf);
}

template <int BM, int EPI, bool OUT_BF16, bool SPLIT = false>
__global__ __launch_bounds__(512, 1) void k_gemm_bf16_pp(const bf16_t* __restrict__ A, int M, int K,
                                                        const bf16_t* __restrict__ Wt, int N,
                                                        const float* __restrict__ bias, GemmBf16Out o, int gm,
                                                        int gn) {
  constexpr int MT = BM / 64;              // 32-row accumulator tiles per wave
  constexpr int NI = (BM + PBN) / 16;      // direct-to-LDS loads (16 rows each) per K step
  constexpr int NW = NI / 8;               // of them per wave
  static_assert(NI % 8 == 0 && (NW == 3 || NW == 4), "load split");
  __shared__ __align__(16) bf16_t S[PNB][BM + PBN][TK];
  __shared__ __align__(16) float bias_s[PBN];  // the tile's bias, staged at its start
  __shared__ int role_s, ready_s;  // SPLIT: the tile's counter before this half arrived; the mark was seen
  static_assert(!SPLIT || (BM == 256 && EPI == EPI_NONE && !OUT_BF16), "split: fp32 y with the residual");
  const int ntiles = SPLIT ? 2 * gm * gn : gm * gn, bid = blockIdx.x, nb = gridDim.x;
  // XCD x = bid % 8 takes the items of the run [x T/8, (x+1) T/8) when 8 divides T and the grid
  const bool runs = ntiles % 8 == 0 && nb % 8 == 0;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = w >> 2, q = w & 3;
  const int fr = lane & 31, fh = lane >> 5;
  const int lrow = lane >> 2, lpos = lane & 3;  // a load's lane i fills row i / 4, position i % 4
  const int nkall = K / TK;
  for (int it = 0;; it++) {
    const int tt = runs ? bid / 8 + it * (nb / 8) : bid + it * nb;
    if (tt >= (runs ? ntiles / 8 : ntiles)) break;
    const int item = runs ? (bid % 8) * (ntiles / 8) + tt : tt;
    // SPLIT: the first half (even item) takes SPLIT_FIRST16 / 16 of the K steps
    const int kfirst = SPLIT ? nkall * SPLIT_FIRST16 / 16 : nkall;
    const int t = SPLIT ? item >> 1 : item, ks0 = SPLIT ? (item & 1) * kfirst : 0;  // tile, first K step
    const int nk = SPLIT ? ((item & 1) ? nkall - kfirst : kfirst) : nkall;  // K steps of this item
    const int m0 = (t / gn) * BM, n0 = (t % gn) * PBN;
    const int arows = min(BM, M - m0), brows = min(PBN, N - n0);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(A + (size_t)m0 * K), (short)0, arows * K * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(Wt + (size_t)n0 * K), (short)0, brows * K * 2, 0x00020000);
    // load ii of a K step fills LDS rows [16 ii, 16 ii + 16) (A rows, then W rows);
    // group g issues [g NI/2, (g+1) NI/2), wave q NW of them.  Steps past the last
    // re-read it into a stage nobody reads again (no branches around loads).
    auto dma = [&](int kt) {
      const int buf = kt % PNB, k0 = (ks0 + min(kt, nk - 1)) * TK;
#pragma unroll
      for (int j = 0; j < NW; j++) {
        const int ii = g * (NI / 2) + q * NW + j;
        const bool isA = ii < BM / 16;
        const int row = (isA ? 16 * ii : 16 * ii - BM) + lrow;
        const int c = lpos ^ ((row >> 2) & 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? ra : rb,
                                                 (__attribute__((address_space(3))) void*)&S[buf][16 * ii][0], 16,
                                                 (row * K + k0 + 8 * c) * 2, 0, 0, 0);
      }
    };
    f32x16_t acc[2][MT];  // [column tile][row tile]: accumulator rows are columns of y, lanes rows of y
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int i = 0; i < MT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][i][r] = 0.f;
    bf16x8_t af[2][MT], bw[2][2];
    auto frags = [&](int kt) {
      const int buf = kt % PNB;
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
#pragma unroll
        for (int i = 0; i < MT; i++)
          af[kk][i] =
              *reinterpret_cast<const bf16x8_t*>(&S[buf][g * (BM / 2) + i * 32 + fr][8 * swz(fr, 2 * kk + fh)]);
#pragma unroll
        for (int j = 0; j < 2; j++)
          bw[kk][j] = *reinterpret_cast<const bf16x8_t*>(&S[buf][BM + q * 64 + j * 32 + fr][8 * swz(fr, 2 * kk + fh)]);
      }
    };
    auto mfma = [&]() {
#pragma unroll
      for (int kk = 0; kk < 2; kk++)
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int j = 0; j < 2; j++)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[kk][j], af[kk][i], acc[j][i], 0, 0, 0);
    };
    // K steps 0 and 1 (group 0 loads the A rows, group 1 the W rows of each), and
    // the bias into LDS: the epilogue then issues no load between its stores
    dma(0);
    dma(1);
    if (tid < PBN) {
      const float bv = (bias && n0 + tid < N) ? bias[n0 + tid] : 0.f;
      bias_s[tid] = bv;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    pp_sync<0>();
    // Step u: group 0 reads its fragments of u and loads u + 2 (phase 2u - 1), then
    // multiplies u (phase 2u); group 1 multiplies u - 1 (phase 2u - 1), then reads
    // and loads (phase 2u).  Stage u % 4 is read in phases 2u - 1 and 2u and
    // refilled (step u + 4) from phase 2u + 3 on; each wave's loads of step u + 1
    // have landed (vmcnt) before the barrier that opens phase 2u + 1.
    if (g == 0) {
      for (int u = 0; u < nk; u++) {
        frags(u);
        dma(u + 2);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        pp_sync<-1>();
        mfma();
        pp_sync<NW>();
      }
    } else {
      for (int u = 0; u < nk; u++) {
        if (u > 0) mfma();
        pp_sync<-1>();
        frags(u);
        dma(u + 2);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        pp_sync<NW>();
      }
      mfma();
    }
    // epilogue: lane (fr, fh), register 4 a + b of acc[j][i] is column
    // n0 + 64 q + 32 j + 8 a + 4 fh + b of row m0 + BM/2 g + 32 i + fr.  Each
    // 32-row chunk i of a wave goes through LDS (bias and GELU applied, rounded
    // for bf16 outputs), in 16-byte units XOR-swizzled by row, and leaves as
    // whole row pieces: 16 lanes x 16 bytes per fp32 row of 64 columns, 8 per
    // bf16 row.  Rows past M and columns past N are dropped by the buffer bounds
    // (offsets past them), not branches; no load sits between the stores (loads
    // and stores share one completion counter).
    pp_sync<0>();  // the last loads have landed and every wave is past its fragment reads
    bool second = false, xok = true;  // SPLIT: this half adds the other's sums and writes y
    if constexpr (SPLIT) {
      const int xcc = hw_xcc();
      if (tid == 0)
        role_s = __hip_atomic_fetch_add(o.cnt + t, 1 + ((xcc + 1) << 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      second = (role_s & 0xf) != 0;
      xok = !second || ((role_s >> 4) & 0xff) == xcc + 1;  // the first half ran on this XCD
      if (second) {
        // the first half has arrived: wait (bounded) until its sums are stored
        if (tid == 0) {
          int ok = 0;
          for (int n = 0; n < (1 << 22) && !ok; n++) {
            ok = (__hip_atomic_load(o.cnt + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & SPLIT_READY) != 0;
            if (!ok) __builtin_amdgcn_s_sleep(2);
          }
          // giving up: the mark may still have come in between (then the sums are
          // there); otherwise the first half, setting it later, clears the counter
          if (!ok)
            ok = (__hip_atomic_fetch_or(o.cnt + t, SPLIT_GAVEUP, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                  SPLIT_READY) != 0;
          if (ok) __hip_atomic_store(o.cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
          if ((!ok || !xok) && o.err)
            __hip_atomic_fetch_or(o.err, ok ? 2 : 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ready_s = ok;
        }
        __syncthreads();
      }
    }
    const bool bad = SPLIT && second && (ready_s == 0 || !xok);  // not ready, or not one XCD: y is NaN
    const int el = opaque_lane(), efr = el & 31, efh = el >> 5;
    int pos0 = 0, D = 0, part = 0;
    if constexpr (EPI == EPI_QKV) {
      D = N / 3;
      pos0 = o.src.pos_off + o.src.pos_mul * *o.src.step;
      part = (n0 + q * 64) / D;  // the wave's 64 columns lie in one of q, K, V (64 | D)
    }
    const int mrows = min(BM, M - m0);
    constexpr int YE = OUT_BF16 ? 2 : 4;
    // SPLIT: the first half writes its sums to ws, the second y (reading ws and the residual)
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
        OUT_BF16 ? static_cast<void*>(o.yh + (size_t)m0 * N)
                 : static_cast<void*>((SPLIT && !second ? o.ws : o.y) + (size_t)m0 * N),
        (short)0, EPI == EPI_QKV ? 0 : mrows * N * YE, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(SPLIT ? o.ws + (size_t)m0 * N : o.y, (short)0, SPLIT ? mrows * N * 4 : 0,
                                          0x00020000);
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(SPLIT ? o.res + (size_t)m0 * N : nullptr), (short)0, SPLIT ? mrows * N * 4 : 0,
        0x00020000);
    // 32 rows x 256 bytes per wave (SPLIT: 16 KB per wave, the other half's sums and the residual)
    char* stg = reinterpret_cast<char*>(&S[0][0][0]) + w * (SPLIT ? 16384 : 8192);
    static_assert(!SPLIT || sizeof(S) >= 8 * 16384, "split staging");
    // read-back role of lane l: fp32 rows 4 k + l / 16 (k < 8), unit l % 16 (4 columns);
    // bf16 rows 8 k + l / 8 (k < 4), unit l % 8 (8 columns).  A buffer's range
    // check covers the vector offset only, so the whole offset goes there: the
    // lane's row and columns, or 2^31 (past every bound: the host keeps a tile's
    // rows under 2^31 bytes) when its columns lie past N.
    constexpr int RK = OUT_BF16 ? 4 : 8, RS = OUT_BF16 ? 8 : 4;
    const int ru = OUT_BF16 ? (el & 7) : (el & 15), rrow0 = OUT_BF16 ? (el >> 3) : (el >> 4);
    const int gcol = n0 + q * 64 + (OUT_BF16 ? 8 : 4) * ru;  // first column of the lane's piece
    auto eoff = [&](int i, int k, int esz) {
      const int lr = g * (BM / 2) + i * 32 + RS * k + rrow0;  // row within the tile
      return gcol < N ? (unsigned)((lr * N + gcol) * esz) : 0x80000000u;
    };
#pragma unroll
    for (int i = 0; i < MT; i++) {
      // 1. this chunk into the wave's staging rows (SPLIT: the raw sums; the
      // second half adds the other half's sums, the bias and the residual there)
      if constexpr (SPLIT) {
        if (second) {
          // the other half's sums and the residual of the chunk by direct-to-LDS
          // loads into the wave's 16 KB (sums, then residual), in the staging
          // layout: load k, lane l fills row 4k + l / 16 at unit position l % 16
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous chunk's read-back is done
#pragma unroll
          for (int k = 0; k < 8; k++) {
            const int cr = 4 * k + rrow0, uc = ru ^ (cr & 15);  // the piece's row and logical unit
            const int lr = g * (BM / 2) + i * 32 + cr, c = n0 + q * 64 + 4 * uc;
            const unsigned off = c < N ? (unsigned)((lr * N + c) * 4) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)(stg + 1024 * k), 16,
                                                     off, 0, 0, 17);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rr, (__attribute__((address_space(3))) void*)(stg + 8192 + 1024 * k), 16, off, 0, 0, 0);
          }
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
          for (int j = 0; j < 2; j++)
#pragma unroll
            for (int a = 0; a < 4; a++) {
              const int u = (8 * j + 2 * a + efh) ^ (efr & 15);
              float4* py = reinterpret_cast<float4*>(stg + efr * 256 + u * 16);
              const float4 pv = *py, rv = *reinterpret_cast<const float4*>(stg + 8192 + efr * 256 + u * 16);
              const float4 bc = *reinterpret_cast<const float4*>(&bias_s[q * 64 + j * 32 + 8 * a + 4 * efh]);
              // ((own + other half) + bias) + residual: the same bits whichever half came first
              float4 yv = make_float4(((acc[j][i][4 * a] + pv.x) + bc.x) + rv.x,
                                      ((acc[j][i][4 * a + 1] + pv.y) + bc.y) + rv.y,
                                      ((acc[j][i][4 * a + 2] + pv.z) + bc.z) + rv.z,
                                      ((acc[j][i][4 * a + 3] + pv.w) + bc.w) + rv.w);
              if (bad) yv = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
              *py = yv;
            }
        }
      }
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int a = 0; a < 4; a++) {
          if (SPLIT && second) break;  // staged above
          const float4 bc = SPLIT ? make_float4(0.f, 0.f, 0.f, 0.f)
                                  : *reinterpret_cast<const float4*>(&bias_s[q * 64 + j * 32 + 8 * a + 4 * efh]);
          const float bcv[4] = {bc.x, bc.y, bc.z, bc.w};
          float v[4];
#pragma unroll
          for (int b = 0; b < 4; b++) {
            v[b] = SPLIT ? acc[j][i][4 * a + b] : acc[j][i][4 * a + b] + bcv[b];
            if constexpr (EPI == EPI_GELU) v[b] = OUT_BF16 ? gelu_for_bf16(v[b]) : gelu_tanh(v[b]);
          }
          if constexpr (OUT_BF16) {
            typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t pk = {(unsigned)__builtin_bit_cast(unsigned short, bf16_rn(v[0])) |
                                    ((unsigned)__builtin_bit_cast(unsigned short, bf16_rn(v[1])) << 16),
                                (unsigned)__builtin_bit_cast(unsigned short, bf16_rn(v[2])) |
                                    ((unsigned)__builtin_bit_cast(unsigned short, bf16_rn(v[3])) << 16)};
            const int u = (4 * j + a) ^ (efr & 7);  // 16-byte unit of the 128-byte row, half fh
            *reinterpret_cast<u32x2_t*>(stg + efr * 128 + u * 16 + efh * 8) = pk;
          } else {
            const int u = (8 * j + 2 * a + efh) ^ (efr & 15);
            *reinterpret_cast<float4*>(stg + efr * 256 + u * 16) = make_float4(v[0], v[1], v[2], v[3]);
          }
        }
      // 2. whole row pieces out (the wave's LDS operations complete in order)
#pragma unroll
      for (int k = 0; k < RK; k++) {
        const int cr = rrow0 + RS * k;  // row within the chunk
        const int row = m0 + g * (BM / 2) + i * 32 + cr;
        if constexpr (OUT_BF16) {
          const u32x4_t x = *reinterpret_cast<const u32x4_t*>(stg + cr * 128 + ((ru ^ (cr & 7)) * 16));
          if constexpr (EPI == EPI_QKV) {
            const int e = gcol - part * D;
            if (row < M && gcol < N) {
              if (part == 0) {
                *reinterpret_cast<u32x4_t*>(o.q + (size_t)row * D + e) = x;
              } else {
                const int bb = row / o.T, pos = pos0 + (row - bb * o.T);
                bf16_t* cache = part == 1 ? o.kc : o.vc;
                if ((unsigned)pos < (unsigned)o.ctx)
                  *reinterpret_cast<u32x4_t*>(cache + (((size_t)bb * o.H + (e >> 6)) * o.ctx + pos) * 64 +
                                              (e & 63)) = x;
              }
            }
          } else {
            __builtin_amdgcn_raw_buffer_store_b128(x, ry, eoff(i, k, 2), 0, 0);
          }
        } else {
          const u32x4_t x = *reinterpret_cast<const u32x4_t*>(stg + cr * 256 + ((ru ^ (cr & 15)) * 16));
          __builtin_amdgcn_raw_buffer_store_b128(x, ry, eoff(i, k, 4), 0, 0);
        }
      }
    }
    if constexpr (SPLIT) {
      if (!second) {
        // every wave's stores of the sums have completed; then the tile is marked ready
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0 &&
            (__hip_atomic_fetch_or(o.cnt + t, SPLIT_READY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & SPLIT_GAVEUP))
          __hip_atomic_store(o.cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // the second half gave up
      }
    }
    // every wave is past its LDS reads and stores before the next tile's loads
    pp_sync<0>();
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

template <int BM, int EPI, bool OUT_BF16, bool SPLIT = false>
static hipError_t launch_pp_tiles(hipStream_t st, int gm, int gn, int nb, const bf16_t* a, int M, int K,
                                  const bf16_t* Wt, int N, const float* bias, const GemmBf16Out& o) {
  hipLaunchKernelGGL((k_gemm_bf16_pp<BM, EPI, OUT_BF16, SPLIT>), dim3(nb), dim3(512), 0, st, a, M, K, Wt, N, bias, o,
                     gm, gn);
  return hipGetLastError();
}

// one block per CU (rounded down to a multiple of 8, the XCD count), at most one per tile
static int pp_blocks(int ntiles) {
  static const int cus = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || v < 8)
      return 8;
    return v / 8 * 8;
  }();
  return ntiles < cus ? ntiles : cus;
}

template <int BM>
static hipError_t launch_pp(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                            const float* bias, int epi, const GemmBf16Out& o) {
  const int gm = (M + BM - 1) / BM, gn = (N + PBN - 1) / PBN, nb = pp_blocks(gm * gn);
  const bool gelu = epi == EPI_GELU;
  if (o.res) return hipErrorInvalidValue;  // residual GEMMs take k_gemm_bf16
  if (epi == EPI_QKV) return launch_pp_tiles<BM, EPI_QKV, true>(st, gm, gn, nb, a, M, K, Wt, N, bias, o);
  if (!gelu && o.y) return launch_pp_tiles<BM, EPI_NONE, false>(st, gm, gn, nb, a, M, K, Wt, N, bias, o);
  if (gelu && o.yh) return launch_pp_tiles<BM, EPI_GELU, true>(st, gm, gn, nb, a, M, K, Wt, N, bias, o);
  if (gelu && o.y) return launch_pp_tiles<BM, EPI_GELU, false>(st, gm, gn, nb, a, M, K, Wt, N, bias, o);
  return hipErrorInvalidValue;  // an epilogue combination no caller uses
}

static hipError_t launch_any(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                             const float* bias, int epi, const GemmBf16Out& o) {
  // bf16 outputs leave as 16-byte pieces of 8 columns
  if (!a || !Wt || M <= 0 || N <= 0 || K <= 0 || K % (2 * TK) != 0 || ((o.yh || o.q) && N % 8 != 0))
    return hipErrorInvalidValue;
  // byte offsets inside a block's rows (operands and outputs) are 32-bit
  if ((size_t)256 * K * 2 > 0x7fffffffu || (size_t)256 * N * 4 > 0x7fffffffu) return hipErrorInvalidValue;
  // The ping-pong kernel without a residual once 256-row tiles give one per CU,
  // or 128-row tiles one per two CUs (C5: qkv and mlp.fc on 256-row tiles; the
  // residual GEMMs attn.proj and mlp.proj measured no faster on it, 32.2 / 90.1
  // against 30.9 / 90.8 us, and stay below); its stores need 16-byte aligned
  // fp32 rows and 8-byte aligned bf16 ones.
  {
    auto al = [](const void* p, unsigned n) { return ((uintptr_t)p & (n - 1)) == 0; };
    const bool pp_ok = !o.res && N % 4 == 0 && al(o.y, 16) && al(o.yh, 8) && al(o.q, 8) && al(o.kc, 8) && al(o.vc, 8);
    const int pn = (N + PBN - 1) / PBN;
    if (pp_ok && ((M + 255) / 256) * pn >= pp_blocks(1 << 30))
      return launch_pp<256>(st, a, M, K, Wt, N, bias, epi, o);
    if (pp_ok && ((M + 127) / 128) * pn >= pp_blocks(1 << 30) / 2)
      return launch_pp<128>(st, a, M, K, Wt, N, bias, epi, o);
  }
  const int gn = (N + TN - 1) / TN;
  // 256-row tiles while they give two tiles per CU (two blocks fit a CU); 128 below
  // that (attn.proj and mlp.proj at N 1024: 512 tiles of 128 rows instead of 256
  // of 256, measured 2 % faster on the whole C5 forward)
  const int gm256 = (M + 255) / 256, gm128 = (M + 127) / 128;
  if (gm256 * gn >= 512) return launch_bm<256>(st, gm256, gn, a, M, K, Wt, N, bias, epi, o);
  return launch_bm<128>(st, gm128, gn, a, M, K, Wt, N, bias, epi, o);
}

hipError_t launch_gemm_bf16_split(hipStream_t st, const bf16_t* a, int M, int K, const bf16_t* Wt, int N,
                                  const float* bias, const float* res, float* y, float* ws, size_t ws_floats,
                                  int* cnt, int cnt_cap) {
  if (!y || !res) return hipErrorInvalidValue;
  // the split when 256 x 256 tiles leave CUs idle and two halves per tile fill them,
  // each half a whole number of 64-deep K steps, both halves of a tile in one XCD's
  // run of items: the 2 gm gn items are dealt to the 8 XCDs in runs of gm gn / 4,
  // which must be even so that no run boundary falls between items 2t and 2t + 1
  // (8 divides gm gn); otherwise the unsplit kernels
  const int gm = (M + 255) / 256, gn = (N + PBN - 1) / PBN, cus = pp_blocks(1 << 30);
  auto al = [](const void* p, unsigned n) { return ((uintptr_t)p & (n - 1)) == 0; };
  const bool split = a && Wt && M > 0 && K > 0 && K % (4 * TK) == 0 && N % 4 == 0 && ws && cnt &&
                     (gm * gn) % 8 == 0 &&
                     ws_floats >= (size_t)M * N && gm * gn <= cnt_cap && gm * gn < cus && 2 * gm * gn >= cus &&
                     al(y, 16) && al(res, 16) && al(ws, 16) && (size_t)256 * K * 2 <= 0x7fffffffu &&
                     (size_t)256 * N * 4 <= 0x7fffffffu;
  if (!split) return launch_gemm_bf16(st, a, M, K, Wt, N, bias, EPI_NONE, res, y, nullptr);
  GemmBf16Out o{};
  o.res = res;
  o.y = y;
  o.ws = ws;
  o.cnt = cnt;
  o.err = cnt + cnt_cap;
  return launch_pp_tiles<256, EPI_NONE, false, true>(st, gm, gn, pp_blocks(2 * gm * gn), a, M, K, Wt, N, bias, o);
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
