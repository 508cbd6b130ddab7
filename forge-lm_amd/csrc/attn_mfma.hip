// attn_mfma.hip -- causal prefill attention on MFMA for head_dim 64 (gfx950).
//
// MultiHeadAttention.Forward over a window (src/LLM.Core/Layers/Layers.cs:191-229,
// ITensorBackend.cs:117-122): per head s = q.k * (1/sqrt(64)), keys past the
// query masked, softmax, o = p @ v.  A block takes 128 queries of one
// (sequence, head); each of its 4 waves owns 32 of them and walks the key tiles
// (64 keys) up to its last query with an online softmax:
//   S^T = K Q^T    MFMA with keys as rows: lane l holds query l % 32 and, in
//                  element r, key (r/4)*8 + (l/32)*4 + r%4 of a 32-key half, so
//                  the softmax statistics of a query stay inside its lane pair
//   O^T += V^T P^T the score registers are the B operand as they are; V^T is
//                  staged in LDS and read in the same key order.
// bf16 sessions: v_mfma_f32_32x32x16_bf16 (q rounded to bf16, fp32 softmax and
// accumulation); fp32 sessions: v_mfma_f32_32x32x2_f32 on exact fp32 values.
#include "kernels.hpp"

#include <math.h>

#include <type_traits>

namespace fh {

namespace {

constexpr int HD = 64;   // head dim
constexpr int BQ = 128;  // queries per block (4 waves x 32)
constexpr int BKV = 64;  // keys per tile

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int acc_row(int lane, int r) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

__device__ __forceinline__ __bf16 to_bf(float f) { return __builtin_bit_cast(__bf16, bf16_rn(f)); }

// Block -> (query block, head, sequence) of a causal prefill launched as one
// grid dimension of nqb * H * B blocks; query block 0 holds the last BQ
// queries (the most keys).  Workgroups reach the 8 XCDs round-robin by linear
// index, so a grid ordered by query block gives one XCD every heaviest block.
// When 8 divides H * B, XCD x takes whole (sequence, head) groups (their K/V
// rows are fetched into its L2 only) and receives its blocks heaviest first:
// query block 0 of each of its groups, then query block 1, and so on, so the
// CUs that finish early pick up the light blocks at the end (longest job first).
// Otherwise block L takes query block L mod nqb of group L / nqb.
struct QBlock {
  int qb, h, b;
};
__device__ __forceinline__ QBlock prefill_block(int L, int nqb, int H) {
  const int G = gridDim.x / nqb;  // H * B
  if (G % 8 == 0) {
    const int xcd = L & 7, s = L >> 3, gx = G / 8, g = xcd * gx + s % gx;
    return {s / gx, g % H, g / H};
  }
  return {L % nqb, (L / nqb) % H, L / (nqb * H)};
}

template <typename KT, typename OT, typename QT>
__global__ __launch_bounds__(256) void k_attn_prefill_mfma(const QT* __restrict__ qp, int qstride, int T, int d, int H,
                                                          int ctx, const KT* __restrict__ kc,
                                                          const KT* __restrict__ vc, OT* __restrict__ o) {
  constexpr bool BF = sizeof(KT) == 2;
  // K tile [key][dim] and V^T tile [dim][key]; fp32 K rows hold the even dims
  // first, then the odd ones (float4 reads per half-wave)
  constexpr int PAD = BF ? 8 : 4;
  typedef typename std::conditional<BF, __bf16, float>::type E;
  __shared__ __align__(16) E Ks[BKV][HD + PAD];
  __shared__ __align__(16) E Vt[HD][BKV + PAD];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (T + BQ - 1) / BQ;
  const QBlock qbk = prefill_block(blockIdx.x, nqb, H);
  const int t0 = (nqb - 1 - qbk.qb) * BQ, h = qbk.h, b = qbk.b;
  const int qw0 = t0 + 32 * w;             // this wave's first query
  const int q = qw0 + (lane & 31), half = lane >> 5;
  const float scale = 0.125f;              // 1 / sqrt(64), exact
  const KT* K = kc + ((size_t)b * H + h) * ctx * HD;
  const KT* V = vc + ((size_t)b * H + h) * ctx * HD;
  // the first T cache rows of this (sequence, head): rows at or past T read as
  // zeros, with no branch around the loads
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(K), (short)0, T * HD * (int)sizeof(KT), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(V), (short)0, T * HD * (int)sizeof(KT), 0x00020000);

  // this lane's q (row q, clamped for the loads)
  const QT* qrow = qp + (size_t)(b * T + min(q, T - 1)) * qstride + h * HD;
  bf16x8_t qb[4];                          // bf16: dims 16kk + 8*half .. +7
  float qf[32];                            // fp32: dims 2s + half
  if constexpr (sizeof(QT) == 2) {
    static_assert(BF, "bf16 q goes with a bf16 cache");
#pragma unroll
    for (int kk = 0; kk < 4; kk++) qb[kk] = *reinterpret_cast<const bf16x8_t*>(qrow + 16 * kk + 8 * half);
  } else if constexpr (BF) {
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 16 * kk + 8 * half);
      const float4 c = *reinterpret_cast<const float4*>(qrow + 16 * kk + 8 * half + 4);
      qb[kk] = bf16x8_t{to_bf(a.x), to_bf(a.y), to_bf(a.z), to_bf(a.w), to_bf(c.x), to_bf(c.y), to_bf(c.z), to_bf(c.w)};
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 4 * i);
      qf[2 * i] = half ? a.y : a.x;
      qf[2 * i + 1] = half ? a.w : a.z;
    }
  }

  f32x16_t ot[2];  // O^T: dims (dt*32 + acc_row) x this lane's query
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) ot[dt][r] = 0.f;
  float m = -INFINITY, l = 0.f;

  const int qlast = min(t0 + BQ, T) - 1;    // last query of the block
  const int nkt = qlast / BKV + 1;
  for (int kt = 0; kt < nkt; kt++) {
    const int k0 = kt * BKV;
    __syncthreads();  // the previous tile is consumed
    // stage K and V^T (rows at or past T read as zeros)
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int idx = tid + 256 * i, key = idx / 8, q8 = idx % 8;  // 8 x 8 bf16 per key row
        const u32x4_t kw = __builtin_amdgcn_raw_buffer_load_b128(rk, ((k0 + key) * HD + 8 * q8) * 2, 0, 0);
        const u32x4_t vw = __builtin_amdgcn_raw_buffer_load_b128(rv, ((k0 + key) * HD + 8 * q8) * 2, 0, 0);
        const uint4 kv = make_uint4(kw.x, kw.y, kw.z, kw.w), vv = make_uint4(vw.x, vw.y, vw.z, vw.w);
        *reinterpret_cast<uint4*>(&Ks[key][8 * q8]) = kv;
        const bf16_t* vh = reinterpret_cast<const bf16_t*>(&vv);
#pragma unroll
        for (int e = 0; e < 8; e++) Vt[8 * q8 + e][key] = __builtin_bit_cast(__bf16, vh[e]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int idx = tid + 256 * i, key = idx / 16, q4 = idx % 16;  // 16 x 4 floats per key row
        const u32x4_t kw = __builtin_amdgcn_raw_buffer_load_b128(rk, ((k0 + key) * HD + 4 * q4) * 4, 0, 0);
        const u32x4_t vw = __builtin_amdgcn_raw_buffer_load_b128(rv, ((k0 + key) * HD + 4 * q4) * 4, 0, 0);
        const float4 kv = make_float4(__uint_as_float(kw.x), __uint_as_float(kw.y), __uint_as_float(kw.z),
                                      __uint_as_float(kw.w));
        const float4 vv = make_float4(__uint_as_float(vw.x), __uint_as_float(vw.y), __uint_as_float(vw.z),
                                      __uint_as_float(vw.w));
        // dims 4q4 .. +3: even ones to 2q4, 2q4+1; odd ones to 32 + 2q4, +1
        Ks[key][2 * q4] = kv.x;
        Ks[key][2 * q4 + 1] = kv.z;
        Ks[key][32 + 2 * q4] = kv.y;
        Ks[key][32 + 2 * q4 + 1] = kv.w;
        Vt[4 * q4 + 0][key] = vv.x;
        Vt[4 * q4 + 1][key] = vv.y;
        Vt[4 * q4 + 2][key] = vv.z;
        Vt[4 * q4 + 3][key] = vv.w;
      }
    }
    __syncthreads();
    if (k0 > qw0 + 31 || qw0 >= T) continue;  // no query of this wave sees a key of the tile

    // ---- S^T = K Q^T for the two 32-key halves ----
    f32x16_t s[2];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
#pragma unroll
      for (int r = 0; r < 16; r++) s[jt][r] = 0.f;
      const int kr = jt * 32 + (lane & 31);  // key row this lane supplies
      if constexpr (BF) {
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&Ks[kr][16 * kk + 8 * half]);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qb[kk], s[jt], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 8; c++) {
          const float4 a = *reinterpret_cast<const float4*>(&Ks[kr][32 * half + 4 * c]);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qf[4 * c + 0], s[jt], 0, 0, 0);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qf[4 * c + 1], s[jt], 0, 0, 0);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qf[4 * c + 2], s[jt], 0, 0, 0);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qf[4 * c + 3], s[jt], 0, 0, 0);
        }
      }
    }
    // ---- scale, causal mask, online softmax (per query = per lane pair) ----
    float mt = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int key = k0 + jt * 32 + acc_row(lane, r);
        const float v = (key <= q && key < T) ? s[jt][r] * scale : -INFINITY;
        s[jt][r] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt);
    const float corr = (m == -INFINITY) ? 0.f : expf(m - mn);
    float ls = 0.f;
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float p = (s[jt][r] == -INFINITY) ? 0.f : expf(s[jt][r] - mn);
        s[jt][r] = p;
        ls += p;
      }
    ls += __shfl_xor(ls, 32, 64);
    l = l * corr + ls;
    m = mn;
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
      for (int r = 0; r < 16; r++) ot[dt][r] *= corr;

    // ---- O^T += V^T P^T: a k step takes, per half-wave, the keys the score
    // registers hold (keys 4*half + {0..3} and 8 + 4*half + {0..3} of 16) ----
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
      const int vr = dt * 32 + (lane & 31);  // V^T row (dim) this lane supplies
      if constexpr (BF) {
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
          for (int kk = 0; kk < 2; kk++) {
            const int kb = jt * 32 + kk * 16 + 4 * half;
            const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(&Vt[vr][kb]);
            const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(&Vt[vr][kb + 8]);
            const bf16x8_t a = bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            const int r0 = 8 * kk;
            const bf16x8_t pb = bf16x8_t{to_bf(s[jt][r0 + 0]), to_bf(s[jt][r0 + 1]), to_bf(s[jt][r0 + 2]),
                                         to_bf(s[jt][r0 + 3]), to_bf(s[jt][r0 + 4]), to_bf(s[jt][r0 + 5]),
                                         to_bf(s[jt][r0 + 6]), to_bf(s[jt][r0 + 7])};
            ot[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, ot[dt], 0, 0, 0);
          }
      } else {
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int key = jt * 32 + acc_row(lane, r);  // the key of score register r in this lane
            ot[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vt[vr][key], s[jt][r], ot[dt], 0, 0, 0);
          }
      }
    }
  }

  if (q >= T) return;
  const float inv = 1.f / l;
  OT* orow = o + (size_t)(b * T + q) * d + h * HD;
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      // elements 4g .. 4g+3 are dims dt*32 + 8g + 4*half + 0..3
      const float4 v = make_float4(ot[dt][4 * g] * inv, ot[dt][4 * g + 1] * inv, ot[dt][4 * g + 2] * inv,
                                   ot[dt][4 * g + 3] * inv);
      if constexpr (sizeof(OT) == 2) {
        const uint32_t lo = (uint32_t)bf16_rn(v.x) | ((uint32_t)bf16_rn(v.y) << 16);
        const uint32_t hi = (uint32_t)bf16_rn(v.z) | ((uint32_t)bf16_rn(v.w) << 16);
        *reinterpret_cast<uint2*>(orow + dt * 32 + 8 * g + 4 * half) = make_uint2(lo, hi);
      } else {
        *reinterpret_cast<float4*>(orow + dt * 32 + 8 * g + 4 * half) = v;
      }
    }
}

// ---------------------------------------------------------------------------
// bf16 sessions with q already in bf16: the same S^T / O^T scheme, software-
// pipelined.  The K and V^T tiles of key tile j + 1 are fetched into registers
// while tile j is multiplied and land in the other half of a double-buffered
// LDS pair (one barrier per tile).  V^T is built in registers: a thread takes
// one dim pair of 8 key rows (4-byte loads, a wave covers whole 128-byte rows)
// and packs them with v_perm into two 16-byte rows of V^T.  Within each group
// of 16 keys V^T holds the keys in the order the score registers hold them
// (0-3, 8-11, 4-7, 12-15), so an A fragment is one 16-byte LDS read.  The
// softmax runs in base 2 on the hardware exp (the scale log2(e) / 8 folded into
// one FMA per score), the causal mask only on tiles that cross the wave's diagonal,
// and P is rounded to bf16 by the hardware packed convert.  Rows at or past T
// read as zeros (bounded buffer loads), so stale cache rows never meet a zero
// weight.  Blocks take query blocks in prefill_block's order (heaviest first per XCD).
// ---------------------------------------------------------------------------
constexpr int KP = HD + 8;  // bf16 per LDS row of K (dims) and V^T (keys): 144 B, 16 rows hit distinct banks

__global__ __launch_bounds__(256, 2) void k_attn_prefill_bf16(const bf16_t* __restrict__ qp, int T, int d, int H,
                                                              int ctx, const bf16_t* __restrict__ kc,
                                                              const bf16_t* __restrict__ vc, bf16_t* __restrict__ o) {
  __shared__ __align__(16) __bf16 Ks[2][BKV][KP];
  __shared__ __align__(16) __bf16 Vt[2][HD][KP];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (T + BQ - 1) / BQ;
  const QBlock qbk = prefill_block(blockIdx.x, nqb, H);
  const int t0 = (nqb - 1 - qbk.qb) * BQ, h = qbk.h, b = qbk.b;
  const int qw0 = t0 + 32 * w;
  const int q = qw0 + (lane & 31), half = lane >> 5;
  const float sl2 = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) * log2(e)
  const size_t head = ((size_t)b * H + h) * ctx * HD;
  // this (sequence, head)'s first T cache rows; rows past T read as zeros
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(kc + head), (short)0, T * HD * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(vc + head), (short)0, T * HD * 2, 0x00020000);

  const bf16_t* qrow = qp + (size_t)(b * T + min(q, T - 1)) * d + h * HD;
  bf16x8_t qb[4];  // dims 16kk + 8*half .. +7
#pragma unroll
  for (int kk = 0; kk < 4; kk++) qb[kk] = *reinterpret_cast<const bf16x8_t*>(qrow + 16 * kk + 8 * half);

  // staging roles: K piece (key kp_key, 16 bytes at dim 8*kp_c) for i = 0, 1;
  // V: dim pair vc2 of keys vkey(u), u = 0..7, to V^T positions vpos .. +7
  const int kp_key = tid >> 3, kp_c = tid & 7;
  const int vc2 = tid & 31, vkq = tid >> 5, vg = vkq >> 1, vsel = vkq & 1;
  auto vkey = [&](int u) { return vg * 16 + vsel * 4 + (u >> 2) * 8 + (u & 3); };
  const int vpos = vg * 16 + vsel * 8;
  uint4 kr[2];
  unsigned vr[8];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rk, ((k0 + kp_key + 32 * i) * HD + 8 * kp_c) * 2, 0, 0);
      kr[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) vr[u] = __builtin_amdgcn_raw_buffer_load_b32(rv, ((k0 + vkey(u)) * HD + 2 * vc2) * 2, 0, 0);
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) *reinterpret_cast<uint4*>(&Ks[buf][kp_key + 32 * i][8 * kp_c]) = kr[i];
    // V^T rows 2*vc2 (low halves) and 2*vc2 + 1 (high halves) of the 8 keys
    const uint4 lo = make_uint4(__builtin_amdgcn_perm(vr[1], vr[0], 0x05040100u),
                                __builtin_amdgcn_perm(vr[3], vr[2], 0x05040100u),
                                __builtin_amdgcn_perm(vr[5], vr[4], 0x05040100u),
                                __builtin_amdgcn_perm(vr[7], vr[6], 0x05040100u));
    const uint4 hi = make_uint4(__builtin_amdgcn_perm(vr[1], vr[0], 0x07060302u),
                                __builtin_amdgcn_perm(vr[3], vr[2], 0x07060302u),
                                __builtin_amdgcn_perm(vr[5], vr[4], 0x07060302u),
                                __builtin_amdgcn_perm(vr[7], vr[6], 0x07060302u));
    *reinterpret_cast<uint4*>(&Vt[buf][2 * vc2][vpos]) = lo;
    *reinterpret_cast<uint4*>(&Vt[buf][2 * vc2 + 1][vpos]) = hi;
  };

  f32x16_t ot[2];  // O^T: dims (dt*32 + acc_row) x this lane's query
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) ot[dt][r] = 0.f;
  float m = -INFINITY, l = 0.f;  // running max (base-2 scaled) and sum

  const int qlast = min(t0 + BQ, T) - 1;
  const int nkt = qlast / BKV + 1;
  fetch(0);
  put(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; kt++) {
    const int k0 = kt * BKV, buf = kt & 1;
    if (kt + 1 < nkt) fetch(k0 + BKV);
    if (k0 <= qw0 + 31 && qw0 < T) {  // some query of this wave sees a key of the tile
      f32x16_t s[2];
#pragma unroll
      for (int jt = 0; jt < 2; jt++) {
#pragma unroll
        for (int r = 0; r < 16; r++) s[jt][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(&Ks[buf][jt * 32 + (lane & 31)][16 * kk + 8 * half]);
          s[jt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qb[kk], s[jt], 0, 0, 0);
        }
      }
      // the maximum is taken on the raw products (the scale is positive) and the
      // scale folded into the exponent: p = 2^(s * log2(e) / 8 - m)
      float mt = -INFINITY;
      if (k0 + BKV - 1 > qw0) {  // the tile crosses this wave's diagonal: mask keys past the query
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int key = k0 + jt * 32 + acc_row(lane, r);
            const float v = key <= q ? s[jt][r] : -INFINITY;
            s[jt][r] = v;
            mt = fmaxf(mt, v);
          }
      } else {
#pragma unroll
        for (int jt = 0; jt < 2; jt++)
#pragma unroll
          for (int r = 0; r < 16; r++) mt = fmaxf(mt, s[jt][r]);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      // a lane whose query precedes every key of the tile keeps mn = m; its
      // first tile (key 0) always has a visible key, so mn is finite here
      const float mn = fmaxf(m, mt * sl2);
      const float corr = __builtin_amdgcn_exp2f(m - mn);
      float ls = 0.f;
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[jt][r], sl2, -mn));
          s[jt][r] = p;
          ls += p;
        }
      ls += __shfl_xor(ls, 32, 64);
      l = l * corr + ls;
      m = mn;
#pragma unroll
      for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) ot[dt][r] *= corr;
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
          const int r0 = 8 * kk;
          const bf16x8_t pb = bf16x8_t{(__bf16)s[jt][r0 + 0], (__bf16)s[jt][r0 + 1], (__bf16)s[jt][r0 + 2],
                                       (__bf16)s[jt][r0 + 3], (__bf16)s[jt][r0 + 4], (__bf16)s[jt][r0 + 5],
                                       (__bf16)s[jt][r0 + 6], (__bf16)s[jt][r0 + 7]};
#pragma unroll
          for (int dt = 0; dt < 2; dt++) {
            const bf16x8_t a =
                *reinterpret_cast<const bf16x8_t*>(&Vt[buf][dt * 32 + (lane & 31)][jt * 32 + kk * 16 + 8 * half]);
            ot[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, ot[dt], 0, 0, 0);
          }
        }
    }
    if (kt + 1 < nkt) put(buf ^ 1);
    __syncthreads();
  }

  if (q >= T) return;
  const float inv = 1.f / l;
  bf16_t* orow = o + (size_t)(b * T + q) * d + h * HD;
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      // elements 4g .. 4g+3 are dims dt*32 + 8g + 4*half + 0..3
      typedef __bf16 bf16x4_t_ __attribute__((ext_vector_type(4)));
      const bf16x4_t_ v = bf16x4_t_{(__bf16)(ot[dt][4 * g] * inv), (__bf16)(ot[dt][4 * g + 1] * inv),
                                    (__bf16)(ot[dt][4 * g + 2] * inv), (__bf16)(ot[dt][4 * g + 3] * inv)};
      *reinterpret_cast<bf16x4_t_*>(orow + dt * 32 + 8 * g + 4 * half) = v;
    }
}

}  // namespace

template <typename KT, typename OT>
hipError_t launch_attn_prefill_mfma(hipStream_t st, const float* qkv, int B, int T, int d, int H, int ctx,
                                    const KT* kcache, const KT* vcache, OT* o) {
  if (B <= 0 || T <= 0 || T > ctx || H <= 0 || d != H * HD || !qkv || !kcache || !vcache || !o ||
      (size_t)T * HD * sizeof(KT) > 0x7fffffffu)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_attn_prefill_mfma<KT, OT, float>), dim3((T + BQ - 1) / BQ * H * B), dim3(256), 0, st, qkv,
                     3 * d, T, d, H, ctx, kcache, vcache, o);
  return hipGetLastError();
}

hipError_t launch_attn_prefill_mfma_q16(hipStream_t st, const bf16_t* q, int B, int T, int d, int H, int ctx,
                                        const bf16_t* kcache, const bf16_t* vcache, bf16_t* o) {
  if (B <= 0 || T <= 0 || T > ctx || H <= 0 || d != H * HD || !q || !kcache || !vcache || !o)
    return hipErrorInvalidValue;
  if ((size_t)T * HD * 2 > 0x7fffffffu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_prefill_bf16, dim3((T + BQ - 1) / BQ * H * B), dim3(256), 0, st, q, T, d, H, ctx, kcache,
                     vcache, o);
  return hipGetLastError();
}

template hipError_t launch_attn_prefill_mfma<float, float>(hipStream_t, const float*, int, int, int, int, int,
                                                           const float*, const float*, float*);
template hipError_t launch_attn_prefill_mfma<bf16_t, float>(hipStream_t, const float*, int, int, int, int, int,
                                                            const bf16_t*, const bf16_t*, float*);
template hipError_t launch_attn_prefill_mfma<bf16_t, bf16_t>(hipStream_t, const float*, int, int, int, int, int,
                                                             const bf16_t*, const bf16_t*, bf16_t*);

}  // namespace fh
