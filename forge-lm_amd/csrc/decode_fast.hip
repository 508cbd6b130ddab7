// decode_fast.hip -- persistent batch-1 fp32 decode step for MI355X (gfx950).
//
// One launch runs a whole decode step of the token loop (GptModel.ForwardLast
// on the cached window, src/LLM.Core/Model/GptModel.cs:202-222, then
// Sampler.Greedy, src/LLM.Core/Inference/Sampler.cs:14-20): 256 blocks (one
// per CU, round-robin over the 8 XCDs) x 256 threads (waves 0..2 hold weight
// tiles, wave 3 is the control wave).  Per layer five phases:
//   A  LN1 + QKV columns (9 of 2304 per block); new K/V row into the cache
//   B  decode attention: (head, key chunk) blocks, online softmax; the last of
//      a head's chunk blocks to arrive combines the chunks into the head's o
//   C  attn.proj columns + residual -> x2
//   D  LN2 + mlp.fc columns + GELU -> h
//   E  mlp.proj columns + residual -> x
// then LN_f + the tied head (64 vocab rows per block) and, in greedy mode, the
// argmax.  At batch 1 every weight is used once per token, so the step is
// bound by HBM bytes plus the chain of cross-CU hand-offs.
//
// Dataflow instead of grid barriers: every value handed from one phase to the
// next is stored as a 64-bit (value, tag) pair in uncached device memory, the
// tag being this launch's sequence number for the producing phase.  A
// consumer's control wave re-reads the pairs it needs until every tag matches,
// then copies the values to LDS; one memory round trip after the last
// producer's store, instead of a barrier plus a separate read.  Because every
// phase reads the outputs of all blocks of the phase before it, no block can
// run a full phase ahead of another, so no buffer is overwritten while a
// reader still needs it.  Attention partials and argmax records are written
// data first, tag (or arrival count) last.
//
// The data waves hold weight tiles in registers: each block's tiles were
// re-laid out once into contiguous column-major blocks, and the next phase's
// tile is requested as soon as the current one is consumed, so HBM streams
// while the control wave waits for the hand-off.  Cached K/V rows are requested
// before q arrives.  Every wait is bounded: past the spin limit the error word
// is set and all blocks leave.
#include <math.h>
#include <stdlib.h>

#include <mutex>
#include <tuple>
#include <vector>

#include "decode_fast.hpp"

namespace fh {

namespace {

constexpr int NB = 256;   // blocks
constexpr int NT = 256;   // threads per block: one wave per SIMD, so 512 registers per wave
constexpr int NW = NT / 64;
constexpr int NDW = NW - 1;  // data waves (the last wave is the control wave)
constexpr int AC = 16;    // attention key chunks per head
constexpr int KG = 8;     // keys per data wave per group (online softmax across groups)
constexpr int TAGS = 128;  // tag values reserved per launch
constexpr long SPIN_LIMIT = 300000;

__device__ __forceinline__ bool err_set(int* err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void raise_err(int* err) {
  __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until this thread's stores are acknowledged by memory
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0); }
// keeps the compiler from reusing values loaded before this point
__device__ __forceinline__ void reload_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void put_pair(uint2* dst, float v, unsigned tag) {
  *dst = make_uint2(__float_as_uint(v), tag);
}

// Reads of the hand-off area go through a raw buffer resource with the
// system-coherent cache policy (SC0|SC1): they miss in the CU's L1 and in L2,
// so a re-read sees other CUs' stores (uncached memory is still cached in L1
// by plain loads).  Out-of-range offsets read as 0.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
struct NcBuf {
  __amdgpu_buffer_rsrc_t r;
  __device__ NcBuf(const void* base, int bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000)) {}
  __device__ __forceinline__ uint4 load4(int byte_off) const {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 17);
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ unsigned load1(int byte_off) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 17);
  }
};

template <int D>
struct Shape {
  static constexpr int KC = D / 256;        // 256-float chunks per K=D column
  static constexpr int KC4 = 4 * D / 256;   // chunks per K=4D column
  static constexpr int QCOL = 3 * D / NB;   // qkv columns per block
  static constexpr int PCOL = D / NB;       // attn.proj / mlp.proj columns per block
  static constexpr int FCOL = 4 * D / NB;   // mlp.fc columns per block
  static constexpr int QCH = QCOL * KC;
  static constexpr int PCH = PCOL * KC;
  static constexpr int FCH = FCOL * KC;
  static constexpr int MCH = PCOL * KC4;
  static constexpr int QMAX = (QCH + NDW - 1) / NDW;
  static constexpr int PMAX = (PCH + NDW - 1) / NDW;
  static constexpr int FMAX = (FCH + NDW - 1) / NDW;
  static constexpr int MMAX = (MCH + NDW - 1) / NDW;
  static constexpr int RMAX = 64;  // vocab rows per block (V <= 16384)
  static constexpr int HMAX = (RMAX * KC + NDW - 1) / NDW;
  static constexpr int PER = (D + NT - 1) / NT;  // LayerNorm elements per thread
  // tile floats per block, in phase order
  static constexpr size_t QT = (size_t)QCOL * D, PT = (size_t)PCOL * D, FT = (size_t)FCOL * D,
                          MT = (size_t)PCOL * 4 * D;
  static constexpr size_t LAYER = (size_t)NB * (QT + PT + FT + MT);
  // compact vector buffer: per layer ln1.w ln1.b qkv.b proj.b ln2.w ln2.b fc.b mproj.b
  static constexpr int V_LN1W = 0, V_LN1B = D, V_QKVB = 2 * D, V_PROJB = 5 * D, V_LN2W = 6 * D, V_LN2B = 7 * D,
                       V_FCB = 8 * D, V_MPB = 12 * D, VL = 13 * D;
};

// exchange layout (uncached): pairs (uint2) and the attention partials
template <int D>
struct Xch {
  static constexpr int X = 0, X2 = D, HH = 2 * D, QKV = 6 * D, O = 9 * D, NPAIR = 10 * D;  // pair offsets
  static constexpr int AP_STRIDE = 68;  // floats per attention partial: o[64], m, l, pad[2]
};

struct KParams {
  RowSrc src;
  const float* tiles;
  const float* vecs;
  const float* tok;
  const float* pos;
  float* kc;
  float* vc;
  float* logits;
  int* out_ids;
  int* out_counts;
  uint2* pairs;      // uncached: x, x2, h, qkv pairs
  float* apart;      // uncached: attention partials [H*AC][68]
  unsigned* hcnt;    // per-head arrival counters of the attention chunk blocks (agent atomics)
  uint4* amax;       // uncached: per-block (value, index, tag, -)
  int uc_bytes;      // size of the uncached area starting at `pairs`
  int off_apart, off_amax;  // byte offsets of the areas above from `pairs`
  unsigned* launch;  // launch counter (agent atomics)
  int* err;
  int V, ctx, H, L, max_new, eos, greedy;
  int* tokens_out;  // same buffer as src.tokens, written by the greedy argmax
  int* step_out;    // same word as src.step
  unsigned long long* trace;  // optional: block 0 timestamps
};

__device__ __forceinline__ void trace_mark(unsigned long long* t, int i) {
  if (t && blockIdx.x == 0 && threadIdx.x == (NT - 64) && i < 256) t[i] = wall_clock64();
}

// Control wave: waits until pairs[0..n) all carry `tag`, then stores the values
// to out[0..n) (LDS).  n must be a multiple of 128 (two pairs per 16-byte load).
// Returns false on spin-limit or a raised error.
template <int N>
__device__ bool wait_pairs(const NcBuf& nc, int pair0, unsigned tag, float* out, int* err) {
  static_assert(N % 128 == 0, "pairs come in 16-byte loads");
  constexpr int R = N / 128;  // 16-byte loads per lane
  const int lane = threadIdx.x & 63;
  uint4 v[R];
  long it = 0;
  for (;;) {
    reload_fence();
#pragma unroll
    for (int r = 0; r < R; r++) v[r] = nc.load4(pair0 * 8 + (r * 64 + lane) * 16);
    bool ok = true;
#pragma unroll
    for (int r = 0; r < R; r++) ok &= (v[r].y == tag) & (v[r].w == tag);
    if (__all(ok)) break;
    if (++it > SPIN_LIMIT || err_set(err)) {
      if (lane == 0) raise_err(err);
      return false;
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int i = 2 * (r * 64 + lane);
    out[i] = __uint_as_float(v[r].x);
    out[i + 1] = __uint_as_float(v[r].z);
  }
  return true;
}

__device__ __forceinline__ float block_sum512(float v, float* red) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NW; i++) s += red[i];
  __syncthreads();
  return s;
}

// LayerNorm of xin[D] (LDS) into xout[D] (LDS) with this thread's parameters
// w[j], b[j] for elements tid + j*NT (biased variance, eps 1e-5).
template <int D>
__device__ void layernorm_regs(const float* xin, float* xout, const float (&w)[Shape<D>::PER],
                               const float (&b)[Shape<D>::PER], float* red) {
  constexpr int PER = Shape<D>::PER;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = threadIdx.x + j * NT;
    if (i < D) s += xin[i];
  }
  const float mu = block_sum512(s, red) / (float)D;
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = threadIdx.x + j * NT;
    if (i < D) {
      const float d = xin[i] - mu;
      v += d * d;
    }
  }
  const float var = block_sum512(v, red);
  const float rs = 1.f / sqrtf(var / (float)D + 1e-5f);
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = threadIdx.x + j * NT;
    if (i < D) xout[i] = (xin[i] - mu) * rs * w[j] + b[j];
  }
  __syncthreads();
}

template <int D>
__device__ __forceinline__ void load_ln(const float* wv, const float* bv, float (&w)[Shape<D>::PER],
                                        float (&b)[Shape<D>::PER]) {
#pragma unroll
  for (int j = 0; j < Shape<D>::PER; j++) {
    const int i = min((int)threadIdx.x + j * NT, D - 1);
    w[j] = wv[i];
    b[j] = bv[i];
  }
}

// Loads this wave's chunks of a tile (chunk = 64 lanes x float4) into registers.
template <int MAX, int NCH>
__device__ __forceinline__ void tile_load(float4 (&r)[MAX], const float* tile) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (w >= NDW) return;
  const float4* t4 = reinterpret_cast<const float4*>(tile);
#pragma unroll
  for (int i = 0; i < MAX; i++) {
    const int ch = min(w + NDW * i, NCH - 1);
    r[i] = t4[ch * 64 + lane];
  }
}

// Chunk dot products against xs (LDS): part[ch] = sum over the chunk's 256 k.
template <int MAX, int NCH, int KCH>
__device__ __forceinline__ void tile_dot(const float4 (&r)[MAX], const float* xs, float* part) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (w >= NDW) return;
#pragma unroll
  for (int i = 0; i < MAX; i++) {
    const int ch = w + NDW * i;
    if (ch < NCH) {
      const int kc = ch % KCH;
      const float4 xv = *reinterpret_cast<const float4*>(xs + kc * 256 + lane * 4);
      const float p = wave_sum_dpp(r[i].x * xv.x + r[i].y * xv.y + r[i].z * xv.z + r[i].w * xv.w);
      if (lane == 0) part[ch] = p;
    }
  }
}

template <int D>
__global__ __launch_bounds__(NT, 1) void k_decode_step(KParams p) {
  using S = Shape<D>;
  using X = Xch<D>;
  __shared__ float xres[D], xs[D], x2s[D], os[D], hs[4 * D];
  __shared__ float part[256];
  __shared__ float red[16];
  __shared__ float qkvs[192];  // this head's q, new k, new v
  __shared__ float wm[NW], wl[NW], wo[NW][64];
  __shared__ float aph[AC * 68];  // the head's attention partials (last arriver only)
  __shared__ int last_s;
  __shared__ float bias_s[2][32];  // this block's qkv, proj, fc, mproj bias slices, by layer parity
  __shared__ int fail_s;

  const int blk = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const bool ctrl = w == NW - 1;
  if (tid == 0) fail_s = 0;
  const unsigned tagbase = __hip_atomic_load(p.launch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * TAGS;
  trace_mark(p.trace, 0);

  const int n = *p.src.step;
  const int pos = p.src.pos_off + p.src.pos_mul * n;  // position of the new token
  int tokid = p.src.tokens[p.src.tok_off + n];
  if ((unsigned)tokid >= (unsigned)p.V) tokid = 0;
  const int H = p.H, ctx = p.ctx;
  const NcBuf nc(p.pairs, p.uc_bytes);
  const bool attn_blk = blk < H * AC;
  const int ah = blk / AC, achunk = blk % AC;
  const int nk = pos + 1, per = (nk + AC - 1) / AC;
  const int j0 = min(nk, achunk * per), j1 = min(nk, j0 + per);
  const int kpw = (j1 - j0 + NDW - 1) / NDW;
  const int a0 = min(j1, j0 + w * kpw), a1 = min(j1, a0 + kpw);  // this data wave's keys

  float4 rq[S::QMAX], rp[S::PMAX], rf[S::FMAX], rm[S::MMAX];
  float l1w[S::PER], l1b[S::PER], l2w[S::PER], l2b[S::PER];
  float kreg[KG], vreg[KG];
  tile_load<S::QMAX, S::QCH>(rq, p.tiles + (size_t)blk * S::QT);
  load_ln<D>(p.vecs + S::V_LN1W, p.vecs + S::V_LN1B, l1w, l1b);

  // x = tok_emb[id] + pos_emb[pos] (every block keeps its own copy)
  for (int i = tid; i < D; i += NT) xres[i] = p.tok[(size_t)tokid * D + i] + p.pos[(size_t)pos * D + i];
  __syncthreads();

  bool ok = true;
  auto fail = [&]() { fail_s = 1; };
#define SYNC_OK()       \
  __syncthreads();      \
  if (fail_s) {         \
    ok = false;         \
    break;              \
  }
#define TM(i) \
  if (l == 1) trace_mark(p.trace, 128 + (i))
  for (int l = 0; l < p.L; l++) {
    const unsigned tA = tagbase + 5 * l, tB = tA + 1, tC = tA + 2, tD = tA + 3, tE = tA + 4;
    const float* vl = p.vecs + (size_t)l * S::VL;
    const float* tl = p.tiles + (size_t)l * S::LAYER;
    const float* t_proj = tl + (size_t)NB * S::QT + (size_t)blk * S::PT;
    const float* t_fc = tl + (size_t)NB * (S::QT + S::PT) + (size_t)blk * S::FT;
    const float* t_mp = tl + (size_t)NB * (S::QT + S::PT + S::FT) + (size_t)blk * S::MT;
    const int ln = min(l + 1, p.L - 1);
    const float* t_qkv_next = p.tiles + (size_t)ln * S::LAYER + (size_t)blk * S::QT;
    const float* vnext = p.vecs + (size_t)ln * S::VL;
    const float* Kc = p.kc + ((size_t)l * H + ah) * ctx * 64;
    const float* Vc = p.vc + ((size_t)l * H + ah) * ctx * 64;

    // ---- A: LN1 + QKV ----
    if (ctrl) {
      constexpr int NBIAS = S::QCOL + 2 * S::PCOL + S::FCOL;
      if (lane < NBIAS) {
        int off;
        if (lane < S::QCOL) off = S::V_QKVB + blk * S::QCOL + lane;
        else if (lane < S::QCOL + S::PCOL) off = S::V_PROJB + blk * S::PCOL + (lane - S::QCOL);
        else if (lane < S::QCOL + S::PCOL + S::FCOL) off = S::V_FCB + blk * S::FCOL + (lane - S::QCOL - S::PCOL);
        else off = S::V_MPB + blk * S::PCOL + (lane - S::QCOL - S::PCOL - S::FCOL);
        bias_s[l & 1][lane] = vl[off];
      }
    }
    load_ln<D>(vl + S::V_LN2W, vl + S::V_LN2B, l2w, l2b);
    if (l > 0 && ctrl && !wait_pairs<D>(nc, X::X, tagbase + 5 * (l - 1) + 4, xres, p.err)) fail();
    SYNC_OK();
    TM(0);
    layernorm_regs<D>(xres, xs, l1w, l1b, red);
    tile_dot<S::QMAX, S::QCH, S::KC>(rq, xs, part);
    tile_load<S::PMAX, S::PCH>(rp, t_proj);
    __syncthreads();
    TM(1);
    if (tid < S::QCOL) {
      const int col = blk * S::QCOL + tid;
      float s = 0.f;
#pragma unroll
      for (int kc = 0; kc < S::KC; kc++) s += part[tid * S::KC + kc];
      s += bias_s[l & 1][tid];
      put_pair(p.pairs + X::QKV + col, s, tA);
      if (col >= D) {  // new K or V row of this position, for later steps
        const int c = col - D, isv = c >= D, cc = isv ? c - D : c, h = cc >> 6, e = cc & 63;
        (isv ? p.vc : p.kc)[(((size_t)l * H + h) * ctx + pos) * 64 + e] = s;
      }
    }

    // ---- B: attention (head ah, key chunk achunk) ----
    if (attn_blk) {
      // cached K/V rows of the first key group do not depend on this step: the
      // data waves request them while the control wave waits for q, k, v
      if (!ctrl) {
#pragma unroll
        for (int i = 0; i < KG; i++) {
          const int j = min(min(a0 + i, max(a0, a1 - 1)), pos);  // in bounds; row pos is replaced
          kreg[i] = Kc[(size_t)j * 64 + lane];
          vreg[i] = Vc[(size_t)j * 64 + lane];
        }
      }
      if (ctrl) {
        // q, k, v of this head: pairs [h*64, h*64+64) in each of the three thirds
        long it = 0;
        uint4 v0, v1, v2;
        for (;;) {
          reload_fence();
          v0 = nc.load4((X::QKV + 0 * D + ah * 64) * 8 + (lane % 32) * 16);
          v1 = nc.load4((X::QKV + 1 * D + ah * 64) * 8 + (lane % 32) * 16);
          v2 = nc.load4((X::QKV + 2 * D + ah * 64) * 8 + (lane % 32) * 16);
          const bool okk = v0.y == tA && v0.w == tA && v1.y == tA && v1.w == tA && v2.y == tA && v2.w == tA;
          if (__all(okk)) break;
          if (++it > SPIN_LIMIT || err_set(p.err)) {
            if (lane == 0) raise_err(p.err);
            fail();
            break;
          }
        }
        if (lane < 32) {
          qkvs[2 * lane] = __uint_as_float(v0.x);
          qkvs[2 * lane + 1] = __uint_as_float(v0.z);
          qkvs[64 + 2 * lane] = __uint_as_float(v1.x);
          qkvs[64 + 2 * lane + 1] = __uint_as_float(v1.z);
          qkvs[128 + 2 * lane] = __uint_as_float(v2.x);
          qkvs[128 + 2 * lane + 1] = __uint_as_float(v2.z);
        }
      }
      SYNC_OK();
      TM(2);
      if (!ctrl) {
        // lane = head dim; this wave's keys a0..a1 in groups of KG (row pos from qkvs)
        const float q = qkvs[lane];
        float m = -INFINITY, lsum = 0.f, acc = 0.f;
        for (int g0 = a0; g0 < a1; g0 += KG) {
          if (g0 != a0) {
#pragma unroll
            for (int i = 0; i < KG; i++) {
              const int j = min(min(g0 + i, a1 - 1), pos);
              kreg[i] = Kc[(size_t)j * 64 + lane];
              vreg[i] = Vc[(size_t)j * 64 + lane];
            }
          }
          float sc[KG];
          float gm = -INFINITY;
#pragma unroll
          for (int i = 0; i < KG; i++) {
            const int j = g0 + i;
            const float kv = (j == pos) ? qkvs[64 + lane] : kreg[i];
            const float sv = wave_sum_dpp(q * kv) * 0.125f;
            sc[i] = (j < a1) ? sv : -INFINITY;
            gm = fmaxf(gm, sc[i]);
          }
          const float nm = fmaxf(m, gm);
          const float corr = (m == -INFINITY) ? 0.f : expf(m - nm);
          lsum *= corr;
          acc *= corr;
#pragma unroll
          for (int i = 0; i < KG; i++) {
            const int j = g0 + i;
            const float pj = (j < a1) ? expf(sc[i] - nm) : 0.f;
            lsum += pj;
            acc += pj * ((j == pos) ? qkvs[128 + lane] : vreg[i]);
          }
          m = nm;
        }
        if (lane == 0) {
          wm[w] = m;
          wl[w] = lsum;
        }
        wo[w][lane] = acc;
      } else {
        if (lane == 0) {
          wm[NW - 1] = -INFINITY;
          wl[NW - 1] = 0.f;
        }
        wo[NW - 1][lane] = 0.f;
      }
      __syncthreads();
      if (tid < 64) {
        float M = -INFINITY;
        for (int i = 0; i < NW; i++) M = fmaxf(M, wm[i]);
        float Ls = 0.f, o = 0.f;
        if (M != -INFINITY) {
          for (int i = 0; i < NW; i++) {
            const float f = (wm[i] == -INFINITY) ? 0.f : expf(wm[i] - M);
            Ls += wl[i] * f;
            o += wo[i][tid] * f;
          }
        }
        float* ap = p.apart + (size_t)blk * X::AP_STRIDE;
        ap[tid] = o;
        if (tid == 0) {
          ap[64] = M;
          ap[65] = Ls;
        }
        stores_done();
      }
      __syncthreads();
      // the last of the head's AC chunk blocks to arrive combines the partials
      // and publishes the head's 64 outputs as tagged pairs
      if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(p.hcnt + ah, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = (old % AC) == AC - 1;
      }
      __syncthreads();
      if (last_s) {
        reload_fence();
        uint4* h4 = reinterpret_cast<uint4*>(aph);
        for (int i = tid; i < AC * X::AP_STRIDE / 4; i += NT)
          h4[i] = nc.load4(p.off_apart + (ah * AC * X::AP_STRIDE / 4 + i) * 16);
        __syncthreads();
        if (tid < 64) {
          float M = -INFINITY;
#pragma unroll
          for (int c = 0; c < AC; c++) M = fmaxf(M, aph[c * X::AP_STRIDE + 64]);
          float Ls = 0.f, o = 0.f;
#pragma unroll
          for (int c = 0; c < AC; c++) {
            const float mc = aph[c * X::AP_STRIDE + 64];
            const float f = (mc == -INFINITY) ? 0.f : expf(mc - M);
            Ls += aph[c * X::AP_STRIDE + 65] * f;
            o += aph[c * X::AP_STRIDE + tid] * f;
          }
          put_pair(p.pairs + X::O + ah * 64 + tid, o / Ls, tB);
        }
      }
    }
    tile_load<S::FMAX, S::FCH>(rf, t_fc);

    // ---- C: attn.proj + residual -> x2 ----
    if (ctrl && !wait_pairs<D>(nc, X::O, tB, os, p.err)) fail();
    SYNC_OK();
    __syncthreads();
    TM(3);
    tile_dot<S::PMAX, S::PCH, S::KC>(rp, os, part);
    tile_load<S::MMAX, S::MCH>(rm, t_mp);
    __syncthreads();
    if (tid < S::PCOL) {
      const int col = blk * S::PCOL + tid;
      float s = 0.f;
#pragma unroll
      for (int kc = 0; kc < S::KC; kc++) s += part[tid * S::KC + kc];
      put_pair(p.pairs + X::X2 + col, (s + bias_s[l & 1][S::QCOL + tid]) + xres[col], tC);
    }

    // ---- D: LN2 + mlp.fc + GELU -> h ----
    if (ctrl && !wait_pairs<D>(nc, X::X2, tC, x2s, p.err)) fail();
    SYNC_OK();
    TM(4);
    layernorm_regs<D>(x2s, xs, l2w, l2b, red);
    tile_dot<S::FMAX, S::FCH, S::KC>(rf, xs, part);
    tile_load<S::QMAX, S::QCH>(rq, t_qkv_next);
    load_ln<D>(vnext + S::V_LN1W, vnext + S::V_LN1B, l1w, l1b);
    __syncthreads();
    if (tid < S::FCOL) {
      const int col = blk * S::FCOL + tid;
      float s = 0.f;
#pragma unroll
      for (int kc = 0; kc < S::KC; kc++) s += part[tid * S::KC + kc];
      put_pair(p.pairs + X::HH + col, gelu_tanh(s + bias_s[l & 1][S::QCOL + S::PCOL + tid]), tD);
    }

    // ---- E: mlp.proj + residual -> x ----
    if (ctrl && !wait_pairs<4 * D>(nc, X::HH, tD, hs, p.err)) fail();
    SYNC_OK();
    TM(5);
    tile_dot<S::MMAX, S::MCH, S::KC4>(rm, hs, part);
    __syncthreads();
    if (tid < S::PCOL) {
      const int col = blk * S::PCOL + tid;
      float s = 0.f;
#pragma unroll
      for (int kc = 0; kc < S::KC4; kc++) s += part[tid * S::KC4 + kc];
      put_pair(p.pairs + X::X + col, (s + bias_s[l & 1][S::QCOL + S::PCOL + S::FCOL + tid]) + x2s[col], tE);
    }
    TM(6);
  }
#undef TM

  if (ok) {
    // ---- head: LN_f + tied projection over this block's vocab rows ----
    const unsigned tH = tagbase + 5 * p.L;
    const int R = p.V / NB;
    const int nch = R * S::KC;
    constexpr int HG = 8;  // head chunks per wave in flight
    const float4* t4 = reinterpret_cast<const float4*>(p.tok + (size_t)blk * R * D);
    float4 rh[HG];
    if (w < NDW) {
#pragma unroll
      for (int i = 0; i < HG; i++) rh[i] = t4[min(w + NDW * i, nch - 1) * 64 + lane];
    }
    const float* vf = p.vecs + (size_t)p.L * S::VL;
    load_ln<D>(vf, vf + D, l1w, l1b);
    if (ctrl && !wait_pairs<D>(nc, X::X, tagbase + 5 * (p.L - 1) + 4, xres, p.err)) fail();
    __syncthreads();
    ok = !fail_s;
    if (ok) {
      layernorm_regs<D>(xres, xs, l1w, l1b, red);
      if (w < NDW) {
        for (int g = 0; g < S::HMAX; g += HG) {
          float4 nx[HG];
#pragma unroll
          for (int i = 0; i < HG; i++) nx[i] = t4[min(w + NDW * (g + HG + i), nch - 1) * 64 + lane];
#pragma unroll
          for (int i = 0; i < HG; i++) {
            const int ch = w + NDW * (g + i);
            if (ch < nch) {
              const int kc = ch % S::KC;
              const float4 xv = *reinterpret_cast<const float4*>(xs + kc * 256 + lane * 4);
              const float q = wave_sum_dpp(rh[i].x * xv.x + rh[i].y * xv.y + rh[i].z * xv.z + rh[i].w * xv.w);
              if (lane == 0) part[ch] = q;
            }
          }
#pragma unroll
          for (int i = 0; i < HG; i++) rh[i] = nx[i];
        }
      }
      __syncthreads();
      if (w == 0) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        if (lane < R) {
          float s = 0.f;
#pragma unroll
          for (int kc = 0; kc < S::KC; kc++) s += part[lane * S::KC + kc];
          const int v = blk * R + lane;
          p.logits[v] = s;
          best = s;
          bi = v;
        }
        wave_argmax(best, bi);
        if (lane == 0) {  // value and index first, tag last
          *reinterpret_cast<uint2*>(&p.amax[blk]) = make_uint2(__float_as_uint(best), (unsigned)bi);
          stores_done();
          reinterpret_cast<unsigned*>(&p.amax[blk])[2] = tH;
        }
      }
      // block 0 collects every block's argmax: it proves all blocks read this
      // launch's counter, so the counter can advance
      if (blk == 0 && ctrl) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        long it = 0;
        bool good = true;
        for (;;) {
          reload_fence();
          bool okk = true;
          best = -INFINITY;
          bi = 0x7fffffff;
          for (int b = lane; b < NB; b += 64) {
            const uint4 a = nc.load4(p.off_amax + 16 * b);
            okk &= a.z == tH;
            argmax_merge(best, bi, __uint_as_float(a.x), (int)a.y);
          }
          if (__all(okk)) break;
          if (++it > SPIN_LIMIT || err_set(p.err)) {
            if (lane == 0) raise_err(p.err);
            good = false;
            break;
          }
        }
        if (good) {
          wave_argmax(best, bi);
          if (lane == 0) {
            if (p.greedy) {
              const int total = p.src.tok_off + 1 + n;  // prompt_len + n
              p.tokens_out[total] = bi;
              if (n < p.max_new) p.out_ids[n] = bi;
              if (p.out_counts[0] < 0 && p.eos >= 0 && bi == p.eos) p.out_counts[0] = n + 1;
              *p.step_out = n + 1;
            }
            __hip_atomic_fetch_add(p.launch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
  }
  (void)fail;
  trace_mark(p.trace, 127);
}

// tile[b][c][k] = W[k][b*ncol + c] for a row-major W [K][N]
__global__ void k_relayout(const float* __restrict__ W, int K, int N, int ncol, float* __restrict__ tile) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)K * N) return;
  const int k = (int)(i % K);
  const size_t bc = i / K;
  const int c = (int)(bc % ncol), b = (int)(bc / ncol);
  tile[i] = W[(size_t)k * N + (size_t)b * ncol + c];
}

__global__ void k_copy(const float* __restrict__ src, float* __restrict__ dst, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// Uncached device memory stays allocated until the process ends (returning it
// to the runtime after a kernel has read it is not safe on this platform);
// released regions go to a per-device free list and are reused.
std::mutex g_uc_mu;
std::vector<std::tuple<int, size_t, void*>> g_uc_free;

void* uc_take(int dev, size_t bytes) {
  {
    std::lock_guard<std::mutex> g(g_uc_mu);
    for (size_t i = 0; i < g_uc_free.size(); i++)
      if (std::get<0>(g_uc_free[i]) == dev && std::get<1>(g_uc_free[i]) >= bytes) {
        void* p = std::get<2>(g_uc_free[i]);
        g_uc_free.erase(g_uc_free.begin() + i);
        return p;
      }
  }
  void* p = nullptr;
  if (hipExtMallocWithFlags(&p, bytes, hipDeviceMallocUncached) != hipSuccess) return nullptr;
  return p;
}

void uc_give(int dev, size_t bytes, void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> g(g_uc_mu);
  g_uc_free.emplace_back(dev, bytes, p);
}

// uncached region layout (bytes)
struct UcLayout {
  size_t pairs, apart, amax, total;
  UcLayout(int D, int H) {
    pairs = 0;
    apart = pairs + (size_t)10 * D * sizeof(uint2);
    amax = (apart + (size_t)H * AC * 68 * sizeof(float) + 255) / 256 * 256;
    total = amax + (size_t)NB * sizeof(uint4);
  }
};

}  // namespace

int FastDecode::init(const fh_model_desc& d, int compute_units) {
  enabled = false;
  D = d.d_model;
  H = d.n_heads;
  L = d.n_layers;
  V = d.vocab_size;
  ctx = d.context_length;
  C = AC;
  blocks = NB;
  const bool shape_ok = d.dtype == FH_DTYPE_F32 && d.max_batch == 1 && D == 768 && D / H == 64 && V % NB == 0 &&
                        V / NB <= 64 && H * AC <= 192 && H * AC <= NB && compute_units >= NB &&
                        5 * L + 2 <= TAGS;
  if (!shape_ok) return FH_OK;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_decode_step<768>, NT, 0) != hipSuccess || occ < 1)
    return FH_OK;
  if (hipGetDevice(&device) != hipSuccess) return FH_ERR_HIP;
  tile_floats = (size_t)12 * D * D * L;
  if (hipMalloc(&tiles, tile_floats * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  const size_t vec_floats = (size_t)13 * D * L + 2 * D;
  if (hipMalloc(&vecs, vec_floats * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  UcLayout u(D, H);
  xch_bytes = u.total;
  uc = static_cast<char*>(uc_take(device, xch_bytes));
  if (!uc) return FH_ERR_OOM;
  if (hipMalloc(&ctl, 256) != hipSuccess) return FH_ERR_OOM;
  if (reset_state() != FH_OK) return FH_ERR_HIP;
  const char* tr = getenv("FORGE_HIP_TRACE");
  if (tr && tr[0] == '1') {
    if (hipMalloc(&trace, 256 * sizeof(unsigned long long)) != hipSuccess) return FH_ERR_OOM;
    if (hipMemset(trace, 0, 256 * sizeof(unsigned long long)) != hipSuccess) return FH_ERR_HIP;
  }
  enabled = true;
  return FH_OK;
}

int FastDecode::build(hipStream_t st, const float* const* params) {
  if (!enabled) return FH_OK;
  const int qcol = 3 * D / NB, pcol = D / NB, fcol = 4 * D / NB;
  auto copy = [&](const float* src, float* dst, int n) {
    hipLaunchKernelGGL(k_copy, dim3((n + 255) / 256), dim3(256), 0, st, src, dst, n);
    return hipGetLastError() == hipSuccess;
  };
  for (int l = 0; l < L; l++) {
    float* tl = tiles + (size_t)l * 12 * D * D;
    const float* const* PL = params + 2 + 12 * l;
    struct {
      const float* W;
      int K, N, ncol;
      float* out;
    } jobs[4] = {
        {PL[2], D, 3 * D, qcol, tl},
        {PL[4], D, D, pcol, tl + (size_t)3 * D * D},
        {PL[8], D, 4 * D, fcol, tl + (size_t)4 * D * D},
        {PL[10], 4 * D, D, pcol, tl + (size_t)8 * D * D},
    };
    for (auto& j : jobs) {
      const size_t tot = (size_t)j.K * j.N;
      hipLaunchKernelGGL(k_relayout, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, j.W, j.K, j.N, j.ncol,
                         j.out);
      if (hipGetLastError() != hipSuccess) return FH_ERR_HIP;
    }
    float* vl = vecs + (size_t)l * 13 * D;
    // ln1.w ln1.b qkv.b proj.b ln2.w ln2.b fc.b mproj.b (registry slots 0,1,3,5,6,7,9,11)
    if (!copy(PL[0], vl, D) || !copy(PL[1], vl + D, D) || !copy(PL[3], vl + 2 * D, 3 * D) ||
        !copy(PL[5], vl + 5 * D, D) || !copy(PL[6], vl + 6 * D, D) || !copy(PL[7], vl + 7 * D, D) ||
        !copy(PL[9], vl + 8 * D, 4 * D) || !copy(PL[11], vl + 12 * D, D))
      return FH_ERR_HIP;
  }
  const float* const* PF = params + 2 + 12 * L;
  if (!copy(PF[0], vecs + (size_t)13 * D * L, D) || !copy(PF[1], vecs + (size_t)13 * D * L + D, D))
    return FH_ERR_HIP;
  return hipStreamSynchronize(st) == hipSuccess ? FH_OK : FH_ERR_HIP;
}

int FastDecode::enqueue(hipStream_t st, const Step& s) {
  if (!enabled) return FH_ERR_STATE;
  if (!s.src.tokens || !s.src.step || !s.tokens || !s.step || !s.kcache || !s.vcache || !s.logits || !s.out_ids ||
      !s.out_counts || s.src.pos_mul != 1 || s.max_new <= 0)
    return FH_ERR_INVALID;
  UcLayout u(D, H);
  KParams k{};
  k.src = s.src;
  k.tiles = tiles;
  k.vecs = vecs;
  k.tok = s.tok_emb;
  k.pos = s.pos_emb;
  k.kc = s.kcache;
  k.vc = s.vcache;
  k.logits = s.logits;
  k.out_ids = s.out_ids;
  k.out_counts = s.out_counts;
  k.pairs = reinterpret_cast<uint2*>(uc + u.pairs);
  k.apart = reinterpret_cast<float*>(uc + u.apart);
  k.hcnt = reinterpret_cast<unsigned*>(ctl) + 32;
  k.amax = reinterpret_cast<uint4*>(uc + u.amax);
  k.uc_bytes = (int)u.total;
  k.off_apart = (int)u.apart;
  k.off_amax = (int)u.amax;
  k.launch = reinterpret_cast<unsigned*>(ctl);
  k.err = reinterpret_cast<int*>(ctl) + 16;
  k.V = V;
  k.ctx = ctx;
  k.H = H;
  k.L = L;
  k.max_new = s.max_new;
  k.eos = s.eos;
  k.greedy = s.greedy;
  k.tokens_out = s.tokens;
  k.step_out = s.step;
  k.trace = trace;
  hipLaunchKernelGGL(k_decode_step<768>, dim3(NB), dim3(NT), 0, st, k);
  return hipGetLastError() == hipSuccess ? FH_OK : FH_ERR_HIP;
}

// Tags of zeroed memory are 0; the launch counter starts at 1, so no live tag
// (counter * 128 + phase) ever equals a stale or cleared one.
int FastDecode::reset_state() {
  const unsigned one = 1;
  if (hipMemset(ctl, 0, 256) != hipSuccess) return FH_ERR_HIP;
  if (hipMemcpy(ctl, &one, sizeof one, hipMemcpyHostToDevice) != hipSuccess) return FH_ERR_HIP;
  if (hipMemset(uc, 0, xch_bytes) != hipSuccess) return FH_ERR_HIP;
  return hipDeviceSynchronize() == hipSuccess ? FH_OK : FH_ERR_HIP;
}

int FastDecode::reset() { return enabled ? reset_state() : FH_OK; }

int FastDecode::check_error() {
  if (!enabled) return FH_OK;
  int h = 0;
  if (hipMemcpy(&h, reinterpret_cast<int*>(ctl) + 16, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
    return FH_ERR_HIP;
  return h ? FH_ERR_HIP : FH_OK;
}

void FastDecode::release() {
  if (tiles) (void)hipFree(tiles);
  if (vecs) (void)hipFree(vecs);
  uc_give(device, xch_bytes, uc);
  if (ctl) (void)hipFree(ctl);
  if (trace) (void)hipFree(trace);
  tiles = vecs = nullptr;
  uc = nullptr;
  ctl = nullptr;
  trace = nullptr;
  enabled = false;
}

}  // namespace fh
