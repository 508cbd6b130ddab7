// decode_fast.hip -- persistent batch-1 fp32 decode step for MI355X (gfx950).
//
// One launch runs a whole decode step of the token loop (GptModel.ForwardLast
// on the cached window, src/LLM.Core/Model/GptModel.cs:202-222, then
// Sampler.Greedy, src/LLM.Core/Inference/Sampler.cs:14-20): 256 blocks, one per
// CU; the dispatcher deals blocks round-robin over the 8 XCDs, so block b is
// slot b / 8 of the 32 blocks on its XCD (read from the hardware).  Each
// block has 256 threads: waves 0..2 hold weight tiles in registers, wave 3 is
// the control wave that collects hand-offs.  Per layer:
//   A  LN1 + QKV: the 192 q/k/v columns of head h are computed by blocks of
//      XCD h % 8 only, so q/k/v reach that head's attention blocks through the
//      XCD's own L2; the new K/V row goes into the cache
//   B  attention of head h by blocks of XCD h % 8: 32 keys per data wave
//      (lane l: dims 4*(l % 16) .. +3 of every fourth key), 96 keys per block,
//      each block publishing a partial (o, max, sum); every block of the XCD
//      combines the partials of all the XCD's heads itself
//   C  attn.proj columns + residual -> x2
//   D  LN2 + mlp.fc columns + GELU -> h
//   E  mlp.proj columns + residual -> x
// then LN_f + the tied head (64 vocab rows per block) and, in greedy mode, the
// argmax.  At batch 1 every weight is used once per token, so the step is
// bound by HBM bytes plus the chain of hand-offs between phases.
//
// Hand-offs without grid barriers: every value passed from one phase to the
// next is stored as a 64-bit (value, tag) pair, the tag being this launch's
// sequence number for the producing phase (launch counter * 128 + phase).  A
// consumer's control wave re-reads the pairs it needs until every tag
// matches, then copies the values to LDS.  Values that cross
// XCDs (x, x2, h, o, the per-block argmax) live in uncached memory; values that
// stay inside one XCD (q/k/v, attention partials) live in ordinary device
// memory, where the XCD's L2 is the coherence point.  Reads of both bypass
// the CU's L1 (buffer loads with the SC0|SC1 policy).  Because every consumer
// needs the outputs of a whole phase before it, no producer can run a full
// phase ahead of a reader, so no pair is overwritten while still needed.  The
// launch counter only grows (also across resets), so stale pairs never match.
//
// The data waves hold every tile of the current layer in registers (each
// block's columns re-laid out once into contiguous column-major tiles) and
// request the next layer's tile as soon as the current one is consumed, so
// HBM streams continuously while the control wave waits.  Cached K/V rows are
// requested before x arrives.  Every wait is bounded: past the spin limit the
// error word is set and all blocks leave.
#include <float.h>
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <tuple>
#include <vector>

#include "decode_fast.hpp"

namespace fh {

namespace {

constexpr int NB = 256;      // blocks
constexpr int NT = 256;      // threads per block: one wave per SIMD
constexpr int NW = NT / 64;
constexpr int NDW = NW - 1;  // data waves (the last wave is the control wave)
constexpr int NX = 8;        // XCDs
constexpr int SLOTS = NB / NX;
constexpr int KPW = 32;            // attention keys per data wave (two lanes per key)
constexpr int KPB = KPW * NDW;     // attention keys per block
constexpr int TAGS = 128;          // tag values reserved per launch
constexpr int PH = 8;              // tagged phases per layer
constexpr long SPIN_LIMIT = 400000;
constexpr int PART = 68;           // pairs per attention partial: o[64], m, l, pad[2]

// vocabulary rows per block of the tied head: ceil(V / 256), at least one per data wave
__host__ __device__ __forceinline__ int head_rows(int V) { return max(NDW, (V + NB - 1) / NB); }

// The sampled kernel keeps the window's ids in LDS (ctx <= 1536) and draws with
// top-k <= KMAX inside the launch.
constexpr int HCAP = 1536;
constexpr int KMAX = 63;

__device__ __forceinline__ bool err_set(int* err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
// The first failing wait records where it was: 1 << 31 | wait << 24 | layer << 16 | block
// (waits: 1 x, 2 q/k/v, 3 attention partials, 5 attn.proj partials, 6 x2, 7 h,
// 8 mlp.proj partials, 9 final x, 10 argmax; 4 is not used), or which check
// failed (11 a token id outside [0, V), 12 two blocks of the launch on the same
// (XCD, slot), 13 the in-kernel sampler met a non-finite logit or an exact tie at
// a top-k threshold: the host then repeats the generation on the per-step path;
// 14 and 15 the sampler's two waits).  A wait that gives up because another block
// already failed records nothing.
enum WaitId { W_X = 1, W_QKV, W_PART, W_O, W_PX2, W_X2, W_H, W_PX, W_XF, W_AMAX, W_TOK, W_XCD, W_SAMPLE, W_SKEYS,
              W_SLIST };
__device__ __forceinline__ int err_code(int wait, int l) {
  return (int)(0x80000000u | ((unsigned)wait << 24) | ((unsigned)(l & 0xff) << 16) | blockIdx.x);
}
__device__ __forceinline__ void raise_err(int* err, int code) {
  int expected = 0;
  __hip_atomic_compare_exchange_strong(err, &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
}
// keeps the compiler from reusing values loaded before this point
__device__ __forceinline__ void reload_fence() { asm volatile("" ::: "memory"); }
// this wave's LDS writes are complete and visible to its own later reads
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ void put_pair(uint2* dst, float v, unsigned tag) {
  *dst = make_uint2(__float_as_uint(v), tag);
}

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

// Reads of the hand-off areas go through a raw buffer resource with the
// SC0|SC1 cache policy: they miss in the CU's L1, so a re-read sees other CUs'
// stores (plain loads would keep hitting a stale L1 line).  Out-of-range
// offsets read as 0.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
template <int AUX>
struct NcBufT {
  __amdgpu_buffer_rsrc_t r;
  __device__ NcBufT(const void* base, int bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000)) {}
  __device__ __forceinline__ uint4 load4(int byte_off) const {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, AUX);
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ uint2 load2(int byte_off) const {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, AUX);
    return make_uint2(v.x, v.y);
  }
};
#ifndef FH_LOCAL_AUX
#define FH_LOCAL_AUX 17
#endif
using NcBuf = NcBufT<17>;            // uncached (cross-XCD) hand-offs
using LcBuf = NcBufT<FH_LOCAL_AUX>;  // XCD-local hand-offs

template <int D, int H>
struct Shape {
  static constexpr int HD = 64;
  static constexpr int KC = D / 256;             // 256-float chunks per K=D column
  static constexpr int HPX = (H + NX - 1) / NX;  // heads per XCD (at most)
  static constexpr int SPH = SLOTS / HPX;        // slots per head
  static constexpr int QCMAX = 3 * HD * HPX / SLOTS;  // qkv columns per block (at most)
  static constexpr int QCW = QCMAX / NDW;              // qkv columns per data wave (at most)
  static constexpr int HX = 4 * D / NX;    // mlp.fc columns (h values) per XCD
  static constexpr int FCOL = HX / SLOTS;  // h values per block
  static constexpr int FCW = FCOL / NDW;   // per data wave
  static constexpr int RSC = D / SLOTS;    // output columns per slot of attn.proj / mlp.proj
  static constexpr int G = RSC / NDW / 4;  // 4-column groups per data wave
  static constexpr int PJ = HPX;           // attn.proj: one 64-row piece per head of the XCD
  static constexpr int MJ = HX / 64;       // mlp.proj: 64-row pieces of the XCD's h slice
  static constexpr int RMAX = 64;          // vocab rows per block (V <= 16384)
  // tile floats per (virtual) block; the 1 KB chunks of attn.proj / mlp.proj hold
  // 4 output columns x 64 rows (lane l: rows 4*(l%16)..+3 of column l/16)
  static constexpr size_t QT = (size_t)QCMAX * D, PT = (size_t)PJ * NDW * G * 256, FT = (size_t)FCOL * D,
                          MT = (size_t)NDW * G * MJ * 256;
  static constexpr size_t LAYER = (size_t)NB * (QT + PT + FT + MT);
  // per-block bias table per layer: qkv[QCMAX] fc[FCOL] proj[RSC] mproj[RSC]
  static constexpr int B_Q = 0, B_F = QCMAX, B_P = QCMAX + FCOL, B_M = QCMAX + FCOL + RSC,
                       BT = QCMAX + FCOL + 2 * RSC;
  static_assert(D == H * HD, "head_dim 64");
  static_assert(D % 256 == 0 && HX % SLOTS == 0 && HX % 64 == 0, "chunked columns");
  static_assert(QCMAX % NDW == 0 && FCOL % NDW == 0 && RSC % (4 * NDW) == 0, "columns split evenly");
  static_assert(SPH * HPX == SLOTS, "slots split evenly over an XCD's heads");
};

// uncached (cross-XCD) pair layout: the per-XCD partial sums of attn.proj and mlp.proj
template <int D>
struct Xu {
  static constexpr int PX2 = 0, PX = NX * D, NPAIR = 2 * NX * D;
};
// per-XCD local pair layout
template <int D, int H>
struct Xl {
  using S = Shape<D, H>;
  static constexpr int QKV = 0;                                   // q, k, v of the XCD's heads
  static constexpr int PARTS = QKV + 3 * S::HD * S::HPX;          // attention partials
  static constexpr int X2 = PARTS + S::HPX * S::SPH * PART;       // x2 (every XCD keeps a copy)
  static constexpr int HH = X2 + D;                               // the XCD's h slice
  static constexpr int X = HH + S::HX;                            // x (every XCD keeps a copy)
  static constexpr int SAMP = X + D;                              // sampler keys: 64 per block of the XCD
  static constexpr int SAMPT = SAMP + SLOTS * 64;                 // the two largest keys of each block
  static constexpr int STRIDE = SAMPT + SLOTS * 2;
};

struct KParams {
  RowSrc src;
  const float* tiles;
  const float* vecs;  // ln_f weight, bias
  const float* btab;
  const float* tok;   // tok_emb, or its copy zero-padded to 256 * R rows (the head reads whole shares)
  const float* pos;
  float* kc;
  float* vc;
  float* logits;
  int* out_ids;
  int* out_counts;
  uint2* uc;          // uncached pairs (Xu), then the argmax records, then the slot claims
  int uc_bytes;
  int off_amax;       // byte offset of the argmax records in uc
  int off_claim;      // byte offset of the (XCD, slot) claim words in uc
  int off_slist;      // byte offset of the sampler's per-XCD top-k lists in uc (8 x 64 records)
  uint2* xl;          // per-XCD pairs (Xl), ordinary device memory
  int xl_bytes;
  unsigned* launch;   // launch counter
  int* err;
  int V, ctx, L, max_new, eos, greedy;
  int Vp;             // 256 * rows per block of the head (V rounded up, at least 768): rows >= V are skipped
  // sampled kernel: Sampler.Sample with top-k after ApplyRepetitionControls (Sampler.cs:29-69, 111-165)
  const double* uniforms;  // [max_new]: the NextDouble of step n
  float temperature, penalty;
  int top_k, ngram;
  int nsteps;         // decode steps of this launch (greedy: the argmax feeds the next step)
  int* tokens_out;    // same buffer as src.tokens, written by the greedy argmax
  int* step_out;      // same word as src.step
  unsigned long long* trace;  // optional: block 0 timestamps
};

// Optional timestamps (FORGE_HIP_TRACE=1): TRACE_PER entries per block, written
// by the control wave (marks 0..15, 30, 31) and data wave 0 (marks 16..29).
constexpr int TRACE_PER = 64;  // control wave marks [0, 32), data wave 0 marks [32, 64)
__device__ __forceinline__ void trace_mark(unsigned long long* t, int i) {
  if (t && threadIdx.x == (NT - 64)) t[blockIdx.x * TRACE_PER + i] = wall_clock64();
}
// data wave 0 keeps its marks in LDS (no extra memory requests in the data
// waves' queue); the control wave writes them out at the end
__device__ __forceinline__ void trace_mark_d(unsigned long long* t, unsigned long long* lds, int i) {
  if (t && threadIdx.x == 0) lds[i] = wall_clock64();
}

#ifndef FH_POLL2
#define FH_POLL2 0
#endif
// The poll loop of every gather: issue(v) requests R 16-byte values per lane,
// good(v) says whether every tag matches (wave-uniform), take(v) stores them.
// With FH_POLL2 a second read is requested before the first is checked, so a
// poll result comes back about twice as often while reads wait behind the
// CU's tile loads.
template <int R, typename Issue, typename Good, typename Take>
__device__ __forceinline__ bool poll(Issue issue, Good good, Take take, int* err, int code, long* npoll) {
  const int lane = threadIdx.x & 63;
  long it = 0;
#if FH_POLL2
  uint4 va[R], vb[R];
  issue(va);
  for (;;) {
    issue(vb);
    if (good(va)) {
      take(va);
      break;
    }
    issue(va);
    if (good(vb)) {
      take(vb);
      break;
    }
    it += 2;
    if ((it & 63) == 0 && (it > SPIN_LIMIT || err_set(err))) {
      if (lane == 0 && it > SPIN_LIMIT) raise_err(err, code);
      return false;
    }
  }
#else
  uint4 v[R];
  for (;;) {
    issue(v);
    if (good(v)) {
      take(v);
      break;
    }
    if ((++it & 63) == 0 && (it > SPIN_LIMIT || err_set(err))) {
      if (lane == 0 && it > SPIN_LIMIT) raise_err(err, code);
      return false;
    }
  }
#endif
  if (npoll) *npoll = it;
  return true;
}

// Control wave: waits until pairs[pair0, pair0 + n) all carry `tag` (n <= N),
// then stores the values to out[0, n) (LDS).
template <int N, typename B>
__device__ bool gather(const B& nc, int pair0, unsigned tag, float* out, int* err, int code, int n = N,
                       long* npoll = nullptr) {
  static_assert(N % 2 == 0, "pairs come in 16-byte loads");
  constexpr int R = (N + 127) / 128;
  const int lane = threadIdx.x & 63;
  return poll<R>(
      [&](uint4(&v)[R]) {
        reload_fence();
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = nc.load4(pair0 * 8 + (r * 64 + lane) * 16);
      },
      [&](const uint4(&v)[R]) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; r++)
          if ((r * 64 + lane) * 2 < n) ok &= (v[r].y == tag) & (v[r].w == tag);
        return __all(ok) != 0;
      },
      [&](const uint4(&v)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const int i = 2 * (r * 64 + lane);
          if (i < n)
            *reinterpret_cast<float2*>(out + i) = make_float2(__uint_as_float(v[r].x), __uint_as_float(v[r].z));
        }
      },
      err, code, npoll);
}

// Control wave: the RSC-column slice [slot*RSC, +RSC) of all NX per-XCD partial
// vectors (pairs at pair0 + x*D + c), into out[x*RSC + c] (LDS).
template <int D, int RSC>
__device__ bool gather_slices(const NcBuf& nc, int pair0, int slot, unsigned tag, float* out, int* err, int code,
                              long* npoll = nullptr) {
  constexpr int Q = RSC / 2;  // 16-byte loads per slice
  constexpr int NQ = NX * Q;
  constexpr int R = (NQ + 63) / 64;
  const int lane = threadIdx.x & 63;
  return poll<R>(
      [&](uint4(&v)[R]) {
        reload_fence();
#pragma unroll
        for (int r = 0; r < R; r++) {
          const int u = min(r * 64 + lane, NQ - 1), x = u / Q, q = u % Q;
          v[r] = nc.load4((pair0 + x * D + slot * RSC + 2 * q) * 8);
        }
      },
      [&](const uint4(&v)[R]) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < R; r++) ok &= (v[r].y == tag) & (v[r].w == tag);
        return __all(ok) != 0;
      },
      [&](const uint4(&v)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
          const int u = r * 64 + lane;
          if (u < NQ) {
            const int x = u / Q, q = u % Q;
            *reinterpret_cast<float2*>(out + x * RSC + 2 * q) =
                make_float2(__uint_as_float(v[r].x), __uint_as_float(v[r].z));
          }
        }
      },
      err, code, npoll);
}

// sum over the 16 lanes of each DPP row (quad permutes, half-row and row mirrors)
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// max over the 16 lanes of each DPP row
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  return v;
}

__device__ __forceinline__ float dot4(const float4 a, const float4 b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// LayerNorm of xin[D] (LDS) for this lane's elements k = c*256 + lane*4 + 0..3
// (c < KC), computed by each wave on its own (biased variance, eps 1e-5,
// ((x - mu) * rs) * w + b as CpuBackend.LayerNormForward).
template <int KC, int D>
__device__ __forceinline__ void ln_lane(const float* xin, const float4 (&w)[KC], const float4 (&b)[KC],
                                        float4 (&xn)[KC]) {
  const int lane = threadIdx.x & 63;
  float4 xv[KC];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++) {
    xv[c] = *reinterpret_cast<const float4*>(xin + c * 256 + lane * 4);
    s += (xv[c].x + xv[c].y) + (xv[c].z + xv[c].w);
  }
  const float mu = wave_sum_dpp(s) * (1.f / (float)D);
  float v = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++) {
    const float a = xv[c].x - mu, bb = xv[c].y - mu, cc = xv[c].z - mu, dd = xv[c].w - mu;
    v += (a * a + bb * bb) + (cc * cc + dd * dd);
  }
  const float var = wave_sum_dpp(v);
  const float rs = __frsqrt_rn(var * (1.f / (float)D) + 1e-5f);
#pragma unroll
  for (int c = 0; c < KC; c++) {
    xn[c].x = (xv[c].x - mu) * rs * w[c].x + b[c].x;
    xn[c].y = (xv[c].y - mu) * rs * w[c].y + b[c].y;
    xn[c].z = (xv[c].z - mu) * rs * w[c].z + b[c].z;
    xn[c].w = (xv[c].w - mu) * rs * w[c].w + b[c].w;
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
// Weight tiles: every tile is read once per token, so its loads carry the
// non-temporal hint (NT) and do not displace the hand-off pairs and KV rows the
// launch re-reads from the L2 (C2: 146.6 -> 140.6 us per token; the head rows and
// the KV loads with the hint measured no different, and the hint on half of the
// layers, the other half left cacheable, 148.5).
__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, int off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// the same through the L2 (the SC1 policy misses the CU's L1): for rows that
// other CUs write during the launch (the KV cache)
__device__ __forceinline__ float4 ld4_l2(__amdgpu_buffer_rsrc_t r, int off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// r[i] = chunk i of a tile (chunk = 64 lanes x float4 = 1 KB).  Loads through a
// buffer resource: one base in scalar registers and constant offsets; with
// real == false the resource is empty and the loads return zeros without
// touching memory (every register is still written on every path).
template <int N>
__device__ __forceinline__ void load_chunks(float4 (&r)[N], const float* tile, bool real) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(tile, real ? N * 1024 : 0);
  const int off = (threadIdx.x & 63) * 16;
#pragma unroll
  for (int i = 0; i < N; i++) r[i] = ld4(rs, off + i * 1024);
}

// GELU (tanh form, CpuBackend.Gelu) with tanh(u) = 1 - 2 / (exp(2u) + 1) on the
// hardware exponential: within a few 1e-7 of the libm form
__device__ __forceinline__ float gelu_fast(float v) {
  const float C = 0.7978845238685608f;  // MathF.Sqrt(2f / MathF.PI) in fp32
  const float u = C * (v + 0.044715f * v * v * v);
  const float t = 1.f - 2.f * __frcp_rn(__expf(2.f * u) + 1.f);
  return 0.5f * v * (1.f + t);
}

// LayerNorm statistics of xin[D] (LDS) for this lane's elements k = c*256 +
// lane*4 + 0..3: d = x - mu, returns rs = 1 / sqrt(var + 1e-5) (biased
// variance, CpuBackend.LayerNormForward).  The LayerNorm weight is folded into
// the tiles and its bias into the bias table, so a column is rs * (d . W') + c.
template <int KC, int D>
__device__ __forceinline__ float ln_center(const float* xin, float4 (&d)[KC]) {
  const int lane = threadIdx.x & 63;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++) {
    d[c] = *reinterpret_cast<const float4*>(xin + c * 256 + lane * 4);
    s += (d[c].x + d[c].y) + (d[c].z + d[c].w);
  }
  const float mu = wave_sum_dpp(s) * (1.f / (float)D);
  float v = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++) {
    d[c].x -= mu;
    d[c].y -= mu;
    d[c].z -= mu;
    d[c].w -= mu;
    v += (d[c].x * d[c].x + d[c].y * d[c].y) + (d[c].z * d[c].z + d[c].w * d[c].w);
  }
  const float var = wave_sum_dpp(v);
  return __frsqrt_rn(var * (1.f / (float)D) + 1e-5f);
}

// Control wave: the attention partials of the XCD's nh heads, nkb key blocks
// each (pairs at pair0 + (j * SPH + kb) * PART + e), into out[(j * SPH + kb) * PART + e].
// RA = loads per lane (ceil(n / 64)) is a template parameter so that every
// load of a poll is issued before the first wait.
template <int D, int H, int RA, typename B>
__device__ bool gather_parts_r(const B& nc, int pair0, int nh, int nkb, unsigned tag, float* out, int* err, int code,
                               long* npoll, unsigned long long* tfirst) {
  using S = Shape<D, H>;
  constexpr int Q = PART / 2;  // 16-byte loads per partial
  const int lane = threadIdx.x & 63;
  const int per = nkb * Q, n = nh * per;
  // byte offset of each of this lane's loads, clamped into range: the extra
  // lanes re-read the last unit, check its tags and store its values again, so
  // no per-lane condition (held in scalar registers) is needed
  int off[RA];
#pragma unroll
  for (int i = 0; i < RA; i++) {
    const int u = min(i * 64 + lane, n - 1), j = u / per, q = u - j * per;
    off[i] = (pair0 + j * S::SPH * PART + 2 * q) * 8;
  }
  uint4 v[RA];
  long it = 0;
  for (;;) {
    reload_fence();
#pragma unroll
    for (int i = 0; i < RA; i++) v[i] = nc.load4(off[i]);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < RA; i++) ok &= (v[i].y == tag) & (v[i].w == tag);
    if (tfirst && it == 0) *tfirst = wall_clock64();
    if (__all(ok)) break;
    if ((++it & 63) == 0 && (it > SPIN_LIMIT || err_set(err))) {
      if (lane == 0 && it > SPIN_LIMIT) raise_err(err, code);
      return false;
    }
  }
  if (npoll) *npoll = it;
#pragma unroll
  for (int i = 0; i < RA; i++) {
    const int u = min(i * 64 + lane, n - 1), j = u / per, q = u - j * per;
    *reinterpret_cast<float2*>(out + j * S::SPH * PART + 2 * q) =
        make_float2(__uint_as_float(v[i].x), __uint_as_float(v[i].z));
  }
  return true;
}

template <int D, int H, typename B>
__device__ bool gather_parts(const B& nc, int pair0, int nh, int nkb, unsigned tag, float* out, int* err, int code,
                             long* npoll = nullptr, unsigned long long* tfirst = nullptr) {
  using S = Shape<D, H>;
  static_assert((S::HPX * S::SPH * PART / 2 + 63) / 64 <= 17, "partial loads per lane");
  // a few sizes keep the code small (extra lanes re-read the last unit)
  const int ra = (nh * nkb * (PART / 2) + 63) / 64;
  if (ra <= 3) return gather_parts_r<D, H, 3>(nc, pair0, nh, nkb, tag, out, err, code, npoll, tfirst);
  if (ra <= 6) return gather_parts_r<D, H, 6>(nc, pair0, nh, nkb, tag, out, err, code, npoll, tfirst);
  if (ra <= 11) return gather_parts_r<D, H, 11>(nc, pair0, nh, nkb, tag, out, err, code, npoll, tfirst);
  return gather_parts_r<D, H, 17>(nc, pair0, nh, nkb, tag, out, err, code, npoll, tfirst);
}

// LDS of one block
template <int D, int H>
struct Lds {
  using S = Shape<D, H>;
  __align__(16) float xres[D];
  __align__(16) float x2s[D];
  __align__(16) float os[S::HD * S::HPX];              // o of the XCD's heads
  __align__(16) float hs[S::HX];                       // the XCD's h slice
  __align__(16) float rsv[NX * S::RSC];                // this slot's columns of the per-XCD partials
  __align__(16) float qkvs[192];                       // this head's q, new k, new v
  __align__(16) float wo[NW][64];                      // per-wave attention partials
  __align__(16) float parts[S::HPX * S::SPH * PART];  // attention partials of the XCD's heads
  float pw[64];                                        // their weights in the combination
  float pl[4];                                         // and each head's softmax denominator
  float wm[NW], wl[NW];
  float bias_s[2][S::BT];
  float hval[S::RMAX];
  __align__(16) float lnf[2 * D];  // ln_f weight, bias
  unsigned long long trd[32];  // data wave 0's trace marks
  int fail;
};

// LDS of the sampled kernel's sampler: the window's ids, the XCD leader's 2048
// gathered values, and the selection scratch
template <bool SAMPLED>
struct SampLds {
  int hist[1];
  float cv[1];
  int cr[1];
};
template <>
struct SampLds<true> {
  int hist[HCAP];
  float cv[NB / NX * 64];
  int cr[NB / NX * 64];
};

// The tied head's rows, per data wave (rows w, w + 3, ... of the block's share).
// ROWS of them stay in LDS for the whole launch (the table does not change
// between steps, so they are read from HBM once per launch instead of once per
// token; 12 fill the LDS the sampled kernel leaves); INFLIGHT of the rest stream
// from HBM at a time.  Both are measured per kernel: the greedy kernel holds 4
// and streams two at a time (145.7 against 147.5 us per token holding none; 6,
// 8 or 12 rows measured 152.7-156.7: the layers' code came out slower; later, with
// the current tile request sites, 2, 3, 5, 6 or 8 rows 141.9-144.0 against 136.6,
// and one, two or three rows in flight 138.2 / 135.7-136.1 / 136.5-136.7), the
// sampled kernel holds 12 and streams two at a time (one or three: 152.7 / 150.4
// against 149.9).
#ifndef FH_HRES_G
#define FH_HRES_G 4
#endif
#ifndef FH_HRES_S
#define FH_HRES_S 12
#endif
#ifndef FH_HG_G
#define FH_HG_G 2
#endif
#ifndef FH_HG_S
#define FH_HG_S 2
#endif
template <bool SAMPLED>
struct HeadRes {
  static constexpr int ROWS = SAMPLED ? FH_HRES_S : FH_HRES_G;
  static constexpr int INFLIGHT = SAMPLED ? FH_HG_S : FH_HG_G;
};
// the LDS rows (only kernels that hold some instantiate it)
template <int N>
__device__ __forceinline__ float* head_rows_lds() {
  __shared__ __align__(16) float rows[N];
  return rows;
}

// What this block and wave do in the step
struct Role {
  int blk, w, lane, xcd, slot, vb;
  int nh, qc, qcw;      // heads of the XCD; qkv columns of the block and of a data wave
  int hj, kb, ah;       // attention: local head, key block, global head
  int n0, pos0;         // first step of the launch and its position
  int nh0;              // ids in the window before the launch's first step (sampled kernel)
  int pos, nk;          // the current token's position and key count
  int nkb;              // key blocks per head (attention blocks) for every token of the launch
  int key0;             // this data wave's first key
  bool wave_keys;
  unsigned tag0;        // tag base of the launch's first token
  int trace_it;         // token/layer iteration the trace marks (token 5, layer 1 when there is one)
  uint2* xl;            // this XCD's local pairs
  int xl0;              // same, as a pair index into p.xl
};

// Control wave: collects every hand-off.  attn: this block computes attention
// (it gathers its head's q/k/v and publishes the block's partial).  After a
// failed wait (sh.fail) it skips the remaining waits and stores but meets
// every barrier: the loops have no early exit, which keeps the compiler's
// load-wait bookkeeping exact across iterations.
// Control wave, head of a token: waits until the NR argmax records (value, index,
// tag, 0) at byte offset `off` all carry `tag`, then returns their (first)
// maximum in best / bi.
template <int NR, typename B>
__device__ bool gather_argmax(const B& nc, int off, unsigned tag, float& best, int& bi, int* err, int code) {
  constexpr int R = (NR + 63) / 64;  // records per lane
  const int lane = threadIdx.x & 63;
  long it = 0;
  for (;;) {
    reload_fence();
    uint4 a[R];
#pragma unroll
    for (int i = 0; i < R; i++) a[i] = nc.load4(off + 16 * min(i * 64 + lane, NR - 1));
    bool ok = true;
    best = -INFINITY;
    bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < R; i++) {
      if (i * 64 + lane < NR) {
        ok &= a[i].z == tag;
        argmax_merge(best, bi, __uint_as_float(a[i].x), (int)a[i].y);
      }
    }
    if (__all(ok)) break;
    if ((++it & 63) == 0 && (it > SPIN_LIMIT || err_set(err))) {
      if (lane == 0 && it > SPIN_LIMIT) raise_err(err, code);
      return false;
    }
  }
  wave_argmax(best, bi);
  return true;
}

// ---- the sampled kernel's sampler (one wave) ----------------------------------------
// Sampler.Sample with top-k (Sampler.cs:29-69) after ApplyRepetitionControls
// (:111-165), spread over the launch's blocks: each block adjusts its own rows and
// publishes them with its two largest values; each XCD's first block selects the
// XCD's k largest, sorted; every block merges the 8 sorted XCD lists into the k
// largest and draws.  The arithmetic is the reference's, in its order: penalty
// (x < 0 ? x * p : x / p), division by T, the threshold = the k-th largest value
// with ties kept, exp(p - max) summed in index order, u = (float)U * sum, the first
// index whose running sum exceeds u.

__device__ __forceinline__ float wave_fmax(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ float wave_fmin(float v) { return -wave_max_dpp(-v); }
// OR over the wave through the same DPP steps as wave_sum_dpp, in every lane
__device__ __forceinline__ uint32_t wave_or_dpp(uint32_t v) {
  int x = (int)v;
  x |= __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x |= __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  return (uint32_t)__builtin_amdgcn_readlane(x, 63);
}
__device__ __forceinline__ uint64_t wave_or64(uint64_t v) {
  return ((uint64_t)wave_or_dpp((uint32_t)(v >> 32)) << 32) | wave_or_dpp((uint32_t)v);
}
// inclusive prefix sum over the wave in lane order: shifts within rows of 16, then
// the last lane of row 0 (2) added to row 1 (3), of row 1 to rows 2 and 3
__device__ __forceinline__ int wave_scan_incl(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
  return x;
}

// ---- one-wave sorting networks: 64 entries, one per lane ----------------------
// (used by the sampled kernel only; marks what the greedy
// kernel's translation unit, decode_fast.hip itself, leaves out)
// The value of lane ^ J: DPP for J < 16 (quad permutes, row shifts into alternate
// 4-lane banks, row rotate by 8); for 16 and 32 the row-swap permutes, which hand
// a lane with bit J clear its partner in the second result, a lane with it set in
// the first (l: the lane index).
template <int J>
__device__ __forceinline__ int lane_xor(int v, int l) {
  if constexpr (J == 1) {
    return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4) {
    const int a = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0x5, false);  // row_shl:4 into banks 0 and 2
    return __builtin_amdgcn_update_dpp(a, v, 0x114, 0xF, 0xA, false);        // row_shr:4 into banks 1 and 3
  } else if constexpr (J == 8) {
    return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (J == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int)((l & 16) ? s[0] : s[1]);
  } else {
    static_assert(J == 32, "distance");
    const auto s = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)((l & 32) ? s[0] : s[1]);
  }
}
// the value of lane 63 - l: mirror within rows of 16 (l ^ 15), then l ^ 16, l ^ 32
__device__ __forceinline__ int lane_rev(int v, int l) {
  const int m = __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);  // row_mirror
  return lane_xor<32>(lane_xor<16>(m, l), l);
}
// The lane index as a value the compiler cannot move out of the token loop: the
// networks' per-lane masks are then recomputed where they are used instead of
// being held (in scalar registers) for the whole kernel.
__device__ __forceinline__ int opaque_lane() {
  int l;
  asm volatile("v_and_b32 %0, 63, %1" : "=v"(l) : "v"((int)threadIdx.x));
  return l;
}
// 1 << 31 in the lanes where bit A of the lane index differs from bit B (B < 0: bit A set)
__device__ __forceinline__ unsigned flip_bits(int l, int A, int B) {
  const unsigned x = B < 0 ? (unsigned)l >> A : ((unsigned)l >> A) ^ ((unsigned)l >> B);
  return (x & 1u) << 31;
}
// Compare-exchange with lane ^ J.  A lane keeps the larger value, or the smaller
// where flip has the sign bit (comparing values with flipped signs reverses the
// order); its payload moves with it.  A partner is taken only when strictly
// better, so equal values stay put and no entry is lost or doubled.
// (PAY false: the value alone, r untouched)
template <int J, bool PAY = true>
__device__ __forceinline__ void cx_val(float& v, int& r, unsigned flip, int l) {
  const float pv = __int_as_float(lane_xor<J>(__float_as_int(v), l));
  const bool take = __uint_as_float(__float_as_uint(pv) ^ flip) > __uint_as_float(__float_as_uint(v) ^ flip);
  v = take ? pv : v;
  if constexpr (PAY) {
    const int pr = lane_xor<J>(r, l);
    r = take ? pr : r;
  }
}
// the same for a non-negative int key kept smallest-first unless flipped (flip: 0 or ~0)
template <int J>
__device__ __forceinline__ void cx_key(int& k, float& v, unsigned flip, int l) {
  const int pk = lane_xor<J>(k, l);
  const float pv = __int_as_float(lane_xor<J>(__float_as_int(v), l));
  const bool take = ((unsigned)pk ^ flip) < ((unsigned)k ^ flip);
  k = take ? pk : k;
  v = take ? pv : v;
}
// bitonic sort of the wave's 64 (value, row) entries, largest value in lane 0:
// at stage (block K, distance J) a lane keeps the larger value when bits J and K
// of its index agree (PAY false: the values alone)
template <bool PAY = true>
__device__ __forceinline__ void sort64_desc(float& v, int& r) {
  const int l = opaque_lane();
#define FH_CX(KB, JB) cx_val<(1 << JB), PAY>(v, r, flip_bits(l, JB, KB), l)
  FH_CX(1, 0);
  FH_CX(2, 1); FH_CX(2, 0);
  FH_CX(3, 2); FH_CX(3, 1); FH_CX(3, 0);
  FH_CX(4, 3); FH_CX(4, 2); FH_CX(4, 1); FH_CX(4, 0);
  FH_CX(5, 4); FH_CX(5, 3); FH_CX(5, 2); FH_CX(5, 1); FH_CX(5, 0);
  FH_CX(-1, 5); FH_CX(-1, 4); FH_CX(-1, 3); FH_CX(-1, 2); FH_CX(-1, 1); FH_CX(-1, 0);
#undef FH_CX
}
// bitonic sort of (key, value) entries by key: W 32 sorts lanes 0..31 smallest
// key first (and 32..63 largest first), W 64 the whole wave smallest key first
template <int W>
__device__ __forceinline__ void sort_key_asc(int& k, float& v) {
  static_assert(W == 32 || W == 64, "width");
  const int l = opaque_lane();
#define FH_CX(KB, JB) cx_key<(1 << JB)>(k, v, (unsigned)((int)flip_bits(l, JB, KB) >> 31), l)
  FH_CX(1, 0);
  FH_CX(2, 1); FH_CX(2, 0);
  FH_CX(3, 2); FH_CX(3, 1); FH_CX(3, 0);
  FH_CX(4, 3); FH_CX(4, 2); FH_CX(4, 1); FH_CX(4, 0);
  FH_CX(5, 4); FH_CX(5, 3); FH_CX(5, 2); FH_CX(5, 1); FH_CX(5, 0);
  if constexpr (W == 64) {
    FH_CX(-1, 5); FH_CX(-1, 4); FH_CX(-1, 3); FH_CX(-1, 2); FH_CX(-1, 1); FH_CX(-1, 0);
  }
#undef FH_CX
}
// The 64 largest of two lists sorted largest-first (a in v/r, b in bv/br), sorted
// largest-first into v/r: a[i] against b[63 - i] keeps the larger of each pair (a
// bitonic sequence holding the 64 largest), then six half-cleaners sort it.
__device__ __forceinline__ void merge64_desc(float& v, int& r, float bv, int br) {
  const int l = opaque_lane();
  const float rv = __int_as_float(lane_rev(__float_as_int(bv), l));
  const int rr = lane_rev(br, l);
  const bool take = rv > v;
  v = take ? rv : v;
  r = take ? rr : r;
  cx_val<32>(v, r, flip_bits(l, 5, -1), l);
  cx_val<16>(v, r, flip_bits(l, 4, -1), l);
  cx_val<8>(v, r, flip_bits(l, 3, -1), l);
  cx_val<4>(v, r, flip_bits(l, 2, -1), l);
  cx_val<2>(v, r, flip_bits(l, 1, -1), l);
  cx_val<1>(v, r, flip_bits(l, 0, -1), l);
}
// the value of lane l ^ 31 (each 32-lane half reversed): row mirror, then l ^ 16
__device__ __forceinline__ int lane_rev32(int v, int l) {
  const int m = __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);  // row_mirror
  return lane_xor<16>(m, l);
}
// Lists of 32 entries, one per 32-lane half, each sorted largest-first.  Each half
// of v/r becomes the 32 largest of its own list and the list in the same half of
// bv/br (FOLD false), or of its list and the other half's (FOLD true, bv/br =
// v/r), sorted largest-first: entry i against the other list's entry 31 - i keeps
// the larger of each pair (a bitonic sequence holding the 32 largest), then five
// half-cleaners within the half sort it.
template <bool FOLD>
__device__ __forceinline__ void merge32_desc(float& v, int& r, float bv, int br) {
  const int l = opaque_lane();
  const float rv = __int_as_float(FOLD ? lane_rev(__float_as_int(bv), l) : lane_rev32(__float_as_int(bv), l));
  const int rr = FOLD ? lane_rev(br, l) : lane_rev32(br, l);
  const bool take = rv > v;
  v = take ? rv : v;
  r = take ? rr : r;
  cx_val<16>(v, r, flip_bits(l, 4, -1), l);
  cx_val<8>(v, r, flip_bits(l, 3, -1), l);
  cx_val<4>(v, r, flip_bits(l, 2, -1), l);
  cx_val<2>(v, r, flip_bits(l, 1, -1), l);
  cx_val<1>(v, r, flip_bits(l, 0, -1), l);
}
// Running sums in lane order with the rounding of a sequential loop: lane j gets
// (((v_0 + v_1) + v_2) + ... ) + v_j for j < W.  Each step shifts the sums one
// lane up the whole wave (DPP wave_shr:1; lane 0 receives 0) and adds the lane's
// own value, so after step s lanes 0..s hold their final sums.  Exact for
// non-negative values (lanes past the entries should hold 0).
template <int W>
__device__ __forceinline__ float seq_prefix(float v) {
  float a = v;
#pragma unroll
  for (int s = 1; s < W; s++)
    a = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x138, 0xF, 0xF, true));
  return a;
}

// The k-th largest (duplicates counted) of the values v[j] of every lane (absent
// entries are -inf and are never counted; at least k are present), and, in cv/cr
// (LDS, cap entries), the entries >= that value with their rows, *n of them.
// A window [lo, M] below the maximum M that holds at least k values is narrowed:
// first the steps M - 2^q / 8 (q < 8), then 8 halvings between the last step that
// held fewer than k and the first that held k (counts by ballot), so it keeps
// little more than k candidates; the k-th largest is the smallest candidate with
// fewer than k candidates above it.
template <int N>
__device__ float wave_topk(const float (&v)[N], const int (&row)[N], int k, float* cv, int* cr, int cap, int* n) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < N; j++) m = fmaxf(m, v[j]);
  const float M = wave_fmax(m);
  auto count_ge = [&](float b) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < N; j++) c += __popcll(__ballot(v[j] >= b));
    return c;
  };
  float lo = M;
  if (count_ge(M) < k) {
    float hi = M;
    lo = -FLT_MAX;
    for (int q = 0; q < 8; q++) {
      const float b = M - (float)(1 << q) * 0.125f;
      if (count_ge(b) >= k) {
        lo = b;
        break;
      }
      hi = b;
    }
    if (lo != -FLT_MAX) {
      for (int h = 0; h < 8; h++) {
        const float mid = lo + (hi - lo) * 0.5f;
        if (count_ge(mid) >= k)
          lo = mid;
        else
          hi = mid;
      }
    }
  }
  // the window's entries into LDS (order of lanes, then registers)
  int w = 0;
#pragma unroll
  for (int j = 0; j < N; j++) {
    const bool in = v[j] >= lo;
    const uint64_t bal = __ballot(in);
    const int pos = w + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
    if (in && pos < cap) {
      cv[pos] = v[j];
      cr[pos] = row[j];
    }
    w += __popcll(bal);
  }
  w = min(w, cap);
  wave_lds_sync();
  // rank in the window: the threshold is the smallest entry with fewer than k above it
  float cand = INFINITY;
  if (w <= 64) {
    const float e = lane < w ? cv[lane] : -INFINITY;
    int above = 0;
    for (int j = 0; j < w; j++) above += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j)) > e ? 1 : 0;
    if (lane < w && above < k) cand = e;
  } else {  // many equal or dense values near the k-th largest
    for (int i = lane; i < w; i += 64) {
      const float e = cv[i];
      int above = 0;
      for (int j = 0; j < w; j++) above += cv[j] > e ? 1 : 0;
      if (above < k) cand = fminf(cand, e);
    }
  }
  const float thr = wave_fmin(cand);
  // keep the entries >= thr (their count is k unless values tie at thr)
  wave_lds_sync();
  int c = 0;
  for (int base = 0; base < w; base += 64) {
    const int i = base + lane;
    const float e = i < w ? cv[i] : -INFINITY;
    const int r = i < w ? cr[i] : 0;
    const bool keep = e >= thr;
    const uint64_t bal = __ballot(keep);
    const int pos = c + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
    wave_lds_sync();  // every lane has read entry i before the kept ones are moved down
    if (keep) {
      cv[pos] = e;
      cr[pos] = r;
    }
    c += __popcll(bal);
  }
  wave_lds_sync();
  *n = c;
  return thr;
}

// ApplyRepetitionControls' masks for rows [row0, row0 + R) of one block over the
// window's T ids hs[0..T): pm the rows the penalty scales (each distinct id once,
// Sampler.cs:117-127), bm the rows the n-gram rule bans (:129-154).  Every lane
// gets both masks.
__device__ void sampler_masks(const KParams& p, const int* hs, int T, int row0, int R, uint64_t& pm, uint64_t& bm) {
  const int lane = threadIdx.x & 63;
  pm = 0;
  bm = 0;
  if (p.penalty != 1.f || p.ngram == 1) {
    uint64_t m = 0;
    for (int i = lane; i < T; i += 64) {
      const int d = hs[i] - row0;
      if ((unsigned)d < (unsigned)R) m |= 1ull << d;
    }
    m = wave_or64(m);
    if (p.penalty != 1.f) pm = m;
    if (p.ngram == 1) bm = m;
  }
  if (p.ngram > 1 && T >= p.ngram - 1) {
    const int pre = p.ngram - 1, suf = T - pre;
    uint64_t m = 0;
    for (int s0 = lane; s0 + p.ngram <= T; s0 += 64) {
      bool match = true;
      for (int j = 0; j < pre; j++)
        if (hs[s0 + j] != hs[suf + j]) {
          match = false;
          break;
        }
      const int d = hs[s0 + pre] - row0;
      if (match && (unsigned)d < (unsigned)R) m |= 1ull << d;
    }
    bm = wave_or64(m);
  }
}

// The 8 published XCD lists (k entries each, largest first, tag `tag`), NR per
// lane: NR 8 puts entry l of list i in lane l of g[i]; NR 4 puts two lists in a
// register, entry l % 32 of list 2 i + l / 32 in lane l (k < 32).  Entries past k
// are -inf (row INT_MAX); lanes past k re-read entry k - 1 and check it too.
template <int NR>
__device__ __forceinline__ bool gather_slists(const NcBuf& nc, const KParams& p, int K, unsigned tag, float* g,
                                              int* gr) {
  static_assert(NR == NX || NR == NX / 2, "lists per register");
  const int lane = threadIdx.x & 63;
  const int e = NR == NX ? lane : (lane & 31);
  const int ec = min(e, K - 1);
  long it = 0;
  for (;;) {
    reload_fence();
    uint4 a[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const int list = NR == NX ? i : 2 * i + (lane >> 5);
      a[i] = nc.load4(p.off_slist + (list * 64 + ec) * 16);
    }
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NR; i++) ok &= (a[i].z == tag) & (a[i].w == tag);
    if (__all(ok)) {
#pragma unroll
      for (int i = 0; i < NR; i++) {
        g[i] = e < K ? __uint_as_float(a[i].x) : -INFINITY;
        gr[i] = e < K ? (int)a[i].y : 0x7fffffff;
      }
      return true;
    }
    if ((++it & 63) == 0 && (it > SPIN_LIMIT || err_set(p.err))) {
      if (lane == 0 && it > SPIN_LIMIT) raise_err(p.err, err_code(W_SLIST, 0));
      return false;
    }
  }
}

// Control wave, sampled kernel, head of token t: this block's rows adjusted and
// published with their two largest values; the XCD's first block selects and
// publishes the XCD's k largest, largest first; with need_id, every block merges
// the 8 XCD lists into the k largest and draws the id.  The host only runs this
// kernel where no row can be all-banned and every XCD has more than k unbanned
// rows.  Returns false after a failed wait or check (the error word is set).
template <int D, int H>
__device__ bool sampler_draw(const KParams& p, const Lds<D, H>& sh, SampLds<true>& sl, const Role& r, unsigned tH,
                             uint64_t pm, uint64_t bm, bool need_id, double u01, int& id) {
#pragma clang fp contract(off)
  using XL = Xl<D, H>;
  const int lane = threadIdx.x & 63;
  const int R = p.Vp / NB, K = p.top_k;
  const int row = r.vb * R + lane;
  const bool valid = lane < R && row < p.V;
  float x = valid ? sh.hval[lane] : 0.f;
  if (__any(valid && !(fabsf(x) <= FLT_MAX))) {  // a NaN or infinite logit: the per-step sampler handles it
    if (lane == 0) raise_err(p.err, err_code(W_SAMPLE, 0));
    return false;
  }
  if ((pm >> lane) & 1ull) x = x < 0.f ? x * p.penalty : x / p.penalty;
  const float pv = (valid && !((bm >> lane) & 1ull)) ? x / p.temperature : -INFINITY;  // banned: -inf
  const unsigned tS1 = tH + 1, tS2 = tH + 2;
  {
    // this block's two largest values (equal when the largest repeats)
    const float m1 = wave_fmax(pv);
    const int l1 = (int)__builtin_ctzll(__ballot(pv == m1));
    const float m2 = wave_fmax(lane == l1 ? -INFINITY : pv);
    put_pair(r.xl + XL::SAMP + r.slot * 64 + lane, pv, tS1);
    if (lane < 2) put_pair(r.xl + XL::SAMPT + r.slot * 2 + lane, lane == 0 ? m1 : m2, tS1);
  }
  char* ucb = reinterpret_cast<char*>(p.uc);
  if (r.slot == 0) {
    // the XCD's k largest of its 32 x 64 values: pair q of the XCD's area is slot
    // q / 64, lane q % 64, i.e. row (8 (q / 64) + xcd) R + q % 64; this lane's
    // 16-byte loads hold pairs 128 i + 2 lane and + 1, its 8-byte load the
    // lane-th of the 64 block maxima
    const LcBuf ncl(p.xl, p.xl_bytes);
    float v[SLOTS];
    int rw[SLOTS];
    float t2;
    {
      long it = 0;
      for (;;) {
        reload_fence();
        uint4 a[SLOTS / 2];
#pragma unroll
        for (int i = 0; i < SLOTS / 2; i++) a[i] = ncl.load4((r.xl0 + XL::SAMP + 128 * i + 2 * lane) * 8);
        const uint2 b = ncl.load2((r.xl0 + XL::SAMPT + lane) * 8);
        bool ok = b.y == tS1;
#pragma unroll
        for (int i = 0; i < SLOTS / 2; i++) {
          ok &= (a[i].y == tS1) & (a[i].w == tS1);
          v[2 * i] = __uint_as_float(a[i].x);
          v[2 * i + 1] = __uint_as_float(a[i].z);
        }
        t2 = __uint_as_float(b.x);
        if (__all(ok)) break;
        if ((++it & 63) == 0 && (it > SPIN_LIMIT || err_set(p.err))) {
          if (lane == 0 && it > SPIN_LIMIT) raise_err(p.err, err_code(W_SKEYS, 0));
          return false;
        }
      }
#pragma unroll
      for (int i = 0; i < SLOTS / 2; i++)
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const int q = 128 * i + 2 * lane + e;
          rw[2 * i + e] = ((q >> 6) * NX + r.xcd) * R + (q & 63);
        }
    }
    // The k-th largest of the 64 block maxima bounds the XCD's k-th largest from
    // below (they are k of the XCD's values), so the XCD's k largest are among the
    // values >= it; when those fit one per lane they are sorted directly, else
    // the threshold search narrows all 2048.
    int dummy = 0;
    sort64_desc<false>(t2, dummy);
    const float tau = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t2), K - 1));
    int w = 0;
    if (tau != -INFINITY) {
      // each lane's candidates go to consecutive places after those of the lanes
      // before it (a wave prefix sum of the counts); the others to a spare place
      int c = 0;
#pragma unroll
      for (int j = 0; j < SLOTS; j++) c += v[j] >= tau ? 1 : 0;
      const int incl = wave_scan_incl(c);
      w = __builtin_amdgcn_readlane(incl, 63);
      if (w <= 64) {
        int pos = incl - c;
#pragma unroll
        for (int j = 0; j < SLOTS; j++) {
          const bool in = v[j] >= tau;
          const int at = in ? pos : 64 + lane;
          sl.cv[at] = v[j];
          sl.cr[at] = rw[j];
          pos += in ? 1 : 0;
        }
      }
    }
    if (tau == -INFINITY || w > 64) {
      int cnt = 0;
      wave_topk<SLOTS>(v, rw, K, sl.cv, sl.cr, SLOTS * 64, &cnt);
      if (cnt != K) {  // values tie at the XCD's k-th largest
        if (lane == 0) raise_err(p.err, err_code(W_SAMPLE, 0));
        return false;
      }
      w = K;
    }
    wave_lds_sync();
    float e = lane < w ? sl.cv[lane] : -INFINITY;
    int er = lane < w ? sl.cr[lane] : 0x7fffffff;
    sort64_desc(e, er);
    // values tie at the XCD's k-th largest (K <= 63, so lane K exists)
    if (__builtin_amdgcn_readlane(__float_as_int(e), K) == __builtin_amdgcn_readlane(__float_as_int(e), K - 1)) {
      if (lane == 0) raise_err(p.err, err_code(W_SAMPLE, 0));
      return false;
    }
    wave_lds_sync();  // every lane has read its candidate before the next token's writes
    if (lane < K)
      *reinterpret_cast<uint4*>(ucb + p.off_slist + (r.xcd * 64 + lane) * 16) =
          make_uint4(__float_as_uint(e), (unsigned)er, tS2, tS2);
  }
  if (!need_id) return true;
  // the k + 1 largest of the 8 lists, largest first, in lanes 0..k of g0/r0
  const NcBuf ncu(p.uc, p.uc_bytes);
  float g0;
  int r0;
  if (K < 32) {
    // two lists per register: three merges of list pairs, then the two halves
    float g[NX / 2];
    int gr[NX / 2];
    if (!gather_slists<NX / 2>(ncu, p, K, tS2, g, gr)) return false;
    merge32_desc<false>(g[0], gr[0], g[1], gr[1]);
    merge32_desc<false>(g[2], gr[2], g[3], gr[3]);
    merge32_desc<false>(g[0], gr[0], g[2], gr[2]);
    merge32_desc<true>(g[0], gr[0], g[0], gr[0]);
    g0 = g[0];
    r0 = gr[0];
  } else {
    // a tree of pairwise merges
    float g[NX];
    int gr[NX];
    if (!gather_slists<NX>(ncu, p, K, tS2, g, gr)) return false;
    merge64_desc(g[0], gr[0], g[1], gr[1]);
    merge64_desc(g[2], gr[2], g[3], gr[3]);
    merge64_desc(g[4], gr[4], g[5], gr[5]);
    merge64_desc(g[6], gr[6], g[7], gr[7]);
    merge64_desc(g[0], gr[0], g[2], gr[2]);
    merge64_desc(g[4], gr[4], g[6], gr[6]);
    merge64_desc(g[0], gr[0], g[4], gr[4]);
    g0 = g[0];
    r0 = gr[0];
  }
  if (__builtin_amdgcn_readlane(__float_as_int(g0), K) == __builtin_amdgcn_readlane(__float_as_int(g0), K - 1)) {
    // values tie at the k-th largest: the reference keeps them all
    if (lane == 0) raise_err(p.err, err_code(W_SAMPLE, 0));
    return false;
  }
  // the kept values in row order (Sampler.cs:52-68 walks the rows in index order:
  // the exps summed one by one, the first row past u)
  const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g0), 0));
  int rs = lane < K ? r0 : 0x7fffffff;
  float ps = lane < K ? g0 : 0.f;
  if (K < 32)
    sort_key_asc<32>(rs, ps);
  else
    sort_key_asc<64>(rs, ps);
  const float ex = lane < K ? expf(ps - mx) : 0.f;
  const float pre = K < 32 ? seq_prefix<32>(ex) : seq_prefix<64>(ex);  // the running sum after row j
  const float acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pre), K - 1));
  const float u = (float)u01 * acc;
  const uint64_t hit = __ballot(lane < K && u < pre);
  id = hit ? __builtin_amdgcn_readlane(rs, (int)__builtin_ctzll(hit)) : p.V - 1;
  return true;
}

template <int D, int H, bool SAMPLED>
__device__ __forceinline__ void ctrl_loop(const KParams& p, Lds<D, H>& sh, SampLds<SAMPLED>& sl, const Role& r,
                                          const bool attn) {
  using S = Shape<D, H>;
  using U = Xu<D>;
  using XL = Xl<D, H>;
  constexpr int RSC = S::RSC;
  const int lane = r.lane;
  const NcBuf ncu(p.uc, p.uc_bytes);
  const LcBuf ncl(p.xl, p.xl_bytes);
  bool dead = false;
  unsigned long long tfirst = 0, tdone = 0, tcomb = 0;
  auto fail = [&]() {
    dead = true;
    sh.fail = 1;
  };
#define TM(i) \
  if (it == r.trace_it) trace_mark(p.trace, (i))
  // tokens t < nsteps, layers l < L: one flat loop
  const int total = p.nsteps * p.L;
  for (int it = 0; it < total; it++) {
    const int t = it / p.L, l = it - t * p.L;
    const unsigned tbase = r.tag0 + (unsigned)t * TAGS;
    const unsigned tb = tbase + PH * l;
    const unsigned tA = tb, tP = tb + 1, tC = tb + 3, tC2 = tb + 4, tD = tb + 5, tE = tb + 6, tE2 = tb + 7;
    // ---- A: x of this layer (every XCD's copy) ----
    for (int i = lane; i < S::BT; i += 64) sh.bias_s[l & 1][i] = p.btab[((size_t)l * NB + r.vb) * S::BT + i];
    if (l > 0 && !dead && !gather<D>(ncl, r.xl0 + XL::X, tb - PH + 7, sh.xres, p.err, err_code(W_X, l), D))
      fail();
    __syncthreads();
    TM(0);
    if (it == r.trace_it + 1) trace_mark(p.trace, 9);
    // Every phase whose data waves publish and then request tiles has a
    // second barrier between the two, so that no published value queues
    // behind the tile loads of another wave of this CU.
    __syncthreads();
    // ---- B: attention of this block's keys; publish the block's partial ----
    if (attn) {
      if (!dead && !gather<192>(ncl, r.xl0 + XL::QKV + r.hj * 192, tA, sh.qkvs, p.err, err_code(W_QKV, l), 192,
                                nullptr))
        fail();
      __syncthreads();
      TM(1);
      __syncthreads();  // the data waves' partials are in wm / wl / wo
      float M = -INFINITY;
#pragma unroll
      for (int i = 0; i < NDW; i++) M = fmaxf(M, sh.wm[i]);
      float Ls = 0.f, o = 0.f;
#pragma unroll
      for (int i = 0; i < NDW; i++) {
        const float f = (sh.wm[i] == -INFINITY) ? 0.f : __expf(sh.wm[i] - M);
        Ls += sh.wl[i] * f;
        o += sh.wo[i][lane] * f;
      }
      if (!dead) {
        uint2* pp = r.xl + XL::PARTS + (r.hj * S::SPH + r.kb) * PART;
        put_pair(pp + lane, o, tP);
        if (lane < PART - 64) put_pair(pp + 64 + lane, lane == 0 ? M : (lane == 1 ? Ls : 0.f), tP);
      }
      TM(2);
      __syncthreads();  // the partial is published before the data waves request K/V
    }
    // ---- C: o of the XCD's heads from every key block's partial ----
    if (!dead &&
        !gather_parts<D, H>(ncl, r.xl0 + XL::PARTS, r.nh, r.nkb, tP, sh.parts, p.err, err_code(W_PART, l), nullptr,
                            (it == r.trace_it && p.trace) ? &tfirst : nullptr))
      fail();
    if (it == r.trace_it && p.trace) tdone = wall_clock64();
    if (!dead) {
      // DPP row j (lanes 16j .. 16j+15) holds head j's partials, lane 16j + c
      // partial c: its weight exp(m - M_j) goes to sh.pw, the row sums l * weight;
      // then lane d sums o[d] over the head's partials (reads issued together,
      // partials past nkb masked)
      static_assert(S::SPH == 16 && S::HPX <= 4, "one DPP row of partials per head");
      wave_lds_sync();
      const int jt = lane >> 4, ct = lane & 15;
      const bool has = jt < r.nh && ct < r.nkb;
      const float mt = has ? sh.parts[(jt * S::SPH + ct) * PART + 64] : -INFINITY;
      const float lt = has ? sh.parts[(jt * S::SPH + ct) * PART + 65] : 0.f;
      const float Mj = row16_max(mt);
      const float f = has ? __expf(mt - Mj) : 0.f;
      const float Lrow = row16_sum(lt * f);
      sh.pw[lane] = f;
      if (ct == 0) sh.pl[jt] = Lrow;
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < S::HPX; j++) {
        if (j < r.nh) {
          const float* pj = sh.parts + j * S::SPH * PART;
          float o = 0.f;
#pragma unroll
          for (int c = 0; c < S::SPH; c++) {
            const float t = pj[c * PART + lane] * sh.pw[j * 16 + c];
            o += c < r.nkb ? t : 0.f;
          }
          sh.os[j * 64 + lane] = o * __frcp_rn(sh.pl[j]);
        }
      }
    }
    if (it == r.trace_it && p.trace) tcomb = wall_clock64();
    __syncthreads();
    TM(3);
    __syncthreads();
    // ---- x2 = x + attn.proj(o) + b: this slot's columns from the 8 XCD partials ----
    if (!dead && !gather_slices<D, RSC>(ncu, U::PX2, r.slot, tC, sh.rsv, p.err, err_code(W_PX2, l))) fail();
    TM(7);
    wave_lds_sync();
    if (!dead && lane < RSC) {
      float sum = 0.f;
#pragma unroll
      for (int x = 0; x < NX; x++) sum += sh.rsv[x * RSC + lane];
      const int col = r.slot * RSC + lane;
      put_pair(r.xl + XL::X2 + col, (sum + sh.bias_s[l & 1][S::B_P + lane]) + sh.xres[col], tC2);
    }
    if (!dead && !gather<D>(ncl, r.xl0 + XL::X2, tC2, sh.x2s, p.err, err_code(W_X2, l), D)) fail();
    __syncthreads();
    TM(4);
    __syncthreads();
    // ---- D: the XCD's h slice ----
    if (!dead && !gather<S::HX>(ncl, r.xl0 + XL::HH, tD, sh.hs, p.err, err_code(W_H, l), S::HX)) fail();
    __syncthreads();
    TM(5);
    __syncthreads();
    // ---- E: x = x2 + mlp.proj(h) + b: this slot's columns from the 8 XCD partials ----
    if (!dead && !gather_slices<D, RSC>(ncu, U::PX, r.slot, tE, sh.rsv, p.err, err_code(W_PX, l))) fail();
    TM(8);
    wave_lds_sync();
    if (!dead && lane < RSC) {
      float sum = 0.f;
#pragma unroll
      for (int x = 0; x < NX; x++) sum += sh.rsv[x * RSC + lane];
      const int col = r.slot * RSC + lane;
      put_pair(r.xl + XL::X + col, (sum + sh.bias_s[l & 1][S::B_M + lane]) + sh.x2s[col], tE2);
    }
    TM(6);
    if (it == r.trace_it && p.trace && lane == 0) {
      p.trace[r.blk * TRACE_PER + 14] = tfirst;
      p.trace[r.blk * TRACE_PER + 15] = tcomb;
      p.trace[r.blk * TRACE_PER + 13] = tdone;
    }
    if (l == p.L - 1) {
      // ---- head of token t: the final x, this block's logits, every block's argmax ----
      if (!dead && !gather<D>(ncl, r.xl0 + XL::X, tb + 7, sh.xres, p.err, err_code(W_XF, 0))) fail();
      const bool thead = it == r.trace_it + p.L - 2;  // the head of the traced token
      if (thead) trace_mark(p.trace, 16);
      __syncthreads();  // x is in xres: the data waves compute this block's logits
      uint64_t pmask = 0, bmask = 0;
      double u01 = 0.0;
      if constexpr (SAMPLED) {
        u01 = p.uniforms[r.n0 + t];  // this step's NextDouble, requested before the waits
        // ApplyRepetitionControls' penalty and n-gram bans for this block's rows
        // (Sampler.cs:117-154) over the window's ids, while the data waves compute
        if (!dead) sampler_masks(p, sl.hist, r.nh0 + t, r.vb * (p.Vp / NB), p.Vp / NB, pmask, bmask);
      }
      __syncthreads();  // hval holds them
      const unsigned tH = tbase + PH * p.L;
      if constexpr (SAMPLED) {
        const bool next = t + 1 < p.nsteps;
        // the next position's embedding row does not depend on the draw: fetched first
        float4 pe4[S::KC];
        if (next) {
          const float* pe = p.pos + (size_t)(r.pos0 + t + 1) * D;
#pragma unroll
          for (int c = 0; c < S::KC; c++) pe4[c] = *reinterpret_cast<const float4*>(pe + c * 256 + lane * 4);
        }
        int bi = 0;
        if (!dead && !sampler_draw<D, H>(p, sh, sl, r, tH, pmask, bmask, next || r.blk == 0, u01, bi)) fail();
        if (!dead && (next || r.blk == 0)) {
          const int n = r.n0 + t;
          if (r.blk == 0 && lane == 0) {
            p.tokens_out[p.src.tok_off + 1 + n] = bi;  // window position prompt_len + n
            if (n < p.max_new) p.out_ids[n] = bi;
            if (p.eos >= 0 && bi == p.eos && p.out_counts[0] < 0) p.out_counts[0] = n + 1;
            *p.step_out = n + 1;
          }
          if (next) {
            if (lane == 0) sl.hist[r.nh0 + t] = bi;  // the window grows by the drawn id
            const float* te = p.tok + (size_t)bi * D;
            float4 a[S::KC];
#pragma unroll
            for (int c = 0; c < S::KC; c++) a[c] = *reinterpret_cast<const float4*>(te + c * 256 + lane * 4);
#pragma unroll
            for (int c = 0; c < S::KC; c++) {
              const float4 b = pe4[c];
              *reinterpret_cast<float4*>(sh.xres + c * 256 + lane * 4) =
                  make_float4(a[c].x + b.x, a[c].y + b.y, a[c].z + b.z, a[c].w + b.w);
            }
          }
        }
      } else if (!dead) {
        // this block's logits (for a host-side sampler) and its argmax record
        const int R = p.Vp / NB;
        float best = -INFINITY;
        int bi = 0x7fffffff;
        if (lane < R && r.blk * R + lane < p.V) {
          const float sv = sh.hval[lane];
          const int v = r.blk * R + lane;
          if (!p.greedy) p.logits[v] = sv;
          best = sv;
          bi = v;
        }
        wave_argmax(best, bi);
        if (lane == 0)
          *reinterpret_cast<uint4*>(reinterpret_cast<char*>(p.uc) + p.off_amax + 16 * r.blk) =
              make_uint4(__float_as_uint(best), (unsigned)bi, tH, 0u);
      }
      if constexpr (!SAMPLED) {
      if (thead) trace_mark(p.trace, 17);
      const bool next = t + 1 < p.nsteps;
      // Every block reduces the 256 uncached records itself (one hop; a two-level
      // reduction through each XCD's L2 measured slower): every block needs the
      // token for the next step; block 0 also records it, and its collection
      // proves all blocks read this launch's counter.
      if (!dead && (next || r.blk == 0)) {
        float best;
        int bi;
        if (!gather_argmax<NB>(ncu, p.off_amax, tH, best, bi, p.err, err_code(W_AMAX, 0))) {
          fail();
        } else if ((unsigned)bi >= (unsigned)p.V) {  // no finite logit: no id to record or feed back
          if (lane == 0) raise_err(p.err, err_code(W_TOK, 0));
          fail();
        } else {
          const int n = r.n0 + t;
          if (r.blk == 0 && lane == 0 && p.greedy) {
            p.tokens_out[p.src.tok_off + 1 + n] = bi;  // window position prompt_len + n
            if (n < p.max_new) p.out_ids[n] = bi;
            if (p.eos >= 0 && bi == p.eos && p.out_counts[0] < 0) p.out_counts[0] = n + 1;
            *p.step_out = n + 1;
          }
          if (thead) trace_mark(p.trace, 18);
          if (next) {
            // x of the next token = tok_emb[id] + pos_emb[pos + 1]
            const int id = bi;
            const float* te = p.tok + (size_t)id * D;
            const float* pe = p.pos + (size_t)(r.pos0 + t + 1) * D;
#pragma unroll
            for (int c = 0; c < S::KC; c++) {
              const int i = c * 256 + lane * 4;
              const float4 a = *reinterpret_cast<const float4*>(te + i);
              const float4 b = *reinterpret_cast<const float4*>(pe + i);
              *reinterpret_cast<float4*>(sh.xres + i) = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
            }
          }
        }
      }
      }  // greedy
      __syncthreads();  // the next token's x is in xres
      if (thead) trace_mark(p.trace, 19);
    }
  }
#undef TM
  // all tokens done: block 0 advances the launch counter past this launch's tags
  if (!dead && r.blk == 0 && lane == 0)
    __hip_atomic_fetch_add(p.launch, (unsigned)p.nsteps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Data waves: weight tiles in registers.  A tile requested right after the
// phase that consumed it has a whole layer to arrive, and a block then issues
// about one tile per phase (in-flight loads delay every hand-off read of the CU,
// so they are spread over the layer):
//   A: rq(l+1)   B (attention blocks): K/V(l+1)   C: rp(l+1)   D: rf(l+1)   E: rm(l+1)
// The sites below move some of them, by measurement.  Every load is unconditional (an empty buffer resource past the last layer),
// so each register has one producer and one consumer per iteration.  After a
// failed wait (sh.fail, read after each barrier) the stores are skipped.
// Load sites of the data loop, in program order within a layer: after A's
// puts, at the start of B and after B (attention blocks), after the puts of
// C, D and E.  A tile requested before its use in the layer is the layer's
// own; after its use, the next layer's (the next token's first after the last).
enum Site : int { S_AEND = 0, S_BSTART = 1, S_BEND = 2, S_CEND = 3, S_DEND = 4, S_EEND = 5 };
// site of each tile, by measurement (sweeps of every combination): non-attention
// blocks request mlp.fc / mlp.proj right after A (their only slack is the
// attention window) and the next layer's qkv after E; attention blocks request
// their attn.proj tiles at the end of B, right before C, and spread the rest over
// the layer (with the weight tiles' non-temporal hint these two sites measured
// 136.3 against 140.3 us per token; the sampled kernel is unchanged by them)
#ifndef FH_NQ
#define FH_NQ S_EEND
#endif
#ifndef FH_NP
#define FH_NP S_CEND
#endif
#ifndef FH_NF
#define FH_NF S_AEND
#endif
#ifndef FH_NM
#define FH_NM S_AEND
#endif
#ifndef FH_AQ
#define FH_AQ S_BSTART
#endif
#ifndef FH_AKV
#define FH_AKV S_BEND
#endif
#ifndef FH_AP
#define FH_AP S_BEND
#endif
#ifndef FH_AF
#define FH_AF S_DEND
#endif
#ifndef FH_AM
#define FH_AM S_EEND
#endif
template <int D, int H, bool ATTN, bool SAMPLED>
__device__ __forceinline__ void data_loop(const KParams& p, Lds<D, H>& sh, Role r) {
  using S = Shape<D, H>;
  using U = Xu<D>;
  using XL = Xl<D, H>;
  constexpr int KC = S::KC, G = S::G;
  constexpr int SQ = ATTN ? FH_AQ : FH_NQ, SP = ATTN ? FH_AP : FH_NP, SF = ATTN ? FH_AF : FH_NF,
                SM = ATTN ? FH_AM : FH_NM, SKV = FH_AKV;
  static_assert(ATTN || (SQ != S_BSTART && SQ != S_BEND && SP != S_BSTART && SP != S_BEND && SF != S_BSTART &&
                         SF != S_BEND && SM != S_BSTART && SM != S_BEND),
                "blocks without attention have no phase B");
  const int w = r.w, lane = r.lane;
  float4 rq[S::QCW * KC], rp[S::PJ * G], rf[S::FCW * KC], rm[G * S::MJ];
  // K/V rows of this wave's keys: register i holds rows key0 + 4i .. key0 + 4i + 3,
  // lane l the dims 4*(l % 16) .. +3 of row key0 + 4i + l / 16 (one 1 KB load each)
  constexpr int NKV = ATTN ? KPW / 4 : 1;
  float4 kr[NKV], vr[NKV];
  auto tile = [&](int l) { return p.tiles + (size_t)l * S::LAYER; };
  // qkv: a block with qcw < QCW columns per wave reads its chunks twice (same
  // addresses, no extra HBM bytes) so the loads stay unconditional
  auto load_q = [&](int l, bool real) {
    constexpr int HALF = S::QCW * KC / 2;
    const float* t = tile(l) + (size_t)r.vb * S::QT + (size_t)w * r.qcw * D;
    const __amdgpu_buffer_rsrc_t lo = make_rsrc(t, real ? HALF * 1024 : 0);
    const __amdgpu_buffer_rsrc_t hi = make_rsrc(r.qcw == S::QCW ? t + HALF * 256 : t, real ? HALF * 1024 : 0);
    const int off = lane * 16;
#pragma unroll
    for (int i = 0; i < HALF; i++) rq[i] = ld4(lo, off + i * 1024);
#pragma unroll
    for (int i = 0; i < HALF; i++) rq[HALF + i] = ld4(hi, off + i * 1024);
  };
  static_assert(S::QCW % 2 == 0, "qkv chunks split in halves");
  // attn.proj chunks are ordered [head piece j][wave][group]: pieces past the
  // XCD's head count lie outside the resource and read as zeros
  auto load_p = [&](int l, bool real) {
    const float* t = tile(l) + (size_t)NB * S::QT + (size_t)r.vb * S::PT;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(t, real ? r.nh * NDW * G * 1024 : 0);
#pragma unroll
    for (int j = 0; j < S::PJ; j++)
#pragma unroll
      for (int g = 0; g < G; g++) rp[j * G + g] = ld4(rs, ((j * NDW + w) * G + g) * 1024 + lane * 16);
  };
  auto load_f = [&](int l, bool real) {
    load_chunks(rf, tile(l) + (size_t)NB * (S::QT + S::PT) + (size_t)r.vb * S::FT + (size_t)w * S::FCW * D, real);
  };
  auto load_m = [&](int l, bool real) {
    load_chunks(rm,
                tile(l) + (size_t)NB * (S::QT + S::PT + S::FT) + (size_t)r.vb * S::MT + (size_t)w * G * S::MJ * 256,
                real);
  };
  // cached K/V rows of this wave's keys in layer l, through buffer resources
  // bounded by the head's ctx rows (rows at or past the new one are masked
  // below; nothing is fetched when real == false)
  auto load_kv = [&](int l, bool real) {
    const size_t hoff = ((size_t)l * H + r.ah) * p.ctx * 64;
    const int bytes = real ? p.ctx * 256 : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.kc + (real ? hoff : 0), bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vc + (real ? hoff : 0), bytes);
    const int off = r.key0 * 256 + lane * 16;
#pragma unroll
    for (int i = 0; i < NKV; i++) kr[i] = ld4_l2(rk, off + 1024 * i);
#pragma unroll
    for (int i = 0; i < NKV; i++) vr[i] = ld4_l2(rv, off + 1024 * i);
  };
#define TD(i) \
  if (it == r.trace_it) trace_mark_d(p.trace, sh.trd, (i))
#define DSYNC()    \
  __syncthreads(); \
  dead = sh.fail != 0
  bool dead = false;
  constexpr int NPF = HeadRes<SAMPLED>::ROWS;
  if constexpr (NPF > 0) {
    // the first NPF head rows this wave owns (w, w + 3, ... of the block's share)
    // are copied to LDS once; launches of one step read every row from HBM
    const int R = p.Vp / NB;
    const float* E = p.tok + (size_t)(SAMPLED ? r.vb : r.blk) * R * D;
    const int npf = p.nsteps > 1 ? min((R - w + NDW - 1) / NDW, NPF) : 0;
    float* hw = head_rows_lds<NDW * NPF * D>() + (size_t)w * NPF * D;
    for (int u0 = 0; u0 < npf; u0 += 4) {
      float4 hv[4 * KC];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int row = w + NDW * min(u0 + u, npf - 1);
#pragma unroll
        for (int c = 0; c < KC; c++)
          hv[u * KC + c] = *reinterpret_cast<const float4*>(E + (size_t)row * D + c * 256 + lane * 4);
      }
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (u0 + u < npf)
#pragma unroll
          for (int c = 0; c < KC; c++)
            *reinterpret_cast<float4*>(hw + (size_t)(u0 + u) * D + c * 256 + lane * 4) = hv[u * KC + c];
    }
  }
  // Iteration l = -1 only requests layer 0's tiles, through the same load
  // statements as every later layer: each tile register has a single load
  // site, so no copy of an in-flight register (and no wait for it) is needed.
  // tokens t < nsteps, layers l < L: one flat loop; iteration -1 only requests tiles
  const int total = p.nsteps * p.L;
  for (int it = -1; it < total; it++) {
    const bool run = it >= 0;
    const int t = run ? it / p.L : 0, l = run ? it - t * p.L : -1;
    r.pos = r.pos0 + t;
    r.nk = r.pos + 1;
    r.wave_keys = ATTN && r.key0 < r.nk;
    const unsigned tb = r.tag0 + (unsigned)t * TAGS + PH * l;
    const unsigned tA = tb, tC = tb + 3, tD = tb + 5, tE = tb + 6;
    const bool more = it + 1 < total;
    const int ln = l + 1 < p.L ? l + 1 : 0;  // the next layer (the next token's first after the last)
    const bool keys_next = r.key0 < (l + 1 < p.L ? r.nk : r.nk + 1);
    // the requests of one site: this layer's tiles (in order of use), then the next layer's
    auto site = [&](auto site_c) {
      constexpr int X = decltype(site_c)::value;
      const int lc = run ? l : 0;
      if constexpr (ATTN) {
        if constexpr (SKV == X && X < S_BSTART) {
          load_kv(lc, run && r.wave_keys);
          reload_fence();
        }
      }
      if constexpr (SP == X && X < S_CEND) {
        load_p(lc, run);
        reload_fence();
      }
      if constexpr (SF == X && X < S_DEND) {
        load_f(lc, run);
        reload_fence();
      }
      if constexpr (SM == X && X < S_EEND) {
        load_m(lc, run);
        reload_fence();
      }
      if constexpr (SQ == X) {
        load_q(ln, more);
        reload_fence();
      }
      if constexpr (ATTN) {
        if constexpr (SKV == X && X >= S_BSTART) {
          load_kv(ln, more && keys_next);
          reload_fence();
        }
      }
      if constexpr (SP == X && X >= S_CEND) {
        load_p(ln, more);
        reload_fence();
      }
      if constexpr (SF == X && X >= S_DEND) {
        load_f(ln, more);
        reload_fence();
      }
      if constexpr (SM == X && X >= S_EEND) {
        load_m(ln, more);
        reload_fence();
      }
    };
    // ---- A: LN1 + QKV ----
    if (run) {
      DSYNC();
      TD(0);
      {
        float4 d[KC];
        const float rs = ln_center<KC, D>(sh.xres, d);
        float val = 0.f;
#pragma unroll
        for (int t = 0; t < S::QCW; t++) {
          if (t < r.qcw) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < KC; c++) acc += dot4(rq[t * KC + c], d[c]);
            const float v = wave_sum_dpp(acc);
            if (lane == t) val = v;
          }
        }
        if (!dead && lane < r.qcw) {
          const int i = r.slot * r.qc + w * r.qcw + lane;  // index in the XCD's column list
          const float s = val * rs + sh.bias_s[l & 1][S::B_Q + w * r.qcw + lane];
          put_pair(r.xl + XL::QKV + i, s, tA);
          const int j = i / 192, rr = i % 192, part = rr / 64, e = rr % 64;
          if (part > 0) {  // new K or V row of this position, for later steps
            const int h = r.xcd + NX * j;
            (part == 2 ? p.vc : p.kc)[(((size_t)l * H + h) * p.ctx + r.pos) * 64 + e] = s;
          }
        }
        TD(1);
      }
      __syncthreads();  // every put of the phase is issued before any tile load
    }
    site(std::integral_constant<int, S_AEND>());
    if (!ATTN && it == r.trace_it && p.trace) {  // trace: when this wave's requested tiles have landed
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      TD(10);
    }
    // ---- B: attention of head ah over key block kb ----
    if constexpr (ATTN) {
      if (run) {
        DSYNC();
        TD(2);
      }
      site(std::integral_constant<int, S_BSTART>());
      if (run) {
        if (r.wave_keys) {
          // lane l: dims 4*(l % 16) .. +3 of keys key0 + 4i + l / 16, i < KPW / 4
          const int g = lane >> 4, d4 = 4 * (lane & 15);
          const float4 q4 = *reinterpret_cast<const float4*>(sh.qkvs + d4);
          const float4 knew = *reinterpret_cast<const float4*>(sh.qkvs + 64 + d4);
          const float4 vnew = *reinterpret_cast<const float4*>(sh.qkvs + 128 + d4);
          float sc[NKV];
          float mloc = -INFINITY;
          if (it == r.trace_it && p.trace) {  // trace: wait for the K/V rows before timing the scores
            float z = kr[0].x + vr[NKV - 1].w;
            asm volatile("" : "+v"(z));
            if (z == 1234.5f) mloc = 0.f;
            TD(11);
          }
#pragma unroll
          for (int i = 0; i < NKV; i++) {
            const int j = r.key0 + 4 * i + g;
            float sp = dot4(q4, j == r.pos ? knew : kr[i]);
            sp = row16_sum(sp);  // all 16 lanes of the row now hold key j's q.k
            sc[i] = j < r.nk ? sp * 0.125f : -INFINITY;
            mloc = fmaxf(mloc, sc[i]);
          }
          const float mw = wave_max_dpp(mloc);
          TD(12);
          float lloc = 0.f;
          float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
          for (int i = 0; i < NKV; i++) {
            const int j = r.key0 + 4 * i + g;
            const float pj = j < r.nk ? __expf(sc[i] - mw) : 0.f;
            lloc += pj;
            // rows past the new one may hold anything (even NaN): never multiplied
            const float4 v = j < r.pos ? vr[i] : (j == r.pos ? vnew : make_float4(0.f, 0.f, 0.f, 0.f));
            o4.x += pj * v.x;
            o4.y += pj * v.y;
            o4.z += pj * v.z;
            o4.w += pj * v.w;
          }
          const float lw = wave_sum_dpp((lane & 15) == 0 ? lloc : 0.f);
          // sum the four key groups (lanes l, l^16, l^32, l^48)
#pragma unroll
          for (int m = 16; m <= 32; m *= 2) {
            o4.x += __shfl_xor(o4.x, m, 64);
            o4.y += __shfl_xor(o4.y, m, 64);
            o4.z += __shfl_xor(o4.z, m, 64);
            o4.w += __shfl_xor(o4.w, m, 64);
          }
          if (lane == 0) {
            sh.wm[w] = mw;
            sh.wl[w] = lw;
          }
          if (g == 0) *reinterpret_cast<float4*>(&sh.wo[w][d4]) = o4;
        } else {
          if (lane == 0) {
            sh.wm[w] = -INFINITY;
            sh.wl[w] = 0.f;
          }
          sh.wo[w][lane] = 0.f;
        }
        TD(3);
      }
      if (run) {
        __syncthreads();  // wm / wl / wo are complete
        __syncthreads();  // the control wave has published the block's partial
      }
      site(std::integral_constant<int, S_BEND>());
    }
    // ---- C: this XCD's part of attn.proj over its heads' o ----
    if (run) {
      TD(13);
      DSYNC();
      TD(4);
      {
        const int d4 = 4 * (lane & 15), rr = lane >> 4;
#pragma unroll
        for (int g = 0; g < G; g++) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < S::PJ; j++) {
            const float d = dot4(rp[j * G + g], *reinterpret_cast<const float4*>(sh.os + j * 64 + d4));
            acc += j < r.nh ? d : 0.f;  // o of a missing head is stale LDS
          }
          acc = row16_sum(acc);
          if (!dead && (lane & 15) == 0)
            put_pair(p.uc + U::PX2 + r.xcd * D + r.slot * S::RSC + w * 4 * G + 4 * g + rr, acc, tC);
        }
        TD(5);
      }
      __syncthreads();  // every put of the phase is issued before any tile load
    }
    site(std::integral_constant<int, S_CEND>());
    // ---- D: LN2 + mlp.fc + GELU -> this XCD's h slice ----
    if (run) {
      DSYNC();
      TD(6);
      {
        float4 d[KC];
        const float rs = ln_center<KC, D>(sh.x2s, d);
        float val = 0.f;
#pragma unroll
        for (int t = 0; t < S::FCW; t++) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < KC; c++) acc += dot4(rf[t * KC + c], d[c]);
          const float v = wave_sum_dpp(acc);
          if (lane == t) val = v;
        }
        if (!dead && lane < S::FCW) {
          const int c = w * S::FCW + lane;
          put_pair(r.xl + XL::HH + r.slot * S::FCOL + c, gelu_fast(val * rs + sh.bias_s[l & 1][S::B_F + c]), tD);
        }
        TD(7);
      }
      __syncthreads();  // every put of the phase is issued before any tile load
    }
    site(std::integral_constant<int, S_DEND>());
    // ---- E: this XCD's part of mlp.proj over its h slice ----
    if (run) {
      DSYNC();
      TD(8);
      {
        const int d4 = 4 * (lane & 15), rr = lane >> 4;
#pragma unroll
        for (int g = 0; g < G; g++) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < S::MJ; j++)
            acc += dot4(rm[g * S::MJ + j], *reinterpret_cast<const float4*>(sh.hs + j * 64 + d4));
          acc = row16_sum(acc);
          if (!dead && (lane & 15) == 0)
            put_pair(p.uc + U::PX + r.xcd * D + r.slot * S::RSC + w * 4 * G + 4 * g + rr, acc, tE);
        }
        TD(9);
      }
      __syncthreads();  // every put of the phase is issued before any tile load
    }
    site(std::integral_constant<int, S_EEND>());
    if (run && l == p.L - 1) {
      // ---- head of token t: LN_f + tied projection over this block's vocab rows ----
      // block b owns rows [b*R, b*R + R) of the head table (tok_emb, zero-padded to
      // 256 * R rows when V is not a multiple of 256; rows >= V are left out of the
      // argmax); R >= 3, so every data wave has rows: w, w+3, ...
      const int R = p.Vp / NB;
      constexpr int HG = HeadRes<SAMPLED>::INFLIGHT;  // rows per wave in flight
      // (the sampled kernel gives block vb the rows of vb: an XCD's blocks know each other's rows)
      const float* E = p.tok + (size_t)(SAMPLED ? r.vb : r.blk) * R * D;
      const int nrow = (R - w + NDW - 1) / NDW;
      // the first npf rows are in LDS; rows npf .. nrow - 1 stream from HBM, the
      // first of them requested before the final x arrives
      const int npf = NPF > 0 && p.nsteps > 1 ? min(nrow, NPF) : 0;
      const float* hw = NPF > 0 ? head_rows_lds<NDW * (NPF > 0 ? NPF : 1) * D>() + (size_t)w * NPF * D : nullptr;
      float4 rh[HG * KC];
#pragma unroll
      for (int u = 0; u < HG; u++) {
        const int row = w + NDW * min(npf + u, nrow - 1);
#pragma unroll
        for (int c = 0; c < KC; c++)
          rh[u * KC + c] = *reinterpret_cast<const float4*>(E + (size_t)row * D + c * 256 + lane * 4);
      }
      __syncthreads();  // the final x is in xres
      dead = sh.fail != 0;
      if (!dead) {
        float4 xn[KC];
        {
          float4 lw[KC], lb[KC];
#pragma unroll
          for (int c = 0; c < KC; c++) {
            lw[c] = *reinterpret_cast<const float4*>(sh.lnf + c * 256 + lane * 4);
            lb[c] = *reinterpret_cast<const float4*>(sh.lnf + D + c * 256 + lane * 4);
          }
          ln_lane<KC, D>(sh.xres, lw, lb, xn);
        }
        // the rows held in LDS first: their arithmetic covers the streamed rows' latency
        for (int u = 0; u < npf; u++) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < KC; c++)
            acc += dot4(*reinterpret_cast<const float4*>(hw + (size_t)u * D + c * 256 + lane * 4), xn[c]);
          const float v = wave_sum_dpp(acc);
          if (lane == 0) sh.hval[w + NDW * u] = v;
        }
        for (int g = npf; g < nrow; g += HG) {
          float4 nx[HG * KC];
#pragma unroll
          for (int u = 0; u < HG; u++) {
            const int row = w + NDW * min(g + HG + u, nrow - 1);
#pragma unroll
            for (int c = 0; c < KC; c++)
              nx[u * KC + c] = *reinterpret_cast<const float4*>(E + (size_t)row * D + c * 256 + lane * 4);
          }
#pragma unroll
          for (int u = 0; u < HG; u++) {
            if (g + u < nrow) {
              float acc = 0.f;
#pragma unroll
              for (int c = 0; c < KC; c++) acc += dot4(rh[u * KC + c], xn[c]);
              const float v = wave_sum_dpp(acc);
              if (lane == 0) sh.hval[w + NDW * (g + u)] = v;
            }
          }
#pragma unroll
          for (int i = 0; i < HG * KC; i++) rh[i] = nx[i];
        }
      }
      if (it == r.trace_it + p.L - 2) trace_mark_d(p.trace, sh.trd, 14);
      __syncthreads();  // hval holds this block's logits
      __syncthreads();  // the next token's x is in xres
    }
  }
#undef TD
#undef DSYNC
}

template <int D, int H, bool SAMPLED>
__global__ __launch_bounds__(NT, 1) void k_decode_step(KParams p) {
  using S = Shape<D, H>;
  using XL = Xl<D, H>;
  __shared__ Lds<D, H> sh;
  __shared__ SampLds<SAMPLED> sl;

  Role r;
  const int tid = threadIdx.x;
  r.blk = blockIdx.x;
  // w is wave-uniform; readfirstlane lets the compiler know, so buffer
  // resources built from it stay in scalar registers
  r.w = __builtin_amdgcn_readfirstlane(tid >> 6);
  r.lane = tid & 63;
  const bool ctrl = r.w == NW - 1;
  // The dispatcher deals consecutive blocks to consecutive XCDs, continuing
  // from wherever the previous dispatch stopped: the XCD comes from the
  // hardware, and blocks b = 8k .. 8k+7 (slot k) land on 8 different XCDs.
  r.xcd = (int)xcc_id() & (NX - 1);
  r.slot = r.blk / NX;
  // every tile and bias depends on (XCD, slot): they are stored under the
  // virtual block id vb; the head rows are indexed by blk
  r.vb = r.slot * NX + r.xcd;
  if (tid < 32) sh.trd[tid] = 0ull;
  if (p.trace && tid == NT - 64) p.trace[r.blk * TRACE_PER + 12] = (unsigned long long)r.xcd;
  r.tag0 = __hip_atomic_load(p.launch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * TAGS;
  trace_mark(p.trace, 30);

  // steps n0 .. n0 + nsteps - 1 at positions pos0 ..
  r.trace_it = p.nsteps > 5 ? 5 * p.L + 1 : 1;
  r.n0 = *p.src.step;
  r.pos0 = p.src.pos_off + p.src.pos_mul * r.n0;  // position of the first new token (>= 1)
  r.pos = r.pos0;
  r.nk = r.pos0 + 1;
  r.nh0 = p.src.tok_off + r.n0 + 1;  // the window: ids 0 .. prompt_len + n0 - 1
  if constexpr (SAMPLED)
    for (int i = tid; i < r.nh0; i += NT) sl.hist[i] = p.src.tokens[i];  // read after the loops' first barrier
  int tokid = p.src.tokens[p.src.tok_off + r.n0];
  bool bad = false;
  if ((unsigned)tokid >= (unsigned)p.V) {  // never read outside the table: report it and run no step
    tokid = 0;
    bad = true;
    if (tid == 0) raise_err(p.err, err_code(W_TOK, 0));
  }
  // Every (XCD, slot) must be taken by exactly one block of the launch: each block
  // swaps this launch's mark into its slot's claim word (uncached, so the swap is
  // device-wide) and fails fast if a block of the same launch got there first.
  if (tid == 0) {
    unsigned* claim = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(p.uc) + p.off_claim) + r.vb;
    const unsigned mark = r.tag0 | 1u;
    if (__hip_atomic_exchange(claim, mark, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == mark) {
      raise_err(p.err, err_code(W_XCD, 0));
      bad = true;
    }
  }
  if (tid == 0) sh.fail = bad ? 1 : 0;  // read by every wave after its first barrier
  r.xl = p.xl + (size_t)r.xcd * XL::STRIDE;
  r.xl0 = r.xcd * XL::STRIDE;
  // qkv columns: the XCD's heads h = xcd + 8j (j < nh) own columns
  // [j*192, j*192+192) of the XCD's list (q, k, v of each head); slot s has qc of them
  r.nh = (H - r.xcd + NX - 1) / NX;
  r.qc = 3 * S::HD * r.nh / SLOTS;
  r.qcw = r.qc / NDW;
  // attention role: local head hj = slot / SPH, key block kb = slot % SPH; the
  // roles cover the keys of the launch's last token (earlier tokens leave the
  // last blocks without keys: they publish empty partials)
  r.hj = r.slot / S::SPH;
  r.kb = r.slot % S::SPH;
  r.ah = r.xcd + NX * r.hj;
  r.nkb = (r.pos0 + p.nsteps + KPB - 1) / KPB;
  const bool attn_blk = r.hj < r.nh && r.kb < r.nkb;
  r.key0 = r.kb * KPB + r.w * KPW;
  r.wave_keys = attn_blk && r.key0 < r.nk;

  // x = tok_emb[id] + pos_emb[pos] (every block keeps its own copy); ln_f
  for (int i = tid; i < D; i += NT) sh.xres[i] = p.tok[(size_t)tokid * D + i] + p.pos[(size_t)r.pos0 * D + i];
  for (int i = tid; i < 2 * D; i += NT) sh.lnf[i] = p.vecs[i];

  // The control wave and the data waves run separate loops, specialised by
  // the block's role, that meet at the same sequence of barriers; after a
  // failed wait every wave runs on to the end without waiting or storing.
  if (ctrl) {
    ctrl_loop<D, H, SAMPLED>(p, sh, sl, r, attn_blk);
  } else {
    if (attn_blk)
      data_loop<D, H, true, SAMPLED>(p, sh, r);
    else
      data_loop<D, H, false, SAMPLED>(p, sh, r);
  }
  if (ctrl && p.trace && r.lane < 32) p.trace[r.blk * TRACE_PER + 32 + r.lane] = sh.trd[r.lane];
  trace_mark(p.trace, 31);
}

#ifdef FH_DECODE_SAMPLED_TU
}  // namespace
// decode_fast_sampled.hip compiles this file for the sampled kernel alone: the
// instantiation and the two entry points the host code below calls.
hipError_t decode_sampled_occupancy(int* occ) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(occ, k_decode_step<768, 12, true>, NT, 0);
}
hipError_t decode_sampled_launch(hipStream_t st, const void* kparams, bool cooperative) {
  if (cooperative) {
    void* args[] = {const_cast<void*>(kparams)};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&k_decode_step<768, 12, true>), dim3(NB),
                                      dim3(NT), args, 0, st);
  }
  hipLaunchKernelGGL((k_decode_step<768, 12, true>), dim3(NB), dim3(NT), 0, st,
                     *static_cast<const KParams*>(kparams));
  return hipGetLastError();
}
}  // namespace fh
#else

__global__ void k_xcc_probe(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// tile[b][c][k] = scale[k] * W[k][map[b*ncol + c]] (0 where map < 0), W row-major
// [K][N]: the LayerNorm weight in front of the matrix folded into its rows
__global__ void k_relayout(const float* __restrict__ W, int K, int N, const int* __restrict__ map, int ncol,
                           const float* __restrict__ scale, float* __restrict__ tile) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)NB * ncol * K) return;
  const int k = (int)(i % K);
  const size_t bc = i / K;
  const int col = map[bc];
  tile[i] = col >= 0 ? scale[k] * W[(size_t)k * N + col] : 0.f;
}

// out[n] = bias[n] + sum_k shift[k] * W[k][n]: the LayerNorm bias in front of
// the matrix folded into the matrix's bias (accumulated in double)
__global__ void k_fold_bias(const float* __restrict__ W, int K, int N, const float* __restrict__ shift,
                            const float* __restrict__ bias, float* __restrict__ out) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  double s = 0.0;
  for (int k = 0; k < K; k++) s += (double)shift[k] * (double)W[(size_t)k * N + n];
  out[n] = (float)((double)bias[n] + s);
}

// chunks of 4 columns x 64 rows: tile[ch*256 + 4l + q] = W[k0 + 4*(l%16) + q][c0 + l/16]
// for desc[ch] = (k0, c0); zeros where k0 < 0.  W row-major [K][N].
__global__ void k_relayout_chunks(const float* __restrict__ W, int N, const int2* __restrict__ desc, int nchunks,
                                  float* __restrict__ tile) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)nchunks * 256) return;
  const int2 d = desc[i / 256];
  const int e = (int)(i % 256), l = e / 4, q = e % 4;
  tile[i] = d.x >= 0 ? W[(size_t)(d.x + 4 * (l % 16) + q) * N + d.y + l / 16] : 0.f;
}

// out[b*bt + off + j] = src[map[b*ncol + j]] for j < ncol (one bias slice of the table)
__global__ void k_gather_bias(const float* __restrict__ src, const int* __restrict__ map, int ncol, int off,
                              int bt, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= NB * ncol) return;
  const int b = i / ncol, j = i % ncol, col = map[i];
  out[b * bt + off + j] = col >= 0 ? src[col] : 0.f;
}

// Fault injection for the host's fallback (FORGE_HIP_INJECT_FUSED_FAILURE=1):
// the launch's error word is set before it starts, as after a wait that exceeded
// its spin limit, so every wait of the launch gives up at once and every block
// runs to its end without waiting.
__global__ void k_set_word(int* p, int v) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *p = v;
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

constexpr int kD = 768, kH = 12;
using S768 = Shape<kD, kH>;

size_t uc_pairs_bytes(int D) { return (size_t)Xu<kD>::NPAIR * sizeof(uint2) * (D / kD); }
size_t uc_amax_off(int D) { return (uc_pairs_bytes(D) + 255) / 256 * 256; }
size_t uc_claim_off(int D) { return uc_amax_off(D) + (size_t)NB * sizeof(uint4); }
size_t uc_slist_off(int D) { return (uc_claim_off(D) + (size_t)NB * sizeof(unsigned) + 255) / 256 * 256; }
size_t uc_total_bytes(int D) { return uc_slist_off(D) + (size_t)NX * 64 * sizeof(uint4); }

// Host maps, all per virtual block vb = slot * 8 + XCD:
//   q  qkv columns by XCD head ownership          f  mlp.fc columns: the XCD's h slice
//   pc attn.proj chunks (head piece, wave, group)  mc mlp.proj chunks (wave, group, row piece)
//   rs the slot's reduce columns (biases of attn.proj / mlp.proj)
struct Maps {
  std::vector<int> q, f, rs;
  std::vector<int2> pc, mc;
};

Maps make_maps(int D, int H) {
  using S = S768;
  Maps m;
  m.q.assign((size_t)NB * S::QCMAX, -1);
  m.f.resize((size_t)NB * S::FCOL);
  m.rs.resize((size_t)NB * S::RSC);
  m.pc.resize((size_t)NB * S::PJ * NDW * S::G);
  m.mc.resize((size_t)NB * NDW * S::G * S::MJ);
  for (int vb = 0; vb < NB; vb++) {
    const int x = vb % NX, s = vb / NX;
    const int nh = (H - x + NX - 1) / NX;
    const int qc = 3 * 64 * nh / SLOTS;
    for (int c = 0; c < qc; c++) {
      const int i = s * qc + c, j = i / 192, r = i % 192, part = r / 64, e = r % 64;
      m.q[(size_t)vb * S::QCMAX + c] = part * D + (x + NX * j) * 64 + e;
    }
    for (int c = 0; c < S::FCOL; c++) m.f[(size_t)vb * S::FCOL + c] = x * S::HX + s * S::FCOL + c;
    for (int c = 0; c < S::RSC; c++) m.rs[(size_t)vb * S::RSC + c] = s * S::RSC + c;
    for (int j = 0; j < S::PJ; j++)
      for (int w = 0; w < NDW; w++)
        for (int g = 0; g < S::G; g++) {
          const int c0 = s * S::RSC + w * 4 * S::G + 4 * g;
          m.pc[(size_t)vb * S::PJ * NDW * S::G + (j * NDW + w) * S::G + g] =
              j < nh ? make_int2((x + NX * j) * 64, c0) : make_int2(-1, -1);
        }
    for (int w = 0; w < NDW; w++)
      for (int g = 0; g < S::G; g++)
        for (int pc = 0; pc < S::MJ; pc++) {
          const int c0 = s * S::RSC + w * 4 * S::G + 4 * g;
          m.mc[(size_t)vb * NDW * S::G * S::MJ + (w * S::G + g) * S::MJ + pc] = make_int2(x * S::HX + 64 * pc, c0);
        }
  }
  return m;
}

}  // namespace

int FastDecode::init(const fh_model_desc& d, int compute_units) {
  enabled = false;
  D = d.d_model;
  H = d.n_heads;
  L = d.n_layers;
  V = d.vocab_size;
  ctx = d.context_length;
  C = KPB;
  blocks = NB;
  // the head gives each block max(3, ceil(V / 256)) <= 64 vocabulary rows
  const bool shape_ok = d.dtype == FH_DTYPE_F32 && d.max_batch == 1 && D == kD && H == kH &&
                        head_rows(V) <= S768::RMAX && (ctx + KPB - 1) / KPB <= S768::SPH &&
                        compute_units >= NB &&
                        PH * L + 1 <= TAGS;
  if (!shape_ok) return FH_OK;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_decode_step<kD, kH, false>, NT, 0) != hipSuccess || occ < 1)
    return FH_OK;
  // This file keeps an instantiation of the sampled kernel as well (checked here,
  // launched from decode_fast_sampled.hip's copy): the greedy kernel's code
  // generation depends on it (compiled without it, the greedy kernel measured
  // 152.9 instead of 147.1 us per token).
  sampled_ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_decode_step<kD, kH, true>, NT, 0) == hipSuccess &&
               occ >= 1 && decode_sampled_occupancy(&occ) == hipSuccess && occ >= 1;
  if (hipGetDevice(&device) != hipSuccess) return FH_ERR_HIP;
  {
    int co = 0;
    cooperative = hipDeviceGetAttribute(&co, hipDeviceAttributeCooperativeLaunch, device) == hipSuccess && co != 0;
    const char* ce = getenv("FORGE_HIP_COOPERATIVE");
    if (ce && ce[0] == '0') cooperative = false;
    const char* fe = getenv("FORGE_HIP_INJECT_FUSED_FAILURE");
    inject_failure = fe && fe[0] == '1';
  }
  {
    // the XCD-local hand-offs need 8 XCDs dealt blocks round-robin (blocks
    // 8k .. 8k+7 on distinct XCDs); keep the generic path otherwise
    unsigned* dx = nullptr;
    std::vector<unsigned> hx(NB);
    if (hipMalloc(&dx, NB * sizeof(unsigned)) != hipSuccess) return FH_ERR_OOM;
    hipLaunchKernelGGL(k_xcc_probe, dim3(NB), dim3(64), 0, 0, dx);
    const bool got = hipGetLastError() == hipSuccess &&
                     hipMemcpy(hx.data(), dx, NB * sizeof(unsigned), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dx);
    if (!got) return FH_ERR_HIP;
    for (int b = 0; b < NB; b++)
      if (hx[b] >= (unsigned)NX || hx[b] != (hx[0] + b) % NX) return FH_OK;
  }
  tile_floats = S768::LAYER * L;
  if (hipMalloc(&tiles, tile_floats * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  if (hipMalloc(&vecs, 2 * (size_t)D * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  if (hipMalloc(&btab, (size_t)L * NB * S768::BT * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  if (head_rows(V) * NB != V) {
    // every block reads whole rows of its share: the rows past V are zeros
    const size_t bytes = (size_t)NB * head_rows(V) * D * sizeof(float);
    if (hipMalloc(&head, bytes) != hipSuccess) return FH_ERR_OOM;
    if (hipMemset(head, 0, bytes) != hipSuccess) return FH_ERR_HIP;
  }
  xch_bytes = uc_total_bytes(D);
  uc = static_cast<char*>(uc_take(device, xch_bytes));
  if (!uc) return FH_ERR_OOM;
  xl_bytes = (size_t)NX * Xl<kD, kH>::STRIDE * sizeof(uint2);
  if (hipMalloc(&xl, xl_bytes) != hipSuccess) return FH_ERR_OOM;
  if (hipMalloc(&ctl, 256) != hipSuccess) return FH_ERR_OOM;
  if (hipMemset(ctl, 0, 256) != hipSuccess) return FH_ERR_HIP;
  counter = 1;
  if (reset_state() != FH_OK) return FH_ERR_HIP;
  const char* tr = getenv("FORGE_HIP_TRACE");
  if (tr && tr[0] == '1') {
    if (hipMalloc(&trace, (size_t)NB * TRACE_PER * sizeof(unsigned long long)) != hipSuccess) return FH_ERR_OOM;
    if (hipMemset(trace, 0, (size_t)NB * TRACE_PER * sizeof(unsigned long long)) != hipSuccess) return FH_ERR_HIP;
  }
  enabled = true;
  return FH_OK;
}

int FastDecode::build(hipStream_t st, const float* const* params) {
  if (!enabled) return FH_OK;
  using S = S768;
  const Maps m = make_maps(D, H);
  char* dmap = nullptr;
  const size_t nq = m.q.size() * 4, nf = m.f.size() * 4, nr = m.rs.size() * 4, np = m.pc.size() * 8,
               nmc = m.mc.size() * 8;
  if (hipMalloc(&dmap, nq + nf + nr + np + nmc + 7 * (size_t)D * sizeof(float)) != hipSuccess) return FH_ERR_OOM;
  int* dq = reinterpret_cast<int*>(dmap);
  int* df = reinterpret_cast<int*>(dmap + nq);
  int* dr = reinterpret_cast<int*>(dmap + nq + nf);
  int2* dp = reinterpret_cast<int2*>(dmap + nq + nf + nr);
  int2* dm = reinterpret_cast<int2*>(dmap + nq + nf + nr + np);
  float* fold = reinterpret_cast<float*>(dmap + nq + nf + nr + np + nmc);  // folded qkv (3D) and fc (4D) biases
  int rc = FH_OK;
  auto copy = [&](const float* src, float* dst, int n) {
    hipLaunchKernelGGL(k_copy, dim3((n + 255) / 256), dim3(256), 0, st, src, dst, n);
    return hipGetLastError() == hipSuccess;
  };
  auto relayout = [&](const float* W, int K, int N, const int* map, int ncol, const float* scale, float* out) {
    const size_t tot = (size_t)NB * ncol * K;
    hipLaunchKernelGGL(k_relayout, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, W, K, N, map, ncol, scale,
                       out);
    return hipGetLastError() == hipSuccess;
  };
  auto fold_bias = [&](const float* W, int K, int N, const float* shift, const float* b, float* out) {
    hipLaunchKernelGGL(k_fold_bias, dim3((N + 255) / 256), dim3(256), 0, st, W, K, N, shift, b, out);
    return hipGetLastError() == hipSuccess;
  };
  auto chunks = [&](const float* W, int N, const int2* desc, int nch, float* out) {
    const size_t tot = (size_t)nch * 256;
    hipLaunchKernelGGL(k_relayout_chunks, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, W, N, desc, nch,
                       out);
    return hipGetLastError() == hipSuccess;
  };
  auto bias = [&](const float* src, const int* map, int ncol, int off, float* out) {
    hipLaunchKernelGGL(k_gather_bias, dim3((NB * ncol + 255) / 256), dim3(256), 0, st, src, map, ncol, off, S::BT,
                       out);
    return hipGetLastError() == hipSuccess;
  };
  if (hipMemcpy(dq, m.q.data(), nq, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(df, m.f.data(), nf, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(dr, m.rs.data(), nr, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(dp, m.pc.data(), np, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(dm, m.mc.data(), nmc, hipMemcpyHostToDevice) != hipSuccess)
    rc = FH_ERR_HIP;
  for (int l = 0; l < L && rc == FH_OK; l++) {
    float* tl = tiles + (size_t)l * S::LAYER;
    const float* const* PL = params + 2 + 12 * l;
    float* bt = btab + (size_t)l * NB * S::BT;
    // registry slots: 0 ln1.w 1 ln1.b 2 qkv.w 3 qkv.b 4 proj.w 5 proj.b 6 ln2.w 7 ln2.b 8 fc.w 9 fc.b 10 mproj.w 11 mproj.b
    // LN1 is folded into qkv (weight into the rows, bias into qkv.b), LN2 into mlp.fc
    const bool good = relayout(PL[2], D, 3 * D, dq, S::QCMAX, PL[0], tl) &&
                      chunks(PL[4], D, dp, (int)m.pc.size(), tl + (size_t)NB * S::QT) &&
                      relayout(PL[8], D, 4 * D, df, S::FCOL, PL[6], tl + (size_t)NB * (S::QT + S::PT)) &&
                      chunks(PL[10], D, dm, (int)m.mc.size(), tl + (size_t)NB * (S::QT + S::PT + S::FT)) &&
                      fold_bias(PL[2], D, 3 * D, PL[1], PL[3], fold) &&
                      fold_bias(PL[8], D, 4 * D, PL[7], PL[9], fold + 3 * D) &&
                      bias(fold, dq, S::QCMAX, S::B_Q, bt) && bias(fold + 3 * D, df, S::FCOL, S::B_F, bt) &&
                      bias(PL[5], dr, S::RSC, S::B_P, bt) && bias(PL[11], dr, S::RSC, S::B_M, bt);
    if (!good) rc = FH_ERR_HIP;
  }
  const float* const* PF = params + 2 + 12 * L;
  if (rc == FH_OK && (!copy(PF[0], vecs, D) || !copy(PF[1], vecs + D, D))) rc = FH_ERR_HIP;
  if (rc == FH_OK && head && hipMemcpyAsync(head, params[0], (size_t)V * D * sizeof(float), hipMemcpyDeviceToDevice,
                                            st) != hipSuccess)
    rc = FH_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) rc = FH_ERR_HIP;
  (void)hipFree(dmap);
  return rc;
}

int FastDecode::enqueue(hipStream_t st, const Step& s) {
  if (!enabled) return FH_ERR_STATE;
  if (!s.src.tokens || !s.src.step || !s.tokens || !s.step || !s.kcache || !s.vcache || !s.logits || !s.out_ids ||
      !s.out_counts || s.src.pos_mul != 1 || s.max_new <= 0 || s.nsteps < 1 || (s.nsteps > 1 && !s.greedy))
    return FH_ERR_INVALID;
  if (s.sampled && !sampler_fits(s.top_k, s.window_end))
    return FH_ERR_INVALID;
  KParams k{};
  k.src = s.src;
  k.tiles = tiles;
  k.vecs = vecs;
  k.btab = btab;
  k.pos = s.pos_emb;
  k.kc = s.kcache;
  k.vc = s.vcache;
  k.logits = s.logits;
  k.out_ids = s.out_ids;
  k.out_counts = s.out_counts;
  k.uc = reinterpret_cast<uint2*>(uc);
  k.uc_bytes = (int)xch_bytes;
  k.off_amax = (int)uc_amax_off(D);
  k.off_claim = (int)uc_claim_off(D);
  k.off_slist = (int)uc_slist_off(D);
  k.xl = reinterpret_cast<uint2*>(xl);
  k.xl_bytes = (int)xl_bytes;
  k.launch = reinterpret_cast<unsigned*>(ctl);
  k.err = reinterpret_cast<int*>(ctl) + 16;
  k.V = V;
  k.tok = head ? head : s.tok_emb;
  k.Vp = NB * head_rows(V);
  k.ctx = ctx;
  k.L = L;
  k.max_new = s.max_new;
  k.eos = s.eos;
  k.greedy = s.greedy;
  k.nsteps = s.nsteps;
  k.tokens_out = s.tokens;
  k.step_out = s.step;
  k.trace = trace;
  k.uniforms = s.uniforms;
  k.temperature = s.temperature;
  k.penalty = s.penalty;
  k.top_k = s.top_k;
  k.ngram = s.ngram;
  static_assert(kD == 768 && kH == 12, "the sampled kernel's instantiation");
  if (inject_failure) {
    // a spin-limit code of wait 1 (x), layer 0, block 0
    hipLaunchKernelGGL(k_set_word, dim3(1), dim3(64), 0, st, k.err, (int)(0x80000000u | (1u << 24)));
    if (hipGetLastError() != hipSuccess) return FH_ERR_HIP;
  }
  // The 256 blocks wait on each other, so they must all be resident at once: a
  // cooperative launch guarantees it (or fails up front).  Stream capture records
  // plain kernel nodes only; the captured per-step launches rely on the occupancy
  // checked at init (one block per CU on >= 256 CUs) and on the session's stream
  // being the only work on the device.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) return FH_ERR_HIP;
  const bool co = cooperative && cap == hipStreamCaptureStatusNone;
  if (s.sampled) return decode_sampled_launch(st, &k, co) == hipSuccess ? FH_OK : FH_ERR_HIP;
  if (co) {
    void* args[] = {&k};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&k_decode_step<kD, kH, false>), dim3(NB),
                                      dim3(NT), args, 0, st) == hipSuccess
               ? FH_OK
               : FH_ERR_HIP;
  }
  hipLaunchKernelGGL((k_decode_step<kD, kH, false>), dim3(NB), dim3(NT), 0, st, k);
  return hipGetLastError() == hipSuccess ? FH_OK : FH_ERR_HIP;
}

int FastDecode::before_launches(int n) {
  if (!enabled || n <= 0) return FH_OK;
  // keep launch counter * 128 far from wrapping in 32 bits
  if (launched + (unsigned long long)n >= (1ull << 24)) {
    launched = 0;
    counter = 1;
    return reset_state();
  }
  launched += (unsigned long long)n;
  return FH_OK;
}

// The launch counter starts at `counter`; every launch advances it by one.  A
// reset continues past every value a failed launch may have used, so no live
// tag (counter * 128 + phase) ever equals a stale one, and zeroed memory (tag
// 0) never matches either.
int FastDecode::reset_state() {
  unsigned cur = 0;
  if (ctl && hipMemcpy(&cur, ctl, sizeof cur, hipMemcpyDeviceToHost) != hipSuccess) return FH_ERR_HIP;
  if (cur + 2 > counter) counter = cur + 2;
  if (hipMemset(ctl, 0, 256) != hipSuccess) return FH_ERR_HIP;
  if (hipMemcpy(ctl, &counter, sizeof counter, hipMemcpyHostToDevice) != hipSuccess) return FH_ERR_HIP;
  if (hipMemset(uc, 0, xch_bytes) != hipSuccess) return FH_ERR_HIP;
  if (hipMemset(xl, 0, xl_bytes) != hipSuccess) return FH_ERR_HIP;
  return hipDeviceSynchronize() == hipSuccess ? FH_OK : FH_ERR_HIP;
}

int FastDecode::reset() { return enabled ? reset_state() : FH_OK; }

// The sampled kernel draws inside the launch when 0 < k <= 63, the window never
// exceeds its history buffer, and every XCD keeps more than k unbanned rows (an
// XCD has 32 * rows-per-block rows, fewer by the padding past V, and at most
// window_end of them are banned or penalised away): then no row set is all-banned and
// every selection has k candidates.
bool FastDecode::sampler_fits(int top_k, int window_end) const {
  const int R = head_rows(V);
  return enabled && sampled_ok && top_k > 0 && top_k <= KMAX && top_k < V && window_end <= HCAP &&
         window_end <= ctx && SLOTS * R - (NB * R - V) - window_end > KMAX;
}

int FastDecode::check_error(unsigned* code) {
  if (code) *code = 0;
  if (!enabled) return FH_OK;
  unsigned h = 0;
  if (hipMemcpy(&h, reinterpret_cast<int*>(ctl) + 16, sizeof h, hipMemcpyDeviceToHost) != hipSuccess)
    return FH_ERR_HIP;
  if (code) *code = h;
  return h ? FH_ERR_HIP : FH_OK;
}

void FastDecode::release() {
  if (tiles) (void)hipFree(tiles);
  if (vecs) (void)hipFree(vecs);
  if (btab) (void)hipFree(btab);
  if (head) (void)hipFree(head);
  if (xl) (void)hipFree(xl);
  uc_give(device, xch_bytes, uc);
  if (ctl) (void)hipFree(ctl);
  if (trace) (void)hipFree(trace);
  tiles = vecs = btab = head = nullptr;
  xl = nullptr;
  uc = nullptr;
  ctl = nullptr;
  trace = nullptr;
  enabled = false;
}

}  // namespace fh
#endif  // FH_DECODE_SAMPLED_TU
