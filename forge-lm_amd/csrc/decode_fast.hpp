// decode_fast.hpp -- persistent batch-1 fp32 decode step (decode_fast.hip).
#pragma once

#include "../../include/forge_hip.h"
#include "common.hpp"

namespace fh {

// The sampled persistent kernel (decode_fast_sampled.hip, a translation unit of
// its own): its occupancy, and a launch of 256 blocks with the kernel's
// parameter block (`kparams` points at it; it is copied at the launch).
hipError_t decode_sampled_occupancy(int* occ);
hipError_t decode_sampled_launch(hipStream_t st, const void* kparams, bool cooperative);

// Device state of the persistent decode path for one session.  It runs one
// batch-1 fp32 decode step per launch: all layers, the tied head and (in
// greedy mode) the argmax, with dataflow hand-offs between phases.  Sessions
// whose shape it was not built for keep `enabled` false and use the generic
// kernels.
struct FastDecode {
  bool enabled = false;
  int D = 0, H = 0, L = 0, V = 0, C = 0, ctx = 0;
  int blocks = 0;
  int device = 0;
  float* tiles = nullptr;            // per-block weight tiles, column-major
  float* vecs = nullptr;             // ln_f weight and bias (LN1 / LN2 are folded into the tiles)
  float* btab = nullptr;             // per-layer, per-block bias slices
  float* head = nullptr;             // copy of tok_emb zero-padded to a whole number of rows per block, when V needs it
  char* uc = nullptr;                // uncached hand-off area (cross-XCD pairs, argmax records)
  size_t xch_bytes = 0;
  void* xl = nullptr;                // per-XCD hand-off area (q/k/v, attention partials)
  size_t xl_bytes = 0;
  void* ctl = nullptr;  // launch counter (word 0), error word (16)
  unsigned counter = 1;                 // launch counter value set at the last reset
  unsigned long long launched = 0;      // launches since that reset
  unsigned long long* trace = nullptr;  // per-block timestamps of the last step (FORGE_HIP_TRACE=1), 256 x 32
  size_t tile_floats = 0;

  int init(const fh_model_desc& d, int compute_units);
  // Builds the tiles from the registry tensors (host array of device fp32 pointers, registry order).
  int build(hipStream_t st, const float* const* params);
  struct Step {
    RowSrc src;          // decode row: tok_off = pos_off = P-1, pos_mul = 1
    const float* tok_emb;
    const float* pos_emb;
    float* kcache;       // [L][H][ctx][hd]
    float* vcache;
    float* logits;       // [V] out
    int* out_ids;        // [max_new]
    int* out_counts;     // [1]
    int max_new;
    int eos;
    int greedy;          // 1: argmax + history update inside the kernel
    int nsteps = 1;      // steps run by the launch (more than one needs greedy): step
                         // n + 1 starts from the argmax of step n, without the host
    int* tokens;         // mutable views of src.tokens / src.step
    int* step;
    // sampled: the launch draws every step itself (Sampler.Sample with top-k after
    // ApplyRepetitionControls) from uniforms[n]; needs sampler_fits(top_k, window_end)
    int sampled = 0;
    const double* uniforms = nullptr;
    float temperature = 0.f, penalty = 1.f;
    int top_k = 0, ngram = 0;
    int window_end = 0;  // the window's length after the launch's last step
  };
  int enqueue(hipStream_t st, const Step& s);
  // Called before n more launches (graph replays included); resets the tag
  // state before the launch counter could wrap.
  int before_launches(int n);
  // FH_ERR_HIP when a wait of the last launches gave up; *code (optional)
  // says which: 1 << 31 | wait << 24 | layer << 16 | block.
  int check_error(unsigned* code = nullptr);
  // The device word check_error reads (for an asynchronous copy on the stream).
  const int* error_word() const { return reinterpret_cast<const int*>(ctl) + 16; }
  int reset();  // fresh launch counter, cleared hand-off area and error word
  // Whether a sampled launch can run these options with windows up to window_end ids.
  bool sampler_fits(int top_k, int window_end) const;
  bool sampled_ok = false;  // the sampled kernel fits on the device
  // launches outside stream capture are cooperative (co-residency of the 256
  // blocks guaranteed, or the launch fails) when the device supports it, unless
  // FORGE_HIP_COOPERATIVE=0
  bool cooperative = false;
  // FORGE_HIP_INJECT_FUSED_FAILURE=1 (fault injection, for the fallback's test):
  // every launch starts with its error word set, so its waits give up at once
  bool inject_failure = false;
  void release();

 private:
  int reset_state();
};

}  // namespace fh
