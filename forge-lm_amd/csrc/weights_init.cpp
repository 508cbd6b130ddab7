// weights_init.cpp -- host-side GptModel random init for fh_session_init_random.
//
// GptModel's constructor (src/LLM.Core/Model/GptModel.cs:38-99) fills the
// registry in order from one seeded System.Random: tok_emb and pos_emb with
// N(0, 0.02), per block the qkv/fc matrices with N(0, 0.02) and the two
// residual projections with N(0, 0.02/sqrt(2L)), LayerNorm weights 1, biases 0.
// Tensor.FillNormal (src/LLM.Core/Tensor/Tensor.cs:79-91) draws Box-Muller
// pairs in double.  System.Random(seed) is the legacy subtractive generator
// (Knuth, TAOCP vol. 2 3.2.2; Numerical Recipes "ran3") with seed constant
// 161803398, a 55-word state and taps 21 apart; NextDouble = sample / (2^31-1).
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <vector>

#pragma clang fp contract(off)

namespace fh {

namespace {

class SubtractiveRandom {
 public:
  explicit SubtractiveRandom(int seed) {
    const int kBig = 2147483647, kSeed = 161803398;
    int sub = (seed == INT32_MIN) ? kBig : std::abs(seed);
    int mj = kSeed - sub;
    state_[55] = mj;
    int mk = 1, ii = 0;
    for (int i = 1; i < 55; i++) {
      ii = (ii + 21) % 55;
      state_[ii] = mk;
      mk = mj - mk;
      if (mk < 0) mk += kBig;
      mj = state_[ii];
    }
    for (int round = 0; round < 4; round++)
      for (int i = 1; i < 56; i++) {
        state_[i] -= state_[1 + (i + 30) % 55];
        if (state_[i] < 0) state_[i] += kBig;
      }
    state_[0] = 0;
  }
  double next_double() {
    const int kBig = 2147483647;
    if (++a_ >= 56) a_ = 1;
    if (++b_ >= 56) b_ = 1;
    int r = state_[a_] - state_[b_];
    if (r == kBig) r--;
    if (r < 0) r += kBig;
    state_[a_] = r;
    return r * (1.0 / kBig);
  }

 private:
  int state_[56];
  int a_ = 0, b_ = 21;
};

void box_muller_fill(float* out, int64_t n, SubtractiveRandom& rng, float stddev) {
  const double two_pi = 2 * M_PI;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = 1.0 - rng.next_double();
    const double u2 = rng.next_double();
    const double radius = std::sqrt(-2.0 * std::log(u1));
    out[i] = (float)(radius * std::cos(two_pi * u2) * (double)stddev);
    if (i + 1 < n) out[i + 1] = (float)(radius * std::sin(two_pi * u2) * (double)stddev);
  }
}

}  // namespace

// Fills `w` (registry order, `numel` floats total) for the given shape.
// `kinds[i]`: 0 = zero, 1 = ones, 2 = normal(0.02), 3 = normal(0.02/sqrt(2L)).
void init_registry_random(int seed, int n_layers, const std::vector<int64_t>& offsets,
                          const std::vector<int64_t>& sizes, const std::vector<int>& kinds, float* w) {
  SubtractiveRandom rng(seed);
  const float base = 0.02f;
  const float resid = 0.02f / std::sqrt(2.f * (float)n_layers);
  for (size_t i = 0; i < offsets.size(); i++) {
    float* p = w + offsets[i];
    switch (kinds[i]) {
      case 0:
        for (int64_t j = 0; j < sizes[i]; j++) p[j] = 0.f;
        break;
      case 1:
        for (int64_t j = 0; j < sizes[i]; j++) p[j] = 1.f;
        break;
      case 2:
        box_muller_fill(p, sizes[i], rng, base);
        break;
      default:
        box_muller_fill(p, sizes[i], rng, resid);
        break;
    }
  }
}

void random_doubles(int seed, int n, double* out) {
  SubtractiveRandom rng(seed);
  for (int i = 0; i < n; i++) out[i] = rng.next_double();
}

}  // namespace fh
