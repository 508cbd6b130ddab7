// decode_fast_sampled.hip -- the sampled persistent decode kernel
// (k_decode_step<768, 12, true> of decode_fast.hip) in a translation unit of its
// own, so that it is compiled with every loop aligned to a 64-byte instruction
// fetch line (-falign-loops=64 in the Makefile).  Its hand-off poll loops run
// faster aligned: 155.5 against 164.2 us per sampled token (top-k 30) on one
// MI355X, where the same option slows the greedy kernel from 147.9 to 149.8 us,
// so the greedy kernel stays in decode_fast.hip without it.
#define FH_DECODE_SAMPLED_TU 1
#include "decode_fast.hip"
