// choices.h — the k routing choices of one token in ascending expert order,
// the order in which the combine and the input-gradient reductions add the
// token's expert rows (the reference adds experts in ascending index,
// FusionLLM models/moe.py:65-76).
#pragma once

#include "fmoe_common.h"

namespace fmoe {

// Load the k choices of token t and return them in ascending expert order
// (the experts of one token are distinct).
struct Choices {
  int e[FMOE_MAX_TOPK];
  int pos[FMOE_MAX_TOPK];
  float w[FMOE_MAX_TOPK];
  int slot[FMOE_MAX_TOPK];
};

__device__ __forceinline__ void load_sorted_choices(const int32_t* idx, const int32_t* pos_of_slot,
                                                    const float* weights, int64_t t, int k,
                                                    Choices& c) {
#pragma unroll
  for (int j = 0; j < FMOE_MAX_TOPK; ++j) {
    if (j < k) {
      const int64_t s = t * k + j;
      c.e[j] = idx[s];
      c.pos[j] = pos_of_slot[s];
      c.w[j] = weights ? weights[s] : 0.0f;
      c.slot[j] = j;
    } else {
      c.e[j] = 0x7fffffff;
      c.pos[j] = 0;
      c.w[j] = 0.0f;
      c.slot[j] = j;
    }
  }
  // k <= 2 (the reference's top-2 configurations): at most one swap.
  if (k <= 2) {
    if (k == 2 && c.e[0] > c.e[1]) {
      int te = c.e[0]; c.e[0] = c.e[1]; c.e[1] = te;
      int tp = c.pos[0]; c.pos[0] = c.pos[1]; c.pos[1] = tp;
      float tw = c.w[0]; c.w[0] = c.w[1]; c.w[1] = tw;
      int ts = c.slot[0]; c.slot[0] = c.slot[1]; c.slot[1] = ts;
    }
    return;
  }
  // Odd-even transposition sort on 8 entries (padding sorts to the end).
#pragma unroll
  for (int pass = 0; pass < FMOE_MAX_TOPK; ++pass) {
#pragma unroll
    for (int j = pass & 1; j + 1 < FMOE_MAX_TOPK; j += 2) {
      if (c.e[j] > c.e[j + 1]) {
        int te = c.e[j]; c.e[j] = c.e[j + 1]; c.e[j + 1] = te;
        int tp = c.pos[j]; c.pos[j] = c.pos[j + 1]; c.pos[j + 1] = tp;
        float tw = c.w[j]; c.w[j] = c.w[j + 1]; c.w[j + 1] = tw;
        int ts = c.slot[j]; c.slot[j] = c.slot[j + 1]; c.slot[j + 1] = ts;
      }
    }
  }
}

}  // namespace fmoe
