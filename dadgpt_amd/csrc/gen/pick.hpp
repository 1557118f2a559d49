// Greedy-pick candidates, shared by the logits projection's epilogue (skinny.hip) and the pick
// kernels (gpt2_ops.hip): a row's best value, its column and the runner-up value. Merging two
// candidates is associative and commutative (ties go to the lower column, as std::max_element
// picks the first maximum: src/generate.cpp:34-37), so any reduction order gives the same pick
// and margin.
#pragma once

#include <hip/hip_runtime.h>

namespace dadgpt::gen {

struct Pick {
  float v1;  // best value
  int i1;    // its column
  float v2;  // runner-up value
};

__device__ __forceinline__ Pick pick_none() {
  return Pick{-__builtin_inff(), 0x7fffffff, -__builtin_inff()};
}

// The better of two candidates (higher value, then lower index) keeps its index; the runner-up
// value is the larger of the loser's best and the winner's runner-up.
__device__ __forceinline__ Pick pick_combine(Pick a, Pick b) {
  const bool b_wins = b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1);
  const Pick& w = b_wins ? b : a;
  const Pick& l = b_wins ? a : b;
  return Pick{w.v1, w.i1, fmaxf(l.v1, w.v2)};
}

__device__ __forceinline__ Pick pick_shfl_xor(const Pick& p, int off) {
  return Pick{__shfl_xor(p.v1, off, 64), __shfl_xor(p.i1, off, 64), __shfl_xor(p.v2, off, 64)};
}

}  // namespace dadgpt::gen
