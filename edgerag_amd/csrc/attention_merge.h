// Merge arithmetic of split attention partials, shared by the merge launches of attention.hip
// (the combine-list and the slotted forms), so that both produce the same bits.
//
// A partial of a (token, query head) over a part of the keys is (m, l, acc[D]): m the
// log2-domain maximum score, l = sum exp2(s - m), acc = sum exp2(s - m) v. Records with m = -inf
// hold no key (an empty slot, or a part past a causal limit).
#pragma once

#include "common.h"

namespace edgerag {

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Partials a thread folds per batch (the (m, l) and acc loads of a batch go out together).
constexpr int kCombineBatch = 16;

// Folds one batch of partial records into the running (m, l, acc): weight exp2(m_k - max) for the
// records that hold keys (take[k] and m_k > -inf); the others are skipped whatever their acc
// holds (a slot never written this step may hold any bits).
__device__ __forceinline__ void merge_partials(const float2 (&ml)[kCombineBatch],
                                               const float4 (&v)[kCombineBatch],
                                               const bool (&take)[kCombineBatch], float& m,
                                               float& l, float4& acc) {
  float mb = m;
#pragma unroll
  for (int k = 0; k < kCombineBatch; ++k)
    if (take[k]) mb = fmaxf(mb, ml[k].x);
  // No branch on mb == -inf (no record so far has seen a key): every weight below is then 0, and
  // a branch here would make the compiler sink the acc loads behind the (m, l) wait.
  const float r = m == -INFINITY ? 0.f : exp2_fast(m - mb);
  l *= r;
  acc.x *= r;
  acc.y *= r;
  acc.z *= r;
  acc.w *= r;
#pragma unroll
  for (int k = 0; k < kCombineBatch; ++k) {
    const bool on = take[k] && ml[k].x != -INFINITY;
    const float w = on ? exp2_fast(ml[k].x - mb) : 0.f;
    l = on ? fmaf(w, ml[k].y, l) : l;
    acc.x = on ? fmaf(w, v[k].x, acc.x) : acc.x;
    acc.y = on ? fmaf(w, v[k].y, acc.y) : acc.y;
    acc.z = on ? fmaf(w, v[k].z, acc.z) : acc.z;
    acc.w = on ? fmaf(w, v[k].w, acc.w) : acc.w;
  }
  m = mb;
}

// The merged output scale: 1 / l (l of a row that saw no key is 0: its output is 0).
__device__ __forceinline__ float merge_inv(float l) { return 1.f / fmaxf(l, 1.17549435e-38f); }

}  // namespace edgerag
