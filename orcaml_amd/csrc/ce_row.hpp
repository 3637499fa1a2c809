// Device helpers shared by the fused softmax cross-entropy kernels: wave64
// reductions and the per-row forward / gradient / argmax of
// python/orca/nn/loss.py:59-100 (the composed CrossEntropyLoss) as the tape
// differentiates it.  Translation units including this file are built with
// -ffp-contract=off: each f32 operation below is the reference's own.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cmath>

namespace orca_hip {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {  // strict `>`: NaN never wins
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float w = __shfl_xor(v, o, 64);
    if (w > v) v = w;
  }
  return v;
}

// Largest value, ties to the lowest index (idx = INT_MAX marks "no candidate").
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float w = __shfl_xor(v, o, 64);
    int wi = __shfl_xor(idx, o, 64);
    if (wi != INT_MAX && (idx == INT_MAX || w > v || (w == v && wi < idx))) {
      v = w;
      idx = wi;
    }
  }
}

// Row argmax with the reference's sequential rule (python/orca/nn/model.py:65-75):
// best starts at r[0]; a later value replaces it only if strictly greater.
// Lanes propose their first strict maximum over c >= 1 (NaN never proposes);
// the winner beats r[0] only if strictly greater, and a NaN r[0] is never beaten.
template <int VPL, class Get>
__device__ __forceinline__ int row_argmax(Get get, int C) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY;
  int bi = INT_MAX;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    int c = lane + 64 * j;
    if (c >= 1 && c < C) {
      float v = get(j);
      if (v == v && (bi == INT_MAX || v > bv)) {
        bv = v;
        bi = c;
      }
    }
  }
  wave_argmax(bv, bi);
  const float first = __shfl(get(0), 0, 64);
  if (bi == INT_MAX) return 0;
  return (bv > first) ? bi : 0;
}

struct CeRowOut {
  float loss;  // -sum_c t_c (p_c - lse): the row's term of the loss before the 1/B mean
  int pred;    // argmax of the logits
  int target;  // target class (label, or argmax of the one-hot row)
};

// One row held by one wave64: x[j] is the logit of column lane + 64 j
// (columns >= C are ignored), tval(j) its target.  Writes the row of
// dL/dlogits to `dr` when non-null.  Every lane returns the same values.
//
// The gradient is the tape's, element by element, through the 22-node
// composition (seed * (1/B), * -1, * target, the identity expands' 0 + g,
// the g / see of LogBackward, the full-gradient-to-ties MaxToShapeBackward).
template <int VPL, class TVal>
__device__ __forceinline__ CeRowOut ce_row(const float (&x)[VPL], int C, TVal tval, bool labels, int label, float inv_b,
                                           float* __restrict__ dr, bool want_argmax) {
  const int lane = threadIdx.x & 63;
  float e[VPL];
  // max_to_shape (init -FLT_MAX, strict >)
  float mx = -FLT_MAX;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (lane + 64 * j < C && x[j] > mx) mx = x[j];
  mx = wave_max(mx);
  // exp(p - max) and its row sum
  float se = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    e[j] = (lane + 64 * j < C) ? expf(x[j] - mx) : 0.0f;
    se = se + e[j];
  }
  se = wave_sum(se);
  const float lg = logf(fmaxf(se, 1e-7f));
  const float lse = mx + lg;
  // per-row loss: sum_c -(t * (p - lse))
  float pb = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (lane + 64 * j < C) pb = pb + (tval(j) * (x[j] - lse)) * -1.0f;
  pb = wave_sum(pb);

  if (dr) {
    const float g_tm = inv_b * -1.0f;
    float gse = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + 64 * j < C) {
        float g_lse = 0.0f + ((g_tm * tval(j)) * -1.0f);
        gse = gse + (0.0f + g_lse) / se;
      }
    gse = wave_sum(gse);
    float gmx = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + 64 * j < C) {
        float g_lse = 0.0f + ((g_tm * tval(j)) * -1.0f);
        float g_sh = gse * e[j];
        gmx = gmx + ((0.0f + g_lse) + (0.0f + (g_sh * -1.0f)));
      }
    gmx = wave_sum(gmx);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      int c = lane + 64 * j;
      if (c < C) {
        float g_ls = g_tm * tval(j);
        float g_sh = gse * e[j];
        float d = (0.0f + g_ls) + (0.0f + g_sh);
        float g3 = 0.0f;
        if (x[j] == mx) g3 = g3 + gmx;
        dr[c] = d + g3;
      }
    }
  }

  CeRowOut out{pb, 0, 0};
  if (want_argmax) {
    out.pred = row_argmax<VPL>([&](int j) { return x[j]; }, C);
    out.target = labels ? label : row_argmax<VPL>(tval, C);
  }
  return out;
}

}  // namespace orca_hip
