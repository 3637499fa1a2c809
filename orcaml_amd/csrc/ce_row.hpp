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

// exp(d) of the softmax terms as 2^(d * log2 e) on the hardware exp2
// (v_exp_f32, 1 ulp): three instructions instead of libm expf's range
// reduction in extended precision, which dominated the instruction count of
// the wide-row kernels.  The rounded product shifts the exponent by at most
// |d * log2 e| * 2^-24, so the relative error is below 1.2e-6 for d > -20
// (every term above 2e-9 of the row's largest) and below 6e-6 down to the
// underflow of the result; exp(0) = 1 and exp(-inf) = 0 exactly, NaN stays
// NaN.
__device__ __forceinline__ float ce_exp(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504088896341f); }

// ---- wave64 reductions on the DPP network (no LDS round trips) ----
// Steps: quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror
// leave every lane of a 16-lane row holding the row's result; row_bcast:15
// into rows 1 and 3 and row_bcast:31 into rows 2 and 3 then complete it in
// lane 63, which is broadcast.  Lanes a masked step does not write get `old`,
// the operation's identity.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ int dpp_i(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(dpp_i<CTRL, ROWS>(__float_as_int(old), __float_as_int(v)));
}

template <class Op>
__device__ __forceinline__ float wave_reduce_f(float v, float identity, Op op) {
  v = op(v, dpp_f<0xb1>(identity, v));
  v = op(v, dpp_f<0x4e>(identity, v));
  v = op(v, dpp_f<0x141>(identity, v));
  v = op(v, dpp_f<0x140>(identity, v));
  v = op(v, dpp_f<0x142, 0xa>(identity, v));
  v = op(v, dpp_f<0x143, 0xc>(identity, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce_f(v, 0.0f, [](float a, float b) { return a + b; });
}

// strict `>`: NaN never wins
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce_f(v, -INFINITY, [](float a, float b) { return b > a ? b : a; });
}

__device__ __forceinline__ int wave_sum_i(int v) {
  v = v + dpp_i<0xb1>(0, v);
  v = v + dpp_i<0x4e>(0, v);
  v = v + dpp_i<0x141>(0, v);
  v = v + dpp_i<0x140>(0, v);
  v = v + dpp_i<0x142, 0xa>(0, v);
  v = v + dpp_i<0x143, 0xc>(0, v);
  return __builtin_amdgcn_readlane(v, 63);
}

// Largest value, ties to the lowest index (idx = INT_MAX marks "no candidate").
// The combine is a total-order maximum, so any reduction tree gives the same pair.
__device__ __forceinline__ void argmax_combine(float& v, int& idx, float w, int wi) {
  if (wi != INT_MAX && (idx == INT_MAX || w > v || (w == v && wi < idx))) {
    v = w;
    idx = wi;
  }
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ void argmax_step(float& v, int& idx) {
  const float w = dpp_f<CTRL, ROWS>(-INFINITY, v);
  const int wi = dpp_i<CTRL, ROWS>(INT_MAX, idx);
  argmax_combine(v, idx, w, wi);
}
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
  argmax_step<0xb1>(v, idx);
  argmax_step<0x4e>(v, idx);
  argmax_step<0x141>(v, idx);
  argmax_step<0x140>(v, idx);
  argmax_step<0x142, 0xa>(v, idx);
  argmax_step<0x143, 0xc>(v, idx);
  v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  idx = __builtin_amdgcn_readlane(idx, 63);
}

// Row-wide reductions for the per-row functions below.  WaveRed: the row is
// held by one wave64.  BlockRed: the row is held by a whole block of NW waves;
// each reduction runs on the DPP network within a wave and then over the
// waves in wave order through LDS (every thread forms the same total), with
// barriers, so every thread of the block must take part in each call.
struct WaveRed {
  __device__ float sum(float v) const { return wave_sum(v); }
  __device__ float max(float v) const { return wave_max(v); }
  __device__ void argmax(float& v, int& idx) const { wave_argmax(v, idx); }
  __device__ bool any(bool b) const { return __any(b); }
  // The value `v` of the row's first thread (lane 0).
  __device__ float first(float v) const { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)); }
};

template <int NW>
struct BlockRed {
  float* f;  // NW floats of LDS
  int* n;    // NW ints of LDS

  __device__ float combine(float v, bool is_max) const {
    const int w = threadIdx.x >> 6;
    __syncthreads();  // the previous reduction's values have been read
    if ((threadIdx.x & 63) == 0) f[w] = v;
    __syncthreads();
    float t = f[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) t = is_max ? (f[k] > t ? f[k] : t) : t + f[k];
    return t;
  }
  __device__ float sum(float v) const { return combine(wave_sum(v), false); }
  __device__ float max(float v) const { return combine(wave_max(v), true); }
  __device__ void argmax(float& v, int& idx) const {
    wave_argmax(v, idx);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      f[w] = v;
      n[w] = idx;
    }
    __syncthreads();
    v = f[0];
    idx = n[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) argmax_combine(v, idx, f[k], n[k]);
  }
  __device__ bool any(bool b) const { return __syncthreads_or(b ? 1 : 0) != 0; }
  __device__ float first(float v) const {
    __syncthreads();
    if (threadIdx.x == 0) f[0] = v;
    __syncthreads();
    return f[0];
  }
};

// Row argmax with the reference's sequential rule (python/orca/nn/model.py:65-75):
// best starts at r[0]; a later value replaces it only if strictly greater.
// Lanes propose their first strict maximum over c >= 1 (NaN never proposes);
// the winner beats r[0] only if strictly greater, and a NaN r[0] is never beaten.
// col(j) is the column of the thread's j-th value, increasing in j; column 0 is
// value 0 of the row's first thread.
template <int VPL, class Get, class Col, class Valid, class R = WaveRed>
__device__ __forceinline__ int row_argmax(Get get, Col col, Valid valid, const R& red = R()) {
  float bv = -INFINITY;
  int bi = INT_MAX;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = col(j);
    if (c >= 1 && valid(j)) {
      float v = get(j);
      if (v == v && (bi == INT_MAX || v > bv)) {
        bv = v;
        bi = c;
      }
    }
  }
  red.argmax(bv, bi);
  const float first = red.first(get(0));
  if (bi == INT_MAX) return 0;
  return (bv > first) ? bi : 0;
}

struct CeRowOut {
  float loss;  // -sum_c t_c (p_c - lse): the row's term of the loss before the 1/B mean
  int pred;    // argmax of the logits
  int target;  // target class (label, or argmax of the one-hot row)
  // ce_row_label only: whether this thread holds `loss` (one thread of the row does);
  // pred and target are held by every thread.
  bool has_loss = true;
};

// One row held by one wave64: x[j] is the logit of column col(j), used where
// valid(j) (the column is < C), tval(j) its target.  Writes element j of the row of
// dL/dlogits through store(j, value) when `grad`.  Every lane returns the
// same values.
//
// The gradient is the tape's, element by element, through the 22-node
// composition (seed * (1/B), * -1, * target, the identity expands' 0 + g,
// the g / see of LogBackward, the full-gradient-to-ties MaxToShapeBackward).
// LogBackward's row sum sum_c (0 + g_lse_c) / se is taken as
// (sum_c (0 + g_lse_c)) / se when se is finite and positive: for one-hot
// targets only the target's term is nonzero, so the two are the same f32
// value; other rows keep one division per element.
template <int VPL, class TVal, class Col, class Valid, class Store, class R = WaveRed>
__device__ __forceinline__ CeRowOut ce_row(const float (&x)[VPL], Valid valid, TVal tval, Col col, bool labels,
                                           int label, float inv_b, bool grad, Store store, bool want_argmax,
                                           const R& red = R()) {
  float e[VPL];
  // max_to_shape (init -FLT_MAX, strict >)
  float mx = -FLT_MAX;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid(j) && x[j] > mx) mx = x[j];
  mx = red.max(mx);
  // exp(p - max) and its row sum
  float se = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    e[j] = valid(j) ? ce_exp(x[j] - mx) : 0.0f;
    se = se + e[j];
  }
  se = red.sum(se);
  const float lg = logf(fmaxf(se, 1e-7f));
  const float lse = mx + lg;
  // per-row loss: sum_c -(t * (p - lse))
  float pb = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid(j)) pb = pb + (tval(j) * (x[j] - lse)) * -1.0f;
  pb = red.sum(pb);

  if (grad) {
    const float g_tm = inv_b * -1.0f;
    float gse = 0.0f;
    if (se > 0.0f && se <= FLT_MAX) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (valid(j)) gse = gse + (0.0f + (0.0f + ((g_tm * tval(j)) * -1.0f)));
      gse = red.sum(gse) / se;
    } else {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (valid(j)) {
          float g_lse = 0.0f + ((g_tm * tval(j)) * -1.0f);
          gse = gse + (0.0f + g_lse) / se;
        }
      gse = red.sum(gse);
    }
    float gmx = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (valid(j)) {
        float g_lse = 0.0f + ((g_tm * tval(j)) * -1.0f);
        float g_sh = gse * e[j];
        gmx = gmx + ((0.0f + g_lse) + (0.0f + (g_sh * -1.0f)));
      }
    gmx = red.sum(gmx);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (valid(j)) {
        float g_ls = g_tm * tval(j);
        float g_sh = gse * e[j];
        float d = (0.0f + g_ls) + (0.0f + g_sh);
        float g3 = 0.0f;
        if (x[j] == mx) g3 = g3 + gmx;
        store(j, d + g3);
      }
    }
  }

  CeRowOut out{pb, 0, 0};
  if (want_argmax) {
    out.pred = row_argmax<VPL>([&](int j) { return x[j]; }, col, valid, red);
    out.target = labels ? label : row_argmax<VPL>(tval, col, valid, red);
  }
  return out;
}

// ce_row for class-index targets, t_c = [c == label]: the same f32 operations
// element by element, without materialising t.  Every term a zero target
// contributes to the row sums (the loss term and LogBackward's sum) is +0,
// which leaves a sum unchanged, so those sums are formed from the label's term
// alone (on its lane; +0 elsewhere) with the same bits as the full sums.  A
// label outside [0, C) leaves every target zero, as its one-hot row would.
//
// x is overwritten with exp(x - max): a thread holds one array of row values
// instead of two, so more rows are resident per CU (more loads in flight).
// What later steps need of x is kept on the side: the label's logit, a bit
// mask of the columns equal to the max, and for the check below the lane's
// smallest value and whether it holds a non-finite one.  reload(j) reads
// x[j] again from memory for rows whose loss terms are irregular.  jl is this
// lane's slot of the label column (col(jl) == label, valid), or -1;
// label_valid says whether some thread of the row has jl >= 0 (0 <= label < C).
// Two of the row sums have one nonzero term, the label's, so they need no
// reduction: the loss term is 0 + pl, held by the label's thread (a row
// without a label column has +0, held by the first thread), and LogBackward's
// sum is 0 + g_lse_t or +0, known to every thread.
template <int VPL, class Col, class Valid, class Store, class Reload, class R = WaveRed>
__device__ __forceinline__ CeRowOut ce_row_label(float (&x)[VPL], Valid valid, Col col, Reload reload, int label,
                                                 int jl, bool label_valid, bool first, float inv_b, bool grad,
                                                 Store store, bool want_argmax, const R& red = R()) {
  static_assert(VPL <= 32, "the max mask holds one bit per value");
  float mx = -FLT_MAX, xmin = FLT_MAX, xl = 0.0f;
  bool nonfinite = false;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid(j)) {
      if (x[j] > mx) mx = x[j];
      xmin = fminf(xmin, x[j]);
      nonfinite = nonfinite || !(fabsf(x[j]) <= FLT_MAX);
      if (j == jl) xl = x[j];
    }
  CeRowOut out{0.0f, 0, label};
  if (want_argmax) out.pred = row_argmax<VPL>([&](int j) { return x[j]; }, col, valid, red);
  mx = red.max(mx);
  float se = 0.0f;
  unsigned at_max = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const float e = valid(j) ? ce_exp(x[j] - mx) : 0.0f;
    if (valid(j) && x[j] == mx) at_max |= 1u << j;
    x[j] = e;
    se = se + e;
  }
  se = red.sum(se);
  const float lg = logf(fmaxf(se, 1e-7f));
  const float lse = mx + lg;
  // A zero target's loss term (0 * (x - lse)) * -1 is +-0 only while x - lse
  // is finite; with an infinite or NaN difference it is NaN, and the full sum
  // is formed as the reference forms it.  The max element's term exp(0) = 1
  // makes se >= 1, so lse >= max >= x and x - lse <= 0 for every finite x:
  // all differences are finite exactly when the lane's values are finite and
  // the smallest difference is (x - lse is monotone in x).
  const float pl = jl >= 0 ? (1.0f * (xl - lse)) * -1.0f : 0.0f;
  const bool irregular = valid(0) && (nonfinite || !(fabsf(xmin - lse) <= FLT_MAX));
  if (red.any(irregular)) {
    float s = 0.0f;
#pragma unroll 1
    for (int j = 0; j < VPL; ++j)  // one reload at a time: the rare path adds no register pressure
      if (valid(j)) s = s + ((j == jl ? 1.0f : 0.0f) * (reload(j) - lse)) * -1.0f;
    out.loss = red.sum(s);
    out.has_loss = first;
  } else {
    out.loss = 0.0f + pl;
    out.has_loss = jl >= 0 || (!label_valid && first);
  }

  if (grad) {
    const float g_tm = inv_b * -1.0f;
    const float g_lse_t = 0.0f + ((g_tm * 1.0f) * -1.0f);  // the label's 0 + ((g_tm * t) * -1)
    const float g_lse_0 = 0.0f + ((g_tm * 0.0f) * -1.0f);  // any other column's (+0)
    float gse;
    if (se > 0.0f && se <= FLT_MAX) {
      gse = (label_valid ? 0.0f + g_lse_t : 0.0f) / se;
    } else {
      gse = 0.0f;
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (valid(j)) gse = gse + (0.0f + (j == jl ? g_lse_t : g_lse_0)) / se;
      gse = red.sum(gse);
    }
    // gse is +0, positive, +inf or NaN and e[j] is in [0, 1] or NaN, so
    // g_sh = gse * e[j] is never negative and never -0.  Then, exactly:
    //   (0 + g_lse) + (0 + (g_sh * -1)) = 0 - g_sh          (zero target: g_lse = +0)
    //   (0 + g_ls) + (0 + g_sh)         = g_sh              (zero target: g_ls = -0)
    //   d + g3 = d where x != max (g3 = +0 and d is never -0),
    // and the target column keeps the full expressions.
    const float g_lse_c = 0.0f + g_lse_t;
    float gmx = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (valid(j)) {
        const float t = 0.0f - gse * x[j];
        gmx = gmx + (j == jl ? g_lse_c + t : t);
      }
    gmx = red.sum(gmx);
    const float g3 = 0.0f + gmx;
    const float g_ls_c = 0.0f + g_tm * 1.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (valid(j)) {
        const float g_sh = gse * x[j];
        const float d = j == jl ? g_ls_c + g_sh : g_sh;
        store(j, (at_max >> j) & 1u ? d + g3 : d);
      }
    }
  }
  return out;
}

}  // namespace orca_hip
