/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, elementwise and shape ops.
 *
 * Restates orca-backend-cpu/src/backend.rs op by op for f32 (line numbers
 * cite that file).  Elementwise ops are parallel over elements like the
 * reference's rayon `par_iter` (the result of each element does not depend on
 * the split).  Shape ops (expand, sum_to_shape, max_to_shape, transpose) are
 * sequential in row-major input order exactly as the reference loops.
 * Compiled with -ffp-contract=off so no multiply-add is fused, matching the
 * reference's separate f32 operations.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline may load this library.
 */
#include "orca_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define PAR_THRESHOLD 32768

#define ELEMENTWISE(n, body)                                        \
  do {                                                              \
    ptrdiff_t n_ = (ptrdiff_t)(n);                                  \
    _Pragma("omp parallel for if (n_ > PAR_THRESHOLD) schedule(static)") \
    for (ptrdiff_t i = 0; i < n_; ++i) { body; }                    \
  } while (0)

void orc_add(const float* a, const float* b, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] + b[i]); }
void orc_sub(const float* a, const float* b, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] - b[i]); }
void orc_mul(const float* a, const float* b, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] * b[i]); }
void orc_div(const float* a, const float* b, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] / b[i]); }
void orc_mul_scalar(const float* a, float s, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] * s); }

/* backend.rs:386 -- `if val > 0 { val } else { zero }`: NaN and -0 give +0. */
void orc_relu(const float* a, float* out, size_t n) { ELEMENTWISE(n, out[i] = a[i] > 0.0f ? a[i] : 0.0f); }

/* backend.rs:434 -- the mask comes from the pre-activation input. */
void orc_relu_backward(const float* g, const float* x, float* out, size_t n) {
  ELEMENTWISE(n, out[i] = x[i] > 0.0f ? g[i] : 0.0f);
}

/* backend.rs:408 */
void orc_sigmoid(const float* a, float* out, size_t n) { ELEMENTWISE(n, out[i] = 1.0f / (1.0f + expf(-a[i]))); }

/* backend.rs:460 -- g * y * (1 - y), left to right. */
void orc_sigmoid_backward(const float* g, const float* y, float* out, size_t n) {
  ELEMENTWISE(n, out[i] = (g[i] * y[i]) * (1.0f - y[i]));
}

/* backend.rs:560 */
void orc_exp(const float* a, float* out, size_t n) { ELEMENTWISE(n, out[i] = expf(a[i])); }

/* backend.rs:577 -- ln(max(x, 1e-7)); f32::max returns the non-NaN operand. */
void orc_log(const float* a, float* out, size_t n) { ELEMENTWISE(n, out[i] = logf(fmaxf(a[i], 1e-7f))); }

/* backend.rs:603 */
void orc_exp_backward(const float* g, const float* y, float* out, size_t n) { ELEMENTWISE(n, out[i] = g[i] * y[i]); }

/* backend.rs:629 -- g / x with no clamp. */
void orc_log_backward(const float* g, const float* x, float* out, size_t n) { ELEMENTWISE(n, out[i] = g[i] / x[i]); }

/* backend.rs:672 */
void orc_sqrt(const float* a, float* out, size_t n) { ELEMENTWISE(n, out[i] = sqrtf(a[i])); }

/* backend.rs:755 */
void orc_sqrt_backward(const float* g, const float* y, float* out, size_t n) {
  ELEMENTWISE(n, out[i] = g[i] / (2.0f * y[i]));
}

/* backend.rs:697 */
void orc_div_backward_lhs(const float* g, const float* r, float* out, size_t n) { ELEMENTWISE(n, out[i] = g[i] / r[i]); }

/* backend.rs:728 -- g * (-l / (r * r)). */
void orc_div_backward_rhs(const float* g, const float* l, const float* r, float* out, size_t n) {
  ELEMENTWISE(n, out[i] = g[i] * (-l[i] / (r[i] * r[i])));
}

/* backend.rs:768-770 -- sequential lhs + rhs. */
void orc_accumulate_grad(const float* a, const float* b, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* backend.rs:1325-1333 */
int orc_has_nan_or_inf(const float* a, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(a[i])) return 1;
  return 0;
}

/* ---------------------------------------------------------------- shapes */

#define MAX_RANK 16

static size_t numel(const size_t* d, size_t r) {
  size_t n = 1;
  for (size_t i = 0; i < r; ++i) n *= d[i];
  return n;
}

/* backend.rs:17-26 -- pad with leading ones; a longer shape yields all ones. */
static void pad_left(const size_t* d, size_t r, size_t target, size_t* out) {
  for (size_t i = 0; i < target; ++i) out[i] = 1;
  if (r <= target)
    for (size_t i = 0; i < r; ++i) out[target - r + i] = d[i];
}

/* backend.rs:28-36 */
static void strides_of(const size_t* d, size_t r, size_t* s) {
  size_t cur = 1;
  for (size_t i = r; i-- > 0;) {
    s[i] = cur;
    cur *= d[i];
  }
}

/* backend.rs:466-497 */
int orc_expand(const float* in, float* out, const size_t* in_dims, size_t in_rank,
               const size_t* out_dims, size_t out_rank) {
  if (out_rank > MAX_RANK || in_rank > MAX_RANK) return ORC_ERR_INTERNAL;
  size_t pin[MAX_RANK], st[MAX_RANK];
  pad_left(in_dims, in_rank, out_rank, pin);
  for (size_t d = 0; d < out_rank; ++d)
    if (pin[d] != 1 && pin[d] != out_dims[d]) return ORC_ERR_SHAPE; /* reference would index out of bounds */
  strides_of(pin, out_rank, st);
  size_t n = numel(out_dims, out_rank);
  for (size_t i = 0; i < n; ++i) {
    size_t rem = i, idx = 0;
    for (size_t d = out_rank; d-- > 0;) {
      size_t c = rem % out_dims[d];
      rem /= out_dims[d];
      if (pin[d] != 1) idx += c * st[d];
    }
    out[i] = in[idx];
  }
  return ORC_OK;
}

/* backend.rs:499-530 -- accumulate into zeros in ascending row-major input order. */
int orc_sum_to_shape(const float* in, float* out, const size_t* in_dims, size_t in_rank,
                     const size_t* out_dims, size_t out_rank) {
  if (out_rank > MAX_RANK || in_rank > MAX_RANK) return ORC_ERR_INTERNAL;
  size_t pout[MAX_RANK], st[MAX_RANK];
  pad_left(out_dims, out_rank, in_rank, pout);
  for (size_t d = 0; d < in_rank; ++d)
    if (pout[d] != 1 && pout[d] != in_dims[d]) return ORC_ERR_SHAPE;
  strides_of(pout, in_rank, st);
  size_t n_out = numel(out_dims, out_rank);
  for (size_t i = 0; i < n_out; ++i) out[i] = 0.0f;
  size_t n = numel(in_dims, in_rank);
  for (size_t i = 0; i < n; ++i) {
    size_t rem = i, idx = 0;
    for (size_t d = in_rank; d-- > 0;) {
      size_t c = rem % in_dims[d];
      rem /= in_dims[d];
      if (pout[d] != 1) idx += c * st[d];
    }
    out[idx] = out[idx] + in[i];
  }
  return ORC_OK;
}

/* Shared index map of max_to_shape and its backward (backend.rs:1347-1367). */
static int max_map_setup(const size_t* in_dims, size_t in_rank, const size_t* out_dims, size_t out_rank,
                         size_t* pout, size_t* st) {
  if (out_rank > in_rank || in_rank > MAX_RANK) return ORC_ERR_SHAPE;
  pad_left(out_dims, out_rank, in_rank, pout);
  for (size_t d = 0; d < in_rank; ++d)
    if (pout[d] != 1 && pout[d] != in_dims[d]) return ORC_ERR_SHAPE;
  strides_of(pout, in_rank, st);
  return ORC_OK;
}

static size_t max_map(size_t i, const size_t* in_dims, size_t in_rank, const size_t* pout, const size_t* st) {
  size_t rem = i, idx = 0;
  for (size_t d = in_rank; d-- > 0;) {
    size_t c = rem % in_dims[d];
    rem /= in_dims[d];
    if (pout[d] != 1) idx += c * st[d];
  }
  return idx;
}

/* backend.rs:1336-1381 -- init f32::MIN, strict `>` so NaN never wins. */
int orc_max_to_shape(const float* in, float* out, const size_t* in_dims, size_t in_rank,
                     const size_t* out_dims, size_t out_rank) {
  size_t pout[MAX_RANK], st[MAX_RANK];
  int rc = max_map_setup(in_dims, in_rank, out_dims, out_rank, pout, st);
  if (rc) return rc;
  size_t n_out = numel(out_dims, out_rank);
  for (size_t i = 0; i < n_out; ++i) out[i] = -FLT_MAX;
  size_t n = numel(in_dims, in_rank);
  for (size_t i = 0; i < n; ++i) {
    size_t o = max_map(i, in_dims, in_rank, pout, st);
    if (in[i] > out[o]) out[o] = in[i];
  }
  return ORC_OK;
}

/* backend.rs:1383-1435 -- every element equal to its max gets the full gradient. */
int orc_max_to_shape_backward(const float* g, const float* x, const float* y, float* out,
                              const size_t* in_dims, size_t in_rank, const size_t* out_dims,
                              size_t out_rank) {
  size_t pout[MAX_RANK], st[MAX_RANK];
  int rc = max_map_setup(in_dims, in_rank, out_dims, out_rank, pout, st);
  if (rc) return rc;
  size_t n = numel(in_dims, in_rank);
  for (size_t i = 0; i < n; ++i) {
    size_t o = max_map(i, in_dims, in_rank, pout, st);
    out[i] = 0.0f;
    if (x[i] == y[o]) out[i] = out[i] + g[o];
  }
  return ORC_OK;
}

/* backend.rs:223-289 -- permuted copy, output-index driven. */
int orc_transpose(const float* in, float* out, const size_t* dims, size_t rank, size_t d0, size_t d1) {
  if (d0 >= rank || d1 >= rank || rank > MAX_RANK) return ORC_ERR_INTERNAL;
  size_t od[MAX_RANK], is[MAX_RANK], os[MAX_RANK];
  for (size_t i = 0; i < rank; ++i) od[i] = dims[i];
  od[d0] = dims[d1];
  od[d1] = dims[d0];
  strides_of(dims, rank, is);
  strides_of(od, rank, os);
  size_t n = numel(dims, rank);
  for (size_t o = 0; o < n; ++o) {
    size_t cur = o, idx = 0;
    for (size_t i = 0; i < rank; ++i) {
      size_t c = cur / os[i];
      cur %= os[i];
      size_t src = (i == d0) ? d1 : (i == d1) ? d0 : i;
      idx += c * is[src];
    }
    out[o] = in[idx];
  }
  return ORC_OK;
}

/* First maximum wins on strict `>` (python/orca/nn/model.py:65-75). */
void orc_argmax_rows(const float* x, size_t B, size_t C, int32_t* out) {
  for (size_t b = 0; b < B; ++b) {
    const float* r = x + b * C;
    size_t best = 0;
    float bv = r[0];
    for (size_t c = 1; c < C; ++c)
      if (r[c] > bv) {
        bv = r[c];
        best = c;
      }
    out[b] = (int32_t)best;
  }
}
