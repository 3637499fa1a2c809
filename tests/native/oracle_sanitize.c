/*
 * CPU sanitizer run of the oracle (its C sources): every entry point on small
 * inputs, with ragged shapes, rank-3 broadcasts, each GEMM summation order and
 * the error returns, built with -fsanitize=address,undefined by
 * tests/test_native_sanitize.py.  Test infrastructure only.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "orca_oracle.h"

#define CHECK(cond)                                                      \
  do {                                                                   \
    if (!(cond)) {                                                       \
      fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
      abort();                                                           \
    }                                                                    \
  } while (0)

static float* filled(size_t n, unsigned seed) {
  float* p = (float*)malloc(sizeof(float) * (n ? n : 1));
  for (size_t i = 0; i < n; ++i) {
    seed = seed * 1103515245u + 12345u;
    p[i] = (float)((int)(seed >> 16) % 2001 - 1000) / 500.0f;
  }
  return p;
}

static void elementwise(void) {
  const size_t n = 1001;
  float *a = filled(n, 1), *b = filled(n, 2), *o = filled(n, 3);
  for (size_t i = 0; i < n; ++i) b[i] = b[i] == 0.0f ? 1.0f : b[i];
  orc_add(a, b, o, n); orc_sub(a, b, o, n); orc_mul(a, b, o, n); orc_div(a, b, o, n);
  orc_mul_scalar(a, -1.0f, o, n); orc_relu(a, o, n); orc_relu_backward(a, b, o, n);
  orc_sigmoid(a, o, n); orc_sigmoid_backward(a, b, o, n); orc_exp(a, o, n); orc_log(a, o, n);
  orc_exp_backward(a, b, o, n); orc_log_backward(a, b, o, n); orc_sqrt(b, o, n);
  orc_sqrt_backward(a, b, o, n); orc_div_backward_lhs(a, b, o, n); orc_div_backward_rhs(a, a, b, o, n);
  orc_accumulate_grad(a, b, o, n);
  CHECK(!orc_has_nan_or_inf(a, n));
  a[n - 1] = INFINITY;
  CHECK(orc_has_nan_or_inf(a, n));
  CHECK(!orc_has_nan_or_inf(a, 0));
  free(a); free(b); free(o);
}

static void shapes(void) {
  const size_t in3[3] = {4, 1, 3}, out4[4] = {2, 4, 5, 3}, r2[2] = {6, 5}, col[2] = {1, 5}, row[2] = {6, 1},
               one[1] = {1}, bad[2] = {6, 4};
  float *x = filled(12, 4), *y = filled(120, 5), *z = filled(30, 6), *w = filled(30, 7);
  CHECK(orc_expand(x, y, in3, 3, out4, 4) == ORC_OK);
  CHECK(orc_sum_to_shape(z, w, r2, 2, col, 2) == ORC_OK);
  CHECK(orc_sum_to_shape(z, w, r2, 2, row, 2) == ORC_OK);
  CHECK(orc_sum_to_shape(z, w, r2, 2, one, 1) == ORC_OK);
  CHECK(orc_max_to_shape(z, w, r2, 2, row, 2) == ORC_OK);
  float g[6], m[6];
  CHECK(orc_max_to_shape(z, m, r2, 2, row, 2) == ORC_OK);
  for (int i = 0; i < 6; ++i) g[i] = 1.0f;
  CHECK(orc_max_to_shape_backward(g, z, m, w, r2, 2, row, 2) == ORC_OK);
  CHECK(orc_transpose(z, w, r2, 2, 0, 1) == ORC_OK);
  CHECK(orc_expand(z, w, r2, 2, bad, 2) != ORC_OK);  /* not broadcastable */
  free(x); free(y); free(z); free(w);
}

static void gemms(void) {
  const size_t ad[3] = {3, 5, 7}, bd[3] = {3, 7, 2}, bd_bad[3] = {3, 6, 2}, bd_rank[2] = {7, 2};
  float *a = filled(105, 8), *b = filled(42, 9), *c = filled(30, 10);
  for (int v = 0; v < 4; ++v) {
    orc_set_gemm_variant(v);
    CHECK(orc_matmul(a, b, c, ad, 3, bd, 3) == ORC_OK);
    const size_t m2[2] = {130, 257}, k2[2] = {257, 67};
    float *p = filled(130 * 257, 11), *q = filled(257 * 67, 12), *r = filled(130 * 67, 13);
    CHECK(orc_matmul(p, q, r, m2, 2, k2, 2) == ORC_OK);
    free(p); free(q); free(r);
  }
  orc_set_gemm_variant(0);
  CHECK(orc_matmul(a, b, c, ad, 3, bd_bad, 3) == ORC_ERR_SHAPE);
  CHECK(orc_matmul(a, b, c, ad, 3, bd_rank, 2) == ORC_ERR_SHAPE);
  free(a); free(b); free(c);
}

static void training(void) {
  const size_t dims[4] = {20, 12, 9, 5}, B = 7, L = 3;
  float* params[6];
  float* grads[6];
  float* ms[6];
  float* vs[6];
  for (size_t l = 0; l < L; ++l) {
    params[2 * l] = filled(dims[l] * dims[l + 1], 20 + (unsigned)l);
    params[2 * l + 1] = filled(dims[l + 1], 30 + (unsigned)l);
  }
  for (int i = 0; i < 6; ++i) {
    const size_t n = i % 2 ? dims[i / 2 + 1] : dims[i / 2] * dims[i / 2 + 1];
    grads[i] = filled(n, 40);
    ms[i] = (float*)calloc(n, sizeof(float));
    vs[i] = (float*)calloc(n, sizeof(float));
  }
  float *x = filled(B * dims[0], 50), *onehot = (float*)calloc(B * dims[3], sizeof(float));
  for (size_t r = 0; r < B; ++r) onehot[r * dims[3] + r % dims[3]] = 1.0f;
  float losses[3], logits[7 * 5];
  int32_t preds[7];
  int64_t correct = 0, t = 0;
  orc_opt sgd = {0, 0.1, 0.0, 0.0, 0.9, 0.999, 1e-8}, adamw = {1, 1e-3, 0.0, 0.01, 0.9, 0.999, 1e-8};
  CHECK(orc_mlp_train(dims, L, B, params, NULL, NULL, NULL, x, onehot, &sgd, 2, losses, grads, logits, preds,
                      &correct) == ORC_OK);
  CHECK(orc_mlp_train(dims, L, B, params, ms, vs, &t, x, onehot, &adamw, 3, losses, grads, logits, preds,
                      &correct) == ORC_OK);
  CHECK(t == 3);
  float loss, dl[7 * 5];
  CHECK(orc_cross_entropy(logits, onehot, B, dims[3], &loss, dl) == ORC_OK);
  orc_argmax_rows(logits, B, dims[3], preds);
  orc_adamw_update(params[0], grads[0], ms[0], vs[0], dims[0] * dims[1], &adamw, 4);
  orc_sgd_update(params[1], grads[1], dims[1], &sgd);
  for (int i = 0; i < 6; ++i) {
    free(params[i]); free(grads[i]); free(ms[i]); free(vs[i]);
  }
  free(x); free(onehot);
}

int main(void) {
  elementwise();
  shapes();
  gemms();
  training();
  printf("oracle sanitizer run: all checks passed (%d threads)\n", orc_num_threads());
  return 0;
}
