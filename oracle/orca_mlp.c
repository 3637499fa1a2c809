/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, one MLP training step in the exact
 * op order the reference executes.
 *
 * Forward follows python/orca/nn/linear.py:74-79 (x @ W, then bias.expand,
 * then `out + b`, whose PyO3 __add__ expands BOTH operands,
 * orca-python/src/lib.rs:513-528), python/orca/nn/activation.py (relu) and
 * python/orca/nn/loss.py:71-96 (composed cross-entropy; `-x` is x * -1,
 * orca-python/src/lib.rs:642-658; `mean` is sum * (1/n as f32), lib.rs:664-669).
 * Backward replays the tape in reverse recording order
 * (orca-autograd/src/tape.rs:107-118) with the backward rules of
 * orca-autograd/src/backend.rs:1379-1793; a node receiving several
 * contributions sums them in arrival order with accumulate_grad
 * (tape.rs:34-47).  Identity expands (shape already equal) are exact copies
 * forward, and their backward is sum_to_shape onto the same shape, i.e.
 * 0 + g.  The update follows python/orca/optim/sgd.py:46-79 and
 * python/orca/optim/adamw.py:48-99 with the f64 scalars rounded to f32 as PyO3
 * does when it extracts `Operand::Scalar(f32)` (orca-python/src/lib.rs:12-16).
 */
#include "orca_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float* falloc(size_t n) { return (float*)malloc((n ? n : 1) * sizeof(float)); }

/* sum_to_shape onto the same shape: 0 + g (the identity ExpandBackward). */
static void identity_sum(const float* g, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = 0.0f + g[i];
}

/* Row-wise sum_to_shape([B,C] -> [B,1]), ascending input order. */
static void row_sum(const float* in, float* out, size_t B, size_t C) {
  size_t in_d[2] = {B, C}, out_d[2] = {B, 1};
  orc_sum_to_shape(in, out, in_d, 2, out_d, 2);
}

/* expand([B,1] -> [B,C]). */
static void row_expand(const float* in, float* out, size_t B, size_t C) {
  size_t in_d[2] = {B, 1}, out_d[2] = {B, C};
  orc_expand(in, out, in_d, 2, out_d, 2);
}

int orc_cross_entropy(const float* p, const float* t, size_t B, size_t C, float* loss, float* dp) {
  size_t n = B * C;
  float *mx = falloc(B), *mxe = falloc(n), *sh = falloc(n), *e = falloc(n), *se = falloc(B);
  float *see = falloc(n), *lg = falloc(n), *lse = falloc(n), *ls = falloc(n), *tm = falloc(n);
  float *nm = falloc(n), *pb = falloc(B), *s = falloc(1);
  float *g1 = falloc(n), *g2 = falloc(n), *g3 = falloc(n), *gb = falloc(B), *gm1 = falloc(n);
  int rc = ORC_ERR_INTERNAL;
  if (!mx || !mxe || !sh || !e || !se || !see || !lg || !lse || !ls || !tm || !nm || !pb || !s || !g1 ||
      !g2 || !g3 || !gb || !gm1)
    goto done;
  size_t pd[2] = {B, C}, rd[2] = {B, 1}, sd[1] = {1};

  /* ---- forward (loss.py:74-96) ---- */
  orc_max_to_shape(p, mx, pd, 2, rd, 2); /* c1 */
  row_expand(mx, mxe, B, C);             /* c2 */
  orc_sub(p, mxe, sh, n);                /* c3,c4 identity expands; c5 */
  orc_exp(sh, e, n);                     /* c6 */
  row_sum(e, se, B, C);                  /* c7 */
  row_expand(se, see, B, C);             /* c8 */
  orc_log(see, lg, n);                   /* c9 */
  orc_add(mxe, lg, lse, n);              /* c10,c11; c12 */
  orc_sub(p, lse, ls, n);                /* c13,c14; c15 */
  orc_mul(t, ls, tm, n);                 /* c16 (target: no node), c17; c18 */
  orc_mul_scalar(tm, -1.0f, nm, n);      /* c19 */
  row_sum(nm, pb, B, C);                 /* c20 */
  orc_sum_to_shape(pb, s, rd, 2, sd, 1); /* c21 */
  float inv_n = 1.0f / (float)B;         /* lib.rs:667, num_elements of [B,1] */
  orc_mul_scalar(s, inv_n, loss, 1);     /* c22 */

  /* ---- backward, reverse recording order ---- */
  float gs = 1.0f * inv_n;                                     /* c22: seed 1 * (1/B) */
  for (size_t b = 0; b < B; ++b) gb[b] = gs;                   /* c21: expand [1] -> [B,1] */
  row_expand(gb, g1, B, C);                                    /* c20: expand -> [B,C] */
  orc_mul_scalar(g1, -1.0f, g2, n);                            /* c19 */
  orc_mul(g2, t, g1, n);                                       /* c18: grad_rhs = g * lhs_primal */
  identity_sum(g1, g2, n);                                     /* c17: g_ls */
  /* c15 Sub: lhs -> c13 gets g_ls, rhs -> c14 gets -g_ls */
  orc_mul_scalar(g2, -1.0f, g3, n);
  identity_sum(g3, g1, n);                                     /* c14: g_lse */
  identity_sum(g2, dp, n);                                     /* c13: first contribution to p */
  /* c12 Add: c10 and c11 both get g_lse; c11 -> g_lg, c10 -> first contribution to mxe */
  identity_sum(g1, g2, n);                                     /* c11: g_lg */
  identity_sum(g1, gm1, n);                                    /* c10: g_mxe (first) */
  orc_log_backward(g2, see, g3, n);                            /* c9: g / see */
  row_sum(g3, gb, B, C);                                       /* c8: ExpandBackward se->see */
  row_expand(gb, g1, B, C);                                    /* c7: SumToShapeBackward */
  orc_exp_backward(g1, e, g2, n);                              /* c6: g * e */
  /* c5 Sub: lhs -> c3 gets g_sh, rhs -> c4 gets -g_sh */
  orc_mul_scalar(g2, -1.0f, g3, n);
  identity_sum(g3, g1, n);                                     /* c4 */
  orc_accumulate_grad(gm1, g1, gm1, n);                        /* mxe: first + second */
  identity_sum(g2, g3, n);                                     /* c3 */
  orc_accumulate_grad(dp, g3, dp, n);                          /* p: first + second */
  row_sum(gm1, gb, B, C);                                      /* c2: ExpandBackward mx->mxe */
  orc_max_to_shape_backward(gb, p, mx, g1, pd, 2, rd, 2);      /* c1 */
  orc_accumulate_grad(dp, g1, dp, n);                          /* p: + third */
  rc = ORC_OK;
done:
  free(mx); free(mxe); free(sh); free(e); free(se); free(see); free(lg); free(lse); free(ls);
  free(tm); free(nm); free(pb); free(s); free(g1); free(g2); free(g3); free(gb); free(gm1);
  return rc;
}

/* sgd.py:74-79: update = g * f32(lr); new = p - update (identity expands). */
void orc_sgd_update(float* p, const float* g, size_t n, const orc_opt* opt) {
  float lr = (float)opt->lr;
  float* upd = falloc(n);
  if (!upd) return;
  orc_mul_scalar(g, lr, upd, n);
  orc_sub(p, upd, p, n);
  free(upd);
}

/* adamw.py:71-94 -- each Python-level op is one f32 pass. */
void orc_adamw_update(float* p, const float* g, float* m, float* v, size_t n, const orc_opt* opt,
                      int64_t t) {
  const float decay = (float)(1.0 - opt->lr * opt->weight_decay);
  const float b1 = (float)opt->beta1, omb1 = (float)(1.0 - opt->beta1);
  const float b2 = (float)opt->beta2, omb2 = (float)(1.0 - opt->beta2);
  const float c1 = (float)(1.0 / (1.0 - pow(opt->beta1, (double)t)));
  const float c2 = (float)(1.0 / (1.0 - pow(opt->beta2, (double)t)));
  const float eps = (float)opt->eps, lr = (float)opt->lr;
  float *d = falloc(n), *a = falloc(n), *b = falloc(n), *mh = falloc(n), *vh = falloc(n);
  if (!d || !a || !b || !mh || !vh) goto done;
  orc_mul_scalar(p, decay, d, n); /* p * (1 - lr*wd) */
  orc_mul_scalar(m, b1, a, n);    /* m * b1 */
  orc_mul_scalar(g, omb1, b, n);  /* g * (1 - b1) */
  orc_add(a, b, m, n);            /* m_new */
  orc_mul_scalar(v, b2, a, n);    /* v * b2 */
  orc_mul(g, g, b, n);            /* g * g */
  orc_mul_scalar(b, omb2, b, n);  /* * (1 - b2) */
  orc_add(a, b, v, n);            /* v_new */
  orc_mul_scalar(m, c1, mh, n);   /* m_hat */
  orc_mul_scalar(v, c2, vh, n);   /* v_hat */
  orc_sqrt(vh, a, n);             /* sqrt(v_hat) */
  for (size_t i = 0; i < n; ++i) b[i] = eps; /* Tensor.scalar(eps).expand */
  orc_add(a, b, a, n);            /* denom */
  orc_div(mh, a, b, n);           /* m_hat / denom */
  orc_mul_scalar(b, lr, b, n);    /* * lr */
  orc_sub(d, b, p, n);            /* decayed - update */
done:
  free(d); free(a); free(b); free(mh); free(vh);
}

int orc_mlp_train(const size_t* dims, size_t L, size_t B, float** params, float** m, float** v,
                  int64_t* t, const float* x, const float* onehot, const orc_opt* opt, int steps,
                  float* losses, float** grads_out, float* logits_out, int32_t* preds, int64_t* correct) {
  if (L == 0 || L > 64 || steps < 0) return ORC_ERR_INTERNAL;
  if (opt->kind == 0 && (opt->momentum != 0.0 || opt->weight_decay != 0.0)) return ORC_ERR_INTERNAL;
  if (opt->kind == 1 && (!m || !v || !t)) return ORC_ERR_INTERNAL;
  const size_t C = dims[L];
  float* pre[64];  /* h_l = a W + b (pre-activation; logits for the last layer) */
  float* act[64];  /* relu(h_l) for l < L-1 */
  float* grads[128];
  memset(pre, 0, sizeof(pre));
  memset(act, 0, sizeof(act));
  memset(grads, 0, sizeof(grads));
  size_t maxw = 0;
  for (size_t l = 0; l <= L; ++l) maxw = dims[l] > maxw ? dims[l] : maxw;
  float *tmp1 = falloc(B * maxw), *tmp2 = falloc(B * maxw), *g = falloc(B * maxw);
  float *ga = falloc(B * maxw), *wt = NULL, *at = NULL;
  int rc = ORC_ERR_INTERNAL;
  if (!tmp1 || !tmp2 || !g || !ga) goto done;
  for (size_t l = 0; l < L; ++l) {
    pre[l] = falloc(B * dims[l + 1]);
    act[l] = falloc(B * dims[l + 1]);
    grads[2 * l] = falloc(dims[l] * dims[l + 1]);
    grads[2 * l + 1] = falloc(dims[l + 1]);
    if (!pre[l] || !act[l] || !grads[2 * l] || !grads[2 * l + 1]) goto done;
  }
  wt = falloc(maxw * maxw);
  at = falloc(B * maxw);
  if (!wt || !at) goto done;

  for (int step = 0; step < steps; ++step) {
    /* ---- forward ---- */
    const float* a = x;
    for (size_t l = 0; l < L; ++l) {
      size_t K = dims[l], N = dims[l + 1];
      size_t ad[2] = {B, K}, wd[2] = {K, N}, bd[2] = {1, N}, od[2] = {B, N};
      if (orc_matmul(a, params[2 * l], tmp1, ad, 2, wd, 2)) goto done;  /* n1 */
      orc_expand(params[2 * l + 1], tmp2, bd, 2, od, 2);                /* n2 */
      orc_add(tmp1, tmp2, pre[l], B * N);                               /* n3,n4 identity; n5 */
      if (l + 1 < L) orc_relu(pre[l], act[l], B * N);                   /* n6 */
      a = (l + 1 < L) ? act[l] : pre[l];
    }
    float loss;
    if (orc_cross_entropy(pre[L - 1], onehot, B, C, &loss, g)) goto done;
    if (losses) losses[step] = loss;
    if (step + 1 == steps) {
      if (logits_out) memcpy(logits_out, pre[L - 1], sizeof(float) * B * C);
      if (preds || correct) {
        int32_t* pr = (int32_t*)malloc(sizeof(int32_t) * B);
        int32_t* tg = (int32_t*)malloc(sizeof(int32_t) * B);
        if (!pr || !tg) { free(pr); free(tg); goto done; }
        orc_argmax_rows(pre[L - 1], B, C, pr);
        orc_argmax_rows(onehot, B, C, tg);
        int64_t c = 0;
        for (size_t b = 0; b < B; ++b) c += pr[b] == tg[b];
        if (preds) memcpy(preds, pr, sizeof(int32_t) * B);
        if (correct) *correct = c;
        free(pr);
        free(tg);
      }
    }

    /* ---- backward: g holds dL/dh_{L-1} ---- */
    for (size_t l = L; l-- > 0;) {
      size_t K = dims[l], N = dims[l + 1];
      size_t od[2] = {B, N}, bd[2] = {1, N};
      /* n5 Add -> n3 and n4 both receive g */
      identity_sum(g, tmp1, B * N);                                      /* n4: g_be */
      identity_sum(g, tmp2, B * N);                                      /* n3: g_z */
      orc_sum_to_shape(tmp1, grads[2 * l + 1], od, 2, bd, 2);            /* n2: bias grad */
      const float* a = (l == 0) ? x : act[l - 1];
      size_t wdims[2] = {K, N}, tdims[2] = {N, K}, adims[2] = {B, K}, atd[2] = {K, B};
      if (l > 0) {                                                       /* n1 lhs: g_a = g_z W^T */
        orc_transpose(params[2 * l], wt, wdims, 2, 0, 1);
        if (orc_matmul(tmp2, wt, ga, od, 2, tdims, 2)) goto done;
      }
      orc_transpose(a, at, adims, 2, 0, 1);                              /* n1 rhs: g_W = a^T g_z */
      if (orc_matmul(at, tmp2, grads[2 * l], atd, 2, od, 2)) goto done;
      if (l > 0) orc_relu_backward(ga, pre[l - 1], g, B * K);            /* previous layer's n6 */
    }

    /* ---- update, parameter order W1, b1, W2, b2, ... (module.py:32-44) ---- */
    if (opt->kind == 1) *t += 1; /* adamw.py:64 */
    for (size_t i = 0; i < 2 * L; ++i) {
      size_t n = (i % 2 == 0) ? dims[i / 2] * dims[i / 2 + 1] : dims[i / 2 + 1];
      if (opt->kind == 0)
        orc_sgd_update(params[i], grads[i], n, opt);
      else
        orc_adamw_update(params[i], grads[i], m[i], v[i], n, opt, *t);
    }
  }
  if (grads_out)
    for (size_t i = 0; i < 2 * L; ++i) {
      size_t n = (i % 2 == 0) ? dims[i / 2] * dims[i / 2 + 1] : dims[i / 2 + 1];
      if (grads_out[i]) memcpy(grads_out[i], grads[i], sizeof(float) * n);
    }
  rc = ORC_OK;
done:
  for (size_t l = 0; l < L; ++l) {
    free(pre[l]);
    free(act[l]);
    free(grads[2 * l]);
    free(grads[2 * l + 1]);
  }
  free(tmp1); free(tmp2); free(g); free(ga); free(wt); free(at);
  return rc;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
