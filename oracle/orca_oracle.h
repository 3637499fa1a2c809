/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the Orca MLP training-step path.
 *
 * This is a C restatement of the reference CPU backend (`orca-backend-cpu`),
 * the autograd tape order (`orca-autograd`) and the Python frontend op
 * sequence (`python/orca/nn`, `python/orca/optim`) for the MLP training step.
 * It exists only to check the HIP backend.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product library never links
 * or calls it.
 *
 * Pinning (see tests/test_oracle.py):
 *   - reference known-answer tests: orca-autograd/tests/autograd_tests.rs:39-50
 *     and :70-87, python/tests/test_api.py:33-61, 196-218, 250-279, 323-346;
 *   - closed forms: CE grad = (softmax - t)/B, equal logits => loss = ln C,
 *     AdamW first step from zero moments, SGD p - lr*g, bias grad = column sums;
 *   - exact-arithmetic GEMM on small integers, fp64 brute force, finite
 *     differences (examples/basics/test_grad_check.py:6-47).
 * `orc_matmul` follows the reference's call contract but not matrixmultiply's
 * blocking order (unpinned third-party order; tolerance only).
 */
#ifndef ORCA_ORACLE_H
#define ORCA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the HIP library's C-ABI. */
#define ORC_OK 0
#define ORC_ERR_SHAPE (-1)
#define ORC_ERR_INTERNAL (-5)

/* ---- elementwise (orca-backend-cpu/src/backend.rs) ---- */
void orc_add(const float* a, const float* b, float* out, size_t n);        /* 104-128 */
void orc_sub(const float* a, const float* b, float* out, size_t n);        /* 291-315 */
void orc_mul(const float* a, const float* b, float* out, size_t n);        /* 340-373 */
void orc_div(const float* a, const float* b, float* out, size_t n);        /* 635-659 */
void orc_mul_scalar(const float* a, float s, float* out, size_t n);        /* 317-338 */
void orc_relu(const float* a, float* out, size_t n);                       /* 375-390 */
void orc_relu_backward(const float* g, const float* x, float* out, size_t n); /* 414-438 */
void orc_sigmoid(const float* a, float* out, size_t n);                    /* 392-412 */
void orc_sigmoid_backward(const float* g, const float* y, float* out, size_t n); /* 440-464 */
void orc_exp(const float* a, float* out, size_t n);                        /* 549-564 */
void orc_log(const float* a, float* out, size_t n);                        /* 566-581 */
void orc_exp_backward(const float* g, const float* y, float* out, size_t n); /* 583-607 */
void orc_log_backward(const float* g, const float* x, float* out, size_t n); /* 609-633 */
void orc_sqrt(const float* a, float* out, size_t n);                       /* 661-676 */
void orc_sqrt_backward(const float* g, const float* y, float* out, size_t n); /* 734-759 */
void orc_div_backward_lhs(const float* g, const float* r, float* out, size_t n); /* 678-701 */
void orc_div_backward_rhs(const float* g, const float* l, const float* r, float* out, size_t n); /* 703-732 */
void orc_accumulate_grad(const float* a, const float* b, float* out, size_t n); /* 761-774 */
int orc_has_nan_or_inf(const float* a, size_t n);                          /* 1316-1334 */

/* ---- shape ops ---- */
int orc_expand(const float* in, float* out, const size_t* in_dims, size_t in_rank,
               const size_t* out_dims, size_t out_rank);                   /* 466-497 */
int orc_sum_to_shape(const float* in, float* out, const size_t* in_dims, size_t in_rank,
                     const size_t* out_dims, size_t out_rank);             /* 499-530 */
int orc_max_to_shape(const float* in, float* out, const size_t* in_dims, size_t in_rank,
                     const size_t* out_dims, size_t out_rank);             /* 1336-1381 */
int orc_max_to_shape_backward(const float* g, const float* x, const float* y, float* out,
                              const size_t* in_dims, size_t in_rank,
                              const size_t* out_dims, size_t out_rank);    /* 1383-1435 */
int orc_transpose(const float* in, float* out, const size_t* dims, size_t rank,
                  size_t d0, size_t d1);                                   /* 223-289 */
int orc_matmul(const float* a, const float* b, float* out, const size_t* a_dims, size_t a_rank,
               const size_t* b_dims, size_t b_rank);                       /* 130-221 */

/* ---- MLP training step: the reference's op order (linear.py:77-86 forward, loss.py:59-100, tape.rs:107-118 reverse walk) ---- */
typedef struct {
  int kind;            /* 0 = SGD, 1 = AdamW */
  double lr;
  double momentum;     /* SGD: must be 0 (configs use vanilla SGD) */
  double weight_decay; /* SGD: must be 0; AdamW: decoupled decay */
  double beta1, beta2, eps;
} orc_opt;

/*
 * Runs `steps` training steps of the MLP dims[0] -> dims[1] -> ... -> dims[L]
 * (ReLU between layers, softmax cross-entropy on one-hot targets) on a fixed
 * batch.  params[2l] is W_l [dims[l], dims[l+1]], params[2l+1] is b_l
 * [1, dims[l+1]]; both are updated in place.  m/v hold AdamW moments (in/out,
 * may be NULL for SGD); *t is AdamW's step counter (in/out).
 * Optional outputs (NULL to skip):
 *   losses[steps]           loss of each step (before that step's update)
 *   grads[2L]               gradients of the LAST step
 *   logits[batch*dims[L]]   logits of the LAST step
 *   preds[batch], *correct  argmax of the last step's logits and accuracy count
 * Returns ORC_OK or an error code.
 */
int orc_mlp_train(const size_t* dims, size_t n_layers, size_t batch, float** params,
                  float** m, float** v, int64_t* t, const float* x, const float* onehot,
                  const orc_opt* opt, int steps, float* losses, float** grads, float* logits,
                  int32_t* preds, int64_t* correct);

/* Composed cross-entropy forward/backward alone on logits [B,C] with one-hot
 * targets (python/orca/nn/loss.py:59-100 + the tape's reverse walk).  Outputs
 * the loss and dL/dlogits. */
int orc_cross_entropy(const float* logits, const float* onehot, size_t B, size_t C,
                      float* loss, float* dlogits);

/* First-max-wins argmax per row (python/orca/nn/model.py:65-75). */
void orc_argmax_rows(const float* x, size_t B, size_t C, int32_t* out);

/* One AdamW / SGD update of a single flat tensor with the reference's op
 * order (python/orca/optim/adamw.py:66-99, sgd.py:46-79). */
void orc_adamw_update(float* p, const float* g, float* m, float* v, size_t n, const orc_opt* opt,
                      int64_t t);
void orc_sgd_update(float* p, const float* g, size_t n, const orc_opt* opt);

/* Selects the GEMM summation order (0 = blocked f32 with FMA, 1 = f64-accumulated
 * dot products, 2 = ascending f32, 3 = descending f32 with FMA); used to measure
 * the spread between valid orders. */
void orc_set_gemm_variant(int variant);

/* Thread count of the OpenMP elementwise ops. */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
