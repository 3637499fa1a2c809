/*
 * orca_hip.h -- C ABI of the MI355X (gfx950) backend for Orca.
 *
 * The reference plugs compute backends in through the Rust `Backend` trait
 * (orca-tensor/src/backend.rs:19-315) whose storages are opaque, cheaply
 * cloned handles that every op borrows and every op returns anew.  This
 * header is the FFI a Rust `HipBackend: Backend` binds: each `orca_hip_<op>`
 * below stands in for the trait method named in its comment, takes the same
 * logical shape / dtype arguments, and returns a NEW device buffer through
 * `out` (allocated from the context's stream-ordered caching allocator; the
 * caller releases it with orca_hip_free, which is what the Rust storage's
 * Drop does).  Inputs are never modified.
 *
 * Error behaviour mirrors orca_core::OrcaError (orca-core/src/error.rs:5-31):
 * every function returns 0 or a negative ORCA_HIP_ERR_* code naming the
 * variant, and orca_hip_last_error() returns the message (thread-local).
 * No function throws across the ABI.
 *
 * All work is enqueued on the context's single in-order HIP stream; only the
 * host-reading calls (to_f32_vec, d2h, has_nan_or_inf, *_read_*) synchronise.
 * Element type on the path is f32 (DType::F32 = 0); other dtypes return
 * ORCA_HIP_ERR_UNSUPPORTED_DTYPE, like the reference's dispatch macros.
 */
#ifndef ORCA_HIP_H
#define ORCA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (orca-core/src/error.rs:5-31) ---- */
#define ORCA_HIP_OK 0
#define ORCA_HIP_ERR_SHAPE (-1)              /* OrcaError::ShapeMismatch */
#define ORCA_HIP_ERR_UNSUPPORTED_DTYPE (-2)  /* OrcaError::UnsupportedDType */
#define ORCA_HIP_ERR_DTYPE_MISMATCH (-3)     /* OrcaError::DTypeMismatch */
#define ORCA_HIP_ERR_DEVICE_MISMATCH (-4)    /* OrcaError::DeviceMismatch */
#define ORCA_HIP_ERR_INTERNAL (-5)           /* OrcaError::InternalError */

/* ---- dtype codes, in orca_core::DType order (orca-core/src/dtype.rs:5-22) ---- */
#define ORCA_HIP_F32 0
#define ORCA_HIP_F64 1
#define ORCA_HIP_F16 2
#define ORCA_HIP_BF16 3
#define ORCA_HIP_I32 4
#define ORCA_HIP_I64 5
#define ORCA_HIP_U8 6
#define ORCA_HIP_BOOL 7

/* Layout of a matmul operand's storage.  TRANSPOSED means the buffer holds
 * the operand with its last two dims swapped: a lazy `transpose` view as
 * produced for MatMulBackward (orca-autograd/src/backend.rs:1467-1495). */
#define ORCA_HIP_VIEW_CONTIGUOUS 0
#define ORCA_HIP_VIEW_TRANSPOSED 1

typedef struct orca_hip_ctx orca_hip_ctx;
typedef struct orca_hip_mlp orca_hip_mlp;
typedef struct orca_hip_event orca_hip_event;

/* ======================= context, memory, host I/O ======================= */

/* Creates a context on HIP device `device` with its own stream and caching
 * allocator.  Replaces GpuBackend::new (orca-backend-gpu/src/backend.rs:53-211)
 * as the process-global backend behind global_backend_gpu()
 * (orca-python/src/lib.rs:23-33). */
int orca_hip_ctx_create(int device, orca_hip_ctx** out);
int orca_hip_ctx_destroy(orca_hip_ctx* ctx);
/* Message of the calling thread's last failure ("" if none). */
const char* orca_hip_last_error(void);
/* The calling thread's last failure as the fields of its orca_core::OrcaError variant
 * (orca-core/src/error.rs:5-31), so a binding can rebuild the variant itself:
 * ShapeMismatch {op, expected, got}; UnsupportedDType {op, dtype}; DTypeMismatch {op,
 * expected = dtype, got = dtype_got}; DeviceMismatch(device 0, device 1) with each device as
 * kind (0 Cpu, 1 Cuda, 2 Gpu; orca-core/src/device.rs:5-12) and index; InternalError(message).
 * Fields a failure does not know are "" or -1.  The strings stay valid until the thread's
 * next failing call. */
typedef struct {
  int code;              /* ORCA_HIP_OK or ORCA_HIP_ERR_* */
  const char* op;
  const char* expected;
  const char* got;
  int dtype;             /* ORCA_HIP_F32 ... */
  int dtype_got;
  int device_kind[2];
  int device_index[2];
  const char* message;   /* the whole message, as orca_hip_last_error */
} orca_hip_error_info;
int orca_hip_last_error_info(orca_hip_error_info* out);
/* Backend::device (orca-tensor/src/backend.rs:25): the HIP ordinal, reported
 * as Device::Gpu(ordinal) so orca-python routes "gpu"/"cuda" here
 * (orca-python/src/lib.rs:91-93). */
int orca_hip_device(const orca_hip_ctx* ctx, int* ordinal);

/* Stream-ordered caching allocator (replaces MemoryPool,
 * orca-backend-gpu/src/pool.rs:8-71).  Blocks are 256-byte aligned; a freed
 * block is reused by later work on the same stream without a hipMalloc. */
int orca_hip_alloc(orca_hip_ctx* ctx, size_t bytes, void** out);
int orca_hip_free(orca_hip_ctx* ctx, void* ptr);
/* orca_hip_free of each of ptrs[0..n) in order (no counterpart in the reference: for a
 * binding that releases dropped storages in batches, one call instead of one per storage). */
int orca_hip_free_many(orca_hip_ctx* ctx, void* const* ptrs, size_t n);
/* Returns cached blocks to the device (synchronises first). */
int orca_hip_empty_cache(orca_hip_ctx* ctx);
/* live bytes, cached bytes, and the number of hipMalloc calls so far. */
int orca_hip_mem_stats(orca_hip_ctx* ctx, size_t* live, size_t* cached, size_t* device_allocs);

int orca_hip_h2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes); /* synchronous */
int orca_hip_d2h(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes); /* synchronous */
int orca_hip_d2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes); /* stream-ordered */
int orca_hip_fill(orca_hip_ctx* ctx, float* dst, float value, size_t n);       /* stream-ordered kernel */
int orca_hip_sync(orca_hip_ctx* ctx);
/* Number of host waits on this context's work so far (every stream or event
 * synchronisation the library performed, including the host-reading calls).
 * No counterpart in the reference: it lets a caller check that a span of calls,
 * such as a backward pass and an optimizer step, never waited for the device. */
int orca_hip_sync_count(const orca_hip_ctx* ctx, uint64_t* count);

/* A second stream per context, and events that order the two.  No counterpart in
 * the reference, whose backend runs on one queue: a binding uses them to run an
 * optimizer update of parameters whose gradients are complete beside the backward's
 * remaining products.  orca_hip_use_side_stream(ctx, b) with b != 0 sends the context's
 * later launches to the side stream, (ctx, 0) back to the context stream.  Host reads and
 * orca_hip_sync first make the context stream wait for the side stream's work.  While
 * launches go to the side stream, every entry point that allocates device memory (its
 * result, or a workspace) fails with ORCA_HIP_ERR_INTERNAL: the caching allocator orders
 * the reuse of a block by the context stream alone, so only non-allocating launches (the
 * orca_hip_adamw_multi / orca_hip_sgd_multi passes, orca_hip_ew_program into buffers
 * allocated beforehand, event records and waits) may run there.
 * orca_hip_event_record marks the current stream's work so far; orca_hip_event_wait
 * makes the current stream wait for such a mark (no host wait); orca_hip_event_release
 * hands the event back for reuse (waits already enqueued are unaffected).  An optimizer pass
 * or elementwise program launched on the side stream takes at most b blocks per CU when
 * b > 0 (room for a product that fills the CUs beside it) and its full grid when b < 0. */
int orca_hip_use_side_stream(orca_hip_ctx* ctx, int blocks_per_cu);
int orca_hip_event_record(orca_hip_ctx* ctx, orca_hip_event** out);
int orca_hip_event_wait(orca_hip_ctx* ctx, orca_hip_event* ev);
int orca_hip_event_release(orca_hip_ctx* ctx, orca_hip_event* ev);

/* =========================== Backend trait ops =========================== */
/* `shape`/`rank` are the logical shape (Shape, orca-core/src/shape.rs:6).
 * `out` receives a new buffer of the result's element count. */

/* Backend::zeros (backend.rs:27) */
int orca_hip_zeros(orca_hip_ctx* ctx, const size_t* shape, size_t rank, int dtype, void** out);
/* Backend::from_f32_slice (backend.rs:30-31); n must equal the shape's elements.
 * Stream-ordered without a host wait: up to 1 KiB travels as a kernel argument,
 * more through the context's pinned staging ring; `data` may be reused on return. */
int orca_hip_from_f32_slice(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const float* data,
                            size_t n, void** out);
/* Backend::to_f32_vec (backend.rs:34): copies n floats to host (synchronises) */
int orca_hip_to_f32_vec(orca_hip_ctx* ctx, const void* storage, size_t n, float* host_out);
/* Backend::from_bytes / to_bytes (backend.rs:296-297), f32 payload; from_bytes
 * uploads like from_f32_slice (no host wait), to_bytes synchronises. */
int orca_hip_from_bytes(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const uint8_t* bytes,
                        size_t n_bytes, int dtype, void** out);
int orca_hip_to_bytes(orca_hip_ctx* ctx, const void* storage, size_t n_bytes, uint8_t* host_out);

/* Backend::matmul (backend.rs:38-45): batched (..., M, K) x (..., K, N) with
 * equal leading dims; lhs_view/rhs_view say whether a buffer holds its
 * operand transposed (ORCA_HIP_VIEW_*). */
int orca_hip_matmul(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* lhs_shape,
                    size_t lhs_rank, const size_t* rhs_shape, size_t rhs_rank, int dtype, int lhs_view,
                    int rhs_view, void** out);
/* Backend::matmul of rank-2 operands (backend.rs:38-45) together with
 * Backend::sum_to_shape(rhs, [K, N] -> [1, N]) (backend.rs:499-530): C = op(lhs) x rhs
 * ([M, K] x [K, N]; lhs_view as above, rhs contiguous) and colsum[n] = sum_k rhs[k][n] in
 * ascending k, the bits sum_to_shape produces.  One call serves MatMulBackward's
 * grad_W = X^T x G and ExpandBackward's bias gradient of the same G
 * (orca-autograd/src/backend.rs:1467-1495, 1684-1697): the column sum rides on
 * the product's loads of G. */
int orca_hip_matmul_colsum(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N,
                           int lhs_view, int dtype, void* colsum, void** out);
/* orca_hip_matmul of rank-2 operands (colsum NULL; either view) or orca_hip_matmul_colsum
 * (colsum non-null; rhs contiguous), and, when done != NULL, an event (*done) that completes
 * with the product's last launch: that launch records it itself when it is the pipelined
 * MFMA kernel, so no marker runs between the product and the next launch; otherwise it is
 * recorded right after.  Give it back with orca_hip_event_release.  No reference
 * counterpart (the reference's backends run on one queue): it lets work on the context's
 * second stream wait for exactly this product. */
int orca_hip_matmul_ev(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N,
                       int lhs_view, int rhs_view, int dtype, void* colsum, void** out, orca_hip_event** done);
/* Backend::transpose (backend.rs:48-55), materialised */
int orca_hip_transpose(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, size_t dim0,
                       size_t dim1, int dtype, void** out);

/* Backend::add / sub / mul / div (backend.rs:57-70, 80-86, 153-159) */
int orca_hip_add(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* shape, size_t rank,
                 int dtype, void** out);
int orca_hip_sub(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* shape, size_t rank,
                 int dtype, void** out);
int orca_hip_mul(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* shape, size_t rank,
                 int dtype, void** out);
int orca_hip_div(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* shape, size_t rank,
                 int dtype, void** out);
/* Backend::mul_scalar (backend.rs:71-77) */
int orca_hip_mul_scalar(orca_hip_ctx* ctx, const void* s, float scalar, const size_t* shape, size_t rank,
                        int dtype, void** out);
/* Backend::relu / sigmoid / exp / log / sqrt (backend.rs:87-93, 135-136, 160) */
int orca_hip_relu(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_sigmoid(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype,
                     void** out);
int orca_hip_exp(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_log(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_sqrt(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, void** out);
/* Backend::relu_backward (backend.rs:96-102): grad * [in_primal > 0] */
int orca_hip_relu_backward(orca_hip_ctx* ctx, const void* grad_out, const void* in_primal,
                           const size_t* shape, size_t rank, int dtype, void** out);
/* Backend::sigmoid_backward (backend.rs:103-109) */
int orca_hip_sigmoid_backward(orca_hip_ctx* ctx, const void* grad_out, const void* out_primal,
                              const size_t* shape, size_t rank, int dtype, void** out);
/* Backend::exp_backward / log_backward (backend.rs:137-150) */
int orca_hip_exp_backward(orca_hip_ctx* ctx, const void* grad_out, const void* out_primal,
                          const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_log_backward(orca_hip_ctx* ctx, const void* grad_out, const void* in_primal,
                          const size_t* shape, size_t rank, int dtype, void** out);
/* Backend::sqrt_backward / div_backward_lhs / div_backward_rhs (backend.rs:161-183) */
int orca_hip_sqrt_backward(orca_hip_ctx* ctx, const void* grad_out, const void* out_primal,
                           const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_div_backward_lhs(orca_hip_ctx* ctx, const void* grad_out, const void* rhs_primal,
                              const size_t* shape, size_t rank, int dtype, void** out);
int orca_hip_div_backward_rhs(orca_hip_ctx* ctx, const void* grad_out, const void* lhs_primal,
                              const void* rhs_primal, const size_t* shape, size_t rank, int dtype,
                              void** out);
/* Backend::accumulate_grad (backend.rs:185): lhs + rhs over n elements */
int orca_hip_accumulate_grad(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t n, void** out);

/* Backend::expand / sum_to_shape / reshape (backend.rs:112-133) */
int orca_hip_expand(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                    const size_t* out_shape, size_t out_rank, int dtype, void** out);
int orca_hip_sum_to_shape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, void** out);
int orca_hip_reshape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                     const size_t* out_shape, size_t out_rank, int dtype, void** out);
/* Backend::max_to_shape / max_to_shape_backward (backend.rs:299-314) */
int orca_hip_max_to_shape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, void** out);
int orca_hip_max_to_shape_backward(orca_hip_ctx* ctx, const void* grad_out, const void* in_primal,
                                   const void* out_primal, const size_t* in_shape, size_t in_rank,
                                   const size_t* out_shape, size_t out_rank, int dtype, void** out);
/* Backend::has_nan_or_inf (backend.rs:298); synchronises */
int orca_hip_has_nan_or_inf(orca_hip_ctx* ctx, const void* s, size_t n, int dtype, int* result);

/* ==================== storage handles: the Backend trait ==================== */
/* The drop-in form of the trait (orca-tensor/src/backend.rs:7-315): a backend object
 * owns the planning state a Rust `HipBackend` would otherwise have to keep above the
 * ABI, and every trait method is one call that takes and returns storage handles.
 *
 * A storage handle stands for `HipBackend::Storage`: reference counted (a binding's clone
 * either takes a reference of its own, orca_hip_storage_retain, or shares one among its
 * clones; the last holder's Drop is orca_hip_storage_release), immutable, and possibly not
 * yet computed.  Behind a handle the backend keeps, invisible to the tape
 * (orca-autograd/src/backend.rs records each op as usual):
 *   - lazy last-two-dims transposes: a view the next matmul reads with the transpose folded
 *     into its loads (MatMulBackward, orca-autograd/src/backend.rs:1467-1495);
 *   - elementwise ops (add ... div_backward_rhs, accumulate_grad, broadcasts, identity
 *     sum_to_shape / max_to_shape) left pending and run as one fused program at their first
 *     use (orca_hip_ew_program), writing every pending value that something else holds;
 *   - products left pending; when their first use is a GEMM epilogue (Linear's bias + ReLU,
 *     ReluBackward's mask) they run with it (orca_hip_gemm);
 *   - the bias gradient sum_to_shape([R, N] -> [1, N]) left pending until the weight
 *     gradient matmul of the same storage computes it (orca_hip_matmul_colsum), each
 *     storage's identity sum_to_shape computed once, and a row sum or maximum onto [R, 1]
 *     of a pending chain run in the chain's launch (orca_hip_ew_program_rows);
 *   - one-element uploads (the backward seed, scalars) kept on the host and applied as
 *     instruction scalars;
 *   - with the fused optimizer passes, the events that let part of an update run on the
 *     context's second stream.
 * Every value has the bits the ops run one by one would give.  Whether a pending value is
 * written out is decided by its reference count: a binding must release a handle as soon
 * as it drops it (as Rust's Drop and CPython's reference counting do).
 *
 * A backend and its storages are used under the backend's own lock, from any thread.  The
 * context must outlive the backend and every storage of it. */
typedef struct orca_hip_backend orca_hip_backend;
typedef struct orca_hip_storage orca_hip_storage;

typedef struct {
  int lazy;         /* elementwise ops and products pending (fused at first use); 0: every op runs at once */
  int deferred;     /* the identity memo, the pending bias column sums and the row reductions with their chain */
  int fold;         /* pending products run with their epilogue chain (needs lazy) */
  int overlap;      /* fused optimizer passes may run part of the update on the second stream */
  double side_frac; /* share of that part run beside the product after its gradients (0..1) */
  int side_bpc;     /* blocks per CU of that share (<= 0: the full grid) */
} orca_hip_backend_options;

/* Defaults: every switch on, side_frac 0.7, side_bpc 3 (the environment variables
 * ORCA_HIP_OVERLAP=0, ORCA_HIP_OPT_SIDE_FRAC=<percent>, ORCA_HIP_OPT_SIDE_BPC=<n> override them). */
int orca_hip_backend_default_options(orca_hip_backend_options* out);
/* Creates a backend on ctx (opts NULL: the defaults).  Replaces GpuBackend::new
 * (orca-backend-gpu/src/backend.rs:53-211) behind global_backend_gpu() (orca-python/src/lib.rs:23-33). */
int orca_hip_backend_create(orca_hip_ctx* ctx, const orca_hip_backend_options* opts, orca_hip_backend** out);
/* Drops the caller's reference; the backend goes when its last storage does. */
int orca_hip_backend_destroy(orca_hip_backend* be);

/* Storage::clone / Drop / len (orca-tensor/src/backend.rs:7-15). */
int orca_hip_storage_retain(orca_hip_storage* s);
int orca_hip_storage_release(orca_hip_storage* s);
int orca_hip_storage_len(const orca_hip_storage* s, size_t* n);
/* State flags of a storage (no counterpart in the reference; for tests and tools). */
#define ORCA_HIP_STORAGE_PENDING 1u     /* not computed yet */
#define ORCA_HIP_STORAGE_TRANSPOSED 2u  /* a lazy transpose view */
#define ORCA_HIP_STORAGE_MARKED 4u      /* written on the second stream; its first use waits there */
#define ORCA_HIP_STORAGE_CONSTANT 8u    /* a one-element value known on the host */
int orca_hip_storage_flags(const orca_hip_storage* s, uint32_t* flags);
/* The device address of a storage's values, computing them first (a transpose view gives
 * its untransposed buffer).  No counterpart in the reference: for interop and tests. */
int orca_hip_storage_device_ptr(orca_hip_backend* be, orca_hip_storage* s, void** ptr);

/* The Backend trait's 42 methods (orca-tensor/src/backend.rs:19-315), in its order.  Shapes
 * and dtypes as the trait passes them; `out` receives a new handle.  Off-path methods (conv2d*,
 * scatter / gather*, cast to another dtype) return ORCA_HIP_ERR_UNSUPPORTED_DTYPE. */
int orca_hip_trait_device(orca_hip_backend* be, int* kind, int* index);  /* Device::Gpu(ordinal) */
int orca_hip_trait_zeros(orca_hip_backend* be, const size_t* shape, size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_from_f32_slice(orca_hip_backend* be, const size_t* shape, size_t rank, const float* data, size_t n,
                                  orca_hip_storage** out);
int orca_hip_trait_to_f32_vec(orca_hip_backend* be, orca_hip_storage* s, float* host, size_t n);
int orca_hip_trait_matmul(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* lhs_shape,
                          size_t lhs_rank, const size_t* rhs_shape, size_t rhs_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_transpose(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, size_t dim0,
                             size_t dim1, int dtype, orca_hip_storage** out);
int orca_hip_trait_add(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_sub(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_mul_scalar(orca_hip_backend* be, orca_hip_storage* s, float scalar, const size_t* shape, size_t rank,
                              int dtype, orca_hip_storage** out);
int orca_hip_trait_mul(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_relu(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype,
                        orca_hip_storage** out);
int orca_hip_trait_sigmoid(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype,
                           orca_hip_storage** out);
/* relu_backward(grad, input), sigmoid_backward(grad, output): lhs is the gradient */
int orca_hip_trait_relu_backward(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                 size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_sigmoid_backward(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                    size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_expand(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_sum_to_shape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                                const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_reshape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                           const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_exp(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype,
                       orca_hip_storage** out);
int orca_hip_trait_log(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype,
                       orca_hip_storage** out);
/* (grad, output) */
int orca_hip_trait_exp_backward(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                size_t rank, int dtype, orca_hip_storage** out);
/* (grad, input) */
int orca_hip_trait_log_backward(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_div(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_sqrt(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype,
                        orca_hip_storage** out);
/* (grad, rhs primal) */
int orca_hip_trait_div_backward_lhs(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                    size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_div_backward_rhs(orca_hip_backend* be, orca_hip_storage* grad, orca_hip_storage* lhs,
                                    orca_hip_storage* rhs, const size_t* shape, size_t rank, int dtype,
                                    orca_hip_storage** out);
/* (grad, output) */
int orca_hip_trait_sqrt_backward(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                                 size_t rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_accumulate_grad(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs,
                                   orca_hip_storage** out);
/* conv2d and its backward (backend.rs:189-236): bias may be NULL (Option::None) */
int orca_hip_trait_conv2d(orca_hip_backend* be, orca_hip_storage* input, orca_hip_storage* weight,
                          orca_hip_storage* bias, const size_t* in_shape, size_t in_rank, const size_t* weight_shape,
                          size_t weight_rank, size_t padding, size_t stride, size_t dilation, size_t groups, int dtype,
                          orca_hip_storage** out);
int orca_hip_trait_conv2d_backward_input(orca_hip_backend* be, orca_hip_storage* grad_out, orca_hip_storage* weight,
                                         const size_t* in_shape, size_t in_rank, const size_t* weight_shape,
                                         size_t weight_rank, size_t padding, size_t stride, size_t dilation,
                                         size_t groups, int dtype, orca_hip_storage** out);
int orca_hip_trait_conv2d_backward_weight(orca_hip_backend* be, orca_hip_storage* grad_out, orca_hip_storage* input,
                                          const size_t* in_shape, size_t in_rank, const size_t* weight_shape,
                                          size_t weight_rank, size_t padding, size_t stride, size_t dilation,
                                          size_t groups, int dtype, orca_hip_storage** out);
int orca_hip_trait_conv2d_backward_bias(orca_hip_backend* be, orca_hip_storage* grad_out, const size_t* out_shape,
                                        size_t out_rank, int dtype, orca_hip_storage** out);
/* cast (backend.rs:239-245): f32 -> f32 returns the storage, anything else is unsupported */
int orca_hip_trait_cast(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int current_dtype,
                        int target_dtype, orca_hip_storage** out);
/* scatter / gather and their backward (backend.rs:248-293) */
int orca_hip_trait_scatter(orca_hip_backend* be, orca_hip_storage* s, size_t dim, orca_hip_storage* index,
                           orca_hip_storage* src, const size_t* shape, size_t rank, const size_t* index_shape,
                           size_t index_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_gather(orca_hip_backend* be, orca_hip_storage* s, size_t dim, orca_hip_storage* index,
                          const size_t* shape, size_t rank, const size_t* index_shape, size_t index_rank, int dtype,
                          orca_hip_storage** out);
int orca_hip_trait_scatter_backward_src(orca_hip_backend* be, orca_hip_storage* grad_out, size_t dim,
                                        orca_hip_storage* index, const size_t* shape, size_t rank,
                                        const size_t* index_shape, size_t index_rank, int dtype,
                                        orca_hip_storage** out);
int orca_hip_trait_scatter_backward_base(orca_hip_backend* be, orca_hip_storage* grad_out, size_t dim,
                                         orca_hip_storage* index, const size_t* shape, size_t rank,
                                         const size_t* index_shape, size_t index_rank, int dtype,
                                         orca_hip_storage** out);
int orca_hip_trait_gather_backward(orca_hip_backend* be, orca_hip_storage* grad_out, size_t dim,
                                   orca_hip_storage* index, const size_t* shape, size_t rank,
                                   const size_t* index_shape, size_t index_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_from_bytes(orca_hip_backend* be, const size_t* shape, size_t rank, const uint8_t* bytes,
                              size_t n_bytes, int dtype, orca_hip_storage** out);
/* to_bytes: the storage's len() * 4 bytes */
int orca_hip_trait_to_bytes(orca_hip_backend* be, orca_hip_storage* s, uint8_t* host, size_t n_bytes);
int orca_hip_trait_has_nan_or_inf(orca_hip_backend* be, orca_hip_storage* s, int dtype, int* result);
int orca_hip_trait_max_to_shape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                                const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out);
int orca_hip_trait_max_to_shape_backward(orca_hip_backend* be, orca_hip_storage* grad, orca_hip_storage* in_primal,
                                         orca_hip_storage* out_primal, const size_t* in_shape, size_t in_rank,
                                         const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out);

/* Inherent HipBackend methods beside the trait (no counterpart in the reference's trait, which
 * has no loss or optimizer op): the opt-in fused paths (nn.CrossEntropyLoss(fused=True),
 * optim.SGD / AdamW(fused=True)) call them when the backend has them. */
/* Mean softmax cross-entropy of [B, C] logits against one-hot targets and, if want_grad,
 * dL/dlogits for a loss seed of 1 (orca_hip_softmax_ce; python/orca/nn/loss.py:59-100). */
int orca_hip_be_softmax_ce(orca_hip_backend* be, orca_hip_storage* logits, orca_hip_storage* onehot, size_t B, size_t C,
                           int want_grad, orca_hip_storage** loss, orca_hip_storage** dlogits);
/* A new storage holding the same values (device to device). */
int orca_hip_be_clone(orca_hip_backend* be, orca_hip_storage* s, orca_hip_storage** out);
/* A flat arena of n floats (set to `value` when fill != 0); view: n floats at `offset` floats of
 * an arena (256-byte aligned when offset is a multiple of 64), sharing its memory;
 * copy_into: dst <- src, device to device, for a slice nothing reads yet. */
int orca_hip_be_arena(orca_hip_backend* be, size_t n, int fill, float value, orca_hip_storage** out);
int orca_hip_be_view(orca_hip_backend* be, orca_hip_storage* arena, size_t offset, size_t n, orca_hip_storage** out);
int orca_hip_be_copy_into(orca_hip_backend* be, orca_hip_storage* dst, orca_hip_storage* src);
/* *exclusive = 1 when no other handle, view or pending work refers to the arena's memory
 * (the caller's handle aside): it can be written without changing a value anybody holds. */
int orca_hip_be_arena_exclusive(orca_hip_backend* be, orca_hip_storage* arena, int* exclusive);
/* One optimizer pass over many parameters (orca_hip_adamw_multi / orca_hip_sgd_multi): rows of
 * (p_src, p_dst, g, m, v, n); p_dst, m and v are written in place (m, v NULL for SGD).  Values
 * derived lazily from the storages written are computed first.  With overlap, the rows whose
 * gradients a weight-gradient product made before the step's last one run on the second stream
 * right after that product; the storages they write carry its event, and their first use makes
 * the context stream wait for it (same kernel, same bits). */
typedef struct {
  orca_hip_storage* p_src;
  orca_hip_storage* p_dst;
  orca_hip_storage* g;
  orca_hip_storage* m;
  orca_hip_storage* v;
  size_t n;
} orca_hip_opt_row;
int orca_hip_be_adamw_multi(orca_hip_backend* be, const orca_hip_opt_row* rows, size_t n_rows, double lr, double beta1,
                            double beta2, double eps, double weight_decay, int64_t t);
int orca_hip_be_sgd_multi(orca_hip_backend* be, const orca_hip_opt_row* rows, size_t n_rows, double lr);
/* In place on p (and m, v): one parameter's update (orca_hip_adamw_step / orca_hip_sgd_step). */
int orca_hip_be_adamw_step(orca_hip_backend* be, orca_hip_storage* p, orca_hip_storage* g, orca_hip_storage* m,
                           orca_hip_storage* v, size_t n, double lr, double beta1, double beta2, double eps,
                           double weight_decay, int64_t t);
int orca_hip_be_sgd_step(orca_hip_backend* be, orca_hip_storage* p, orca_hip_storage* g, size_t n, double lr);

/* ================ fused elementwise programs (lazy trait ops) ================ */
/* The elementwise trait ops (Backend::add ... div_backward_rhs, accumulate_grad,
 * and sum_to_shape / max_to_shape onto the input's own shape) applied per
 * element as a straight-line program over registers, one launch for a whole
 * chain: the backend's storages defer elementwise ops and run them together
 * at their first non-elementwise use, which the tape never sees
 * (orca-autograd/src/backend.rs:74-118 records each op as usual).  Each
 * instruction is the same f32 operation as the op's own kernel, so results are
 * bit-identical to running the ops one by one. */
#define ORCA_HIP_EW_ADD 0          /* a + b (also accumulate_grad) */
#define ORCA_HIP_EW_SUB 1          /* a - b */
#define ORCA_HIP_EW_MUL 2          /* a * b */
#define ORCA_HIP_EW_DIV 3          /* a / b (also div_backward_lhs) */
#define ORCA_HIP_EW_MUL_SCALAR 4   /* a * scalar */
#define ORCA_HIP_EW_RELU 5         /* a > 0 ? a : 0 */
#define ORCA_HIP_EW_RELU_BW 6      /* b > 0 ? a : 0   (a = grad, b = input) */
#define ORCA_HIP_EW_EXP 7
#define ORCA_HIP_EW_LOG 8          /* ln(max(a, 1e-7)) */
#define ORCA_HIP_EW_SQRT 9
#define ORCA_HIP_EW_SIGMOID 10
#define ORCA_HIP_EW_EXP_BW 11      /* a * b   (b = output) */
#define ORCA_HIP_EW_LOG_BW 12      /* a / b   (b = input) */
#define ORCA_HIP_EW_SQRT_BW 13     /* a / (2 b) */
#define ORCA_HIP_EW_SIGMOID_BW 14  /* (a * b) * (1 - b) */
#define ORCA_HIP_EW_DIV_BW_RHS 15  /* a * (-b / (c * c)) */
#define ORCA_HIP_EW_SUM_VISIT 16   /* 0 + a   (sum_to_shape onto the same shape) */
#define ORCA_HIP_EW_MAX_VISIT 17   /* a > -FLT_MAX ? a : -FLT_MAX   (max_to_shape onto the same shape) */
#define ORCA_HIP_EW_COPY 18        /* a   (Backend::expand: the broadcast is the input's index map) */
#define ORCA_HIP_EW_ADD_SCALAR 19  /* a + scalar   (add of an expanded one-element constant) */
#define ORCA_HIP_EW_MAX_INPUTS 8
#define ORCA_HIP_EW_MAX_OUTPUTS 8
#define ORCA_HIP_EW_MAX_OPS 64
#define ORCA_HIP_EW_MAX_REGS 16

typedef struct {
  uint8_t op;       /* ORCA_HIP_EW_* */
  uint8_t dst;      /* register written */
  uint8_t a, b, c;  /* registers read (b, c when the op takes them) */
  uint8_t pad[3];
  float scalar;     /* ORCA_HIP_EW_MUL_SCALAR's factor, ORCA_HIP_EW_ADD_SCALAR's addend */
} orca_hip_ew_instr;

/* An input of a program: element e of the n reads ptr[(e / div) % mod], so a
 * plain input has div = 1, mod = n, and a broadcast of a contiguous block of
 * dims (Backend::expand, orca-backend-cpu/src/backend.rs:466-497: a bias row
 * [1, N] -> [B, N] is div = 1, mod = N; a column [B, 1] -> [B, N] is div = N,
 * mod = B; a single value is mod = 1) reads its mod values in place. */
typedef struct {
  const float* ptr;
  uint64_t div, mod;
} orca_hip_ew_input;

/* Runs one program over n elements: input i is loaded into register i, the
 * instructions run in order, and output o (n floats) receives register
 * out_regs[o].  No counterpart in the reference (its backend runs each op as
 * its own pass); the Backend trait's storages call it. */
int orca_hip_ew_program(orca_hip_ctx* ctx, size_t n, const orca_hip_ew_input* inputs, size_t n_inputs,
                        float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                        const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs);
/* orca_hip_ew_program over a [rows, cols] block (n = rows * cols), and in the same launch
 * reduced[r] = the sum (reduce_max = 0) or the maximum (reduce_max = 1) over row r of
 * register red_reg: Backend::sum_to_shape / max_to_shape of the program's value to
 * [rows, 1] (backend.rs:112-133, 299-314) with their bits -- a sum from +0 in ascending
 * column order, a maximum from -FLT_MAX that a value replaces only when greater.
 * 1 <= cols <= 64.  No reference counterpart: it runs a chain and the row reduction after
 * it (a loss's softmax) as one launch. */
int orca_hip_ew_program_rows(orca_hip_ctx* ctx, size_t rows, size_t cols, const orca_hip_ew_input* inputs,
                             size_t n_inputs, float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                             const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs, int red_reg,
                             int reduce_max, float* reduced);

/* Run-time compilation of fused programs.  No counterpart in the reference:
 * controls for callers that want to choose or observe how programs run.  A
 * program structure that recurs (same opcodes, operand registers, outputs and
 * input accesses; scalars and sizes may differ) is compiled by hipRTC into a
 * straight-line kernel with the same per-element functions, so the results
 * are the interpreter's bit for bit.  mode 0: interpret every program; 1
 * (default, or ORCA_HIP_EW_JIT at context creation): compile a structure at
 * its second use; 2: at its first.  Without hipRTC, or when a compile fails,
 * the structure stays on the interpreter. */
int orca_hip_ew_set_jit(orca_hip_ctx* ctx, int mode);
/* Launches so far on the interpreter and on compiled kernels, structures
 * compiled, and compiles that failed (any output may be null). */
int orca_hip_ew_jit_stats(orca_hip_ctx* ctx, uint64_t* interpreted, uint64_t* compiled_launches,
                          uint64_t* compiles, uint64_t* failures);
/* The HIP source compiled for a program over n elements (inputs' pointers are
 * not read), NUL-terminated into buf (len bytes; *needed = its full size + 1),
 * and the text of the functor header it includes as "ew_ops.hpp".  Needs no
 * GPU. */
int orca_hip_ew_jit_source(size_t n, const orca_hip_ew_input* inputs, size_t n_inputs, const uint8_t* out_regs,
                           size_t n_outputs, const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs,
                           char* buf, size_t len, size_t* needed);
int orca_hip_ew_jit_headers(const char** ew_ops_text);

/* ===================== fused kernels beyond the trait ===================== */
/* Buffer-level entry points: the caller owns every output buffer. */

/* GEMM epilogues. */
#define ORCA_HIP_EPI_NONE 0      /* C = acc */
#define ORCA_HIP_EPI_BIAS 1      /* C = acc + bias[n] */
#define ORCA_HIP_EPI_BIAS_RELU 2 /* C = relu(acc + bias[n])  (x > 0 ? x : 0) */
#define ORCA_HIP_EPI_RELU_MASK 3 /* C = mask[m][n] > 0 ? acc : 0  (ReLU backward on the product) */
#define ORCA_HIP_EPI_BIAS_RELU_PRE 4 /* pre[m][n] = acc + bias[n] and C = relu(pre)  (pre has C's ldc):
                                        a Linear + ReLU whose pre-activation is kept for ReLU backward */
#define ORCA_HIP_EPI_RELU_MASK_PRE 5 /* pre[m][n] = acc and C = mask[m][n] > 0 ? acc : 0: ReLU backward on a
                                        product that is kept as well (a gradient the tape holds) */

typedef struct {
  int kind;            /* ORCA_HIP_EPI_* */
  const float* bias;   /* [N] for EPI_BIAS / EPI_BIAS_RELU */
  const float* mask;   /* [M][ldmask] for EPI_RELU_MASK: the ReLU output (or pre-activation) */
  size_t ldmask;
  float* colsum;       /* optional [N]: column sums of op(B) over K in ascending k, the bits
                          sum_to_shape gives (bias gradient of dW = X^T dY) */
  float* pre;          /* [M][ldc] for EPI_BIAS_RELU_PRE (acc + bias) and EPI_RELU_MASK_PRE (acc) */
  orca_hip_event** done; /* optional: receives an event completing with the product's last launch,
                            as orca_hip_matmul_ev's (no reference counterpart) */
} orca_hip_epilogue;

/* C[M,N] = op(A)[M,K] . op(B)[K,N] in f32 on the fp32 MFMA units.
 * trans_a = 0: A is row-major [M][lda]; 1: A is stored [K][lda] (A^T).
 * trans_b = 0: B is row-major [K][ldb]; 1: B is stored [N][ldb] (B^T).
 * This is the Linear layer's three products: Y = X W (+b, ReLU) with (0,0),
 * dX = dY W^T (ReLU mask) with (0,1) and dW = X^T dY (+ bias colsum) with (1,0)
 * (MatMulBackward, orca-autograd/src/backend.rs:1449-1499). */
int orca_hip_gemm(orca_hip_ctx* ctx, int trans_a, int trans_b, size_t M, size_t N, size_t K, const float* A,
                  size_t lda, const float* B, size_t ldb, float* C, size_t ldc, const orca_hip_epilogue* epi);

/* The backward of a Linear with at most 16 outputs (a classifier head), as the separate
 * products compute it but from one grid: dW[K][C] = H^T G with H [B][K] and G [B][C]
 * (MatMulBackward's grad_W, orca-autograd/src/backend.rs:1467-1495), db[C] = the column sums
 * of G in ascending row order (ExpandBackward's sum_to_shape, 1684-1697; optional), and
 * dH[B][K] = G W^T with W [K][C] (grad_X) through an optional ReLU mask (mask[b][k] > 0, and
 * dH_pre = the unmasked product when non-null: orca_hip_gemm's EPI_RELU_MASK and
 * EPI_RELU_MASK_PRE).  Every value has the bits of orca_hip_matmul_colsum and orca_hip_gemm
 * computing them one by one: the same kernels' sums in one launch, plus the weight gradient's
 * slice reduction.  `done` (optional) as orca_hip_matmul_ev's.  Requires 1 <= C <= 16.  No
 * reference counterpart: it takes the launches of three trait calls. */
int orca_hip_narrow_linear_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* G, size_t C,
                                    const float* W, const float* mask, float* dH, float* dH_pre, float* dW, float* db,
                                    orca_hip_event** done);

/* Fused softmax cross-entropy forward + gradient, one wavefront per row
 * (replaces the ~21-op composition of python/orca/nn/loss.py:59-100 and its
 * tape backward).  Targets are either one-hot rows `onehot` [B][C] or class
 * indices `labels` [B] (exactly one non-NULL).  Writes, each optional:
 * loss[1] = mean over rows, dlogits[B][C] = dL/dlogits, preds[B] = first-max
 * argmax (python/orca/nn/model.py:65-75), correct[1] = #rows with
 * preds == target class.  All outputs are device pointers. */
int orca_hip_softmax_ce(orca_hip_ctx* ctx, const float* logits, size_t B, size_t C, const float* onehot,
                        const int32_t* labels, float* loss, float* dlogits, int32_t* preds, int64_t* correct);

/* Fused classifier head, forward: the last nn.Linear when it has at most 16
 * outputs, logits[B][C] = H[B][K] W[K][C] + bias (python/orca/nn/linear.py:77-86),
 * followed by everything orca_hip_softmax_ce computes (loss, dlogits, preds,
 * correct; each optional except logits), in one kernel that streams H once.
 * Requires 1 <= C <= 16, K a multiple of 4, H and W 16-byte aligned. */
int orca_hip_head_forward_ce(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W,
                             const float* bias, size_t C, const float* onehot, const int32_t* labels, float* logits,
                             float* loss, float* dlogits, int32_t* preds, int64_t* correct);
/* Its backward in one kernel that streams H once: dW[K][C] = H^T dlogits
 * (MatMulBackward, orca-autograd/src/backend.rs:1449-1499), db[C] = column sums
 * of dlogits (optional; ExpandBackward's sum_to_shape, 1684-1697) and, when
 * dH != NULL, dH[B][K] = dlogits W^T, times [H > 0] if relu_mask (ReluBackward
 * of the layer below, 1624-1646: H is its output).  Same shape rules as the
 * forward; dH 16-byte aligned. */
int orca_hip_head_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, size_t C,
                           const float* dlogits, int relu_mask, float* dH, float* dW, float* db);

/* dpre = grad * [pre > 0] and, if colsum != NULL, colsum[n] = sum over rows of
 * dpre (ReluBackward + the bias ExpandBackward's sum_to_shape,
 * orca-autograd/src/backend.rs:1633-1645, 1684-1697). */
int orca_hip_relu_bw_colsum(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                            float* dpre, float* colsum);
/* The same results as orca_hip_relu_bw_colsum, with no device allocation: no
 * counterpart in the reference (whose backends allocate freely); it is for
 * callers that cannot allocate -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The column-sum partials live in a
 * fixed device array of 2^20 floats (4 MiB) per GPU, held until the process
 * ends, so with colsum != NULL ceil(rows / 64) * cols must not exceed 1048576
 * (larger calls fail with ORCA_HIP_ERR_INTERNAL before anything is launched).
 * Every call on a GPU shares that GPU's array: a call's stream first waits on the
 * device (no host wait) for the work of the previous call that used it, from any
 * context or stream, so calls issued one after another on the host never overlap
 * on the array.  The array and that event are set up at a GPU's first call. */
int orca_hip_relu_bw_colsum_noalloc(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows,
                                    size_t cols, float* dpre, float* colsum);

/* One AdamW step over flat buffers, same f32 op order as
 * python/orca/optim/adamw.py:71-94 with the f64 scalars rounded to f32 as
 * PyO3 does (orca-python/src/lib.rs:12-16).  t is the step count after
 * increment (adamw.py:64). */
int orca_hip_adamw_step(orca_hip_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, double lr,
                        double beta1, double beta2, double eps, double weight_decay, int64_t t);
/* One vanilla SGD step p -= f32(lr) * g (python/orca/optim/sgd.py:74-79). */
int orca_hip_sgd_step(orca_hip_ctx* ctx, float* p, const float* g, size_t n, double lr);

/* The optimizer's loop over parameters (python/orca/optim/adamw.py:66-99,
 * sgd.py:46-79) as one launch per ORCA_HIP_OPT_MAX_SEGMENTS parameters: each
 * segment reads p_src and g (and m, v for AdamW) and writes p_dst (which may be
 * p_src) and m, v in place, with the per-element arithmetic of
 * orca_hip_adamw_step / orca_hip_sgd_step, so the same bits.  Segments must
 * not overlap one another.  m and v are ignored by SGD. */
#define ORCA_HIP_OPT_MAX_SEGMENTS 32
typedef struct {
  const float* p_src;
  float* p_dst;
  const float* g;
  float* m;
  float* v;
  size_t n;
} orca_hip_opt_segment;
int orca_hip_adamw_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr, double beta1,
                         double beta2, double eps, double weight_decay, int64_t t);
int orca_hip_sgd_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr);

/* ===================== device-resident MLP training step ===================== */
/* nn.Sequential(Linear, ReLU, ..., Linear) + CrossEntropyLoss + SGD/AdamW
 * (python/orca/nn/{linear,activation,container,loss}.py, python/orca/optim)
 * with parameters, gradients and moments in flat device arenas and every
 * intermediate preallocated: a step is a fixed sequence of kernel launches
 * with no host synchronisation and no allocation. */
typedef struct {
  int kind;            /* 0 = SGD (momentum = weight_decay = 0), 1 = AdamW */
  double lr;
  double weight_decay; /* AdamW only */
  double beta1, beta2, eps;
} orca_hip_optim;

/* dims[0..n_layers]: features per layer (e.g. 784, H, H, 10). */
int orca_hip_mlp_create(orca_hip_ctx* ctx, const size_t* dims, size_t n_layers, size_t batch,
                        const orca_hip_optim* opt, orca_hip_mlp** out);
int orca_hip_mlp_destroy(orca_hip_mlp* mlp);
/* Parameter index i: W_{i/2} for even i ([dims[l]][dims[l+1]]), b_{i/2} ([1][dims[l+1]]) for odd i.
 * set_param, set_moment and set_batch upload stream-ordered with no host wait (the host data may
 * be reused on return): a checkpoint restore of every tensor never waits for the device, and the
 * next step runs after the uploads.  The get_* calls synchronise. */
int orca_hip_mlp_param_numel(const orca_hip_mlp* mlp, size_t index, size_t* n);
int orca_hip_mlp_set_param(orca_hip_mlp* mlp, size_t index, const float* host, size_t n);
int orca_hip_mlp_get_param(orca_hip_mlp* mlp, size_t index, float* host, size_t n);
int orca_hip_mlp_get_grad(orca_hip_mlp* mlp, size_t index, float* host, size_t n);
/* which = 0: first moment m, 1: second moment v */
int orca_hip_mlp_get_moment(orca_hip_mlp* mlp, int which, size_t index, float* host, size_t n);
/* Checkpoint restore of the AdamW moments.  No reference counterpart: the
 * reference optimizer keeps m and v in Python lists (python/orca/optim/adamw.py:30-31)
 * and does not save them; here they can be saved and restored with the step count. */
int orca_hip_mlp_set_moment(orca_hip_mlp* mlp, int which, size_t index, const float* host, size_t n);
/* Uploads the batch: x [batch][dims[0]] and either one-hot targets
 * [batch][dims[L]] or class labels [batch] (one of the two non-NULL). */
int orca_hip_mlp_set_batch(orca_hip_mlp* mlp, const float* x, const float* onehot, const int32_t* labels);
/* Device pointers of the resident batch, for callers that fill it on device. */
int orca_hip_mlp_batch_ptrs(orca_hip_mlp* mlp, float** x, int32_t** labels);
/* One forward + backward + optimizer step, enqueued; no host sync. */
int orca_hip_mlp_step(orca_hip_mlp* mlp);
/* Loss and correct-prediction count of the last step (synchronises). */
int orca_hip_mlp_read_metrics(orca_hip_mlp* mlp, float* loss, int64_t* correct);
/* Logits [batch][dims[L]] and predictions [batch] of the last step (synchronises). */
int orca_hip_mlp_get_logits(orca_hip_mlp* mlp, float* host, size_t n);
int orca_hip_mlp_get_preds(orca_hip_mlp* mlp, int32_t* host, size_t n);
/* Forward activations of the last step: layer l < L-1 gives the ReLU output
 * [batch][dims[l+1]], layer L-1 the logits [batch][dims[L]] (synchronises). */
int orca_hip_mlp_get_activation(orca_hip_mlp* mlp, size_t layer, float* host, size_t n);
/* AdamW step counter t (python/orca/optim/adamw.py:33, 64); set restores it from a checkpoint. */
int orca_hip_mlp_get_step_count(const orca_hip_mlp* mlp, int64_t* t);
int orca_hip_mlp_set_step_count(orca_hip_mlp* mlp, int64_t t);
/* One rank's share of a data-parallel step whose optimizer state is sharded over `count`
 * ranks: each optimizer pass of orca_hip_mlp_step updates only slice `index` of `count` of
 * its parameter range (cut at multiples of 64 floats; the slices of all indices cover every
 * parameter once), with the whole update's bits there.  The other slices keep the values
 * they hold when this is called (set_param writes them too); in a data-parallel run the
 * ranks' all-gather would write them.  count = 1 restores the whole update.  No reference
 * counterpart: the reference's optimizers update every parameter (python/orca/optim/
 * adamw.py:66-99), as each rank of a replicated data-parallel step does. */
int orca_hip_mlp_set_update_shard(orca_hip_mlp* mlp, size_t index, size_t count);

/* ===================== kernel timing ===================== */
/* When enabled, each GEMM / fused-kernel launch is bracketed by HIP events on
 * the context stream.  The report is a JSON object
 * {"num_cus": n, "kernels": [{"name", "launches", "total_ms", "flops", "bytes"}...]}
 * with the algorithmic flops / bytes of the launches and the device's compute-unit
 * count, which sizes the GEMM grids and K splits (synchronises). */
int orca_hip_prof_enable(orca_hip_ctx* ctx, int enable);
int orca_hip_prof_reset(orca_hip_ctx* ctx);
int orca_hip_prof_report(orca_hip_ctx* ctx, char* buf, size_t len);
/* Elapsed device time between two markers on the context stream. */
int orca_hip_timer_start(orca_hip_ctx* ctx);
int orca_hip_timer_stop(orca_hip_ctx* ctx, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* ORCA_HIP_H */
