//! Raw declarations of the entry points of include/orca_hip.h this crate calls: the context,
//! the error report, and the storage-handle API (backends, storages, the trait's 42 methods and
//! the inherent fused methods).  Each returns ORCA_HIP_OK (0) or a negative ORCA_HIP_ERR_* code,
//! with the failure's fields available from `orca_hip_last_error_info` on the same thread.
use std::os::raw::{c_char, c_int};

#[repr(C)]
pub struct OrcaHipCtx {
    _private: [u8; 0],
}
#[repr(C)]
pub struct OrcaHipBackend {
    _private: [u8; 0],
}
#[repr(C)]
pub struct OrcaHipStorage {
    _private: [u8; 0],
}

pub const ORCA_HIP_OK: c_int = 0;
pub const ORCA_HIP_ERR_SHAPE: c_int = -1;
pub const ORCA_HIP_ERR_UNSUPPORTED_DTYPE: c_int = -2;
pub const ORCA_HIP_ERR_DTYPE_MISMATCH: c_int = -3;
pub const ORCA_HIP_ERR_DEVICE_MISMATCH: c_int = -4;
pub const ORCA_HIP_ERR_INTERNAL: c_int = -5;

/// orca_hip_backend_options
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct BackendOptions {
    pub lazy: c_int,
    pub deferred: c_int,
    pub fold: c_int,
    pub overlap: c_int,
    pub side_frac: f64,
    pub side_bpc: c_int,
}

/// orca_hip_error_info
#[repr(C)]
pub struct ErrorInfo {
    pub code: c_int,
    pub op: *const c_char,
    pub expected: *const c_char,
    pub got: *const c_char,
    pub dtype: c_int,
    pub dtype_got: c_int,
    pub device_kind: [c_int; 2],
    pub device_index: [c_int; 2],
    pub message: *const c_char,
}

/// orca_hip_opt_row
#[repr(C)]
pub struct OptRow {
    pub p_src: *mut OrcaHipStorage,
    pub p_dst: *mut OrcaHipStorage,
    pub g: *mut OrcaHipStorage,
    pub m: *mut OrcaHipStorage,
    pub v: *mut OrcaHipStorage,
    pub n: usize,
}

extern "C" {
    // ---- context and errors
    pub fn orca_hip_ctx_create(device: c_int, out: *mut *mut OrcaHipCtx) -> c_int;
    pub fn orca_hip_ctx_destroy(ctx: *mut OrcaHipCtx) -> c_int;
    pub fn orca_hip_sync(ctx: *mut OrcaHipCtx) -> c_int;
    pub fn orca_hip_last_error() -> *const c_char;
    pub fn orca_hip_last_error_info(out: *mut ErrorInfo) -> c_int;

    // ---- backends and storage handles
    pub fn orca_hip_backend_default_options(out: *mut BackendOptions) -> c_int;
    pub fn orca_hip_backend_create(
        ctx: *mut OrcaHipCtx,
        opts: *const BackendOptions,
        out: *mut *mut OrcaHipBackend,
    ) -> c_int;
    pub fn orca_hip_backend_destroy(be: *mut OrcaHipBackend) -> c_int;
    pub fn orca_hip_storage_retain(s: *mut OrcaHipStorage) -> c_int;
    pub fn orca_hip_storage_release(s: *mut OrcaHipStorage) -> c_int;
    pub fn orca_hip_storage_len(s: *const OrcaHipStorage, n: *mut usize) -> c_int;
    pub fn orca_hip_storage_flags(s: *const OrcaHipStorage, flags: *mut u32) -> c_int;
    pub fn orca_hip_storage_device_ptr(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        ptr: *mut *mut std::os::raw::c_void,
    ) -> c_int;

    // ---- the Backend trait (orca-tensor/src/backend.rs:19-315), in its order
    pub fn orca_hip_trait_device(be: *mut OrcaHipBackend, kind: *mut c_int, index: *mut c_int) -> c_int;
    pub fn orca_hip_trait_zeros(
        be: *mut OrcaHipBackend,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_from_f32_slice(
        be: *mut OrcaHipBackend,
        shape: *const usize,
        rank: usize,
        data: *const f32,
        n: usize,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_to_f32_vec(be: *mut OrcaHipBackend, s: *mut OrcaHipStorage, host: *mut f32, n: usize)
        -> c_int;
    pub fn orca_hip_trait_matmul(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        lhs_shape: *const usize,
        lhs_rank: usize,
        rhs_shape: *const usize,
        rhs_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_transpose(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dim0: usize,
        dim1: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_add(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sub(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_mul_scalar(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        scalar: f32,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_mul(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_relu(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sigmoid(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_relu_backward(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sigmoid_backward(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_expand(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sum_to_shape(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_reshape(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_exp(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_log(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_exp_backward(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_log_backward(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_div(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sqrt(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_div_backward_lhs(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_div_backward_rhs(
        be: *mut OrcaHipBackend,
        grad: *mut OrcaHipStorage,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_sqrt_backward(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_accumulate_grad(
        be: *mut OrcaHipBackend,
        lhs: *mut OrcaHipStorage,
        rhs: *mut OrcaHipStorage,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_conv2d(
        be: *mut OrcaHipBackend,
        input: *mut OrcaHipStorage,
        weight: *mut OrcaHipStorage,
        bias: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        weight_shape: *const usize,
        weight_rank: usize,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_conv2d_backward_input(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        weight: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        weight_shape: *const usize,
        weight_rank: usize,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_conv2d_backward_weight(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        input: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        weight_shape: *const usize,
        weight_rank: usize,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_conv2d_backward_bias(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_cast(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        current_dtype: c_int,
        target_dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_scatter(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        dim: usize,
        index: *mut OrcaHipStorage,
        src: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        index_shape: *const usize,
        index_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_gather(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        dim: usize,
        index: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        index_shape: *const usize,
        index_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_scatter_backward_src(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        dim: usize,
        index: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        index_shape: *const usize,
        index_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_scatter_backward_base(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        dim: usize,
        index: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        index_shape: *const usize,
        index_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_gather_backward(
        be: *mut OrcaHipBackend,
        grad_out: *mut OrcaHipStorage,
        dim: usize,
        index: *mut OrcaHipStorage,
        shape: *const usize,
        rank: usize,
        index_shape: *const usize,
        index_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_from_bytes(
        be: *mut OrcaHipBackend,
        shape: *const usize,
        rank: usize,
        bytes: *const u8,
        n_bytes: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_to_bytes(be: *mut OrcaHipBackend, s: *mut OrcaHipStorage, host: *mut u8, n_bytes: usize)
        -> c_int;
    pub fn orca_hip_trait_has_nan_or_inf(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        dtype: c_int,
        result: *mut c_int,
    ) -> c_int;
    pub fn orca_hip_trait_max_to_shape(
        be: *mut OrcaHipBackend,
        s: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_trait_max_to_shape_backward(
        be: *mut OrcaHipBackend,
        grad: *mut OrcaHipStorage,
        in_primal: *mut OrcaHipStorage,
        out_primal: *mut OrcaHipStorage,
        in_shape: *const usize,
        in_rank: usize,
        out_shape: *const usize,
        out_rank: usize,
        dtype: c_int,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;

    // ---- inherent methods beside the trait (the opt-in fused loss and optimizers)
    pub fn orca_hip_be_softmax_ce(
        be: *mut OrcaHipBackend,
        logits: *mut OrcaHipStorage,
        onehot: *mut OrcaHipStorage,
        b: usize,
        c: usize,
        want_grad: c_int,
        loss: *mut *mut OrcaHipStorage,
        dlogits: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_be_clone(be: *mut OrcaHipBackend, s: *mut OrcaHipStorage, out: *mut *mut OrcaHipStorage) -> c_int;
    pub fn orca_hip_be_arena(
        be: *mut OrcaHipBackend,
        n: usize,
        fill: c_int,
        value: f32,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_be_view(
        be: *mut OrcaHipBackend,
        arena: *mut OrcaHipStorage,
        offset: usize,
        n: usize,
        out: *mut *mut OrcaHipStorage,
    ) -> c_int;
    pub fn orca_hip_be_copy_into(be: *mut OrcaHipBackend, dst: *mut OrcaHipStorage, src: *mut OrcaHipStorage) -> c_int;
    pub fn orca_hip_be_arena_exclusive(be: *mut OrcaHipBackend, arena: *mut OrcaHipStorage, exclusive: *mut c_int)
        -> c_int;
    pub fn orca_hip_be_adamw_multi(
        be: *mut OrcaHipBackend,
        rows: *const OptRow,
        n_rows: usize,
        lr: f64,
        beta1: f64,
        beta2: f64,
        eps: f64,
        weight_decay: f64,
        t: i64,
    ) -> c_int;
    pub fn orca_hip_be_sgd_multi(be: *mut OrcaHipBackend, rows: *const OptRow, n_rows: usize, lr: f64) -> c_int;
    pub fn orca_hip_be_adamw_step(
        be: *mut OrcaHipBackend,
        p: *mut OrcaHipStorage,
        g: *mut OrcaHipStorage,
        m: *mut OrcaHipStorage,
        v: *mut OrcaHipStorage,
        n: usize,
        lr: f64,
        beta1: f64,
        beta2: f64,
        eps: f64,
        weight_decay: f64,
        t: i64,
    ) -> c_int;
    pub fn orca_hip_be_sgd_step(
        be: *mut OrcaHipBackend,
        p: *mut OrcaHipStorage,
        g: *mut OrcaHipStorage,
        n: usize,
        lr: f64,
    ) -> c_int;
}
