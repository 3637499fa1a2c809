//! `HipBackend: Backend` (orca-tensor/src/backend.rs:19-315): each trait method is one call into
//! liborca_hip.so's storage-handle API, which keeps the planning that makes the composed step
//! fast (lazy transposes, fused elementwise chains, GEMM epilogue folds, deferred bias column
//! sums, host constants) behind the handles.  The inherent methods beside the trait serve the
//! opt-in fused loss and optimizers.
use std::fmt;
use std::os::raw::c_int;
use std::ptr;
use std::sync::Arc;

use orca_core::{DType, Device, Result, Shape};
use orca_tensor::Backend;

use crate::error::{check, dtype_code};
use crate::ffi;
use crate::storage::HipStorage;

struct Raw {
    be: *mut ffi::OrcaHipBackend,
    ordinal: usize,
}

// The library serialises every call on a backend with its own lock.
unsafe impl Send for Raw {}
unsafe impl Sync for Raw {}

impl Drop for Raw {
    fn drop(&mut self) {
        unsafe {
            ffi::orca_hip_backend_destroy(self.be);
        }
    }
}

/// The MI355X backend: cheap to clone, usable from any thread.
#[derive(Clone)]
pub struct HipBackend {
    raw: Arc<Raw>,
}

impl fmt::Debug for HipBackend {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "HipBackend(gpu:{})", self.raw.ordinal)
    }
}

fn dims(shape: &Shape) -> (*const usize, usize) {
    (shape.0.as_ptr(), shape.0.len())
}

impl HipBackend {
    /// A backend on HIP device 0 (GpuBackend::new's counterpart, orca-backend-gpu/src/backend.rs:53).
    pub fn new() -> Result<Self> {
        Self::with_device(0)
    }

    /// A backend on HIP device `ordinal`.  Its context (stream, caching allocator) lives for the
    /// process, as the reference's global backend does (orca-python/src/lib.rs:23-33).
    pub fn with_device(ordinal: usize) -> Result<Self> {
        let mut ctx = ptr::null_mut();
        check(unsafe { ffi::orca_hip_ctx_create(ordinal as c_int, &mut ctx) })?;
        let mut be = ptr::null_mut();
        check(unsafe { ffi::orca_hip_backend_create(ctx, ptr::null(), &mut be) })?;
        Ok(HipBackend { raw: Arc::new(Raw { be, ordinal }) })
    }

    fn be(&self) -> *mut ffi::OrcaHipBackend {
        self.raw.be
    }

    /// Runs one entry point that returns a new storage handle.
    fn out(&self, call: impl FnOnce(*mut *mut ffi::OrcaHipStorage) -> c_int) -> Result<HipStorage> {
        let mut out = ptr::null_mut();
        check(call(&mut out))?;
        Ok(HipStorage::adopt(out))
    }

    // ---- inherent methods beside the trait (no counterpart in the reference's trait) ----

    /// Mean softmax cross-entropy of [b, c] logits against one-hot targets and, if want_grad,
    /// dL/dlogits for a loss seed of 1, in one kernel (python/orca/nn/loss.py:59-100 fused).
    pub fn softmax_ce(
        &self,
        logits: &HipStorage,
        onehot: &HipStorage,
        b: usize,
        c: usize,
        want_grad: bool,
    ) -> Result<(HipStorage, Option<HipStorage>)> {
        let (mut loss, mut grad) = (ptr::null_mut(), ptr::null_mut());
        check(unsafe {
            ffi::orca_hip_be_softmax_ce(self.be(), logits.raw(), onehot.raw(), b, c, want_grad as c_int, &mut loss, &mut grad)
        })?;
        Ok((HipStorage::adopt(loss), if want_grad { Some(HipStorage::adopt(grad)) } else { None }))
    }

    /// A new storage with the same values.
    pub fn clone_storage(&self, s: &HipStorage) -> Result<HipStorage> {
        self.out(|o| unsafe { ffi::orca_hip_be_clone(self.be(), s.raw(), o) })
    }

    /// A flat arena of n floats (filled with `fill` when given) for the fused optimizers.
    pub fn arena(&self, n: usize, fill: Option<f32>) -> Result<HipStorage> {
        self.out(|o| unsafe { ffi::orca_hip_be_arena(self.be(), n, fill.is_some() as c_int, fill.unwrap_or(0.0), o) })
    }

    /// n floats at `offset` of an arena, sharing its memory.
    pub fn view(&self, arena: &HipStorage, offset: usize, n: usize) -> Result<HipStorage> {
        self.out(|o| unsafe { ffi::orca_hip_be_view(self.be(), arena.raw(), offset, n, o) })
    }

    /// dst <- src on the device (dst: a fresh arena slice nothing reads yet).
    pub fn copy_into(&self, dst: &HipStorage, src: &HipStorage) -> Result<()> {
        check(unsafe { ffi::orca_hip_be_copy_into(self.be(), dst.raw(), src.raw()) })
    }

    /// Whether nothing but `arena` refers to its memory (it can be written without changing a held value).
    pub fn arena_exclusive(&self, arena: &HipStorage) -> Result<bool> {
        let mut v: c_int = 0;
        check(unsafe { ffi::orca_hip_be_arena_exclusive(self.be(), arena.raw(), &mut v) })?;
        Ok(v != 0)
    }

    /// One AdamW pass over many parameters: rows of (p_src, p_dst, g, m, v, n); p_dst, m and v
    /// are written (python/orca/optim/adamw.py:66-99, same f32 operations).
    #[allow(clippy::too_many_arguments)]
    pub fn adamw_multi(
        &self,
        rows: &[(&HipStorage, &HipStorage, &HipStorage, &HipStorage, &HipStorage, usize)],
        lr: f64,
        beta1: f64,
        beta2: f64,
        eps: f64,
        weight_decay: f64,
        t: i64,
    ) -> Result<()> {
        let table: Vec<ffi::OptRow> = rows
            .iter()
            .map(|(ps, pd, g, m, v, n)| ffi::OptRow {
                p_src: ps.raw(),
                p_dst: pd.raw(),
                g: g.raw(),
                m: m.raw(),
                v: v.raw(),
                n: *n,
            })
            .collect();
        check(unsafe {
            ffi::orca_hip_be_adamw_multi(self.be(), table.as_ptr(), table.len(), lr, beta1, beta2, eps, weight_decay, t)
        })
    }

    /// One SGD pass over many parameters: rows of (p_src, p_dst, g, n) (python/orca/optim/sgd.py:46-79).
    pub fn sgd_multi(&self, rows: &[(&HipStorage, &HipStorage, &HipStorage, usize)], lr: f64) -> Result<()> {
        let table: Vec<ffi::OptRow> = rows
            .iter()
            .map(|(ps, pd, g, n)| ffi::OptRow {
                p_src: ps.raw(),
                p_dst: pd.raw(),
                g: g.raw(),
                m: ptr::null_mut(),
                v: ptr::null_mut(),
                n: *n,
            })
            .collect();
        check(unsafe { ffi::orca_hip_be_sgd_multi(self.be(), table.as_ptr(), table.len(), lr) })
    }
}

impl Backend for HipBackend {
    type Storage = HipStorage;

    fn device(&self) -> Device {
        Device::Gpu(self.raw.ordinal)
    }

    fn zeros(&self, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_zeros(self.be(), d, r, dtype_code(dtype), o) })
    }

    fn from_f32_slice(&self, shape: &Shape, data: &[f32]) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_from_f32_slice(self.be(), d, r, data.as_ptr(), data.len(), o) })
    }

    fn to_f32_vec(&self, storage: &HipStorage) -> Result<Vec<f32>> {
        let mut v = vec![0.0f32; storage.len_elements()];
        check(unsafe { ffi::orca_hip_trait_to_f32_vec(self.be(), storage.raw(), v.as_mut_ptr(), v.len()) })?;
        Ok(v)
    }

    fn matmul(
        &self,
        lhs: &HipStorage,
        rhs: &HipStorage,
        lhs_shape: &Shape,
        rhs_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (ld, lr) = dims(lhs_shape);
        let (rd, rr) = dims(rhs_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_matmul(self.be(), lhs.raw(), rhs.raw(), ld, lr, rd, rr, dtype_code(dtype), o)
        })
    }

    fn transpose(&self, storage: &HipStorage, shape: &Shape, dim0: usize, dim1: usize, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_transpose(self.be(), storage.raw(), d, r, dim0, dim1, dtype_code(dtype), o)
        })
    }

    fn add(&self, lhs: &HipStorage, rhs: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_add(self.be(), lhs.raw(), rhs.raw(), d, r, dtype_code(dtype), o) })
    }

    fn sub(&self, lhs: &HipStorage, rhs: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_sub(self.be(), lhs.raw(), rhs.raw(), d, r, dtype_code(dtype), o) })
    }

    fn mul_scalar(&self, storage: &HipStorage, scalar: f32, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_mul_scalar(self.be(), storage.raw(), scalar, d, r, dtype_code(dtype), o)
        })
    }

    fn mul(&self, lhs: &HipStorage, rhs: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_mul(self.be(), lhs.raw(), rhs.raw(), d, r, dtype_code(dtype), o) })
    }

    fn relu(&self, storage: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_relu(self.be(), storage.raw(), d, r, dtype_code(dtype), o) })
    }

    fn sigmoid(&self, storage: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_sigmoid(self.be(), storage.raw(), d, r, dtype_code(dtype), o) })
    }

    fn relu_backward(&self, grad_out: &HipStorage, in_primal: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_relu_backward(self.be(), grad_out.raw(), in_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn sigmoid_backward(
        &self,
        grad_out: &HipStorage,
        out_primal: &HipStorage,
        shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_sigmoid_backward(self.be(), grad_out.raw(), out_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn expand(&self, storage: &HipStorage, in_shape: &Shape, out_shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_expand(self.be(), storage.raw(), id, ir, od, or, dtype_code(dtype), o) })
    }

    fn sum_to_shape(&self, storage: &HipStorage, in_shape: &Shape, out_shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_sum_to_shape(self.be(), storage.raw(), id, ir, od, or, dtype_code(dtype), o)
        })
    }

    fn reshape(&self, storage: &HipStorage, in_shape: &Shape, out_shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_reshape(self.be(), storage.raw(), id, ir, od, or, dtype_code(dtype), o) })
    }

    fn exp(&self, storage: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_exp(self.be(), storage.raw(), d, r, dtype_code(dtype), o) })
    }

    fn log(&self, storage: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_log(self.be(), storage.raw(), d, r, dtype_code(dtype), o) })
    }

    fn exp_backward(&self, grad_out: &HipStorage, out_primal: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_exp_backward(self.be(), grad_out.raw(), out_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn log_backward(&self, grad_out: &HipStorage, in_primal: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_log_backward(self.be(), grad_out.raw(), in_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn div(&self, lhs: &HipStorage, rhs: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_div(self.be(), lhs.raw(), rhs.raw(), d, r, dtype_code(dtype), o) })
    }

    fn sqrt(&self, storage: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_sqrt(self.be(), storage.raw(), d, r, dtype_code(dtype), o) })
    }

    fn div_backward_lhs(&self, grad_out: &HipStorage, rhs_primal: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_div_backward_lhs(self.be(), grad_out.raw(), rhs_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn div_backward_rhs(
        &self,
        grad_out: &HipStorage,
        lhs_primal: &HipStorage,
        rhs_primal: &HipStorage,
        shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_div_backward_rhs(
                self.be(),
                grad_out.raw(),
                lhs_primal.raw(),
                rhs_primal.raw(),
                d,
                r,
                dtype_code(dtype),
                o,
            )
        })
    }

    fn sqrt_backward(&self, grad_out: &HipStorage, out_primal: &HipStorage, shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_sqrt_backward(self.be(), grad_out.raw(), out_primal.raw(), d, r, dtype_code(dtype), o)
        })
    }

    fn accumulate_grad(&self, lhs: &HipStorage, rhs: &HipStorage) -> Result<HipStorage> {
        self.out(|o| unsafe { ffi::orca_hip_trait_accumulate_grad(self.be(), lhs.raw(), rhs.raw(), o) })
    }

    fn conv2d(
        &self,
        input: &HipStorage,
        weight: &HipStorage,
        bias: Option<&HipStorage>,
        in_shape: &Shape,
        weight_shape: &Shape,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (wd, wr) = dims(weight_shape);
        let b = bias.map_or(ptr::null_mut(), |b| b.raw());
        self.out(|o| unsafe {
            ffi::orca_hip_trait_conv2d(
                self.be(),
                input.raw(),
                weight.raw(),
                b,
                id,
                ir,
                wd,
                wr,
                padding,
                stride,
                dilation,
                groups,
                dtype_code(dtype),
                o,
            )
        })
    }

    fn conv2d_backward_input(
        &self,
        grad_out: &HipStorage,
        weight: &HipStorage,
        in_shape: &Shape,
        weight_shape: &Shape,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (wd, wr) = dims(weight_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_conv2d_backward_input(
                self.be(),
                grad_out.raw(),
                weight.raw(),
                id,
                ir,
                wd,
                wr,
                padding,
                stride,
                dilation,
                groups,
                dtype_code(dtype),
                o,
            )
        })
    }

    fn conv2d_backward_weight(
        &self,
        grad_out: &HipStorage,
        input: &HipStorage,
        in_shape: &Shape,
        weight_shape: &Shape,
        padding: usize,
        stride: usize,
        dilation: usize,
        groups: usize,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (wd, wr) = dims(weight_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_conv2d_backward_weight(
                self.be(),
                grad_out.raw(),
                input.raw(),
                id,
                ir,
                wd,
                wr,
                padding,
                stride,
                dilation,
                groups,
                dtype_code(dtype),
                o,
            )
        })
    }

    fn conv2d_backward_bias(&self, grad_out: &HipStorage, out_shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe { ffi::orca_hip_trait_conv2d_backward_bias(self.be(), grad_out.raw(), od, or, dtype_code(dtype), o) })
    }

    fn cast(&self, storage: &HipStorage, shape: &Shape, current_dtype: DType, target_dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_cast(self.be(), storage.raw(), d, r, dtype_code(current_dtype), dtype_code(target_dtype), o)
        })
    }

    fn scatter(
        &self,
        storage: &HipStorage,
        dim: usize,
        index: &HipStorage,
        src: &HipStorage,
        shape: &Shape,
        index_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        let (xd, xr) = dims(index_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_scatter(self.be(), storage.raw(), dim, index.raw(), src.raw(), d, r, xd, xr, dtype_code(dtype), o)
        })
    }

    fn gather(
        &self,
        storage: &HipStorage,
        dim: usize,
        index: &HipStorage,
        shape: &Shape,
        index_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        let (xd, xr) = dims(index_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_gather(self.be(), storage.raw(), dim, index.raw(), d, r, xd, xr, dtype_code(dtype), o)
        })
    }

    fn scatter_backward_src(
        &self,
        grad_out: &HipStorage,
        dim: usize,
        index: &HipStorage,
        shape: &Shape,
        index_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        let (xd, xr) = dims(index_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_scatter_backward_src(self.be(), grad_out.raw(), dim, index.raw(), d, r, xd, xr, dtype_code(dtype), o)
        })
    }

    fn scatter_backward_base(
        &self,
        grad_out: &HipStorage,
        dim: usize,
        index: &HipStorage,
        shape: &Shape,
        index_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        let (xd, xr) = dims(index_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_scatter_backward_base(self.be(), grad_out.raw(), dim, index.raw(), d, r, xd, xr, dtype_code(dtype), o)
        })
    }

    fn gather_backward(
        &self,
        grad_out: &HipStorage,
        dim: usize,
        index: &HipStorage,
        shape: &Shape,
        index_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        let (xd, xr) = dims(index_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_gather_backward(self.be(), grad_out.raw(), dim, index.raw(), d, r, xd, xr, dtype_code(dtype), o)
        })
    }

    fn from_bytes(&self, shape: &Shape, bytes: &[u8], dtype: DType) -> Result<HipStorage> {
        let (d, r) = dims(shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_from_bytes(self.be(), d, r, bytes.as_ptr(), bytes.len(), dtype_code(dtype), o)
        })
    }

    fn to_bytes(&self, storage: &HipStorage) -> Result<Vec<u8>> {
        let mut v = vec![0u8; 4 * storage.len_elements()];
        check(unsafe { ffi::orca_hip_trait_to_bytes(self.be(), storage.raw(), v.as_mut_ptr(), v.len()) })?;
        Ok(v)
    }

    fn has_nan_or_inf(&self, storage: &HipStorage, dtype: DType) -> Result<bool> {
        let mut v: c_int = 0;
        check(unsafe { ffi::orca_hip_trait_has_nan_or_inf(self.be(), storage.raw(), dtype_code(dtype), &mut v) })?;
        Ok(v != 0)
    }

    fn max_to_shape(&self, storage: &HipStorage, in_shape: &Shape, out_shape: &Shape, dtype: DType) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_max_to_shape(self.be(), storage.raw(), id, ir, od, or, dtype_code(dtype), o)
        })
    }

    fn max_to_shape_backward(
        &self,
        grad_out: &HipStorage,
        in_primal: &HipStorage,
        out_primal: &HipStorage,
        in_shape: &Shape,
        out_shape: &Shape,
        dtype: DType,
    ) -> Result<HipStorage> {
        let (id, ir) = dims(in_shape);
        let (od, or) = dims(out_shape);
        self.out(|o| unsafe {
            ffi::orca_hip_trait_max_to_shape_backward(
                self.be(),
                grad_out.raw(),
                in_primal.raw(),
                out_primal.raw(),
                id,
                ir,
                od,
                or,
                dtype_code(dtype),
                o,
            )
        })
    }
}
