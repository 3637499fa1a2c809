//! MI355X (gfx950) backend for Orca.
//!
//! `HipBackend` implements `orca_tensor::Backend` (orca-tensor/src/backend.rs:19-315) with one
//! call per trait method into liborca_hip.so (include/orca_hip.h, "storage handles"): the
//! library owns the storages' device memory and their planning (lazy transposes, fused
//! elementwise chains, GEMM epilogue folds, deferred bias column sums), so `Autodiff<HipBackend>`
//! and the orca-python frontend run unchanged on the MI355X.  Every value has the bits the
//! trait's ops run one by one give; errors map onto all five `OrcaError` variants.
pub mod backend;
pub mod error;
pub mod ffi;
pub mod storage;

pub use backend::HipBackend;
pub use storage::HipStorage;
