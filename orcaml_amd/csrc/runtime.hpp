// Host runtime shared by every translation unit of liborca_hip.so: error
// mapping onto orca_core::OrcaError codes, the per-device context with its
// stream-ordered caching allocator, and optional per-launch event timing.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/orca_hip.h"

namespace orca_hip {

// The fields of an orca_core::OrcaError variant (orca-core/src/error.rs:5-31)
// beyond its code: ShapeMismatch {op, expected, got}, UnsupportedDType {op,
// dtype}, DTypeMismatch {op, expected, got} (dtype codes in dtype / dtype_got),
// DeviceMismatch (two devices as kind + index: 0 = Cpu, 1 = Cuda, 2 = Gpu).
struct ErrorFields {
  std::string op, expected, got;
  int dtype = -1, dtype_got = -1;
  int device_kind[2] = {-1, -1}, device_index[2] = {-1, -1};
};

// An error carrying one of the ORCA_HIP_ERR_* codes and, where known, its variant's fields.
struct Error : std::runtime_error {
  int code;
  ErrorFields fields;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
  Error(int c, const std::string& m, ErrorFields f) : std::runtime_error(m), code(c), fields(std::move(f)) {}
};

void set_last_error(const std::string& msg);
void set_last_error(const std::string& msg, int code, const ErrorFields& fields);
const char* last_error_cstr();  // the calling thread's last message
void last_error_info(orca_hip_error_info* out);  // the calling thread's last error, with its fields

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }
// OrcaError::ShapeMismatch, with the reference's message ("Shape mismatch during {op}: expected {e}, got {g}").
[[noreturn]] void fail_shape(const std::string& op, const std::string& expected, const std::string& got);
// OrcaError::UnsupportedDType ("Unsupported dtype for {op}: {dtype}").
[[noreturn]] void fail_dtype(const std::string& op, int dtype);
// OrcaError::DeviceMismatch of two GPUs ("Device mismatch: ... Got gpu:{a} and gpu:{b}").
[[noreturn]] void fail_device(int gpu_a, int gpu_b);
// The name of a dtype code in orca_core::DType's Display form ("float32", "bfloat16", ...,
// orca-core/src/dtype.rs:146-160).
const char* dtype_name(int dtype);

#define ORCA_HIP_CHECK(expr)                                                                   \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess)                                                                      \
      ::orca_hip::fail(ORCA_HIP_ERR_INTERNAL, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

// Output buffers allocated by the entry point that is running on this thread
// (new_output): kept when it succeeds, returned to the allocator when it fails,
// so an op that rejects its arguments after allocating its result leaks nothing.
void outputs_begin();
void outputs_commit();
void outputs_abort();

// Runs f, converting exceptions into a status code + thread-local message.
template <class F>
int guard(F&& f) {
  outputs_begin();
  try {
    f();
    outputs_commit();
    return ORCA_HIP_OK;
  } catch (const Error& e) {
    outputs_abort();
    set_last_error(e.what(), e.code, e.fields);
    return e.code;
  } catch (const std::exception& e) {
    outputs_abort();
    set_last_error(std::string("internal error: ") + e.what());
    return ORCA_HIP_ERR_INTERNAL;
  } catch (...) {
    outputs_abort();
    set_last_error("internal error: unknown exception");
    return ORCA_HIP_ERR_INTERNAL;
  }
}

// Size-class caching allocator.  All work of a context runs on one in-order
// stream, so a block returned here can be handed to the next request at once:
// any later kernel using it is ordered after every earlier kernel that used
// it.  Blocks are 256-byte aligned (hipMalloc alignment).
//
// Every release ticks a clock.  A block released at tick t was last used by work
// enqueued before that release, so work on another stream that first waits for an
// event recorded on the context stream when the clock read c >= t may use it.
class CachingAllocator {
 public:
  void* allocate(size_t bytes, hipStream_t stream);
  // A cached block released at or before tick `clock`, oldest first, or null (this never
  // allocates device memory).
  void* allocate_released_by(size_t bytes, uint64_t clock);
  // How many cached blocks of this size were released at or before tick `clock`.
  size_t count_released_by(size_t bytes, uint64_t clock);
  uint64_t clock();
  void release(void* p);
  void empty(hipStream_t stream);
  size_t size_of(void* p);
  // Where p points: into a live block (*extent = bytes from p to its end), into
  // a block that was freed and is held in the cache, or into neither (memory
  // this allocator did not hand out).
  enum class Where { kLive, kFreed, kUnknown };
  Where locate(const void* p, size_t* extent);
  // Bytes from p to the end of the live allocation containing p (0 if none does).
  size_t extent_from(const void* p);
  void stats(size_t* live, size_t* cached, size_t* mallocs);
  ~CachingAllocator();

  static size_t round_size(size_t bytes);
  // Counts the stream synchronisation that empty() performs (the owning context's counter).
  std::atomic<uint64_t>* sync_counter = nullptr;

 private:
  std::mutex mu_;
  std::map<void*, size_t> live_;  // ordered: extent_from finds the block around an interior pointer
  struct Cached {
    void* p;
    uint64_t released;  // the clock tick of its release
  };
  // per size class in release order (a multimap keeps equal keys in insertion order)
  std::multimap<size_t, Cached> cached_;
  std::map<void*, size_t> cached_at_;  // the cached blocks by address, for locate()
  size_t live_bytes_ = 0, cached_bytes_ = 0, mallocs_ = 0;
  uint64_t clock_ = 0;
};

// Pinned host memory through which uploads reach the device without a host
// wait: the caller's bytes are copied into a free region of the ring, the
// region is copied to the device on the stream, and an event recorded after
// that copy marks when the region may be reused.  The host waits only when
// every region is still in flight (back-pressure), and each such wait is
// counted like any other.
class StagingRing {
 public:
  // Enqueues dst <- src (bytes) on `stream`; src may be reused on return.
  void upload(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes, hipStream_t stream);
  ~StagingRing();

  static constexpr size_t kCapacity = size_t(16) << 20;  // pinned bytes held per context
  static constexpr size_t kChunk = size_t(4) << 20;      // largest single region

 private:
  struct Region {
    size_t begin, end;
    hipEvent_t done;
  };
  // Offset of a free region of `need` bytes, waiting for the oldest copies if none is free.
  size_t reserve(orca_hip_ctx* ctx, size_t need);
  void retire_finished();
  std::mutex mu_;
  char* base_ = nullptr;
  size_t head_ = 0;
  std::deque<Region> inflight_;
  std::vector<hipEvent_t> spare_;
};

// Per-kernel timing aggregation (enabled by orca_hip_prof_enable).
struct Profiler {
  struct Pending {
    std::string name;
    hipEvent_t start, stop;
    double flops, bytes;
  };
  struct Agg {
    long launches = 0;
    double total_ms = 0, flops = 0, bytes = 0;
  };
  bool enabled = false;
  std::vector<Pending> pending;
  std::vector<hipEvent_t> pool;
  std::map<std::string, Agg> agg;

  hipEvent_t get_event();
  void drain();  // requires the stream to be synchronised
  ~Profiler();
};

struct EwJitCache;

}  // namespace orca_hip

struct orca_hip_ctx {
  int device = 0;
  int num_cus = 256;
  hipStream_t stream = nullptr;
  orca_hip::CachingAllocator alloc;
  orca_hip::Profiler prof;
  hipEvent_t timer_start = nullptr, timer_stop = nullptr;
  std::mutex mu;
  // Tuning switches read once when the context is created (environment):
  // ORCA_HIP_GEMM_FAST=0 sends every product through the generic GEMM kernel,
  // ORCA_HIP_GEMM_TILE=128x128|128x64 fixes the generic kernel's tile (0 = by grid size).
  bool gemm_generic_only = false;
  int gemm_tile_bn = 0;
  // ORCA_HIP_GEMM_SMALL_TILES=0 keeps the K split for small products instead of 64 x 64 tiles.
  bool gemm_small_tiles = true;
  // ORCA_HIP_GEMM_SKINNY=0 keeps the K split for few-row products instead of the skinny kernel.
  bool gemm_skinny = true;
  // ORCA_HIP_GEMM_NARROW=0 keeps products with N <= 16 (or K <= 16 against B^T) on the tiled kernels.
  bool gemm_narrow = true;
  // ORCA_HIP_GEMM_BAND: 0 keeps weight gradients X^T dY of 784-like row counts on the
  // 128 x 128 tiles; 1 prefers the eight-band grid (every CU), 2 the 112-row tiles
  // (the CUs the 128 x 128 grid leaves free stay free) where both apply.
  int gemm_band = 2;
  // Host waits on this context's work so far (stream or event synchronisations).
  std::atomic<uint64_t> host_syncs{0};
  orca_hip::StagingRing staging;
  // Fused elementwise programs compiled at run time (ewprog.hip), released with
  // the context.  ORCA_HIP_EW_JIT (or orca_hip_ew_set_jit): 0 interprets every
  // program, 1 compiles a program structure at its second use, 2 at its first.
  orca_hip::EwJitCache* ew_jit = nullptr;
  int ew_jit_mode = 1;
  // A second stream (default priority) for work that runs beside the context
  // stream: while launches go to it (orca_hip_use_side_stream), `main` holds
  // the context stream.  `side_last` marks the side stream's work so far;
  // host reads and synchronisations first make the context stream wait for it.
  hipStream_t side = nullptr;
  hipStream_t main = nullptr;
  hipEvent_t side_last = nullptr;
  bool side_joined = true;
  // Blocks per CU of an optimizer pass launched on the side stream (0: the full grid).
  int side_bpc = 0;
  // Released ordering events, reused by orca_hip_event_record.
  std::vector<hipEvent_t> event_pool;
};

namespace orca_hip {

// Unloads the context's compiled elementwise programs (ewprog.hip).
void ew_jit_release(orca_hip_ctx* ctx);

// Makes ctx's device current for the calling thread.
void bind(orca_hip_ctx* ctx);

// Brackets one launch with events when profiling is on (on `stream`, the
// context stream when null).
class ProfScope {
 public:
  ProfScope(orca_hip_ctx* ctx, const char* name, double flops, double bytes, hipStream_t stream = nullptr);
  ~ProfScope();

 private:
  orca_hip_ctx* ctx_;
  hipStream_t stream_;
  Profiler::Pending rec_;
  bool on_;
};

// A block from the context's caching allocator for work on the context stream.
// The allocator orders the reuse of a released block by the context stream alone,
// so this fails (InternalError) while launches go to the side stream
// (orca_hip_use_side_stream): a block released after side-stream work could be
// handed to context-stream work that the side stream has not finished with.
void* ctx_allocate(orca_hip_ctx* ctx, size_t bytes);
// For work that will run on the side stream after waiting for an event recorded on the
// context stream when the allocator's clock read `clock`: a cached block released by then
// (its last users are all before that event), or null.  Called while launches still go to
// the context stream, like ctx_allocate.
void* ctx_allocate_released_by(orca_hip_ctx* ctx, size_t bytes, uint64_t clock);
size_t ctx_count_released_by(orca_hip_ctx* ctx, size_t bytes, uint64_t clock);
uint64_t ctx_release_clock(orca_hip_ctx* ctx);
// An unrecorded event for ordering the context's two streams (from the context's pool;
// orca_hip_event_release gives it back).
hipEvent_t take_order_event(orca_hip_ctx* ctx);

// RAII device buffer from the context allocator (freed stream-ordered).
class Scratch {
 public:
  Scratch(orca_hip_ctx* ctx, size_t bytes) : ctx_(ctx), p_(bytes ? ctx_allocate(ctx, bytes) : nullptr) {}
  ~Scratch() {
    if (p_) ctx_->alloc.release(p_);
  }
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  template <class T>
  T* as() const {
    return static_cast<T*>(p_);
  }

 private:
  orca_hip_ctx* ctx_;
  void* p_;
};

// Fails with ShapeMismatch when [p, p + bytes) runs past the end of the
// context allocation that contains p, so a wrong size or leading dimension
// is reported instead of launching out of bounds, and with InternalError when
// p points into a block that was freed (a use after free through the ABI).
// Memory the context did not allocate is not checked.
void check_extent(orca_hip_ctx* ctx, const void* p, size_t bytes, const char* what);
// Extent of a row-major [rows][ld] operand whose rows hold `cols` used values.
inline size_t matrix_bytes(size_t rows, size_t cols, size_t ld) {
  return rows == 0 || cols == 0 ? 0 : ((rows - 1) * ld + cols) * sizeof(float);
}

inline void check_ctx(const orca_hip_ctx* ctx) {
  if (!ctx) fail(ORCA_HIP_ERR_INTERNAL, "null orca_hip_ctx");
}

inline void check_f32(int dtype, const char* op) {
  if (dtype != ORCA_HIP_F32) fail_dtype(op, dtype);
}

size_t numel(const size_t* shape, size_t rank);
std::string shape_str(const size_t* shape, size_t rank);

// Grid size for grid-stride element loops.
inline unsigned grid_for(size_t work_items, unsigned block, unsigned max_blocks) {
  size_t g = (work_items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > max_blocks) g = max_blocks;
  return static_cast<unsigned>(g);
}

// Every host wait the library performs goes through these two, which count it
// in ctx->host_syncs (reported by orca_hip_sync_count).
void host_sync(orca_hip_ctx* ctx, hipStream_t stream = nullptr);
// The context stream waits for the side stream's work so far (no host wait).
void join_side(orca_hip_ctx* ctx);
void host_wait_event(orca_hip_ctx* ctx, hipEvent_t ev);
// Stream-ordered host-to-device copy that does not wait for the device: small
// payloads travel as a kernel argument, larger ones through the staging ring.
// The host buffer may be reused as soon as this returns.
void upload_async(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes);

// Allocates a fresh output buffer of n floats for a trait op.
float* new_output(orca_hip_ctx* ctx, size_t n);

// ---- launchers shared between translation units (device pointers, async) ----
void launch_fill(orca_hip_ctx* ctx, float* dst, float v, size_t n);
void launch_copy(orca_hip_ctx* ctx, float* dst, const float* src, size_t n);
// colsum[c] = sum_r src[r*ld + c] in ascending r (the sum_to_shape order).
void launch_colsum(orca_hip_ctx* ctx, const float* src, size_t rows, size_t cols, size_t ld, float* colsum);

struct GemmEpi {
  int kind = ORCA_HIP_EPI_NONE;
  const float* bias = nullptr;
  const float* mask = nullptr;
  size_t ldmask = 0;
  float* colsum = nullptr;
  float* pre = nullptr;  // EPI_BIAS_RELU_PRE: acc + bias; EPI_RELU_MASK_PRE: acc (C's ldc)
  // Column sums in ascending row order (bit-identical to sum_to_shape) even
  // when K is split: the split product then takes them in a separate pass.
  bool exact_colsum = false;
  // Optional caller-owned workspace for split-K partials (see
  // gemm_workspace_floats); without it they come from the context cache.
  float* ws = nullptr;
  size_t ws_floats = 0;
  // Optional event that the product records on ctx->stream once its last
  // launch has run: bound to that launch's completion when the pipelined
  // kernel is the last one (no separate marker between it and the next
  // launch), else recorded after it.
  hipEvent_t done = nullptr;
  // Banded weight gradient grid where both forms apply (gemm_band's values): 0 the
  // context's preference, 1 every CU (nothing runs beside the product), 2 the grid
  // that leaves CUs free for work on another stream.
  int band = 0;
};
// Workspace floats gemm() needs for this product (0 when K is not split).
size_t gemm_workspace_floats(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K,
                             const float* A, size_t lda, size_t sa, const float* B, size_t ldb, size_t sb,
                             size_t batch, bool colsum, int epi_kind = ORCA_HIP_EPI_NONE);
// Batched GEMM: C[b] = op(A[b]) op(B[b]) with element strides sa/sb/sc between batch entries.
void gemm(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K, const float* A,
          size_t lda, size_t sa, const float* B, size_t ldb, size_t sb, float* C, size_t ldc, size_t sc,
          size_t batch, const GemmEpi& epi);

// row_loss / row_correct: optional caller-owned [B] workspaces (else from the context cache).
void softmax_ce(orca_hip_ctx* ctx, const float* logits, size_t B, size_t C, const float* onehot,
                const int32_t* labels, float* loss, float* dlogits, int32_t* preds, int64_t* correct,
                float* row_loss = nullptr, int* row_correct = nullptr);

// Fused classifier head (last Linear with at most HEAD_MAX_CLASSES outputs +
// softmax cross-entropy); see head.hip.
constexpr size_t HEAD_MAX_CLASSES = 16;
struct HeadWorkspace {
  float* row_loss = nullptr;   // [B] per-row loss terms
  int* row_correct = nullptr;  // [B] per-row prediction == target
};
bool head_supported(size_t B, size_t K, size_t C);
// logits, dlogits, preds and the per-row terms in ws (no host sync).
void head_forward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, const float* bias, size_t C,
                  const float* onehot, const int32_t* labels, float* logits, float* dlogits, int32_t* preds,
                  const HeadWorkspace& ws);
// loss = mean of the row terms, correct = their count (one small kernel).
void head_finish(orca_hip_ctx* ctx, const HeadWorkspace& ws, size_t B, float* loss, int64_t* correct);
// dW, db, dH; when `finish` is set, also what head_finish computes.
void head_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, size_t C,
                   const float* dlogits, bool mask, float* dH, float* dW, float* db, const HeadWorkspace* finish,
                   float* loss, int64_t* correct, float* dh_colsum = nullptr);

// AdamW's per-step f32 scalars: the f64 expressions of python/orca/optim/adamw.py:64-94
// rounded to f32 as PyO3 passes them.
struct AdamWScalars {
  float decay, b1, omb1, b2, omb2, c1, c2, eps, lr;
};
AdamWScalars adamw_scalars(double lr, double b1, double b2, double eps, double wd, int64_t t);
// Writes s to device memory `dst` with a one-thread kernel on `stream` (by-value
// argument: a captured graph that reads dst sees each step's values).
void adamw_store_scalars(orca_hip_ctx* ctx, AdamWScalars* dst, const AdamWScalars& s, hipStream_t stream);

// Optimizer passes over flat buffers, on `stream` (the context stream when null).
// adamw: the scalars come from (lr, ..., t), or from device memory when dev_scalars is set;
// the parameters are read from p_src when it is set (and written to p), else updated in place;
// blocks_per_cu > 0 bounds the grid to that many blocks per CU (an update beside a GEMM).
void adamw(orca_hip_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, double lr, double b1,
           double b2, double eps, double wd, int64_t t, hipStream_t stream = nullptr,
           const AdamWScalars* dev_scalars = nullptr, const float* p_src = nullptr, int blocks_per_cu = 0);
void sgd(orca_hip_ctx* ctx, float* p, const float* g, size_t n, double lr, hipStream_t stream = nullptr);

}  // namespace orca_hip
