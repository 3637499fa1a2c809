// Host-only part of the runtime shared by every translation unit of
// liborca_hip.so: error messages, the caching allocator and its extent checks,
// per-launch event timing, counted host waits, the pinned staging ring and the
// per-call output tracking.  It launches no kernel, so it also builds with a
// plain C++ compiler against a HIP API stand-in for the sanitizer test
// (tests/native).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "runtime.hpp"

namespace orca_hip {

static thread_local std::string g_last_error;
static thread_local int g_last_code = ORCA_HIP_OK;
static thread_local ErrorFields g_last_fields;

void set_last_error(const std::string& msg) {
  g_last_error = msg;
  g_last_code = ORCA_HIP_ERR_INTERNAL;
  g_last_fields = ErrorFields{};
}

void set_last_error(const std::string& msg, int code, const ErrorFields& fields) {
  g_last_error = msg;
  g_last_code = code;
  g_last_fields = fields;
}

void last_error_info(orca_hip_error_info* out) {
  out->code = g_last_error.empty() ? ORCA_HIP_OK : g_last_code;
  out->op = g_last_fields.op.c_str();
  out->expected = g_last_fields.expected.c_str();
  out->got = g_last_fields.got.c_str();
  out->dtype = g_last_fields.dtype;
  out->dtype_got = g_last_fields.dtype_got;
  for (int i = 0; i < 2; ++i) {
    out->device_kind[i] = g_last_fields.device_kind[i];
    out->device_index[i] = g_last_fields.device_index[i];
  }
  out->message = g_last_error.c_str();
}

const char* dtype_name(int dtype) {  // orca-core/src/dtype.rs Display
  static const char* names[] = {"float32", "float64", "float16", "bfloat16", "int32", "int64", "uint8", "bool"};
  return dtype >= 0 && dtype < 8 ? names[dtype] : "unknown";
}

void fail_shape(const std::string& op, const std::string& expected, const std::string& got) {
  ErrorFields f;
  f.op = op;
  f.expected = expected;
  f.got = got;
  throw Error(ORCA_HIP_ERR_SHAPE, "Shape mismatch during " + op + ": expected " + expected + ", got " + got,
              std::move(f));
}

void fail_dtype(const std::string& op, int dtype) {
  ErrorFields f;
  f.op = op;
  f.dtype = dtype;
  throw Error(ORCA_HIP_ERR_UNSUPPORTED_DTYPE, "Unsupported dtype for " + op + ": " + dtype_name(dtype), std::move(f));
}

void fail_device(int gpu_a, int gpu_b) {
  ErrorFields f;
  f.device_kind[0] = f.device_kind[1] = 2;  // Device::Gpu
  f.device_index[0] = gpu_a;
  f.device_index[1] = gpu_b;
  throw Error(ORCA_HIP_ERR_DEVICE_MISMATCH,
              "Device mismatch: tensors must be on the same device. Got gpu:" + std::to_string(gpu_a) + " and gpu:" +
                  std::to_string(gpu_b),
              std::move(f));
}

size_t numel(const size_t* shape, size_t rank) {
  size_t n = 1;
  for (size_t i = 0; i < rank; ++i) n *= shape[i];
  return n;
}

std::string shape_str(const size_t* shape, size_t rank) {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < rank; ++i) os << (i ? ", " : "") << shape[i];
  os << "]";
  return os.str();
}

void bind(orca_hip_ctx* ctx) {
  check_ctx(ctx);
  ORCA_HIP_CHECK(hipSetDevice(ctx->device));
}

// ------------------------------------------------------------ allocator
size_t CachingAllocator::round_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (1u << 20)) return (bytes + 255) & ~size_t(255);
  // Above 1 MiB: a granule of 1/8 of the leading power of two, at least 1 MiB
  // (at most 12.5 % slack from 8 MiB on).
  size_t p = size_t(1) << (63 - __builtin_clzll(bytes));
  size_t g = std::max<size_t>(p / 8, 1u << 20);
  return (bytes + g - 1) / g * g;
}

void* CachingAllocator::allocate(size_t bytes, hipStream_t stream) {
  size_t r = round_size(bytes);
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto hi = cached_.upper_bound(r);
    if (hi != cached_.begin() && std::prev(hi)->first == r) {  // the most recently released
      auto it = std::prev(hi);
      void* p = it->second.p;
      cached_.erase(it);
      cached_at_.erase(p);
      cached_bytes_ -= r;
      live_[p] = r;
      live_bytes_ += r;
      return p;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, r);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    empty(stream);  // give cached blocks back and retry once
    e = hipMalloc(&p, r);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      fail(ORCA_HIP_ERR_INTERNAL, "device allocation of " + std::to_string(r) + " bytes failed: " +
                                      hipGetErrorString(e));
    }
  }
  std::lock_guard<std::mutex> lk(mu_);
  ++mallocs_;
  live_[p] = r;
  live_bytes_ += r;
  return p;
}

void* CachingAllocator::allocate_released_by(size_t bytes, uint64_t clock) {
  const size_t r = round_size(bytes);
  std::lock_guard<std::mutex> lk(mu_);
  auto it = cached_.find(r);  // the oldest release of this size
  if (it == cached_.end() || it->second.released > clock) return nullptr;
  void* p = it->second.p;
  cached_.erase(it);
  cached_at_.erase(p);
  cached_bytes_ -= r;
  live_[p] = r;
  live_bytes_ += r;
  return p;
}

size_t CachingAllocator::count_released_by(size_t bytes, uint64_t clock) {
  const size_t r = round_size(bytes);
  std::lock_guard<std::mutex> lk(mu_);
  size_t n = 0;
  for (auto it = cached_.lower_bound(r); it != cached_.end() && it->first == r && it->second.released <= clock; ++it)
    ++n;
  return n;
}

uint64_t CachingAllocator::clock() {
  std::lock_guard<std::mutex> lk(mu_);
  return clock_;
}

void CachingAllocator::release(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  if (it == live_.end()) fail(ORCA_HIP_ERR_INTERNAL, "orca_hip_free: pointer not owned by this context");
  size_t r = it->second;
  live_.erase(it);
  live_bytes_ -= r;
  cached_.emplace(r, Cached{p, ++clock_});
  cached_at_[p] = r;
  cached_bytes_ += r;
}

size_t CachingAllocator::size_of(void* p) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  return it == live_.end() ? 0 : it->second;
}

// Bytes from p to the end of the block of `blocks` (address -> size) that contains p, or 0.
static size_t extent_in(const std::map<void*, size_t>& blocks, const void* p) {
  auto it = blocks.upper_bound(const_cast<void*>(p));
  if (it == blocks.begin()) return 0;
  --it;
  const char* base = static_cast<const char*>(it->first);
  const char* q = static_cast<const char*>(p);
  if (q >= base && q < base + it->second) return static_cast<size_t>(base + it->second - q);
  return 0;
}

CachingAllocator::Where CachingAllocator::locate(const void* p, size_t* extent) {
  std::lock_guard<std::mutex> lk(mu_);
  if (size_t e = extent_in(live_, p)) {
    *extent = e;
    return Where::kLive;
  }
  *extent = 0;
  return extent_in(cached_at_, p) ? Where::kFreed : Where::kUnknown;
}

size_t CachingAllocator::extent_from(const void* p) {
  std::lock_guard<std::mutex> lk(mu_);
  return extent_in(live_, p);
}

void check_extent(orca_hip_ctx* ctx, const void* p, size_t bytes, const char* what) {
  if (!p || !bytes) return;
  size_t have = 0;
  switch (ctx->alloc.locate(p, &have)) {
    case CachingAllocator::Where::kLive:
      if (bytes > have)
        fail(ORCA_HIP_ERR_SHAPE, std::string("Shape mismatch during ") + what + ": the access spans " +
                                     std::to_string(bytes) + " bytes but the buffer has " + std::to_string(have) +
                                     " from this pointer");
      break;
    case CachingAllocator::Where::kFreed:
      fail(ORCA_HIP_ERR_INTERNAL, std::string("Internal error: ") + what +
                                      " was given a pointer into a buffer that has been freed");
    case CachingAllocator::Where::kUnknown:
      break;
  }
}

void CachingAllocator::empty(hipStream_t stream) {
  if (stream) {
    if (sync_counter) sync_counter->fetch_add(1, std::memory_order_relaxed);
    (void)hipStreamSynchronize(stream);
  }
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& kv : cached_) (void)hipFree(kv.second.p);
  cached_.clear();
  cached_at_.clear();
  cached_bytes_ = 0;
}

void CachingAllocator::stats(size_t* live, size_t* cached, size_t* mallocs) {
  std::lock_guard<std::mutex> lk(mu_);
  if (live) *live = live_bytes_;
  if (cached) *cached = cached_bytes_;
  if (mallocs) *mallocs = mallocs_;
}

CachingAllocator::~CachingAllocator() {
  for (auto& kv : cached_) (void)hipFree(kv.second.p);
  for (auto& kv : live_) (void)hipFree(kv.first);
}

// ------------------------------------------------------------ profiler
hipEvent_t Profiler::get_event() {
  if (!pool.empty()) {
    hipEvent_t e = pool.back();
    pool.pop_back();
    return e;
  }
  // Timing only: no system-scope fence at record, so the stop event of a kernel
  // does not add a cache write-back to its measured duration or to the next launch.
  hipEvent_t e;
  ORCA_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  return e;
}

void Profiler::drain() {
  for (auto& p : pending) {
    float ms = 0.f;
    ORCA_HIP_CHECK(hipEventElapsedTime(&ms, p.start, p.stop));
    Agg& a = agg[p.name];
    a.launches += 1;
    a.total_ms += ms;
    a.flops += p.flops;
    a.bytes += p.bytes;
    pool.push_back(p.start);
    pool.push_back(p.stop);
  }
  pending.clear();
}

Profiler::~Profiler() {
  for (auto& p : pending) {
    (void)hipEventDestroy(p.start);
    (void)hipEventDestroy(p.stop);
  }
  for (auto e : pool) (void)hipEventDestroy(e);
}

ProfScope::ProfScope(orca_hip_ctx* ctx, const char* name, double flops, double bytes, hipStream_t stream)
    : ctx_(ctx), stream_(stream ? stream : ctx->stream), on_(ctx->prof.enabled) {
  if (!on_) return;
  rec_.name = name;
  rec_.flops = flops;
  rec_.bytes = bytes;
  rec_.start = ctx->prof.get_event();
  rec_.stop = ctx->prof.get_event();
  ORCA_HIP_CHECK(hipEventRecord(rec_.start, stream_));
}

ProfScope::~ProfScope() {
  if (!on_) return;
  if (hipEventRecord(rec_.stop, stream_) == hipSuccess) ctx_->prof.pending.push_back(rec_);
}

// ------------------------------------------------------------ host waits and uploads
void join_side(orca_hip_ctx* ctx) {
  if (ctx->side && !ctx->side_joined && !ctx->main) {
    ORCA_HIP_CHECK(hipStreamWaitEvent(ctx->stream, ctx->side_last, 0));
    ctx->side_joined = true;
  }
}

void host_sync(orca_hip_ctx* ctx, hipStream_t stream) {
  ctx->host_syncs.fetch_add(1, std::memory_order_relaxed);
  if (!stream || stream == ctx->stream) join_side(ctx);
  ORCA_HIP_CHECK(hipStreamSynchronize(stream ? stream : ctx->stream));
}

void host_wait_event(orca_hip_ctx* ctx, hipEvent_t ev) {
  ctx->host_syncs.fetch_add(1, std::memory_order_relaxed);
  ORCA_HIP_CHECK(hipEventSynchronize(ev));
}

void StagingRing::retire_finished() {
  while (!inflight_.empty()) {
    const hipError_t q = hipEventQuery(inflight_.front().done);
    if (q == hipErrorNotReady) return;
    ORCA_HIP_CHECK(q);
    spare_.push_back(inflight_.front().done);
    inflight_.pop_front();
  }
}

size_t StagingRing::reserve(orca_hip_ctx* ctx, size_t need) {
  for (;;) {
    retire_finished();
    if (inflight_.empty()) {
      head_ = 0;
      return 0;
    }
    // The regions in flight occupy [tail, head_) in ring order; head_ == tail
    // with regions in flight means the ring is full.
    const size_t tail = inflight_.front().begin;
    if (head_ > tail) {
      if (kCapacity - head_ >= need) return head_;
      if (tail >= need) return 0;
    } else if (head_ < tail && tail - head_ >= need) {
      return head_;
    }
    host_wait_event(ctx, inflight_.front().done);  // back-pressure: wait for the oldest copy
  }
}

void StagingRing::upload(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(mu_);
  if (!base_) ORCA_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&base_), kCapacity, hipHostMallocDefault));
  char* d = static_cast<char*>(dst);
  const char* h = static_cast<const char*>(src);
  while (bytes) {
    const size_t part = std::min(bytes, kChunk);
    const size_t need = (part + 255) & ~size_t(255);
    const size_t off = reserve(ctx, need);
    std::memcpy(base_ + off, h, part);
    ORCA_HIP_CHECK(hipMemcpyAsync(d, base_ + off, part, hipMemcpyHostToDevice, stream));
    hipEvent_t ev;
    if (spare_.empty()) {
      ORCA_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    } else {
      ev = spare_.back();
      spare_.pop_back();
    }
    ORCA_HIP_CHECK(hipEventRecord(ev, stream));
    inflight_.push_back(Region{off, off + need, ev});
    head_ = off + need;
    d += part;
    h += part;
    bytes -= part;
  }
}

StagingRing::~StagingRing() {
  // The owning context has synchronised its stream before it is destroyed.
  for (auto& r : inflight_) (void)hipEventDestroy(r.done);
  for (auto e : spare_) (void)hipEventDestroy(e);
  if (base_) (void)hipHostFree(base_);
}

namespace {
struct CallOutputs {
  int depth = 0;
  std::vector<std::pair<orca_hip_ctx*, void*>> made;
};
thread_local CallOutputs g_outputs;
}  // namespace

void outputs_begin() {
  if (g_outputs.depth++ == 0) g_outputs.made.clear();
}

void outputs_commit() {
  if (--g_outputs.depth == 0) g_outputs.made.clear();
}

void outputs_abort() {
  if (--g_outputs.depth != 0) return;
  for (auto& cp : g_outputs.made) {
    try {
      cp.first->alloc.release(cp.second);
    } catch (...) {
    }
  }
  g_outputs.made.clear();
}

void* ctx_allocate(orca_hip_ctx* ctx, size_t bytes) {
  if (ctx->main)
    fail(ORCA_HIP_ERR_INTERNAL,
         "Internal error: a device allocation was requested while launches go to the side stream "
         "(only non-allocating launches may run there)");
  return ctx->alloc.allocate(bytes, ctx->stream);
}

void* ctx_allocate_released_by(orca_hip_ctx* ctx, size_t bytes, uint64_t clock) {
  if (ctx->main)
    fail(ORCA_HIP_ERR_INTERNAL,
         "Internal error: a device allocation was requested while launches go to the side stream "
         "(only non-allocating launches may run there)");
  return ctx->alloc.allocate_released_by(bytes, clock);
}

size_t ctx_count_released_by(orca_hip_ctx* ctx, size_t bytes, uint64_t clock) {
  return ctx->alloc.count_released_by(bytes, clock);
}

uint64_t ctx_release_clock(orca_hip_ctx* ctx) { return ctx->alloc.clock(); }

float* new_output(orca_hip_ctx* ctx, size_t n) {
  void* p = ctx_allocate(ctx, n * sizeof(float));
  g_outputs.made.emplace_back(ctx, p);
  return static_cast<float*>(p);
}


const char* last_error_cstr() { return g_last_error.c_str(); }

}  // namespace orca_hip
