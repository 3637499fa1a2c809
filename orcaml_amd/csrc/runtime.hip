// Context, caching allocator, host I/O, timing and the small copy/fill
// kernels of liborca_hip.so.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <sstream>

#include "runtime.hpp"

namespace orca_hip {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }

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
  // Above 1 MiB: granule of 1/8 of the leading power of two (<= 12.5% slack).
  size_t p = size_t(1) << (63 - __builtin_clzll(bytes));
  size_t g = std::max<size_t>(p / 8, 1u << 20);
  return (bytes + g - 1) / g * g;
}

void* CachingAllocator::allocate(size_t bytes, hipStream_t stream) {
  size_t r = round_size(bytes);
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = cached_.find(r);
    if (it != cached_.end()) {
      void* p = it->second;
      cached_.erase(it);
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

void CachingAllocator::release(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  if (it == live_.end()) fail(ORCA_HIP_ERR_INTERNAL, "orca_hip_free: pointer not owned by this context");
  size_t r = it->second;
  live_.erase(it);
  live_bytes_ -= r;
  cached_.emplace(r, p);
  cached_bytes_ += r;
}

size_t CachingAllocator::size_of(void* p) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  return it == live_.end() ? 0 : it->second;
}

size_t CachingAllocator::extent_from(const void* p) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.upper_bound(const_cast<void*>(p));
  if (it == live_.begin()) return 0;
  --it;
  const char* base = static_cast<const char*>(it->first);
  const char* q = static_cast<const char*>(p);
  if (q >= base && q < base + it->second) return static_cast<size_t>(base + it->second - q);
  return 0;
}

void check_extent(orca_hip_ctx* ctx, const void* p, size_t bytes, const char* what) {
  if (!p || !bytes) return;
  const size_t have = ctx->alloc.extent_from(p);
  if (have && bytes > have)
    fail(ORCA_HIP_ERR_SHAPE, std::string("Shape mismatch during ") + what + ": the access spans " +
                                 std::to_string(bytes) + " bytes but the buffer has " + std::to_string(have) +
                                 " from this pointer");
}

void CachingAllocator::empty(hipStream_t stream) {
  if (stream) (void)hipStreamSynchronize(stream);
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& kv : cached_) (void)hipFree(kv.second);
  cached_.clear();
  cached_bytes_ = 0;
}

void CachingAllocator::stats(size_t* live, size_t* cached, size_t* mallocs) {
  std::lock_guard<std::mutex> lk(mu_);
  if (live) *live = live_bytes_;
  if (cached) *cached = cached_bytes_;
  if (mallocs) *mallocs = mallocs_;
}

CachingAllocator::~CachingAllocator() {
  for (auto& kv : cached_) (void)hipFree(kv.second);
  for (auto& kv : live_) (void)hipFree(kv.first);
}

// ------------------------------------------------------------ profiler
hipEvent_t Profiler::get_event() {
  if (!pool.empty()) {
    hipEvent_t e = pool.back();
    pool.pop_back();
    return e;
  }
  hipEvent_t e;
  ORCA_HIP_CHECK(hipEventCreate(&e));
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

// ------------------------------------------------------------ small kernels
__global__ void fill_kernel(float* __restrict__ dst, float v, size_t n) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = v;
}

__global__ void copy_kernel(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// One thread per column, rows in ascending order: the accumulation order of
// orca-backend-cpu's sum_to_shape (backend.rs:519-527) for [R,C] -> [1,C].

void launch_fill(orca_hip_ctx* ctx, float* dst, float v, size_t n) {
  if (n == 0) return;
  unsigned g = grid_for(n, 256, 4096);
  hipLaunchKernelGGL(fill_kernel, dim3(g), dim3(256), 0, ctx->stream, dst, v, n);
  ORCA_HIP_CHECK(hipGetLastError());
}

void launch_copy(orca_hip_ctx* ctx, float* dst, const float* src, size_t n) {
  if (n == 0) return;
  unsigned g = grid_for(n, 256, 4096);
  hipLaunchKernelGGL(copy_kernel, dim3(g), dim3(256), 0, ctx->stream, dst, src, n);
  ORCA_HIP_CHECK(hipGetLastError());
}


float* new_output(orca_hip_ctx* ctx, size_t n) {
  return static_cast<float*>(ctx->alloc.allocate(n * sizeof(float), ctx->stream));
}

}  // namespace orca_hip

using namespace orca_hip;

// ============================================================== C ABI
extern "C" {

const char* orca_hip_last_error(void) { return g_last_error.c_str(); }

int orca_hip_ctx_create(int device, orca_hip_ctx** out) {
  return guard([&] {
    if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    int count = 0;
    ORCA_HIP_CHECK(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
      fail(ORCA_HIP_ERR_INTERNAL, "HIP device " + std::to_string(device) + " not present (" +
                                      std::to_string(count) + " visible)");
    ORCA_HIP_CHECK(hipSetDevice(device));
    hipDeviceProp_t prop;
    ORCA_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    auto* ctx = new orca_hip_ctx();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&ctx->timer_start);
    if (e == hipSuccess) e = hipEventCreate(&ctx->timer_stop);
    if (e != hipSuccess) {
      delete ctx;
      fail(ORCA_HIP_ERR_INTERNAL, std::string("context setup failed: ") + hipGetErrorString(e));
    }
    *out = ctx;
  });
}

int orca_hip_ctx_destroy(orca_hip_ctx* ctx) {
  return guard([&] {
    if (!ctx) return;
    bind(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->timer_start) (void)hipEventDestroy(ctx->timer_start);
    if (ctx->timer_stop) (void)hipEventDestroy(ctx->timer_stop);
    hipStream_t s = ctx->stream;
    delete ctx;  // allocator and profiler release their resources
    if (s) (void)hipStreamDestroy(s);
  });
}

int orca_hip_device(const orca_hip_ctx* ctx, int* ordinal) {
  return guard([&] {
    check_ctx(ctx);
    if (!ordinal) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    *ordinal = ctx->device;
  });
}

int orca_hip_alloc(orca_hip_ctx* ctx, size_t bytes, void** out) {
  return guard([&] {
    bind(ctx);
    if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    *out = ctx->alloc.allocate(bytes, ctx->stream);
  });
}

int orca_hip_free(orca_hip_ctx* ctx, void* ptr) {
  return guard([&] {
    check_ctx(ctx);
    ctx->alloc.release(ptr);
  });
}

int orca_hip_empty_cache(orca_hip_ctx* ctx) {
  return guard([&] {
    bind(ctx);
    ctx->alloc.empty(ctx->stream);
  });
}

int orca_hip_mem_stats(orca_hip_ctx* ctx, size_t* live, size_t* cached, size_t* device_allocs) {
  return guard([&] {
    check_ctx(ctx);
    ctx->alloc.stats(live, cached, device_allocs);
  });
}

int orca_hip_h2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    bind(ctx);
    if (!bytes) return;
    check_extent(ctx, dst, bytes, "h2d");
    ORCA_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    ORCA_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int orca_hip_d2h(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    bind(ctx);
    if (!bytes) return;
    check_extent(ctx, src, bytes, "d2h");
    ORCA_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    ORCA_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int orca_hip_d2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    bind(ctx);
    if (!bytes) return;
    check_extent(ctx, dst, bytes, "d2d");
    check_extent(ctx, src, bytes, "d2d");
    ORCA_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  });
}

int orca_hip_fill(orca_hip_ctx* ctx, float* dst, float value, size_t n) {
  return guard([&] {
    bind(ctx);
    check_extent(ctx, dst, n * sizeof(float), "fill");
    launch_fill(ctx, dst, value, n);
  });
}

int orca_hip_sync(orca_hip_ctx* ctx) {
  return guard([&] {
    bind(ctx);
    ORCA_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int orca_hip_prof_enable(orca_hip_ctx* ctx, int enable) {
  return guard([&] {
    check_ctx(ctx);
    ctx->prof.enabled = enable != 0;
  });
}

int orca_hip_prof_reset(orca_hip_ctx* ctx) {
  return guard([&] {
    bind(ctx);
    ORCA_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    ctx->prof.drain();
    ctx->prof.agg.clear();
  });
}

int orca_hip_prof_report(orca_hip_ctx* ctx, char* buf, size_t len) {
  return guard([&] {
    bind(ctx);
    ORCA_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    ctx->prof.drain();
    std::ostringstream os;
    os << "{\"num_cus\": " << ctx->num_cus << ", \"kernels\": [";
    bool first = true;
    for (auto& kv : ctx->prof.agg) {
      os << (first ? "" : ", ") << "{\"name\": \"" << kv.first << "\", \"launches\": " << kv.second.launches
         << ", \"total_ms\": " << kv.second.total_ms << ", \"flops\": " << kv.second.flops
         << ", \"bytes\": " << kv.second.bytes << "}";
      first = false;
    }
    os << "]}";
    std::string s = os.str();
    if (!buf || len < s.size() + 1) fail(ORCA_HIP_ERR_INTERNAL, "report buffer too small (" + std::to_string(s.size() + 1) + " bytes needed)");
    std::memcpy(buf, s.c_str(), s.size() + 1);
  });
}

int orca_hip_timer_start(orca_hip_ctx* ctx) {
  return guard([&] {
    bind(ctx);
    ORCA_HIP_CHECK(hipEventRecord(ctx->timer_start, ctx->stream));
  });
}

int orca_hip_timer_stop(orca_hip_ctx* ctx, float* ms) {
  return guard([&] {
    bind(ctx);
    ORCA_HIP_CHECK(hipEventRecord(ctx->timer_stop, ctx->stream));
    ORCA_HIP_CHECK(hipEventSynchronize(ctx->timer_stop));
    ORCA_HIP_CHECK(hipEventElapsedTime(ms, ctx->timer_start, ctx->timer_stop));
  });
}

}  // extern "C"
