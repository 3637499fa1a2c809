// Context and host I/O entry points, stream-ordered uploads and the small
// copy / fill kernels of liborca_hip.so (the host-only runtime is in
// runtime_host.cpp).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "runtime.hpp"

namespace orca_hip {
// Up to 1 KiB of host data handed to the device as a kernel argument: it is
// captured at launch, so nothing is left for the host to keep alive or wait for.
struct SmallPayload {
  uint32_t words;
  uint32_t data[256];
};

__global__ void store_payload_kernel(uint32_t* __restrict__ dst, SmallPayload p) {
  for (uint32_t i = threadIdx.x; i < p.words; i += blockDim.x) dst[i] = p.data[i];
}

void upload_async(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!bytes) return;
  if (bytes % 4 == 0 && bytes <= sizeof(SmallPayload::data) && reinterpret_cast<uintptr_t>(dst) % 4 == 0) {
    SmallPayload p;
    p.words = static_cast<uint32_t>(bytes / 4);
    std::memcpy(p.data, src, bytes);
    hipLaunchKernelGGL(store_payload_kernel, dim3(1), dim3(64), 0, ctx->stream, static_cast<uint32_t*>(dst), p);
    ORCA_HIP_CHECK(hipGetLastError());
    return;
  }
  ctx->staging.upload(ctx, dst, src, bytes, ctx->stream);
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


}  // namespace orca_hip

using namespace orca_hip;

// Events that order the two streams of one context: no system-scope fence at
// record (the kernels' own release and acquire are at device scope).
static constexpr unsigned kOrderEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;

namespace orca_hip {
hipEvent_t take_order_event(orca_hip_ctx* ctx) {
  hipEvent_t ev = nullptr;
  if (!ctx->event_pool.empty()) {
    ev = ctx->event_pool.back();
    ctx->event_pool.pop_back();
  } else {
    ORCA_HIP_CHECK(hipEventCreateWithFlags(&ev, kOrderEventFlags));
  }
  return ev;
}
}  // namespace orca_hip

// ============================================================== C ABI
extern "C" {

const char* orca_hip_last_error(void) { return last_error_cstr(); }

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
    ctx->alloc.sync_counter = &ctx->host_syncs;
    if (const char* v = std::getenv("ORCA_HIP_GEMM_FAST")) ctx->gemm_generic_only = v[0] == '0';
    if (const char* v = std::getenv("ORCA_HIP_GEMM_SMALL_TILES")) ctx->gemm_small_tiles = v[0] != '0';
    if (const char* v = std::getenv("ORCA_HIP_GEMM_SKINNY")) ctx->gemm_skinny = v[0] != '0';
    if (const char* v = std::getenv("ORCA_HIP_GEMM_NARROW")) ctx->gemm_narrow = v[0] != '0';
    if (const char* v = std::getenv("ORCA_HIP_GEMM_BAND")) ctx->gemm_band = v[0] == '0' ? 0 : v[0] == '1' ? 1 : 2;
    if (const char* v = std::getenv("ORCA_HIP_EW_JIT")) ctx->ew_jit_mode = v[0] == '0' ? 0 : v[0] == '2' ? 2 : 1;
    if (const char* v = std::getenv("ORCA_HIP_GEMM_TILE")) {
      if (std::strcmp(v, "128x128") == 0) ctx->gemm_tile_bn = 128;
      if (std::strcmp(v, "128x64") == 0) ctx->gemm_tile_bn = 64;
    }
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
    if (ctx->main) ctx->stream = ctx->main;
    if (ctx->side) (void)hipStreamSynchronize(ctx->side);
    (void)hipStreamSynchronize(ctx->stream);
    ew_jit_release(ctx);
    if (ctx->timer_start) (void)hipEventDestroy(ctx->timer_start);
    if (ctx->timer_stop) (void)hipEventDestroy(ctx->timer_stop);
    if (ctx->side_last) (void)hipEventDestroy(ctx->side_last);
    for (hipEvent_t ev : ctx->event_pool) (void)hipEventDestroy(ev);
    hipStream_t s = ctx->stream, side = ctx->side;
    delete ctx;  // allocator and profiler release their resources
    if (s) (void)hipStreamDestroy(s);
    if (side) (void)hipStreamDestroy(side);
  });
}

int orca_hip_use_side_stream(orca_hip_ctx* ctx, int blocks_per_cu) {
  return guard([&] {
    bind(ctx);
    if (blocks_per_cu) {
      if (ctx->main) fail(ORCA_HIP_ERR_INTERNAL, "launches already go to the side stream");
      if (!ctx->side) {
        ORCA_HIP_CHECK(hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking));
        ORCA_HIP_CHECK(hipEventCreateWithFlags(&ctx->side_last, kOrderEventFlags));
      }
      ctx->main = ctx->stream;
      ctx->stream = ctx->side;
      ctx->side_bpc = blocks_per_cu > 0 ? blocks_per_cu : 0;
    } else {
      if (!ctx->main) fail(ORCA_HIP_ERR_INTERNAL, "launches do not go to the side stream");
      ORCA_HIP_CHECK(hipEventRecord(ctx->side_last, ctx->side));
      ctx->side_joined = false;
      ctx->stream = ctx->main;
      ctx->main = nullptr;
    }
  });
}

int orca_hip_event_record(orca_hip_ctx* ctx, orca_hip_event** out) {
  return guard([&] {
    bind(ctx);
    if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    hipEvent_t ev = take_order_event(ctx);
    const hipError_t e = hipEventRecord(ev, ctx->stream);
    if (e != hipSuccess) {
      (void)hipEventDestroy(ev);
      ORCA_HIP_CHECK(e);
    }
    *out = reinterpret_cast<orca_hip_event*>(ev);
  });
}

int orca_hip_event_wait(orca_hip_ctx* ctx, orca_hip_event* ev) {
  return guard([&] {
    bind(ctx);
    if (!ev) fail(ORCA_HIP_ERR_INTERNAL, "null event");
    ORCA_HIP_CHECK(hipStreamWaitEvent(ctx->stream, reinterpret_cast<hipEvent_t>(ev), 0));
  });
}

// A wait already enqueued keeps the record it was enqueued after, so a released
// event can be recorded again.
int orca_hip_event_release(orca_hip_ctx* ctx, orca_hip_event* ev) {
  return guard([&] {
    check_ctx(ctx);
    if (ev) ctx->event_pool.push_back(reinterpret_cast<hipEvent_t>(ev));
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
    *out = ctx_allocate(ctx, bytes);
  });
}

int orca_hip_free(orca_hip_ctx* ctx, void* ptr) {
  return guard([&] {
    check_ctx(ctx);
    ctx->alloc.release(ptr);
  });
}

int orca_hip_free_many(orca_hip_ctx* ctx, void* const* ptrs, size_t n) {
  return guard([&] {
    check_ctx(ctx);
    if (n && !ptrs) fail(ORCA_HIP_ERR_INTERNAL, "free_many: null pointer array");
    for (size_t i = 0; i < n; ++i) ctx->alloc.release(ptrs[i]);
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
    host_sync(ctx);
  });
}

int orca_hip_d2h(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    bind(ctx);
    if (!bytes) return;
    check_extent(ctx, src, bytes, "d2h");
    join_side(ctx);
    ORCA_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    host_sync(ctx);
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
    host_sync(ctx);
  });
}

int orca_hip_sync_count(const orca_hip_ctx* ctx, uint64_t* count) {
  return guard([&] {
    check_ctx(ctx);
    if (!count) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    *count = ctx->host_syncs.load(std::memory_order_relaxed);
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
    host_sync(ctx);
    ctx->prof.drain();
    ctx->prof.agg.clear();
  });
}

int orca_hip_prof_report(orca_hip_ctx* ctx, char* buf, size_t len) {
  return guard([&] {
    bind(ctx);
    host_sync(ctx);
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
    host_wait_event(ctx, ctx->timer_stop);
    ORCA_HIP_CHECK(hipEventElapsedTime(ms, ctx->timer_start, ctx->timer_stop));
  });
}

}  // extern "C"
