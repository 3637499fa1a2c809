// CPU sanitizer test of the host-only runtime (orcaml_amd/csrc/runtime_host.cpp)
// against the HIP API stand-in in tests/native/hip_stub: the caching allocator and
// its extent checks, the error guard and per-call output release, the
// out-of-memory retry, counted host waits, the pinned staging ring (including
// its back-pressure waits and chunking) and the profiler's bookkeeping.  Built
// with -fsanitize=address,undefined by tests/test_native_sanitize.py.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

#include "runtime.hpp"

using namespace orca_hip;

#define CHECK(cond)                                                          \
  do {                                                                       \
    if (!(cond)) {                                                           \
      std::fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
      std::abort();                                                          \
    }                                                                        \
  } while (0)

static size_t live_bytes(orca_hip_ctx& ctx) {
  size_t live = 0, cached = 0, mallocs = 0;
  ctx.alloc.stats(&live, &cached, &mallocs);
  return live;
}

static void allocator_and_extents(orca_hip_ctx& ctx) {
  CHECK(CachingAllocator::round_size(1) == 256 && CachingAllocator::round_size(1000) == 1024);
  for (size_t b = 1; b < (size_t(64) << 20); b = b * 3 + 7) {
    const size_t r = CachingAllocator::round_size(b);
    // granule: 256 B up to 1 MiB, then max(1 MiB, 1/8 of the leading power of two)
    CHECK(r >= b && r % 256 == 0 && (b <= (size_t(1) << 20) ? r - b < 256 : r - b < std::max(b / 8, size_t(1) << 20)));
  }
  void* a = ctx.alloc.allocate(1000, nullptr);
  CHECK(a && live_bytes(ctx) == 1024);
  ctx.alloc.release(a);
  void* b = ctx.alloc.allocate(1024, nullptr);  // same size class: the cached block comes back
  CHECK(b == a);
  size_t ext = 0;
  CHECK(ctx.alloc.locate(static_cast<char*>(b) + 100, &ext) == CachingAllocator::Where::kLive && ext == 924);
  int rc = guard([&] { check_extent(&ctx, static_cast<char*>(b) + 100, 925, "overrun"); });
  CHECK(rc == ORCA_HIP_ERR_SHAPE && std::strstr(last_error_cstr(), "Shape mismatch during overrun"));
  rc = guard([&] { check_extent(&ctx, static_cast<char*>(b) + 100, 924, "fits"); });
  CHECK(rc == ORCA_HIP_OK);
  ctx.alloc.release(b);
  CHECK(ctx.alloc.locate(static_cast<char*>(b) + 8, &ext) == CachingAllocator::Where::kFreed);
  rc = guard([&] { check_extent(&ctx, static_cast<char*>(b) + 8, 4, "after free"); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && std::strstr(last_error_cstr(), "freed"));
  int local = 0;
  rc = guard([&] { check_extent(&ctx, &local, 4, "foreign"); });  // memory the allocator never saw
  CHECK(rc == ORCA_HIP_OK);
  rc = guard([&] { ctx.alloc.release(&local); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && std::strstr(last_error_cstr(), "not owned"));
  CHECK(ctx.alloc.extent_from(b) == 0);
}

static void outputs_released_on_failure(orca_hip_ctx& ctx) {
  const size_t before = live_bytes(ctx);
  int rc = guard([&] {
    new_output(&ctx, 300);
    new_output(&ctx, 5000);
    fail(ORCA_HIP_ERR_SHAPE, "rejected after allocating");
  });
  CHECK(rc == ORCA_HIP_ERR_SHAPE && live_bytes(ctx) == before);
  float* kept = nullptr;
  rc = guard([&] { kept = new_output(&ctx, 300); });
  CHECK(rc == ORCA_HIP_OK && kept && live_bytes(ctx) == before + 1280);
  ctx.alloc.release(kept);
  // an exception that is not an Error still releases and maps to InternalError
  rc = guard([&] {
    new_output(&ctx, 64);
    throw std::runtime_error("boom");
  });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && live_bytes(ctx) == before && std::strstr(last_error_cstr(), "boom"));
}

static void out_of_memory_retry(orca_hip_ctx& ctx) {
  void* c = ctx.alloc.allocate(size_t(3) << 20, nullptr);
  ctx.alloc.release(c);  // cached
  const uint64_t syncs = ctx.host_syncs.load();
  hip_stub::fail_next_mallocs() = 1;  // first hipMalloc fails: the cache is emptied and the call retried
  void* d = ctx.alloc.allocate(size_t(5) << 20, reinterpret_cast<hipStream_t>(&ctx));
  CHECK(d && ctx.host_syncs.load() == syncs + 1);
  size_t live = 0, cached = 0, mallocs = 0;
  ctx.alloc.stats(&live, &cached, &mallocs);
  CHECK(cached == 0);
  ctx.alloc.release(d);
  hip_stub::fail_next_mallocs() = 2;  // both attempts fail: an InternalError, nothing leaked
  const int rc = guard([&] { ctx.alloc.allocate(size_t(7) << 20, nullptr); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && std::strstr(last_error_cstr(), "allocation"));
}

static void staging_ring(orca_hip_ctx& ctx) {
  // Sizes around the region and ring sizes, odd byte counts included.
  const size_t sizes[] = {3, 1024, 4099, StagingRing::kChunk - 1, StagingRing::kChunk, StagingRing::kChunk + 5,
                          StagingRing::kCapacity, 3 * StagingRing::kCapacity + 12345};
  for (int delay : {0, 1, 5}) {
    hip_stub::event_delay() = delay;
    for (size_t n : sizes) {
      std::vector<unsigned char> src(n), dst(n, 0);
      for (size_t i = 0; i < n; ++i) src[i] = static_cast<unsigned char>(i * 131 + n + delay);
      const uint64_t before = ctx.host_syncs.load();
      ctx.staging.upload(&ctx, dst.data(), src.data(), n, nullptr);
      CHECK(std::memcmp(dst.data(), src.data(), n) == 0);
      const uint64_t waits = ctx.host_syncs.load() - before;
      if (delay == 0) CHECK(waits == 0);  // finished copies are retired without waiting
      if (n <= StagingRing::kChunk / 2) CHECK(waits <= 1);  // one region: at most the oldest copy is awaited
    }
  }
  // many small uploads recycle regions in ring order
  hip_stub::event_delay() = 2;
  std::vector<float> host(777), dev(777);
  for (int i = 0; i < 5000; ++i) {
    for (size_t k = 0; k < host.size(); ++k) host[k] = float(i) + float(k);
    ctx.staging.upload(&ctx, dev.data(), host.data(), host.size() * sizeof(float), nullptr);
    CHECK(dev[0] == float(i) && dev[776] == float(i) + 776.0f);
  }
  hip_stub::event_delay() = 0;
}

static void waits_and_profiler(orca_hip_ctx& ctx) {
  const uint64_t before = ctx.host_syncs.load();
  host_sync(&ctx);
  hipEvent_t e;
  CHECK(hipEventCreate(&e) == hipSuccess);
  host_wait_event(&ctx, e);
  CHECK(hipEventDestroy(e) == hipSuccess);
  CHECK(ctx.host_syncs.load() == before + 2);
  ctx.prof.enabled = true;
  for (int i = 0; i < 3; ++i) ProfScope ps(&ctx, "k", 10.0, 20.0);
  ctx.prof.drain();
  CHECK(ctx.prof.agg["k"].launches == 3 && ctx.prof.agg["k"].flops == 30.0);
  ctx.prof.enabled = false;
}

// A host wait on the context stream first makes it wait for the side stream's
// work (once per recording), and not while launches go to the side stream.
static void side_stream_join(orca_hip_ctx& ctx) {
  hipStream_t side = reinterpret_cast<hipStream_t>(&ctx);  // any non-null handle: the stand-in ignores it
  CHECK(hipEventCreate(&ctx.side_last) == hipSuccess);
  CHECK(hipEventRecord(ctx.side_last, side) == hipSuccess);
  ctx.side = side;
  ctx.side_joined = false;
  const long waits = hip_stub::stream_waits();
  host_sync(&ctx);
  CHECK(hip_stub::stream_waits() == waits + 1 && ctx.side_joined);
  host_sync(&ctx);
  CHECK(hip_stub::stream_waits() == waits + 1);
  ctx.side_joined = false;
  ctx.main = side;  // launches on the side stream (the stand-in handle): no join
  join_side(&ctx);
  CHECK(hip_stub::stream_waits() == waits + 1 && !ctx.side_joined);
  // and no allocation: the allocator orders block reuse by the context stream alone
  const size_t live_before = live_bytes(ctx);
  int rc = guard([&] { new_output(&ctx, 16); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && std::strstr(last_error_cstr(), "side stream") && live_bytes(ctx) == live_before);
  rc = guard([&] { Scratch s(&ctx, 64); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL && live_bytes(ctx) == live_before);
  rc = guard([&] { ctx_allocate(&ctx, 64); });
  CHECK(rc == ORCA_HIP_ERR_INTERNAL);
  ctx.main = nullptr;
  join_side(&ctx);
  CHECK(hip_stub::stream_waits() == waits + 2 && ctx.side_joined);
  CHECK(hipEventDestroy(ctx.side_last) == hipSuccess);
  ctx.side_last = nullptr;
  ctx.side = nullptr;
}

int main() {
  {
    orca_hip_ctx ctx;
    ctx.alloc.sync_counter = &ctx.host_syncs;
    allocator_and_extents(ctx);
    outputs_released_on_failure(ctx);
    out_of_memory_retry(ctx);
    staging_ring(ctx);
    waits_and_profiler(ctx);
    side_stream_join(ctx);
    ctx.alloc.empty(nullptr);
  }  // the context's destructor frees every block, event and the pinned ring
  CHECK(hip_stub::device_mallocs() == hip_stub::device_frees());
  std::printf("runtime host test: all checks passed\n");
  return 0;
}
