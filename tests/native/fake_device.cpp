// A host stand-in of liborca_hip.so's buffer-level entry points (test infrastructure):
// "device" memory is host memory from the context's caching allocator (over the HIP
// stand-in in hip_stub/), and every kernel is computed with the oracle's C ops
// (oracle/orca_ops.c), one array pass per op.  Linked with the storage layer
// (orcaml_amd/csrc/storage.cpp) and the host runtime it makes a CPU library with the
// same storage-handle ABI, so the planner's decisions -- which chains become one
// program, which values a program writes, which products fold into an epilogue,
// when constants upload, what runs on the second stream -- can be checked on the
// CPU.  Each launch is appended to a text log (fake_log_text).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "orca_oracle.h"
#include "runtime.hpp"

using namespace orca_hip;

namespace {
std::string g_log;

void logf(const std::string& line) {
  g_log += line;
  g_log += '\n';
}

float* F(const void* p) { return static_cast<float*>(const_cast<void*>(p)); }

// ---- a happens-before check of a context's two streams.  Launches are synchronous here,
// so an order that only the real GPU would get wrong has to be checked: every launch
// declares the byte ranges it reads and writes, and an access on one stream to a range that
// the other stream touched after the last of its points this stream waited for (an event,
// or a host read's join) is logged as "RACE <launch> ...".
struct Range {
  uintptr_t lo, hi;
  uint64_t main_write, main_read, side_write, side_read;  // each stream's launch count at its last access
};
struct Streams {
  uint64_t main_clock = 0, side_clock = 0;            // launches so far on each stream
  uint64_t side_knows_main = 0, main_knows_side = 0;  // the other stream's launches each has waited for
  uint64_t side_at_switch = 0;                        // side launches when launches last went back
  std::vector<Range> ranges;
};
std::map<const orca_hip_ctx*, Streams> g_streams;
std::map<uintptr_t, std::pair<bool, uint64_t>> g_event_at;  // event -> (recorded on the side stream, clock)
std::string g_launch = "?";
uint64_t g_races = 0;

bool on_side(const orca_hip_ctx* ctx) { return ctx->main != nullptr; }

void launch(orca_hip_ctx* ctx, const std::string& what) {
  Streams& st = g_streams[ctx];
  if (on_side(ctx))
    ++st.side_clock;
  else
    ++st.main_clock;
  g_launch = what;
}

void touch(orca_hip_ctx* ctx, const void* p, size_t bytes, bool write) {
  if (!p || !bytes) return;
  Streams& st = g_streams[ctx];
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p), hi = lo + bytes;
  const bool side = on_side(ctx);
  size_t exact = st.ranges.size();
  for (size_t i = 0; i < st.ranges.size(); ++i) {
    const Range& r = st.ranges[i];
    if (r.hi <= lo || r.lo >= hi) continue;
    const bool race = side ? (r.main_write > st.side_knows_main || (write && r.main_read > st.side_knows_main))
                           : (r.side_write > st.main_knows_side || (write && r.side_read > st.main_knows_side));
    if (race) {
      ++g_races;
      logf("RACE " + g_launch + (write ? " writes" : " reads") + (side ? " on the side stream" : " on the context stream"));
    }
    if (r.lo == lo && r.hi == hi) exact = i;
  }
  if (exact == st.ranges.size()) st.ranges.push_back(Range{lo, hi, 0, 0, 0, 0});
  Range& r = st.ranges[exact];
  const uint64_t now = side ? st.side_clock : st.main_clock;
  (side ? (write ? r.side_write : r.side_read) : (write ? r.main_write : r.main_read)) = now;
}
void R(orca_hip_ctx* ctx, const void* p, size_t bytes) { touch(ctx, p, bytes, false); }
void W(orca_hip_ctx* ctx, const void* p, size_t bytes) { touch(ctx, p, bytes, true); }

void event_at(orca_hip_ctx* ctx, orca_hip_event* ev) {
  const Streams& st = g_streams[ctx];
  g_event_at[reinterpret_cast<uintptr_t>(ev)] = {on_side(ctx), on_side(ctx) ? st.side_clock : st.main_clock};
}

// A host read or sync: the library first makes the context stream wait for the side stream.
void join(orca_hip_ctx* ctx) {
  Streams& st = g_streams[ctx];
  st.main_knows_side = std::max(st.main_knows_side, st.side_at_switch);
}


float* out_buf(orca_hip_ctx* ctx, size_t n, void** out) {
  if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
  float* o = new_output(ctx, n ? n : 1);
  *out = o;
  W(ctx, o, 4 * n);
  return o;
}

// op(X) as a contiguous row-major [rows][cols] array: X stored [rows][ld] (trans = 0) or
// [cols][ld] (trans = 1).
std::vector<float> dense(const float* X, size_t rows, size_t cols, size_t ld, bool trans) {
  std::vector<float> d(rows * cols);
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < cols; ++c) d[r * cols + c] = trans ? X[c * ld + r] : X[r * ld + c];
  return d;
}

// C = op(A) op(B), the oracle's matmul on contiguous copies (the same sums for every caller).
std::vector<float> product(const float* A, bool ta, size_t lda, const float* B, bool tb, size_t ldb, size_t M,
                           size_t N, size_t K) {
  std::vector<float> a = dense(A, M, K, lda, ta), b = dense(B, K, N, ldb, tb), c(M * N);
  const size_t ad[2] = {M, K}, bd[2] = {K, N};
  if (M && N) {
    if (K == 0) {
      std::fill(c.begin(), c.end(), 0.0f);
    } else if (orc_matmul(a.data(), b.data(), c.data(), ad, 2, bd, 2) != 0) {
      fail(ORCA_HIP_ERR_INTERNAL, "oracle matmul failed");
    }
  }
  return c;
}

// Rethrows a failed nested entry point's error.
void ck_fake(int rc) {
  if (rc != ORCA_HIP_OK) fail(rc, last_error_cstr());
}

void check_oracle(int rc, const char* op) {
  if (rc != 0) fail(ORCA_HIP_ERR_SHAPE, std::string("Shape mismatch during ") + op + " (oracle)");
}
}  // namespace

extern "C" {

// ---- instrumentation
int fake_log_text(char* buf, size_t len, size_t* needed) {
  if (needed) *needed = g_log.size() + 1;
  if (!buf || len < g_log.size() + 1) return ORCA_HIP_ERR_INTERNAL;
  std::memcpy(buf, g_log.c_str(), g_log.size() + 1);
  return ORCA_HIP_OK;
}
void fake_log_clear(void) { g_log.clear(); }
// Accesses that the two streams' order did not cover, since the library was loaded.
uint64_t fake_race_count(void) { return g_races; }

// ---- context and memory
const char* orca_hip_last_error(void) { return last_error_cstr(); }

int orca_hip_ctx_create(int device, orca_hip_ctx** out) {
  return guard([&] {
    if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    auto* ctx = new orca_hip_ctx();
    ctx->device = device;
    ctx->alloc.sync_counter = &ctx->host_syncs;
    ctx->stream = reinterpret_cast<hipStream_t>(ctx);
    *out = ctx;
  });
}

int orca_hip_ctx_destroy(orca_hip_ctx* ctx) {
  return guard([&] {
    if (!ctx) return;
    if (ctx->main) ctx->stream = ctx->main;
    g_streams.erase(ctx);
    delete ctx;
  });
}

int orca_hip_device(const orca_hip_ctx* ctx, int* ordinal) {
  return guard([&] {
    check_ctx(ctx);
    *ordinal = ctx->device;
  });
}

int orca_hip_alloc(orca_hip_ctx* ctx, size_t bytes, void** out) {
  return guard([&] {
    check_ctx(ctx);
    *out = ctx_allocate(ctx, bytes);
  });
}

int orca_hip_free(orca_hip_ctx* ctx, void* p) {
  return guard([&] {
    check_ctx(ctx);
    ctx->alloc.release(p);
  });
}

int orca_hip_free_many(orca_hip_ctx* ctx, void* const* ptrs, size_t n) {
  return guard([&] {
    check_ctx(ctx);
    for (size_t i = 0; i < n; ++i) ctx->alloc.release(ptrs[i]);
  });
}

int orca_hip_mem_stats(orca_hip_ctx* ctx, size_t* live, size_t* cached, size_t* device_allocs) {
  return guard([&] { ctx->alloc.stats(live, cached, device_allocs); });
}

int orca_hip_sync(orca_hip_ctx* ctx) {
  return guard([&] {
    host_sync(ctx);
    join(ctx);
  });
}

int orca_hip_sync_count(const orca_hip_ctx* ctx, uint64_t* count) {
  return guard([&] { *count = ctx->host_syncs.load(); });
}

int orca_hip_h2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    check_extent(ctx, dst, bytes, "h2d");
    join(ctx);
    launch(ctx, "h2d");
    W(ctx, dst, bytes);
    std::memcpy(dst, src, bytes);
  });
}

int orca_hip_d2h(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    check_extent(ctx, src, bytes, "d2h");
    join(ctx);
    launch(ctx, "d2h");
    R(ctx, src, bytes);
    std::memcpy(dst, src, bytes);
  });
}

int orca_hip_d2d(orca_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    check_extent(ctx, dst, bytes, "d2d");
    check_extent(ctx, src, bytes, "d2d");
    launch(ctx, "d2d");
    R(ctx, src, bytes);
    W(ctx, dst, bytes);
    std::memmove(dst, src, bytes);
    logf("d2d " + std::to_string(bytes));
  });
}

int orca_hip_fill(orca_hip_ctx* ctx, float* dst, float value, size_t n) {
  return guard([&] {
    check_extent(ctx, dst, 4 * n, "fill");
    launch(ctx, "fill");
    W(ctx, dst, 4 * n);
    for (size_t i = 0; i < n; ++i) dst[i] = value;
  });
}

// ---- streams and events: launches are synchronous here; the log records which stream
int orca_hip_use_side_stream(orca_hip_ctx* ctx, int blocks_per_cu) {
  return guard([&] {
    if (blocks_per_cu) {
      if (ctx->main) fail(ORCA_HIP_ERR_INTERNAL, "launches already go to the side stream");
      ctx->main = ctx->stream;
      ctx->stream = reinterpret_cast<hipStream_t>(reinterpret_cast<char*>(ctx) + 1);
      ctx->side_bpc = blocks_per_cu > 0 ? blocks_per_cu : 0;
      logf("side " + std::to_string(blocks_per_cu));
    } else {
      if (!ctx->main) fail(ORCA_HIP_ERR_INTERNAL, "launches do not go to the side stream");
      g_streams[ctx].side_at_switch = g_streams[ctx].side_clock;
      ctx->stream = ctx->main;
      ctx->main = nullptr;
      logf("main");
    }
  });
}

orca_hip_event* next_event() {
  static uintptr_t next = 16;
  next += 16;
  return reinterpret_cast<orca_hip_event*>(next);
}

int orca_hip_event_record(orca_hip_ctx* ctx, orca_hip_event** out) {
  return guard([&] {
    *out = next_event();
    event_at(ctx, *out);
    logf("record " + std::to_string(reinterpret_cast<uintptr_t>(*out)) + (ctx->main ? " side" : ""));
  });
}

int orca_hip_event_wait(orca_hip_ctx* ctx, orca_hip_event* ev) {
  return guard([&] {
    auto it = g_event_at.find(reinterpret_cast<uintptr_t>(ev));
    if (it != g_event_at.end()) {
      Streams& st = g_streams[ctx];
      if (it->second.first && !on_side(ctx)) st.main_knows_side = std::max(st.main_knows_side, it->second.second);
      if (!it->second.first && on_side(ctx)) st.side_knows_main = std::max(st.side_knows_main, it->second.second);
    }
    logf("wait " + std::to_string(reinterpret_cast<uintptr_t>(ev)) + (ctx->main ? " side" : ""));
  });
}

int orca_hip_event_release(orca_hip_ctx*, orca_hip_event*) { return ORCA_HIP_OK; }

// ---- trait kernels
int orca_hip_zeros(orca_hip_ctx* ctx, const size_t* shape, size_t rank, int dtype, void** out) {
  return guard([&] {
    check_f32(dtype, "zeros");
    const size_t n = numel(shape, rank);
    launch(ctx, "zeros");
    float* o = out_buf(ctx, n, out);
    for (size_t i = 0; i < n; ++i) o[i] = 0.0f;
  });
}

int orca_hip_from_f32_slice(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const float* data, size_t n,
                            void** out) {
  return guard([&] {
    if (numel(shape, rank) != n) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during from_f32_slice");
    launch(ctx, "upload");
    float* o = out_buf(ctx, n, out);
    if (n) std::memcpy(o, data, 4 * n);
    logf("upload " + std::to_string(n));
  });
}

int orca_hip_to_f32_vec(orca_hip_ctx* ctx, const void* s, size_t n, float* host) {
  return guard([&] {
    check_extent(ctx, s, 4 * n, "to_f32_vec");
    join(ctx);
    launch(ctx, "to_f32_vec");
    R(ctx, s, 4 * n);
    if (n) std::memcpy(host, s, 4 * n);
  });
}

int orca_hip_from_bytes(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const uint8_t* bytes, size_t n_bytes,
                        int dtype, void** out) {
  return guard([&] {
    check_f32(dtype, "from_bytes");
    const size_t n = numel(shape, rank);
    if (n_bytes != 4 * n) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during from_bytes");
    launch(ctx, "from_bytes");
    float* o = out_buf(ctx, n, out);
    if (n) std::memcpy(o, bytes, n_bytes);
  });
}

int orca_hip_to_bytes(orca_hip_ctx* ctx, const void* s, size_t n_bytes, uint8_t* host) {
  return guard([&] {
    check_extent(ctx, s, n_bytes, "to_bytes");
    join(ctx);
    launch(ctx, "to_bytes");
    R(ctx, s, n_bytes);
    if (n_bytes) std::memcpy(host, s, n_bytes);
  });
}

int orca_hip_has_nan_or_inf(orca_hip_ctx* ctx, const void* s, size_t n, int dtype, int* result) {
  return guard([&] {
    check_f32(dtype, "has_nan_or_inf");
    join(ctx);
    launch(ctx, "has_nan_or_inf");
    R(ctx, s, 4 * n);
    *result = orc_has_nan_or_inf(F(s), n);
  });
}

int orca_hip_matmul(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* ls, size_t lr, const size_t* rs,
                    size_t rr, int dtype, int lv, int rv, void** out) {
  return guard([&] {
    check_f32(dtype, "matmul");
    if (lr != 2 || rr != 2) fail(ORCA_HIP_ERR_INTERNAL, "the stand-in multiplies 2-D operands only");
    const size_t M = ls[0], K = ls[1], N = rs[1];
    if (rs[0] != K) fail_shape("matmul", std::to_string(K), std::to_string(rs[0]));
    launch(ctx, "matmul");
    R(ctx, lhs, 4 * M * K);
    R(ctx, rhs, 4 * K * N);
    std::vector<float> c = product(F(lhs), lv != 0, lv ? M : K, F(rhs), rv != 0, rv ? K : N, M, N, K);
    float* o = out_buf(ctx, M * N, out);
    std::copy(c.begin(), c.end(), o);
    logf("matmul " + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K) + " " +
         std::to_string(lv) + std::to_string(rv));
  });
}

int orca_hip_matmul_colsum(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N,
                           int lhs_view, int dtype, void* colsum, void** out) {
  return guard([&] {
    check_f32(dtype, "matmul_colsum");
    launch(ctx, "matmul_colsum");
    R(ctx, lhs, 4 * M * K);
    R(ctx, rhs, 4 * K * N);
    W(ctx, colsum, 4 * N);
    std::vector<float> c = product(F(lhs), lhs_view != 0, lhs_view ? M : K, F(rhs), false, N, M, N, K);
    float* o = out_buf(ctx, M * N, out);
    std::copy(c.begin(), c.end(), o);
    const size_t in[2] = {K, N}, cs[2] = {1, N};
    check_oracle(orc_sum_to_shape(F(rhs), F(colsum), in, 2, cs, 2), "matmul_colsum");
    logf("matmul_colsum " + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K) + " " +
         std::to_string(lhs_view));
  });
}

// Products that hand back an event completing with them: "bound N" follows the launch's
// log line (a real launch records it itself).
int orca_hip_matmul_ev(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N, int lv,
                       int rv, int dtype, void* colsum, void** out, orca_hip_event** done) {
  return guard([&] {
    if (done) *done = nullptr;
    if (colsum && rv) fail(ORCA_HIP_ERR_INTERNAL, "matmul_ev: a column sum needs a contiguous rhs");
    if (colsum) {
      ck_fake(orca_hip_matmul_colsum(ctx, lhs, rhs, M, K, N, lv, dtype, colsum, out));
    } else {
      const size_t ls[2] = {M, K}, rs[2] = {K, N};
      ck_fake(orca_hip_matmul(ctx, lhs, rhs, ls, 2, rs, 2, dtype, lv, rv, out));
    }
    if (done) {
      *done = next_event();
      event_at(ctx, *done);
      logf("bound " + std::to_string(reinterpret_cast<uintptr_t>(*done)));
    }
  });
}

int orca_hip_gemm(orca_hip_ctx* ctx, int ta, int tb, size_t M, size_t N, size_t K, const float* A, size_t lda,
                  const float* B, size_t ldb, float* C, size_t ldc, const orca_hip_epilogue* epi) {
  return guard([&] {
    launch(ctx, "gemm");
    R(ctx, A, 4 * (ta ? K * lda : M * lda));
    R(ctx, B, 4 * (tb ? N * ldb : K * ldb));
    W(ctx, C, 4 * M * ldc);
    std::vector<float> p = product(A, ta != 0, lda, B, tb != 0, ldb, M, N, K);
    const int kind = epi ? epi->kind : ORCA_HIP_EPI_NONE;
    if (epi) {
      R(ctx, epi->bias, 4 * N);
      R(ctx, epi->mask, 4 * M * epi->ldmask);
      W(ctx, epi->pre, 4 * M * ldc);
      W(ctx, epi->colsum, 4 * N);
    }
    std::vector<float> v(M * N), bias_row(M * N);
    if (kind == ORCA_HIP_EPI_BIAS || kind == ORCA_HIP_EPI_BIAS_RELU || kind == ORCA_HIP_EPI_BIAS_RELU_PRE) {
      const size_t bd[2] = {1, N}, od[2] = {M, N};
      check_oracle(orc_expand(epi->bias, bias_row.data(), bd, 2, od, 2), "gemm bias");
      orc_add(p.data(), bias_row.data(), v.data(), M * N);
      if (kind == ORCA_HIP_EPI_BIAS_RELU_PRE)
        for (size_t r = 0; r < M; ++r) std::copy(&v[r * N], &v[r * N] + N, epi->pre + r * ldc);
      if (kind != ORCA_HIP_EPI_BIAS) orc_relu(v.data(), v.data(), M * N);
    } else if (kind == ORCA_HIP_EPI_RELU_MASK || kind == ORCA_HIP_EPI_RELU_MASK_PRE) {
      std::vector<float> mk = dense(epi->mask, M, N, epi->ldmask, false);
      if (kind == ORCA_HIP_EPI_RELU_MASK_PRE)
        for (size_t r = 0; r < M; ++r) std::copy(&p[r * N], &p[r * N] + N, epi->pre + r * ldc);
      orc_relu_backward(p.data(), mk.data(), v.data(), M * N);
    } else {
      v = p;
    }
    for (size_t r = 0; r < M; ++r) std::copy(&v[r * N], &v[r * N] + N, C + r * ldc);
    if (epi && epi->colsum) {
      std::vector<float> b = dense(B, K, N, ldb, tb != 0);
      const size_t in[2] = {K, N}, cs[2] = {1, N};
      check_oracle(orc_sum_to_shape(b.data(), epi->colsum, in, 2, cs, 2), "gemm colsum");
    }
    logf("gemm " + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K) + " " + std::to_string(ta) +
         std::to_string(tb) + " epi " + std::to_string(kind) + (epi && epi->colsum ? " colsum" : "") +
         (ctx->main ? " side" : ""));
    if (epi && epi->done) {
      *epi->done = next_event();
      event_at(ctx, *epi->done);
      logf("bound " + std::to_string(reinterpret_cast<uintptr_t>(*epi->done)));
    }
  });
}

// The three products one by one, as the library's grid computes them (the same sums).
int orca_hip_narrow_linear_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* G, size_t C,
                                    const float* Wc, const float* mask, float* dH, float* dH_pre, float* dW, float* db,
                                    orca_hip_event** done) {
  return guard([&] {
    if (done) *done = nullptr;
    launch(ctx, "narrow_linear_backward");
    R(ctx, H, 4 * B * K);
    R(ctx, G, 4 * B * C);
    R(ctx, Wc, 4 * K * C);
    R(ctx, mask, 4 * B * K);
    W(ctx, dH, 4 * B * K);
    W(ctx, dH_pre, 4 * B * K);
    W(ctx, dW, 4 * K * C);
    W(ctx, db, 4 * C);
    std::vector<float> w = product(H, true, K, G, false, C, K, C, B);
    std::copy(w.begin(), w.end(), dW);
    if (db) {
      const size_t in[2] = {B, C}, cs[2] = {1, C};
      check_oracle(orc_sum_to_shape(G, db, in, 2, cs, 2), "narrow_linear_backward colsum");
    }
    std::vector<float> h = product(G, false, C, Wc, true, C, B, K, C);
    if (mask) {
      if (dH_pre) std::copy(h.begin(), h.end(), dH_pre);
      orc_relu_backward(h.data(), mask, dH, B * K);
    } else {
      std::copy(h.begin(), h.end(), dH);
    }
    logf("narrow_linear_backward " + std::to_string(B) + "x" + std::to_string(K) + "x" + std::to_string(C) +
         (mask ? (dH_pre ? " mask pre" : " mask") : "") + (db ? " colsum" : ""));
    if (done) {
      *done = next_event();
      event_at(ctx, *done);
      logf("bound " + std::to_string(reinterpret_cast<uintptr_t>(*done)));
    }
  });
}

int orca_hip_transpose(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, size_t d0, size_t d1,
                       int dtype, void** out) {
  return guard([&] {
    check_f32(dtype, "transpose");
    const size_t n = numel(shape, rank);
    launch(ctx, "transpose");
    R(ctx, s, 4 * n);
    float* o = out_buf(ctx, n, out);
    check_oracle(orc_transpose(F(s), o, shape, rank, d0, d1), "transpose");
    logf("transpose " + std::to_string(n));
  });
}

#define FAKE_EW1(NAME, FN)                                                                                     \
  int orca_hip_##NAME(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, void** out) { \
    return guard([&] {                                                                                         \
      check_f32(dtype, #NAME);                                                                                 \
      const size_t n = numel(shape, rank);                                                                     \
      launch(ctx, #NAME);                                                                                      \
      R(ctx, s, 4 * n);                                                                                        \
      FN(F(s), out_buf(ctx, n, out), n);                                                                       \
      logf(std::string("op ") + #NAME);                                                                        \
    });                                                                                                        \
  }
#define FAKE_EW2(NAME, FN)                                                                                   \
  int orca_hip_##NAME(orca_hip_ctx* ctx, const void* a, const void* b, const size_t* shape, size_t rank, int dtype, \
                      void** out) {                                                                          \
    return guard([&] {                                                                                       \
      check_f32(dtype, #NAME);                                                                               \
      const size_t n = numel(shape, rank);                                                                   \
      launch(ctx, #NAME);                                                                                    \
      R(ctx, a, 4 * n);                                                                                      \
      R(ctx, b, 4 * n);                                                                                      \
      FN(F(a), F(b), out_buf(ctx, n, out), n);                                                               \
      logf(std::string("op ") + #NAME);                                                                      \
    });                                                                                                      \
  }
FAKE_EW1(relu, orc_relu)
FAKE_EW1(sigmoid, orc_sigmoid)
FAKE_EW1(exp, orc_exp)
FAKE_EW1(log, orc_log)
FAKE_EW1(sqrt, orc_sqrt)
FAKE_EW2(add, orc_add)
FAKE_EW2(sub, orc_sub)
FAKE_EW2(mul, orc_mul)
FAKE_EW2(div, orc_div)
FAKE_EW2(relu_backward, orc_relu_backward)
FAKE_EW2(sigmoid_backward, orc_sigmoid_backward)
FAKE_EW2(exp_backward, orc_exp_backward)
FAKE_EW2(log_backward, orc_log_backward)
FAKE_EW2(sqrt_backward, orc_sqrt_backward)
FAKE_EW2(div_backward_lhs, orc_div_backward_lhs)

int orca_hip_mul_scalar(orca_hip_ctx* ctx, const void* s, float scalar, const size_t* shape, size_t rank, int dtype,
                        void** out) {
  return guard([&] {
    check_f32(dtype, "mul_scalar");
    const size_t n = numel(shape, rank);
    launch(ctx, "mul_scalar");
    R(ctx, s, 4 * n);
    orc_mul_scalar(F(s), scalar, out_buf(ctx, n, out), n);
    logf("op mul_scalar");
  });
}

int orca_hip_div_backward_rhs(orca_hip_ctx* ctx, const void* g, const void* l, const void* r, const size_t* shape,
                              size_t rank, int dtype, void** out) {
  return guard([&] {
    check_f32(dtype, "div_backward_rhs");
    const size_t n = numel(shape, rank);
    launch(ctx, "div_backward_rhs");
    R(ctx, g, 4 * n);
    R(ctx, l, 4 * n);
    R(ctx, r, 4 * n);
    orc_div_backward_rhs(F(g), F(l), F(r), out_buf(ctx, n, out), n);
    logf("op div_backward_rhs");
  });
}

int orca_hip_accumulate_grad(orca_hip_ctx* ctx, const void* a, const void* b, size_t n, void** out) {
  return guard([&] {
    launch(ctx, "accumulate_grad");
    R(ctx, a, 4 * n);
    R(ctx, b, 4 * n);
    orc_accumulate_grad(F(a), F(b), out_buf(ctx, n, out), n);
    logf("op accumulate_grad");
  });
}

#define FAKE_RESHAPE(NAME, FN)                                                                             \
  int orca_hip_##NAME(orca_hip_ctx* ctx, const void* s, const size_t* in, size_t ir, const size_t* os, size_t orank, \
                      int dtype, void** out) {                                                             \
    return guard([&] {                                                                                     \
      check_f32(dtype, #NAME);                                                                             \
      launch(ctx, #NAME);                                                                                  \
      R(ctx, s, 4 * numel(in, ir));                                                                        \
      check_oracle(FN(F(s), out_buf(ctx, numel(os, orank), out), in, ir, os, orank), #NAME);               \
      logf(std::string("op ") + #NAME);                                                                    \
    });                                                                                                    \
  }
FAKE_RESHAPE(expand, orc_expand)
FAKE_RESHAPE(sum_to_shape, orc_sum_to_shape)
FAKE_RESHAPE(max_to_shape, orc_max_to_shape)

int orca_hip_max_to_shape_backward(orca_hip_ctx* ctx, const void* g, const void* x, const void* y, const size_t* in,
                                   size_t ir, const size_t* os, size_t orank, int dtype, void** out) {
  return guard([&] {
    check_f32(dtype, "max_to_shape_backward");
    launch(ctx, "max_to_shape_backward");
    R(ctx, g, 4 * numel(os, orank));
    R(ctx, x, 4 * numel(in, ir));
    R(ctx, y, 4 * numel(os, orank));
    check_oracle(orc_max_to_shape_backward(F(g), F(x), F(y), out_buf(ctx, numel(in, ir), out), in, ir, os, orank),
                 "max_to_shape_backward");
    logf("op max_to_shape_backward");
  });
}

// ---- fused programs: each instruction is the op's own array pass
// The interpreter: the registers after the program ran over n elements.
std::vector<std::vector<float>> fake_program(orca_hip_ctx* ctx, size_t n, const orca_hip_ew_input* inputs,
                                             size_t n_inputs, size_t n_outputs, const orca_hip_ew_instr* instrs,
                                             size_t n_instrs, size_t n_regs) {
  if (n_inputs > ORCA_HIP_EW_MAX_INPUTS || n_outputs > ORCA_HIP_EW_MAX_OUTPUTS || n_instrs > ORCA_HIP_EW_MAX_OPS ||
      n_regs > ORCA_HIP_EW_MAX_REGS || n_inputs > n_regs)
    fail(ORCA_HIP_ERR_INTERNAL, "program exceeds the interpreter's limits");
  std::vector<std::vector<float>> reg(n_regs, std::vector<float>(n));
  for (size_t i = 0; i < n_inputs; ++i) R(ctx, inputs[i].ptr, 4 * std::min<uint64_t>(inputs[i].mod, n ? n : 1));
  for (size_t i = 0; i < n_inputs; ++i) {
    const orca_hip_ew_input& in = inputs[i];
    if (!in.mod || !in.div) fail(ORCA_HIP_ERR_INTERNAL, "bad input map");
    check_extent(ctx, in.ptr, 4 * std::min<uint64_t>(in.mod, n ? n : 1), "ew_program input");
    for (size_t e = 0; e < n; ++e) reg[i][e] = in.ptr[(e / in.div) % in.mod];
  }
  std::vector<float> tmp(n);
  for (size_t k = 0; k < n_instrs; ++k) {
    const orca_hip_ew_instr& I = instrs[k];
    if (I.dst >= n_regs || I.a >= n_regs || I.b >= n_regs || I.c >= n_regs)
      fail(ORCA_HIP_ERR_INTERNAL, "register out of range");
    const float *a = reg[I.a].data(), *b = reg[I.b].data(), *c = reg[I.c].data();
    float* d = tmp.data();
    switch (I.op) {
      case ORCA_HIP_EW_ADD: orc_add(a, b, d, n); break;
      case ORCA_HIP_EW_SUB: orc_sub(a, b, d, n); break;
      case ORCA_HIP_EW_MUL: orc_mul(a, b, d, n); break;
      case ORCA_HIP_EW_DIV: orc_div(a, b, d, n); break;
      case ORCA_HIP_EW_MUL_SCALAR: orc_mul_scalar(a, I.scalar, d, n); break;
      case ORCA_HIP_EW_RELU: orc_relu(a, d, n); break;
      case ORCA_HIP_EW_RELU_BW: orc_relu_backward(a, b, d, n); break;
      case ORCA_HIP_EW_EXP: orc_exp(a, d, n); break;
      case ORCA_HIP_EW_LOG: orc_log(a, d, n); break;
      case ORCA_HIP_EW_SQRT: orc_sqrt(a, d, n); break;
      case ORCA_HIP_EW_SIGMOID: orc_sigmoid(a, d, n); break;
      case ORCA_HIP_EW_EXP_BW: orc_exp_backward(a, b, d, n); break;
      case ORCA_HIP_EW_LOG_BW: orc_log_backward(a, b, d, n); break;
      case ORCA_HIP_EW_SQRT_BW: orc_sqrt_backward(a, b, d, n); break;
      case ORCA_HIP_EW_SIGMOID_BW: orc_sigmoid_backward(a, b, d, n); break;
      case ORCA_HIP_EW_DIV_BW_RHS: orc_div_backward_rhs(a, b, c, d, n); break;
      case ORCA_HIP_EW_SUM_VISIT: {
        const size_t dims[1] = {n};
        check_oracle(orc_sum_to_shape(a, d, dims, 1, dims, 1), "sum visit");
        break;
      }
      case ORCA_HIP_EW_MAX_VISIT: {
        const size_t dims[1] = {n};
        check_oracle(orc_max_to_shape(a, d, dims, 1, dims, 1), "max visit");
        break;
      }
      case ORCA_HIP_EW_COPY: std::copy(a, a + n, d); break;
      case ORCA_HIP_EW_ADD_SCALAR: {
        std::vector<float> sc(n, I.scalar);
        orc_add(a, sc.data(), d, n);
        break;
      }
      default: fail(ORCA_HIP_ERR_INTERNAL, "unknown opcode");
    }
    reg[I.dst].swap(tmp);
  }
  return reg;
}

void fake_outputs(orca_hip_ctx* ctx, size_t n, const std::vector<std::vector<float>>& reg, float* const* outputs,
                  const uint8_t* out_regs, size_t n_outputs) {
  for (size_t o = 0; o < n_outputs; ++o) {
    if (out_regs[o] >= reg.size()) fail(ORCA_HIP_ERR_INTERNAL, "output register out of range");
    check_extent(ctx, outputs[o], 4 * n, "ew_program output");
    W(ctx, outputs[o], 4 * n);
    std::copy(reg[out_regs[o]].begin(), reg[out_regs[o]].end(), outputs[o]);
  }
}

int orca_hip_ew_program(orca_hip_ctx* ctx, size_t n, const orca_hip_ew_input* inputs, size_t n_inputs,
                        float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                        const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs) {
  return guard([&] {
    launch(ctx, "program");
    auto reg = fake_program(ctx, n, inputs, n_inputs, n_outputs, instrs, n_instrs, n_regs);
    fake_outputs(ctx, n, reg, outputs, out_regs, n_outputs);
    logf("program " + std::to_string(n_inputs) + " " + std::to_string(n_outputs) + " " + std::to_string(n_instrs) +
         " " + std::to_string(n_regs) + (ctx->main ? " side" : ""));
  });
}

// The program, then the rows of one register reduced as the oracle's sum_to_shape / max_to_shape.
int orca_hip_ew_program_rows(orca_hip_ctx* ctx, size_t rows, size_t cols, const orca_hip_ew_input* inputs,
                             size_t n_inputs, float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                             const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs, int red_reg,
                             int reduce_max, float* reduced) {
  return guard([&] {
    if (cols == 0 || cols > 64 || red_reg < 0 || (size_t)red_reg >= n_regs)
      fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: bad arguments");
    launch(ctx, "program_rows");
    const size_t n = rows * cols;
    auto reg = fake_program(ctx, n, inputs, n_inputs, n_outputs, instrs, n_instrs, n_regs);
    fake_outputs(ctx, n, reg, outputs, out_regs, n_outputs);
    W(ctx, reduced, 4 * rows);
    const size_t in[2] = {rows, cols}, os[2] = {rows, 1};
    check_oracle(reduce_max ? orc_max_to_shape(reg[red_reg].data(), reduced, in, 2, os, 2)
                            : orc_sum_to_shape(reg[red_reg].data(), reduced, in, 2, os, 2),
                 "ew_program_rows");
    logf("program_rows " + std::to_string(n_inputs) + " " + std::to_string(n_outputs) + " " +
         std::to_string(n_instrs) + " " + std::to_string(n_regs) + (reduce_max ? " max" : " sum") +
         (ctx->main ? " side" : ""));
  });
}

// ---- fused loss and optimizers
int orca_hip_softmax_ce(orca_hip_ctx* ctx, const float* logits, size_t B, size_t C, const float* onehot,
                        const int32_t* labels, float* loss, float* dlogits, int32_t* preds, int64_t* correct) {
  return guard([&] {
    if (!onehot || labels || preds || correct) fail(ORCA_HIP_ERR_INTERNAL, "the stand-in takes one-hot targets only");
    launch(ctx, "softmax_ce");
    R(ctx, logits, 4 * B * C);
    R(ctx, onehot, 4 * B * C);
    W(ctx, loss, 4);
    W(ctx, dlogits, 4 * B * C);
    std::vector<float> d(B * C);
    float l = 0.0f;
    if (orc_cross_entropy(logits, onehot, B, C, &l, d.data()) != 0) fail(ORCA_HIP_ERR_INTERNAL, "oracle CE failed");
    if (loss) *loss = l;
    if (dlogits) std::copy(d.begin(), d.end(), dlogits);
    logf("softmax_ce");
  });
}

static orc_opt make_opt(int kind, double lr, double b1, double b2, double eps, double wd) {
  orc_opt o{};
  o.kind = kind;
  o.lr = lr;
  o.weight_decay = wd;
  o.beta1 = b1;
  o.beta2 = b2;
  o.eps = eps;
  return o;
}

int orca_hip_adamw_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr, double beta1,
                         double beta2, double eps, double weight_decay, int64_t t) {
  return guard([&] {
    const orc_opt o = make_opt(1, lr, beta1, beta2, eps, weight_decay);
    size_t total = 0;
    launch(ctx, "adamw_multi");
    for (size_t i = 0; i < n_segs; ++i) {
      const orca_hip_opt_segment& s = segs[i];
      R(ctx, s.p_src, 4 * s.n);
      R(ctx, s.g, 4 * s.n);
      R(ctx, s.m, 4 * s.n);
      R(ctx, s.v, 4 * s.n);
    }
    for (size_t i = 0; i < n_segs; ++i) {
      const orca_hip_opt_segment& s = segs[i];
      W(ctx, s.p_dst, 4 * s.n);
      W(ctx, s.m, 4 * s.n);
      W(ctx, s.v, 4 * s.n);
    }
    for (size_t i = 0; i < n_segs; ++i) {
      const orca_hip_opt_segment& s = segs[i];
      std::vector<float> p(s.p_src, s.p_src + s.n);
      orc_adamw_update(p.data(), s.g, s.m, s.v, s.n, &o, t);
      std::copy(p.begin(), p.end(), s.p_dst);
      total += s.n;
    }
    logf("adamw_multi " + std::to_string(n_segs) + " " + std::to_string(total) + (ctx->main ? " side" : ""));
  });
}

int orca_hip_sgd_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr) {
  return guard([&] {
    const orc_opt o = make_opt(0, lr, 0, 0, 0, 0);
    size_t total = 0;
    launch(ctx, "sgd_multi");
    for (size_t i = 0; i < n_segs; ++i) {
      const orca_hip_opt_segment& s = segs[i];
      R(ctx, s.p_src, 4 * s.n);
      R(ctx, s.g, 4 * s.n);
    }
    for (size_t i = 0; i < n_segs; ++i) W(ctx, segs[i].p_dst, 4 * segs[i].n);
    for (size_t i = 0; i < n_segs; ++i) {
      const orca_hip_opt_segment& s = segs[i];
      std::vector<float> p(s.p_src, s.p_src + s.n);
      orc_sgd_update(p.data(), s.g, s.n, &o);
      std::copy(p.begin(), p.end(), s.p_dst);
      total += s.n;
    }
    logf("sgd_multi " + std::to_string(n_segs) + " " + std::to_string(total) + (ctx->main ? " side" : ""));
  });
}

int orca_hip_adamw_step(orca_hip_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, double lr,
                        double beta1, double beta2, double eps, double weight_decay, int64_t t) {
  return guard([&] {
    launch(ctx, "adamw_step");
    R(ctx, g, 4 * n);
    W(ctx, p, 4 * n);
    W(ctx, m, 4 * n);
    W(ctx, v, 4 * n);
    const orc_opt o = make_opt(1, lr, beta1, beta2, eps, weight_decay);
    orc_adamw_update(p, g, m, v, n, &o, t);
    logf("adamw_step");
  });
}

int orca_hip_sgd_step(orca_hip_ctx* ctx, float* p, const float* g, size_t n, double lr) {
  return guard([&] {
    launch(ctx, "sgd_step");
    R(ctx, g, 4 * n);
    W(ctx, p, 4 * n);
    const orc_opt o = make_opt(0, lr, 0, 0, 0, 0);
    orc_sgd_update(p, g, n, &o);
    logf("sgd_step");
  });
}

}  // extern "C"
