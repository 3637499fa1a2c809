// Backend trait ops of the HIP backend: the elementwise family and the shape
// ops (expand, sum_to_shape, max_to_shape and its backward, transpose).
//
// Semantics follow orca-backend-cpu/src/backend.rs (line numbers cite it):
// relu is `x > 0 ? x : 0`, log clamps its input at 1e-7, log_backward does
// not clamp, max_to_shape starts from -FLT_MAX and only a strictly greater
// value replaces the running max, max_to_shape_backward hands the full
// gradient to every element equal to the max, and sum_to_shape / max_to_shape
// visit inputs in ascending row-major order -- here one thread owns one output
// element (for column reductions, one lane combining LDS-staged rows), so those
// reductions are bit-identical to the reference's loops.
// Built with -ffp-contract=off: no multiply-add is fused.
#include <cfloat>
#include <cmath>

#include "ew_ops.hpp"
#include "runtime.hpp"

namespace orca_hip {
namespace {

constexpr int kMaxRank = 8;
constexpr unsigned kBlock = 256;
constexpr int RED_UNROLL = 128;  // loads in flight per thread of a single-axis reduction

// ---------------------------------------------------------------- kernels
// float4 path: n4 full vectors, tail elements handled by the first threads.
template <class Op>
__global__ void __launch_bounds__(kBlock) ew1_kernel(const float* __restrict__ a, float* __restrict__ out, size_t n, Op op) {
  size_t n4 = n / 4, stride = (size_t)gridDim.x * blockDim.x, t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const float4* a4 = reinterpret_cast<const float4*>(a);
  float4* o4 = reinterpret_cast<float4*>(out);
  for (size_t i = t; i < n4; i += stride) {
    float4 x = a4[i];
    o4[i] = make_float4(op(x.x), op(x.y), op(x.z), op(x.w));
  }
  for (size_t i = 4 * n4 + t; i < n; i += stride) out[i] = op(a[i]);
}

template <class Op>
__global__ void __launch_bounds__(kBlock) ew2_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out, size_t n, Op op) {
  size_t n4 = n / 4, stride = (size_t)gridDim.x * blockDim.x, t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const float4* a4 = reinterpret_cast<const float4*>(a);
  const float4* b4 = reinterpret_cast<const float4*>(b);
  float4* o4 = reinterpret_cast<float4*>(out);
  for (size_t i = t; i < n4; i += stride) {
    float4 x = a4[i], y = b4[i];
    o4[i] = make_float4(op(x.x, y.x), op(x.y, y.y), op(x.z, y.z), op(x.w, y.w));
  }
  for (size_t i = 4 * n4 + t; i < n; i += stride) out[i] = op(a[i], b[i]);
}

template <class Op>
__global__ void __launch_bounds__(kBlock) ew3_kernel(const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ c,
                                                     float* __restrict__ out, size_t n, Op op) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = op(a[i], b[i], c[i]);
}

// Scalar-pointer fallbacks (inputs not 16-byte aligned).
template <class Op>
__global__ void ew1_scalar_kernel(const float* a, float* out, size_t n, Op op) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = op(a[i]);
}
template <class Op>
__global__ void ew2_scalar_kernel(const float* a, const float* b, float* out, size_t n, Op op) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = op(a[i], b[i]);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <class Op>
void run_ew1(orca_hip_ctx* ctx, const char* name, const float* a, float* out, size_t n, Op op) {
  if (n == 0) return;
  check_extent(ctx, a, n * sizeof(float), name);
  ProfScope ps(ctx, name, 0.0, 8.0 * n);
  if (aligned16(a) && aligned16(out)) {
    unsigned g = grid_for((n + 3) / 4, kBlock, ctx->num_cus * 16);
    hipLaunchKernelGGL(ew1_kernel<Op>, dim3(g), dim3(kBlock), 0, ctx->stream, a, out, n, op);
  } else {
    unsigned g = grid_for(n, kBlock, ctx->num_cus * 16);
    hipLaunchKernelGGL(ew1_scalar_kernel<Op>, dim3(g), dim3(kBlock), 0, ctx->stream, a, out, n, op);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

template <class Op>
void run_ew2(orca_hip_ctx* ctx, const char* name, const float* a, const float* b, float* out, size_t n, Op op) {
  if (n == 0) return;
  check_extent(ctx, a, n * sizeof(float), name);
  check_extent(ctx, b, n * sizeof(float), name);
  ProfScope ps(ctx, name, 0.0, 12.0 * n);
  if (aligned16(a) && aligned16(b) && aligned16(out)) {
    unsigned g = grid_for((n + 3) / 4, kBlock, ctx->num_cus * 16);
    hipLaunchKernelGGL(ew2_kernel<Op>, dim3(g), dim3(kBlock), 0, ctx->stream, a, b, out, n, op);
  } else {
    unsigned g = grid_for(n, kBlock, ctx->num_cus * 16);
    hipLaunchKernelGGL(ew2_scalar_kernel<Op>, dim3(g), dim3(kBlock), 0, ctx->stream, a, b, out, n, op);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

// ---------------------------------------------------------------- shape ops
struct Dims {
  int rank;
  int64_t d[kMaxRank];
};

// expand: out index -> in index, broadcast dims have in-stride 0 (backend.rs:486-494).
struct ExpandArgs {
  int rank;
  int64_t out_dims[kMaxRank];
  int64_t in_strides[kMaxRank];
};

__global__ void expand_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n, ExpandArgs a) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, idx = 0;
    for (int d = a.rank - 1; d >= 0; --d) {
      size_t c = rem % (size_t)a.out_dims[d];
      rem /= (size_t)a.out_dims[d];
      idx += c * (size_t)a.in_strides[d];
    }
    out[i] = in[idx];
  }
}

// The broadcasts the Linear layer, the loss and the optimizer make on every
// step, as copies without index arithmetic: rows (out[r][c] = in[c], a bias
// [1, N] expanded to [B, N]), columns (out[r][c] = in[r], [B, 1] to [B, C])
// and a single value.
__global__ void expand_rows_kernel(const float* __restrict__ in, float* __restrict__ out, size_t rows, size_t cols,
                                   bool vec) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (size_t r = blockIdx.y; r < rows; r += gridDim.y) {
    if (vec) {
      const float4* i4 = reinterpret_cast<const float4*>(in);
      float4* o4 = reinterpret_cast<float4*>(out + r * cols);
      for (size_t c = t0; c < cols / 4; c += stride) o4[c] = i4[c];
    } else {
      for (size_t c = t0; c < cols; c += stride) out[r * cols + c] = in[c];
    }
  }
}

// A one-element input everywhere (e.g. eps expanded to a parameter's shape).
__global__ void expand_scalar_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n, bool vec) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const float v = in[0];
  if (vec) {
    float4* o4 = reinterpret_cast<float4*>(out);
    for (size_t i = t0; i < n / 4; i += stride) o4[i] = make_float4(v, v, v, v);
    for (size_t i = 4 * (n / 4) + t0; i < n; i += stride) out[i] = v;
  } else {
    for (size_t i = t0; i < n; i += stride) out[i] = v;
  }
}

__global__ void expand_cols_kernel(const float* __restrict__ in, float* __restrict__ out, size_t rows, size_t cols) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (size_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float v = in[r];
    for (size_t c = t0; c < cols; c += stride) out[r * cols + c] = v;
  }
}

// One thread per output element; the reduced coordinates are walked as an
// odometer in row-major order, i.e. ascending input index (backend.rs:519-527,
// 1355-1372).
struct ReduceArgs {
  int rank;                       // input rank
  int64_t in_strides[kMaxRank];   // contiguous strides of the input
  int n_kept;                     // kept (non-reduced) dims, outer to inner
  int64_t kept_dims[kMaxRank];
  int64_t kept_strides[kMaxRank];  // input strides of the kept dims
  int n_red;                      // reduced dims, outer to inner
  int64_t red_dims[kMaxRank];
  int64_t red_strides[kMaxRank];
  int64_t red_count;
};

template <bool IS_MAX>
__global__ void reduce_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n_out, ReduceArgs a) {
  size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  size_t rem = o, base = 0;
  for (int d = a.n_kept - 1; d >= 0; --d) {
    size_t c = rem % (size_t)a.kept_dims[d];
    rem /= (size_t)a.kept_dims[d];
    base += c * (size_t)a.kept_strides[d];
  }
  float acc = IS_MAX ? -FLT_MAX : 0.0f;
  auto step = [&](float v) {
    if (IS_MAX) {
      if (v > acc) acc = v;
    } else {
      acc = acc + v;
    }
  };
  if (a.n_red == 1) {
    // RED_UNROLL loads in flight, then combined in index order: the same
    // sequence of operations as one load at a time.
    const float* p = in + base;
    const size_t st = (size_t)a.red_strides[0];
    const int64_t n = a.red_count;
    int64_t j = 0;
    for (; j + RED_UNROLL <= n; j += RED_UNROLL) {
      float v[RED_UNROLL];
#pragma unroll
      for (int u = 0; u < RED_UNROLL; ++u) v[u] = p[(size_t)(j + u) * st];
#pragma unroll
      for (int u = 0; u < RED_UNROLL; ++u) step(v[u]);
    }
    for (; j < n; ++j) step(p[(size_t)j * st]);
  } else {
    int64_t c[kMaxRank] = {0};
    size_t off = base;
    for (int64_t j = 0; j < a.red_count; ++j) {
      float v = in[off];
      if (IS_MAX) {
        if (v > acc) acc = v;
      } else {
        acc = acc + v;
      }
      for (int d = a.n_red - 1; d >= 0; --d) {  // odometer step
        off += (size_t)a.red_strides[d];
        if (++c[d] < a.red_dims[d]) break;
        off -= (size_t)(a.red_dims[d] * a.red_strides[d]);
        c[d] = 0;
      }
    }
  }
  out[o] = acc;
}

// Column reduction of a row-strided matrix (contiguous kept axis, one reduced axis of stride
// `st`), e.g. a bias gradient [rows, cols] -> [1, cols]. One thread per column leaves a
// 4096-column matrix with 64 waves; here every thread of a 256-thread block stages a
// CR_COLS-column slab through LDS (one 128-byte line per row, transposed so that each column's
// rows are contiguous, double-buffered, two slabs' loads in flight), and lane c of wave 0
// combines column c's values in row order: the same sequence of operations as reduce_kernel,
// so the result is bit-identical.  A matrix of at most 16 columns (a classifier head's
// bias gradient) takes slabs of 16 columns x 1024 rows instead of 32 x 128: the chain of
// additions is the same, with 8x fewer slab round trips in front of it.
constexpr int CR_THREADS = 256;
constexpr int CR_COLS = 32;
constexpr int CR_ROWS = 128;
constexpr int CR_NARROW_COLS = 16;
constexpr int CR_NARROW_ROWS = 1024;

template <bool IS_MAX, int CR_COLS_T = CR_COLS, int CR_ROWS_T = CR_ROWS>
__global__ void __launch_bounds__(CR_THREADS)
    colreduce_kernel(const float* __restrict__ in, float* __restrict__ out, size_t cols, int64_t rows, size_t st) {
  constexpr int CR_COLS = CR_COLS_T, CR_ROWS = CR_ROWS_T;
  constexpr int CR_LD = CR_ROWS + 4;               // LDS floats per staged column (16-byte aligned, offset banks)
  constexpr int GROUPS = CR_THREADS / CR_COLS;     // row quads loaded side by side
  constexpr int QUADS = CR_ROWS / (4 * GROUPS);    // row quads per thread per slab
  __shared__ __align__(16) float buf[2][CR_COLS * CR_LD];
  const int t = threadIdx.x;
  const int lc = t % CR_COLS, rg = t / CR_COLS;
  const size_t c = (size_t)blockIdx.x * CR_COLS + lc;
  const bool col_ok = c < cols;
  const int64_t n_slabs = (rows + CR_ROWS - 1) / CR_ROWS;
  // Rows past the end and columns past the edge load a clamped (in-bounds) element instead
  // of branching around the load: their values are never combined or stored.
  const float* src = in + (col_ok ? c : cols - 1);
  auto load = [&](int64_t k, float4 (&v)[QUADS]) {
#pragma unroll
    for (int q = 0; q < QUADS; ++q) {
      const int64_t r = k * CR_ROWS + 4 * (rg + GROUPS * q);
      v[q].x = src[(size_t)min(r, rows - 1) * st];
      v[q].y = src[(size_t)min(r + 1, rows - 1) * st];
      v[q].z = src[(size_t)min(r + 2, rows - 1) * st];
      v[q].w = src[(size_t)min(r + 3, rows - 1) * st];
    }
  };
  auto stash = [&](int b, const float4 (&v)[QUADS]) {
    float4* dst = reinterpret_cast<float4*>(buf[b] + lc * CR_LD);
#pragma unroll
    for (int q = 0; q < QUADS; ++q) dst[rg + GROUPS * q] = v[q];
  };
  float acc = IS_MAX ? -FLT_MAX : 0.0f;
  auto step = [&](float x) {
    if (IS_MAX) {
      if (x > acc) acc = x;
    } else {
      acc = acc + x;
    }
  };
  auto combine = [&](int64_t k) {
    const int n = (int)min((int64_t)CR_ROWS, rows - k * CR_ROWS);
    const float* col = buf[k & 1] + t * CR_LD;
    const float4* col4 = reinterpret_cast<const float4*>(col);
    int q = 0;
    for (; q + 8 <= n / 4; q += 8) {
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = col4[q + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        step(x[u].x);
        step(x[u].y);
        step(x[u].z);
        step(x[u].w);
      }
    }
    for (int r = 4 * q; r < n; ++r) step(col[r]);
  };
  // Slab k sits in LDS buffer k & 1; `cur` held slab k (already staged) and receives slab
  // k + 2, `nxt` holds slab k + 1 (in flight), staged after slab k is combined.
  auto iter = [&](int64_t k, float4 (&cur)[QUADS], const float4 (&nxt)[QUADS]) {
    if (k + 2 < n_slabs) load(k + 2, cur);
    if (t < CR_COLS) combine(k);
    if (k + 1 < n_slabs) stash((int)((k + 1) & 1), nxt);
    __syncthreads();
  };
  float4 va[QUADS], vb[QUADS];
  load(0, va);
  if (n_slabs > 1) load(1, vb);
  stash(0, va);
  __syncthreads();
  for (int64_t k = 0; k < n_slabs; k += 2) {
    iter(k, va, vb);
    if (k + 1 < n_slabs) iter(k + 1, vb, va);
  }
  if (t < CR_COLS && col_ok) out[c] = acc;
}

// max_to_shape_backward: thread per input element (backend.rs:1407-1424).
__global__ void max_bw_kernel(const float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ y,
                              float* __restrict__ out, size_t n, Dims in_dims, ExpandArgs map) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, o = 0;
    for (int d = in_dims.rank - 1; d >= 0; --d) {
      size_t c = rem % (size_t)in_dims.d[d];
      rem /= (size_t)in_dims.d[d];
      o += c * (size_t)map.in_strides[d];
    }
    float r = 0.0f;
    if (x[i] == y[o]) r = r + g[o];
    out[i] = r;
  }
}

// General transpose: thread per output element (backend.rs:264-284).
struct TransposeArgs {
  int rank;
  int64_t out_dims[kMaxRank];
  int64_t src_strides[kMaxRank];  // input stride of the input dim feeding output dim d
};

__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n, TransposeArgs a) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, idx = 0;
    for (int d = a.rank - 1; d >= 0; --d) {
      size_t c = rem % (size_t)a.out_dims[d];
      rem /= (size_t)a.out_dims[d];
      idx += c * (size_t)a.src_strides[d];
    }
    out[i] = in[idx];
  }
}

// Batched 2-D transpose of the last two dims through a padded LDS tile.
__global__ void transpose2d_kernel(const float* __restrict__ in, float* __restrict__ out, size_t rows, size_t cols) {
  __shared__ float tile[32][33];
  size_t b = blockIdx.z;
  const float* src = in + b * rows * cols;
  float* dst = out + b * rows * cols;
  size_t c0 = (size_t)blockIdx.x * 32, r0 = (size_t)blockIdx.y * 32;
  int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
  for (int k = ty; k < 32; k += 8) {
    size_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    size_t c = c0 + k, r = r0 + tx;  // output row c, column r
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][k];
  }
}

__global__ void nan_inf_kernel(const float* __restrict__ a, size_t n, int* __restrict__ flag) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  bool bad = false;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) bad |= !isfinite(a[i]);
  if (bad) *flag = 1;  // every writer stores the same value
}

__global__ void zero_int_kernel(int* p) { *p = 0; }

// ---------------------------------------------------------------- host helpers
void check_rank(size_t rank, const char* op) {
  if (rank > (size_t)kMaxRank)
    fail(ORCA_HIP_ERR_INTERNAL, std::string(op) + ": rank " + std::to_string(rank) + " exceeds " +
                                    std::to_string(kMaxRank));
}

// backend.rs:17-26: left-pad with ones; a longer shape pads to all ones.
void pad_left(const size_t* d, size_t r, size_t target, int64_t* out) {
  for (size_t i = 0; i < target; ++i) out[i] = 1;
  if (r <= target)
    for (size_t i = 0; i < r; ++i) out[target - r + i] = (int64_t)d[i];
}

void contiguous_strides(const int64_t* d, int rank, int64_t* s) {
  int64_t cur = 1;
  for (int i = rank - 1; i >= 0; --i) {
    s[i] = cur;
    cur *= d[i];
  }
}

// The kept/reduced split of an `in -> out` reduction (sum_to_shape / max_to_shape).
ReduceArgs make_reduce(const size_t* in_shape, size_t in_rank, const size_t* out_shape, size_t out_rank,
                       const char* op) {
  check_rank(in_rank, op);
  check_rank(out_rank, op);
  int64_t pout[kMaxRank], ind[kMaxRank];
  pad_left(out_shape, out_rank, in_rank, pout);
  for (size_t i = 0; i < in_rank; ++i) ind[i] = (int64_t)in_shape[i];
  for (size_t i = 0; i < in_rank; ++i)
    if (pout[i] != 1 && pout[i] != ind[i])
      fail(ORCA_HIP_ERR_SHAPE, std::string("Shape mismatch during ") + op + ": expected a shape reducible from " +
                                   shape_str(in_shape, in_rank) + ", got " + shape_str(out_shape, out_rank));
  ReduceArgs a{};
  a.rank = (int)in_rank;
  contiguous_strides(ind, (int)in_rank, a.in_strides);
  a.red_count = 1;
  for (size_t i = 0; i < in_rank; ++i) {
    if (pout[i] != 1) {
      a.kept_dims[a.n_kept] = ind[i];
      a.kept_strides[a.n_kept] = a.in_strides[i];
      ++a.n_kept;
    } else if (ind[i] != 1) {
      a.red_dims[a.n_red] = ind[i];
      a.red_strides[a.n_red] = a.in_strides[i];
      a.red_count *= ind[i];
      ++a.n_red;
    }
  }
  if (a.n_red == 0) {  // nothing reduced: a single visit per output
    a.n_red = 1;
    a.red_dims[0] = 1;
    a.red_strides[0] = 0;
  }
  // Adjacent dims that tile memory contiguously become one dim: the odometer then visits the
  // same elements in the same order, with fewer index steps (and [B, S, N] -> [N] reaches the
  // one-axis paths).
  auto merge = [](int& n, int64_t* dims, int64_t* strides) {
    int m = 0;
    for (int d = 1; d < n; ++d) {
      if (strides[m] == strides[d] * dims[d]) {
        dims[m] *= dims[d];
        strides[m] = strides[d];
      } else {
        ++m;
        dims[m] = dims[d];
        strides[m] = strides[d];
      }
    }
    if (n > 0) n = m + 1;
  };
  merge(a.n_kept, a.kept_dims, a.kept_strides);
  merge(a.n_red, a.red_dims, a.red_strides);
  return a;
}

const float* as_f(const void* p) { return static_cast<const float*>(p); }

}  // namespace

// colsum[c] = sum_r src[r * ld + c] in ascending r, through colreduce_kernel:
// the same sequence of f32 additions as sum_to_shape's loop.
void launch_colsum(orca_hip_ctx* ctx, const float* src, size_t rows, size_t cols, size_t ld, float* colsum) {
  if (cols == 0) return;
  if (rows == 0) {
    launch_fill(ctx, colsum, 0.0f, cols);
    return;
  }
  ProfScope ps(ctx, "colsum_rows", 0.0, 4.0 * (double)rows * cols + 4.0 * cols);
  if (cols <= CR_NARROW_COLS) {
    hipLaunchKernelGGL((colreduce_kernel<false, CR_NARROW_COLS, CR_NARROW_ROWS>), dim3(1), dim3(CR_THREADS), 0,
                       ctx->stream, src, colsum, cols, (int64_t)rows, ld);
  } else {
    const unsigned g = (unsigned)((cols + CR_COLS - 1) / CR_COLS);
    hipLaunchKernelGGL(colreduce_kernel<false>, dim3(g), dim3(CR_THREADS), 0, ctx->stream, src, colsum, cols,
                       (int64_t)rows, ld);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

}  // namespace orca_hip

using namespace orca_hip;

#define EW1_ENTRY(NAME, OPEXPR)                                                                      \
  int orca_hip_##NAME(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, int dtype, \
                      void** out) {                                                                  \
    return guard([&] {                                                                               \
      bind(ctx);                                                                                     \
      check_f32(dtype, #NAME);                                                                       \
      size_t n = numel(shape, rank);                                                                 \
      float* o = new_output(ctx, n);                                                                 \
      run_ew1(ctx, "ew_" #NAME, as_f(s), o, n, OPEXPR);                                              \
      *out = o;                                                                                      \
    });                                                                                              \
  }

#define EW2_ENTRY(NAME, OPEXPR)                                                                          \
  int orca_hip_##NAME(orca_hip_ctx* ctx, const void* a, const void* b, const size_t* shape, size_t rank, \
                      int dtype, void** out) {                                                           \
    return guard([&] {                                                                                   \
      bind(ctx);                                                                                         \
      check_f32(dtype, #NAME);                                                                           \
      size_t n = numel(shape, rank);                                                                     \
      float* o = new_output(ctx, n);                                                                     \
      run_ew2(ctx, "ew_" #NAME, as_f(a), as_f(b), o, n, OPEXPR);                                         \
      *out = o;                                                                                          \
    });                                                                                                  \
  }

extern "C" {

// backend.rs:104-128, 291-315, 340-373, 635-659
EW2_ENTRY(add, OpAdd{})
EW2_ENTRY(sub, OpSub{})
EW2_ENTRY(mul, OpMul{})
EW2_ENTRY(div, OpDiv{})
// backend.rs:414-438, 440-464, 583-633, 678-701, 734-759
EW2_ENTRY(relu_backward, OpReluBw{})
EW2_ENTRY(sigmoid_backward, OpSigBw{})
EW2_ENTRY(exp_backward, OpExpBw{})
EW2_ENTRY(log_backward, OpLogBw{})
EW2_ENTRY(sqrt_backward, OpSqrtBw{})
EW2_ENTRY(div_backward_lhs, OpDiv{})
// backend.rs:375-412, 549-581, 661-676
EW1_ENTRY(relu, OpRelu{})
EW1_ENTRY(sigmoid, OpSigmoid{})
EW1_ENTRY(exp, OpExp{})
EW1_ENTRY(log, OpLog{})
EW1_ENTRY(sqrt, OpSqrt{})

// backend.rs:317-338
int orca_hip_mul_scalar(orca_hip_ctx* ctx, const void* s, float scalar, const size_t* shape, size_t rank, int dtype,
                        void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "mul_scalar");
    size_t n = numel(shape, rank);
    float* o = new_output(ctx, n);
    run_ew1(ctx, "ew_mul_scalar", as_f(s), o, n, OpScale{scalar});
    *out = o;
  });
}

// backend.rs:703-732
int orca_hip_div_backward_rhs(orca_hip_ctx* ctx, const void* g, const void* l, const void* r, const size_t* shape,
                              size_t rank, int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "div_backward_rhs");
    size_t n = numel(shape, rank);
    for (const void* a : {g, l, r}) check_extent(ctx, a, n * sizeof(float), "div_backward_rhs");
    float* o = new_output(ctx, n);
    if (n) {
      unsigned gsz = grid_for(n, kBlock, ctx->num_cus * 16);
      hipLaunchKernelGGL(ew3_kernel<OpDivBwRhs>, dim3(gsz), dim3(kBlock), 0, ctx->stream, as_f(g), as_f(l), as_f(r),
                         o, n, OpDivBwRhs{});
      ORCA_HIP_CHECK(hipGetLastError());
    }
    *out = o;
  });
}

// backend.rs:761-774 (no shape: the storages' element count)
int orca_hip_accumulate_grad(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t n, void** out) {
  return guard([&] {
    bind(ctx);
    float* o = new_output(ctx, n);
    run_ew2(ctx, "ew_accumulate_grad", as_f(lhs), as_f(rhs), o, n, OpAdd{});
    *out = o;
  });
}

// backend.rs:73-85
int orca_hip_zeros(orca_hip_ctx* ctx, const size_t* shape, size_t rank, int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "zeros");
    size_t n = numel(shape, rank);
    float* o = new_output(ctx, n);
    launch_fill(ctx, o, 0.0f, n);
    *out = o;
  });
}

// backend.rs:87-89
int orca_hip_from_f32_slice(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const float* data, size_t n,
                            void** out) {
  return guard([&] {
    bind(ctx);
    size_t want = numel(shape, rank);
    if (n != want)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during from_f32_slice: expected " + std::to_string(want) +
                                   " elements, got " + std::to_string(n));
    float* o = new_output(ctx, n);
    upload_async(ctx, o, data, n * sizeof(float));  // stream-ordered, no host wait
    *out = o;
  });
}

// backend.rs:91-102
int orca_hip_to_f32_vec(orca_hip_ctx* ctx, const void* s, size_t n, float* host_out) {
  return guard([&] {
    bind(ctx);
    if (!n) return;
    check_extent(ctx, s, n * sizeof(float), "to_f32_vec");
    join_side(ctx);
    ORCA_HIP_CHECK(hipMemcpyAsync(host_out, s, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    host_sync(ctx);
  });
}

int orca_hip_from_bytes(orca_hip_ctx* ctx, const size_t* shape, size_t rank, const uint8_t* bytes, size_t n_bytes,
                        int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "from_bytes");
    size_t want = numel(shape, rank) * sizeof(float);
    if (n_bytes != want)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during from_bytes: expected " + std::to_string(want) +
                                   " bytes, got " + std::to_string(n_bytes));
    float* o = new_output(ctx, want / sizeof(float));
    upload_async(ctx, o, bytes, want);  // stream-ordered, no host wait
    *out = o;
  });
}

int orca_hip_to_bytes(orca_hip_ctx* ctx, const void* s, size_t n_bytes, uint8_t* host_out) {
  return guard([&] {
    bind(ctx);
    if (!n_bytes) return;
    check_extent(ctx, s, n_bytes, "to_bytes");
    join_side(ctx);
    ORCA_HIP_CHECK(hipMemcpyAsync(host_out, s, n_bytes, hipMemcpyDeviceToHost, ctx->stream));
    host_sync(ctx);
  });
}

// backend.rs:466-497
int orca_hip_expand(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank, const size_t* out_shape,
                    size_t out_rank, int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "expand");
    check_rank(in_rank, "expand");
    check_rank(out_rank, "expand");
    int64_t pin[kMaxRank], st[kMaxRank];
    pad_left(in_shape, in_rank, out_rank, pin);
    for (size_t d = 0; d < out_rank; ++d)
      if (pin[d] != 1 && pin[d] != (int64_t)out_shape[d])
        fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during expand: expected a shape broadcastable to " +
                                     shape_str(out_shape, out_rank) + ", got " + shape_str(in_shape, in_rank));
    contiguous_strides(pin, (int)out_rank, st);
    ExpandArgs a{};
    a.rank = (int)out_rank;
    for (size_t d = 0; d < out_rank; ++d) {
      a.out_dims[d] = (int64_t)out_shape[d];
      a.in_strides[d] = pin[d] == 1 ? 0 : st[d];
    }
    check_extent(ctx, s, numel(in_shape, in_rank) * sizeof(float), "expand");
    size_t n = numel(out_shape, out_rank);
    float* o = new_output(ctx, n);
    if (n) {
      ProfScope ps(ctx, "expand", 0.0, 8.0 * n);
      // The output as [rows, cols] with cols its last dim: a row broadcast
      // takes the input only along the last dim, a column broadcast only
      // along the others (the input's last dim is 1).
      const size_t cols = out_rank ? out_shape[out_rank - 1] : 1, rows = cols ? n / cols : 0;
      bool row_bc = out_rank >= 1 && pin[out_rank - 1] == (int64_t)cols, col_bc = out_rank >= 2 && pin[out_rank - 1] == 1;
      for (size_t d = 0; d + 1 < out_rank; ++d) {
        if (pin[d] != 1) row_bc = false;
        if (pin[d] != (int64_t)out_shape[d]) col_bc = false;
      }
      const unsigned gy = (unsigned)std::min<size_t>(rows, 65535);
      if (numel(in_shape, in_rank) == 1 && n > 1) {
        const bool vec = aligned16(o);
        unsigned g = grid_for(vec ? (n + 3) / 4 : n, kBlock, ctx->num_cus * 16);
        hipLaunchKernelGGL(expand_scalar_kernel, dim3(g), dim3(kBlock), 0, ctx->stream, as_f(s), o, n, vec);
      } else if (row_bc && rows > 1) {
        const bool vec = cols % 4 == 0 && aligned16(s) && aligned16(o);
        const size_t per_row = vec ? cols / 4 : cols;
        const unsigned gx = (unsigned)std::min<size_t>((per_row + kBlock - 1) / kBlock, 64);
        hipLaunchKernelGGL(expand_rows_kernel, dim3(gx, gy), dim3(kBlock), 0, ctx->stream, as_f(s), o, rows, cols, vec);
      } else if (col_bc && cols > 1) {
        const unsigned gx = (unsigned)std::min<size_t>((cols + kBlock - 1) / kBlock, 64);
        hipLaunchKernelGGL(expand_cols_kernel, dim3(gx, gy), dim3(kBlock), 0, ctx->stream, as_f(s), o, rows, cols);
      } else {
        unsigned g = grid_for(n, kBlock, ctx->num_cus * 16);
        hipLaunchKernelGGL(expand_kernel, dim3(g), dim3(kBlock), 0, ctx->stream, as_f(s), o, n, a);
      }
      ORCA_HIP_CHECK(hipGetLastError());
    }
    *out = o;
  });
}

static int reduce_entry(orca_hip_ctx* ctx, bool is_max, const void* s, const size_t* in_shape, size_t in_rank,
                        const size_t* out_shape, size_t out_rank, int dtype, void** out) {
  const char* op = is_max ? "max_to_shape" : "sum_to_shape";
  return guard([&] {
    bind(ctx);
    check_f32(dtype, op);
    if (is_max && out_rank > in_rank)
      fail(ORCA_HIP_ERR_SHAPE, std::string("Shape mismatch during ") + op + ": output rank exceeds input rank");
    ReduceArgs a = make_reduce(in_shape, in_rank, out_shape, out_rank, op);
    check_extent(ctx, s, numel(in_shape, in_rank) * sizeof(float), op);
    size_t n_out = numel(out_shape, out_rank);
    float* o = new_output(ctx, n_out);
    if (n_out) {
      size_t n_in = numel(in_shape, in_rank);
      if (n_in == 0) {
        launch_fill(ctx, o, is_max ? -FLT_MAX : 0.0f, n_out);
      } else {
        // Out-of-range output slots (rank padding quirk) stay zero like the reference.
        if ((size_t)a.red_count * n_out != n_in) launch_fill(ctx, o, 0.0f, n_out);
        if (a.red_count == 1 && n_out == n_in && a.n_kept == 1 && a.kept_strides[0] == 1) {
          if (is_max)
            run_ew1(ctx, op, as_f(s), o, n_in, OpMaxVisit{});
          else
            run_ew1(ctx, op, as_f(s), o, n_in, OpSumVisit{});
          *out = o;
          return;
        }
        size_t n_threads = n_in / (size_t)a.red_count;
        ProfScope ps(ctx, op, 0.0, 4.0 * (n_in + n_out));
        unsigned g = (unsigned)((n_threads + 63) / 64);
        if (a.n_red == 1 && a.n_kept == 1 && a.kept_strides[0] == 1 && a.red_count >= CR_ROWS) {
          const unsigned gc = (unsigned)((n_threads + CR_COLS - 1) / CR_COLS);
          const size_t st = (size_t)a.red_strides[0];
          if (n_threads <= CR_NARROW_COLS) {
            if (is_max)
              hipLaunchKernelGGL((colreduce_kernel<true, CR_NARROW_COLS, CR_NARROW_ROWS>), dim3(1), dim3(CR_THREADS),
                                 0, ctx->stream, as_f(s), o, n_threads, a.red_count, st);
            else
              hipLaunchKernelGGL((colreduce_kernel<false, CR_NARROW_COLS, CR_NARROW_ROWS>), dim3(1), dim3(CR_THREADS),
                                 0, ctx->stream, as_f(s), o, n_threads, a.red_count, st);
          } else if (is_max)
            hipLaunchKernelGGL(colreduce_kernel<true>, dim3(gc), dim3(CR_THREADS), 0, ctx->stream, as_f(s), o,
                               n_threads, a.red_count, st);
          else
            hipLaunchKernelGGL(colreduce_kernel<false>, dim3(gc), dim3(CR_THREADS), 0, ctx->stream, as_f(s), o,
                               n_threads, a.red_count, st);
        } else if (is_max)
          hipLaunchKernelGGL(reduce_kernel<true>, dim3(g), dim3(64), 0, ctx->stream, as_f(s), o, n_threads, a);
        else
          hipLaunchKernelGGL(reduce_kernel<false>, dim3(g), dim3(64), 0, ctx->stream, as_f(s), o, n_threads, a);
        ORCA_HIP_CHECK(hipGetLastError());
      }
    }
    *out = o;
  });
}

// backend.rs:499-530
int orca_hip_sum_to_shape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, void** out) {
  return reduce_entry(ctx, false, s, in_shape, in_rank, out_shape, out_rank, dtype, out);
}

// backend.rs:1336-1381
int orca_hip_max_to_shape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, void** out) {
  return reduce_entry(ctx, true, s, in_shape, in_rank, out_shape, out_rank, dtype, out);
}

// backend.rs:1383-1435
int orca_hip_max_to_shape_backward(orca_hip_ctx* ctx, const void* g, const void* x, const void* y,
                                   const size_t* in_shape, size_t in_rank, const size_t* out_shape, size_t out_rank,
                                   int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "max_to_shape_backward");
    if (out_rank > in_rank) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during max_to_shape_backward: output rank exceeds input rank");
    check_rank(in_rank, "max_to_shape_backward");
    check_extent(ctx, g, numel(out_shape, out_rank) * sizeof(float), "max_to_shape_backward (grad)");
    check_extent(ctx, x, numel(in_shape, in_rank) * sizeof(float), "max_to_shape_backward (input)");
    check_extent(ctx, y, numel(out_shape, out_rank) * sizeof(float), "max_to_shape_backward (output)");
    int64_t pout[kMaxRank], st[kMaxRank];
    pad_left(out_shape, out_rank, in_rank, pout);
    for (size_t d = 0; d < in_rank; ++d)
      if (pout[d] != 1 && pout[d] != (int64_t)in_shape[d])
        fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during max_to_shape_backward: " + shape_str(out_shape, out_rank) +
                                     " is not a reduction of " + shape_str(in_shape, in_rank));
    contiguous_strides(pout, (int)in_rank, st);
    Dims dims{};
    ExpandArgs map{};
    dims.rank = (int)in_rank;
    for (size_t d = 0; d < in_rank; ++d) {
      dims.d[d] = (int64_t)in_shape[d];
      map.in_strides[d] = pout[d] == 1 ? 0 : st[d];
    }
    size_t n = numel(in_shape, in_rank);
    float* o = new_output(ctx, n);
    if (n) {
      unsigned gsz = grid_for(n, kBlock, ctx->num_cus * 16);
      hipLaunchKernelGGL(max_bw_kernel, dim3(gsz), dim3(kBlock), 0, ctx->stream, as_f(g), as_f(x), as_f(y), o, n, dims,
                         map);
      ORCA_HIP_CHECK(hipGetLastError());
    }
    *out = o;
  });
}

// backend.rs:532-547 -- a copy here (a Rust shim returns a clone of the storage instead)
int orca_hip_reshape(orca_hip_ctx* ctx, const void* s, const size_t* in_shape, size_t in_rank, const size_t* out_shape,
                     size_t out_rank, int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    size_t n = numel(in_shape, in_rank), m = numel(out_shape, out_rank);
    if (n != m)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during reshape: expected " + std::to_string(n) + " elements, got " +
                                   std::to_string(m) + " elements");
    (void)dtype;
    float* o = new_output(ctx, n);
    launch_copy(ctx, o, as_f(s), n);
    *out = o;
  });
}

// backend.rs:223-289
int orca_hip_transpose(orca_hip_ctx* ctx, const void* s, const size_t* shape, size_t rank, size_t d0, size_t d1,
                       int dtype, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "transpose");
    if (d0 >= rank || d1 >= rank) fail(ORCA_HIP_ERR_INTERNAL, "Invalid transpose dimensions");
    check_rank(rank, "transpose");
    size_t n = numel(shape, rank);
    check_extent(ctx, s, n * sizeof(float), "transpose");
    float* o = new_output(ctx, n);
    if (n) {
      ProfScope ps(ctx, "transpose", 0.0, 8.0 * n);
      size_t lo = d0 < d1 ? d0 : d1, hi = d0 < d1 ? d1 : d0;
      if (rank >= 2 && lo == rank - 2 && hi == rank - 1) {
        size_t rows = shape[rank - 2], cols = shape[rank - 1], batch = n / (rows * cols);
        dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32), (unsigned)batch);
        hipLaunchKernelGGL(transpose2d_kernel, grid, dim3(256), 0, ctx->stream, as_f(s), o, rows, cols);
      } else {
        int64_t ind[kMaxRank], ist[kMaxRank];
        for (size_t i = 0; i < rank; ++i) ind[i] = (int64_t)shape[i];
        contiguous_strides(ind, (int)rank, ist);
        TransposeArgs a{};
        a.rank = (int)rank;
        for (size_t i = 0; i < rank; ++i) {
          size_t src = i == d0 ? d1 : (i == d1 ? d0 : i);
          a.out_dims[i] = ind[src];
          a.src_strides[i] = ist[src];
        }
        unsigned g = grid_for(n, kBlock, ctx->num_cus * 16);
        hipLaunchKernelGGL(transpose_kernel, dim3(g), dim3(kBlock), 0, ctx->stream, as_f(s), o, n, a);
      }
      ORCA_HIP_CHECK(hipGetLastError());
    }
    *out = o;
  });
}

// backend.rs:1316-1334
int orca_hip_has_nan_or_inf(orca_hip_ctx* ctx, const void* s, size_t n, int dtype, int* result) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "has_nan_or_inf");
    if (!result) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    join_side(ctx);  // the scan below reads what the side stream may have written
    Scratch flag(ctx, sizeof(int));
    hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(1), 0, ctx->stream, flag.as<int>());
    if (n) {
      unsigned g = grid_for(n, kBlock, ctx->num_cus * 8);
      hipLaunchKernelGGL(nan_inf_kernel, dim3(g), dim3(kBlock), 0, ctx->stream, as_f(s), n, flag.as<int>());
    }
    ORCA_HIP_CHECK(hipGetLastError());
    int h = 0;
    ORCA_HIP_CHECK(hipMemcpyAsync(&h, flag.as<int>(), sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    host_sync(ctx);
    *result = h;
  });
}

}  // extern "C"
