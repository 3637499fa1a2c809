// Fused kernels beyond the Backend trait:
//  * softmax cross-entropy forward + gradient + argmax, one wave64 per row,
//    replacing the ~21-op composition of python/orca/nn/loss.py:59-100 and
//    the tape's backward through it;
//  * ReLU-mask backward with the bias-gradient column sum;
//  * single-pass AdamW / SGD over flat parameter arenas.
// Built with -ffp-contract=off so the per-element arithmetic is the
// reference's separate f32 operations.
#include <cfloat>
#include <cmath>

#include <map>
#include <mutex>

#include "ce_row.hpp"
#include "runtime.hpp"

namespace orca_hip {
// Fixed device scratch of orca_hip_relu_bw_colsum_noalloc: 2^20 floats (4 MiB)
// per GPU, held until the process ends.
constexpr size_t kStaticScratchFloats = size_t(1) << 20;
}  // namespace orca_hip

// One copy per GPU the library runs on.  In host code this name only stands in
// for the symbol: kernels receive the per-device address that static_scratch()
// resolves with hipGetSymbolAddress.
static __device__ __align__(256) float scratch[orca_hip::kStaticScratchFloats];

namespace orca_hip {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// One wave per row.  Logits stay in registers, VPL values per lane: column
// c = lane + 64 j (scalar loads), or, when VEC (C a multiple of 4 and 16-byte
// aligned rows), c = 256 (j / 4) + 4 lane + j % 4 so that logits and the
// gradient move as float4s.  Their loads and stores are ordinary ones: the
// logits usually come straight from the product before (still in the
// memory-side cache) and the gradient goes straight to the one after, which
// measured faster than non-temporal accesses (43.6 against 47.1 us on
// [8192, 4096], repeated launches).  FULL: C == 64 VPL, every slot is a
// column (no bounds checks).
// LABELS: class-index targets (compared), else one-hot rows (read where used).
template <int VPL, bool VEC, bool FULL, bool LABELS>
__global__ void __launch_bounds__(256) softmax_ce_kernel(const float* __restrict__ logits, int B, int C,
                                                         const float* __restrict__ onehot,
                                                         const int32_t* __restrict__ labels, float inv_b,
                                                         float* __restrict__ row_loss, float* __restrict__ dlogits,
                                                         int32_t* __restrict__ preds, int* __restrict__ row_correct) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= B) return;
  const float* xr = logits + (int64_t)row * C;
  const float* tr = LABELS ? nullptr : onehot + (int64_t)row * C;
  float* dr = dlogits ? dlogits + (int64_t)row * C : nullptr;
  const int label = LABELS ? labels[row] : -1;
  auto col = [&](int j) -> int { return VEC ? (j >> 2) * 256 + lane * 4 + (j & 3) : lane + 64 * j; };
  auto valid = [&](int j) -> bool { return FULL || col(j) < C; };
  auto tval = [&](int j) -> float {
    if (!valid(j)) return 0.0f;
    return LABELS ? (col(j) == label ? 1.0f : 0.0f) : tr[col(j)];
  };
  float x[VPL];
  if (VEC) {
#pragma unroll
    for (int q = 0; q < VPL / 4; ++q) {
      const int c0 = q * 256 + lane * 4;
      floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (FULL || c0 < C) v = *reinterpret_cast<const floatx4*>(xr + c0);
      x[4 * q] = v.x;
      x[4 * q + 1] = v.y;
      x[4 * q + 2] = v.z;
      x[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) x[j] = valid(j) ? xr[col(j)] : 0.0f;
  }
  float buf[4];
  auto store = [&](int j, float v) {
    if (VEC) {
      buf[j & 3] = v;
      if ((j & 3) == 3)
        *reinterpret_cast<floatx4*>(dr + col(j) - 3) = floatx4{buf[0], buf[1], buf[2], buf[3]};
    } else {
      dr[col(j)] = v;
    }
  };
  CeRowOut r;
  if constexpr (LABELS) {
    // The label's slot: col(j) = label for j = jl on one lane.
    int jl = -1;
    if (label >= 0 && label < C) {
      if (VEC && (((label & 255) >> 2) == lane)) jl = 4 * (label >> 8) + (label & 3);
      if (!VEC && (label & 63) == lane) jl = label >> 6;
    }
    r = ce_row_label<VPL>(x, valid, col, [&](int j) { return xr[col(j)]; }, label, jl, label >= 0 && label < C,
                          lane == 0, inv_b, dr != nullptr, store, preds || row_correct);
  } else {
    r = ce_row<VPL>(x, valid, tval, col, false, label, inv_b, dr != nullptr, store, preds || row_correct);
    r.has_loss = lane == 0;
  }
  if (r.has_loss) row_loss[row] = r.loss;
  if (lane == 0) {
    if (preds) preds[row] = r.pred;
    if (row_correct) row_correct[row] = (r.pred == r.target) ? 1 : 0;
  }
}

// Rows of 1025..4096 logits: one 256-thread block per row, 16 values per
// thread (VEC: float4 column groups tid + 256 q, so every load and store is a
// coalesced float4; otherwise columns tid + 256 j).  The row reductions run
// across the block's 4 waves (BlockRed); with 16 values a thread holds few
// registers, so many rows are in flight.
template <bool VEC, bool FULL, bool LABELS>
__global__ void __launch_bounds__(256) softmax_ce_block_kernel(const float* __restrict__ logits, int B, int C,
                                                               const float* __restrict__ onehot,
                                                               const int32_t* __restrict__ labels, float inv_b,
                                                               float* __restrict__ row_loss,
                                                               float* __restrict__ dlogits,
                                                               int32_t* __restrict__ preds,
                                                               int* __restrict__ row_correct) {
  constexpr int VPT = 16;
  __shared__ float red_f[4];
  __shared__ int red_i[4];
  const BlockRed<4> red{red_f, red_i};
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const float* xr = logits + (int64_t)row * C;
  const float* tr = LABELS ? nullptr : onehot + (int64_t)row * C;
  float* dr = dlogits ? dlogits + (int64_t)row * C : nullptr;
  const int label = LABELS ? labels[row] : -1;
  auto col = [&](int j) -> int { return VEC ? (j >> 2) * 1024 + tid * 4 + (j & 3) : tid + 256 * j; };
  auto valid = [&](int j) -> bool { return FULL || col(j) < C; };
  float x[VPT];
  if (VEC) {
#pragma unroll
    for (int q = 0; q < VPT / 4; ++q) {
      const int c0 = q * 1024 + tid * 4;
      floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (FULL || c0 < C) v = *reinterpret_cast<const floatx4*>(xr + c0);
      x[4 * q] = v.x;
      x[4 * q + 1] = v.y;
      x[4 * q + 2] = v.z;
      x[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) x[j] = valid(j) ? xr[col(j)] : 0.0f;
  }
  float buf[4];
  auto store = [&](int j, float v) {
    if (VEC) {
      buf[j & 3] = v;
      if ((j & 3) == 3)
        *reinterpret_cast<floatx4*>(dr + col(j) - 3) = floatx4{buf[0], buf[1], buf[2], buf[3]};
    } else {
      dr[col(j)] = v;
    }
  };
  const bool want_argmax = preds || row_correct;
  CeRowOut r;
  if constexpr (LABELS) {
    // The label's slot: col(j) = label for j = jl on one thread.
    int jl = -1;
    if (label >= 0 && label < C) {
      if (VEC && (((label & 1023) >> 2) == tid)) jl = 4 * (label >> 10) + (label & 3);
      if (!VEC && (label & 255) == tid) jl = label >> 8;
    }
    r = ce_row_label<VPT>(x, valid, col, [&](int j) { return xr[col(j)]; }, label, jl, label >= 0 && label < C,
                          tid == 0, inv_b, dr != nullptr, store, want_argmax, red);
  } else {
    auto tval = [&](int j) -> float { return valid(j) ? tr[col(j)] : 0.0f; };
    r = ce_row<VPT>(x, valid, tval, col, false, label, inv_b, dr != nullptr, store, want_argmax, red);
    r.has_loss = tid == 0;
  }
  if (r.has_loss) row_loss[row] = r.loss;
  if (tid == 0) {
    if (preds) preds[row] = r.pred;
    if (row_correct) row_correct[row] = (r.pred == r.target) ? 1 : 0;
  }
}

// loss = (sum of row losses) * (1/B); correct = number of matching rows.
__global__ void __launch_bounds__(1024) ce_finish_kernel(const float* __restrict__ row_loss,
                                                          const int* __restrict__ row_correct, int B, float inv_b,
                                                          float* __restrict__ loss, int64_t* __restrict__ correct) {
  __shared__ float ls[1024];
  __shared__ long long cs[1024];
  const int t = threadIdx.x;
  const int per = (B + 1023) / 1024;
  float s = 0.0f;
  long long c = 0;
  for (int k = 0; k < per; ++k) {
    int r = t * per + k;
    if (r < B) {
      s = s + row_loss[r];
      if (row_correct) c += row_correct[r];
    }
  }
  ls[t] = s;
  cs[t] = c;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (t < w) {
      ls[t] = ls[t] + ls[t + w];
      cs[t] += cs[t + w];
    }
    __syncthreads();
  }
  if (t == 0) {
    if (loss) *loss = ls[0] * inv_b;
    if (correct) *correct = cs[0];
  }
}

constexpr int kRowsPerChunk = 64;  // rows per column-sum partial of the ReLU-backward kernels

// dpre = pre > 0 ? g : 0 and per-chunk column partial sums (4 columns per
// thread).  Rows go RB_UNROLL at a time, all loads issued before any use;
// g and pre are read with ordinary loads, dpre is written with non-temporal
// stores ([8192, 4096]: 62.0 us against 67.8 with non-temporal loads too,
// 77.1 with ordinary stores too).
constexpr int RB_UNROLL = 8;

__global__ void __launch_bounds__(256) relu_bw_colsum_vec_kernel(const float4* __restrict__ g, const float4* __restrict__ pre,
                                                                 size_t rows, size_t cols4, int rows_per_chunk,
                                                                 float4* __restrict__ dpre, float4* __restrict__ partial) {
  size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols4) return;
  size_t r0 = (size_t)blockIdx.y * rows_per_chunk;
  size_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
  const floatx4* gv = reinterpret_cast<const floatx4*>(g);
  const floatx4* pv = reinterpret_cast<const floatx4*>(pre);
  floatx4* dv = reinterpret_cast<floatx4*>(dpre);
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (size_t rb = r0; rb < r1; rb += RB_UNROLL) {
    floatx4 ga[RB_UNROLL], pa[RB_UNROLL];
#pragma unroll
    for (int u = 0; u < RB_UNROLL; ++u) {
      const size_t r = rb + u;
      if (r < r1) {
        ga[u] = gv[r * cols4 + c];
        pa[u] = pv[r * cols4 + c];
      }
    }
#pragma unroll
    for (int u = 0; u < RB_UNROLL; ++u) {
      const size_t r = rb + u;
      if (r < r1) {
        const floatx4 gg = ga[u], pp = pa[u];
        const floatx4 d = {pp.x > 0.0f ? gg.x : 0.0f, pp.y > 0.0f ? gg.y : 0.0f, pp.z > 0.0f ? gg.z : 0.0f,
                           pp.w > 0.0f ? gg.w : 0.0f};
        __builtin_nontemporal_store(d, dv + r * cols4 + c);
        s.x = s.x + d.x;
        s.y = s.y + d.y;
        s.z = s.z + d.z;
        s.w = s.w + d.w;
      }
    }
  }
  if (partial) partial[(size_t)blockIdx.y * cols4 + c] = s;
}

__global__ void __launch_bounds__(256) relu_bw_colsum_scalar_kernel(const float* __restrict__ g, const float* __restrict__ pre,
                                                                    size_t rows, size_t cols, int rows_per_chunk,
                                                                    float* __restrict__ dpre, float* __restrict__ partial) {
  size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  size_t r0 = (size_t)blockIdx.y * rows_per_chunk;
  size_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
  float s = 0.0f;
  for (size_t r = r0; r < r1; ++r) {
    float d = pre[r * cols + c] > 0.0f ? g[r * cols + c] : 0.0f;
    dpre[r * cols + c] = d;
    s = s + d;
  }
  if (partial) partial[(size_t)blockIdx.y * cols + c] = s;
}

// colsum[c] from the per-chunk partials: a 256-thread block takes
// CR_PARTS_COLS columns, and the CR_PARTS threads of a column each add one
// contiguous quarter of the chunks in chunk order (RB_UNROLL loads issued
// before their adds); the quarters are then added in order,
// ((q0 + q1) + q2) + q3 -- a fixed order, so the result is deterministic.
constexpr int CR_PARTS = 4;
constexpr int CR_PARTS_COLS = 256 / CR_PARTS;
__global__ void __launch_bounds__(256) chunk_reduce_kernel(const float* __restrict__ partial, int chunks, size_t cols,
                                                           float* __restrict__ out) {
  __shared__ float q[CR_PARTS][CR_PARTS_COLS];
  const int lc = threadIdx.x % CR_PARTS_COLS, part = threadIdx.x / CR_PARTS_COLS;
  const size_t c = (size_t)blockIdx.x * CR_PARTS_COLS + lc;
  const int per = (chunks + CR_PARTS - 1) / CR_PARTS;
  const int k_begin = part * per, k_end = min(chunks, k_begin + per);
  float s = 0.0f;
  if (c < cols) {
    for (int k0 = k_begin; k0 < k_end; k0 += RB_UNROLL) {
      float v[RB_UNROLL];
#pragma unroll
      for (int u = 0; u < RB_UNROLL; ++u) v[u] = k0 + u < k_end ? partial[(size_t)(k0 + u) * cols + c] : 0.0f;
#pragma unroll
      for (int u = 0; u < RB_UNROLL; ++u)
        if (k0 + u < k_end) s = s + v[u];
    }
  }
  q[part][lc] = s;
  __syncthreads();
  if (part == 0 && c < cols) {
    float t = q[0][lc];
#pragma unroll
    for (int p = 1; p < CR_PARTS; ++p) t = t + q[p][lc];
    out[c] = t;
  }
}

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, const AdamWScalars& k) {
  float d = p * k.decay;                // p * (1 - lr*wd)
  float mn = (m * k.b1) + (g * k.omb1); // m*b1 + g*(1-b1)
  float vn = (v * k.b2) + ((g * g) * k.omb2);
  float mh = mn * k.c1;
  float vh = vn * k.c2;
  float den = sqrtf(vh) + k.eps;
  float u = (mh / den) * k.lr;
  p = d - u;
  m = mn;
  v = vn;
}

// One float4 of every array per thread, a flat grid, and non-temporal loads
// and stores: the arrays are streamed once per step, so they bypass cache
// allocation.  (Measured on 2^28 parameters: 6.2 TB/s, against 5.2 TB/s for
// a grid-stride loop with ordinary accesses.)
// p_src holds the parameters read, p receives the updated ones (the same
// buffer for an update in place; each element is read before it is written
// by the same thread).
template <bool DEV>
__global__ void __launch_bounds__(256) adamw_vec_kernel(float4* p, const float4* p_src, const float4* __restrict__ g,
                                                        float4* __restrict__ m, float4* __restrict__ v, size_t n4,
                                                        AdamWScalars ka, const AdamWScalars* __restrict__ kd) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const AdamWScalars k = DEV ? *kd : ka;
  floatx4 pp = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p_src) + i);
  const floatx4 gg = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(g) + i);
  floatx4 mm = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(m) + i);
  floatx4 vv = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(v) + i);
  float pa[4] = {pp.x, pp.y, pp.z, pp.w}, ma[4] = {mm.x, mm.y, mm.z, mm.w}, va[4] = {vv.x, vv.y, vv.z, vv.w};
  const float ga[4] = {gg.x, gg.y, gg.z, gg.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) adamw_elem(pa[j], ga[j], ma[j], va[j], k);
  __builtin_nontemporal_store(floatx4{pa[0], pa[1], pa[2], pa[3]}, reinterpret_cast<floatx4*>(p) + i);
  __builtin_nontemporal_store(floatx4{ma[0], ma[1], ma[2], ma[3]}, reinterpret_cast<floatx4*>(m) + i);
  __builtin_nontemporal_store(floatx4{va[0], va[1], va[2], va[3]}, reinterpret_cast<floatx4*>(v) + i);
}

// Bounded-grid variant for an update that runs beside a GEMM on another
// stream: a few 256-thread blocks per CU, each thread streaming ADAMW_RES_U
// float4 of every array per iteration (all loads issued before the
// arithmetic).  The launch holds few registers per SIMD, so a GEMM launched
// while it runs can still place its blocks; a flat grid of one float4 per
// thread fills every SIMD's register file and delays such a GEMM.
constexpr int ADAMW_RES_U = 4;
template <bool DEV>
__global__ void __launch_bounds__(256) adamw_res_kernel(float4* p, const float4* p_src, const float4* __restrict__ g,
                                                        float4* __restrict__ m, float4* __restrict__ v, size_t n4,
                                                        AdamWScalars ka, const AdamWScalars* __restrict__ kd) {
  const AdamWScalars k = DEV ? *kd : ka;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  auto update4 = [&](floatx4 pp, floatx4 gg, floatx4 mm, floatx4 vv, size_t j) {
    float pa[4] = {pp.x, pp.y, pp.z, pp.w}, ma[4] = {mm.x, mm.y, mm.z, mm.w}, va[4] = {vv.x, vv.y, vv.z, vv.w};
    const float ga[4] = {gg.x, gg.y, gg.z, gg.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) adamw_elem(pa[e], ga[e], ma[e], va[e], k);
    __builtin_nontemporal_store(floatx4{pa[0], pa[1], pa[2], pa[3]}, reinterpret_cast<floatx4*>(p) + j);
    __builtin_nontemporal_store(floatx4{ma[0], ma[1], ma[2], ma[3]}, reinterpret_cast<floatx4*>(m) + j);
    __builtin_nontemporal_store(floatx4{va[0], va[1], va[2], va[3]}, reinterpret_cast<floatx4*>(v) + j);
  };
  auto ld = [](const float4* a, size_t j) { return __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(a) + j); };
  for (; i + (ADAMW_RES_U - 1) * stride < n4; i += ADAMW_RES_U * stride) {
    floatx4 pp[ADAMW_RES_U], gg[ADAMW_RES_U], mm[ADAMW_RES_U], vv[ADAMW_RES_U];
#pragma unroll
    for (int u = 0; u < ADAMW_RES_U; ++u) {
      const size_t j = i + u * stride;
      pp[u] = ld(p_src, j);
      gg[u] = ld(g, j);
      mm[u] = ld(m, j);
      vv[u] = ld(v, j);
    }
#pragma unroll
    for (int u = 0; u < ADAMW_RES_U; ++u) update4(pp[u], gg[u], mm[u], vv[u], i + u * stride);
  }
  for (; i < n4; i += stride) update4(ld(p_src, i), ld(g, i), ld(m, i), ld(v, i), i);
}

template <bool DEV>
__global__ void adamw_scalar_kernel(float* p, const float* p_src, const float* __restrict__ g, float* __restrict__ m,
                                    float* __restrict__ v, size_t begin, size_t n, AdamWScalars ka,
                                    const AdamWScalars* __restrict__ kd) {
  const AdamWScalars k = DEV ? *kd : ka;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = begin + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float pp = p_src[i], mm = m[i], vv = v[i];
    adamw_elem(pp, g[i], mm, vv, k);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
  }
}

__global__ void adamw_store_scalars_kernel(AdamWScalars* dst, AdamWScalars s) { *dst = s; }

// Many parameters in one launch (the optimizer's per-parameter loop,
// python/orca/optim/adamw.py:66-99 and sgd.py:46-79, as one pass): segment i
// covers float4 groups [start4[i], start4[i + 1]) of the launch's index space
// and ceil(n / 4) groups of its own arrays.  A thread finds its segment by
// binary search over the (uniform) table; whole groups of 16-byte-aligned
// segments take float4 accesses, the rest (a segment's last partial group,
// unaligned segments) element by element.  Same per-element arithmetic as the
// one-parameter kernels, so the same bits.
constexpr int kOptSegs = ORCA_HIP_OPT_MAX_SEGMENTS;
struct OptSegs {
  const float* ps[kOptSegs];
  float* pd[kOptSegs];
  const float* g[kOptSegs];
  float* m[kOptSegs];
  float* v[kOptSegs];
  uint64_t n[kOptSegs];
  uint64_t start4[kOptSegs + 1];
  uint32_t vec_mask;  // bit i: segment i's arrays are all 16-byte aligned
  int count;
};

__device__ __forceinline__ int opt_segment(const OptSegs& s, uint64_t q) {
  int lo = 0, hi = s.count - 1;  // the last i with start4[i] <= q
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s.start4[mid] <= q) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <bool ADAMW>
__device__ __forceinline__ void opt_multi_group(const OptSegs& s, const AdamWScalars& k, float lr, uint64_t q) {
  const int i = opt_segment(s, q);
  const uint64_t e0 = 4 * (q - s.start4[i]);
  const uint64_t n = s.n[i];
  if (((s.vec_mask >> i) & 1) && e0 + 4 <= n) {
    const uint64_t j = e0 / 4;
    const floatx4 pp = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(s.ps[i]) + j);
    const floatx4 gg = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(s.g[i]) + j);
    if (ADAMW) {
      const floatx4 mm = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(s.m[i]) + j);
      const floatx4 vv = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(s.v[i]) + j);
      float pa[4] = {pp.x, pp.y, pp.z, pp.w}, ma[4] = {mm.x, mm.y, mm.z, mm.w}, va[4] = {vv.x, vv.y, vv.z, vv.w};
      const float ga[4] = {gg.x, gg.y, gg.z, gg.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) adamw_elem(pa[u], ga[u], ma[u], va[u], k);
      __builtin_nontemporal_store(floatx4{pa[0], pa[1], pa[2], pa[3]}, reinterpret_cast<floatx4*>(s.pd[i]) + j);
      __builtin_nontemporal_store(floatx4{ma[0], ma[1], ma[2], ma[3]}, reinterpret_cast<floatx4*>(s.m[i]) + j);
      __builtin_nontemporal_store(floatx4{va[0], va[1], va[2], va[3]}, reinterpret_cast<floatx4*>(s.v[i]) + j);
    } else {
      floatx4 r;
      r.x = pp.x - gg.x * lr;
      r.y = pp.y - gg.y * lr;
      r.z = pp.z - gg.z * lr;
      r.w = pp.w - gg.w * lr;
      __builtin_nontemporal_store(r, reinterpret_cast<floatx4*>(s.pd[i]) + j);
    }
    return;
  }
  for (uint64_t e = e0; e < e0 + 4 && e < n; ++e) {
    if (ADAMW) {
      float pp = s.ps[i][e], mm = s.m[i][e], vv = s.v[i][e];
      adamw_elem(pp, s.g[i][e], mm, vv, k);
      s.pd[i][e] = pp;
      s.m[i][e] = mm;
      s.v[i][e] = vv;
    } else {
      s.pd[i][e] = s.ps[i][e] - s.g[i][e] * lr;
    }
  }
}

// One float4 group per thread on the full grid; a bounded grid (a pass beside
// other work) strides over the groups.
template <bool ADAMW>
__global__ void __launch_bounds__(256) opt_multi_kernel(OptSegs s, AdamWScalars k, float lr) {
  const uint64_t total = s.start4[s.count], stride = (uint64_t)gridDim.x * 256;
  for (uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x; q < total; q += stride) opt_multi_group<ADAMW>(s, k, lr, q);
}

__global__ void __launch_bounds__(256) sgd_vec_kernel(float4* __restrict__ p, const float4* __restrict__ g, size_t n4, float lr) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const floatx4 pp = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p) + i);
  const floatx4 gg = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(g) + i);
  floatx4 r;
  r.x = pp.x - gg.x * lr;
  r.y = pp.y - gg.y * lr;
  r.z = pp.z - gg.z * lr;
  r.w = pp.w - gg.w * lr;
  __builtin_nontemporal_store(r, reinterpret_cast<floatx4*>(p) + i);
}

__global__ void sgd_scalar_kernel(float* __restrict__ p, const float* __restrict__ g, size_t begin, size_t n, float lr) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = begin + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = p[i] - g[i] * lr;
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

void softmax_ce(orca_hip_ctx* ctx, const float* logits, size_t B, size_t C, const float* onehot, const int32_t* labels,
                float* loss, float* dlogits, int32_t* preds, int64_t* correct, float* ws_row_loss,
                int* ws_row_correct) {
  if ((onehot == nullptr) == (labels == nullptr))
    fail(ORCA_HIP_ERR_INTERNAL, "softmax_ce needs exactly one of one-hot targets or labels");
  if (B == 0 || C == 0) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during softmax_ce: empty logits");
  if (C > 4096) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during softmax_ce: expected at most 4096 classes, got " + std::to_string(C));
  if (B > (size_t)INT32_MAX) fail(ORCA_HIP_ERR_SHAPE, "softmax_ce: too many rows");
  Scratch row_loss_s(ctx, ws_row_loss ? 0 : sizeof(float) * B);
  Scratch row_correct_s(ctx, ws_row_correct ? 0 : sizeof(int) * B);
  float* row_loss = ws_row_loss ? ws_row_loss : row_loss_s.as<float>();
  int* row_correct = ws_row_correct ? ws_row_correct : row_correct_s.as<int>();
  const float inv_b = 1.0f / (float)B;
  const int rows_per_block = 4;
  dim3 grid((unsigned)((B + rows_per_block - 1) / rows_per_block));
  int* rc = correct ? row_correct : nullptr;
  {
    ProfScope ps(ctx, "softmax_ce", 0.0, 4.0 * (double)B * C * (dlogits ? 2 : 1) + 4.0 * B);
#define CE_LAUNCH(VPL, VEC, FULL)                                                                           \
  do {                                                                                                      \
    if (labels)                                                                                             \
      hipLaunchKernelGGL((softmax_ce_kernel<VPL, VEC, FULL, true>), grid, dim3(256), 0, ctx->stream, logits, \
                         (int)B, (int)C, onehot, labels, inv_b, row_loss, dlogits, preds, rc);                 \
    else                                                                                                    \
      hipLaunchKernelGGL((softmax_ce_kernel<VPL, VEC, FULL, false>), grid, dim3(256), 0, ctx->stream, logits, \
                         (int)B, (int)C, onehot, labels, inv_b, row_loss, dlogits, preds, rc);                 \
  } while (0)
    const bool vec = C % 4 == 0 && aligned16(logits) && (!dlogits || aligned16(dlogits));
    if (C <= 64) {
      if (C == 64) CE_LAUNCH(1, false, true);
      else CE_LAUNCH(1, false, false);
    } else if (C <= 256) {
      if (vec) CE_LAUNCH(4, true, false);
      else CE_LAUNCH(4, false, false);
    } else if (C <= 1024) {
      if (vec) CE_LAUNCH(16, true, false);
      else CE_LAUNCH(16, false, false);
    } else {
#define CE_BLOCK_LAUNCH(VEC, FULL)                                                                            \
  do {                                                                                                        \
    if (labels)                                                                                               \
      hipLaunchKernelGGL((softmax_ce_block_kernel<VEC, FULL, true>), dim3((unsigned)B), dim3(256), 0, ctx->stream, \
                         logits, (int)B, (int)C, onehot, labels, inv_b, row_loss, dlogits, preds, rc);           \
    else                                                                                                      \
      hipLaunchKernelGGL((softmax_ce_block_kernel<VEC, FULL, false>), dim3((unsigned)B), dim3(256), 0, ctx->stream, \
                         logits, (int)B, (int)C, onehot, labels, inv_b, row_loss, dlogits, preds, rc);           \
  } while (0)
      if (vec && C == 4096) CE_BLOCK_LAUNCH(true, true);
      else if (vec) CE_BLOCK_LAUNCH(true, false);
      else CE_BLOCK_LAUNCH(false, false);
#undef CE_BLOCK_LAUNCH
    }
#undef CE_LAUNCH
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (loss || correct) {
    hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(1024), 0, ctx->stream, row_loss, rc, (int)B,
                       inv_b, loss, correct);
    ORCA_HIP_CHECK(hipGetLastError());
  }
}

AdamWScalars adamw_scalars(double lr, double b1, double b2, double eps, double wd, int64_t t) {
  if (t < 1) fail(ORCA_HIP_ERR_INTERNAL, "adamw step count must be >= 1");
  AdamWScalars k;
  k.decay = (float)(1.0 - lr * wd);
  k.b1 = (float)b1;
  k.omb1 = (float)(1.0 - b1);
  k.b2 = (float)b2;
  k.omb2 = (float)(1.0 - b2);
  k.c1 = (float)(1.0 / (1.0 - std::pow(b1, (double)t)));
  k.c2 = (float)(1.0 / (1.0 - std::pow(b2, (double)t)));
  k.eps = (float)eps;
  k.lr = (float)lr;
  return k;
}

void adamw_store_scalars(orca_hip_ctx* ctx, AdamWScalars* dst, const AdamWScalars& s, hipStream_t stream) {
  hipLaunchKernelGGL(adamw_store_scalars_kernel, dim3(1), dim3(1), 0, stream ? stream : ctx->stream, dst, s);
  ORCA_HIP_CHECK(hipGetLastError());
}

void adamw(orca_hip_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, double lr, double b1, double b2,
           double eps, double wd, int64_t t, hipStream_t stream, const AdamWScalars* dev_scalars, const float* p_src,
           int blocks_per_cu) {
  if (!stream) stream = ctx->stream;
  if (n == 0) return;
  if (!p_src) p_src = p;
  const AdamWScalars k = dev_scalars ? AdamWScalars{} : adamw_scalars(lr, b1, b2, eps, wd, t);
  // Launches on another stream than the context's run beside other work: their
  // device time is reported under a name of its own.
  ProfScope ps(ctx, stream == ctx->stream ? "adamw" : "adamw_overlapped", 0.0, 28.0 * (double)n, stream);
  size_t done = 0;
  if (aligned16(p) && aligned16(p_src) && aligned16(g) && aligned16(m) && aligned16(v)) {
    size_t n4 = n / 4;
    if (n4) {
      const size_t gsz = (n4 + 255) / 256;
      if (gsz > 0x7fffffffu) fail(ORCA_HIP_ERR_INTERNAL, "adamw: buffer too large for one launch");
      auto* p4 = reinterpret_cast<float4*>(p);
      auto* g4 = reinterpret_cast<const float4*>(g);
      auto* m4 = reinterpret_cast<float4*>(m);
      auto* v4 = reinterpret_cast<float4*>(v);
      auto* s4 = reinterpret_cast<const float4*>(p_src);
      if (blocks_per_cu > 0) {
        const size_t rg = std::min(gsz, (size_t)ctx->num_cus * (size_t)blocks_per_cu);
        if (dev_scalars)
          hipLaunchKernelGGL(adamw_res_kernel<true>, dim3((unsigned)rg), dim3(256), 0, stream, p4, s4, g4, m4, v4, n4,
                             k, dev_scalars);
        else
          hipLaunchKernelGGL(adamw_res_kernel<false>, dim3((unsigned)rg), dim3(256), 0, stream, p4, s4, g4, m4, v4,
                             n4, k, dev_scalars);
      } else if (dev_scalars)
        hipLaunchKernelGGL(adamw_vec_kernel<true>, dim3((unsigned)gsz), dim3(256), 0, stream, p4, s4, g4, m4, v4, n4,
                           k, dev_scalars);
      else
        hipLaunchKernelGGL(adamw_vec_kernel<false>, dim3((unsigned)gsz), dim3(256), 0, stream, p4, s4, g4, m4, v4,
                           n4, k, dev_scalars);
    }
    done = 4 * n4;
  }
  if (done < n) {
    unsigned gsz = grid_for(n - done, 256, ctx->num_cus * 8);
    if (dev_scalars)
      hipLaunchKernelGGL(adamw_scalar_kernel<true>, dim3(gsz), dim3(256), 0, stream, p, p_src, g, m, v, done, n, k,
                         dev_scalars);
    else
      hipLaunchKernelGGL(adamw_scalar_kernel<false>, dim3(gsz), dim3(256), 0, stream, p, p_src, g, m, v, done, n, k,
                         dev_scalars);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

// One launch per kOptSegs segments; each segment's arrays are checked against
// the allocations they point into.
void opt_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, bool adamw_, const AdamWScalars& k,
               float lr) {
  if (n_segs && !segs) fail(ORCA_HIP_ERR_INTERNAL, "optimizer: null segment table");
  for (size_t b = 0; b < n_segs; b += kOptSegs) {
    OptSegs t{};
    uint64_t total4 = 0;
    double bytes = 0.0;
    for (size_t i = b; i < n_segs && t.count < kOptSegs; ++i) {
      const orca_hip_opt_segment& sg = segs[i];
      const size_t nb = sg.n * sizeof(float);
      check_extent(ctx, sg.p_src, nb, "optimizer (p_src)");
      check_extent(ctx, sg.p_dst, nb, "optimizer (p_dst)");
      check_extent(ctx, sg.g, nb, "optimizer (g)");
      if (adamw_) {
        check_extent(ctx, sg.m, nb, "optimizer (m)");
        check_extent(ctx, sg.v, nb, "optimizer (v)");
      }
      if (sg.n && (!sg.p_src || !sg.p_dst || !sg.g || (adamw_ && (!sg.m || !sg.v))))
        fail(ORCA_HIP_ERR_INTERNAL, "optimizer: null array in segment " + std::to_string(i));
      const int c = t.count++;
      t.ps[c] = sg.p_src;
      t.pd[c] = sg.p_dst;
      t.g[c] = sg.g;
      t.m[c] = sg.m;
      t.v[c] = sg.v;
      t.n[c] = sg.n;
      t.start4[c] = total4;
      total4 += (sg.n + 3) / 4;
      const bool vec = aligned16(sg.p_src) && aligned16(sg.p_dst) && aligned16(sg.g) &&
                       (!adamw_ || (aligned16(sg.m) && aligned16(sg.v)));
      if (vec) t.vec_mask |= 1u << c;
      bytes += (adamw_ ? 28.0 : 12.0) * (double)sg.n;
    }
    t.start4[t.count] = total4;
    if (total4 == 0) continue;
    // On the side stream the pass may run beside a product that fills the CUs: a
    // bounded grid leaves it room to launch its own blocks.
    const uint64_t full = (total4 + 255) / 256;
    const uint64_t blocks =
        ctx->main && ctx->side_bpc > 0 ? std::min<uint64_t>(full, (uint64_t)ctx->side_bpc * ctx->num_cus) : full;
    if (blocks > 0x7fffffffu) fail(ORCA_HIP_ERR_INTERNAL, "optimizer: too many parameters for one launch");
    ProfScope ps(ctx, ctx->main ? (adamw_ ? "adamw_multi_overlapped" : "sgd_multi_overlapped")
                                : (adamw_ ? "adamw_multi" : "sgd_multi"),
                 0.0, bytes);
    if (adamw_)
      hipLaunchKernelGGL(opt_multi_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, t, k, lr);
    else
      hipLaunchKernelGGL(opt_multi_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, t, k, lr);
    ORCA_HIP_CHECK(hipGetLastError());
  }
}

void sgd(orca_hip_ctx* ctx, float* p, const float* g, size_t n, double lr, hipStream_t stream) {
  if (!stream) stream = ctx->stream;
  if (n == 0) return;
  const float flr = (float)lr;
  ProfScope ps(ctx, stream == ctx->stream ? "sgd" : "sgd_overlapped", 0.0, 12.0 * (double)n, stream);
  size_t done = 0;
  if (aligned16(p) && aligned16(g)) {
    size_t n4 = n / 4;
    if (n4) {
      const size_t gsz = (n4 + 255) / 256;
      if (gsz > 0x7fffffffu) fail(ORCA_HIP_ERR_INTERNAL, "sgd: buffer too large for one launch");
      hipLaunchKernelGGL(sgd_vec_kernel, dim3((unsigned)gsz), dim3(256), 0, stream, reinterpret_cast<float4*>(p),
                         reinterpret_cast<const float4*>(g), n4, flr);
    }
    done = 4 * n4;
  }
  if (done < n) {
    unsigned gsz = grid_for(n - done, 256, ctx->num_cus * 8);
    hipLaunchKernelGGL(sgd_scalar_kernel, dim3(gsz), dim3(256), 0, stream, p, g, done, n, flr);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

// ReLU-backward + bias column sum, shared by the allocating and the
// allocation-free entry points.
void relu_bw_colsum_check(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                          const float* dpre, const float* colsum);
size_t relu_bw_colsum_partial_floats(size_t rows, size_t cols, bool colsum);
void relu_bw_colsum_launch(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                           float* dpre, float* colsum, float* part);

// One GPU's copy of `scratch`: its device address (hipGetSymbolAddress) and an event that
// marks the work of the last call that used it, on whichever stream that call ran.  Both are
// set up once per device (which the caller has made current) and kept for the life of the
// process; `mu` orders the calls' bookkeeping on the host.
struct StaticScratch {
  float* ptr = nullptr;
  hipEvent_t last_use = nullptr;
  bool used = false;
  std::mutex mu;
};

StaticScratch& static_scratch(int device) {
  static std::mutex mu;
  static std::map<int, StaticScratch> by_device;
  std::lock_guard<std::mutex> lk(mu);
  auto it = by_device.find(device);
  if (it != by_device.end() && it->second.ptr) return it->second;
  StaticScratch& s = by_device[device];
  float* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    fail(ORCA_HIP_ERR_INTERNAL, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
  ORCA_HIP_CHECK(hipEventCreateWithFlags(&s.last_use, hipEventDisableTiming));
  s.ptr = ptr;
  return s;
}

}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_softmax_ce(orca_hip_ctx* ctx, const float* logits, size_t B, size_t C, const float* onehot,
                        const int32_t* labels, float* loss, float* dlogits, int32_t* preds, int64_t* correct) {
  return guard([&] {
    bind(ctx);
    check_extent(ctx, logits, B * C * sizeof(float), "softmax_ce (logits)");
    check_extent(ctx, onehot, B * C * sizeof(float), "softmax_ce (onehot)");
    check_extent(ctx, labels, B * sizeof(int32_t), "softmax_ce (labels)");
    check_extent(ctx, dlogits, B * C * sizeof(float), "softmax_ce (dlogits)");
    check_extent(ctx, preds, B * sizeof(int32_t), "softmax_ce (preds)");
    check_extent(ctx, loss, sizeof(float), "softmax_ce (loss)");
    check_extent(ctx, correct, sizeof(int64_t), "softmax_ce (correct)");
    softmax_ce(ctx, logits, B, C, onehot, labels, loss, dlogits, preds, correct);
  });
}

int orca_hip_relu_bw_colsum(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                            float* dpre, float* colsum) {
  return guard([&] {
    bind(ctx);
    relu_bw_colsum_check(ctx, grad, pre, rows, cols, dpre, colsum);
    const size_t need = relu_bw_colsum_partial_floats(rows, cols, colsum != nullptr);
    std::unique_ptr<Scratch> partial;
    if (need) partial.reset(new Scratch(ctx, sizeof(float) * need));
    relu_bw_colsum_launch(ctx, grad, pre, rows, cols, dpre, colsum, need ? partial->as<float>() : nullptr);
  });
}

int orca_hip_relu_bw_colsum_noalloc(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows,
                                    size_t cols, float* dpre, float* colsum) {
  return guard([&] {
    bind(ctx);
    const size_t need = relu_bw_colsum_partial_floats(rows, cols, colsum != nullptr);
    if (need > kStaticScratchFloats)
      fail(ORCA_HIP_ERR_INTERNAL, "relu_bw_colsum_noalloc: ceil(rows / 64) * cols = " + std::to_string(need) +
                                      " column-sum partials exceed the fixed device scratch of " +
                                      std::to_string(kStaticScratchFloats) + " floats");
    relu_bw_colsum_check(ctx, grad, pre, rows, cols, dpre, colsum);
    if (!need) {  // no column sum: the scratch is not touched
      relu_bw_colsum_launch(ctx, grad, pre, rows, cols, dpre, colsum, nullptr);
      return;
    }
    // The GPU's one scratch is shared by every context and stream on it: this call's stream
    // first waits (on the device) for the last call that used it, and this call's work is
    // then the one the next call waits for.  The kernels overwrite every partial they later
    // read, so nothing has to start at zero.
    StaticScratch& s = static_scratch(ctx->device);
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.used) ORCA_HIP_CHECK(hipStreamWaitEvent(ctx->stream, s.last_use, 0));
    relu_bw_colsum_launch(ctx, grad, pre, rows, cols, dpre, colsum, s.ptr);
    ORCA_HIP_CHECK(hipEventRecord(s.last_use, ctx->stream));
    s.used = true;
  });
}

}  // extern "C"

namespace orca_hip {

void relu_bw_colsum_check(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                          const float* dpre, const float* colsum) {
  check_extent(ctx, grad, rows * cols * sizeof(float), "relu_bw_colsum (grad)");
  check_extent(ctx, pre, rows * cols * sizeof(float), "relu_bw_colsum (pre)");
  check_extent(ctx, dpre, rows * cols * sizeof(float), "relu_bw_colsum (dpre)");
  check_extent(ctx, colsum, cols * sizeof(float), "relu_bw_colsum (colsum)");
  if ((rows * cols != 0) && (!grad || !pre || !dpre))
    fail(ORCA_HIP_ERR_INTERNAL, "relu_bw_colsum: null grad, pre-activation or output");
  if ((rows + kRowsPerChunk - 1) / kRowsPerChunk > 65535) fail(ORCA_HIP_ERR_INTERNAL, "relu_bw_colsum: too many rows");
}

size_t relu_bw_colsum_partial_floats(size_t rows, size_t cols, bool colsum) {
  if (!colsum || rows == 0 || cols == 0) return 0;
  return (rows + kRowsPerChunk - 1) / kRowsPerChunk * cols;
}

// dpre (and colsum when non-null) on the context stream; `part` holds the
// per-chunk column partials (relu_bw_colsum_partial_floats of them).
void relu_bw_colsum_launch(orca_hip_ctx* ctx, const float* grad, const float* pre, size_t rows, size_t cols,
                           float* dpre, float* colsum, float* part) {
    if (rows == 0 || cols == 0) {
      if (colsum) launch_fill(ctx, colsum, 0.0f, cols);
      return;
    }
    const int rows_per_chunk = kRowsPerChunk;
    const size_t chunks = (rows + rows_per_chunk - 1) / rows_per_chunk;
    {
      ProfScope ps(ctx, "relu_bw_colsum", 0.0, 12.0 * (double)rows * cols + (colsum ? 4.0 * cols : 0.0));
      if (cols % 4 == 0 && aligned16(grad) && aligned16(pre) && aligned16(dpre)) {
        size_t cols4 = cols / 4;
        dim3 grid((unsigned)((cols4 + 255) / 256), (unsigned)chunks);
        hipLaunchKernelGGL(relu_bw_colsum_vec_kernel, grid, dim3(256), 0, ctx->stream,
                           reinterpret_cast<const float4*>(grad), reinterpret_cast<const float4*>(pre), rows, cols4,
                           rows_per_chunk, reinterpret_cast<float4*>(dpre), reinterpret_cast<float4*>(part));
      } else {
        dim3 grid((unsigned)((cols + 255) / 256), (unsigned)chunks);
        hipLaunchKernelGGL(relu_bw_colsum_scalar_kernel, grid, dim3(256), 0, ctx->stream, grad, pre, rows, cols,
                           rows_per_chunk, dpre, part);
      }
      ORCA_HIP_CHECK(hipGetLastError());
    }
    if (colsum) {
      ProfScope ps(ctx, "colsum_chunks", 0.0, 4.0 * (double)chunks * cols + 4.0 * cols);
      hipLaunchKernelGGL(chunk_reduce_kernel, dim3((unsigned)((cols + CR_PARTS_COLS - 1) / CR_PARTS_COLS)), dim3(256),
                         0, ctx->stream, part, (int)chunks, cols, colsum);
      ORCA_HIP_CHECK(hipGetLastError());
    }
}

}  // namespace orca_hip

extern "C" {

int orca_hip_adamw_step(orca_hip_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, double lr,
                        double beta1, double beta2, double eps, double weight_decay, int64_t t) {
  return guard([&] {
    bind(ctx);
    for (const void* a : {(const void*)p, (const void*)g, (const void*)m, (const void*)v})
      check_extent(ctx, a, n * sizeof(float), "adamw_step");
    adamw(ctx, p, g, m, v, n, lr, beta1, beta2, eps, weight_decay, t);
  });
}

int orca_hip_sgd_step(orca_hip_ctx* ctx, float* p, const float* g, size_t n, double lr) {
  return guard([&] {
    bind(ctx);
    check_extent(ctx, p, n * sizeof(float), "sgd_step");
    check_extent(ctx, g, n * sizeof(float), "sgd_step");
    sgd(ctx, p, g, n, lr);
  });
}

int orca_hip_adamw_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr, double beta1,
                         double beta2, double eps, double weight_decay, int64_t t) {
  return guard([&] {
    bind(ctx);
    opt_multi(ctx, segs, n_segs, true, adamw_scalars(lr, beta1, beta2, eps, weight_decay, t), 0.0f);
  });
}

int orca_hip_sgd_multi(orca_hip_ctx* ctx, const orca_hip_opt_segment* segs, size_t n_segs, double lr) {
  return guard([&] {
    bind(ctx);
    opt_multi(ctx, segs, n_segs, false, AdamWScalars{}, (float)lr);
  });
}

}  // extern "C"
