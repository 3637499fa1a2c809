// Fused classifier head: the last nn.Linear of an MLP when it has few
// outputs (C <= 16 classes), together with the softmax cross-entropy.
//
// With C this small the layer's three products are not GEMM-shaped: every
// one of them streams the [B, K] activation H once and does C multiply-adds
// per element of it, so they are HBM-bound.  Two kernels cover the layer:
//
//   head_forward_kernel   logits = H W + b (python/orca/nn/linear.py:77-86),
//                         then per row the loss term, dL/dlogits and the
//                         argmax of the composed CrossEntropyLoss
//                         (python/orca/nn/loss.py:59-100); the block that
//                         finishes last adds the row terms into the mean loss
//                         and the correct-prediction count.
//   head_backward_kernel  dW = H^T dlogits, db = colsum(dlogits) and
//                         dH = (dlogits W^T) * [H > 0] (MatMulBackward,
//                         ExpandBackward's sum_to_shape and ReluBackward,
//                         orca-autograd/src/backend.rs:1449-1499, 1684-1697,
//                         1624-1646), reading H once.
//
// Both are deterministic: every sum runs in a fixed order.  The mean loss
// needs every row's term, so it is added up after the forward kernel: by
// block 0 of the backward kernel in a training step, or by a one-block
// kernel when the forward runs alone.
#include <cstdint>

#include "ce_row.hpp"
#include "runtime.hpp"

namespace orca_hip {
namespace {

constexpr int HEAD_THREADS = 256;  // 4 waves
constexpr int HEAD_PANEL = 16;     // columns of H per backward block
constexpr int BWD_UNROLL = 4;      // rows per thread whose loads are in flight together

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Rows per forward block (one wave per row in the loss phase): 4, or 2 for
// C > 10 so that the accumulators and W's slice stay in registers.
template <int C>
constexpr int fwd_rows() {
  return C <= 10 ? 4 : 2;
}
// Float4 column groups of H per forward W chunk: the chunk's 4 x groups rows
// of W (groups x C float4s) are staged in LDS, at most 40 KiB.
template <int C>
constexpr int fwd_chunk_groups() {
  return C <= 10 ? 256 : 128;
}
template <int C>
constexpr int fwd_smem_floats() {
  return fwd_chunk_groups<C>() * 4 * C > fwd_rows<C>() * C * HEAD_THREADS ? fwd_chunk_groups<C>() * 4 * C
                                                                            : fwd_rows<C>() * C * HEAD_THREADS;
}

// Blocks are handed to the 8 XCDs round-robin; with nb a multiple of 8 this
// gives XCD x the consecutive work items x * nb/8 ... so neighbours that
// share cache lines share an L2.  (A performance mapping only: any bijection
// is correct.)
__device__ __forceinline__ int xcd_local_index(int b, int nb) {
  return (nb & 7) ? b : (b & 7) * (nb >> 3) + (b >> 3);
}

// Sum of n_out columns of a [n_out][256] LDS array, one output per 4 threads:
// thread t < 4 n_out adds the 64 values of quarter t % 4 of row t / 4 in
// index order, then the 4 quarters combine as (q0 + q1) + (q2 + q3).  Every
// thread of the block must call it; the result is valid on threads with
// t % 4 == 0.
__device__ __forceinline__ float sum_rows_256(const float* red, int n_out) {
  const int t = threadIdx.x;
  float v = 0.0f;
  if (t < 4 * n_out) {
    const floatx4* src = reinterpret_cast<const floatx4*>(red + (t >> 2) * HEAD_THREADS + (t & 3) * 64);
    floatx4 a[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = src[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) v = (((v + a[i].x) + a[i].y) + a[i].z) + a[i].w;
  }
  v = v + __shfl_xor(v, 1, 64);
  v = v + __shfl_xor(v, 2, 64);
  return v;
}

// loss = (sum of row terms) * (1/B) and the correct-row count, by one block.
__device__ void finish_rows(const float* __restrict__ row_loss, const int* __restrict__ row_correct, int B, float inv_b,
                            float* loss, int64_t* correct, float* red_f, int* red_i) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int per = (B + HEAD_THREADS - 1) / HEAD_THREADS;
  float s = 0.0f;
  int n = 0;
  for (int k = 0; k < per; ++k) {
    const int r = tid * per + k;
    if (r < B) {
      s = s + row_loss[r];
      n += row_correct[r];
    }
  }
  s = wave_sum(s);
  n = wave_sum_i(n);
  if (lane == 0) {
    red_f[wave] = s;
    red_i[wave] = n;
  }
  __syncthreads();
  if (tid == 0) {
    float t = red_f[0];
    int64_t c = red_i[0];
    for (int w = 1; w < HEAD_THREADS / 64; ++w) {
      t = t + red_f[w];
      c += red_i[w];
    }
    if (loss) *loss = t * inv_b;
    if (correct) *correct = c;
  }
}

struct HeadFwdParams {
  const float* H;  // [B][K]
  const float* W;  // [K][C]
  const float* bias;
  const float* onehot;    // [B][C] or null
  const int32_t* labels;  // [B] or null
  float* logits;          // [B][C]
  float* dlogits;         // [B][C] or null
  int32_t* preds;         // [B] or null
  float* row_loss;        // [B]
  int* row_correct;       // [B]
  int B, K;
  float inv_b;
};

// Block = fwd_rows<C>() rows x all of K.  K is walked in chunks of G float4
// column groups; chunk i+1's H and W are loaded into registers while chunk i
// is multiplied out.  The chunk's rows of W go through LDS (coalesced float4
// loads in, a 4C-float slice per thread out); thread t multiplies column
// group t of the chunk for every row.  The 256 partial sums of each logit
// are added up by sum_rows_256 (fixed order); the bias is added after the
// product, as a separate f32 operation.
template <int C>
__global__ void __launch_bounds__(HEAD_THREADS) head_forward_kernel(HeadFwdParams p) {
  constexpr int R = fwd_rows<C>(), G = fwd_chunk_groups<C>();
  constexpr int WPT = (G * C + HEAD_THREADS - 1) / HEAD_THREADS;  // staged float4s per thread
  __shared__ __attribute__((aligned(16))) float smem[fwd_smem_floats<C>()];
  __shared__ float logit[R * C];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * R;
  const int nrows = min(R, p.B - r0);
  const int K4 = p.K >> 2;
  const int nchunks = (K4 + G - 1) / G;

  float acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = 0.0f;

  floatx4 hn[R], wn[WPT];
  auto load_chunk = [&](int ch) {
    const int g0 = ch * G, ng = min(G, K4 - g0);
#pragma unroll
    for (int r = 0; r < R; ++r)
      hn[r] = (tid < ng && r < nrows)
                  ? *reinterpret_cast<const floatx4*>(p.H + (int64_t)(r0 + r) * p.K + 4 * (g0 + tid))
                  : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const floatx4* src = reinterpret_cast<const floatx4*>(p.W + (int64_t)g0 * 4 * C);
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      const int i = tid + HEAD_THREADS * j;
      wn[j] = i < ng * C ? src[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  // Blocks start at different chunks so they do not all read the same rows
  // of W from L2 at the same moment.
  const int rot = blockIdx.x % nchunks;
  load_chunk(rot);
  for (int i = 0; i < nchunks; ++i) {
    const int ch = (i + rot) % nchunks;
    const int ng = min(G, K4 - ch * G);
    __syncthreads();  // the previous chunk's W slices have been read
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      const int i = tid + HEAD_THREADS * j;
      if (i < G * C) reinterpret_cast<floatx4*>(smem)[i] = wn[j];
    }
    floatx4 h[R];
#pragma unroll
    for (int r = 0; r < R; ++r) h[r] = hn[r];
    __syncthreads();
    if (i + 1 < nchunks) load_chunk((ch + 1) % nchunks);
    if (tid < ng) {
      const floatx4* ws = reinterpret_cast<const floatx4*>(smem + tid * 4 * C);
      float w[4 * C];
#pragma unroll
      for (int j = 0; j < C; ++j) {
        const floatx4 v = ws[j];
        w[4 * j] = v.x;
        w[4 * j + 1] = v.y;
        w[4 * j + 2] = v.z;
        w[4 * j + 3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < C; ++c) {
          float a = acc[r][c];
          a = fmaf(h[r].x, w[c], a);
          a = fmaf(h[r].y, w[C + c], a);
          a = fmaf(h[r].z, w[2 * C + c], a);
          a = fmaf(h[r].w, w[3 * C + c], a);
          acc[r][c] = a;
        }
    }
  }

  // Reduce the 256 partial sums of each of the R x C logits.
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) smem[(r * C + c) * HEAD_THREADS + tid] = acc[r][c];
  __syncthreads();
  const float z = sum_rows_256(smem, R * C);
  if ((tid & 3) == 0 && tid < 4 * R * C) logit[tid >> 2] = z;
  __syncthreads();

  // Loss phase: wave w < rows owns row r0 + w; lane c < C holds logit c.
  if (wave < nrows) {
    const int row = r0 + wave;
    float x[1];
    x[0] = 0.0f;
    if (lane < C) {
      x[0] = logit[wave * C + lane] + p.bias[lane];
      p.logits[(int64_t)row * C + lane] = x[0];
    }
    const float* tr = p.onehot ? p.onehot + (int64_t)row * C : nullptr;
    const int label = p.labels ? p.labels[row] : -1;
    auto tval = [&](int j) -> float {
      const int c = lane + 64 * j;
      if (c >= C) return 0.0f;
      return tr ? tr[c] : (c == label ? 1.0f : 0.0f);
    };
    float* dr = p.dlogits ? p.dlogits + (int64_t)row * C : nullptr;
    const CeRowOut o = ce_row<1>(
        x, [&](int) { return lane < C; }, tval, [&](int j) { return lane + 64 * j; }, p.labels != nullptr, label,
        p.inv_b, dr != nullptr, [&](int, float v) { dr[lane] = v; }, true);
    if (lane == 0) {
      p.row_loss[row] = o.loss;
      p.row_correct[row] = o.pred == o.target ? 1 : 0;
      if (p.preds) p.preds[row] = o.pred;
    }
  }
}

struct HeadFinish {
  const float* row_loss;
  const int* row_correct;
  float* loss;       // or null
  int64_t* correct;  // or null
  float inv_b;
};

__global__ void __launch_bounds__(HEAD_THREADS) head_finish_kernel(HeadFinish f, int B) {
  __shared__ float red_f[HEAD_THREADS / 64];
  __shared__ int red_i[HEAD_THREADS / 64];
  finish_rows(f.row_loss, f.row_correct, B, f.inv_b, f.loss, f.correct, red_f, red_i);
}

struct HeadBwdParams {
  const float* H;   // [B][K] (ReLU output of the layer below: also the mask)
  const float* W;   // [K][C]
  const float* dl;  // [B][C] dL/dlogits
  float* dH;        // [B][K] or null
  float* dW;        // [K][C]
  float* db;        // [C] or null
  HeadFinish fin;   // block 0 also finishes the forward's loss when fin.loss or fin.correct is set
  int B, K;
  int mask;
};

// C floats of row `row` of dl, with the widest loads the row alignment allows.
template <int C>
__device__ __forceinline__ void load_dl_row(const float* __restrict__ dl, int row, float (&d)[C]) {
  const float* r = dl + (int64_t)row * C;
  if constexpr (C % 4 == 0) {
#pragma unroll
    for (int j = 0; j < C / 4; ++j) {
      const floatx4 v = reinterpret_cast<const floatx4*>(r)[j];
      d[4 * j] = v.x;
      d[4 * j + 1] = v.y;
      d[4 * j + 2] = v.z;
      d[4 * j + 3] = v.w;
    }
  } else if constexpr (C % 2 == 0) {
#pragma unroll
    for (int j = 0; j < C / 2; ++j) {
      const floatx2 v = reinterpret_cast<const floatx2*>(r)[j];
      d[2 * j] = v.x;
      d[2 * j + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) d[c] = r[c];
  }
}

// Block = 16 columns of H (a panel) x all B rows, so no block depends on
// another.  Thread t owns the float4 column group q = t % 4 of the panel and
// rows t / 4, + 64, ...; it keeps W's 4 x C slice for its columns and
// accumulates 4 x C products of dW, loading BWD_UNROLL rows at a time before
// using any of them.  The 64 row-lane partials of each dW entry are added by
// sum_rows_256 (fixed order).  Adjacent panels share 128-byte lines of H and
// dH, so they run on one XCD.
template <int C>
__global__ void __launch_bounds__(HEAD_THREADS) head_backward_kernel(HeadBwdParams p) {
  constexpr int ROW_LANES = HEAD_THREADS / 4;
  constexpr int PASS = C <= 10 ? 4 * C : 2 * C;  // dW values per thread reduced per LDS pass
  __shared__ __attribute__((aligned(16))) float red[PASS * HEAD_THREADS];
  __shared__ float red_f[HEAD_THREADS / 64];
  __shared__ int red_i[HEAD_THREADS / 64];
  const int tid = threadIdx.x;
  const int q = tid & 3, rl = tid >> 2;
  const int panel = xcd_local_index(blockIdx.x, gridDim.x);
  const int k0 = panel * HEAD_PANEL;
  const int k = k0 + 4 * q;
  const bool kin = k < p.K;
  const bool do_db = p.db != nullptr && panel == 0;

  float w[4 * C];
  if (kin) {
    const floatx4* wp = reinterpret_cast<const floatx4*>(p.W + (int64_t)k * C);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const floatx4 v = wp[j];
      w[4 * j] = v.x;
      w[4 * j + 1] = v.y;
      w[4 * j + 2] = v.z;
      w[4 * j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4 * C; ++j) w[j] = 0.0f;
  }
  float acc[4 * C];
#pragma unroll
  for (int j = 0; j < 4 * C; ++j) acc[j] = 0.0f;
  float adb[C];
#pragma unroll
  for (int c = 0; c < C; ++c) adb[c] = 0.0f;

  // Blocks start at different row groups so they do not all read the same
  // rows of dlogits at the same moment.
  constexpr int GROUP = ROW_LANES * BWD_UNROLL;
  const int ngroups = (p.B + GROUP - 1) / GROUP;
  const int rot = blockIdx.x % ngroups;
  for (int gi = 0; gi < ngroups; ++gi) {
    const int base = ((gi + rot) % ngroups) * GROUP + rl;
    float d[BWD_UNROLL][C];
    floatx4 h[BWD_UNROLL];
#pragma unroll
    for (int u = 0; u < BWD_UNROLL; ++u) {
      const int row = base + u * ROW_LANES;
      if (row < p.B) {
        load_dl_row<C>(p.dl, row, d[u]);
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c) d[u][c] = 0.0f;
      }
      h[u] = row < p.B && kin ? *reinterpret_cast<const floatx4*>(p.H + (int64_t)row * p.K + k)
                              : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < BWD_UNROLL; ++u) {
      const int row = base + u * ROW_LANES;
      if (row >= p.B) break;
      const float hv[4] = {h[u].x, h[u].y, h[u].z, h[u].w};
      if (kin && p.dH) {
        float dz[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float s = d[u][0] * w[e * C];
#pragma unroll
          for (int c = 1; c < C; ++c) s = fmaf(d[u][c], w[e * C + c], s);
          dz[e] = (!p.mask || hv[e] > 0.0f) ? s : 0.0f;
        }
        *reinterpret_cast<floatx4*>(p.dH + (int64_t)row * p.K + k) = floatx4{dz[0], dz[1], dz[2], dz[3]};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[e * C + c] = fmaf(hv[e], d[u][c], acc[e * C + c]);
      if (do_db && q == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c) adb[c] = adb[c] + d[u][c];
      }
    }
  }

  // dW entry (4 q + e, c) = sum over the 64 row lanes of acc[e * C + c] on
  // the threads with that q.  LDS row (jj, q) holds those 64 partials for
  // j = j0 + jj (j = e * C + c); thread t adds LDS row t in row-lane order.
#pragma unroll
  for (int j0 = 0; j0 < 4 * C; j0 += PASS) {
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < PASS; ++jj) red[(jj * 4 + q) * 64 + rl] = acc[j0 + jj];
    __syncthreads();
    if (tid < PASS * 4) {
      const floatx4* src = reinterpret_cast<const floatx4*>(red + tid * 64);
      floatx4 a[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) a[i] = src[i];
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) v = (((v + a[i].x) + a[i].y) + a[i].z) + a[i].w;
      const int j = j0 + (tid >> 2), qq = tid & 3;
      const int kk = k0 + 4 * qq + j / C;
      if (kk < p.K) p.dW[(int64_t)kk * C + j % C] = v;
    }
  }
  if (do_db) {
    __syncthreads();
    if (q == 0) {
#pragma unroll
      for (int c = 0; c < C; ++c) red[c * 64 + rl] = adb[c];
    }
    __syncthreads();
    if (tid < C) {
      const floatx4* src = reinterpret_cast<const floatx4*>(red + tid * 64);
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const floatx4 a = src[i];
        v = (((v + a.x) + a.y) + a.z) + a.w;
      }
      p.db[tid] = v;
    }
  }
  if (blockIdx.x == 0 && (p.fin.loss || p.fin.correct)) {
    __syncthreads();
    finish_rows(p.fin.row_loss, p.fin.row_correct, p.B, p.fin.inv_b, p.fin.loss, p.fin.correct, red_f, red_i);
  }
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

bool head_supported(size_t B, size_t K, size_t C) {
  return C >= 1 && C <= HEAD_MAX_CLASSES && K >= 4 && K % 4 == 0 && B >= 1 && B <= (size_t)INT32_MAX / 2 &&
         K <= (size_t)INT32_MAX / 4;
}

void head_forward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, const float* bias, size_t C,
                  const float* onehot, const int32_t* labels, float* logits, float* dlogits, int32_t* preds,
                  const HeadWorkspace& ws) {
  if (!head_supported(B, K, C)) fail(ORCA_HIP_ERR_SHAPE, "head_forward: unsupported shape");
  if ((onehot == nullptr) == (labels == nullptr))
    fail(ORCA_HIP_ERR_INTERNAL, "head_forward needs exactly one of one-hot targets or labels");
  if (!aligned16(H) || !aligned16(W)) fail(ORCA_HIP_ERR_INTERNAL, "head_forward: H and W must be 16-byte aligned");
  HeadFwdParams p{};
  p.H = H;
  p.W = W;
  p.bias = bias;
  p.onehot = onehot;
  p.labels = labels;
  p.logits = logits;
  p.dlogits = dlogits;
  p.preds = preds;
  p.row_loss = ws.row_loss;
  p.row_correct = ws.row_correct;
  p.B = (int)B;
  p.K = (int)K;
  p.inv_b = 1.0f / (float)B;
  const unsigned rows = C <= 10 ? 4u : 2u;  // fwd_rows<C>()
  const dim3 grid((unsigned)((B + rows - 1) / rows));
  ProfScope ps(ctx, "head_fwd_ce", 2.0 * (double)B * K * C,
               4.0 * ((double)B * K + (double)K * C + C + (double)B * C * (dlogits ? 3 : 2)));
  switch (C) {
#define HEAD_FWD_CASE(N)                                                                        \
  case N:                                                                                       \
    hipLaunchKernelGGL(head_forward_kernel<N>, grid, dim3(HEAD_THREADS), 0, ctx->stream, p);   \
    break;
    HEAD_FWD_CASE(1) HEAD_FWD_CASE(2) HEAD_FWD_CASE(3) HEAD_FWD_CASE(4) HEAD_FWD_CASE(5) HEAD_FWD_CASE(6)
    HEAD_FWD_CASE(7) HEAD_FWD_CASE(8) HEAD_FWD_CASE(9) HEAD_FWD_CASE(10) HEAD_FWD_CASE(11) HEAD_FWD_CASE(12)
    HEAD_FWD_CASE(13) HEAD_FWD_CASE(14) HEAD_FWD_CASE(15) HEAD_FWD_CASE(16)
#undef HEAD_FWD_CASE
    default:
      fail(ORCA_HIP_ERR_SHAPE, "head_forward: unsupported class count");
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

void head_finish(orca_hip_ctx* ctx, const HeadWorkspace& ws, size_t B, float* loss, int64_t* correct) {
  if (!loss && !correct) return;
  HeadFinish f{ws.row_loss, ws.row_correct, loss, correct, 1.0f / (float)B};
  hipLaunchKernelGGL(head_finish_kernel, dim3(1), dim3(HEAD_THREADS), 0, ctx->stream, f, (int)B);
  ORCA_HIP_CHECK(hipGetLastError());
}

void head_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, size_t C,
                   const float* dlogits, bool mask, float* dH, float* dW, float* db, const HeadWorkspace* finish,
                   float* loss, int64_t* correct) {
  if (!head_supported(B, K, C)) fail(ORCA_HIP_ERR_SHAPE, "head_backward: unsupported shape");
  if (!aligned16(H) || !aligned16(W) || (dH && !aligned16(dH)))
    fail(ORCA_HIP_ERR_INTERNAL, "head_backward: H, W and dH must be 16-byte aligned");
  if (C % 4 == 0 ? !aligned16(dlogits) : (C % 2 == 0 && (reinterpret_cast<uintptr_t>(dlogits) & 7) != 0))
    fail(ORCA_HIP_ERR_INTERNAL, "head_backward: dlogits is not aligned for its row length");
  const size_t panels = (K + HEAD_PANEL - 1) / HEAD_PANEL;
  HeadBwdParams p{};
  p.H = H;
  p.W = W;
  p.dl = dlogits;
  p.dH = dH;
  p.dW = dW;
  p.db = db;
  if (finish) p.fin = HeadFinish{finish->row_loss, finish->row_correct, loss, correct, 1.0f / (float)B};
  p.B = (int)B;
  p.K = (int)K;
  p.mask = mask ? 1 : 0;
  const dim3 grid((unsigned)panels);
  ProfScope ps(ctx, "head_bwd", 4.0 * (double)B * K * C,
               4.0 * ((double)B * K * (dH ? 2 : 1) + (double)B * C + 2.0 * K * C + C));
  switch (C) {
#define HEAD_BWD_CASE(N)                                                                        \
  case N:                                                                                       \
    hipLaunchKernelGGL(head_backward_kernel<N>, grid, dim3(HEAD_THREADS), 0, ctx->stream, p);  \
    break;
    HEAD_BWD_CASE(1) HEAD_BWD_CASE(2) HEAD_BWD_CASE(3) HEAD_BWD_CASE(4) HEAD_BWD_CASE(5) HEAD_BWD_CASE(6)
    HEAD_BWD_CASE(7) HEAD_BWD_CASE(8) HEAD_BWD_CASE(9) HEAD_BWD_CASE(10) HEAD_BWD_CASE(11) HEAD_BWD_CASE(12)
    HEAD_BWD_CASE(13) HEAD_BWD_CASE(14) HEAD_BWD_CASE(15) HEAD_BWD_CASE(16)
#undef HEAD_BWD_CASE
    default:
      fail(ORCA_HIP_ERR_SHAPE, "head_backward: unsupported class count");
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_head_forward_ce(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W,
                             const float* bias, size_t C, const float* onehot, const int32_t* labels, float* logits,
                             float* loss, float* dlogits, int32_t* preds, int64_t* correct) {
  return guard([&] {
    bind(ctx);
    if (!H || !W || !bias || !logits) fail(ORCA_HIP_ERR_INTERNAL, "head_forward_ce: null buffer");
    if (!head_supported(B, K, C))
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during head_forward_ce: expected 1..16 classes and K a multiple of 4, got K=" +
                                   std::to_string(K) + " C=" + std::to_string(C));
    check_extent(ctx, H, B * K * sizeof(float), "head_forward_ce (H)");
    check_extent(ctx, W, K * C * sizeof(float), "head_forward_ce (W)");
    check_extent(ctx, bias, C * sizeof(float), "head_forward_ce (bias)");
    check_extent(ctx, onehot, B * C * sizeof(float), "head_forward_ce (onehot)");
    check_extent(ctx, labels, B * sizeof(int32_t), "head_forward_ce (labels)");
    check_extent(ctx, logits, B * C * sizeof(float), "head_forward_ce (logits)");
    check_extent(ctx, dlogits, B * C * sizeof(float), "head_forward_ce (dlogits)");
    check_extent(ctx, preds, B * sizeof(int32_t), "head_forward_ce (preds)");
    check_extent(ctx, loss, sizeof(float), "head_forward_ce (loss)");
    check_extent(ctx, correct, sizeof(int64_t), "head_forward_ce (correct)");
    Scratch rows_f(ctx, sizeof(float) * B), rows_i(ctx, sizeof(int) * B);
    HeadWorkspace ws{rows_f.as<float>(), rows_i.as<int>()};
    head_forward(ctx, H, B, K, W, bias, C, onehot, labels, logits, dlogits, preds, ws);
    head_finish(ctx, ws, B, loss, correct);
  });
}

int orca_hip_head_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, size_t C,
                           const float* dlogits, int relu_mask, float* dH, float* dW, float* db) {
  return guard([&] {
    bind(ctx);
    if (!H || !W || !dlogits || !dW) fail(ORCA_HIP_ERR_INTERNAL, "head_backward: null buffer");
    if (!head_supported(B, K, C))
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during head_backward: expected 1..16 classes and K a multiple of 4, got K=" +
                                   std::to_string(K) + " C=" + std::to_string(C));
    check_extent(ctx, H, B * K * sizeof(float), "head_backward (H)");
    check_extent(ctx, W, K * C * sizeof(float), "head_backward (W)");
    check_extent(ctx, dlogits, B * C * sizeof(float), "head_backward (dlogits)");
    check_extent(ctx, dH, B * K * sizeof(float), "head_backward (dH)");
    check_extent(ctx, dW, K * C * sizeof(float), "head_backward (dW)");
    check_extent(ctx, db, C * sizeof(float), "head_backward (db)");
    head_backward(ctx, H, B, K, W, C, dlogits, relu_mask != 0, dH, dW, db, nullptr, nullptr, nullptr);
  });
}

}  // extern "C"
