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
//                         (python/orca/nn/loss.py:59-100).
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

constexpr int FWD_THREADS = 512;  // 8 waves
constexpr int FWD_GPT = 2;        // float4 column groups of H per thread per pass
constexpr int BWD_THREADS = 512;  // 8 waves: 4 column groups x 128 row lanes
constexpr int BWD_ROW_LANES = BWD_THREADS / 4;
constexpr int HEAD_PANEL = 16;                            // columns of H per backward block
constexpr int FINISH_THREADS = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Rows per forward block (one wave per row in the loss phase): 4, or 2 for
// C > 10 so that a thread's W slices and accumulators stay in registers.
template <int C>
constexpr int fwd_rows() {
  return C <= 10 ? 4 : 2;
}
// Rows per backward thread per row group (a group is 128 x that many rows):
// 8, or 4 for C > 10, again to stay in registers.
template <int C>
constexpr int bwd_rows() {
  return C <= 10 ? 8 : 4;
}

// Blocks are handed to the 8 XCDs round-robin; with nb a multiple of 8 this
// gives XCD x the consecutive work items x * nb/8 ... so neighbours that
// share cache lines share an L2.  (A performance mapping only: any bijection
// is correct.)
__device__ __forceinline__ int xcd_local_index(int b, int nb) {
  return (nb & 7) ? b : (b & 7) * (nb >> 3) + (b >> 3);
}

// ---- wave folds: sums over groups of lanes without LDS ----
// The lanes that differ only in lane bits M, M/2, ..., LO (powers of two)
// form a group, and wave_fold adds each of N values over the group.  While
// the count is even a step halves it: the lane with bit M clear keeps the
// first half (adding its partner's copy), the partner the second half, so
// the group's lanes end up with different slices.  Once the count is odd a
// step adds the partner's whole set and both lanes hold the same sums.  A
// lane's slice starts at `base`; fold_shared(N, M, LO) is the mask of the
// lane bits whose lanes hold identical slices.  Every sum has an order fixed
// by the lane indices.
constexpr int fold_len(int n, int m, int lo) {
  return m < lo ? n : (n % 2 == 0 ? fold_len(n / 2, m / 2, lo) : fold_len(n, m / 2, lo));
}
constexpr int fold_shared(int n, int m, int lo) {
  return m < lo ? 0 : (n % 2 == 0 ? fold_shared(n / 2, m / 2, lo) : (m | fold_shared(n, m / 2, lo)));
}

template <int N, int M, int LO>
__device__ __forceinline__ void wave_fold(const float (&v)[N], float (&out)[fold_len(N, M, LO)], int& base) {
  if constexpr (M < LO) {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = v[j];
  } else if constexpr (N % 2 == 0) {
    constexpr int HN = N / 2;
    const bool up = (threadIdx.x & M) != 0;
    float nv[HN];
#pragma unroll
    for (int j = 0; j < HN; ++j) {
      const float send = up ? v[j] : v[j + HN];
      const float keep = up ? v[j + HN] : v[j];
      nv[j] = keep + __shfl_xor(send, M, 64);
    }
    if (up) base += HN;
    wave_fold<HN, M / 2, LO>(nv, out, base);
  } else {
    float nv[N];
#pragma unroll
    for (int j = 0; j < N; ++j) nv[j] = v[j] + __shfl_xor(v[j], M, 64);
    wave_fold<N, M / 2, LO>(nv, out, base);
  }
}

// Adds N per-lane values over the lanes of each wave that differ in lane
// bits M..LO, then over the block's waves: part receives one row of N sums
// per wave (and per value of the lane bits below LO), and thread t < n_out
// later adds the rows of its column in wave order.
template <int N, int M, int LO>
__device__ __forceinline__ void fold_to_lds(const float (&v)[N], float* part, int row_stride, int row) {
  constexpr int NF = fold_len(N, M, LO);
  constexpr int SHARED = fold_shared(N, M, LO);
  float out[NF];
  int base = 0;
  wave_fold<N, M, LO>(v, out, base);
  if ((threadIdx.x & SHARED) == 0) {
#pragma unroll
    for (int j = 0; j < NF; ++j) part[row * row_stride + base + j] = out[j];
  }
}

// loss = (sum of row terms) * (1/B) and the correct-row count, by one block
// (any multiple of 64 threads up to 1024).
__device__ void finish_rows(const float* __restrict__ row_loss, const int* __restrict__ row_correct, int B, float inv_b,
                            float* loss, int64_t* correct, float* red_f, int* red_i) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nt = blockDim.x;
  const int per = (B + nt - 1) / nt;
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
    for (int w = 1; w < nt / 64; ++w) {
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

// Block = fwd_rows<C>() rows x all of K, 512 threads.  Thread t multiplies
// the float4 column groups t, t + 512 (then t + 1024, ... for K > 4096) of
// every row: the rows' H values and W's 4 x C slice for those columns come
// straight from memory, all of a pass's loads issued before the first use,
// so a block waits for memory once per pass (once in all for K <= 4096).
// The per-thread partial logits are added over each wave's lanes by a wave
// fold and over the 8 waves in wave order; the bias is added after the
// product, as a separate f32 operation.  Then one wave per row runs the
// softmax cross-entropy.
template <int C>
__global__ void __launch_bounds__(FWD_THREADS) head_forward_kernel(HeadFwdParams p) {
  constexpr int R = fwd_rows<C>(), NV = R * C;
  constexpr int NW = FWD_THREADS / 64;
  __shared__ float part[NW * NV];
  __shared__ float logit[NV];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * R;
  const int nrows = min(R, p.B - r0);
  const int K4 = p.K >> 2;
  const floatx4* W4 = reinterpret_cast<const floatx4*>(p.W);

  float acc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = 0.0f;

  for (int g0 = tid; g0 < K4; g0 += FWD_GPT * FWD_THREADS) {
    floatx4 h[FWD_GPT][R], w[FWD_GPT][C];
#pragma unroll
    for (int s = 0; s < FWD_GPT; ++s) {
      const int g = g0 + s * FWD_THREADS;
      const bool in = g < K4;
#pragma unroll
      for (int r = 0; r < R; ++r)
        h[s][r] = in && r < nrows ? *reinterpret_cast<const floatx4*>(p.H + (int64_t)(r0 + r) * p.K + 4 * g)
                                  : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < C; ++j) w[s][j] = in ? W4[(int64_t)g * C + j] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int s = 0; s < FWD_GPT; ++s) {
      float wf[4 * C];  // W rows 4g .. 4g+3, C values each
#pragma unroll
      for (int j = 0; j < C; ++j) {
        wf[4 * j] = w[s][j].x;
        wf[4 * j + 1] = w[s][j].y;
        wf[4 * j + 2] = w[s][j].z;
        wf[4 * j + 3] = w[s][j].w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < C; ++c) {
          float a = acc[r * C + c];
          a = fmaf(h[s][r].x, wf[c], a);
          a = fmaf(h[s][r].y, wf[C + c], a);
          a = fmaf(h[s][r].z, wf[2 * C + c], a);
          a = fmaf(h[s][r].w, wf[3 * C + c], a);
          acc[r * C + c] = a;
        }
    }
  }

  fold_to_lds<NV, 32, 1>(acc, part, NV, wave);
  __syncthreads();
  if (tid < NV) {
    float z = part[tid];
#pragma unroll
    for (int w = 1; w < NW; ++w) z = z + part[w * NV + tid];
    logit[tid] = z;
  }
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

__global__ void __launch_bounds__(FINISH_THREADS) head_finish_kernel(HeadFinish f, int B) {
  __shared__ float red_f[FINISH_THREADS / 64];
  __shared__ int red_i[FINISH_THREADS / 64];
  finish_rows(f.row_loss, f.row_correct, B, f.inv_b, f.loss, f.correct, red_f, red_i);
}

struct HeadBwdParams {
  const float* H;   // [B][K] (ReLU output of the layer below: also the mask)
  const float* W;   // [K][C]
  const float* dl;  // [B][C] dL/dlogits
  float* dH;        // [B][K] or null
  float* dW;        // [K][C]
  float* db;        // [C] or null
  float* dh_colsum; // [K] column sums of dH (the bias gradient of the layer below) or null
  HeadFinish fin;   // block 0 also finishes the forward's loss when fin.loss or fin.correct is set
  int B, K;
  int mask;
  int dl_vec;  // dl is 16-byte aligned: staged with float4 loads
};

// Block = 16 columns of H (a panel) x all B rows, so no block depends on
// another; 512 threads: column group q = t % 4 of the panel, row lane
// t / 4.  Rows go in groups of 1024 (512 when C > 10): the group's rows of
// dlogits are staged in LDS and each thread loads its 8 (4) rows of H, all
// before the first use.
// A thread keeps W's 4 x C slice for its columns, writes
// dH = (dlogits W^T) * [H > 0] for its rows and accumulates its 4 x C
// products of dW in row order; the row lanes are then added by a wave fold
// and the 8 waves in wave order.  With dh_colsum the block also adds up its
// 16 columns of dH over all rows the same way (each thread its rows in
// order, then the fold and the waves): the bias gradient of the layer below,
// which its weight-gradient product then need not compute.  Adjacent panels share 128-byte lines of H
// and dH, so they run on one XCD.
template <int C>
__global__ void __launch_bounds__(BWD_THREADS) head_backward_kernel(HeadBwdParams p) {
  constexpr int NW = BWD_THREADS / 64;
  constexpr int NV = 4 * C;
  constexpr int BWD_ROWS = bwd_rows<C>();
  constexpr int BWD_GROUP = BWD_ROW_LANES * BWD_ROWS;
  constexpr int SPT = (BWD_GROUP * C / 4 + BWD_THREADS - 1) / BWD_THREADS;  // staged float4s per thread
  __shared__ __attribute__((aligned(16))) float dls[BWD_GROUP * C];
  __shared__ float part[NW * 4 * NV];
  __shared__ float red_f[NW];
  __shared__ int red_i[NW];
  const int tid = threadIdx.x, wave = tid >> 6;
  const int q = tid & 3, rl = tid >> 2;
  const int panel = xcd_local_index(blockIdx.x, gridDim.x);
  const int k0 = panel * HEAD_PANEL;
  const int k = k0 + 4 * q;
  const bool kin = k < p.K;
  const bool do_db = p.db != nullptr && panel == 0;

  float w[NV];
  {
    const floatx4* wp = reinterpret_cast<const floatx4*>(p.W + (int64_t)k * C);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const floatx4 v = kin ? wp[j] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      w[4 * j] = v.x;
      w[4 * j + 1] = v.y;
      w[4 * j + 2] = v.z;
      w[4 * j + 3] = v.w;
    }
  }
  float acc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = 0.0f;
  float adb[C];
#pragma unroll
  for (int c = 0; c < C; ++c) adb[c] = 0.0f;
  float adz[4] = {0.0f, 0.0f, 0.0f, 0.0f};

  const int ngroups = (p.B + BWD_GROUP - 1) / BWD_GROUP;
  for (int gi = 0; gi < ngroups; ++gi) {
    const int g0 = gi * BWD_GROUP;
    const int cnt = min(BWD_GROUP, p.B - g0) * C;  // floats of dlogits in this group
    const float* src = p.dl + (int64_t)g0 * C;
    floatx4 st[SPT];
    floatx4 h[BWD_ROWS];
    if (p.dl_vec) {
#pragma unroll
      for (int j = 0; j < SPT; ++j) {
        const int e = 4 * (tid + BWD_THREADS * j);
        if (e + 3 < cnt) {
          st[j] = *reinterpret_cast<const floatx4*>(src + e);
        } else {
          float t[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) t[i] = e + i < cnt ? src[e + i] : 0.0f;
          st[j] = floatx4{t[0], t[1], t[2], t[3]};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < BWD_ROWS; ++u) {
      const int row = g0 + rl + BWD_ROW_LANES * u;
      h[u] = row < p.B && kin ? *reinterpret_cast<const floatx4*>(p.H + (int64_t)row * p.K + k)
                              : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();  // the previous group's rows of dls have been read
    if (p.dl_vec) {
#pragma unroll
      for (int j = 0; j < SPT; ++j) {
        const int i4 = tid + BWD_THREADS * j;
        if (4 * i4 < BWD_GROUP * C) reinterpret_cast<floatx4*>(dls)[i4] = st[j];
      }
    } else {
      for (int e = tid; e < BWD_GROUP * C; e += BWD_THREADS) dls[e] = e < cnt ? src[e] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < BWD_ROWS; ++u) {
      const int lr = rl + BWD_ROW_LANES * u;
      const int row = g0 + lr;
      if (row >= p.B) break;
      float d[C];
      const float* dr = dls + lr * C;
      if constexpr (C % 4 == 0) {
#pragma unroll
        for (int j = 0; j < C / 4; ++j) {
          const floatx4 v = reinterpret_cast<const floatx4*>(dr)[j];
          d[4 * j] = v.x;
          d[4 * j + 1] = v.y;
          d[4 * j + 2] = v.z;
          d[4 * j + 3] = v.w;
        }
      } else if constexpr (C % 2 == 0) {
#pragma unroll
        for (int j = 0; j < C / 2; ++j) {
          const floatx2 v = reinterpret_cast<const floatx2*>(dr)[j];
          d[2 * j] = v.x;
          d[2 * j + 1] = v.y;
        }
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c) d[c] = dr[c];
      }
      const float hv[4] = {h[u].x, h[u].y, h[u].z, h[u].w};
      if (kin && p.dH) {
        float dz[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float s = d[0] * w[e * C];
#pragma unroll
          for (int c = 1; c < C; ++c) s = fmaf(d[c], w[e * C + c], s);
          dz[e] = (!p.mask || hv[e] > 0.0f) ? s : 0.0f;
        }
        *reinterpret_cast<floatx4*>(p.dH + (int64_t)row * p.K + k) = floatx4{dz[0], dz[1], dz[2], dz[3]};
        if (p.dh_colsum) {
#pragma unroll
          for (int e = 0; e < 4; ++e) adz[e] = adz[e] + dz[e];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[e * C + c] = fmaf(hv[e], d[c], acc[e * C + c]);
      if (do_db && q == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c) adb[c] = adb[c] + d[c];
      }
    }
  }

  // dW entry (4 q + e, c) = the sum over all row lanes of acc[e * C + c] on
  // the threads with that q.  Lane bits 2..5 are the wave's 16 row lanes and
  // bits 0..1 are q, so the fold runs over bits 32..4; part row (wave, q).
  fold_to_lds<NV, 32, 4>(acc, part, NV, wave * 4 + q);
  __syncthreads();
  if (tid < 4 * NV) {  // tid = q * NV + j: dW[k0 + 4 q + j / C][j % C] = dW[k0 * C + tid]
    const int qq = tid / NV, j = tid % NV;
    float v = part[qq * NV + j];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) v = v + part[(w2 * 4 + qq) * NV + j];
    if (k0 + 4 * qq + j / C < p.K) p.dW[(int64_t)k0 * C + tid] = v;
  }
  if (p.dh_colsum) {
    __syncthreads();  // part is read above
    fold_to_lds<4, 32, 4>(adz, part, 4, wave * 4 + q);
    __syncthreads();
    if (tid < 16) {  // column k0 + tid = k0 + 4 qq + e
      const int qq = tid / 4, e = tid % 4;
      float v = part[qq * 4 + e];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) v = v + part[(w2 * 4 + qq) * 4 + e];
      if (k0 + tid < p.K) p.dh_colsum[k0 + tid] = v;
    }
  }
  if (do_db) {
    __syncthreads();
    fold_to_lds<C, 32, 4>(adb, part, C, wave * 4 + q);
    __syncthreads();
    if (tid < C) {  // the q = 0 rows of part hold the partial sums
      float v = part[tid];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) v = v + part[w2 * 4 * C + tid];
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
    hipLaunchKernelGGL(head_forward_kernel<N>, grid, dim3(FWD_THREADS), 0, ctx->stream, p);    \
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
  hipLaunchKernelGGL(head_finish_kernel, dim3(1), dim3(FINISH_THREADS), 0, ctx->stream, f, (int)B);
  ORCA_HIP_CHECK(hipGetLastError());
}

void head_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* W, size_t C,
                   const float* dlogits, bool mask, float* dH, float* dW, float* db, const HeadWorkspace* finish,
                   float* loss, int64_t* correct, float* dh_colsum) {
  if (!head_supported(B, K, C)) fail(ORCA_HIP_ERR_SHAPE, "head_backward: unsupported shape");
  if (!aligned16(H) || !aligned16(W) || (dH && !aligned16(dH)))
    fail(ORCA_HIP_ERR_INTERNAL, "head_backward: H, W and dH must be 16-byte aligned");
  const size_t panels = (K + HEAD_PANEL - 1) / HEAD_PANEL;
  HeadBwdParams p{};
  p.H = H;
  p.W = W;
  p.dl = dlogits;
  p.dH = dH;
  p.dW = dW;
  p.db = db;
  if (dh_colsum && !dH) fail(ORCA_HIP_ERR_INTERNAL, "head_backward: dH column sums without dH");
  p.dh_colsum = dh_colsum;
  if (finish) p.fin = HeadFinish{finish->row_loss, finish->row_correct, loss, correct, 1.0f / (float)B};
  p.B = (int)B;
  p.K = (int)K;
  p.mask = mask ? 1 : 0;
  p.dl_vec = aligned16(dlogits) ? 1 : 0;
  const dim3 grid((unsigned)panels);
  ProfScope ps(ctx, "head_bwd", 4.0 * (double)B * K * C,
               4.0 * ((double)B * K * (dH ? 2 : 1) + (double)B * C + 2.0 * K * C + C));
  switch (C) {
#define HEAD_BWD_CASE(N)                                                                        \
  case N:                                                                                       \
    hipLaunchKernelGGL(head_backward_kernel<N>, grid, dim3(BWD_THREADS), 0, ctx->stream, p);   \
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
