// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), used for
// the Linear layer's three products (orca-autograd/src/backend.rs:1449-1499):
//   Y  = X W      (+ bias, ReLU)           trans_a = 0, trans_b = 0
//   dX = dY W^T   (ReLU-mask epilogue)     trans_a = 0, trans_b = 1
//   dW = X^T dY   (+ bias column sum)      trans_a = 1, trans_b = 0
// The transposes never materialise: each operand is copied from global
// memory into LDS in the layout it already has ("k-fast" rows of K
// contiguous values, or "mn-fast" rows of M/N contiguous values) and the
// MFMA fragments are read out of whichever layout it is.
//
// Tiling: a 256-thread block (4 wave64s as 2 x 2) owns a 128 x 128 tile of C;
// each wave owns 64 x 64 = 2 x 2 MFMA 32x32 blocks (64 accumulator VGPRs per
// lane).  K advances in slabs of 32 held in double-buffered LDS (72 KiB, so
// two blocks fit in one CU's 160 KiB).  The next slab's global loads are
// issued before the current slab's 64 MFMAs per wave and land in the other
// LDS buffer afterwards; one barrier per slab.
//
// Within a slab, MFMA step s (0..15) gives lane half h = lane/32 the k index
// h*16 + s, for both operands, so a lane's A (or B^T) fragment for the whole
// slab is 16 contiguous floats of a k-fast row: four ds_read_b128.  Rows of
// k-fast tiles are padded to 36 floats and k-rows 16..31 of mn-fast tiles are
// shifted by 32 floats so both halves of a wave hit disjoint LDS banks.
#include <cstdint>

#include "runtime.hpp"

namespace orca_hip {
namespace {

constexpr int BM = 128, BN = 128, BK = 32, NTHREADS = 256;
constexpr int LDK = BK + 4;        // pitch of k-fast tile rows (floats)
constexpr int MN_GAP = 32;         // shift of k-rows 16..31 in mn-fast tiles
constexpr int TILE = BM * LDK;     // floats per operand buffer (>= BK * BM + MN_GAP)
static_assert(BK * BM + MN_GAP <= TILE, "mn-fast tile must fit the buffer");

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct GemmParams {
  const float* A;
  const float* B;
  float* C;  // output, or split-K workspace [batch][splits][M][N]
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;
  int M, N, K;
  int k_chunk;  // K per split, a multiple of BK
  int splits;
  int epi;
  const float* bias;
  const float* mask;
  int64_t ldmask;
  float* colsum;  // [splits][N]
  int vec_a, vec_b;
};

__device__ __forceinline__ int mn_off(int k) { return k * BM + (k >= 16 ? MN_GAP : 0); }

// Stage one BK slab of an operand into registers.  KFAST: rows of the source
// hold K contiguous values (row r = m or n), else rows hold M/N contiguous
// values (row r = k).
template <bool KFAST>
__device__ __forceinline__ void load_slab(const float* __restrict__ src, int64_t ld, int row0_mn, int lim_mn, int k0,
                                          int klim, bool vec, float4 (&r)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int idx = tid + NTHREADS * j;
    int mn, k;
    if (KFAST) {
      mn = row0_mn + (idx >> 3);
      k = k0 + (idx & 7) * 4;
    } else {
      k = k0 + (idx >> 5);
      mn = row0_mn + (idx & 31) * 4;
    }
    if (KFAST) {
      const float* p = src + (int64_t)mn * ld + k;
      if (vec && mn < lim_mn && k + 4 <= klim) {
        r[j] = *reinterpret_cast<const float4*>(p);
      } else {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = (mn < lim_mn && k + e < klim) ? p[e] : 0.0f;
        r[j] = make_float4(t[0], t[1], t[2], t[3]);
      }
    } else {
      const float* p = src + (int64_t)k * ld + mn;
      if (vec && k < klim && mn + 4 <= lim_mn) {
        r[j] = *reinterpret_cast<const float4*>(p);
      } else {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = (k < klim && mn + e < lim_mn) ? p[e] : 0.0f;
        r[j] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
  }
}

template <bool KFAST>
__device__ __forceinline__ void store_slab(float* __restrict__ s, const float4 (&r)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int idx = tid + NTHREADS * j;
    int off = KFAST ? (idx >> 3) * LDK + (idx & 7) * 4 : mn_off(idx >> 5) + (idx & 31) * 4;
    *reinterpret_cast<float4*>(s + off) = r[j];
  }
}

// Fragment of one 32-row (or 32-column) MFMA block for the whole slab:
// f[s] = operand(row = base + lane%32, k = h*16 + s).
template <bool KFAST>
__device__ __forceinline__ void read_frag(const float* __restrict__ s, int base, float (&f)[16]) {
  const int lane = threadIdx.x & 63, h = lane >> 5, i = lane & 31;
  if (KFAST) {
    const float* p = s + (base + i) * LDK + h * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 v = *reinterpret_cast<const float4*>(p + 4 * q);
      f[4 * q + 0] = v.x;
      f[4 * q + 1] = v.y;
      f[4 * q + 2] = v.z;
      f[4 * q + 3] = v.w;
    }
  } else {
    const float* p = s + h * (16 * BM + MN_GAP) + base + i;
#pragma unroll
    for (int q = 0; q < 16; ++q) f[q] = p[q * BM];
  }
}

// TA: A stored [K][lda] (A^T), else [M][lda].  TB: B stored [N][ldb] (B^T), else [K][ldb].
template <bool TA, bool TB>
__global__ void __launch_bounds__(NTHREADS) gemm_mfma_f32_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) float smem[2][2][TILE];  // [buffer][A|B]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, i = lane & 31;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int bz = blockIdx.z, batch = bz / p.splits, split = bz % p.splits;

  const float* A = p.A + batch * p.sa;
  const float* B = p.B + batch * p.sb;
  const int kb = split * p.k_chunk;
  const int ke = min(p.K, kb + p.k_chunk);
  const int nslabs = (ke - kb + BK - 1) / BK;
  const bool vec_a = p.vec_a != 0, vec_b = p.vec_b != 0;
  const bool do_colsum = p.colsum != nullptr && blockIdx.y == 0 && !TB;

  floatx16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;
  float cs = 0.0f;  // bias column sum (threads 0..127 own column n0 + tid)

  float4 ra[4], rb[4];
  // A tile: rows m (k-fast) when !TA, rows k (m-fast) when TA.
  load_slab<!TA>(A, p.lda, m0, p.M, kb, ke, vec_a, ra);
  load_slab<TB>(B, p.ldb, n0, p.N, kb, ke, vec_b, rb);
  store_slab<!TA>(smem[0][0], ra);
  store_slab<TB>(smem[0][1], rb);
  __syncthreads();

  for (int t = 0; t < nslabs; ++t) {
    const int cur = t & 1;
    const int k0 = kb + t * BK;
    const bool more = t + 1 < nslabs;
    if (more) {
      load_slab<!TA>(A, p.lda, m0, p.M, k0 + BK, ke, vec_a, ra);
      load_slab<TB>(B, p.ldb, n0, p.N, k0 + BK, ke, vec_b, rb);
    }
    const float* sa = smem[cur][0];
    const float* sb = smem[cur][1];
    if (do_colsum && tid < BN) {
      const int kv = min(BK, ke - k0);
      for (int k = 0; k < kv; ++k) cs = cs + sb[mn_off(k) + tid];
    }
    float fa[2][16], fb[2][16];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) read_frag<!TA>(sa, wm * 64 + mt * 32, fa[mt]);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) read_frag<TB>(sb, wn * 64 + nt * 32, fb[nt]);
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mt][s], fb[nt][s], acc[mt][nt], 0, 0, 0);
    if (more) {
      store_slab<!TA>(smem[cur ^ 1][0], ra);
      store_slab<TB>(smem[cur ^ 1][1], rb);
    }
    __syncthreads();
  }

  // One partial per K-chunk when K is split (reduced in chunk order on the host side).
  if (do_colsum && tid < BN && n0 + tid < p.N) p.colsum[(int64_t)split * p.N + n0 + tid] = cs;

  // Epilogue.  Lane (h, i), register r of block (mt, nt) holds
  // C[wm*64 + mt*32 + (r/4)*8 + h*4 + r%4][wn*64 + nt*32 + i].
  float* C = p.C + batch * p.sc;
  if (p.splits > 1) C = p.C + (int64_t)bz * p.M * p.N;  // raw partial sums, ld = N
  const int64_t ldc = p.splits > 1 ? p.N : p.ldc;
  const int epi = p.splits > 1 ? ORCA_HIP_EPI_NONE : p.epi;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + wn * 64 + nt * 32 + i;
      if (col >= p.N) continue;
      float bias = 0.0f;
      if (epi == ORCA_HIP_EPI_BIAS || epi == ORCA_HIP_EPI_BIAS_RELU) bias = p.bias[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + mt * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        if (row >= p.M) continue;
        float v = acc[mt][nt][r];
        if (epi == ORCA_HIP_EPI_BIAS) {
          v = v + bias;
        } else if (epi == ORCA_HIP_EPI_BIAS_RELU) {
          v = v + bias;
          v = v > 0.0f ? v : 0.0f;
        } else if (epi == ORCA_HIP_EPI_RELU_MASK) {
          v = p.mask[(int64_t)row * p.ldmask + col] > 0.0f ? v : 0.0f;
        }
        C[(int64_t)row * ldc + col] = v;
      }
    }
}

// Sums split-K partials in split order and applies the epilogue.
struct SplitReduceParams {
  const float* ws;
  float* C;
  int64_t ldc, sc;
  int M, N, splits;
  int epi;
  const float* bias;
  const float* mask;
  int64_t ldmask;
};

__global__ void splitk_reduce_kernel(SplitReduceParams p, size_t total) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t mn = (size_t)p.M * p.N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    size_t b = idx / mn, rem = idx % mn;
    int row = (int)(rem / p.N), col = (int)(rem % p.N);
    const float* w = p.ws + b * p.splits * mn + rem;
    float v = w[0];
    for (int s = 1; s < p.splits; ++s) v = v + w[s * mn];
    if (p.epi == ORCA_HIP_EPI_BIAS) {
      v = v + p.bias[col];
    } else if (p.epi == ORCA_HIP_EPI_BIAS_RELU) {
      v = v + p.bias[col];
      v = v > 0.0f ? v : 0.0f;
    } else if (p.epi == ORCA_HIP_EPI_RELU_MASK) {
      v = p.mask[(int64_t)row * p.ldmask + col] > 0.0f ? v : 0.0f;
    }
    p.C[b * p.sc + (int64_t)row * p.ldc + col] = v;
  }
}

// colsum[n] = sum over K-chunks, in chunk order, of the per-chunk column sums.
__global__ void colsum_split_reduce_kernel(const float* __restrict__ part, int splits, int N, float* __restrict__ out) {
  int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float v = part[n];
  for (int s = 1; s < splits; ++s) v = v + part[(int64_t)s * N + n];
  out[n] = v;
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

const char* kernel_name(bool ta, bool tb) {
  if (!ta && !tb) return "gemm_nn";
  if (!ta && tb) return "gemm_nt";
  if (ta && !tb) return "gemm_tn";
  return "gemm_tt";
}

}  // namespace

void gemm(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K, const float* A, size_t lda,
          size_t sa, const float* B, size_t ldb, size_t sb, float* C, size_t ldc, size_t sc, size_t batch,
          const GemmEpi& epi) {
  if (M == 0 || N == 0 || batch == 0) return;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > 65535)
    fail(ORCA_HIP_ERR_INTERNAL, "gemm dimensions exceed the kernel's index range");
  if (K == 0) {  // empty product: C = epilogue(0)
    for (size_t b = 0; b < batch; ++b) {
      if (epi.kind == ORCA_HIP_EPI_NONE || epi.kind == ORCA_HIP_EPI_RELU_MASK) {
        if (ldc == N) launch_fill(ctx, C + b * sc, 0.0f, M * N);
        else for (size_t r = 0; r < M; ++r) launch_fill(ctx, C + b * sc + r * ldc, 0.0f, N);
      } else {
        fail(ORCA_HIP_ERR_INTERNAL, "gemm with K = 0 and a bias epilogue is not supported");
      }
    }
    if (epi.colsum) launch_fill(ctx, epi.colsum, 0.0f, N);
    return;
  }
  const size_t mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
  if (mt > 65535) fail(ORCA_HIP_ERR_INTERNAL, "gemm: too many row tiles");

  // Split K when the tile grid cannot fill the CUs and K is long enough.
  int splits = 1;
  const size_t tiles = mt * nt * batch;
  const size_t target = (size_t)ctx->num_cus;
  if (tiles < target / 2 && K >= 4 * (size_t)BK) {
    size_t want = (target + tiles - 1) / tiles;
    size_t max_by_k = K / (2 * BK);
    splits = (int)std::min<size_t>(std::min<size_t>(want, max_by_k), 64);
    if (splits < 1) splits = 1;
  }
  int k_chunk = (int)K;
  if (splits > 1) {
    size_t per = (K + splits - 1) / splits;
    per = (per + BK - 1) / BK * BK;
    splits = (int)((K + per - 1) / per);
    k_chunk = (int)per;
  }

  GemmParams p{};
  p.A = A;
  p.B = B;
  p.lda = (int64_t)lda;
  p.ldb = (int64_t)ldb;
  p.ldc = (int64_t)ldc;
  p.sa = (int64_t)sa;
  p.sb = (int64_t)sb;
  p.sc = (int64_t)sc;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.k_chunk = k_chunk;
  p.splits = splits;
  p.epi = epi.kind;
  p.bias = epi.bias;
  p.mask = epi.mask;
  p.ldmask = (int64_t)epi.ldmask;
  const bool fold_colsum = epi.colsum != nullptr && batch == 1 && !trans_b;
  std::unique_ptr<Scratch> colsum_ws;
  if (fold_colsum && splits > 1) {
    colsum_ws.reset(new Scratch(ctx, sizeof(float) * splits * N));
    p.colsum = colsum_ws->as<float>();
  } else {
    p.colsum = fold_colsum ? epi.colsum : nullptr;
  }
  p.vec_a = aligned16(A) && lda % 4 == 0 && (batch == 1 || sa % 4 == 0);
  p.vec_b = aligned16(B) && ldb % 4 == 0 && (batch == 1 || sb % 4 == 0);

  std::unique_ptr<Scratch> ws;
  if (splits > 1) {
    ws.reset(new Scratch(ctx, sizeof(float) * batch * splits * M * N));
    p.C = ws->as<float>();
  } else {
    p.C = C;
  }

  dim3 grid((unsigned)nt, (unsigned)mt, (unsigned)(batch * splits));
  {
    ProfScope ps(ctx, kernel_name(trans_a, trans_b), 2.0 * (double)M * N * K * batch,
                 4.0 * (double)batch * (M * K + K * N + M * N));
    if (!trans_a && !trans_b)
      hipLaunchKernelGGL((gemm_mfma_f32_kernel<false, false>), grid, dim3(NTHREADS), 0, ctx->stream, p);
    else if (!trans_a && trans_b)
      hipLaunchKernelGGL((gemm_mfma_f32_kernel<false, true>), grid, dim3(NTHREADS), 0, ctx->stream, p);
    else if (trans_a && !trans_b)
      hipLaunchKernelGGL((gemm_mfma_f32_kernel<true, false>), grid, dim3(NTHREADS), 0, ctx->stream, p);
    else
      hipLaunchKernelGGL((gemm_mfma_f32_kernel<true, true>), grid, dim3(NTHREADS), 0, ctx->stream, p);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (splits > 1) {
    SplitReduceParams r{};
    r.ws = p.C;
    r.C = C;
    r.ldc = (int64_t)ldc;
    r.sc = (int64_t)sc;
    r.M = (int)M;
    r.N = (int)N;
    r.splits = splits;
    r.epi = epi.kind;
    r.bias = epi.bias;
    r.mask = epi.mask;
    r.ldmask = (int64_t)epi.ldmask;
    size_t total = batch * M * N;
    ProfScope ps(ctx, "gemm_splitk_reduce", 0.0, 4.0 * (double)total * (splits + 1));
    unsigned g = grid_for(total, 256, ctx->num_cus * 8);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(g), dim3(256), 0, ctx->stream, r, total);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (fold_colsum && splits > 1) {
    hipLaunchKernelGGL(colsum_split_reduce_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, ctx->stream,
                       p.colsum, splits, (int)N, epi.colsum);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  // Column sums that the GEMM could not fold in (batched, or B^T storage).
  if (epi.colsum && !fold_colsum) {
    if (batch != 1) fail(ORCA_HIP_ERR_INTERNAL, "gemm colsum epilogue requires batch == 1");
    if (trans_b) fail(ORCA_HIP_ERR_INTERNAL, "gemm colsum epilogue requires row-major B");
    launch_colsum(ctx, B, K, N, ldb, epi.colsum);
  }
}

}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_gemm(orca_hip_ctx* ctx, int trans_a, int trans_b, size_t M, size_t N, size_t K, const float* A, size_t lda,
                  const float* B, size_t ldb, float* C, size_t ldc, const orca_hip_epilogue* epi) {
  return guard([&] {
    bind(ctx);
    if ((trans_a ? lda < M : lda < K) || (trans_b ? ldb < K : ldb < N) || ldc < N)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during gemm: leading dimension smaller than the row length");
    GemmEpi e;
    if (epi) {
      e.kind = epi->kind;
      e.bias = epi->bias;
      e.mask = epi->mask;
      e.ldmask = epi->ldmask;
      e.colsum = epi->colsum;
      if (e.kind < ORCA_HIP_EPI_NONE || e.kind > ORCA_HIP_EPI_RELU_MASK)
        fail(ORCA_HIP_ERR_INTERNAL, "unknown gemm epilogue " + std::to_string(e.kind));
      if ((e.kind == ORCA_HIP_EPI_BIAS || e.kind == ORCA_HIP_EPI_BIAS_RELU) && !e.bias)
        fail(ORCA_HIP_ERR_INTERNAL, "bias epilogue without a bias pointer");
      if (e.kind == ORCA_HIP_EPI_RELU_MASK && (!e.mask || e.ldmask < N))
        fail(ORCA_HIP_ERR_INTERNAL, "mask epilogue without a valid mask");
    }
    gemm(ctx, trans_a != 0, trans_b != 0, M, N, K, A, lda, 0, B, ldb, 0, C, ldc, 0, 1, e);
  });
}

// orca-backend-cpu/src/backend.rs:130-221 (contract), with lazy-transpose views.
int orca_hip_matmul(orca_hip_ctx* ctx, const void* lhs, const void* rhs, const size_t* lhs_shape, size_t lhs_rank,
                    const size_t* rhs_shape, size_t rhs_rank, int dtype, int lhs_view, int rhs_view, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "matmul");
    if (lhs_rank < 2 || rhs_rank < 2) fail(ORCA_HIP_ERR_INTERNAL, "Matmul requires at least 2D shapes");
    if (lhs_rank != rhs_rank)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during matmul: expected Same rank for batched matmul, got " +
                                   std::to_string(lhs_rank) + "D and " + std::to_string(rhs_rank) + "D");
    size_t batch = 1;
    for (size_t i = 0; i + 2 < lhs_rank; ++i) {
      if (lhs_shape[i] != rhs_shape[i]) fail(ORCA_HIP_ERR_INTERNAL, "Matmul batch dimensions must match");
      batch *= lhs_shape[i];
    }
    size_t M = lhs_shape[lhs_rank - 2], K = lhs_shape[lhs_rank - 1];
    size_t K2 = rhs_shape[rhs_rank - 2], N = rhs_shape[rhs_rank - 1];
    if (K != K2)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during matmul: expected Inner dimensions must match: " +
                                   std::to_string(K) + " == " + std::to_string(K2) + ", got " + std::to_string(K) +
                                   " != " + std::to_string(K2));
    const bool ta = lhs_view == ORCA_HIP_VIEW_TRANSPOSED, tb = rhs_view == ORCA_HIP_VIEW_TRANSPOSED;
    float* o = new_output(ctx, batch * M * N);
    GemmEpi e;
    gemm(ctx, ta, tb, M, N, K, static_cast<const float*>(lhs), ta ? M : K, M * K, static_cast<const float*>(rhs),
         tb ? K : N, K * N, o, N, M * N, batch, e);
    *out = o;
  });
}

}  // extern "C"
