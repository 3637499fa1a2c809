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
// Tiling: a 256-thread block (4 wave64s as 2 x 2) owns a 128 x 128 or
// 128 x 64 tile of C (the smaller tile when the larger one cannot give every
// CU two blocks); each wave owns 2 x 2 (or 2 x 1) MFMA 32x32 blocks.  K
// advances in slabs of 32 held in double-buffered LDS (72 / 54 KiB, so two
// blocks fit in one CU's 160 KiB).  The next slab's global loads are issued
// before the current slab's MFMAs and land in the other LDS buffer
// afterwards; one barrier per slab.  Interior blocks of aligned operands load
// without bounds checks (a uniform branch); edge blocks zero-fill.
//
// Within a slab, MFMA step s (0..15) gives lane half h = lane/32 the k index
// h*16 + s, for both operands, so a lane's A (or B^T) fragment for the whole
// slab is 16 contiguous floats of a k-fast row: four ds_read_b128.  Rows of
// k-fast tiles are padded to 36 floats and k-rows 16..31 of mn-fast tiles are
// shifted by 32 floats so both halves of a wave hit disjoint LDS banks.
#include <cstdint>
#include <cstdlib>
#include <string>
#include <type_traits>

#include <hip/hip_ext.h>

#include "runtime.hpp"

namespace orca_hip {
namespace {

constexpr int BK = 32, NTHREADS = 256;
constexpr int LDK = BK + 4;  // pitch of k-fast tile rows (floats)
constexpr int MN_GAP = 32;   // shift of k-rows 16..31 in mn-fast tiles

typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native 4-float vector: copies stay SSA values (HIP's float4 struct copies
// lower to memcpy, which can pin a register stage in scratch).
typedef float floatx4 __attribute__((ext_vector_type(4)));

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
  float* pre;     // EPI_BIAS_RELU_PRE: acc + bias; EPI_RELU_MASK_PRE: acc (with ldc)
  float* colsum;  // [splits][N]
  int vec_a, vec_b;
};

// Floats of one operand buffer: P rows of a k-fast tile, or BK rows of P in a mn-fast tile.
constexpr int tile_floats(int P) { return P * LDK > BK * P + MN_GAP ? P * LDK : BK * P + MN_GAP; }

template <int P>
__device__ __forceinline__ int mn_off(int k) {
  return k * P + (k >= 16 ? MN_GAP : 0);
}

// Stage one BK slab of an operand (P rows/cols of M or N) into registers.
// KFAST: rows of the source hold K contiguous values (row = m or n), else rows
// hold M/N contiguous values (row = k).  `fast` (uniform per block) means the
// whole slab is in bounds and 16-byte aligned: plain float4 loads.
template <bool KFAST, int P>
__device__ __forceinline__ void load_slab(const float* __restrict__ src, int64_t ld, int row0_mn, int lim_mn, int k0,
                                          int klim, bool fast, float4 (&r)[P / 32]) {
  const int tid = threadIdx.x;
  constexpr int PER_ROW = P / 4;  // float4s per mn-fast row
#pragma unroll
  for (int j = 0; j < P / 32; ++j) {
    const int idx = tid + NTHREADS * j;
    int mn, k;
    if (KFAST) {
      mn = row0_mn + (idx >> 3);
      k = k0 + (idx & 7) * 4;
    } else {
      k = k0 + idx / PER_ROW;
      mn = row0_mn + (idx % PER_ROW) * 4;
    }
    const float* p = KFAST ? src + (int64_t)mn * ld + k : src + (int64_t)k * ld + mn;
    if (fast) {
      r[j] = *reinterpret_cast<const float4*>(p);
    } else {
      float t[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = KFAST ? (mn < lim_mn && k + e < klim) : (k < klim && mn + e < lim_mn);
        t[e] = in ? p[e] : 0.0f;
      }
      r[j] = make_float4(t[0], t[1], t[2], t[3]);
    }
  }
}

template <bool KFAST, int P, typename V>
__device__ __forceinline__ void store_slab(float* __restrict__ s, const V (&r)[P / 32]) {
  const int tid = threadIdx.x;
  constexpr int PER_ROW = P / 4;
#pragma unroll
  for (int j = 0; j < P / 32; ++j) {
    const int idx = tid + NTHREADS * j;
    const int off = KFAST ? (idx >> 3) * LDK + (idx & 7) * 4 : mn_off<P>(idx / PER_ROW) + (idx % PER_ROW) * 4;
    *reinterpret_cast<V*>(s + off) = r[j];
  }
}

// Half a slab of one 32-row (or 32-column) MFMA block's fragment:
// f[q] = operand(row = base + lane%32, k = h*16 + 8*half + q), q = 0..7.
template <bool KFAST, int P>
__device__ __forceinline__ void read_frag(const float* __restrict__ s, int base, int half, float (&f)[8]) {
  const int lane = threadIdx.x & 63, h = lane >> 5, i = lane & 31;
  if (KFAST) {
    const float* p = s + (base + i) * LDK + h * 16 + half * 8;
    const float4 v0 = *reinterpret_cast<const float4*>(p);
    const float4 v1 = *reinterpret_cast<const float4*>(p + 4);
    f[0] = v0.x; f[1] = v0.y; f[2] = v0.z; f[3] = v0.w;
    f[4] = v1.x; f[5] = v1.y; f[6] = v1.z; f[7] = v1.w;
  } else {
    const float* p = s + h * (16 * P + MN_GAP) + half * 8 * P + base + i;
#pragma unroll
    for (int q = 0; q < 8; ++q) f[q] = p[q * P];
  }
}

// Epilogue of one wave: MT x NT accumulator blocks, lane (h, i), register r
// of block (mt, nt) holding C[row0 + mt*32 + (r/4)*8 + h*4 + r%4][col0 + nt*32 + i].
// EPI is a compile-time constant and FULL (every row < M, every column < N)
// drops the per-element checks, so the stores are straight-line code: all
// mask loads are issued before the first store and no store waits on another
// (vmcnt counts stores as well as loads, so a load between two stores would
// make each store wait for the one before it).
template <int EPI, bool FULL, int MT, int NT>
__device__ __forceinline__ void store_acc(const floatx16 (&acc)[MT][NT], float* __restrict__ C, int64_t ldc, int row0,
                                          int col0, int M, int N, const float* __restrict__ bias,
                                          const float* __restrict__ mask, int64_t ldmask, float* __restrict__ pre) {
  const int lane = threadIdx.x & 63, h = lane >> 5, i = lane & 31;
  auto row_of = [&](int mt, int r) { return row0 + mt * 32 + (r >> 2) * 8 + h * 4 + (r & 3); };
  auto col_of = [&](int nt) { return col0 + nt * 32 + i; };
  auto in = [&](int mt, int nt, int r) { return FULL || (row_of(mt, r) < M && col_of(nt) < N); };
  float bv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    bv[nt] = (EPI == ORCA_HIP_EPI_BIAS || EPI == ORCA_HIP_EPI_BIAS_RELU || EPI == ORCA_HIP_EPI_BIAS_RELU_PRE) &&
                     (FULL || col_of(nt) < N)
                 ? bias[col_of(nt)]
                 : 0.0f;
  constexpr bool MASK = EPI == ORCA_HIP_EPI_RELU_MASK || EPI == ORCA_HIP_EPI_RELU_MASK_PRE;
  float mk[MT][NT][MASK ? 16 : 1];
  if (MASK) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mk[mt][nt][r & (MASK ? 15 : 0)] = in(mt, nt, r) ? mask[(int64_t)row_of(mt, r) * ldmask + col_of(nt)] : 0.0f;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = acc[mt][nt][r];
        if (EPI == ORCA_HIP_EPI_BIAS) {
          v = v + bv[nt];
        } else if (EPI == ORCA_HIP_EPI_BIAS_RELU) {
          v = v + bv[nt];
          v = v > 0.0f ? v : 0.0f;
        } else if (EPI == ORCA_HIP_EPI_RELU_MASK) {
          v = mk[mt][nt][r & (MASK ? 15 : 0)] > 0.0f ? v : 0.0f;
        } else if (EPI == ORCA_HIP_EPI_RELU_MASK_PRE) {
          if (in(mt, nt, r)) pre[(int64_t)row_of(mt, r) * ldc + col_of(nt)] = v;
          v = mk[mt][nt][r & (MASK ? 15 : 0)] > 0.0f ? v : 0.0f;
        } else if (EPI == ORCA_HIP_EPI_BIAS_RELU_PRE) {
          v = v + bv[nt];
          if (in(mt, nt, r)) pre[(int64_t)row_of(mt, r) * ldc + col_of(nt)] = v;
          v = v > 0.0f ? v : 0.0f;
        }
        if (in(mt, nt, r)) C[(int64_t)row_of(mt, r) * ldc + col_of(nt)] = v;
      }
}

// The block's epilogue: the kind is uniform, so one specialised store path runs.
template <int MT, int NT>
__device__ __forceinline__ void write_tile(const floatx16 (&acc)[MT][NT], float* C, int64_t ldc, int epi, int row0,
                                           int col0, bool full, const GemmParams& p) {
#define ORCA_STORE_ACC(E)                                                                          \
  do {                                                                                             \
    if (full)                                                                                      \
      store_acc<E, true>(acc, C, ldc, row0, col0, p.M, p.N, p.bias, p.mask, p.ldmask, p.pre);      \
    else                                                                                           \
      store_acc<E, false>(acc, C, ldc, row0, col0, p.M, p.N, p.bias, p.mask, p.ldmask, p.pre);     \
  } while (0)
  switch (epi) {
    case ORCA_HIP_EPI_BIAS: ORCA_STORE_ACC(ORCA_HIP_EPI_BIAS); break;
    case ORCA_HIP_EPI_BIAS_RELU: ORCA_STORE_ACC(ORCA_HIP_EPI_BIAS_RELU); break;
    case ORCA_HIP_EPI_RELU_MASK: ORCA_STORE_ACC(ORCA_HIP_EPI_RELU_MASK); break;
    case ORCA_HIP_EPI_BIAS_RELU_PRE: ORCA_STORE_ACC(ORCA_HIP_EPI_BIAS_RELU_PRE); break;
    case ORCA_HIP_EPI_RELU_MASK_PRE: ORCA_STORE_ACC(ORCA_HIP_EPI_RELU_MASK_PRE); break;
    default: ORCA_STORE_ACC(ORCA_HIP_EPI_NONE); break;
  }
#undef ORCA_STORE_ACC
}

// TA: A stored [K][lda] (A^T), else [M][lda].  TB: B stored [N][ldb] (B^T), else [K][ldb].
// Block tile BM x BN, four waves as 2 x 2, wave tile (BM/2) x (BN/2) = MT x NT
// MFMA 32x32 blocks.
template <int BM, int BN, bool TA, bool TB>
__global__ void __launch_bounds__(NTHREADS) gemm_mfma_f32_kernel(GemmParams p) {
  constexpr int MT = BM / 64, NT = BN / 64;
  constexpr int A_TILE = tile_floats(BM), B_TILE = tile_floats(BN);
  __shared__ __attribute__((aligned(16))) float smem[2][A_TILE + B_TILE];  // [buffer][A | B]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, i = lane & 31;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int bz = blockIdx.z, batch = bz / p.splits, split = bz % p.splits;

  const float* A = p.A + batch * p.sa;
  const float* B = p.B + batch * p.sb;
  const int kb = split * p.k_chunk;
  const int ke = min(p.K, kb + p.k_chunk);
  const int nslabs = (ke - kb + BK - 1) / BK;
  // Interior blocks with aligned operands take the unchecked load path.
  const bool a_in = p.vec_a != 0 && m0 + BM <= p.M;
  const bool b_in = p.vec_b != 0 && n0 + BN <= p.N;
  const bool do_colsum = p.colsum != nullptr && blockIdx.y == 0 && !TB;

  floatx16 acc[MT][NT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;
  float cs = 0.0f;  // bias column sum (threads 0..BN-1 own column n0 + tid)

  // Global loads run two slabs ahead: slab t+2 is fetched into one register
  // stage while slab t is multiplied out of LDS and slab t+1 (the other
  // stage) waits to be stored into the free LDS buffer.  The loop handles two
  // slabs per trip so each register stage is a fixed set of VGPRs.
  auto load = [&](int t, float4 (&ra)[BM / 32], float4 (&rb)[BN / 32]) {
    const int k0 = kb + t * BK;
    const bool kfull = k0 + BK <= ke;
    // A tile: rows m (k-fast) when !TA, rows k (m-fast) when TA.
    load_slab<!TA, BM>(A, p.lda, m0, p.M, k0, ke, a_in && kfull, ra);
    load_slab<TB, BN>(B, p.ldb, n0, p.N, k0, ke, b_in && kfull, rb);
  };
  auto store = [&](float* s, const float4 (&ra)[BM / 32], const float4 (&rb)[BN / 32]) {
    store_slab<!TA, BM>(s, ra);
    store_slab<TB, BN>(s + A_TILE, rb);
  };
  auto compute = [&](const float* s, int t) {
    const float* sa = s;
    const float* sb = s + A_TILE;
    if (do_colsum && tid < BN) {
      const int kv = min(BK, ke - (kb + t * BK));
      for (int k = 0; k < kv; ++k) cs = cs + sb[mn_off<BN>(k) + tid];
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      float fa[MT][8], fb[NT][8];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) read_frag<!TA, BM>(sa, wm * (BM / 2) + mt * 32, half, fa[mt]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) read_frag<TB, BN>(sb, wn * (BN / 2) + nt * 32, half, fb[nt]);
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mt][q], fb[nt][q], acc[mt][nt], 0, 0, 0);
    }
  };

  float4 ra0[BM / 32], rb0[BN / 32], ra1[BM / 32], rb1[BN / 32];
  load(0, ra0, rb0);
  store(smem[0], ra0, rb0);
  if (nslabs > 1) load(1, ra1, rb1);
  __syncthreads();
  int t = 0;
  for (; t + 1 < nslabs; t += 2) {
    // LDS[0] holds slab t, stage 1 holds slab t+1.
    if (t + 2 < nslabs) load(t + 2, ra0, rb0);
    compute(smem[0], t);
    store(smem[1], ra1, rb1);
    __syncthreads();
    // LDS[1] holds slab t+1, stage 0 holds slab t+2.
    if (t + 3 < nslabs) load(t + 3, ra1, rb1);
    compute(smem[1], t + 1);
    if (t + 2 < nslabs) store(smem[0], ra0, rb0);
    __syncthreads();
  }
  if (t < nslabs) compute(smem[0], t);  // odd slab count: the last slab sits in LDS[0]

  // One partial per K-chunk when K is split (reduced in chunk order on the host side).
  if (do_colsum && tid < BN && n0 + tid < p.N) p.colsum[(int64_t)split * p.N + n0 + tid] = cs;

  float* C = p.C + batch * p.sc;
  if (p.splits > 1) C = p.C + (int64_t)bz * p.M * p.N;  // raw partial sums, ld = N
  const int64_t ldc = p.splits > 1 ? p.N : p.ldc;
  const int epi = p.splits > 1 ? ORCA_HIP_EPI_NONE : p.epi;
  write_tile(acc, C, ldc, epi, m0 + wm * (BM / 2), n0 + wn * (BN / 2), m0 + BM <= p.M && n0 + BN <= p.N, p);
}

// ---------------------------------------------------------------------------
// Pipelined kernel for products with M, N, K multiples of 4 and 16-byte
// aligned operands: edge rows are clamped instead of checked, only the last,
// partial K slab is loaded with a check (zero fill), global loads use a
// uniform per-slab base plus 32-bit per-lane offsets, and a
// software pipeline built so each wave always has MFMAs queued while it issues
// memory work.  Per slab t (one register stage R, two LDS buffers L0/L1):
//   region A: store R (slab t+1, loaded one slab earlier) into L[(t+1)%2];
//             load slab t+2 -> R; read the second half-slab fragments of t;
//             32 MFMAs on the first half of t; barrier
//   region B: read the first half-slab fragments of t+1 from L[(t+1)%2]; 32
//             MFMAs on the second half of t.
// The barrier sits between the two MFMA groups, so its wait overlaps queued
// MFMAs, and the next slab's first fragments arrive under the current slab's
// last MFMAs.  sched_group_barrier interleaves one memory instruction after
// each MFMA.  L[(t+1)%2] was last read before the barrier of slab t-1, so the
// store in region A of slab t cannot overwrite fragments still to be read.
template <bool KFAST>
struct BufOperand {
  const char* base;  // uniform: the operand's first element
  uint32_t voff[4];  // byte offsets of this thread's four float4s in slab 0
  uint32_t slab_bytes;

  // Rows (M or N) past `lim_mn` are clamped to the last valid row (or float4),
  // so every load stays inside the operand; they only feed rows / columns of
  // C that are never stored.  lim_mn is a multiple of 4.
  __device__ __forceinline__ void init(const float* b, int64_t ld, int row0_mn, int lim_mn, int kb) {
    base = reinterpret_cast<const char*>(b);
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = tid + NTHREADS * j;
      int64_t off;
      if (KFAST)
        off = (int64_t)min(row0_mn + (idx >> 3), lim_mn - 1) * ld + kb + (idx & 7) * 4;
      else
        off = (int64_t)(kb + (idx >> 5)) * ld + min(row0_mn + (idx & 31) * 4, lim_mn - 4);
      voff[j] = (uint32_t)(off * 4);
    }
    slab_bytes = KFAST ? (uint32_t)(BK * 4) : (uint32_t)(BK * ld * 4);
  }
  // A whole slab: uniform slab base + 32-bit lane offset (global_load_dwordx4).
  __device__ __forceinline__ void load(int t, floatx4 (&r)[4]) const {
    const char* slab = base + (size_t)slab_bytes * (uint32_t)t;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = *reinterpret_cast<const floatx4*>(slab + voff[j]);
  }
  // The chunk's last, partial slab: k offsets >= klen (a multiple of 4) are
  // zero-filled without touching memory.
  __device__ __forceinline__ void load_tail(int t, int klen, floatx4 (&r)[4]) const {
    const char* slab = base + (size_t)slab_bytes * (uint32_t)t;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = t * BK + (KFAST ? (tid & 7) * 4 : (tid >> 5) + 8 * j);
      r[j] = kk < klen ? *reinterpret_cast<const floatx4*>(slab + voff[j]) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
};

template <bool TA, bool TB, bool COLSUM>
__global__ void __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(2))) gemm_mfma_f32_fast_kernel(GemmParams p) {
  constexpr int BM = 128, BN = 128, MT = 2, NT = 2;
  constexpr int A_TILE = tile_floats(BM), B_TILE = tile_floats(BN);
  __shared__ __attribute__((aligned(16))) float smem[2][A_TILE + B_TILE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, i = lane & 31;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int bz = blockIdx.z, batch = bz / p.splits, split = bz % p.splits;
  const int kb = split * p.k_chunk;
  const int klen = min(p.K, kb + p.k_chunk) - kb;
  const int nfull = klen / BK;            // whole slabs
  const int n = (klen + BK - 1) / BK;     // slabs, the last one possibly partial
  const bool do_colsum = COLSUM && blockIdx.y == 0;

  BufOperand<!TA> opa;
  BufOperand<TB> opb;
  opa.init(p.A + batch * p.sa, p.lda, m0, p.M, kb);
  opb.init(p.B + batch * p.sb, p.ldb, n0, p.N, kb);

  floatx16 acc[MT][NT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;
  float cs = 0.0f;

  floatx4 ra[4], rb[4];
  float f0a[MT][8], f0b[NT][8], f1a[MT][8], f1b[NT][8];

  auto store = [&](float* s) {
    store_slab<!TA, BM>(s, ra);
    store_slab<TB, BN>(s + A_TILE, rb);
  };
  auto load = [&](int t) {
    opa.load(t, ra);
    opb.load(t, rb);
  };
  auto load_any = [&](int t) {  // uniform branch: whole or partial slab
    if (t < nfull) {
      load(t);
    } else {
      opa.load_tail(t, klen, ra);
      opb.load_tail(t, klen, rb);
    }
  };
  auto frags = [&](const float* s, int half, float (&fa)[MT][8], float (&fb)[NT][8]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) read_frag<!TA, BM>(s, wm * (BM / 2) + mt * 32, half, fa[mt]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) read_frag<TB, BN>(s + A_TILE, wn * (BN / 2) + nt * 32, half, fb[nt]);
  };
  auto mfma = [&](const float (&fa)[MT][8], const float (&fb)[NT][8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mt][q], fb[nt][q], acc[mt][nt], 0, 0, 0);
  };
  auto colsum = [&](const float* s) {
    if (do_colsum && tid < BN) {
      const float* sb = s + A_TILE;
#pragma unroll
      for (int k = 0; k < BK; ++k) cs = cs + sb[mn_off<BN>(k) + tid];
    }
  };
  // Memory instructions of region A: 8 LDS stores, 8 VMEM loads, the
  // half-slab fragment reads (A k-fast: 4 x b128, m-fast: 16 x b32; same for B).
  constexpr int RD = (!TA ? 4 : 16) + (TB ? 4 : 16);
  auto interleave_a = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    }
#pragma unroll
    for (int j = 0; j < (RD < 16 ? RD : 16); ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, RD > 16 ? 2 : 1, 0);  // DS read
    }
  };
  auto interleave_b = [&]() {
#pragma unroll
    for (int j = 0; j < (RD < 16 ? RD : 16); ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, RD > 16 ? 2 : 1, 0);
    }
  };

  // One slab; P = t % 2 selects the LDS buffer.  FULL: slabs t+1 and t+2
  // exist (no runtime checks inside the straight-line body).
  auto body = [&](auto P_, int t, bool full) {
    constexpr int P = decltype(P_)::value;
    float* lcur = smem[P];
    float* lnxt = smem[P ^ 1];
    if (full) {
      store(lnxt);
      load(t + 2);
      frags(lcur, 1, f1a, f1b);
      mfma(f0a, f0b);
      interleave_a();
    } else {
      if (t + 1 < n) store(lnxt);
      if (t + 2 < n) load_any(t + 2);
      frags(lcur, 1, f1a, f1b);
      mfma(f0a, f0b);
    }
    colsum(lcur);
    __syncthreads();
    if (full) {
      frags(lnxt, 0, f0a, f0b);
      mfma(f1a, f1b);
      interleave_b();
    } else {
      if (t + 1 < n) frags(lnxt, 0, f0a, f0b);
      mfma(f1a, f1b);
    }
  };

  // Prologue: slab 0 into L0 and its first fragments; slab 1 in flight in R.
  load_any(0);
  store(smem[0]);
  if (n > 1) load_any(1);
  __syncthreads();
  frags(smem[0], 0, f0a, f0b);

  // Full bodies load only whole slabs (t + 3 < nfull); the last slabs,
  // including a partial one, run through the checked tail bodies.
  int t = 0;
  for (; t + 3 < nfull; t += 2) {
    body(std::integral_constant<int, 0>{}, t, true);
    body(std::integral_constant<int, 1>{}, t + 1, true);
  }
  if (t < n) body(std::integral_constant<int, 0>{}, t, false);
  if (t + 1 < n) body(std::integral_constant<int, 1>{}, t + 1, false);
  if (t + 2 < n) body(std::integral_constant<int, 0>{}, t + 2, false);
  if (t + 3 < n) body(std::integral_constant<int, 1>{}, t + 3, false);

  if (do_colsum && tid < BN && n0 + tid < p.N) p.colsum[(int64_t)split * p.N + n0 + tid] = cs;

  float* C = p.C + batch * p.sc;
  if (p.splits > 1) C = p.C + (int64_t)bz * p.M * p.N;
  const int64_t ldc = p.splits > 1 ? p.N : p.ldc;
  const int epi = p.splits > 1 ? ORCA_HIP_EPI_NONE : p.epi;
  write_tile(acc, C, ldc, epi, m0 + wm * (BM / 2), n0 + wn * (BN / 2), m0 + BM <= p.M && n0 + BN <= p.N, p);
}

// ---------------------------------------------------------------------------
// Banded weight gradients: C = A^T B with A stored [K][lda] (X of a layer whose
// input count M is not a multiple of 128, e.g. 784 = 28 x 28) and B stored
// [K][ldb] (dY, N a multiple of 128), one K chunk, pipelined as the kernel
// above.  With 128 x 128 tiles M = 784 takes 7 tile rows, the last one 16/128
// full, and each busy CU runs four MFMA 32 x 32 blocks per SIMD and k step.
// Both forms below use 32 x 32 blocks for 96 rows of a block's 128 columns
// (wave w: columns 32 w .. 32 w + 31, three blocks) and 16 x 16 x 4 blocks for
// 16 more rows:
//   ROWS112 (M = 112 R, R <= 7): block (c, r) owns rows 112 r .. 112 r + 111;
//     wave w's last 16 rows are two 16 x 16 blocks with the full k range.  7 x
//     N/128 blocks (224 for N = 4096, CUs left free for work beside it, as the
//     128 x 128 grid leaves them), 3 x 1024 + 2 x 256 MFMA cycles per SIMD and
//     slab instead of 4 x 1024.
//   EIGHT (M = 768 + E, 4 <= E <= 16): block (c, r), r < 8, owns rows 96 r ..
//     96 r + 95 and the E leftover rows 768 .. M - 1 of its 16 columns 128 c +
//     16 r .. + 15: one 16 x 16 block whose k range the four waves share (wave
//     w: k = 8 w .. 8 w + 7 of every slab), the partial sums added in wave order
//     at the end.  8 x N/128 blocks (256 for N = 4096: every CU), 3 x 1024 + 64
//     MFMA cycles per SIMD and slab.
// A's LDS rows hold the 96 band values, then the 16 others (pitch 112).
// COLSUM: the bias gradient, colsum[n] = sum of B's column n in ascending k from
// +0 (the additions of sum_to_shape, so the same bits).  EIGHT: on a fifth wave
// per block that does nothing else, the 16 columns 128 c + 16 r .. + 15; it
// reads each slab's B tile between the same barriers as the MFMA waves, and its
// dependent adds issue on SIMD 0 beside wave 0's matrix instructions.  ROWS112
// (whose waves need more than half a SIMD's registers, so a fifth one does not
// fit): one more row of N/128 blocks, each summing its 128 columns straight from
// global memory, one per thread, on CUs the product's blocks leave free.
constexpr int BAND_M = 96, BAND_EX = 16, BAND_AP = BAND_M + BAND_EX, BAND_ROWS = 8 * BAND_M;
constexpr int BAND_EIGHT = 0, BAND_ROWS112 = 1;

typedef float floatx2 __attribute__((ext_vector_type(2)));

// A of a banded product: per slab and thread three float4s of the block's 96
// band rows (32 k rows x 24 float4) and one float2 of its 16 other rows (32 x 8)
// starting at m_ex; rows past M - 1 repeat the last valid pair (never stored).
struct BandOperandA {
  const char* base;
  uint32_t voff[4];
  uint32_t slab_bytes;
  __device__ __forceinline__ void init(const float* a, int64_t lda, int m0, int m_ex, int M) {
    base = reinterpret_cast<const char*>(a);
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int idx = tid + NTHREADS * j;
      voff[j] = (uint32_t)(((int64_t)(idx / 24) * lda + m0 + (idx % 24) * 4) * 4);
    }
    voff[3] = (uint32_t)(((int64_t)(tid >> 3) * lda + min(m_ex + (tid & 7) * 2, M - 2)) * 4);
    slab_bytes = (uint32_t)(BK * lda * 4);
  }
  __device__ __forceinline__ void load(int t, floatx4 (&r)[3], floatx2& e) const {
    const char* slab = base + (size_t)slab_bytes * (uint32_t)t;
#pragma unroll
    for (int j = 0; j < 3; ++j) r[j] = *reinterpret_cast<const floatx4*>(slab + voff[j]);
    e = *reinterpret_cast<const floatx2*>(slab + voff[3]);
  }
  // The last, partial slab: k offsets >= klen are zero-filled without touching memory.
  __device__ __forceinline__ void load_tail(int t, int klen, floatx4 (&r)[3], floatx2& e) const {
    const char* slab = base + (size_t)slab_bytes * (uint32_t)t;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int kk = t * BK + (tid + NTHREADS * j) / 24;
      r[j] = kk < klen ? *reinterpret_cast<const floatx4*>(slab + voff[j]) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int kk = t * BK + (tid >> 3);
    e = kk < klen ? *reinterpret_cast<const floatx2*>(slab + voff[3]) : floatx2{0.0f, 0.0f};
  }
};

template <int MODE, bool COLSUM>
__global__ void __launch_bounds__(COLSUM && MODE == BAND_EIGHT ? NTHREADS + 64 : NTHREADS)
__attribute__((amdgpu_waves_per_eu(MODE == BAND_EIGHT ? 2 : 1))) gemm_tn_band_kernel(GemmParams p) {
  constexpr bool EIGHT = MODE == BAND_EIGHT;
  constexpr int MT = BAND_M / 32;
  constexpr int NX = EIGHT ? 1 : 2;  // 16 x 16 blocks per wave
  constexpr int A_TILE = BK * BAND_AP + MN_GAP, B_TILE = BK * 128 + MN_GAP;
  __shared__ __attribute__((aligned(16))) float smem[2][A_TILE + B_TILE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int band = blockIdx.y, n0 = blockIdx.x * 128;
  const int m0 = EIGHT ? band * BAND_M : band * BAND_AP;
  const int m_ex = EIGHT ? BAND_ROWS : m0 + BAND_M;  // first of the 16 other rows
  const int klen = p.K;
  const int nfull = klen / BK;
  const int n = (klen + BK - 1) / BK;

  if (EIGHT && COLSUM && wave == 4) {
    // Slab t sits in smem[t % 2] from barrier t (the prologue's is barrier 0)
    // until barrier t + 1, after which region A of slab t + 1 overwrites it.
    // The MFMA waves pass n + 3 barriers: the prologue's, one per slab and two
    // around the leftover-row reduction.  Lanes 16 .. 63 repeat lanes 0 .. 15.
    const int c0 = 16 * band + (lane & 15);
    float cs = 0.0f;
    __syncthreads();
    for (int t = 0; t < n; ++t) {
      const float* sb = smem[t & 1] + A_TILE + c0;
#pragma unroll
      for (int k = 0; k < BK; ++k) cs = cs + sb[mn_off<128>(k)];
      __syncthreads();
    }
    if (lane < 16) p.colsum[n0 + c0] = cs;
    __syncthreads();
    __syncthreads();
    return;
  }
  if (!EIGHT && COLSUM && m0 >= p.M) {
    // The column-sum row: threads 0 .. 127 each add one column of B in row order,
    // the next 16 rows' loads in flight while 16 are added.
    if (tid < 128) {
      const float* src = p.B + n0 + tid;
      float cs = 0.0f, v[16], w[16];
      int k = 0;
      auto fetch = [&](float (&d)[16], int k0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) d[u] = src[(int64_t)(k0 + u) * p.ldb];
      };
      if (klen >= 16) fetch(v, 0);
      for (; k + 32 <= klen; k += 32) {
        fetch(w, k + 16);
#pragma unroll
        for (int u = 0; u < 16; ++u) cs = cs + v[u];
        if (k + 48 <= klen) fetch(v, k + 32);
#pragma unroll
        for (int u = 0; u < 16; ++u) cs = cs + w[u];
      }
      if (k + 16 <= klen) {
#pragma unroll
        for (int u = 0; u < 16; ++u) cs = cs + v[u];
        k += 16;
      }
      for (; k < klen; ++k) cs = cs + src[(int64_t)k * p.ldb];
      p.colsum[n0 + tid] = cs;
    }
    return;
  }

  BandOperandA opa;
  BufOperand<false> opb;
  opa.init(p.A, p.lda, m0, m_ex, p.M);
  opb.init(p.B, p.ldb, n0, p.N, 0);

  floatx16 acc[MT][1];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][0][r] = 0.0f;
  floatx4 accx[NX];
#pragma unroll
  for (int x = 0; x < NX; ++x) accx[x] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  floatx4 ra[3], rb[4];
  floatx2 re;
  float f0a[MT][8], f0b[8], f1a[MT][8], f1b[8];
  // 16 x 16 fragments of a half slab: EIGHT one step (A, B), ROWS112 four
  // steps of A and of the wave's two column blocks of B.
  constexpr int XS = EIGHT ? 1 : 4;
  float x0a[XS], x0b[XS][NX], x1a[XS], x1b[XS][NX];

  // LDS offsets of this thread's A stores (k row, column).
  int soff[4];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int idx = tid + NTHREADS * j;
    soff[j] = mn_off<BAND_AP>(idx / 24) + (idx % 24) * 4;
  }
  soff[3] = mn_off<BAND_AP>(tid >> 3) + BAND_M + (tid & 7) * 2;
  // 16 x 16 x 4 lane layout: lane (g, c) = (lane / 16, lane % 16) holds A[row c][k g]
  // and B[k g][column c]; EIGHT's k is 8 w + 4 half + g, ROWS112's 16 half + 4 s + g.
  const int xg = lane >> 4, xc = lane & 15;
  const int xcol = EIGHT ? 16 * band + xc : 32 * wave + xc;  // column within the tile

  auto store = [&](float* s) {
#pragma unroll
    for (int j = 0; j < 3; ++j) *reinterpret_cast<floatx4*>(s + soff[j]) = ra[j];
    *reinterpret_cast<floatx2*>(s + soff[3]) = re;
    store_slab<false, 128>(s + A_TILE, rb);
  };
  auto load = [&](int t) {
    opa.load(t, ra, re);
    opb.load(t, rb);
  };
  auto load_any = [&](int t) {  // uniform branch: whole or partial slab
    if (t < nfull) {
      load(t);
    } else {
      opa.load_tail(t, klen, ra, re);
      opb.load_tail(t, klen, rb);
    }
  };
  auto frags = [&](const float* s, int half, float (&fa)[MT][8], float (&fb)[8], float (&xa)[XS],
                   float (&xb)[XS][NX]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) read_frag<false, BAND_AP>(s, mt * 32, half, fa[mt]);
    read_frag<false, 128>(s + A_TILE, wave * 32, half, fb);
#pragma unroll
    for (int st = 0; st < XS; ++st) {
      const int kk = EIGHT ? 8 * wave + 4 * half + xg : 16 * half + 4 * st + xg;
      xa[st] = s[mn_off<BAND_AP>(kk) + BAND_M + xc];
#pragma unroll
      for (int x = 0; x < NX; ++x) xb[st][x] = s[A_TILE + mn_off<128>(kk) + xcol + 16 * x];
    }
  };
  auto mfma = [&](const float (&fa)[MT][8], const float (&fb)[8], const float (&xa)[XS], const float (&xb)[XS][NX]) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mt][q], fb[q], acc[mt][0], 0, 0, 0);
      if (!EIGHT && (q & 1)) {  // ROWS112: the 16 x 16 steps spread among the 32 x 32 ones
#pragma unroll
        for (int x = 0; x < NX; ++x)
          accx[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[q >> 1], xb[q >> 1][x], accx[x], 0, 0, 0);
      }
    }
    if (EIGHT) accx[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[0], xb[0][0], accx[0], 0, 0, 0);
  };
  // Region A: 8 LDS stores, 8 VMEM loads and the half-slab fragments among its
  // matrix instructions (EIGHT: 25 and 34 scalar LDS reads; ROWS112: 32 and 44).
  constexpr int NMF = EIGHT ? 25 : 32, NRD = EIGHT ? 34 : 44;
  auto interleave_a = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
#pragma unroll
    for (int j = 0; j < NMF - 16; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, (NRD - 32 + NMF - 17) / (NMF - 16), 0);
    }
  };
  auto interleave_b = [&]() {
#pragma unroll
    for (int j = 0; j < (NRD + 1) / 2; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };

  auto body = [&](auto P_, int t, bool full) {
    constexpr int P = decltype(P_)::value;
    float* lcur = smem[P];
    float* lnxt = smem[P ^ 1];
    if (full) {
      store(lnxt);
      load(t + 2);
      frags(lcur, 1, f1a, f1b, x1a, x1b);
      mfma(f0a, f0b, x0a, x0b);
      interleave_a();
    } else {
      if (t + 1 < n) store(lnxt);
      if (t + 2 < n) load_any(t + 2);
      frags(lcur, 1, f1a, f1b, x1a, x1b);
      mfma(f0a, f0b, x0a, x0b);
    }
    __syncthreads();
    if (full) {
      frags(lnxt, 0, f0a, f0b, x0a, x0b);
      mfma(f1a, f1b, x1a, x1b);
      interleave_b();
    } else {
      if (t + 1 < n) frags(lnxt, 0, f0a, f0b, x0a, x0b);
      mfma(f1a, f1b, x1a, x1b);
    }
  };

  load_any(0);
  store(smem[0]);
  if (n > 1) load_any(1);
  __syncthreads();
  frags(smem[0], 0, f0a, f0b, x0a, x0b);

  int t = 0;
  for (; t + 3 < nfull; t += 2) {
    body(std::integral_constant<int, 0>{}, t, true);
    body(std::integral_constant<int, 1>{}, t + 1, true);
  }
  if (t < n) body(std::integral_constant<int, 0>{}, t, false);
  if (t + 1 < n) body(std::integral_constant<int, 1>{}, t + 1, false);
  if (t + 2 < n) body(std::integral_constant<int, 0>{}, t + 2, false);
  if (t + 3 < n) body(std::integral_constant<int, 1>{}, t + 3, false);

  // The 16 x 16 blocks: lane (g, c) holds rows 4 g .. 4 g + 3 of column c.
  if (EIGHT) {  // the four waves' partial sums, added in wave order
    __syncthreads();
    float* red = smem[0];
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave * 256 + (4 * xg + j) * 16 + xc] = accx[0][j];
    __syncthreads();
    const int row = BAND_ROWS + (tid >> 4);
    const float v = ((red[tid] + red[256 + tid]) + red[512 + tid]) + red[768 + tid];
    if (row < p.M) p.C[(int64_t)row * p.ldc + n0 + 16 * band + (tid & 15)] = v;
  } else {
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        p.C[(int64_t)(m_ex + 4 * xg + j) * p.ldc + n0 + xcol + 16 * x] = accx[x][j];
  }
  write_tile(acc, p.C, p.ldc, p.epi, m0, n0 + 32 * wave, true, p);
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
  float* pre;            // EPI_BIAS_RELU_PRE: acc + bias; EPI_RELU_MASK_PRE: acc (with ldc)
  const float* cs_part;  // per-split column sums [splits][N] of a folded bias gradient, or null
  float* cs_out;         // their in-order sum [N]
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
    } else if (p.epi == ORCA_HIP_EPI_BIAS_RELU_PRE) {
      v = v + p.bias[col];
      p.pre[b * p.sc + (int64_t)row * p.ldc + col] = v;
      v = v > 0.0f ? v : 0.0f;
    } else if (p.epi == ORCA_HIP_EPI_RELU_MASK_PRE) {
      p.pre[b * p.sc + (int64_t)row * p.ldc + col] = v;
      v = p.mask[(int64_t)row * p.ldmask + col] > 0.0f ? v : 0.0f;
    }
    p.C[b * p.sc + (int64_t)row * p.ldc + col] = v;
  }
}

// The same sums four columns at a time: N, ldc, sc and ldmask are multiples of
// 4 and C, the partials and the mask are 16-byte aligned; total4 < 2^31 so the
// float4 index and its row / column split stay 32-bit.  Each float4 component
// takes exactly the scalar kernel's adds, in the same split order.  With a
// folded bias gradient the first N threads also sum its per-split column sums
// in split order (what colsum_split_reduce_kernel does, without its launch).
__global__ void splitk_reduce_vec_kernel(SplitReduceParams p, uint32_t total4) {
  const uint32_t n4 = (uint32_t)p.N >> 2, mn4 = (uint32_t)p.M * n4;
  const size_t mn = (size_t)p.M * p.N;
  const uint32_t stride = gridDim.x * blockDim.x;
  if (p.cs_part) {
    for (uint32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < (uint32_t)p.N; n += stride) {
      float v = p.cs_part[n];
      for (int s = 1; s < p.splits; ++s) v = v + p.cs_part[(size_t)s * p.N + n];
      p.cs_out[n] = v;
    }
  }
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total4; idx += stride) {
    const uint32_t b = idx / mn4, rem4 = idx - b * mn4;
    const uint32_t row = rem4 / n4, col = (rem4 - row * n4) * 4;
    const float* w = p.ws + b * p.splits * mn + (size_t)rem4 * 4;
    floatx4 v = *reinterpret_cast<const floatx4*>(w);
#pragma unroll 4
    for (int s = 1; s < p.splits; ++s) v = v + *reinterpret_cast<const floatx4*>(w + s * mn);
    if (p.epi == ORCA_HIP_EPI_BIAS || p.epi == ORCA_HIP_EPI_BIAS_RELU || p.epi == ORCA_HIP_EPI_BIAS_RELU_PRE) {
      const floatx4 bv = {p.bias[col], p.bias[col + 1], p.bias[col + 2], p.bias[col + 3]};
      v = v + bv;
      if (p.epi == ORCA_HIP_EPI_BIAS_RELU_PRE)
        *reinterpret_cast<floatx4*>(p.pre + b * p.sc + (int64_t)row * p.ldc + col) = v;
      if (p.epi != ORCA_HIP_EPI_BIAS) {
        v.x = v.x > 0.0f ? v.x : 0.0f;
        v.y = v.y > 0.0f ? v.y : 0.0f;
        v.z = v.z > 0.0f ? v.z : 0.0f;
        v.w = v.w > 0.0f ? v.w : 0.0f;
      }
    } else if (p.epi == ORCA_HIP_EPI_RELU_MASK || p.epi == ORCA_HIP_EPI_RELU_MASK_PRE) {
      if (p.epi == ORCA_HIP_EPI_RELU_MASK_PRE)
        *reinterpret_cast<floatx4*>(p.pre + b * p.sc + (int64_t)row * p.ldc + col) = v;
      const floatx4 m = *reinterpret_cast<const floatx4*>(p.mask + (int64_t)row * p.ldmask + col);
      v.x = m.x > 0.0f ? v.x : 0.0f;
      v.y = m.y > 0.0f ? v.y : 0.0f;
      v.z = m.z > 0.0f ? v.z : 0.0f;
      v.w = m.w > 0.0f ? v.w : 0.0f;
    }
    *reinterpret_cast<floatx4*>(p.C + b * p.sc + (int64_t)row * p.ldc + col) = v;
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

// Skinny products (few rows, short K, A row-major): C[M, N] = A[M, K] op(B),
// op(B) = B [K][N] (TB = false) or B stored [N][K] (TB = true).  One 32 x 32
// tile of C per block of SK_WAVES waves, so an M = 256, N = 1024 product is
// 256 blocks with no K split.  Wave w multiplies the k range [w kq, (w + 1) kq)
// straight from global memory in MFMA fragment order: for each group of 8 k,
// lane (i, h) = (l % 32, l / 32) holds A[m0 + i][k8 + 4h .. + 3] (one float4)
// and the four B values of the same k for column n0 + i, and MFMA step j
// (0..3) multiplies k = k8 + 4h + j.  Steps 0 and 2 accumulate into one
// register block and 1 and 3 into another (two independent chains), added at
// the end; the waves' tiles are summed through LDS in wave order.  SK_DEPTH
// groups of loads are in flight while one is multiplied.
// Rows and columns past M / N are clamped to the last valid one (never
// stored); k past the wave's range reads as zero.
struct SkinnyParams {
  const float* A;
  const float* B;
  float* C;
  int64_t lda, ldb, ldc;
  int M, N, K, kq;
  int vec;  // A (and B when TB) rows 16-byte aligned with lda, ldb multiples of 4
  int epi;
  const float* bias;
  const float* mask;
  int64_t ldmask;
  float* pre;  // EPI_BIAS_RELU_PRE: acc + bias; EPI_RELU_MASK_PRE: acc (with ldc)
};

template <bool TB>
__device__ __forceinline__ void skinny_load(const SkinnyParams& p, int row_a, int col_b, int k, int kend, floatx4& a,
                                            floatx4& b) {
  if (p.vec && k + 4 <= kend) {
    a = *reinterpret_cast<const floatx4*>(p.A + (int64_t)row_a * p.lda + k);
    if (TB) {
      b = *reinterpret_cast<const floatx4*>(p.B + (int64_t)col_b * p.ldb + k);
    } else {
      const float* bp = p.B + (int64_t)k * p.ldb + col_b;
      b = floatx4{bp[0], bp[p.ldb], bp[2 * p.ldb], bp[3 * p.ldb]};
    }
  } else {
    float av[4], bv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = k + e < kend;
      av[e] = in ? p.A[(int64_t)row_a * p.lda + k + e] : 0.0f;
      bv[e] = in ? (TB ? p.B[(int64_t)col_b * p.ldb + k + e] : p.B[(int64_t)(k + e) * p.ldb + col_b]) : 0.0f;
    }
    a = floatx4{av[0], av[1], av[2], av[3]};
    b = floatx4{bv[0], bv[1], bv[2], bv[3]};
  }
}

constexpr int SK_WAVES = 8;   // waves per skinny block, each an eighth of K
constexpr int SK_DEPTH = 4;   // 8-k groups of loads in flight per wave

template <bool TB>
__global__ void __launch_bounds__(64 * SK_WAVES) gemm_skinny_kernel(SkinnyParams p) {
  __shared__ float red[SK_WAVES][32 * 32];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, i = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int row_a = min(m0 + i, p.M - 1), col_b = min(n0 + i, p.N - 1);
  const int kbeg = w * p.kq, kend = min(p.K, kbeg + p.kq);
  floatx16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc0[r] = 0.0f;
    acc1[r] = 0.0f;
  }
  if (kbeg < kend) {
    floatx4 a[SK_DEPTH], b[SK_DEPTH];
#pragma unroll
    for (int d = 0; d < SK_DEPTH; ++d) skinny_load<TB>(p, row_a, col_b, kbeg + 8 * d + 4 * h, kend, a[d], b[d]);
    for (int base = kbeg; base < kend; base += 8 * SK_DEPTH) {
#pragma unroll
      for (int d = 0; d < SK_DEPTH; ++d) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d].x, b[d].x, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d].y, b[d].y, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d].z, b[d].z, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d].w, b[d].w, acc1, 0, 0, 0);
        // refill this slot with the group SK_DEPTH ahead (zeros past the wave's range)
        skinny_load<TB>(p, row_a, col_b, base + 8 * (d + SK_DEPTH) + 4 * h, kend, a[d], b[d]);
      }
    }
  }
  // register r of lane (i, h) holds C[(r / 4) * 8 + h * 4 + r % 4][i] of this wave's tile
#pragma unroll
  for (int r = 0; r < 16; ++r) red[w][((r >> 2) * 8 + h * 4 + (r & 3)) * 32 + i] = acc0[r] + acc1[r];
  __syncthreads();
  // thread t < 256: row t / 8, columns 4 (t % 8) .. + 3
  if (tid >= 256) return;
  const int row = tid >> 3, c4 = (tid & 7) * 4;
  const int m = m0 + row;
  if (m >= p.M) return;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int o = row * 32 + c4 + e;
    float t = red[0][o];
#pragma unroll
    for (int q = 1; q < SK_WAVES; ++q) t = t + red[q][o];
    v[e] = t;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = n0 + c4 + e;
    if (n >= p.N) break;
    float x = v[e];
    if (p.epi == ORCA_HIP_EPI_BIAS) {
      x = x + p.bias[n];
    } else if (p.epi == ORCA_HIP_EPI_BIAS_RELU) {
      x = x + p.bias[n];
      x = x > 0.0f ? x : 0.0f;
    } else if (p.epi == ORCA_HIP_EPI_RELU_MASK) {
      x = p.mask[(int64_t)m * p.ldmask + n] > 0.0f ? x : 0.0f;
    } else if (p.epi == ORCA_HIP_EPI_BIAS_RELU_PRE) {
      x = x + p.bias[n];
      p.pre[(int64_t)m * p.ldc + n] = x;
      x = x > 0.0f ? x : 0.0f;
    } else if (p.epi == ORCA_HIP_EPI_RELU_MASK_PRE) {
      p.pre[(int64_t)m * p.ldc + n] = x;
      x = p.mask[(int64_t)m * p.ldmask + n] > 0.0f ? x : 0.0f;
    }
    p.C[(int64_t)m * p.ldc + n] = x;
  }
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// Profiler names: "gemm_<op(A)><op(B)>", "_pipe" for the pipelined 128 x 128 kernel.
// ---------------------------------------------------------------------------
// Narrow products, which tile badly on the matrix cores: N <= 16 with a
// row-major B (X W of a classifier head, X^T dY of its weight gradient) and
// K <= 16 against B^T (dY W^T back through it).  They are memory-bound: each
// streams its large operand once, with fp32 FMAs on the vector units.  The
// small operand is staged through LDS with coalesced loads, padded with zeros
// to NP = 4, 8 or 16 columns (padding terms are never stored), and every sum
// has a fixed order, so results do not depend on timing.
constexpr int NW_MAX = 16;     // largest narrow N (NN, TN) or K (NT)
constexpr int NW_THREADS = 256;
constexpr int NN_ROWS = 16;    // rows of C per NN block: 4 per wave
constexpr int NN_CHUNK = 256;  // k per NN pass: lane l takes k0 + l + 64 j, j < 4
constexpr int TN_CHUNK = 64;   // k rows of A per TN pass: 16 per wave
constexpr int NW_MAX_SLICES = 64;
constexpr int NT_ROW_GROUP = 16;  // rows of an NT block whose mask values are loaded together

inline int narrow_pad(size_t n) { return n <= 4 ? 4 : n <= 8 ? 8 : 16; }

// C[M x N] = A[M x K] B[K x N], N <= NP.  Block (x, y): K slice x, rows 16 y ..
// 16 y + 15, wave w owning rows 16 y + 4 w .. + 3.  Per 256-k chunk the block
// stages B's rows in LDS (row stride NP + 4 floats: conflict-free float4 reads
// for NP >= 8), lane l reads A at k0 + l + 64 j (coalesced) and accumulates
// 4 x NP sums in k order; then the 64 lanes of each output are added in lane
// order.  The next chunk's loads are in flight while a chunk is computed.
// With one slice the result is C, else part[slice][M][N] (ldo = N), summed in
// slice order by gemm_narrow_reduce_kernel.
template <int NP>
__global__ void __launch_bounds__(NW_THREADS) gemm_nn_narrow_kernel(const float* __restrict__ A, int64_t lda,
                                                                     const float* __restrict__ B, int64_t ldb,
                                                                     float* __restrict__ out, int64_t ldo, int M, int N,
                                                                     int K, int kslice, const float* __restrict__ bias) {
  constexpr int BS = NP == 4 ? 4 : NP + 4;
  constexpr int RED = 4 * NP + 1;
  constexpr int SMEM = NN_CHUNK * BS > 4 * 64 * RED ? NN_CHUNK * BS : 4 * 64 * RED;
  constexpr int PER_T = NN_CHUNK * NP / NW_THREADS;  // staged B values per thread
  __shared__ __align__(16) float smem[SMEM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int k_beg = blockIdx.x * kslice, k_end = min(K, k_beg + kslice);
  float* o = out + (int64_t)blockIdx.x * M * N;  // this slice's partials (C itself with one slice)
  float bv[PER_T], a[4][4];
  // B values first: the LDS writes wait for them and not for A
  auto load = [&](int k0, int m0) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int e = tid + i * NW_THREADS, r = e / NP, n = e % NP, k = k0 + r;
      bv[i] = k < k_end && n < N ? B[(int64_t)k * ldb + n] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + lane + 64 * j;
        a[r][j] = m0 + r < M && k < k_end ? A[(int64_t)(m0 + r) * lda + k] : 0.0f;
      }
  };
  for (int g = blockIdx.y; g * NN_ROWS < M; g += gridDim.y) {
    const int m0 = g * NN_ROWS + 4 * w;  // this wave's first row
    float acc[4][NP];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int n = 0; n < NP; ++n) acc[r][n] = 0.0f;
    load(k_beg, m0);
    for (int k0 = k_beg; k0 < k_end; k0 += NN_CHUNK) {
      __syncthreads();  // the previous chunk's (or row group's) LDS reads are done
#pragma unroll
      for (int i = 0; i < PER_T; ++i) {
        const int e = tid + i * NW_THREADS;
        smem[(e / NP) * BS + e % NP] = bv[i];
      }
      float ac[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) ac[r][j] = a[r][j];
      __syncthreads();
      if (k0 + NN_CHUNK < k_end) load(k0 + NN_CHUNK, m0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* brow = smem + (lane + 64 * j) * BS;
        float b[NP];
#pragma unroll
        for (int q = 0; q < NP / 4; ++q) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(brow + 4 * q);
          b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int n = 0; n < NP; ++n) acc[r][n] = fmaf(ac[r][j], b[n], acc[r][n]);
      }
    }
    __syncthreads();  // all B reads done before the partials overwrite the staging area
    float* red = smem + w * 64 * RED;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int n = 0; n < NP; ++n) red[lane * RED + r * NP + n] = acc[r][n];
    __syncthreads();
    for (int q = lane; q < 4 * NP; q += 64) {
      const int r = q / NP, n = q % NP;
      if (m0 + r < M && n < N) {
        float sum = red[q];
        for (int t = 1; t < 64; ++t) sum = sum + red[t * RED + q];
        if (bias) sum = sum + bias[n];  // the bias epilogue (one slice only)
        o[(int64_t)(m0 + r) * ldo + n] = sum;
      }
    }
  }
}

// C[M x N] = A[M x K] B^T with B stored [N][K], K <= KP.  Thread t of block
// (x, y) owns column 256 x + t (its row of B in registers) for rows
// rows_per_block y .. + rows_per_block - 1, whose A values are staged in LDS
// (`as`, 64 x KP floats) per pass of 64 rows and read as broadcasts.  Each output
// is a dot product over k in order; a wave's stores cover 64 consecutive columns
// of a row.
template <int KP>
__device__ __forceinline__ void nt_smallk_block(int bx, int by, float* as, const float* __restrict__ A, int64_t lda,
                                                const float* __restrict__ B, int64_t ldb, float* __restrict__ C,
                                                int64_t ldc, int M, int N, int K, int rows_per_block,
                                                const float* __restrict__ mask, int64_t ldmask,
                                                float* __restrict__ pre) {
  constexpr int PASS = 64;
  const int tid = threadIdx.x;
  const int n = bx * NW_THREADS + tid;
  float b[KP];
#pragma unroll
  for (int k = 0; k < KP; ++k) b[k] = n < N && k < K ? B[(int64_t)n * ldb + k] : 0.0f;
  const int m_beg = by * rows_per_block, m_end = min(M, m_beg + rows_per_block);
  for (int p0 = m_beg; p0 < m_end; p0 += PASS) {
    const int cnt = min(PASS, m_end - p0);
    float av[PASS * KP / NW_THREADS];
#pragma unroll
    for (int i = 0; i < PASS * KP / NW_THREADS; ++i) {
      const int e = tid + i * NW_THREADS, t = e / KP, k = e % KP;
      av[i] = t < cnt && k < K ? A[(int64_t)(p0 + t) * lda + k] : 0.0f;
    }
    __syncthreads();  // the previous pass's LDS reads are done
#pragma unroll
    for (int i = 0; i < PASS * KP / NW_THREADS; ++i) as[tid + i * NW_THREADS] = av[i];
    __syncthreads();
    if (n >= N) continue;
    float* dst = C + (int64_t)p0 * ldc + n;
    // Rows in groups of 16, the group's mask values loaded before its first row is
    // computed (a load per row ahead of each store would chain the rows on memory), and
    // the next group's while this one is computed.
    float mk[NT_ROW_GROUP], mk_next[NT_ROW_GROUP];
    auto load_mask = [&](int t0, float (&m)[NT_ROW_GROUP]) {
#pragma unroll
      for (int j = 0; j < NT_ROW_GROUP; ++j)
        m[j] = t0 + j < cnt ? mask[(int64_t)(p0 + t0 + j) * ldmask + n] : 0.0f;
    };
    if (mask) load_mask(0, mk);
    for (int t0 = 0; t0 < cnt; t0 += NT_ROW_GROUP) {
      if (mask && t0 + NT_ROW_GROUP < cnt) load_mask(t0 + NT_ROW_GROUP, mk_next);
#pragma unroll
      for (int j = 0; j < NT_ROW_GROUP; ++j) {
        const int t = t0 + j;
        if (t >= cnt) break;
        float a[KP];
#pragma unroll
        for (int q = 0; q < KP / 4; ++q) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(as + t * KP + 4 * q);
          a[4 * q] = v.x, a[4 * q + 1] = v.y, a[4 * q + 2] = v.z, a[4 * q + 3] = v.w;
        }
        float c = 0.0f;
#pragma unroll
        for (int k = 0; k < KP; ++k) c = fmaf(a[k], b[k], c);
        if (pre) pre[(int64_t)(p0 + t) * ldc + n] = c;  // the product itself, kept beside the masked one
        if (mask) c = mk[j] > 0.0f ? c : 0.0f;          // the ReLU-mask epilogue
        dst[(int64_t)t * ldc] = c;
      }
      if (mask) {
#pragma unroll
        for (int j = 0; j < NT_ROW_GROUP; ++j) mk[j] = mk_next[j];
      }
    }
  }
}

template <int KP>
__global__ void __launch_bounds__(NW_THREADS) gemm_nt_smallk_kernel(const float* __restrict__ A, int64_t lda,
                                                                     const float* __restrict__ B, int64_t ldb,
                                                                     float* __restrict__ C, int64_t ldc, int M, int N,
                                                                     int K, int rows_per_block,
                                                                     const float* __restrict__ mask, int64_t ldmask,
                                                                     float* __restrict__ pre) {
  __shared__ __align__(16) float as[64 * KP];
  nt_smallk_block<KP>(blockIdx.x, blockIdx.y, as, A, lda, B, ldb, C, ldc, M, N, K, rows_per_block, mask, ldmask, pre);
}

// C[M x N] = A^T B with A stored [K][M], B [K][N], N <= NP.  Block (x, y):
// columns 64 COLS x .. + 64 COLS - 1 (COLS per lane: a float4 or float2 of an A
// row when aligned) and K slice y.  Per 64-row chunk the block stages B's rows in
// LDS (`bs`, TN_CHUNK x NP floats) and wave w takes chunk rows 16 w .. 16 w + 15;
// with PIPE the next chunk's loads are in flight while a chunk is computed.  The
// lane's sums run in k order, then the 4 waves are added in wave order: waves 1, 2
// and 3 hand theirs to wave 0 in turn through `red` (64 x (COLS NP + 1) floats), and
// wave 0 stores.  Each output's sums are the same for every COLS and PIPE.  With one
// slice the result is C, else part[slice][M][N] (ldo = N).
template <int NP, int COLS, bool PIPE>
__device__ __forceinline__ void tn_narrow_block(int bx, int by, float* bs, float* red, const float* __restrict__ A,
                                                int64_t lda, const float* __restrict__ B, int64_t ldb,
                                                float* __restrict__ out, int64_t ldo, int M, int N, int K, int kslice,
                                                int vec_a) {
  static_assert(COLS == 2 || COLS == 4, "two or four columns per lane");
  constexpr int RED = COLS * NP + 1;
  constexpr int PER_WAVE = TN_CHUNK / 4;
  constexpr int PER_T = TN_CHUNK * NP / NW_THREADS;  // staged B values per thread
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int m0 = bx * 64 * COLS + COLS * lane;
  const int k_beg = by * kslice, k_end = min(K, k_beg + kslice);
  const bool vec = vec_a && m0 + COLS - 1 < M;
  float acc[COLS][NP];
#pragma unroll
  for (int i = 0; i < COLS; ++i)
#pragma unroll
    for (int n = 0; n < NP; ++n) acc[i][n] = 0.0f;
  float bv[PER_T], a[PER_WAVE][COLS];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int e = tid + i * NW_THREADS, r = e / NP, n = e % NP, k = k0 + r;
      bv[i] = k < k_end && n < N ? B[(int64_t)k * ldb + n] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < PER_WAVE; ++r) {
      const int k = k0 + PER_WAVE * w + r;
      const float* row = A + (int64_t)k * lda + m0;
      if (k < k_end && vec) {
        if (COLS == 4) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(row);
          a[r][0] = v.x, a[r][1] = v.y, a[r][COLS > 2 ? 2 : 0] = v.z, a[r][COLS > 3 ? 3 : 0] = v.w;
        } else {
          const float2 v = *reinterpret_cast<const float2*>(row);
          a[r][0] = v.x, a[r][1] = v.y;
        }
      } else {
#pragma unroll
        for (int i = 0; i < COLS; ++i) a[r][i] = k < k_end && m0 + i < M ? row[i] : 0.0f;
      }
    }
  };
  auto compute = [&](const float (&ac)[PER_WAVE][COLS]) {
#pragma unroll
    for (int r = 0; r < PER_WAVE; ++r) {
      const float* brow = bs + (PER_WAVE * w + r) * NP;
      float b[NP];
#pragma unroll
      for (int q = 0; q < NP / 4; ++q) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(brow + 4 * q);
        b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int i = 0; i < COLS; ++i)
#pragma unroll
        for (int n = 0; n < NP; ++n) acc[i][n] = fmaf(ac[r][i], b[n], acc[i][n]);
    }
  };
  if (PIPE && k_beg < k_end) load(k_beg);
  for (int k0 = k_beg; k0 < k_end; k0 += TN_CHUNK) {
    if (!PIPE) load(k0);
    __syncthreads();  // the previous chunk's B reads are done
#pragma unroll
    for (int i = 0; i < PER_T; ++i) bs[tid + i * NW_THREADS] = bv[i];
    if (PIPE) {
      float ac[PER_WAVE][COLS];
#pragma unroll
      for (int r = 0; r < PER_WAVE; ++r)
#pragma unroll
        for (int i = 0; i < COLS; ++i) ac[r][i] = a[r][i];
      __syncthreads();
      if (k0 + TN_CHUNK < k_end) load(k0 + TN_CHUNK);
      compute(ac);
    } else {
      __syncthreads();
      compute(a);
    }
  }
  float* mine = red + lane * RED;
  for (int src = 1; src < 4; ++src) {
    __syncthreads();  // wave 0 has read the previous hand-over
    if (w == src) {
#pragma unroll
      for (int i = 0; i < COLS; ++i)
#pragma unroll
        for (int n = 0; n < NP; ++n) mine[i * NP + n] = acc[i][n];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int i = 0; i < COLS; ++i)
#pragma unroll
        for (int n = 0; n < NP; ++n) acc[i][n] = acc[i][n] + mine[i * NP + n];
    }
  }
  if (w == 0) {
    float* o = out + (int64_t)by * M * N;
#pragma unroll
    for (int i = 0; i < COLS; ++i) {
      const int m = m0 + i;
      if (m < M) {
#pragma unroll
        for (int n = 0; n < NP; ++n)
          if (n < N) o[(int64_t)m * ldo + n] = acc[i][n];
      }
    }
  }
}

template <int NP>
__global__ void __launch_bounds__(NW_THREADS) gemm_tn_narrow_kernel(const float* __restrict__ A, int64_t lda,
                                                                     const float* __restrict__ B, int64_t ldb,
                                                                     float* __restrict__ out, int64_t ldo, int M, int N,
                                                                     int K, int kslice, int vec_a) {
  __shared__ __align__(16) float bs[TN_CHUNK * NP];
  __shared__ float red[64 * (4 * NP + 1)];
  tn_narrow_block<NP, 4, true>(blockIdx.x, blockIdx.y, bs, red, A, lda, B, ldb, out, ldo, M, N, K, kslice, vec_a);
}

// C[m][n] = sum over slices s (in order) of part[s][m][n] (+ bias[n] when given).
__global__ void __launch_bounds__(NW_THREADS) gemm_narrow_reduce_kernel(const float* __restrict__ part, int slices,
                                                                         float* __restrict__ C, int64_t ldc, int M,
                                                                         int N, const float* __restrict__ bias) {
  const int64_t total = (int64_t)M * N;
  for (int64_t e = (int64_t)blockIdx.x * NW_THREADS + threadIdx.x; e < total; e += (int64_t)gridDim.x * NW_THREADS) {
    float sum = part[e];
    for (int s0 = 1; s0 < slices; s0 += 8) {  // 8 loads in flight, added in slice order
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = s0 + i < slices ? part[(int64_t)(s0 + i) * total + e] : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (s0 + i < slices) sum = sum + v[i];
    }
    if (bias) sum = sum + bias[e % N];  // the bias epilogue
    C[(e / N) * ldc + e % N] = sum;
  }
}

// colsum[c] = the sum over rows r of G[r][c] (row stride ldg) in ascending r, for C <= 16
// columns: the additions of sum_to_shape's loop (and of colreduce_kernel), so the same bits.
// Chunks of 256 rows are staged transposed in LDS (`st`, 16 x CS_LD floats) and thread c adds
// its column's values in row order.
constexpr int CS_ROWS = 256, CS_LD = CS_ROWS + 4;
__device__ __forceinline__ void colsum_narrow_block(float* st, const float* __restrict__ G, int64_t ldg, int rows, int C,
                                                    float* __restrict__ colsum) {
  constexpr int PER_T = CS_ROWS * NW_MAX / NW_THREADS;
  const int t = threadIdx.x;
  float acc = 0.0f;
  float v[PER_T];
  auto load = [&](int r0) {  // chunk r0's values, thread t taking elements t, t + 256, ...
    const int total = min(CS_ROWS, rows - r0) * C;
#pragma unroll
    for (int j = 0; j < PER_T; ++j) {
      const int e = t + j * NW_THREADS;
      v[j] = e < total ? G[(int64_t)(r0 + e / C) * ldg + e % C] : 0.0f;
    }
  };
  if (rows > 0) load(0);
  for (int r0 = 0; r0 < rows; r0 += CS_ROWS) {
    const int cnt = min(CS_ROWS, rows - r0), total = cnt * C;
    __syncthreads();  // the previous chunk has been added up
#pragma unroll
    for (int j = 0; j < PER_T; ++j) {
      const int e = t + j * NW_THREADS;
      if (e < total) st[(e % C) * CS_LD + e / C] = v[j];
    }
    __syncthreads();
    if (r0 + CS_ROWS < rows) load(r0 + CS_ROWS);  // the next chunk's loads in flight during the adds
    if (t < C) {
      const float* col = st + t * CS_LD;
      int r = 0;
      for (; r + 32 <= cnt; r += 32) {
        floatx4 x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const floatx4*>(col + r + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc = acc + x[u].x;
          acc = acc + x[u].y;
          acc = acc + x[u].z;
          acc = acc + x[u].w;
        }
      }
      for (; r < cnt; ++r) acc = acc + col[r];
    }
  }
  if (t < C) colsum[t] = acc;
}

// The three products of a narrow Linear's backward in one grid (block roles by index): the
// column sum of G (one block), the weight gradient's slices (tn_narrow_block) and the input
// gradient's row groups (nt_smallk_block), each role the same code as its own kernel.
struct NarrowLinearBwArgs {
  const float* H;   // [B][K]
  const float* G;   // [B][C]
  const float* W;   // [K][C]
  const float* mask;
  float* dw_out;    // dW, or its slice partials
  float* dH;
  float* dH_pre;
  float* db;
  int B, K, C;
  int tn_gx, tn_blocks, tn_kslice, tn_vec;
  int nt_gx, nt_blocks, nt_rows;
};

template <int NP>
__global__ void __launch_bounds__(NW_THREADS, 4) narrow_linear_bw_kernel(NarrowLinearBwArgs a) {
  constexpr int TN_SMEM = TN_CHUNK * NP + 64 * (2 * NP + 1);
  constexpr int CS_SMEM = NW_MAX * CS_LD;
  constexpr int SMEM = TN_SMEM > CS_SMEM ? TN_SMEM : CS_SMEM;
  __shared__ __align__(16) float smem[SMEM];
  int b = blockIdx.x;
  if (a.db) {
    if (b == 0) {
      colsum_narrow_block(smem, a.G, a.C, a.B, a.C, a.db);
      return;
    }
    --b;
  }
  if (b < a.tn_blocks) {
    // two columns per lane and no prefetch: fewer registers, so the input-gradient blocks
    // beside it keep their occupancy (the sums are those of the weight gradient's own kernel)
    tn_narrow_block<NP, 2, false>(b % a.tn_gx, b / a.tn_gx, smem, smem + TN_CHUNK * NP, a.H, a.K, a.G, a.C,
                                  a.dw_out, a.C, a.K, a.C, a.B, a.tn_kslice, a.tn_vec);
    return;
  }
  b -= a.tn_blocks;
  nt_smallk_block<NP>(b % a.nt_gx, b / a.nt_gx, smem, a.G, a.C, a.W, a.C, a.dH, a.K, a.B, a.K, a.C, a.nt_rows, a.mask,
                      a.K, a.dH_pre);
}

const char* kernel_name(bool ta, bool tb, bool pipelined) {
  static const char* names[2][4] = {{"gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt"},
                                    {"gemm_nn_pipe", "gemm_nt_pipe", "gemm_tn_pipe", "gemm_tt_pipe"}};
  return names[pipelined ? 1 : 0][(ta ? 2 : 0) + (tb ? 1 : 0)];
}

}  // namespace

namespace {

// Kernel, tile and K split of one product.
struct GemmPlan {
  bool fast;
  bool skinny;  // 32 x 32 tiles on gemm_skinny_kernel, no K split
  int band;     // 0, or 1 + the gemm_tn_band_kernel mode of a banded X^T dY (no K split)
  int narrow;   // 0, or a narrow product: 1 NN (N <= 16), 2 NT (K <= 16), 3 TN (N <= 16)
  size_t BM, BN, mt, nt;
  int splits, k_chunk;  // for a narrow TN product: K slices and rows per slice
};

GemmPlan plan_gemm(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K, const float* A,
                   size_t lda, size_t sa, const float* B, size_t ldb, size_t sb, size_t batch,
                   int epi_kind = ORCA_HIP_EPI_NONE, int band_pref = 0) {
  GemmPlan g{};
  // Narrow products (one batch entry; a bias on X W, a ReLU mask on dY W^T) take the vector-unit kernels.
  if (ctx->gemm_narrow && batch == 1 && K > 0) {
    const bool none = epi_kind == ORCA_HIP_EPI_NONE;
    if (!trans_a && !trans_b && N <= NW_MAX && (none || epi_kind == ORCA_HIP_EPI_BIAS)) g.narrow = 1;
    else if (!trans_a && trans_b && K <= NW_MAX &&
             (none || epi_kind == ORCA_HIP_EPI_RELU_MASK || epi_kind == ORCA_HIP_EPI_RELU_MASK_PRE))
      g.narrow = 2;
    else if (trans_a && !trans_b && N <= NW_MAX && none) g.narrow = 3;
  }
  if (g.narrow) {
    // K slices (narrow NN and TN) so that the grid holds about two blocks per CU
    g.splits = 1;
    g.k_chunk = (int)K;
    if (g.narrow != 2) {
      const size_t chunk = g.narrow == 1 ? NN_CHUNK : TN_CHUNK;
      const size_t other = g.narrow == 1 ? (M + NN_ROWS - 1) / NN_ROWS : (M + 255) / 256;
      const size_t want = std::max<size_t>(1, (2 * (size_t)ctx->num_cus + other - 1) / other);
      const size_t chunks = (K + chunk - 1) / chunk;
      const size_t slices = std::min<size_t>(std::min(want, chunks), NW_MAX_SLICES);
      const size_t per = (chunks + slices - 1) / slices * chunk;
      g.k_chunk = (int)per;
      g.splits = (int)((K + per - 1) / per);
    }
    return g;
  }
  const bool vec_a = aligned16(A) && lda % 4 == 0 && (batch == 1 || sa % 4 == 0);
  const bool vec_b = aligned16(B) && ldb % 4 == 0 && (batch == 1 || sb % 4 == 0);
  // Products with M, N, K multiples of 4 and 16-byte aligned operands take the
  // pipelined 128 x 128 kernel, whose per-lane offsets are 32-bit byte offsets
  // within one operand.
  const size_t a_rows = trans_a ? K : M, b_rows = trans_b ? N : K;
  g.fast = M % 4 == 0 && N % 4 == 0 && K % 4 == 0 && vec_a && vec_b && a_rows * lda * 4 < 0xffffffffull &&
           b_rows * ldb * 4 < 0xffffffffull && !ctx->gemm_generic_only;
  // Generic kernel tile: 128 x 128 when that gives every CU a block, else
  // 128 x 64 (twice the blocks), unless the context fixes it (tuning).
  const size_t target = (size_t)ctx->num_cus;
  const size_t t128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  int bn = t128 >= target ? 128 : 64;
  if (ctx->gemm_tile_bn) bn = ctx->gemm_tile_bn;
  if (g.fast) bn = 128;
  // A weight gradient X^T dY (no epilogue) whose banded grid is one round between
  // half and all of the CUs (so it takes no K split) runs banded: 112-row tiles for
  // M = 112 R (R <= 7: as many tiles as 128 rows need, each 12.5 % smaller), or
  // eight 96-row bands plus 16 x 16 blocks for M = 768 + E, whichever the context
  // prefers when both apply.
  const size_t band_cols = N / 128;
  if (g.fast && ctx->gemm_band && trans_a && !trans_b && batch == 1 && epi_kind == ORCA_HIP_EPI_NONE &&
      N % 128 == 0) {
    const size_t r112 = M / BAND_AP;
    const bool rows112 = M % BAND_AP == 0 && r112 >= 1 && r112 <= 7 && r112 * band_cols <= target &&
                         2 * r112 * band_cols > target;
    const bool eight = M > (size_t)BAND_ROWS && M <= (size_t)(BAND_ROWS + BAND_EX) && 8 * band_cols <= target &&
                       16 * band_cols > target;
    if (rows112 || eight) {
      const int pref = band_pref ? band_pref : ctx->gemm_band;
      const bool use_eight = eight && (!rows112 || pref == 1);
      g.band = 1 + (use_eight ? BAND_EIGHT : BAND_ROWS112);
      g.BM = use_eight ? BAND_M : BAND_AP;
      g.BN = 128;
      g.mt = use_eight ? 8 : r112;
      g.nt = band_cols;
      g.splits = 1;
      g.k_chunk = (int)K;
      return g;
    }
  }
  size_t BM = 128;
  // Short products (K <= 512) whose 128 x 128 grid leaves at least half the
  // CUs idle take 64 x 64 tiles on the generic kernel instead of splitting K,
  // when those tiles alone give three quarters of the CUs a block: the K
  // split's partial sums and their reduce launch are gone (the weight
  // gradients of a 256-row batch).  With fewer tiles, or a long K, the
  // generic kernel's K loop costs more than the split saves.
  const size_t t64 = ((M + 63) / 64) * ((N + 63) / 64) * batch;
  if (ctx->gemm_small_tiles && K <= 512 && t128 <= target / 2 && 4 * t64 >= 3 * target) {
    g.fast = false;
    BM = 64;
    bn = 64;
  }
  // Few rows and a short K (A row-major): when 32 x 32 tiles give between a
  // half and two blocks per CU, the skinny kernel takes the product whole, with
  // no K split (with more of its tiles the 128 x 128 split is faster).
  const size_t t32 = ((M + 31) / 32) * ((N + 31) / 32);
  if (ctx->gemm_skinny && !trans_a && batch == 1 && BM == 128 && t128 <= target / 2 && M <= 256 && K <= 1024 &&
      2 * t32 >= target && t32 <= 2 * target) {
    g.skinny = true;
    g.fast = false;
    BM = 32;
    bn = 32;
  }
  g.BM = BM;
  g.BN = (size_t)bn;
  g.mt = (M + BM - 1) / BM;
  g.nt = (N + g.BN - 1) / g.BN;
  // Split K when the tile grid leaves at least half the CUs idle and K is long
  // enough (a grid of exactly half the CUs halves its time with two chunks;
  // between half and all of them a split would not shorten the longest CU).
  g.splits = 1;
  const size_t tiles = g.mt * g.nt * batch;
  if (BM == 128 && !g.skinny && tiles <= target / 2 && K >= 4 * (size_t)BK) {
    size_t want = (target + tiles - 1) / tiles;
    size_t max_by_k = K / (2 * BK);
    g.splits = (int)std::min<size_t>(std::min<size_t>(want, max_by_k), 64);
    if (g.splits < 1) g.splits = 1;
  }
  g.k_chunk = (int)K;
  if (g.splits > 1) {
    size_t per = (K + g.splits - 1) / g.splits;
    per = (per + BK - 1) / BK * BK;
    g.splits = (int)((K + per - 1) / per);
    g.k_chunk = (int)per;
  }
  return g;
}

// Workspace floats of a planned product: split-K partials, then per-split column sums.
size_t plan_workspace_floats(const GemmPlan& g, size_t M, size_t N, size_t batch, bool colsum) {
  if (g.splits <= 1) return 0;
  if (g.narrow) return (size_t)g.splits * M * N;  // TN slice partials (its column sum is a separate pass)
  return batch * (size_t)g.splits * M * N + (colsum ? (size_t)g.splits * N : 0);
}

}  // namespace

namespace {

// The grid of a narrow NT product: about two blocks per CU, each walking `rows` rows with
// its columns of B in registers.
void nt_grid(orca_hip_ctx* ctx, size_t M, size_t N, size_t& gx, size_t& gy, size_t& rows) {
  gx = (N + NW_THREADS - 1) / NW_THREADS;
  const size_t want = std::max<size_t>(1, (2 * (size_t)ctx->num_cus + gx - 1) / gx);
  rows = std::max<size_t>((M + want - 1) / want, (M + 65534) / 65535);
  gy = (M + rows - 1) / rows;
  if (gx > 0x7fffffff) fail(ORCA_HIP_ERR_INTERNAL, "gemm: too many columns");
}

// A narrow product (plan.narrow): one launch, plus the slice reduction of a
// sliced product and, when asked for, the exact column sum of B.
template <int NP>
void launch_narrow(orca_hip_ctx* ctx, const GemmPlan& plan, size_t M, size_t N, size_t K, const float* A,
                   size_t lda, const float* B, size_t ldb, float* out, int64_t ldo, int vec, const GemmEpi& epi) {
  if (plan.narrow == 1) {
    const unsigned gy = (unsigned)std::min<size_t>((M + NN_ROWS - 1) / NN_ROWS, 65535);
    hipLaunchKernelGGL(gemm_nn_narrow_kernel<NP>, dim3((unsigned)plan.splits, gy), dim3(NW_THREADS), 0, ctx->stream,
                       A, (int64_t)lda, B, (int64_t)ldb, out, ldo, (int)M, (int)N, (int)K, plan.k_chunk,
                       plan.splits == 1 && epi.kind == ORCA_HIP_EPI_BIAS ? epi.bias : nullptr);
  } else if (plan.narrow == 2) {
    size_t gx, gy, rows;
    nt_grid(ctx, M, N, gx, gy, rows);
    hipLaunchKernelGGL(gemm_nt_smallk_kernel<NP>, dim3((unsigned)gx, (unsigned)gy), dim3(NW_THREADS), 0, ctx->stream,
                       A, (int64_t)lda, B, (int64_t)ldb, out, ldo, (int)M, (int)N, (int)K, (int)rows,
                       epi.kind == ORCA_HIP_EPI_RELU_MASK || epi.kind == ORCA_HIP_EPI_RELU_MASK_PRE ? epi.mask : nullptr,
                       (int64_t)epi.ldmask, epi.kind == ORCA_HIP_EPI_RELU_MASK_PRE ? epi.pre : nullptr);
  } else {
    hipLaunchKernelGGL(gemm_tn_narrow_kernel<NP>, dim3((unsigned)((M + 255) / 256), (unsigned)plan.splits),
                       dim3(NW_THREADS), 0, ctx->stream, A, (int64_t)lda, B, (int64_t)ldb, out, ldo, (int)M, (int)N,
                       (int)K, plan.k_chunk, vec);
  }
  ORCA_HIP_CHECK(hipGetLastError());
}

void gemm_narrow(orca_hip_ctx* ctx, const GemmPlan& plan, size_t M, size_t N, size_t K, const float* A, size_t lda,
                 const float* B, size_t ldb, float* C, size_t ldc, const GemmEpi& epi) {
  static const char* names[4] = {"", "gemm_nn_narrow", "gemm_nt_smallk", "gemm_tn_narrow"};
  std::string pname;
  if (ctx->prof.enabled)
    pname = std::string(names[plan.narrow]) + " " + std::to_string(M) + "x" + std::to_string(N) + "x" +
            std::to_string(K);
  const int slices = plan.splits;
  std::unique_ptr<Scratch> scratch;
  float* out = C;
  int64_t ldo = (int64_t)ldc;
  if (slices > 1) {
    const size_t need = (size_t)slices * M * N;
    if (epi.ws) {
      if (epi.ws_floats < need) fail(ORCA_HIP_ERR_INTERNAL, "gemm: workspace too small for the planned slices");
      out = epi.ws;
    } else {
      scratch.reset(new Scratch(ctx, sizeof(float) * need));
      out = scratch->as<float>();
    }
    ldo = (int64_t)N;
  }
  {
    ProfScope ps(ctx, pname.c_str(), 2.0 * (double)M * N * K,
                 4.0 * (double)(M * K + K * N + (slices > 1 ? slices : 1) * M * N));
    const int vec = aligned16(A) && lda % 4 == 0;  // float4 rows of A (narrow TN)
    const int np = narrow_pad(plan.narrow == 2 ? K : N);
    if (np == 4) launch_narrow<4>(ctx, plan, M, N, K, A, lda, B, ldb, out, ldo, vec, epi);
    else if (np == 8) launch_narrow<8>(ctx, plan, M, N, K, A, lda, B, ldb, out, ldo, vec, epi);
    else launch_narrow<16>(ctx, plan, M, N, K, A, lda, B, ldb, out, ldo, vec, epi);
  }
  if (slices > 1) {
    ProfScope ps(ctx, "gemm_narrow_reduce", 0.0, 4.0 * (double)M * N * (slices + 1));
    const unsigned g = grid_for(M * N, NW_THREADS, ctx->num_cus * 4);
    hipLaunchKernelGGL(gemm_narrow_reduce_kernel, dim3(g), dim3(NW_THREADS), 0, ctx->stream, out, slices, C,
                       (int64_t)ldc, (int)M, (int)N, epi.kind == ORCA_HIP_EPI_BIAS ? epi.bias : nullptr);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (epi.colsum) {  // only a row-major B has one: the bias gradient, in ascending row order
    if (plan.narrow == 2) fail(ORCA_HIP_ERR_INTERNAL, "gemm colsum epilogue requires row-major B");
    launch_colsum(ctx, B, K, N, ldb, epi.colsum);
  }
}

// dW = H^T G (+ db, the column sums of G) and dH = G W^T (+ ReLU mask) in one grid plus the
// weight gradient's slice reduction, with the plans the separate products would take (so the
// same sums).  False when either product would not run on the narrow kernels.
bool narrow_linear_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* G, size_t C,
                            const float* W, const float* mask, float* dH, float* dH_pre, float* dW, float* db) {
  const int nt_kind = mask ? (dH_pre ? ORCA_HIP_EPI_RELU_MASK_PRE : ORCA_HIP_EPI_RELU_MASK) : ORCA_HIP_EPI_NONE;
  const GemmPlan tn = plan_gemm(ctx, true, false, K, C, B, H, K, 0, G, C, 0, 1, ORCA_HIP_EPI_NONE);
  const GemmPlan nt = plan_gemm(ctx, false, true, B, K, C, G, C, 0, W, C, 0, 1, nt_kind);
  if (tn.narrow != 3 || nt.narrow != 2 || B == 0 || K == 0 || C == 0) return false;
  NarrowLinearBwArgs a{};
  a.H = H;
  a.G = G;
  a.W = W;
  a.mask = mask;
  a.dH = dH;
  a.dH_pre = mask ? dH_pre : nullptr;
  a.db = db;
  a.B = (int)B;
  a.K = (int)K;
  a.C = (int)C;
  a.tn_gx = (int)((K + 127) / 128);  // 128 columns per block (two per lane)
  a.tn_blocks = a.tn_gx * tn.splits;
  a.tn_kslice = tn.k_chunk;
  a.tn_vec = (reinterpret_cast<uintptr_t>(H) & 7) == 0 && K % 2 == 0;
  size_t gx, gy, rows;
  nt_grid(ctx, B, K, gx, gy, rows);
  a.nt_gx = (int)gx;
  a.nt_blocks = (int)(gx * gy);
  a.nt_rows = (int)rows;
  std::unique_ptr<Scratch> scratch;
  a.dw_out = dW;
  if (tn.splits > 1) {
    scratch.reset(new Scratch(ctx, sizeof(float) * (size_t)tn.splits * K * C));
    a.dw_out = scratch->as<float>();
  }
  const size_t blocks = (db ? 1 : 0) + (size_t)a.tn_blocks + (size_t)a.nt_blocks;
  if (blocks > 0x7fffffff) fail(ORCA_HIP_ERR_INTERNAL, "narrow_linear_backward: too many blocks");
  {
    ProfScope ps(ctx, "narrow_linear_bw", 2.0 * 2.0 * (double)B * K * C,
                 4.0 * (double)(B * K * (mask ? 2 : 1) + B * C + 2 * K * C + B * K * (dH_pre ? 2 : 1) +
                                (tn.splits > 1 ? tn.splits * K * C : 0)));
    const int np = narrow_pad(C);
    if (np == 4)
      hipLaunchKernelGGL(narrow_linear_bw_kernel<4>, dim3((unsigned)blocks), dim3(NW_THREADS), 0, ctx->stream, a);
    else if (np == 8)
      hipLaunchKernelGGL(narrow_linear_bw_kernel<8>, dim3((unsigned)blocks), dim3(NW_THREADS), 0, ctx->stream, a);
    else
      hipLaunchKernelGGL(narrow_linear_bw_kernel<16>, dim3((unsigned)blocks), dim3(NW_THREADS), 0, ctx->stream, a);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (tn.splits > 1) {
    ProfScope ps(ctx, "gemm_narrow_reduce", 0.0, 4.0 * (double)K * C * (tn.splits + 1));
    const unsigned g = grid_for(K * C, NW_THREADS, ctx->num_cus * 4);
    hipLaunchKernelGGL(gemm_narrow_reduce_kernel, dim3(g), dim3(NW_THREADS), 0, ctx->stream, a.dw_out, tn.splits, dW,
                       (int64_t)C, (int)K, (int)C, nullptr);
    ORCA_HIP_CHECK(hipGetLastError());
  }
  return true;
}

}  // namespace

size_t gemm_workspace_floats(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K,
                             const float* A, size_t lda, size_t sa, const float* B, size_t ldb, size_t sb,
                             size_t batch, bool colsum, int epi_kind) {
  if (M == 0 || N == 0 || batch == 0 || K == 0) return 0;
  const GemmPlan g = plan_gemm(ctx, trans_a, trans_b, M, N, K, A, lda, sa, B, ldb, sb, batch, epi_kind);
  return plan_workspace_floats(g, M, N, batch, colsum && batch == 1 && !trans_b);
}

namespace {
// gemm() without epi.done; sets `bound` when the pipelined kernel was
// launched with epi.done as its completion event.
void gemm_launch(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K, const float* A,
                 size_t lda, size_t sa, const float* B, size_t ldb, size_t sb, float* C, size_t ldc, size_t sc,
                 size_t batch, const GemmEpi& epi, bool& bound) {
  if (M == 0 || N == 0 || batch == 0) return;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || batch > 65535)
    fail(ORCA_HIP_ERR_INTERNAL, "gemm dimensions exceed the kernel's index range");
  if (K == 0) {  // empty product: C = epilogue(0)
    for (size_t b = 0; b < batch; ++b) {
      if (epi.kind == ORCA_HIP_EPI_NONE || epi.kind == ORCA_HIP_EPI_RELU_MASK ||
          epi.kind == ORCA_HIP_EPI_RELU_MASK_PRE) {
        for (float* out : {C, epi.kind == ORCA_HIP_EPI_RELU_MASK_PRE ? epi.pre : nullptr}) {
          if (!out) continue;
          if (ldc == N) launch_fill(ctx, out + b * sc, 0.0f, M * N);
          else for (size_t r = 0; r < M; ++r) launch_fill(ctx, out + b * sc + r * ldc, 0.0f, N);
        }
      } else {
        fail(ORCA_HIP_ERR_INTERNAL, "gemm with K = 0 and a bias epilogue is not supported");
      }
    }
    if (epi.colsum) launch_fill(ctx, epi.colsum, 0.0f, N);
    return;
  }
  const GemmPlan plan = plan_gemm(ctx, trans_a, trans_b, M, N, K, A, lda, sa, B, ldb, sb, batch, epi.kind, epi.band);
  if (plan.narrow) {
    gemm_narrow(ctx, plan, M, N, K, A, lda, B, ldb, C, ldc, epi);
    return;
  }
  if (plan.skinny) {
    SkinnyParams q{};
    q.A = A;
    q.B = B;
    q.C = C;
    q.lda = (int64_t)lda;
    q.ldb = (int64_t)ldb;
    q.ldc = (int64_t)ldc;
    q.M = (int)M;
    q.N = (int)N;
    q.K = (int)K;
    q.kq = (int)(((K + SK_WAVES - 1) / SK_WAVES + 7) / 8 * 8);
    q.vec = aligned16(A) && lda % 4 == 0 && (!trans_b || (aligned16(B) && ldb % 4 == 0));
    q.epi = epi.kind;
    q.bias = epi.bias;
    q.mask = epi.mask;
    q.ldmask = (int64_t)epi.ldmask;
    q.pre = epi.pre;
    {
      std::string pname;
      if (ctx->prof.enabled)
        pname = std::string(trans_b ? "gemm_nt_skinny " : "gemm_nn_skinny ") + std::to_string(M) + "x" +
                std::to_string(N) + "x" + std::to_string(K);
      ProfScope ps(ctx, pname.c_str(), 2.0 * (double)M * N * K, 4.0 * (double)(M * K + K * N + M * N));
      dim3 grid((unsigned)plan.nt, (unsigned)plan.mt);
      if (trans_b)
        hipLaunchKernelGGL(gemm_skinny_kernel<true>, grid, dim3(64 * SK_WAVES), 0, ctx->stream, q);
      else
        hipLaunchKernelGGL(gemm_skinny_kernel<false>, grid, dim3(64 * SK_WAVES), 0, ctx->stream, q);
      ORCA_HIP_CHECK(hipGetLastError());
    }
    if (epi.colsum) {  // only a row-major B has one (the bias gradient of X^T dY, which is not skinny)
      if (trans_b) fail(ORCA_HIP_ERR_INTERNAL, "gemm colsum epilogue requires row-major B");
      launch_colsum(ctx, B, K, N, ldb, epi.colsum);
    }
    return;
  }
  const bool fast = plan.fast;
  const int bn = (int)plan.BN;
  const size_t mt = plan.mt, nt = plan.nt;
  if (mt > 65535) fail(ORCA_HIP_ERR_INTERNAL, "gemm: too many row tiles");
  const int splits = plan.splits, k_chunk = plan.k_chunk;
  const bool vec_a = aligned16(A) && lda % 4 == 0 && (batch == 1 || sa % 4 == 0);
  const bool vec_b = aligned16(B) && ldb % 4 == 0 && (batch == 1 || sb % 4 == 0);

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
  p.pre = epi.pre;
  const bool fold_colsum = epi.colsum != nullptr && batch == 1 && !trans_b && (splits == 1 || !epi.exact_colsum);
  // Split-K partials (and per-split column sums) go to the caller's workspace
  // when it provides one, else to blocks from the context cache.
  const size_t ws_need = plan_workspace_floats(plan, M, N, batch, fold_colsum);
  std::unique_ptr<Scratch> scratch;
  float* ws = nullptr;
  if (ws_need) {
    if (epi.ws) {
      if (epi.ws_floats < ws_need) fail(ORCA_HIP_ERR_INTERNAL, "gemm: workspace too small for the planned split");
      ws = epi.ws;
    } else {
      scratch.reset(new Scratch(ctx, sizeof(float) * ws_need));
      ws = scratch->as<float>();
    }
  }
  p.colsum = fold_colsum ? (splits > 1 ? ws + batch * (size_t)splits * M * N : epi.colsum) : nullptr;
  p.vec_a = vec_a;
  p.vec_b = vec_b;
  p.C = splits > 1 ? ws : C;

  dim3 grid((unsigned)nt, (unsigned)mt, (unsigned)(batch * splits));
  {
    // Profiler records carry the product's shape: "gemm_tn_pipe 4096x4096x1024".
    std::string pname;
    if (ctx->prof.enabled) {
      pname = std::string(plan.band == 1 + BAND_EIGHT     ? "gemm_tn_band8"
                          : plan.band == 1 + BAND_ROWS112 ? "gemm_tn_band112"
                                                          : kernel_name(trans_a, trans_b, fast)) +
              " " +
              std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K);
      if (batch > 1) pname += "x" + std::to_string(batch);
    }
    ProfScope ps(ctx, pname.c_str(), 2.0 * (double)M * N * K * batch,
                 4.0 * (double)batch * (M * K + K * N + M * N));
#define GEMM_LAUNCH(BM_, BN_, TA_, TB_) \
  hipLaunchKernelGGL((gemm_mfma_f32_kernel<BM_, BN_, TA_, TB_>), grid, dim3(NTHREADS), 0, ctx->stream, p)
#define GEMM_DISPATCH(BM_, BN_)                                      \
  do {                                                               \
    if (!trans_a && !trans_b) GEMM_LAUNCH(BM_, BN_, false, false);   \
    else if (!trans_a && trans_b) GEMM_LAUNCH(BM_, BN_, false, true); \
    else if (trans_a && !trans_b) GEMM_LAUNCH(BM_, BN_, true, false); \
    else GEMM_LAUNCH(BM_, BN_, true, true);                          \
  } while (0)
#define FAST_LAUNCH(TA_, TB_, CS_)                                                                        \
  do {                                                                                                     \
    if (bind)                                                                                              \
      hipExtLaunchKernelGGL((gemm_mfma_f32_fast_kernel<TA_, TB_, CS_>), grid, dim3(NTHREADS), 0, ctx->stream, \
                            nullptr, epi.done, 0, p);                                                      \
    else                                                                                                   \
      hipLaunchKernelGGL((gemm_mfma_f32_fast_kernel<TA_, TB_, CS_>), grid, dim3(NTHREADS), 0, ctx->stream, p); \
  } while (0)
    // The pipelined kernel is the product's last launch unless a split
    // reduce or a separate column sum follows it.
    const bool bind = epi.done && splits == 1 && (!epi.colsum || fold_colsum);
#define BAND_LAUNCH(MODE_, CS_)                                                                          \
  do {                                                                                                    \
    const dim3 threads(CS_ && MODE_ == BAND_EIGHT ? NTHREADS + 64 : NTHREADS);                           \
    const dim3 bgrid(grid.x, grid.y + (CS_ && MODE_ == BAND_ROWS112 ? 1 : 0));                            \
    if (bind)                                                                                             \
      hipExtLaunchKernelGGL((gemm_tn_band_kernel<MODE_, CS_>), bgrid, threads, 0, ctx->stream, nullptr, epi.done, \
                            0, p);                                                                        \
    else                                                                                                  \
      hipLaunchKernelGGL((gemm_tn_band_kernel<MODE_, CS_>), bgrid, threads, 0, ctx->stream, p);           \
  } while (0)
    if (plan.band) {
      bound = bind;
      const bool eight = plan.band == 1 + BAND_EIGHT;
      if (eight && p.colsum) BAND_LAUNCH(BAND_EIGHT, true);
      else if (eight) BAND_LAUNCH(BAND_EIGHT, false);
      else if (p.colsum) BAND_LAUNCH(BAND_ROWS112, true);
      else BAND_LAUNCH(BAND_ROWS112, false);
    } else if (fast) {
      bound = bind;
      // The column sum reads only B's LDS tile (row-major B), so it folds in
      // whatever A's layout is.
      const bool cs = p.colsum != nullptr;
      if (!trans_a && !trans_b && cs) FAST_LAUNCH(false, false, true);
      else if (!trans_a && !trans_b) FAST_LAUNCH(false, false, false);
      else if (!trans_a && trans_b) FAST_LAUNCH(false, true, false);
      else if (trans_a && !trans_b && cs) FAST_LAUNCH(true, false, true);
      else if (trans_a && !trans_b) FAST_LAUNCH(true, false, false);
      else FAST_LAUNCH(true, true, false);
    } else if (plan.BM == 64) {
      GEMM_DISPATCH(64, 64);
    } else if (bn == 128) {
      GEMM_DISPATCH(128, 128);
    } else {
      GEMM_DISPATCH(128, 64);
    }
#undef BAND_LAUNCH
#undef FAST_LAUNCH
#undef GEMM_DISPATCH
#undef GEMM_LAUNCH
    ORCA_HIP_CHECK(hipGetLastError());
  }
  bool colsum_reduced = false;
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
    r.pre = epi.pre;
    size_t total = batch * M * N;
    ProfScope ps(ctx, "gemm_splitk_reduce", 0.0, 4.0 * (double)total * (splits + 1));
    const bool vec = N % 4 == 0 && ldc % 4 == 0 && (batch == 1 || sc % 4 == 0) && aligned16(C) && aligned16(r.ws) &&
                     ((epi.kind != ORCA_HIP_EPI_RELU_MASK && epi.kind != ORCA_HIP_EPI_RELU_MASK_PRE) ||
                      (aligned16(epi.mask) && epi.ldmask % 4 == 0)) &&
                     (!epi.pre || aligned16(epi.pre)) && total / 4 < (size_t)INT32_MAX;
    if (vec) {
      if (fold_colsum) {
        r.cs_part = p.colsum;
        r.cs_out = epi.colsum;
        colsum_reduced = true;
      }
      unsigned g = grid_for(total / 4, 256, ctx->num_cus * 8);
      hipLaunchKernelGGL(splitk_reduce_vec_kernel, dim3(g), dim3(256), 0, ctx->stream, r, (uint32_t)(total / 4));
    } else {
      unsigned g = grid_for(total, 256, ctx->num_cus * 8);
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(g), dim3(256), 0, ctx->stream, r, total);
    }
    ORCA_HIP_CHECK(hipGetLastError());
  }
  if (fold_colsum && splits > 1 && !colsum_reduced) {
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
}  // namespace

void gemm(orca_hip_ctx* ctx, bool trans_a, bool trans_b, size_t M, size_t N, size_t K, const float* A, size_t lda,
          size_t sa, const float* B, size_t ldb, size_t sb, float* C, size_t ldc, size_t sc, size_t batch,
          const GemmEpi& epi) {
  bool bound = false;
  gemm_launch(ctx, trans_a, trans_b, M, N, K, A, lda, sa, B, ldb, sb, C, ldc, sc, batch, epi, bound);
  if (epi.done && !bound) ORCA_HIP_CHECK(hipEventRecord(epi.done, ctx->stream));
}

namespace {
// gemm() of one 2-D product, handing back through `done` (when non-null) an event that
// completes with the product's last launch (bound to it when gemm() can bind it).
void gemm_with_event(orca_hip_ctx* ctx, bool ta, bool tb, size_t M, size_t N, size_t K, const float* A, size_t lda,
                     const float* B, size_t ldb, float* C, size_t ldc, GemmEpi& e, orca_hip_event** done) {
  if (done) {
    *done = nullptr;
    e.done = take_order_event(ctx);
  }
  try {
    gemm(ctx, ta, tb, M, N, K, A, lda, 0, B, ldb, 0, C, ldc, 0, 1, e);
  } catch (...) {
    if (e.done) ctx->event_pool.push_back(e.done);
    throw;
  }
  if (done) *done = reinterpret_cast<orca_hip_event*>(e.done);
}
}  // namespace

}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_gemm(orca_hip_ctx* ctx, int trans_a, int trans_b, size_t M, size_t N, size_t K, const float* A, size_t lda,
                  const float* B, size_t ldb, float* C, size_t ldc, const orca_hip_epilogue* epi) {
  return guard([&] {
    bind(ctx);
    if ((trans_a ? lda < M : lda < K) || (trans_b ? ldb < K : ldb < N) || ldc < N)
      fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during gemm: leading dimension smaller than the row length");
    check_extent(ctx, A, matrix_bytes(trans_a ? K : M, trans_a ? M : K, lda), "gemm (A)");
    check_extent(ctx, B, matrix_bytes(trans_b ? N : K, trans_b ? K : N, ldb), "gemm (B)");
    check_extent(ctx, C, matrix_bytes(M, N, ldc), "gemm (C)");
    GemmEpi e;
    if (epi) {
      e.kind = epi->kind;
      e.bias = epi->bias;
      e.mask = epi->mask;
      e.ldmask = epi->ldmask;
      e.colsum = epi->colsum;
      e.exact_colsum = true;
      const bool has_bias = e.kind == ORCA_HIP_EPI_BIAS || e.kind == ORCA_HIP_EPI_BIAS_RELU ||
                            e.kind == ORCA_HIP_EPI_BIAS_RELU_PRE;
      const bool has_mask = e.kind == ORCA_HIP_EPI_RELU_MASK || e.kind == ORCA_HIP_EPI_RELU_MASK_PRE;
      if (e.kind < ORCA_HIP_EPI_NONE || e.kind > ORCA_HIP_EPI_RELU_MASK_PRE)
        fail(ORCA_HIP_ERR_INTERNAL, "unknown gemm epilogue " + std::to_string(e.kind));
      if (has_bias && !e.bias) fail(ORCA_HIP_ERR_INTERNAL, "bias epilogue without a bias pointer");
      if (has_mask && (!e.mask || e.ldmask < N)) fail(ORCA_HIP_ERR_INTERNAL, "mask epilogue without a valid mask");
      if (e.kind == ORCA_HIP_EPI_BIAS_RELU_PRE || e.kind == ORCA_HIP_EPI_RELU_MASK_PRE) {
        if (!epi->pre) fail(ORCA_HIP_ERR_INTERNAL, "pre-activation epilogue without a pre pointer");
        e.pre = epi->pre;
        check_extent(ctx, e.pre, matrix_bytes(M, N, ldc), "gemm (pre)");
      }
      if (has_bias) check_extent(ctx, e.bias, N * sizeof(float), "gemm (bias)");
      if (has_mask) check_extent(ctx, e.mask, matrix_bytes(M, N, e.ldmask), "gemm (mask)");
      check_extent(ctx, e.colsum, N * sizeof(float), "gemm (colsum)");
    }
    gemm_with_event(ctx, trans_a != 0, trans_b != 0, M, N, K, A, lda, B, ldb, C, ldc, e, epi ? epi->done : nullptr);
  });
}

// orca-backend-cpu/src/backend.rs:130-221 (contract), with lazy-transpose views.
// Backend::matmul of [M, K] x [K, N] plus sum_to_shape(rhs, [K, N] -> [1, N])
// (backend.rs:499-530) in one product: the column sum is folded into the
// GEMM's loads of rhs when K is not split, else taken in a separate pass.
int orca_hip_matmul_colsum(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N,
                           int lhs_view, int dtype, void* colsum, void** out) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "matmul");
    if (!colsum) fail(ORCA_HIP_ERR_INTERNAL, "matmul_colsum: null column-sum output");
    const bool ta = lhs_view == ORCA_HIP_VIEW_TRANSPOSED;
    check_extent(ctx, lhs, M * K * sizeof(float), "matmul (lhs)");
    check_extent(ctx, rhs, K * N * sizeof(float), "matmul (rhs)");
    check_extent(ctx, colsum, N * sizeof(float), "matmul_colsum (colsum)");
    float* o = new_output(ctx, M * N);
    if (M == 0) {  // no product, but the column sum still covers rhs
      launch_colsum(ctx, static_cast<const float*>(rhs), K, N, N, static_cast<float*>(colsum));
      *out = o;
      return;
    }
    GemmEpi e;
    e.colsum = static_cast<float*>(colsum);
    e.exact_colsum = true;
    gemm(ctx, ta, false, M, N, K, static_cast<const float*>(lhs), ta ? M : K, 0, static_cast<const float*>(rhs), N,
         0, o, N, 0, 1, e);
    *out = o;
  });
}

int orca_hip_narrow_linear_backward(orca_hip_ctx* ctx, const float* H, size_t B, size_t K, const float* G, size_t C,
                                    const float* W, const float* mask, float* dH, float* dH_pre, float* dW, float* db,
                                    orca_hip_event** done) {
  return guard([&] {
    bind(ctx);
    if (done) *done = nullptr;
    if (C < 1 || C > NW_MAX) fail(ORCA_HIP_ERR_INTERNAL, "narrow_linear_backward: needs 1 <= C <= 16");
    if (!H || !G || !W || !dH || !dW) fail(ORCA_HIP_ERR_INTERNAL, "narrow_linear_backward: null operand");
    check_extent(ctx, H, B * K * sizeof(float), "narrow_linear_backward (H)");
    check_extent(ctx, G, B * C * sizeof(float), "narrow_linear_backward (G)");
    check_extent(ctx, W, K * C * sizeof(float), "narrow_linear_backward (W)");
    check_extent(ctx, mask, B * K * sizeof(float), "narrow_linear_backward (mask)");
    check_extent(ctx, dH, B * K * sizeof(float), "narrow_linear_backward (dH)");
    check_extent(ctx, dH_pre, B * K * sizeof(float), "narrow_linear_backward (dH_pre)");
    check_extent(ctx, dW, K * C * sizeof(float), "narrow_linear_backward (dW)");
    check_extent(ctx, db, C * sizeof(float), "narrow_linear_backward (db)");
    if (!narrow_linear_backward(ctx, H, B, K, G, C, W, mask, dH, dH_pre, dW, db))
      fail(ORCA_HIP_ERR_INTERNAL, "narrow_linear_backward: the products do not take the narrow kernels");
    if (done) {
      hipEvent_t ev = take_order_event(ctx);
      const hipError_t er = hipEventRecord(ev, ctx->stream);
      if (er != hipSuccess) {
        ctx->event_pool.push_back(ev);
        ORCA_HIP_CHECK(er);
      }
      *done = reinterpret_cast<orca_hip_event*>(ev);
    }
  });
}

// orca_hip_matmul of rank-2 operands or orca_hip_matmul_colsum, with an event completing
// with the product (for the storage layer's second-stream work).
int orca_hip_matmul_ev(orca_hip_ctx* ctx, const void* lhs, const void* rhs, size_t M, size_t K, size_t N,
                       int lhs_view, int rhs_view, int dtype, void* colsum, void** out, orca_hip_event** done) {
  return guard([&] {
    bind(ctx);
    check_f32(dtype, "matmul");
    if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    const bool ta = lhs_view == ORCA_HIP_VIEW_TRANSPOSED, tb = rhs_view == ORCA_HIP_VIEW_TRANSPOSED;
    if (colsum && tb) fail(ORCA_HIP_ERR_INTERNAL, "matmul_ev: a column sum needs a contiguous rhs");
    check_extent(ctx, lhs, M * K * sizeof(float), "matmul (lhs)");
    check_extent(ctx, rhs, K * N * sizeof(float), "matmul (rhs)");
    check_extent(ctx, colsum, N * sizeof(float), "matmul_colsum (colsum)");
    float* o = new_output(ctx, M * N);
    GemmEpi e;
    if (colsum) {
      e.colsum = static_cast<float*>(colsum);
      e.exact_colsum = true;
    }
    if (M == 0 || N == 0) {  // no product; a column sum still covers rhs
      if (colsum && N) launch_colsum(ctx, static_cast<const float*>(rhs), K, N, N, static_cast<float*>(colsum));
      if (done) {
        *done = nullptr;
        hipEvent_t ev = take_order_event(ctx);
        const hipError_t er = hipEventRecord(ev, ctx->stream);
        if (er != hipSuccess) {
          ctx->event_pool.push_back(ev);
          ORCA_HIP_CHECK(er);
        }
        *done = reinterpret_cast<orca_hip_event*>(ev);
      }
      *out = o;
      return;
    }
    gemm_with_event(ctx, ta, tb, M, N, K, static_cast<const float*>(lhs), ta ? M : K, static_cast<const float*>(rhs),
                    tb ? K : N, o, N, e, done);
    *out = o;
  });
}

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
    check_extent(ctx, lhs, batch * M * K * sizeof(float), "matmul (lhs)");
    check_extent(ctx, rhs, batch * K * N * sizeof(float), "matmul (rhs)");
    float* o = new_output(ctx, batch * M * N);
    GemmEpi e;
    gemm(ctx, ta, tb, M, N, K, static_cast<const float*>(lhs), ta ? M : K, M * K, static_cast<const float*>(rhs),
         tb ? K : N, K * N, o, N, M * N, batch, e);
    *out = o;
  });
}

}  // extern "C"
