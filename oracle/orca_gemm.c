/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, batched f32 GEMM.
 *
 * Restates the contract of orca-backend-cpu/src/backend.rs:130-221: C[b] =
 * A[b] . B[b] for row-major (..., M, K) x (..., K, N), alpha = 1, beta = 0,
 * one single-threaded sgemm per batch entry (the reference links the
 * `matrixmultiply` 0.3 crate without its `threading` feature,
 * orca-backend-cpu/Cargo.toml:11).  The blocking order of that crate is not
 * reproduced (it is not vendored and its version is unpinned), so results
 * match the reference to rounding, not bit for bit; integer-valued inputs
 * give exact results for any order, which is how tests pin this function.
 * Cache-blocked with packed panels so the CPU baseline keeps an
 * sgemm-class cost structure.
 */
#include "orca_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MR 4
#define NR 16
#define KC 256
#define MC 96
#define NC 1024

typedef float v8 __attribute__((vector_size(32)));

#define GEMM_BODY                                                                          \
  {                                                                                        \
    float* bp = (float*)aligned_alloc(64, sizeof(float) * KC * NC);                        \
    float* ap = (float*)aligned_alloc(64, sizeof(float) * KC * MC);                        \
    if (!bp || !ap) {                                                                      \
      free(bp);                                                                            \
      free(ap);                                                                            \
      return -1;                                                                           \
    }                                                                                      \
    for (size_t i = 0; i < M * N; ++i) C[i] = 0.0f;                                        \
    for (size_t jc = 0; jc < N; jc += NC) {                                                \
      size_t nc = N - jc < NC ? N - jc : NC;                                               \
      size_t npan = (nc + NR - 1) / NR;                                                    \
      for (size_t pc = 0; pc < K; pc += KC) {                                              \
        size_t kc = K - pc < KC ? K - pc : KC;                                             \
        /* pack B[pc:pc+kc, jc:jc+nc] into NR-wide panels, zero padded */                  \
        for (size_t jp = 0; jp < npan; ++jp)                                               \
          for (size_t k = 0; k < kc; ++k) {                                                \
            float* dst = bp + (jp * kc + k) * NR;                                          \
            const float* src = B + (pc + k) * N + jc + jp * NR;                            \
            size_t w = nc - jp * NR < NR ? nc - jp * NR : NR;                              \
            for (size_t j = 0; j < w; ++j) dst[j] = src[j];                                \
            for (size_t j = w; j < NR; ++j) dst[j] = 0.0f;                                 \
          }                                                                                \
        for (size_t ic = 0; ic < M; ic += MC) {                                            \
          size_t mc = M - ic < MC ? M - ic : MC;                                           \
          size_t mpan = (mc + MR - 1) / MR;                                                \
          for (size_t ip = 0; ip < mpan; ++ip)                                             \
            for (size_t k = 0; k < kc; ++k) {                                              \
              float* dst = ap + (ip * kc + k) * MR;                                        \
              for (size_t r = 0; r < MR; ++r) {                                            \
                size_t row = ic + ip * MR + r;                                             \
                dst[r] = (ip * MR + r < mc) ? A[row * K + pc + k] : 0.0f;                  \
              }                                                                            \
            }                                                                              \
          for (size_t ip = 0; ip < mpan; ++ip)                                             \
            for (size_t jp = 0; jp < npan; ++jp) {                                         \
              v8 acc[MR][2];                                                               \
              memset(acc, 0, sizeof(acc));                                                 \
              const float* a = ap + ip * kc * MR;                                          \
              const float* b = bp + jp * kc * NR;                                          \
              for (size_t k = 0; k < kc; ++k) {                                            \
                v8 b0, b1;                                                                 \
                memcpy(&b0, b + k * NR, 32);                                               \
                memcpy(&b1, b + k * NR + 8, 32);                                           \
                for (size_t r = 0; r < MR; ++r) {                                          \
                  v8 av = {a[k * MR + r], a[k * MR + r], a[k * MR + r], a[k * MR + r],     \
                           a[k * MR + r], a[k * MR + r], a[k * MR + r], a[k * MR + r]};    \
                  acc[r][0] += av * b0;                                                    \
                  acc[r][1] += av * b1;                                                    \
                }                                                                          \
              }                                                                            \
              for (size_t r = 0; r < MR; ++r) {                                            \
                size_t row = ic + ip * MR + r;                                             \
                if (ip * MR + r >= mc) break;                                              \
                size_t w = nc - jp * NR < NR ? nc - jp * NR : NR;                          \
                float tmp[NR];                                                             \
                memcpy(tmp, &acc[r][0], 32);                                               \
                memcpy(tmp + 8, &acc[r][1], 32);                                           \
                float* c = C + row * N + jc + jp * NR;                                     \
                for (size_t j = 0; j < w; ++j) c[j] += tmp[j];                             \
              }                                                                            \
            }                                                                              \
        }                                                                                  \
      }                                                                                    \
    }                                                                                      \
    free(bp);                                                                              \
    free(ap);                                                                              \
    return 0;                                                                              \
  }

__attribute__((target("avx2,fma"))) static int sgemm_avx2(size_t M, size_t N, size_t K, const float* A,
                                                          const float* B, float* C) GEMM_BODY

static int sgemm_generic(size_t M, size_t N, size_t K, const float* A, const float* B, float* C) GEMM_BODY

/* Summation-order variants used only to measure how far valid f32 GEMMs drive
 * a training run apart: 0 = packed/blocked f32 with fused multiply-adds
 * (default), 1 = each dot product accumulated in f64 and rounded once, 2 = each
 * dot product in f32 in ascending k with a separate multiply and add (the
 * textbook loop), 3 = each dot product in f32 in descending k with fused
 * multiply-adds.  Variants 1-3 split the rows over OpenMP threads, which does
 * not change any element's order. */
static int g_variant = 0;
void orc_set_gemm_variant(int v) { g_variant = v; }

__attribute__((optimize("fp-contract=off"))) static int sgemm_f32_ascending(size_t M, size_t N, size_t K,
                                                                           const float* A, const float* B, float* C) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < M; ++i) {
    float* c = C + i * N;
    for (size_t j = 0; j < N; ++j) c[j] = 0.0f;
    for (size_t k = 0; k < K; ++k) {
      const float a = A[i * K + k];
      const float* b = B + k * N;
      for (size_t j = 0; j < N; ++j) {
        const float prod = a * b[j];
        c[j] = c[j] + prod;
      }
    }
  }
  return 0;
}

#define DESCENDING_FMA_BODY                                                        \
  {                                                                                \
    _Pragma("omp parallel for schedule(static)") for (size_t i = 0; i < M; ++i) {  \
      float* c = C + i * N;                                                        \
      for (size_t j = 0; j < N; ++j) c[j] = 0.0f;                                  \
      for (size_t k = K; k-- > 0;) {                                               \
        const float a = A[i * K + k];                                              \
        const float* b = B + k * N;                                                \
        for (size_t j = 0; j < N; ++j) c[j] = fmaf(a, b[j], c[j]);                 \
      }                                                                            \
    }                                                                              \
    return 0;                                                                      \
  }

__attribute__((target("avx2,fma"))) static int sgemm_desc_avx2(size_t M, size_t N, size_t K, const float* A,
                                                               const float* B, float* C) DESCENDING_FMA_BODY
static int sgemm_desc_generic(size_t M, size_t N, size_t K, const float* A, const float* B,
                              float* C) DESCENDING_FMA_BODY

static int sgemm_f32_descending_fma(size_t M, size_t N, size_t K, const float* A, const float* B, float* C) {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return sgemm_desc_avx2(M, N, K, A, B, C);
  return sgemm_desc_generic(M, N, K, A, B, C);
}

static int sgemm_f64acc(size_t M, size_t N, size_t K, const float* A, const float* B, float* C) {
  int failed = 0;
#pragma omp parallel
  {
    double* row = (double*)malloc(sizeof(double) * N);
    if (!row) {
#pragma omp atomic write
      failed = 1;
    }
#pragma omp for schedule(static)
    for (size_t i = 0; i < M; ++i) {
      if (!row) continue;
      for (size_t j = 0; j < N; ++j) row[j] = 0.0;
      for (size_t k = 0; k < K; ++k) {
        double a = A[i * K + k];
        const float* b = B + k * N;
        for (size_t j = 0; j < N; ++j) row[j] += a * (double)b[j];
      }
      for (size_t j = 0; j < N; ++j) C[i * N + j] = (float)row[j];
    }
    free(row);
  }
  return failed ? -1 : 0;
}

static int sgemm(size_t M, size_t N, size_t K, const float* A, const float* B, float* C) {
  if (M == 0 || N == 0) return 0;
  if (g_variant == 1) return sgemm_f64acc(M, N, K, A, B, C);
  if (g_variant == 2) return sgemm_f32_ascending(M, N, K, A, B, C);
  if (g_variant == 3) return sgemm_f32_descending_fma(M, N, K, A, B, C);
  if (K == 0) {
    memset(C, 0, sizeof(float) * M * N);
    return 0;
  }
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return sgemm_avx2(M, N, K, A, B, C);
  return sgemm_generic(M, N, K, A, B, C);
}

/* backend.rs:162-220 -- rank >= 2, equal batch dims, (..., M, K) x (..., K, N). */
int orc_matmul(const float* a, const float* b, float* out, const size_t* a_dims, size_t a_rank,
               const size_t* b_dims, size_t b_rank) {
  if (a_rank < 2 || b_rank < 2) return ORC_ERR_INTERNAL;
  if (a_rank != b_rank) return ORC_ERR_SHAPE;
  size_t batch = 1;
  for (size_t i = 0; i + 2 < a_rank; ++i) {
    if (a_dims[i] != b_dims[i]) return ORC_ERR_INTERNAL;
    batch *= a_dims[i];
  }
  size_t M = a_dims[a_rank - 2], K = a_dims[a_rank - 1], N = b_dims[b_rank - 1];
  if (b_dims[b_rank - 2] != K) return ORC_ERR_SHAPE;
  for (size_t i = 0; i < batch; ++i)
    if (sgemm(M, N, K, a + i * M * K, b + i * K * N, out + i * M * N)) return ORC_ERR_INTERNAL;
  return ORC_OK;
}
