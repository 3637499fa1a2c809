// The per-element operations of the Backend trait's elementwise ops, shared by
// their one-op kernels (ops.hip) and the fused elementwise-program interpreter
// (ewprog.hip), so both give the same bits.  Semantics follow
// orca-backend-cpu/src/backend.rs: relu is `x > 0 ? x : 0` (375-390), log
// clamps its input at 1e-7 (566-581), log_backward does not clamp (609-633).
// Every translation unit is built with -ffp-contract=off.
#pragma once

#include <cfloat>
#include <cmath>

namespace orca_hip {

struct OpAdd { __device__ float operator()(float a, float b) const { return a + b; } };
struct OpSub { __device__ float operator()(float a, float b) const { return a - b; } };
struct OpMul { __device__ float operator()(float a, float b) const { return a * b; } };
struct OpDiv { __device__ float operator()(float a, float b) const { return a / b; } };
struct OpReluBw { __device__ float operator()(float g, float x) const { return x > 0.0f ? g : 0.0f; } };
struct OpExpBw { __device__ float operator()(float g, float y) const { return g * y; } };
struct OpLogBw { __device__ float operator()(float g, float x) const { return g / x; } };
struct OpSqrtBw { __device__ float operator()(float g, float y) const { return g / (2.0f * y); } };
struct OpSigBw { __device__ float operator()(float g, float y) const { return (g * y) * (1.0f - y); } };
struct OpRelu { __device__ float operator()(float x) const { return x > 0.0f ? x : 0.0f; } };
struct OpExp { __device__ float operator()(float x) const { return expf(x); } };
struct OpLog { __device__ float operator()(float x) const { return logf(fmaxf(x, 1e-7f)); } };
struct OpSqrt { __device__ float operator()(float x) const { return sqrtf(x); } };
struct OpSigmoid { __device__ float operator()(float x) const { return 1.0f / (1.0f + expf(-x)); } };
struct OpScale {
  float s;
  __device__ float operator()(float x) const { return x * s; }
};
struct OpAddScalar {
  float s;
  __device__ float operator()(float x) const { return x + s; }
};
// One visit per output of sum_to_shape / max_to_shape (nothing reduced): the first step of
// the reduction from its start value, so -0 becomes +0 and NaN / -inf become -FLT_MAX.
struct OpSumVisit { __device__ float operator()(float x) const { return 0.0f + x; } };
struct OpMaxVisit { __device__ float operator()(float x) const { return x > -FLT_MAX ? x : -FLT_MAX; } };
struct OpDivBwRhs {  // g * (-l / (r * r))
  __device__ float operator()(float g, float l, float r) const { return g * (-l / (r * r)); }
};

}  // namespace orca_hip
