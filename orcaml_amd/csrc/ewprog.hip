// Fused elementwise programs: a chain of the Backend trait's elementwise ops
// (orca-backend-cpu/src/backend.rs: add 104-128 ... div_backward_rhs 703-732)
// run as one pass over the elements.  The program is uniform over the grid
// (kernel arguments, read with scalar loads); each instruction applies the
// same functor as the op's own kernel (ew_ops.hpp), so the bits are those of
// the ops run one by one.  Registers live in VGPRs: the register file holds
// one 16-wide vector per component (plane j = component j of every
// register), and a register index, uniform over the wave, selects within the
// planes in place (s_set_gpr_idx) -- no scratch memory and no LDS traffic.
#include <cstdint>

#include "ew_ops.hpp"
#include "runtime.hpp"

namespace orca_hip {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
constexpr int kEwBlock = 256;
static_assert(ORCA_HIP_EW_MAX_REGS == 16, "one register per lane of a 16-wide plane");

// How element e of an input is read: in[(e / div) % mod].
enum : uint8_t {
  kPlain,      // in[e]
  kScalar,     // mod 1: in[0]
  kIndexed,    // n < 2^31: the division and the remainder by multiply and shift (Magic)
  kIndexed64,  // 64-bit division and remainder
  kRow4,       // kIndexed with div 1, mod % 4 == 0: 4 consecutive elements from one aligned float4
  kGroup4,     // kIndexed with div % 4 == 0: the 4 elements of an aligned group read one value
};

// floor(x / d) for 0 <= x < 2^31 as (x * m) >> s, with l = ceil(log2 d), s = 31 + l and
// m = ceil(2^s / d) < 2^32 (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, theorem 4.2: 2^s <= m d <= 2^s + 2^l makes it exact for
// every x below 2^31).
struct Magic {
  uint32_t m, s;
};

struct EwProgram {
  const float* in[ORCA_HIP_EW_MAX_INPUTS];
  uint64_t div[ORCA_HIP_EW_MAX_INPUTS], mod[ORCA_HIP_EW_MAX_INPUTS];
  Magic div_magic[ORCA_HIP_EW_MAX_INPUTS], mod_magic[ORCA_HIP_EW_MAX_INPUTS];
  uint8_t mode[ORCA_HIP_EW_MAX_INPUTS];
  float* out[ORCA_HIP_EW_MAX_OUTPUTS];
  uint8_t out_reg[ORCA_HIP_EW_MAX_OUTPUTS];
  uint32_t n_in, n_out, n_ops;
  orca_hip_ew_instr ins[ORCA_HIP_EW_MAX_OPS];
};

// Registers of 4 consecutive elements (RegFile4) or of one (RegFile1).
struct RegFile4 {
  typedef floatx4 V;
  floatx16 x, y, z, w;
  __device__ __forceinline__ V get(uint32_t r) const { return V{x[r], y[r], z[r], w[r]}; }
  __device__ __forceinline__ void set(uint32_t r, V v) {
    x[r] = v.x;
    y[r] = v.y;
    z[r] = v.z;
    w[r] = v.w;
  }
};
struct RegFile1 {
  typedef float V;
  floatx16 x;
  __device__ __forceinline__ V get(uint32_t r) const { return x[r]; }
  __device__ __forceinline__ void set(uint32_t r, V v) { x[r] = v; }
};

// f applied to each component.
template <class F>
__device__ __forceinline__ float lanes(F f, float a, float b, float c) {
  return f(a, b, c);
}
template <class F>
__device__ __forceinline__ floatx4 lanes(F f, floatx4 a, floatx4 b, floatx4 c) {
  return floatx4{f(a.x, b.x, c.x), f(a.y, b.y, c.y), f(a.z, b.z, c.z), f(a.w, b.w, c.w)};
}

#define EW_OP1(CODE, F) \
  case CODE:            \
    return lanes([](float x, float, float) { return F{}(x); }, a, b, c)
#define EW_OP2(CODE, F) \
  case CODE:            \
    return lanes([](float x, float y, float) { return F{}(x, y); }, a, b, c)

// All three operands are read before the switch: reading them inside the cases
// (fewer register moves on paper) measured 2-3x slower, the compiler's control
// flow for that form costing more than the moves saved.
template <class V>
__device__ __forceinline__ V ew_apply(const orca_hip_ew_instr& I, V a, V b, V c) {
  switch (I.op) {
    EW_OP2(ORCA_HIP_EW_ADD, OpAdd);
    EW_OP2(ORCA_HIP_EW_SUB, OpSub);
    EW_OP2(ORCA_HIP_EW_MUL, OpMul);
    EW_OP2(ORCA_HIP_EW_DIV, OpDiv);
    case ORCA_HIP_EW_MUL_SCALAR: {
      const float s = I.scalar;
      return lanes([s](float x, float, float) { return OpScale{s}(x); }, a, b, c);
    }
    EW_OP1(ORCA_HIP_EW_RELU, OpRelu);
    EW_OP2(ORCA_HIP_EW_RELU_BW, OpReluBw);
    EW_OP1(ORCA_HIP_EW_EXP, OpExp);
    EW_OP1(ORCA_HIP_EW_LOG, OpLog);
    EW_OP1(ORCA_HIP_EW_SQRT, OpSqrt);
    EW_OP1(ORCA_HIP_EW_SIGMOID, OpSigmoid);
    EW_OP2(ORCA_HIP_EW_EXP_BW, OpExpBw);
    EW_OP2(ORCA_HIP_EW_LOG_BW, OpLogBw);
    EW_OP2(ORCA_HIP_EW_SQRT_BW, OpSqrtBw);
    EW_OP2(ORCA_HIP_EW_SIGMOID_BW, OpSigBw);
    case ORCA_HIP_EW_DIV_BW_RHS:
      return lanes([](float x, float y, float z) { return OpDivBwRhs{}(x, y, z); }, a, b, c);
    EW_OP1(ORCA_HIP_EW_SUM_VISIT, OpSumVisit);
    EW_OP1(ORCA_HIP_EW_MAX_VISIT, OpMaxVisit);
    default:
      return a;  // ORCA_HIP_EW_COPY
  }
}
#undef EW_OP1
#undef EW_OP2

__device__ __forceinline__ uint32_t magic_div(uint32_t x, Magic g) {
  return (uint32_t)(((uint64_t)x * g.m) >> g.s);
}

// (e / div) % mod of input i for e < 2^31.
__device__ __forceinline__ uint32_t ew_index32(const EwProgram& p, uint32_t i, uint32_t e) {
  const uint32_t q = magic_div(e, p.div_magic[i]);
  return q - magic_div(q, p.mod_magic[i]) * (uint32_t)p.mod[i];
}

__device__ __forceinline__ float ew_input(const EwProgram& p, uint32_t i, size_t e) {
  switch (p.mode[i]) {
    case kPlain: return p.in[i][e];
    case kScalar: return p.in[i][0];
    case kIndexed64: return p.in[i][(e / p.div[i]) % p.mod[i]];
    default: return p.in[i][ew_index32(p, i, (uint32_t)e)];
  }
}

// Elements 4 idx .. 4 idx + 3 of input i (16-byte aligned, n a multiple of 4 past idx).
__device__ __forceinline__ floatx4 ew_input4(const EwProgram& p, uint32_t i, size_t idx) {
  const size_t e = 4 * idx;
  switch (p.mode[i]) {
    case kPlain: return reinterpret_cast<const floatx4*>(p.in[i])[idx];
    case kScalar: {
      const float v = p.in[i][0];
      return floatx4{v, v, v, v};
    }
    case kRow4: return *reinterpret_cast<const floatx4*>(p.in[i] + ew_index32(p, i, (uint32_t)e));
    case kGroup4: {
      const float v = p.in[i][ew_index32(p, i, (uint32_t)e)];
      return floatx4{v, v, v, v};
    }
    default:
      return floatx4{ew_input(p, i, e), ew_input(p, i, e + 1), ew_input(p, i, e + 2), ew_input(p, i, e + 3)};
  }
}

__device__ __forceinline__ floatx4 ew_load(const EwProgram& p, uint32_t i, size_t idx, floatx4*) {
  return ew_input4(p, i, idx);
}
__device__ __forceinline__ float ew_load(const EwProgram& p, uint32_t i, size_t idx, float*) {
  return ew_input(p, i, idx);
}

// Runs the program on element group idx: 4 elements 4 idx .. (RegFile4, 16-byte
// aligned buffers) or element idx (RegFile1).
template <class R>
__device__ __forceinline__ void ew_run(const EwProgram& p, size_t idx) {
  typedef typename R::V V;
  R rf;
  for (uint32_t i = 0; i < p.n_in; ++i) rf.set(i, ew_load(p, i, idx, (V*)nullptr));
  for (uint32_t k = 0; k < p.n_ops; ++k) {
    const orca_hip_ew_instr I = p.ins[k];
    rf.set(I.dst, ew_apply<V>(I, rf.get(I.a), rf.get(I.b), rf.get(I.c)));
  }
  for (uint32_t o = 0; o < p.n_out; ++o) reinterpret_cast<V*>(p.out[o])[idx] = rf.get(p.out_reg[o]);
}

__global__ void __launch_bounds__(kEwBlock) ew_program_vec_kernel(EwProgram p, size_t n) {
  const size_t n4 = n / 4, stride = (size_t)gridDim.x * kEwBlock;
  for (size_t i = (size_t)blockIdx.x * kEwBlock + threadIdx.x; i < n4; i += stride) ew_run<RegFile4>(p, i);
  // the last n % 4 elements, one per thread of block 0
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) ew_run<RegFile1>(p, 4 * n4 + threadIdx.x);
}

__global__ void __launch_bounds__(kEwBlock) ew_program_scalar_kernel(EwProgram p, size_t n) {
  const size_t stride = (size_t)gridDim.x * kEwBlock;
  for (size_t i = (size_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride) ew_run<RegFile1>(p, i);
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// Magic of a divisor 1 <= d <= 2^31.
Magic magic_for(uint64_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t two_s = uint64_t(1) << (31 + l);
  return Magic{(uint32_t)((two_s + d - 1) / d), 31 + l};
}

}  // namespace
}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_ew_program(orca_hip_ctx* ctx, size_t n, const orca_hip_ew_input* inputs, size_t n_inputs,
                        float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                        const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs) {
  return guard([&] {
    bind(ctx);
    if (n_inputs > ORCA_HIP_EW_MAX_INPUTS || n_outputs > ORCA_HIP_EW_MAX_OUTPUTS || n_instrs > ORCA_HIP_EW_MAX_OPS ||
        n_regs > ORCA_HIP_EW_MAX_REGS || n_regs < n_inputs || n_regs == 0 || n_outputs == 0)
      fail(ORCA_HIP_ERR_INTERNAL, "ew_program: program exceeds the interpreter's limits");
    if ((n_inputs && !inputs) || !outputs || !out_regs || (n_instrs && !instrs))
      fail(ORCA_HIP_ERR_INTERNAL, "ew_program: null program array");
    EwProgram p{};
    p.n_in = (uint32_t)n_inputs;
    p.n_out = (uint32_t)n_outputs;
    p.n_ops = (uint32_t)n_instrs;
    bool vec = true;
    for (size_t i = 0; i < n_inputs; ++i) {
      const orca_hip_ew_input& in = inputs[i];
      if (n && (!in.ptr || in.div == 0 || in.mod == 0)) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: invalid input");
      const bool plain = in.div == 1 && in.mod == n;
      if (n && !plain && in.mod > n) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: broadcast input larger than the output");
      check_extent(ctx, in.ptr, (plain ? n : in.mod) * sizeof(float), "ew_program (input)");
      p.in[i] = in.ptr;
      p.div[i] = in.div;
      p.mod[i] = in.mod;
      if (plain) {
        p.mode[i] = kPlain;
      } else if (in.mod == 1) {
        p.mode[i] = kScalar;
      } else if (n >= (uint64_t(1) << 31) || in.div >= (uint64_t(1) << 31)) {
        p.mode[i] = kIndexed64;
      } else {
        // here mod < n < 2^31 and div < 2^31
        p.div_magic[i] = magic_for(in.div);
        p.mod_magic[i] = magic_for(in.mod);
        p.mode[i] = (in.div == 1 && in.mod % 4 == 0) ? kRow4 : (in.div % 4 == 0) ? kGroup4 : kIndexed;
      }
      vec = vec && aligned16(in.ptr);
    }
    for (size_t o = 0; o < n_outputs; ++o) {
      if (!outputs[o] && n) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: null output");
      if (out_regs[o] >= n_regs) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: output register out of range");
      check_extent(ctx, outputs[o], n * sizeof(float), "ew_program (output)");
      p.out[o] = outputs[o];
      p.out_reg[o] = out_regs[o];
      vec = vec && aligned16(outputs[o]);
    }
    for (size_t k = 0; k < n_instrs; ++k) {
      const orca_hip_ew_instr& I = instrs[k];
      if (I.op > ORCA_HIP_EW_COPY || I.dst >= n_regs || I.a >= n_regs || I.b >= n_regs || I.c >= n_regs)
        fail(ORCA_HIP_ERR_INTERNAL, "ew_program: instruction " + std::to_string(k) + " is invalid");
      p.ins[k] = I;
    }
    if (n == 0) return;
    ProfScope ps(ctx, "ew_program", 0.0, 4.0 * (double)n * (n_inputs + n_outputs));
    if (vec) {
      const unsigned g = grid_for((n + 3) / 4, kEwBlock, ctx->num_cus * 8);
      hipLaunchKernelGGL(ew_program_vec_kernel, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, n);
    } else {
      const unsigned g = grid_for(n, kEwBlock, ctx->num_cus * 8);
      hipLaunchKernelGGL(ew_program_scalar_kernel, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, n);
    }
    ORCA_HIP_CHECK(hipGetLastError());
  });
}

}  // extern "C"
