// Fused elementwise programs: a chain of the Backend trait's elementwise ops
// (orca-backend-cpu/src/backend.rs: add 104-128 ... div_backward_rhs 703-732)
// run as one pass over the elements.  The program is uniform over the grid
// (kernel arguments, read with scalar loads); each instruction applies the
// same functor as the op's own kernel (ew_ops.hpp), so the bits are those of
// the ops run one by one.  Registers live in VGPRs: the register file holds
// one 16-wide vector per component (plane j = component j of every
// register), and a register index, uniform over the wave, selects within the
// planes in place (s_set_gpr_idx) -- no scratch memory and no LDS traffic.
#include <dlfcn.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

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
    case ORCA_HIP_EW_ADD_SCALAR: {
      const float s = I.scalar;
      return lanes([s](float x, float, float) { return OpAddScalar{s}(x); }, a, b, c);
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

// The program over a [rows, cols] block and the row reduction of one register: each block
// takes rows_per_block whole rows, one thread per element (coalesced as the plain kernel);
// the reduced register's values go through LDS and thread r of the block combines its
// row's values in column order as sum_to_shape's and max_to_shape's loops do (a sum from
// +0, a maximum from -FLT_MAX that a value replaces only when greater), so reduced[r] has
// the bits of that reduction of the program's value.
template <bool IS_MAX>
__global__ void __launch_bounds__(kEwBlock) ew_program_rows_kernel(EwProgram p, size_t rows, uint32_t cols,
                                                                    uint32_t rows_per_block, uint32_t red_reg,
                                                                    float* __restrict__ reduced) {
  __shared__ float vals[kEwBlock];
  const size_t r0 = (size_t)blockIdx.x * rows_per_block;
  const uint32_t nr = rows - r0 < rows_per_block ? (uint32_t)(rows - r0) : rows_per_block;
  const uint32_t t = threadIdx.x;
  if (t < nr * cols) {
    const size_t e = r0 * cols + t;
    RegFile1 rf;
    for (uint32_t i = 0; i < p.n_in; ++i) rf.set(i, ew_input(p, i, e));
    for (uint32_t k = 0; k < p.n_ops; ++k) {
      const orca_hip_ew_instr I = p.ins[k];
      rf.set(I.dst, ew_apply<float>(I, rf.get(I.a), rf.get(I.b), rf.get(I.c)));
    }
    for (uint32_t o = 0; o < p.n_out; ++o) p.out[o][e] = rf.get(p.out_reg[o]);
    vals[t] = rf.get(red_reg);
  }
  __syncthreads();
  if (t < nr) {
    float acc = IS_MAX ? -FLT_MAX : 0.0f;
    for (uint32_t c = 0; c < cols; ++c) {
      const float v = vals[t * cols + c];
      if (IS_MAX) {
        if (v > acc) acc = v;
      } else {
        acc = acc + v;
      }
    }
    reduced[r0 + t] = acc;
  }
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// Magic of a divisor 1 <= d <= 2^31.
Magic magic_for(uint64_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t two_s = uint64_t(1) << (31 + l);
  return Magic{(uint32_t)((two_s + d - 1) / d), 31 + l};
}

// The access of an input (plain inputs have div 1, mod n).
uint8_t input_mode(size_t n, uint64_t div, uint64_t mod) {
  if (div == 1 && mod == n) return kPlain;
  if (mod == 1) return kScalar;
  if (n >= (uint64_t(1) << 31) || div >= (uint64_t(1) << 31)) return kIndexed64;
  return (div == 1 && mod % 4 == 0) ? kRow4 : (div % 4 == 0) ? kGroup4 : kIndexed;
}

// Checks a program against the limits and that every register is written
// before it is read (inputs are registers 0 .. n_inputs - 1).
void check_program(size_t n_inputs, const uint8_t* out_regs, size_t n_outputs, const orca_hip_ew_instr* instrs,
                   size_t n_instrs, size_t n_regs) {
  if (n_inputs > ORCA_HIP_EW_MAX_INPUTS || n_outputs > ORCA_HIP_EW_MAX_OUTPUTS || n_instrs > ORCA_HIP_EW_MAX_OPS ||
      n_regs > ORCA_HIP_EW_MAX_REGS || n_regs < n_inputs || n_regs == 0 || n_outputs == 0)
    fail(ORCA_HIP_ERR_INTERNAL, "ew_program: program exceeds the interpreter's limits");
  if (!out_regs || (n_instrs && !instrs)) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: null program array");
  uint32_t written = n_inputs ? (1u << n_inputs) - 1 : 0;
  auto readable = [&](uint8_t r) { return r < n_regs && ((written >> r) & 1); };
  for (size_t k = 0; k < n_instrs; ++k) {
    const orca_hip_ew_instr& I = instrs[k];
    const bool three = I.op == ORCA_HIP_EW_DIV_BW_RHS;
    const bool two = three || I.op == ORCA_HIP_EW_ADD || I.op == ORCA_HIP_EW_SUB || I.op == ORCA_HIP_EW_MUL ||
                     I.op == ORCA_HIP_EW_DIV || I.op == ORCA_HIP_EW_RELU_BW || I.op == ORCA_HIP_EW_EXP_BW ||
                     I.op == ORCA_HIP_EW_LOG_BW || I.op == ORCA_HIP_EW_SQRT_BW || I.op == ORCA_HIP_EW_SIGMOID_BW;
    if (I.op > ORCA_HIP_EW_ADD_SCALAR || I.dst >= n_regs || I.b >= n_regs || I.c >= n_regs || !readable(I.a) ||
        (two && !readable(I.b)) || (three && !readable(I.c)))
      fail(ORCA_HIP_ERR_INTERNAL, "ew_program: instruction " + std::to_string(k) + " is invalid");
    written |= 1u << I.dst;
  }
  for (size_t o = 0; o < n_outputs; ++o)
    if (!readable(out_regs[o])) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: output register out of range");
}

}  // namespace

// ---------------------------------------------------------------------------
// Run-time compiled programs.  A program structure (opcodes, operand
// registers, outputs, each input's access) that recurs is compiled once into a
// straight-line kernel by hipRTC: every instruction becomes one SSA value of
// the same functor from ew_ops.hpp (the header's text is compiled in), so the
// bits are the interpreter's; the scalars, input pointers and index constants
// are kernel arguments, so one kernel serves every size and every step.  The
// compile options are those of the library's own build (-O3,
// -ffp-contract=off, no packed FP32), for which hipRTC and hipcc emit the same
// instructions.  hipRTC is loaded with dlopen at the first compile; without it,
// or when a compile fails, the program stays on the interpreter.

// Kernel arguments of a compiled program.  The generated source declares the
// same struct from the same token list.
#define ORCA_EW_JIT_ARGS_FIELDS                                                                              \
  const float* in[8];                                                                                     \
  unsigned long long div[8];                                                                              \
  unsigned long long mod[8];                                                                              \
  unsigned int dm[8], ds[8], mm[8], ms[8];                                                                \
  float* out[8];                                                                                          \
  float sc[64];                                                                                           \
  unsigned long long n;
#define ORCA_EW_STR2(...) #__VA_ARGS__
#define ORCA_EW_STR(...) ORCA_EW_STR2(__VA_ARGS__)

namespace {

struct JitArgs {
  ORCA_EW_JIT_ARGS_FIELDS
};
static_assert(sizeof(JitArgs::in) / sizeof(JitArgs::in[0]) == ORCA_HIP_EW_MAX_INPUTS, "inputs");
static_assert(sizeof(JitArgs::out) / sizeof(JitArgs::out[0]) == ORCA_HIP_EW_MAX_OUTPUTS, "outputs");
static_assert(sizeof(JitArgs::sc) / sizeof(JitArgs::sc[0]) == ORCA_HIP_EW_MAX_OPS, "scalars");

const char kEwOpsText[] =
#include "ew_ops_text.inc"
    ;

const char kJitPrelude[] =
    "#include \"ew_ops.hpp\"\n"
    "typedef float floatx4 __attribute__((ext_vector_type(4)));\n"
    "using namespace orca_hip;\n"
    "struct JitArgs { " ORCA_EW_STR(ORCA_EW_JIT_ARGS_FIELDS) " };\n"
    "__device__ __forceinline__ unsigned mdiv(unsigned x, unsigned m, unsigned s) {\n"
    "  return (unsigned)(((unsigned long long)x * m) >> s);\n"
    "}\n"
    "__device__ __forceinline__ unsigned ix32(const JitArgs& p, int i, unsigned e) {\n"
    "  const unsigned q = mdiv(e, p.dm[i], p.ds[i]);\n"
    "  return q - mdiv(q, p.mm[i], p.ms[i]) * (unsigned)p.mod[i];\n"
    "}\n"
    "__device__ __forceinline__ unsigned long long ix64(const JitArgs& p, int i, unsigned long long e) {\n"
    "  return (e / p.div[i]) % p.mod[i];\n"
    "}\n"
    "__device__ __forceinline__ floatx4 bc4(float v) { return floatx4{v, v, v, v}; }\n"
    "template <class F> __device__ __forceinline__ float L1(F f, float a) { return f(a); }\n"
    "template <class F> __device__ __forceinline__ floatx4 L1(F f, floatx4 a) {\n"
    "  return floatx4{f(a.x), f(a.y), f(a.z), f(a.w)};\n"
    "}\n"
    "template <class F> __device__ __forceinline__ float L2(F f, float a, float b) { return f(a, b); }\n"
    "template <class F> __device__ __forceinline__ floatx4 L2(F f, floatx4 a, floatx4 b) {\n"
    "  return floatx4{f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w)};\n"
    "}\n"
    "template <class F> __device__ __forceinline__ float L3(F f, float a, float b, float c) { return f(a, b, c); }\n"
    "template <class F> __device__ __forceinline__ floatx4 L3(F f, floatx4 a, floatx4 b, floatx4 c) {\n"
    "  return floatx4{f(a.x, b.x, c.x), f(a.y, b.y, c.y), f(a.z, b.z, c.z), f(a.w, b.w, c.w)};\n"
    "}\n";

// Functor and arity of an opcode (the scalar ops and ORCA_HIP_EW_COPY are written inline).
struct JitOp {
  int arity;
  const char* functor;
};
JitOp jit_op(uint8_t op) {
  switch (op) {
    case ORCA_HIP_EW_ADD: return {2, "OpAdd{}"};
    case ORCA_HIP_EW_SUB: return {2, "OpSub{}"};
    case ORCA_HIP_EW_MUL: return {2, "OpMul{}"};
    case ORCA_HIP_EW_DIV: return {2, "OpDiv{}"};
    case ORCA_HIP_EW_MUL_SCALAR: return {1, nullptr};
    case ORCA_HIP_EW_ADD_SCALAR: return {1, nullptr};
    case ORCA_HIP_EW_RELU: return {1, "OpRelu{}"};
    case ORCA_HIP_EW_RELU_BW: return {2, "OpReluBw{}"};
    case ORCA_HIP_EW_EXP: return {1, "OpExp{}"};
    case ORCA_HIP_EW_LOG: return {1, "OpLog{}"};
    case ORCA_HIP_EW_SQRT: return {1, "OpSqrt{}"};
    case ORCA_HIP_EW_SIGMOID: return {1, "OpSigmoid{}"};
    case ORCA_HIP_EW_EXP_BW: return {2, "OpExpBw{}"};
    case ORCA_HIP_EW_LOG_BW: return {2, "OpLogBw{}"};
    case ORCA_HIP_EW_SQRT_BW: return {2, "OpSqrtBw{}"};
    case ORCA_HIP_EW_SIGMOID_BW: return {2, "OpSigBw{}"};
    case ORCA_HIP_EW_DIV_BW_RHS: return {3, "OpDivBwRhs{}"};
    case ORCA_HIP_EW_SUM_VISIT: return {1, "OpSumVisit{}"};
    case ORCA_HIP_EW_MAX_VISIT: return {1, "OpMaxVisit{}"};
    default: return {1, nullptr};  // ORCA_HIP_EW_COPY
  }
}

// Loads of input i (access `mode`) for element e: the 4-element group q (vec) or one element.
std::string jit_load(int i, uint8_t mode, bool vec) {
  const std::string in = "p.in[" + std::to_string(i) + "]", is = std::to_string(i);
  const std::string i32 = "ix32(p, " + is + ", (unsigned)(e", i64 = "ix64(p, " + is + ", e";
  if (!vec) {
    switch (mode) {
      case kPlain: return in + "[e]";
      case kScalar: return in + "[0]";
      case kIndexed64: return in + "[" + i64 + ")]";
      default: return in + "[" + i32 + "))]";
    }
  }
  switch (mode) {
    case kPlain: return "reinterpret_cast<const floatx4*>(" + in + ")[q]";
    case kScalar: return "bc4(" + in + "[0])";
    case kRow4: return "*reinterpret_cast<const floatx4*>(" + in + " + " + i32 + ")))";
    case kGroup4: return "bc4(" + in + "[" + i32 + "))])";
    case kIndexed64: {
      std::string r = "floatx4{";
      for (int j = 0; j < 4; ++j) r += (j ? ", " : "") + in + "[" + i64 + " + " + std::to_string(j) + ")]";
      return r + "}";
    }
    default: {
      std::string r = "floatx4{";
      for (int j = 0; j < 4; ++j) r += (j ? ", " : "") + in + "[" + i32 + " + " + std::to_string(j) + "))]";
      return r + "}";
    }
  }
}

// The body of one element (vec = false) or one 4-element group q (vec = true) at element e.
std::string jit_body(size_t n_in, const uint8_t* modes, size_t n_out, const uint8_t* out_regs,
                     const orca_hip_ew_instr* instrs, size_t n_instrs, bool vec, const char* indent) {
  std::string b;
  std::vector<std::string> name(ORCA_HIP_EW_MAX_REGS);
  const char* V = vec ? "floatx4" : "float";
  for (size_t i = 0; i < n_in; ++i) {
    name[i] = "x" + std::to_string(i);
    b += std::string(indent) + "const " + V + " " + name[i] + " = " + jit_load((int)i, modes[i], vec) + ";\n";
  }
  for (size_t k = 0; k < n_instrs; ++k) {
    const orca_hip_ew_instr& I = instrs[k];
    const JitOp op = jit_op(I.op);
    const std::string t = "t" + std::to_string(k);
    std::string expr;
    if (I.op == ORCA_HIP_EW_MUL_SCALAR)
      expr = "L1(OpScale{p.sc[" + std::to_string(k) + "]}, " + name[I.a] + ")";
    else if (I.op == ORCA_HIP_EW_ADD_SCALAR)
      expr = "L1(OpAddScalar{p.sc[" + std::to_string(k) + "]}, " + name[I.a] + ")";
    else if (!op.functor)
      expr = name[I.a];
    else if (op.arity == 1)
      expr = std::string("L1(") + op.functor + ", " + name[I.a] + ")";
    else if (op.arity == 2)
      expr = std::string("L2(") + op.functor + ", " + name[I.a] + ", " + name[I.b] + ")";
    else
      expr = std::string("L3(") + op.functor + ", " + name[I.a] + ", " + name[I.b] + ", " + name[I.c] + ")";
    b += std::string(indent) + "const " + V + " " + t + " = " + expr + ";\n";
    name[I.dst] = t;
  }
  for (size_t o = 0; o < n_out; ++o) {
    const std::string out = "p.out[" + std::to_string(o) + "]";
    b += std::string(indent) +
         (vec ? "reinterpret_cast<floatx4*>(" + out + ")[q] = " : out + "[e] = ") + name[out_regs[o]] + ";\n";
  }
  return b;
}

// The source of a program's two kernels: ew_fused_vec (16-byte aligned
// buffers, 4 elements per thread, the last n % 4 in block 0) and
// ew_fused_scalar (any alignment).  Both stride over the grid.
std::string jit_source(size_t n_in, const uint8_t* modes, size_t n_out, const uint8_t* out_regs,
                       const orca_hip_ew_instr* instrs, size_t n_instrs) {
  std::string s = kJitPrelude;
  s += "extern \"C\" __global__ void __launch_bounds__(256) ew_fused_vec(JitArgs p) {\n"
       "  const unsigned long long n = p.n, n4 = n / 4, stride = (unsigned long long)gridDim.x * 256;\n"
       "  for (unsigned long long q = (unsigned long long)blockIdx.x * 256 + threadIdx.x; q < n4; q += stride) {\n"
       "    const unsigned long long e = 4 * q;\n";
  s += jit_body(n_in, modes, n_out, out_regs, instrs, n_instrs, true, "    ");
  s += "  }\n"
       "  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {\n"
       "    const unsigned long long e = 4 * n4 + threadIdx.x;\n";
  s += jit_body(n_in, modes, n_out, out_regs, instrs, n_instrs, false, "    ");
  s += "  }\n"
       "}\n"
       "extern \"C\" __global__ void __launch_bounds__(256) ew_fused_scalar(JitArgs p) {\n"
       "  const unsigned long long n = p.n, stride = (unsigned long long)gridDim.x * 256;\n"
       "  for (unsigned long long e = (unsigned long long)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {\n";
  s += jit_body(n_in, modes, n_out, out_regs, instrs, n_instrs, false, "    ");
  s += "  }\n"
       "}\n";
  return s;
}

// hipRTC, loaded on first use.
struct Hiprtc {
  bool ok = false;
  decltype(&hiprtcCreateProgram) create = nullptr;
  decltype(&hiprtcCompileProgram) compile = nullptr;
  decltype(&hiprtcGetProgramLogSize) log_size = nullptr;
  decltype(&hiprtcGetProgramLog) log = nullptr;
  decltype(&hiprtcGetCodeSize) code_size = nullptr;
  decltype(&hiprtcGetCode) code = nullptr;
  decltype(&hiprtcDestroyProgram) destroy = nullptr;
};
const Hiprtc& hiprtc() {
  static const Hiprtc h = [] {
    Hiprtc r;
    void* lib = dlopen("libhiprtc.so.7", RTLD_NOW | RTLD_LOCAL);
    if (!lib) lib = dlopen("libhiprtc.so", RTLD_NOW | RTLD_LOCAL);
    if (!lib) return r;
    r.create = reinterpret_cast<decltype(r.create)>(dlsym(lib, "hiprtcCreateProgram"));
    r.compile = reinterpret_cast<decltype(r.compile)>(dlsym(lib, "hiprtcCompileProgram"));
    r.log_size = reinterpret_cast<decltype(r.log_size)>(dlsym(lib, "hiprtcGetProgramLogSize"));
    r.log = reinterpret_cast<decltype(r.log)>(dlsym(lib, "hiprtcGetProgramLog"));
    r.code_size = reinterpret_cast<decltype(r.code_size)>(dlsym(lib, "hiprtcGetCodeSize"));
    r.code = reinterpret_cast<decltype(r.code)>(dlsym(lib, "hiprtcGetCode"));
    r.destroy = reinterpret_cast<decltype(r.destroy)>(dlsym(lib, "hiprtcDestroyProgram"));
    r.ok = r.create && r.compile && r.log_size && r.log && r.code_size && r.code && r.destroy;
    return r;
  }();
  return h;
}

// Compiles a program's source to a code object; empty with *log set on failure.
std::string jit_compile(const std::string& src, std::string* log) {
  const Hiprtc& rtc = hiprtc();
  if (!rtc.ok) {
    *log = "hipRTC not available";
    return {};
  }
  const char* headers[] = {kEwOpsText, "#pragma once\n#define FLT_MAX 3.40282347e+38F\n", "#pragma once\n"};
  const char* names[] = {"ew_ops.hpp", "cfloat", "cmath"};
  hiprtcProgram prog = nullptr;
  if (rtc.create(&prog, src.c_str(), "ew_fused.hip", 3, headers, names) != HIPRTC_SUCCESS) {
    *log = "hiprtcCreateProgram failed";
    return {};
  }
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops"};
  std::string code;
  if (rtc.compile(prog, 7, opts) == HIPRTC_SUCCESS) {
    size_t size = 0;
    if (rtc.code_size(prog, &size) == HIPRTC_SUCCESS && size) {
      code.resize(size);
      if (rtc.code(prog, &code[0]) != HIPRTC_SUCCESS) code.clear();
    }
  }
  if (code.empty()) {
    size_t size = 0;
    if (rtc.log_size(prog, &size) == HIPRTC_SUCCESS && size) {
      log->resize(size);
      rtc.log(prog, &(*log)[0]);
    }
  }
  rtc.destroy(&prog);
  return code;
}

struct JitEntry {
  uint32_t uses = 0;
  bool failed = false;
  hipModule_t module = nullptr;
  hipFunction_t vec = nullptr, scalar = nullptr;
};

// Structure key of a program: input accesses, output registers, instructions without their scalars.
std::string jit_key(size_t n_in, const uint8_t* modes, size_t n_out, const uint8_t* out_regs,
                    const orca_hip_ew_instr* instrs, size_t n_instrs) {
  std::string k;
  k.reserve(4 + n_in + n_out + 5 * n_instrs);
  k.push_back((char)n_in);
  k.push_back((char)n_out);
  k.push_back((char)n_instrs);
  k.append(reinterpret_cast<const char*>(modes), n_in);
  k.append(reinterpret_cast<const char*>(out_regs), n_out);
  for (size_t i = 0; i < n_instrs; ++i) {
    const orca_hip_ew_instr& I = instrs[i];
    const char c[5] = {(char)I.op, (char)I.dst, (char)I.a, (char)I.b, (char)I.c};
    k.append(c, 5);
  }
  return k;
}

}  // namespace

struct EwJitCache {
  std::mutex mu;
  std::unordered_map<std::string, JitEntry> programs;
  uint64_t interpreted = 0, compiled_launches = 0, compiles = 0, failures = 0;
};

void ew_jit_release(orca_hip_ctx* ctx) {
  if (!ctx->ew_jit) return;
  for (auto& kv : ctx->ew_jit->programs)
    if (kv.second.module) (void)hipModuleUnload(kv.second.module);
  delete ctx->ew_jit;
  ctx->ew_jit = nullptr;
}

namespace {

// The compiled kernel of this program (the aligned or the general one), or
// null when it runs on the interpreter.  Compiles at the use the context's
// mode asks for.
hipFunction_t jit_kernel(orca_hip_ctx* ctx, const EwProgram& p, bool vec) {
  if (ctx->ew_jit_mode <= 0) return nullptr;
  if (!ctx->ew_jit) ctx->ew_jit = new EwJitCache();
  EwJitCache& c = *ctx->ew_jit;
  std::lock_guard<std::mutex> lk(c.mu);
  JitEntry& e = c.programs[jit_key(p.n_in, p.mode, p.n_out, p.out_reg, p.ins, p.n_ops)];
  ++e.uses;
  // At most kMaxCompiled structures per context get a module of their own; past that
  // (a workload that keeps building new chain shapes) new structures stay interpreted.
  constexpr uint64_t kMaxCompiled = 4096;
  if (!e.module && !e.failed && c.compiles < kMaxCompiled && (ctx->ew_jit_mode >= 2 || e.uses >= 2)) {
    std::string log;
    const std::string code = jit_compile(jit_source(p.n_in, p.mode, p.n_out, p.out_reg, p.ins, p.n_ops), &log);
    hipModule_t m = nullptr;
    if (!code.empty() && hipModuleLoadData(&m, code.data()) == hipSuccess) {
      hipFunction_t fv = nullptr, fs = nullptr;
      if (hipModuleGetFunction(&fv, m, "ew_fused_vec") == hipSuccess &&
          hipModuleGetFunction(&fs, m, "ew_fused_scalar") == hipSuccess) {
        e.module = m;
        e.vec = fv;
        e.scalar = fs;
        ++c.compiles;
      } else {
        (void)hipModuleUnload(m);
      }
    }
    (void)hipGetLastError();
    if (!e.module) {
      e.failed = true;
      if (c.failures++ == 0)  // said once per context; the structure stays on the interpreter
        std::fprintf(stderr, "orca_hip: compiling a fused elementwise program failed, interpreting it instead: %.800s\n",
                     log.empty() ? "module load failed" : log.c_str());
    }
  }
  if (!e.module) {
    ++c.interpreted;
    return nullptr;
  }
  ++c.compiled_launches;
  return vec ? e.vec : e.scalar;
}

}  // namespace
}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_ew_program_rows(orca_hip_ctx* ctx, size_t rows, size_t cols, const orca_hip_ew_input* inputs,
                             size_t n_inputs, float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                             const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs, int red_reg,
                             int reduce_max, float* reduced) {
  return guard([&] {
    bind(ctx);
    check_program(n_inputs, out_regs, n_outputs, instrs, n_instrs, n_regs);
    if ((n_inputs && !inputs) || !outputs) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: null program array");
    if (cols == 0 || cols > 64) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: needs 1 <= cols <= 64");
    if (rows > ((size_t)1 << 31) / cols) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: too many elements");
    if (red_reg < 0 || (size_t)red_reg >= n_regs) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: bad register");
    bool readable = red_reg < (int)n_inputs;
    for (size_t k = 0; k < n_instrs; ++k) readable = readable || instrs[k].dst == red_reg;
    if (!readable) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: the reduced register is never written");
    const size_t n = rows * cols;
    check_extent(ctx, reduced, rows * sizeof(float), "ew_program_rows (reduced)");
    if (rows && !reduced) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: null reduced output");
    EwProgram p{};
    p.n_in = (uint32_t)n_inputs;
    p.n_out = (uint32_t)n_outputs;
    p.n_ops = (uint32_t)n_instrs;
    for (size_t i = 0; i < n_inputs; ++i) {
      const orca_hip_ew_input& in = inputs[i];
      if (n && (!in.ptr || in.div == 0 || in.mod == 0)) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: invalid input");
      const bool plain = in.div == 1 && in.mod == n;
      if (n && !plain && in.mod > n) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: broadcast input larger than the output");
      check_extent(ctx, in.ptr, (plain ? n : in.mod) * sizeof(float), "ew_program_rows (input)");
      p.in[i] = in.ptr;
      p.div[i] = in.div;
      p.mod[i] = in.mod;
      p.mode[i] = n ? input_mode(n, in.div, in.mod) : (uint8_t)kPlain;
      if (p.mode[i] == kRow4 || p.mode[i] == kGroup4) p.mode[i] = kIndexed;  // one element at a time here
      if (p.mode[i] == kIndexed) {
        p.div_magic[i] = magic_for(in.div);
        p.mod_magic[i] = magic_for(in.mod);
      }
    }
    for (size_t o = 0; o < n_outputs; ++o) {
      if (!outputs[o] && n) fail(ORCA_HIP_ERR_INTERNAL, "ew_program_rows: null output");
      check_extent(ctx, outputs[o], n * sizeof(float), "ew_program_rows (output)");
      p.out[o] = outputs[o];
      p.out_reg[o] = out_regs[o];
    }
    for (size_t k = 0; k < n_instrs; ++k) p.ins[k] = instrs[k];
    if (rows == 0) return;
    ProfScope ps(ctx, ctx->main ? "ew_program_rows_overlapped" : "ew_program_rows", 0.0,
                 4.0 * (double)n * (n_inputs + n_outputs) + 4.0 * rows);
    // whole rows per block: rows_per_block * cols <= kEwBlock elements
    const uint32_t rpb = (uint32_t)(kEwBlock / cols);
    const unsigned g = (unsigned)((rows + rpb - 1) / rpb);
    if (reduce_max)
      hipLaunchKernelGGL(ew_program_rows_kernel<true>, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, rows,
                         (uint32_t)cols, rpb, (uint32_t)red_reg, reduced);
    else
      hipLaunchKernelGGL(ew_program_rows_kernel<false>, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, rows,
                         (uint32_t)cols, rpb, (uint32_t)red_reg, reduced);
    ORCA_HIP_CHECK(hipGetLastError());
  });
}

int orca_hip_ew_program(orca_hip_ctx* ctx, size_t n, const orca_hip_ew_input* inputs, size_t n_inputs,
                        float* const* outputs, const uint8_t* out_regs, size_t n_outputs,
                        const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs) {
  return guard([&] {
    bind(ctx);
    check_program(n_inputs, out_regs, n_outputs, instrs, n_instrs, n_regs);
    if ((n_inputs && !inputs) || !outputs) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: null program array");
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
      p.mode[i] = n ? input_mode(n, in.div, in.mod) : (uint8_t)kPlain;
      if (p.mode[i] == kRow4 || p.mode[i] == kGroup4 || p.mode[i] == kIndexed) {
        // here mod < n < 2^31 and div < 2^31
        p.div_magic[i] = magic_for(in.div);
        p.mod_magic[i] = magic_for(in.mod);
      }
      vec = vec && aligned16(in.ptr);
    }
    for (size_t o = 0; o < n_outputs; ++o) {
      if (!outputs[o] && n) fail(ORCA_HIP_ERR_INTERNAL, "ew_program: null output");
      check_extent(ctx, outputs[o], n * sizeof(float), "ew_program (output)");
      p.out[o] = outputs[o];
      p.out_reg[o] = out_regs[o];
      vec = vec && aligned16(outputs[o]);
    }
    for (size_t k = 0; k < n_instrs; ++k) p.ins[k] = instrs[k];
    if (n == 0) return;
    ProfScope ps(ctx, ctx->main ? "ew_program_overlapped" : "ew_program", 0.0, 4.0 * (double)n * (n_inputs + n_outputs));
    // On the side stream a bounded grid leaves room for a product running beside it (the
    // kernels stride over the grid, so any grid covers n).
    const unsigned cap = ctx->main && ctx->side_bpc > 0 ? (unsigned)(ctx->side_bpc * ctx->num_cus) : ctx->num_cus * 8;
    const unsigned g = vec ? grid_for((n + 3) / 4, kEwBlock, cap) : grid_for(n, kEwBlock, cap);
    if (hipFunction_t fn = jit_kernel(ctx, p, vec)) {
      JitArgs a{};
      for (size_t i = 0; i < n_inputs; ++i) {
        a.in[i] = p.in[i];
        a.div[i] = p.div[i];
        a.mod[i] = p.mod[i];
        a.dm[i] = p.div_magic[i].m;
        a.ds[i] = p.div_magic[i].s;
        a.mm[i] = p.mod_magic[i].m;
        a.ms[i] = p.mod_magic[i].s;
      }
      for (size_t o = 0; o < n_outputs; ++o) a.out[o] = p.out[o];
      for (size_t k = 0; k < n_instrs; ++k) a.sc[k] = p.ins[k].scalar;
      a.n = n;
      void* args[] = {&a};
      ORCA_HIP_CHECK(hipModuleLaunchKernel(fn, g, 1, 1, kEwBlock, 1, 1, 0, ctx->stream, args, nullptr));
    } else if (vec) {
      hipLaunchKernelGGL(ew_program_vec_kernel, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, n);
    } else {
      hipLaunchKernelGGL(ew_program_scalar_kernel, dim3(g), dim3(kEwBlock), 0, ctx->stream, p, n);
    }
    ORCA_HIP_CHECK(hipGetLastError());
  });
}

int orca_hip_ew_set_jit(orca_hip_ctx* ctx, int mode) {
  return guard([&] {
    check_ctx(ctx);
    if (mode < 0 || mode > 2) fail(ORCA_HIP_ERR_INTERNAL, "ew_set_jit: mode must be 0, 1 or 2");
    ctx->ew_jit_mode = mode;
  });
}

int orca_hip_ew_jit_stats(orca_hip_ctx* ctx, uint64_t* interpreted, uint64_t* compiled_launches, uint64_t* compiles,
                          uint64_t* failures) {
  return guard([&] {
    check_ctx(ctx);
    uint64_t v[4] = {0, 0, 0, 0};
    if (ctx->ew_jit) {
      std::lock_guard<std::mutex> lk(ctx->ew_jit->mu);
      v[0] = ctx->ew_jit->interpreted;
      v[1] = ctx->ew_jit->compiled_launches;
      v[2] = ctx->ew_jit->compiles;
      v[3] = ctx->ew_jit->failures;
    }
    if (interpreted) *interpreted = v[0];
    if (compiled_launches) *compiled_launches = v[1];
    if (compiles) *compiles = v[2];
    if (failures) *failures = v[3];
  });
}

int orca_hip_ew_jit_source(size_t n, const orca_hip_ew_input* inputs, size_t n_inputs, const uint8_t* out_regs,
                           size_t n_outputs, const orca_hip_ew_instr* instrs, size_t n_instrs, size_t n_regs, char* buf,
                           size_t len, size_t* needed) {
  return guard([&] {
    check_program(n_inputs, out_regs, n_outputs, instrs, n_instrs, n_regs);
    if (n_inputs && !inputs) fail(ORCA_HIP_ERR_INTERNAL, "ew_jit_source: null inputs");
    uint8_t modes[ORCA_HIP_EW_MAX_INPUTS];
    for (size_t i = 0; i < n_inputs; ++i) {
      if (inputs[i].div == 0 || inputs[i].mod == 0) fail(ORCA_HIP_ERR_INTERNAL, "ew_jit_source: invalid input");
      modes[i] = input_mode(n, inputs[i].div, inputs[i].mod);
    }
    const std::string src = jit_source(n_inputs, modes, n_outputs, out_regs, instrs, n_instrs);
    if (needed) *needed = src.size() + 1;
    if (buf && len) {
      const size_t m = std::min(len - 1, src.size());
      std::memcpy(buf, src.data(), m);
      buf[m] = '\0';
    }
  });
}

int orca_hip_ew_jit_headers(const char** ew_ops_text) {
  return guard([&] {
    if (!ew_ops_text) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    *ew_ops_text = kEwOpsText;
  });
}

}  // extern "C"
