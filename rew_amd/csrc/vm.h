// Fused elementwise programs ("VM") shared by the host planner and the HIP
// kernels.
//
// A program evaluates a DAG of elementwise ops at every point of a kernel's
// index space.  Leaves read materialized tensors through affine index maps
// (the composition of the reshape / transpose / broadcast_in_dim / slice /
// reverse ops rew emitted on the way), so view ops never touch HBM.  The
// opcode stream is wave-uniform: every lane runs the same instruction, the
// dispatch on opcode and register number is scalar control flow, and each
// lane carries kVec consecutive elements of the innermost dimension so the
// interpretation cost is spread over 64 x kVec elements.
#pragma once

#ifndef __HIPCC_RTC__
#include <stdint.h>
#endif

namespace rew {
namespace vm {

constexpr int kMaxLeaves = 12;
constexpr int kMaxIns = 120;
constexpr int kMaxRegs = 16;
constexpr int kMaxOuts = 4;
constexpr int kRank = 8;
constexpr int kVec = 4;

// Opcodes.  Register values are 32-bit: floats as IEEE binary32 (bf16/f16
// values are held as their exactly-representable f32 value, re-rounded after
// every op whose StableHLO result type is bf16/f16), integers and booleans
// as 32-bit two's complement.
enum Op : uint8_t {
  OP_NOP = 0,
  OP_LOAD,      // dst <- leaf[imm]
  OP_CONST,     // dst <- imm bits
  OP_IOTA,      // dst <- affine coordinate value of leaf[imm] (an index map)
  // float binary
  OP_ADDF, OP_SUBF, OP_MULF, OP_DIVF, OP_MAXF, OP_MINF, OP_POWF, OP_REMF,
  OP_ATAN2F,
  // signed / unsigned integer binary
  OP_ADDI, OP_SUBI, OP_MULI, OP_DIVI, OP_REMI, OP_MAXI, OP_MINI, OP_DIVU,
  OP_REMU, OP_MAXU, OP_MINU, OP_AND, OP_OR, OP_XOR, OP_SHL, OP_SHRA, OP_SHRL,
  // float unary
  OP_NEGF, OP_ABSF, OP_EXPF, OP_LOGF, OP_SQRTF, OP_RSQRTF, OP_TANHF,
  OP_LOGISTICF, OP_SINF, OP_COSF, OP_TANF, OP_EXPM1F, OP_LOG1PF, OP_CBRTF,
  OP_CEILF, OP_FLOORF, OP_SIGNF, OP_ROUNDAFZF, OP_ROUNDEVENF, OP_ISFINITEF,
  // integer unary
  OP_NEGI, OP_ABSI, OP_NOT, OP_NOTB, OP_CLZ, OP_POPCNT, OP_SIGNI,
  // comparisons (aux = direction) -> bool
  OP_CMPF, OP_CMPI, OP_CMPU,
  OP_SELECT,    // dst <- a ? b : c
  OP_CLAMPF,    // dst <- min(max(b, a), c)   (StableHLO clamp(min, x, max))
  OP_CLAMPI,
  OP_CLAMPU,
  // conversions / roundings
  OP_RBF16,     // round f32 value to bf16 precision (RNE)
  OP_RF16,      // round f32 value to f16 precision
  OP_F2I,       // f32 -> int32 (truncate toward zero, saturating)
  OP_F2U,       // f32 -> uint32
  OP_I2F,       // int32 -> f32
  OP_U2F,       // uint32 -> f32
  OP_TOBOOL,    // int != 0
  OP_FTOBOOL,   // float != 0
  OP_SEXT8, OP_ZEXT8, OP_SEXT16, OP_ZEXT16,  // integer narrowing
  OP_COUNT
};

enum Cmp : uint8_t { CMP_EQ = 0, CMP_NE, CMP_LT, CMP_LE, CMP_GT, CMP_GE };

struct Ins {
  uint8_t op, dst, a, b, c, aux;
  uint16_t pad;
  uint32_t imm;
};

// Leaf addressing modes.
enum LeafMode : uint8_t {
  LM_CONTIG = 0,  // innermost kernel dim has stride 1 and vector alignment
  LM_BCAST,       // innermost kernel dim has stride 0
  LM_STRIDED,     // any strides over the kernel's index space
  LM_VIRTUAL      // linear index of the kernel space re-split over vdim[]
};

// 32-bit magic-number division for n < 2^31.
struct FastDiv {
  uint32_t d, m, s;
};

struct Leaf {
  const void* ptr;      // nullptr for OP_IOTA leaves
  uint8_t dtype;        // rew dtype code
  uint8_t mode;         // LeafMode
  uint8_t vrank;        // LM_VIRTUAL only
  uint8_t pad;
  int32_t off;          // element offset
  int32_t clamp_hi;     // >= 0: clamp element offsets into [0, clamp_hi]
  int32_t stride[kRank];  // over kernel dims (or over vdim for LM_VIRTUAL)
  FastDiv vdim[kRank];    // LM_VIRTUAL only
};

struct Out {
  void* ptr;
  uint8_t dtype;
  uint8_t reg;
  uint8_t pad[2];
  int32_t off;          // element offset (kernel space linear index + off)
};

struct Program {
  uint16_t n_ins;
  uint8_t n_leaves;
  uint8_t n_outs;
  Ins ins[kMaxIns];
  Leaf leaf[kMaxLeaves];
  Out out[kMaxOuts];
};

// Kernel index space: rank dims, outermost first.
struct Space {
  int32_t rank;
  int64_t numel;
  FastDiv dim[kRank];
};

}  // namespace vm
}  // namespace rew
