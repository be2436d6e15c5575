// The per-element evaluator of a bt_program: a straight line of instructions over 16 registers of 32-bit values, in
// one dtype. The program sits in the kernel arguments, so instruction fields are uniform across a wavefront, and the
// register index switches below become scalar branches rather than indexed (scratch) register access.
#pragma once
#include "common.h"
#include <math.h>

namespace bt {

__device__ __forceinline__ uint32_t reg_get(const uint32_t (&r)[BT_MAX_REGS], int i) {
  switch (i) {
    case 0: return r[0]; case 1: return r[1]; case 2: return r[2]; case 3: return r[3];
    case 4: return r[4]; case 5: return r[5]; case 6: return r[6]; case 7: return r[7];
    case 8: return r[8]; case 9: return r[9]; case 10: return r[10]; case 11: return r[11];
    case 12: return r[12]; case 13: return r[13]; case 14: return r[14]; default: return r[15];
  }
}

__device__ __forceinline__ void reg_set(uint32_t (&r)[BT_MAX_REGS], int i, uint32_t v) {
  switch (i) {
    case 0: r[0] = v; break; case 1: r[1] = v; break; case 2: r[2] = v; break; case 3: r[3] = v; break;
    case 4: r[4] = v; break; case 5: r[5] = v; break; case 6: r[6] = v; break; case 7: r[7] = v; break;
    case 8: r[8] = v; break; case 9: r[9] = v; break; case 10: r[10] = v; break; case 11: r[11] = v; break;
    case 12: r[12] = v; break; case 13: r[13] = v; break; case 14: r[14] = v; break; default: r[15] = v; break;
  }
}

// The stored matrix that batch entry b of the result reads.
__device__ __forceinline__ int64_t operand_matrix(const bt_operand &o, int64_t b) {
  if (o.rep == 1 && o.cyc == 0) return b;  // the common case, without a division
  int64_t m = b / o.rep;
  return o.cyc ? m % o.cyc : m;
}

__device__ __forceinline__ const void *operand_at(const bt_operand &o, int64_t b, int64_t r, int64_t c) {
  int64_t at = operand_matrix(o, b) * o.sb + r * o.sr + c * o.sc;
  int size = o.dtype == BT_BF16 ? 2 : 4;
  return (const void *)(o.ptr + (uint64_t)(at * size));
}

// An input value in the program's dtype, as raw bits.
template <int DT>
__device__ __forceinline__ uint32_t load_operand(const bt_operand &o, int64_t b, int64_t r, int64_t c) {
  const void *p = operand_at(o, b, r, c);
  if (o.dtype == BT_BF16) {
    uint32_t bits = *(const uint16_t *)p;
    if (DT == BT_INT32) return (uint32_t)(int32_t)rintf(bf16_value(bits));
    return bits << 16;
  }
  uint32_t v = *(const uint32_t *)p;
  if (o.dtype == BT_INT32 && DT != BT_INT32) {
    float f = (float)(int32_t)v;
    return __float_as_uint(DT == BT_BF16 ? round_packed(f) : f);
  }
  if (o.dtype == BT_FP32 && DT == BT_INT32) return (uint32_t)(int32_t)rintf(__uint_as_float(v));
  if (o.dtype == BT_FP32 && DT == BT_BF16) return __float_as_uint(round_packed(__uint_as_float(v)));
  return v;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}

// One instruction's float result, before the dtype's rounding.
__device__ __forceinline__ float float_op(int op, float a, float b, float c) {
  switch (op) {
    case BT_OP_ADD: return a + b;
    case BT_OP_SUB: return a - b;
    case BT_OP_MUL: return a * b;
    case BT_OP_DIV: return a / b;
    case BT_OP_MAX: return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
    case BT_OP_MIN: return (a != a || b != b) ? __builtin_nanf("") : fminf(a, b);
    case BT_OP_CMPLT: return a < b ? 1.0f : 0.0f;
    case BT_OP_CMPLE: return a <= b ? 1.0f : 0.0f;
    case BT_OP_CMPNE: return a != b ? 1.0f : 0.0f;
    case BT_OP_CMPEQ: return a == b ? 1.0f : 0.0f;
    case BT_OP_NEG: return -a;
    case BT_OP_RELU: return a > 0.0f ? a : 0.0f;
    case BT_OP_EXP: return expf(a);
    case BT_OP_EXP2: return exp2f(a);
    case BT_OP_LOG: return logf(a);
    case BT_OP_LOG2: return log2f(a);
    case BT_OP_SQRT: return sqrtf(a);
    case BT_OP_RECIP: return 1.0f / a;
    case BT_OP_RSQRT: return 1.0f / sqrtf(a);
    case BT_OP_SIN: return sinf(a);
    case BT_OP_COS: return cosf(a);
    case BT_OP_SIGMOID: return 1.0f / (1.0f + expf(-a));
    case BT_OP_SILU: return a / (1.0f + expf(-a));
    case BT_OP_GELU: return gelu_tanh(a);
    case BT_OP_TANH: return tanhf(a);
    case BT_OP_FTOB: return round_packed(a);
    default: return a;
  }
}

__device__ __forceinline__ int32_t int_op(int op, int32_t a, int32_t b) {
  switch (op) {
    case BT_OP_ADD: return (int32_t)((uint32_t)a + (uint32_t)b);
    case BT_OP_SUB: return (int32_t)((uint32_t)a - (uint32_t)b);
    case BT_OP_MUL: return (int32_t)((uint32_t)a * (uint32_t)b);
    case BT_OP_MAX: return a > b ? a : b;
    case BT_OP_MIN: return a < b ? a : b;
    case BT_OP_CMPLT: return a < b;
    case BT_OP_CMPLE: return a <= b;
    case BT_OP_CMPNE: return a != b;
    case BT_OP_CMPEQ: return a == b;
    case BT_OP_NEG: return (int32_t)(0u - (uint32_t)a);
    case BT_OP_RELU: return a > 0 ? a : 0;
    default: return a;
  }
}

// ---- evaluation of V elements at once ------------------------------------------------------------------------------
// A program runs in two phases: every input is fetched for all V elements first, so the loads are in flight together
// and their latencies overlap, then the instructions run over the V values each, so decoding an instruction and
// selecting its registers (uniform scalar branches) is paid once per V elements.

template <int V> struct Vals { uint32_t x[V]; };

// The register file of one element: a vector, so that reading or writing register i (a uniform index from the
// instruction) is a register-relative move (v_movrels / v_movreld) rather than an access to scratch memory.
typedef uint32_t regfile __attribute__((ext_vector_type(BT_MAX_REGS)));
typedef uint32_t prefile __attribute__((ext_vector_type(BT_MAX_INPUTS)));

template <int V>
__device__ __forceinline__ Vals<V> regs_get(const regfile (&r)[V], int i) {
  Vals<V> o;
#pragma unroll
  for (int v = 0; v < V; v++) o.x[v] = r[v][i];
  return o;
}

template <int V>
__device__ __forceinline__ void regs_set(regfile (&r)[V], int i, const Vals<V> &x) {
#pragma unroll
  for (int v = 0; v < V; v++) r[v][i] = x.x[v];
}

template <int V>
__device__ __forceinline__ Vals<V> pre_get(const prefile (&p)[V], int i) {
  Vals<V> o;
#pragma unroll
  for (int v = 0; v < V; v++) o.x[v] = p[v][i];
  return o;
}

// Where each of V elements sits in the result: batch entry, row, column, and whether it exists.
template <int V> struct Coords {
  int64_t b[V], r[V], c[V];
  bool ok[V];
};

// Every input of prog at the V elements; 0 where an element does not exist.
template <int DT, int V>
__device__ __forceinline__ void fetch_inputs(const bt_program &prog, const Coords<V> &at, prefile (&pre)[V]) {
#pragma unroll
  for (int k = 0; k < BT_MAX_INPUTS; k++) {
#pragma unroll
    for (int v = 0; v < V; v++)
      pre[v][k] = k < prog.n_inputs && at.ok[v] ? load_operand<DT>(prog.in[k], at.b[v], at.r[v], at.c[v]) : 0u;
  }
}

// The transcendental and other long operations, kept out of line: each expands to dozens of instructions, and inlined
// into every op's branch they would make the evaluator larger than the instruction cache.
__device__ __forceinline__ float long_op_inline(int op, float a) {
  switch (op) {
    case BT_OP_EXP: return expf(a);
    case BT_OP_EXP2: return exp2f(a);
    case BT_OP_LOG: return logf(a);
    case BT_OP_LOG2: return log2f(a);
    case BT_OP_SQRT: return sqrtf(a);
    case BT_OP_RECIP: return 1.0f / a;
    case BT_OP_RSQRT: return 1.0f / sqrtf(a);
    case BT_OP_SIN: return sinf(a);
    case BT_OP_COS: return cosf(a);
    case BT_OP_SIGMOID: return 1.0f / (1.0f + expf(-a));
    case BT_OP_SILU: return a / (1.0f + expf(-a));
    case BT_OP_GELU: return gelu_tanh(a);
    case BT_OP_TANH: return tanhf(a);
    default: return a;
  }
}
__device__ __attribute__((noinline)) float long_op(int op, float a) { return long_op_inline(op, a); }

// One instruction over V values. op is uniform, so the switch is a scalar branch around straight vector code. INL
// inlines the long operations too: for callers that hold many live registers (a GEMM's accumulators), which a call
// would have to save to memory.
template <int DT, int V, bool INL = false>
__device__ __forceinline__ Vals<V> apply_op(int op, const Vals<V> &a, const Vals<V> &b) {
  Vals<V> o;
  if (DT == BT_INT32) {
#pragma unroll
    for (int v = 0; v < V; v++) o.x[v] = (uint32_t)int_op(op, (int32_t)a.x[v], (int32_t)b.x[v]);
    return o;
  }
  float f[V], x[V], y[V];
#pragma unroll
  for (int v = 0; v < V; v++) { x[v] = __uint_as_float(a.x[v]); y[v] = __uint_as_float(b.x[v]); }
#define BT_OP(code, expr)                              \
  case code:                                           \
    _Pragma("unroll") for (int v = 0; v < V; v++) {    \
      const float A = x[v], B = y[v];                  \
      (void)B;                                         \
      f[v] = (expr);                                   \
    }                                                  \
    break;
  switch (op) {
    BT_OP(BT_OP_ADD, A + B)
    BT_OP(BT_OP_SUB, A - B)
    BT_OP(BT_OP_MUL, A * B)
    BT_OP(BT_OP_DIV, A / B)
    BT_OP(BT_OP_MAX, (A != A || B != B) ? __builtin_nanf("") : fmaxf(A, B))
    BT_OP(BT_OP_MIN, (A != A || B != B) ? __builtin_nanf("") : fminf(A, B))
    BT_OP(BT_OP_CMPLT, A < B ? 1.0f : 0.0f)
    BT_OP(BT_OP_CMPLE, A <= B ? 1.0f : 0.0f)
    BT_OP(BT_OP_CMPNE, A != B ? 1.0f : 0.0f)
    BT_OP(BT_OP_CMPEQ, A == B ? 1.0f : 0.0f)
    BT_OP(BT_OP_NEG, -A)
    BT_OP(BT_OP_RELU, A > 0.0f ? A : 0.0f)
    BT_OP(BT_OP_FTOB, round_packed(A))
    default:
#pragma unroll
      for (int v = 0; v < V; v++) f[v] = INL ? long_op_inline(op, x[v]) : long_op(op, x[v]);
  }
#undef BT_OP
#pragma unroll
  for (int v = 0; v < V; v++) o.x[v] = __float_as_uint(DT == BT_BF16 ? round_packed(f[v]) : f[v]);
  return o;
}

// Runs prog on V elements whose inputs are in pre. io holds the incoming value (register 0: a matmul epilogue's
// result) and receives the result register's bits.
template <int DT, int V, bool INL = false>
__device__ __forceinline__ void eval_program(const bt_program &prog, const prefile (&pre)[V], uint32_t (&io)[V]) {
  regfile regs[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    regs[v] = (regfile)(0u);
    regs[v][0] = io[v];
  }
  for (int i = 0; i < prog.n_inst; i++) {
    const bt_inst in = prog.inst[i];
    Vals<V> o;
    if (in.op == BT_OP_LOAD) o = pre_get<V>(pre, in.a);
    else if (in.op == BT_OP_CONST) {
#pragma unroll
      for (int v = 0; v < V; v++) o.x[v] = in.imm;
    } else if (in.op == BT_OP_MOV) o = regs_get<V>(regs, in.a);
    else if (in.op == BT_OP_WHERE) {
      const Vals<V> cnd = regs_get<V>(regs, in.a), t = regs_get<V>(regs, in.b), e = regs_get<V>(regs, in.c);
#pragma unroll
      for (int v = 0; v < V; v++) {
        const bool on = DT == BT_INT32 ? cnd.x[v] != 0 : __uint_as_float(cnd.x[v]) != 0.0f;
        o.x[v] = on ? t.x[v] : e.x[v];
      }
    } else {
      o = apply_op<DT, V, INL>(in.op, regs_get<V>(regs, in.a), regs_get<V>(regs, in.b));
    }
    regs_set<V>(regs, in.dst, o);
  }
  const Vals<V> res = regs_get<V>(regs, prog.result);
#pragma unroll
  for (int v = 0; v < V; v++) io[v] = res.x[v];
}

// Runs prog at V elements: fetch, then evaluate. io as for eval_program.
template <int DT, int V, bool INL = false>
__device__ __forceinline__ void run_program_v(const bt_program &prog, const Coords<V> &at, uint32_t (&io)[V]) {
  prefile pre[V];
  fetch_inputs<DT, V>(prog, at, pre);
  eval_program<DT, V, INL>(prog, pre, io);
}

// Runs prog at element (b, r, c). acc, if the program reads register 0 as a preloaded value (a matmul epilogue), is
// placed there first. Returns the result register's bits.
template <int DT, bool INL = false>
__device__ __forceinline__ uint32_t run_program(const bt_program &prog, int64_t b, int64_t r, int64_t c,
                                                uint32_t acc) {
  Coords<1> at;
  at.b[0] = b, at.r[0] = r, at.c[0] = c, at.ok[0] = true;
  uint32_t io[1] = {acc};
  run_program_v<DT, 1, INL>(prog, at, io);
  return io[0];
}

// ---- evaluation over row segments ----------------------------------------------------------------------------------
// For results large enough to fill the chip many times: a thread evaluates SEG neighbouring columns c0 .. c0 + SEG - 1
// of one row. Each input's address is worked out once per segment; an input whose columns are contiguous is read with
// 16-byte loads, a broadcast one (column stride 0) with one load, any other value by value. The inputs are fetched by
// a loop that is not unrolled, which keeps the code small; the latency of one input's loads is hidden by the many
// other waves in flight.
constexpr int SEG = 8;

// A raw element of an input (bf16 bits in the low half, or 32 bits) as the program's dtype: the conversions of
// load_operand.
template <int DT>
__device__ __forceinline__ uint32_t convert_raw(uint32_t raw, int dtype) {
  if (dtype == BT_BF16) {
    if (DT == BT_INT32) return (uint32_t)(int32_t)rintf(bf16_value(raw & 0xFFFFu));
    return raw << 16;
  }
  if (dtype == BT_INT32 && DT != BT_INT32) {
    const float f = (float)(int32_t)raw;
    return __float_as_uint(DT == BT_BF16 ? round_packed(f) : f);
  }
  if (dtype == BT_FP32 && DT == BT_INT32) return (uint32_t)(int32_t)rintf(__uint_as_float(raw));
  if (dtype == BT_FP32 && DT == BT_BF16) return __float_as_uint(round_packed(__uint_as_float(raw)));
  return raw;
}

// The inputs of prog for the segment (b, r, c0 .. c0 + n - 1), n <= SEG; 0 past n.
template <int DT>
__device__ __forceinline__ void fetch_segment(const bt_program &prog, int64_t b, int64_t r, int64_t c0, int n,
                                              prefile (&pre)[SEG]) {
#pragma unroll
  for (int v = 0; v < SEG; v++) pre[v] = (prefile)(0u);
#pragma unroll 1
  for (int k = 0; k < prog.n_inputs; k++) {
    const bt_operand &o = prog.in[k];
    const int64_t at = operand_matrix(o, b) * o.sb + r * o.sr + c0 * o.sc;
    uint32_t raw[SEG];
    if (o.dtype == BT_BF16) {
      const uint16_t *p = (const uint16_t *)o.ptr + at;
      if (o.sc == 1 && n == SEG && ((uintptr_t)p & 15) == 0) {
        const uint4 w = *(const uint4 *)p;
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int v = 0; v < SEG; v++) raw[v] = ws[v / 2] >> (16 * (v & 1)) & 0xFFFFu;
      } else if (o.sc == 0) {
        const uint32_t x = *p;
#pragma unroll
        for (int v = 0; v < SEG; v++) raw[v] = x;
      } else {
#pragma unroll
        for (int v = 0; v < SEG; v++) raw[v] = v < n ? p[v * o.sc] : 0u;
      }
    } else {
      const uint32_t *p = (const uint32_t *)o.ptr + at;
      if (o.sc == 1 && n == SEG && ((uintptr_t)p & 15) == 0) {
        const uint4 w0 = *(const uint4 *)p, w1 = *(const uint4 *)(p + 4);
        raw[0] = w0.x, raw[1] = w0.y, raw[2] = w0.z, raw[3] = w0.w;
        raw[4] = w1.x, raw[5] = w1.y, raw[6] = w1.z, raw[7] = w1.w;
      } else if (o.sc == 0) {
        const uint32_t x = *p;
#pragma unroll
        for (int v = 0; v < SEG; v++) raw[v] = x;
      } else {
#pragma unroll
        for (int v = 0; v < SEG; v++) raw[v] = v < n ? p[v * o.sc] : 0u;
      }
    }
#pragma unroll
    for (int v = 0; v < SEG; v++) pre[v][k] = convert_raw<DT>(raw[v], o.dtype);
  }
}

// The stored bits of a value computed in DT, for an output of dtype `dtype` (the conversions of store_value).
template <int DT>
__device__ __forceinline__ uint32_t stored_bits(uint32_t v, int dtype) {
  if (dtype == BT_BF16) return bf16_packed(DT == BT_INT32 ? (float)(int32_t)v : __uint_as_float(v));
  if (dtype == BT_FP32) return __float_as_uint(DT == BT_INT32 ? (float)(int32_t)v : __uint_as_float(v));
  if (DT == BT_INT32) return v;
  const float f = rintf(__uint_as_float(v));
  return (uint32_t)(f != f ? 0 : f >= 2147483648.0f ? 2147483647 : f < -2147483648.0f ? (-2147483647 - 1) : (int32_t)f);
}

// Stores the segment's n values, with 16-byte stores when the output's columns are contiguous and aligned.
template <int DT>
__device__ __forceinline__ void store_segment(const bt_operand &out, int64_t b, int64_t r, int64_t c0, int n,
                                              const uint32_t (&io)[SEG]) {
  const int64_t at = operand_matrix(out, b) * out.sb + r * out.sr + c0 * out.sc;
  uint32_t w[SEG];
#pragma unroll
  for (int v = 0; v < SEG; v++) w[v] = stored_bits<DT>(io[v], out.dtype);
  if (out.dtype == BT_BF16) {
    uint16_t *p = (uint16_t *)out.ptr + at;
    if (out.sc == 1 && n == SEG && ((uintptr_t)p & 15) == 0) {
      *(uint4 *)p = make_uint4(w[0] | w[1] << 16, w[2] | w[3] << 16, w[4] | w[5] << 16, w[6] | w[7] << 16);
      return;
    }
#pragma unroll
    for (int v = 0; v < SEG; v++)
      if (v < n) p[v * out.sc] = (uint16_t)w[v];
  } else {
    uint32_t *p = (uint32_t *)out.ptr + at;
    if (out.sc == 1 && n == SEG && ((uintptr_t)p & 15) == 0) {
      *(uint4 *)p = make_uint4(w[0], w[1], w[2], w[3]);
      *(uint4 *)(p + 4) = make_uint4(w[4], w[5], w[6], w[7]);
      return;
    }
#pragma unroll
    for (int v = 0; v < SEG; v++)
      if (v < n) p[v * out.sc] = w[v];
  }
}

// n / d for 32-bit n, with a multiplier and shift the host computed for d (the round-up method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994): q = (umulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s;
};
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.s);
}
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) s++;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}

// Stores a result computed in DT as out's dtype at element offset `at`.
template <int DT>
__device__ __forceinline__ void store_value(const bt_operand &out, int64_t at, uint32_t v) {
  if (out.dtype == BT_BF16) {
    float f = DT == BT_INT32 ? (float)(int32_t)v : __uint_as_float(v);
    ((uint16_t *)out.ptr)[at] = (uint16_t)bf16_packed(f);
  } else if (out.dtype == BT_FP32) {
    ((float *)out.ptr)[at] = DT == BT_INT32 ? (float)(int32_t)v : __uint_as_float(v);
  } else {
    int32_t i;
    if (DT == BT_INT32) i = (int32_t)v;
    else {
      float f = rintf(__uint_as_float(v));
      i = f != f ? 0 : f >= 2147483648.0f ? 2147483647 : f < -2147483648.0f ? (-2147483647 - 1) : (int32_t)f;
    }
    ((int32_t *)out.ptr)[at] = i;
  }
}

}  // namespace bt
