// Exact GELU of bf16 values by table, shared by the MLP kernels:
// nn.GELU() (0.5 x (1 + erf(x / sqrt 2)), models/mlp.py:152-172) applied to a
// bf16 tensor, i.e. computed in fp32 and rounded to bf16.
#pragma once

#include "common.h"

namespace terra {
namespace {

// GELU of a bf16 input by table.  The fc1 output is rounded to bf16 before
// the activation, so GELU sees one of 2^16 inputs; for 2^-22 <= |x| < 32 the
// bf16 result is read from a table that each workgroup fills at start with
// the module's formula, 0.5 x (1 + erf(x / sqrt 2)) in fp32 rounded to bf16
// (the value PyTorch's GPU kernel computes for a bf16 input).  Outside that
// range the bf16 result has a closed form: 0.5 x for |x| < 2^-22 (the fp32
// value is 0.5 x (1 + d) with |d| < 2^-22, and 0.5 x is a bf16 value, so it
// rounds to 0.5 x); x for x >= 32 (erf = 1 in fp32); -0 for x <= -32 (erf =
// -1 in fp32); -inf gives NaN (-inf * 0) and NaN stays NaN.
constexpr uint32_t kGeluLo = 0x3480;   // bf16 bits of 2^-22
constexpr uint32_t kGeluHi = 0x4200;   // bf16 bits of 32
constexpr int kGeluSpan = (int)(kGeluHi - kGeluLo);  // 3456 entries per sign
constexpr int kGeluBytes = 2 * kGeluSpan * 2;

// Fills the GELU table (see kGeluLo): entry sign * kGeluSpan + (mag - kGeluLo).
__device__ __forceinline__ void gelu_table_fill(uint16_t* table, int tid, int nthreads) {
  for (int e = tid; e < 2 * kGeluSpan; e += nthreads) {
    const uint32_t sign = e >= kGeluSpan ? 0x8000u : 0u;
    const uint32_t bits = sign | (kGeluLo + (uint32_t)(e - (sign ? kGeluSpan : 0)));
    const float x = bf16_bits_to_f32((uint16_t)bits);
    table[e] = f32_to_bf16_bits(x * 0.5f * (1.f + erff(x * 0.70710678118654752f)));
  }
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Table lookups for the two bf16 values of `p` (two GELU results, packed the
// same way), with packed 16-bit index arithmetic.  `dmax` collects mag - kGeluLo
// per half (wrapping below kGeluLo): a value >= kGeluSpan marks an input
// outside the table, whose lookup here is clamped and wrong.
__device__ __forceinline__ uint32_t gelu_pair_table(uint32_t p, const uint16_t* table, u16x2& dmax) {
  const u16x2 v = __builtin_bit_cast(u16x2, p);
  const u16x2 d = (v & (u16x2)0x7fff) - (u16x2)(uint16_t)kGeluLo;
  dmax = __builtin_elementwise_max(dmax, d);
  const u16x2 idx = __builtin_elementwise_min(d, (u16x2)(uint16_t)(kGeluSpan - 1)) + (v >> 15) * (u16x2)(uint16_t)kGeluSpan;
  const u16x2 off = idx << 1;  // byte offsets (< 2^15)
  const uint8_t* t = reinterpret_cast<const uint8_t*>(table);
  return (uint32_t)*reinterpret_cast<const uint16_t*>(t + off.x) |
         ((uint32_t)*reinterpret_cast<const uint16_t*>(t + off.y) << 16);
}

// bf16 bits of GELU(x) for the bf16 bits of any x (the table or the closed forms).
__device__ __forceinline__ uint32_t gelu_bf16(uint32_t b, const uint16_t* table) {
  const uint32_t mag = b & 0x7fffu;
  const uint32_t sign = b >> 15;
  const uint32_t d = mag - kGeluLo;  // wraps below kGeluLo
  const uint32_t idx = (d < (uint32_t)kGeluSpan ? d : 0u) + (sign ? kGeluSpan : 0);
  const uint32_t tab = table[idx];
  const uint32_t half = __builtin_bit_cast(uint16_t, (__bf16)(0.5f * bf16_bits_to_f32((uint16_t)b)));
  const uint32_t big = b == 0xff80u ? 0x7fc0u : ((sign && mag <= 0x7f80u) ? 0x8000u : b);
  return mag < kGeluLo ? half : (mag < kGeluHi ? tab : big);
}

}  // namespace
}  // namespace terra
