// Shared helpers of the gfx950 kernels: error reporting for the C ABI,
// fast division by launch-time constants, bf16 conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <hip/hip_fp16.h>

#include "../../include/terra_swin.h"

namespace terra {

// Records the message returned by terra_last_error() for this thread and
// returns `status`, so validation code can `return fail(...)`.
int fail(int status, const char* fmt, ...);
void clear_error();

// Element size in bytes of a terra_dtype, or 0 if unknown.
inline int dtype_size(int dtype) {
  switch (dtype) {
    case TERRA_DTYPE_F32: return 4;
    case TERRA_DTYPE_F16: return 2;
    case TERRA_DTYPE_BF16: return 2;
    case TERRA_DTYPE_U8: return 1;
    default: return 0;
  }
}

// Unsigned division by a divisor fixed at launch time (Granlund–Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994):
//   n / d == (umulhi(n, m) + n) >> s   for all 32-bit n,
// with s = ceil(log2 d) and m = floor(2^32 * (2^s - d) / d) + 1.
struct FastDiv {
  uint32_t d, m, s;
  FastDiv() : d(1), m(0), s(0) {}
  explicit FastDiv(uint32_t div) : d(div) {
    s = 0;
    while ((1ull << s) < div) ++s;
    m = (uint32_t)(((1ull << 32) * ((1ull << s) - div)) / div + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint32_t hi = __umulhi(n, m);
    return (uint32_t)(((uint64_t)hi + n) >> s);
  }
  __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

// float -> bf16 bits, round to nearest even (what torch does on a cast).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// DPP move of a float between lanes of a row (kCtrl: the DPP control word).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// Sum over the 8 aligned lanes of one LayerNorm token group, in registers
// (DPP) rather than through the LDS crossbar: partners l^1 and l^2 (quad
// permutes [1,0,3,2] and [2,3,0,1]), then the other quad of the group (half-row
// mirror, lane i <-> 7 - i).  Each step adds the same two values on both
// partners, so all 8 lanes end with the same, order-independent result.  The
// whole group must be active.
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp_move<0xb1>(v);
  v += dpp_move<0x4e>(v);
  return v + dpp_move<0x141>(v);
}

// ---- streaming stores ------------------------------------------------------
// Output streams are written through buffer stores carrying the sc1 cache-
// policy bit.  Measured on MI355X (201 MB arrays, 16-byte accesses):
// nontemporal loads + sc1 stores copy at 7.2 TB/s, against 6.0-6.4 TB/s with
// nontemporal stores and 5.6-5.8 TB/s with plain ones; a 3-read/1-write
// stream goes from 6.5 to 7.2 TB/s.  The buffer descriptor also bounds every
// store to [base, base + bytes): out-of-range lanes are dropped by the
// hardware.
constexpr int kCacheNt = 2;    // nt: streaming (loads)
constexpr int kCacheSc1 = 16;  // sc1 (stores)
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit records, gfx950

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferWord3);
}

typedef uint32_t stream_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t stream_u32x2 __attribute__((ext_vector_type(2)));

// A 16-byte store with the nt policy.  For 128-byte row slices spread over
// a strided tensor (the attention backward's gradients: three tensors, one
// slice per token row and head pair) it measured 272 us against 278 us with
// sc1 and 288 us with sc0 or no policy bits (c3); contiguous streams favour
// sc1 (above).
template <typename T>
__device__ __forceinline__ void stream_store_nt(const T& v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  static_assert(sizeof(T) == 16, "16-byte stores");
  stream_u32x4 w;
  __builtin_memcpy(&w, &v, 16);
  __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, kCacheNt);
}

// Stores `v` at byte offset `off` of the descriptor's range.
template <typename T>
__device__ __forceinline__ void stream_store_sc1(T v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 16) {
    stream_u32x4 w;
    __builtin_memcpy(&w, &v, 16);
    __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, kCacheSc1);
  } else if constexpr (sizeof(T) == 8) {
    stream_u32x2 w;
    __builtin_memcpy(&w, &v, 8);
    __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, kCacheSc1);
  } else if constexpr (sizeof(T) == 4) {
    uint32_t w;
    __builtin_memcpy(&w, &v, 4);
    __builtin_amdgcn_raw_buffer_store_b32(w, r, off, 0, kCacheSc1);
  } else if constexpr (sizeof(T) == 2) {
    uint16_t w;
    __builtin_memcpy(&w, &v, 2);
    __builtin_amdgcn_raw_buffer_store_b16(w, r, off, 0, kCacheSc1);
  } else {
    static_assert(sizeof(T) == 1, "1, 2, 4, 8 or 16-byte stores");
    uint8_t w;
    __builtin_memcpy(&w, &v, 1);
    __builtin_amdgcn_raw_buffer_store_b8(w, r, off, 0, kCacheSc1);
  }
}

// Derived sizes of a validated terra_swin_geom.
struct GeomDims {
  int64_t Hp, Wp;      // padded frame
  int64_t nWh, nWw;    // frame windows per column / row
  int64_t rows;        // emitted window rows (win_rows resolved)
  int64_t nWe;         // emitted windows per image
};

// Checks the shape fields of `geom` (positive sizes, whole windows, shift
// and window-row / valid-window ranges inside the frame) and fills `dims`.
int validate_geom(const terra_swin_geom* geom, GeomDims* dims);

}  // namespace terra
