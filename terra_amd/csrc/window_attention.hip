// Fused per-window multi-head attention forward for gfx950.
//
// One wavefront computes one (window, head) item.  With the window padded to
// 64 tokens and head dim D:
//
//   S^T = K Q^T      v_mfma_f32_16x16x32_bf16 (bf16) / 16x16x4_f32 (fp32),
//                    4x4 tiles of 16x16; both operands are read straight from
//                    global memory as contiguous 16-byte rows of q and k.
//   S   = S*scale + bias + mask (fp32, in registers; the relative-position
//         bias table of the head and the window's mask terms are applied per
//         element), padded keys excluded, row softmax in fp32 with the row
//         spread over 4 lanes x 16 registers.
//   O^T = V^T P^T    P (from the S^T accumulator layout) is already in MFMA
//                    operand order; V is staged once in LDS and read
//                    transposed.  The O^T accumulator layout gives each lane 4
//                    consecutive channels of one token row, stored as one
//                    8-byte (bf16) / 16-byte (fp32) write into [B_, N, C].
//
// Accumulator layout of a 16x16 MFMA tile (lane l, g = l/16, c = l%16):
// element (row 4g + r, col c), r = 0..3.  In S^T the row is the key j and
// the column the query i, so lane l holds queries i = 16*it + c and keys
// j = 16*jt + 4g + r.
#include "common.h"

#include <math.h>

namespace terra {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kNPad = 64;      // window tokens padded to 4 tiles of 16
constexpr int kTableMax = 225; // (2*8-1)^2: windows up to 8x8
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_stride, k_stride, v_stride, o_stride;
  const float* bias_table;
  const float* explicit_mask;
  const uint64_t* land_bits;
  int32_t items;      // num_windows * heads
  int32_t heads;
  int32_t N;          // token rows per window
  int32_t n_geo;      // window_h * window_w (bias / mask extent)
  int32_t window_h, window_w;
  int32_t table_size; // (2Wh-1)(2Ww-1)
  int32_t n_real;
  float scale, mask_value, pad_key_value;
  int32_t mask_mode, mask_windows;
  int32_t frame_h, frame_w, shift_h, shift_w;
  int32_t win_row_begin, win_rows, win_cols;
};

__device__ __forceinline__ int region(int coord, int extent, int ws, int shift) {
  // Swin shift-mask slices (0:-ws), (-ws:-shift), (-shift:) of one axis.
  return coord < extent - ws ? 0 : (coord < extent - shift ? 1 : 2);
}

template <bool kBf16> struct EltTraits;
template <> struct EltTraits<true> { using T = uint16_t; };
template <> struct EltTraits<false> { using T = float; };

template <bool kBf16, int D>
struct alignas(16) LdsLayout {
  using T = typename EltTraits<kBf16>::T;
  // Row pitch of the per-wave V tile: 16 extra bytes make the 4 row groups
  // read by one instruction fall into disjoint LDS bank ranges.
  static constexpr int kPitch = D + 16 / (int)sizeof(T);
  T v[kWaves][kNPad * kPitch];
  float table[kWaves][kTableMax];
};

template <bool kBf16, int D>
__global__ __launch_bounds__(kThreads) void window_attn_kernel(const AttnParams p) {
  using T = typename EltTraits<kBf16>::T;
  using L = LdsLayout<kBf16, D>;
  __shared__ L lds;
  constexpr int kPitch = L::kPitch;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;

  const int item_raw = blockIdx.x * kWaves + wave;
  const bool live = item_raw < p.items;
  const int item = live ? item_raw : p.items - 1;
  const int w = item / p.heads;
  const int h = item - w * p.heads;

  const T* qw = reinterpret_cast<const T*>(p.q) + (int64_t)w * p.N * p.q_stride + (int64_t)h * D;
  const T* kw = reinterpret_cast<const T*>(p.k) + (int64_t)w * p.N * p.k_stride + (int64_t)h * D;
  const T* vw = reinterpret_cast<const T*>(p.v) + (int64_t)w * p.N * p.v_stride + (int64_t)h * D;

  // ---- global loads: K and Q fragments straight into registers, V rows ----
  // bf16: lane (c, g) holds row 16*t + c, channels [8g, 8g+8) of each 32-wide
  // k-step.  fp32: lane holds channels [g*D/4, (g+1)*D/4) (k order permuted
  // identically in both operands, which leaves the dot products unchanged).
  constexpr int kKSteps = kBf16 ? D / 32 : 1;
  constexpr int kFragU4 = kBf16 ? 1 : D / 16;  // 16-byte loads per fragment row part
  uint4 kf[4][kKSteps * kFragU4];
  uint4 qf[4][kKSteps * kFragU4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 16 * t + c16;
    const bool ok = row < p.N;
#pragma unroll
    for (int s = 0; s < kKSteps * kFragU4; ++s) {
      int col;
      if constexpr (kBf16) col = 32 * s + 8 * g;
      else col = g * (D / 4) + 4 * s;
      kf[t][s] = ok ? *reinterpret_cast<const uint4*>(kw + (int64_t)row * p.k_stride + col) : make_uint4(0, 0, 0, 0);
      qf[t][s] = ok ? *reinterpret_cast<const uint4*>(qw + (int64_t)row * p.q_stride + col) : make_uint4(0, 0, 0, 0);
    }
  }
  // V: the 64 x D tile as 16-byte chunks, kChunksPerRow per row.
  constexpr int kChunksPerRow = D * (int)sizeof(T) / 16;
  constexpr int kVLoads = kNPad * kChunksPerRow / 64;
  uint4 vr[kVLoads];
#pragma unroll
  for (int u = 0; u < kVLoads; ++u) {
    const int chunk = lane + 64 * u;
    const int row = chunk / kChunksPerRow;
    const int col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
    vr[u] = row < p.N ? *reinterpret_cast<const uint4*>(vw + (int64_t)row * p.v_stride + col) : make_uint4(0, 0, 0, 0);
  }

  // ---- per-token geometry, one token per lane, shared through shuffles ----
  const int t_geo = lane < p.n_geo ? lane : p.n_geo - 1;
  const int ti = t_geo / p.window_w;
  const int tj = t_geo - ti * p.window_w;
  const int rel_w = 2 * p.window_w - 1;
  const int my_base = (ti + p.window_h - 1) * rel_w + tj + p.window_w - 1;  // idx = base(i) - off(j)
  const int my_off = ti * rel_w + tj;

  // Window position in the frame (shift mask) and mask flags.
  bool use_shift = false;
  int my_rid = 0;
  if (p.mask_mode == TERRA_MASK_SHIFT) {
    const int per_img = p.win_rows * p.win_cols;
    const int wl = w % per_img;
    const int wr = wl / p.win_cols + p.win_row_begin;
    const int wc = wl - (wl / p.win_cols) * p.win_cols;
    use_shift = (wr + 1) * p.window_h > p.frame_h - p.window_h || (wc + 1) * p.window_w > p.frame_w - p.window_w;
    my_rid = 3 * region(wr * p.window_h + ti, p.frame_h, p.window_h, p.shift_h) +
             region(wc * p.window_w + tj, p.frame_w, p.window_w, p.shift_w);
  }
  const uint64_t land = p.land_bits != nullptr ? p.land_bits[w % p.mask_windows] : 0ull;
  const float* emask = p.mask_mode == TERRA_MASK_EXPLICIT
                           ? p.explicit_mask + (int64_t)(w % p.mask_windows) * p.n_geo * p.n_geo
                           : nullptr;

  // Stage this head's bias-table column in LDS (wave-local).
  float* tab = lds.table[wave];
  if (p.bias_table != nullptr) {
    for (int e = lane; e < p.table_size; e += 64) tab[e] = p.bias_table[(int64_t)e * p.heads + h];
  }

  // ---- S^T = K Q^T ----
  f32x4 acc[4][4];  // [it][jt]
#pragma unroll
  for (int it = 0; it < 4; ++it)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) acc[it][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int it = 0; it < 4; ++it) {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      if constexpr (kBf16) {
#pragma unroll
        for (int s = 0; s < kKSteps; ++s) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, kf[jt][s]);
          const bf16x8 b = __builtin_bit_cast(bf16x8, qf[it][s]);
          acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[it][jt], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int s = 0; s < kFragU4; ++s) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = __uint_as_float(reinterpret_cast<const uint32_t*>(&kf[jt][s])[e]);
            const float b = __uint_as_float(reinterpret_cast<const uint32_t*>(&qf[it][s])[e]);
            acc[it][jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[it][jt], 0, 0, 0);
          }
        }
      }
    }
  }

  // V rows -> LDS (row-major, padded pitch).
  T* vt = lds.v[wave];
#pragma unroll
  for (int u = 0; u < kVLoads; ++u) {
    const int chunk = lane + 64 * u;
    const int row = chunk / kChunksPerRow;
    const int col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
    *reinterpret_cast<uint4*>(vt + row * kPitch + col) = vr[u];
  }
  __syncthreads();

  // ---- scale, bias, mask, softmax (fp32) ----
  const bool has_bias = p.bias_table != nullptr;
  const bool has_mask = use_shift || land != 0ull || emask != nullptr;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int i = 16 * it + c16;
    const int i_geo = i < p.n_geo ? i : p.n_geo - 1;
    const int base_i = __shfl(my_base, i_geo);
    const int rid_i = __shfl(my_rid, i_geo);
    float mx = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jt + 4 * g + r;
        const int j_geo = j < p.n_geo ? j : p.n_geo - 1;
        const bool in_geo = i < p.n_geo && j < p.n_geo;
        float x = acc[it][jt][r] * p.scale;
        if (has_bias) {
          const int off_j = __shfl(my_off, j_geo);
          const float b = tab[base_i - off_j];
          x += in_geo ? b : 0.f;
        }
        if (has_mask) {
          float m = 0.f;
          if (emask != nullptr) m = in_geo ? emask[i_geo * p.n_geo + j_geo] : 0.f;
          if (use_shift) {
            const int rid_j = __shfl(my_rid, j_geo);
            m += (in_geo && rid_i != rid_j) ? p.mask_value : 0.f;
          }
          if (j < p.n_geo && ((land >> j) & 1ull)) m += p.mask_value;
          x += m;
        }
        if (j >= p.n_real) x = p.pad_key_value;
        if (j >= p.N) x = -INFINITY;
        acc[it][jt][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mb = mx * kLog2e;
    float sum = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[it][jt][r], kLog2e, -mb));
        acc[it][jt][r] = e;
        sum += e;
      }
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[it][jt][r] *= inv;
  }

  // ---- O^T = V^T P^T ----
  constexpr int kCT = D / 16;
  f32x4 oacc[kCT][4];  // [ct][it]
#pragma unroll
  for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
    for (int it = 0; it < 4; ++it) oacc[ct][it] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (kBf16) {
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      // P^T fragment: k-slot e -> key 32*js + 16*(e/4) + 4g + e%4.
      bf16x8 pf[4];
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        uint16_t bits[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) bits[e] = f32_to_bf16_bits(acc[it][2 * js + (e >> 2)][e & 3]);
        pf[it] = __builtin_bit_cast(bf16x8, bits);
      }
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct) {
        uint16_t bits[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * js + 16 * (e >> 2) + 4 * g + (e & 3);
          bits[e] = vt[j * kPitch + 16 * ct + c16];
        }
        const bf16x8 a = __builtin_bit_cast(bf16x8, bits);
#pragma unroll
        for (int it = 0; it < 4; ++it)
          oacc[ct][it] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pf[it], oacc[ct][it], 0, 0, 0);
      }
    }
  } else {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jt + 4 * g + r;
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
          const float a = vt[j * kPitch + 16 * ct + c16];
#pragma unroll
          for (int it = 0; it < 4; ++it)
            oacc[ct][it] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, acc[it][jt][r], oacc[ct][it], 0, 0, 0);
        }
      }
    }
  }

  // ---- store O: lane holds O[i = 16*it + c16][16*ct + 4g .. +4] ----
  if (live) {
    T* ow = reinterpret_cast<T*>(p.o) + (int64_t)w * p.N * p.o_stride + (int64_t)h * D;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int i = 16 * it + c16;
      if (i < p.N) {
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
          T* dst = ow + (int64_t)i * p.o_stride + 16 * ct + 4 * g;
          if constexpr (kBf16) {
            uint2 pk;
            pk.x = (uint32_t)f32_to_bf16_bits(oacc[ct][it][0]) | ((uint32_t)f32_to_bf16_bits(oacc[ct][it][1]) << 16);
            pk.y = (uint32_t)f32_to_bf16_bits(oacc[ct][it][2]) | ((uint32_t)f32_to_bf16_bits(oacc[ct][it][3]) << 16);
            *reinterpret_cast<uint2*>(dst) = pk;
          } else {
            *reinterpret_cast<float4*>(dst) =
                make_float4(oacc[ct][it][0], oacc[ct][it][1], oacc[ct][it][2], oacc[ct][it][3]);
          }
        }
      }
    }
  }
}

template <bool kBf16, int D>
void launch(const AttnParams& p, hipStream_t s) {
  const int blocks = (p.items + kWaves - 1) / kWaves;
  window_attn_kernel<kBf16, D><<<blocks, kThreads, 0, s>>>(p);
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype,
                                   const terra_swin_attn_desc* desc, const float* bias_table,
                                   const float* explicit_mask, const uint64_t* land_bits,
                                   void* stream) {
  clear_error();
  if (desc == nullptr) return fail(TERRA_ERR_NULL, "desc is NULL");
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr)
    return fail(TERRA_ERR_NULL, "q, k, v and o must be non-NULL");
  if (dtype != TERRA_DTYPE_BF16 && dtype != TERRA_DTYPE_F32)
    return fail(TERRA_ERR_DTYPE, "attention supports bf16 and f32 activations (got dtype %d)", dtype);
  const terra_swin_attn_desc& d = *desc;
  if (d.num_windows <= 0 || d.tokens <= 0 || d.channels <= 0 || d.heads <= 0)
    return fail(TERRA_ERR_SHAPE, "num_windows/tokens/channels/heads must be positive");
  if (d.tokens > kNPad) return fail(TERRA_ERR_UNSUPPORTED, "tokens per window %d > %d", d.tokens, kNPad);
  if (d.channels % d.heads != 0)
    return fail(TERRA_ERR_SHAPE, "channels %d not divisible by heads %d", d.channels, d.heads);
  const int D = d.channels / d.heads;
  if (D != 32 && D != 64) return fail(TERRA_ERR_UNSUPPORTED, "head dim %d not in {32, 64}", D);
  if (d.window_h <= 0 || d.window_w <= 0 || d.window_h > 8 || d.window_w > 8)
    return fail(TERRA_ERR_UNSUPPORTED, "window %dx%d outside 1..8", d.window_h, d.window_w);
  const int n_geo = d.window_h * d.window_w;
  if (n_geo > d.tokens)
    return fail(TERRA_ERR_SHAPE, "window %dx%d has more than %d tokens", d.window_h, d.window_w, d.tokens);
  if (d.n_real <= 0 || d.n_real > d.tokens)
    return fail(TERRA_ERR_SHAPE, "n_real %d outside [1, %d]", d.n_real, d.tokens);
  const int64_t min_stride = d.channels;
  if (d.q_stride < min_stride || d.k_stride < min_stride || d.v_stride < min_stride || d.o_stride < min_stride)
    return fail(TERRA_ERR_SHAPE, "row strides must be >= channels");
  const int elt = dtype_size(dtype);
  const int vec = 16 / elt;
  if (d.q_stride % vec || d.k_stride % vec || d.v_stride % vec || d.o_stride % vec)
    return fail(TERRA_ERR_ALIGN, "row strides must be multiples of %d elements", vec);
  for (const void* ptr : {q, k, v, (const void*)o})
    if ((uintptr_t)ptr % 16 != 0) return fail(TERRA_ERR_ALIGN, "q/k/v/o must be 16-byte aligned");
  if (d.mask_mode != TERRA_MASK_NONE && d.mask_mode != TERRA_MASK_SHIFT && d.mask_mode != TERRA_MASK_EXPLICIT)
    return fail(TERRA_ERR_SHAPE, "unknown mask_mode %d", d.mask_mode);
  if ((d.mask_mode == TERRA_MASK_EXPLICIT || land_bits != nullptr) && d.mask_windows <= 0)
    return fail(TERRA_ERR_SHAPE, "mask_windows must be positive with an explicit mask or land bits");
  if (d.mask_mode == TERRA_MASK_EXPLICIT && explicit_mask == nullptr)
    return fail(TERRA_ERR_NULL, "explicit mask mode without a mask");
  if (d.mask_mode == TERRA_MASK_EXPLICIT && d.num_windows % d.mask_windows != 0)
    return fail(TERRA_ERR_SHAPE, "num_windows %d not divisible by mask windows %d", d.num_windows, d.mask_windows);
  if (d.mask_mode == TERRA_MASK_SHIFT) {
    if (d.win_rows <= 0 || d.win_cols <= 0 || d.frame_h <= 0 || d.frame_w <= 0)
      return fail(TERRA_ERR_SHAPE, "shift mask needs a positive frame and window grid");
    if (d.frame_h % d.window_h || d.frame_w % d.window_w)
      return fail(TERRA_ERR_SHAPE, "frame %dx%d not a multiple of the window", d.frame_h, d.frame_w);
    if (d.win_cols != d.frame_w / d.window_w)
      return fail(TERRA_ERR_SHAPE, "win_cols %d != frame_w / window_w", d.win_cols);
    if (d.win_row_begin < 0 || (d.win_row_begin + d.win_rows) * d.window_h > d.frame_h)
      return fail(TERRA_ERR_SHAPE, "window rows outside the frame");
    if (d.shift_h <= 0 || d.shift_h >= d.window_h || d.shift_w <= 0 || d.shift_w >= d.window_w)
      return fail(TERRA_ERR_SHAPE, "shift mask needs 0 < shift < window (got %d, %d)", d.shift_h, d.shift_w);
    if (d.num_windows % (d.win_rows * d.win_cols) != 0)
      return fail(TERRA_ERR_SHAPE, "num_windows %d not a multiple of the %d windows per image", d.num_windows,
                  d.win_rows * d.win_cols);
  }
  if (bias_table != nullptr && (uintptr_t)bias_table % 4 != 0)
    return fail(TERRA_ERR_ALIGN, "bias_table must be 4-byte aligned");
  const int64_t items = (int64_t)d.num_windows * d.heads;
  if (items >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "too many window-heads for one launch");

  AttnParams p;
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_stride = d.q_stride; p.k_stride = d.k_stride; p.v_stride = d.v_stride; p.o_stride = d.o_stride;
  p.bias_table = bias_table;
  p.explicit_mask = d.mask_mode == TERRA_MASK_EXPLICIT ? explicit_mask : nullptr;
  p.land_bits = land_bits;
  p.items = (int32_t)items;
  p.heads = d.heads;
  p.N = d.tokens;
  p.n_geo = n_geo;
  p.window_h = d.window_h; p.window_w = d.window_w;
  p.table_size = (2 * d.window_h - 1) * (2 * d.window_w - 1);
  p.n_real = d.n_real;
  p.scale = d.scale; p.mask_value = d.mask_value; p.pad_key_value = d.pad_key_value;
  p.mask_mode = d.mask_mode; p.mask_windows = d.mask_windows > 0 ? d.mask_windows : 1;
  p.frame_h = d.frame_h; p.frame_w = d.frame_w; p.shift_h = d.shift_h; p.shift_w = d.shift_w;
  p.win_row_begin = d.win_row_begin; p.win_rows = d.win_rows; p.win_cols = d.win_cols;

  hipStream_t s = (hipStream_t)stream;
  if (dtype == TERRA_DTYPE_BF16) {
    if (D == 32) launch<true, 32>(p, s);
    else launch<true, 64>(p, s);
  } else {
    if (D == 32) launch<false, 32>(p, s);
    else launch<false, 64>(p, s);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
