// Device building blocks of the window-attention core shared by the
// stand-alone attention kernels and the fused block kernel: MFMA fragment
// conventions, the closed-form Swin mask and relative-position bias terms,
// and the log2-domain softmax over one query half.
//
// MFMA v_mfma_f32_16x16x32_bf16 (lane l, g = l/16, c = l%16): the A operand
// lane holds row c, k = 8g..8g+7; the B operand lane holds column c, the same
// k; the accumulator lane holds rows 4g + r (r = 0..3) of column c.  Any
// permutation of the k slots applied to both operands leaves the product
// unchanged, which the kernels use to feed accumulators back as operands.
#pragma once

#include "common.h"

#include <math.h>

namespace terra {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kNPad = 64;       // window tokens padded to 4 tiles of 16
constexpr int kTableMax = 228;  // >= (2*8-1)^2 = 225, multiple of 4
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
  float scale_l2e;    // scale * log2(e)
  float mask_l2e;     // mask_value * log2(e)
  float pad_key_l2e;  // pad_key_value * log2(e)
  int32_t mask_mode, mask_windows;
  int32_t frame_h, frame_w, shift_h, shift_w;
  int32_t win_row_begin, win_rows, win_cols;
  // window-tile kernel
  int32_t group;      // heads per workgroup
  int32_t groups;     // head groups per window
};

__device__ __forceinline__ int region(int coord, int extent, int ws, int shift) {
  // Swin shift-mask slices (0:-ws), (-ws:-shift), (-shift:) of one axis.
  return coord < extent - ws ? 0 : (coord < extent - shift ? 1 : 2);
}

// max(a, b) propagating NaN (IEEE 754-2019 maximum).  On gfx950 a chain of
// these becomes v_maximum3_f32, two inputs per instruction, with nothing
// else: with fmaxf (maxNum) the compiler quiets every operand it cannot prove
// canonical first (MFMA results, values from other lanes), one extra VALU op
// each.  A softmax row max is the same either way, except that a NaN score
// now makes its row NaN, as torch's max does.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Reductions over the 4 lanes l, l^16, l^32, l^48 that share a query row.
// v_permlane16_swap / v_permlane32_swap with both operands = v return the
// value of the own 16-lane (32-lane) half and of the partner half, so one
// VALU op per step replaces an LDS-crossbar shuffle.
__device__ __forceinline__ float xor_max(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = max_nan(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  const uint32_t c = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return max_nan(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

__device__ __forceinline__ float xor_sum(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
  const uint32_t c = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

// ---- LayerNorm statistics from packed bf16 rows -----------------------------
// A lane's partial moments of one token's values, accumulated from the packed
// bf16 pairs by dot products (v_dot2_f32_bf16 against (1, 1) and against the
// pair itself): the products are exact in fp32 and only the sums round.  Two
// chains each (even / odd words), so consecutive words do not wait on each
// other.
struct Bf16Moments {
  float s1a = 0.f, s1b = 0.f, s2a = 0.f, s2b = 0.f;

  template <int kOdd>
  __device__ __forceinline__ void add(uint32_t w) {
    const bf16x2 x2 = __builtin_bit_cast(bf16x2, w);
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3f803f80u);
    if (kOdd) {
      s1b = __builtin_amdgcn_fdot2_f32_bf16(x2, ones, s1b, false);
      s2b = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, s2b, false);
    } else {
      s1a = __builtin_amdgcn_fdot2_f32_bf16(x2, ones, s1a, false);
      s2a = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, s2a, false);
    }
  }
  __device__ __forceinline__ void add4(const uint4& r) {
    add<0>(r.x);
    add<1>(r.y);
    add<0>(r.z);
    add<1>(r.w);
  }
};

// mean and var of a token whose values lie on an 8-lane group (inv_c = 1 / C),
// from each lane's moments: var = E[x^2] - mean^2, which loses accuracy to
// cancellation when the mean is large against the spread (the sums carry a
// relative error of a few 2^-24 of mean^2 + var).  token_stats_recheck says
// whether any lane of the wave has mean^2 > 64 var, i.e. could be off by more
// than about 1e-4 of var; the wave then recomputes var from centred values
// (centred_sq4 over the same chunks, group8_sum, times inv_c).  Every lane of
// the wave must take part.
__device__ __forceinline__ void token_stats8(const Bf16Moments& m, float inv_c, float& mean, float& var) {
  mean = group8_sum(m.s1a + m.s1b) * inv_c;
  var = group8_sum(m.s2a + m.s2b) * inv_c - mean * mean;
}

__device__ __forceinline__ bool token_stats_recheck(float mean, float var) {
  return __builtin_amdgcn_ballot_w64(mean * mean > 64.f * var) != 0;
}

// sq + the sum of (x - mean)^2 over the eight bf16 values of a chunk.
__device__ __forceinline__ float centred_sq4(const uint4& r, float mean, float sq) {
  const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float dl = __uint_as_float(w4[i] << 16) - mean;
    const float dh = __uint_as_float(w4[i] & 0xffff0000u) - mean;
    sq = __builtin_fmaf(dl, dl, sq);
    sq = __builtin_fmaf(dh, dh, sq);
  }
  return sq;
}

// y = (x rstd - mean rstd) gamma + beta of a chunk's eight bf16 values (two
// FMAs per value: nmr = -mean rstd), rounded once to bf16.
__device__ __forceinline__ uint4 normalize_chunk(const uint4& r, float rstd, float nmr, const float (&gm)[8],
                                                 const float (&bt)[8]) {
  const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(w4[i] << 16), hi = __uint_as_float(w4[i] & 0xffff0000u);
    o[i] = pack_bf16x2(__builtin_fmaf(__builtin_fmaf(lo, rstd, nmr), gm[2 * i], bt[2 * i]),
                       __builtin_fmaf(__builtin_fmaf(hi, rstd, nmr), gm[2 * i + 1], bt[2 * i + 1]));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Mask state of one window (uniform across the wave).
struct WindowMaskState {
  bool use_shift;     // window touches the last window row / column of the frame
  bool use_mask;      // shift boundary or any land key
  int wr, wc;         // window row / column in the frame
  uint64_t land;      // land bit per key
};

__device__ __forceinline__ WindowMaskState window_mask_state(const AttnParams& p, int w, bool analytic,
                                                             bool read_land = true) {
  WindowMaskState m;
  m.use_shift = false;
  m.wr = m.wc = 0;
  if (analytic && p.mask_mode == TERRA_MASK_SHIFT) {
    const int per_img = p.win_rows * p.win_cols;
    const int wl = w % per_img;
    const int rr = wl / p.win_cols;
    m.wr = rr + p.win_row_begin;
    m.wc = wl - rr * p.win_cols;
    m.use_shift = (m.wr + 2) * p.window_h > p.frame_h || (m.wc + 2) * p.window_w > p.frame_w;
  }
  m.land = (read_land && p.land_bits != nullptr) ? p.land_bits[w % p.mask_windows] : 0ull;
  m.use_mask = m.use_shift || m.land != 0ull;
  return m;
}

// Per-lane index terms of the window geometry.
//   kWs8: closed form for 8x8 windows.
//   generic: lane t computes token t's terms, other lanes fetch them with
//   shuffles; bias index idx(i, j) = base(i) - off(j).
template <bool kWs8>
struct LaneGeom {
  const float* tab8;      // kWs8: bias pointer so that offsets 30*(it-jt) - r + 93 >= 0
  const float* tab;       // generic: this head's bias column (x log2e)
  int g_base, g_rid;      // generic: this lane's token terms (shuffle sources)
  int off_j[kWs8 ? 1 : 4][4];
  uint64_t rid_pack;      // 4-bit region id of key (jt, r) at bit 4*(4*jt + r)
  uint64_t land_lane;     // land bit of key (jt, r) at bit 16*jt + r
};

template <bool kWs8>
__device__ __forceinline__ void lane_geom_init(LaneGeom<kWs8>& lg, const AttnParams& p, const WindowMaskState& m,
                                               const float* tab, int lane) {
  const int g = lane >> 4, c16 = lane & 15;
  lg.tab = tab;
  lg.g_base = lg.g_rid = 0;
  int g_off = 0;
  if constexpr (kWs8) {
    const int lane_base = 15 * ((c16 >> 3) - (g >> 1) + 7) + (c16 & 7) - 4 * (g & 1) + 7;  // in [93, 134]
    lg.tab8 = tab + (lane_base - 93);
  } else {
    lg.tab8 = tab;
    const int t = lane < p.n_geo ? lane : p.n_geo - 1;
    const int ti = t / p.window_w;
    const int tj = t - ti * p.window_w;
    const int rel_w = 2 * p.window_w - 1;
    lg.g_base = (ti + p.window_h - 1) * rel_w + tj + p.window_w - 1;
    g_off = ti * rel_w + tj;
    if (m.use_shift)
      lg.g_rid = 3 * region(m.wr * p.window_h + ti, p.frame_h, p.window_h, p.shift_h) +
                 region(m.wc * p.window_w + tj, p.frame_w, p.window_w, p.shift_w);
  }
  lg.rid_pack = 0;
  lg.land_lane = m.land >> (4 * g);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jt + 4 * g + r;
      int rid;
      if constexpr (kWs8) {
        rid = m.use_shift ? 3 * region(m.wr * 8 + 2 * jt + (g >> 1), p.frame_h, 8, p.shift_h) +
                                region(m.wc * 8 + 4 * (g & 1) + r, p.frame_w, 8, p.shift_w)
                          : 0;
      } else {
        const int jg = j < p.n_geo ? j : p.n_geo - 1;
        lg.off_j[jt][r] = __shfl(g_off, jg);
        rid = __shfl(lg.g_rid, jg);
      }
      lg.rid_pack |= (uint64_t)rid << (4 * (4 * jt + r));
    }
  }
}

// Turns the raw scores of query tiles it = 2*half + {0, 1} into unnormalised
// probabilities in place and returns 1/rowsum per tile.
template <bool kWs8, bool kExplicit>
__device__ __forceinline__ void softmax_half(f32x4 (&s)[2][4], float (&inv)[2], int half, const AttnParams& p,
                                             const WindowMaskState& m, const LaneGeom<kWs8>& lg,
                                             const float* emask, int lane) {
  const int g = lane >> 4, c16 = lane & 15;
  int base_i[2] = {0, 0}, rid_i[2] = {0, 0};
  bool i_geo[2] = {true, true};
#pragma unroll
  for (int il = 0; il < 2; ++il) {
    const int it = 2 * half + il;
    const int i = 16 * it + c16;
    if constexpr (kWs8) {
      if (m.use_shift)
        rid_i[il] = 3 * region(m.wr * 8 + 2 * it + (c16 >> 3), p.frame_h, 8, p.shift_h) +
                    region(m.wc * 8 + (c16 & 7), p.frame_w, 8, p.shift_w);
    } else {
      const int ig = i < p.n_geo ? i : p.n_geo - 1;
      i_geo[il] = i < p.n_geo;
      base_i[il] = __shfl(lg.g_base, ig);
      rid_i[il] = __shfl(lg.g_rid, ig);
    }
  }
  // Pass 1, branch-free: y = s * scale * log2e + bias * log2e.
#pragma unroll
  for (int il = 0; il < 2; ++il) {
    const int it = 2 * half + il;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float b;
        if constexpr (kWs8) {
          b = lg.tab8[30 * (it - jt) - r + 93];
        } else {
          const int j = 16 * jt + 4 * g + r;
          b = lg.tab[base_i[il] - lg.off_j[jt][r]];  // clamped indices: always in range
          b = (i_geo[il] && j < p.n_geo) ? b : 0.f;
        }
        s[il][jt][r] = __builtin_fmaf(s[il][jt][r], p.scale_l2e, b);
      }
    }
  }
  // Pass 2 (only windows with a shift boundary or land keys): + mask.
  if constexpr (kExplicit) {
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int i = 16 * (2 * half + il) + c16;
      const int ig = i < p.n_geo ? i : p.n_geo - 1;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        float mrow[4];
        if constexpr (kWs8) {
          // 8x8 windows: n_geo == 64, and the launchers take this path only
          // for a 16-byte aligned mask (global or staged in LDS), so a lane's
          // four keys are one load.
          const float4 e4 = *reinterpret_cast<const float4*>(emask + i * 64 + 16 * jt + 4 * g);
          mrow[0] = e4.x; mrow[1] = e4.y; mrow[2] = e4.z; mrow[3] = e4.w;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = 16 * jt + 4 * g + r;
            mrow[r] = emask[ig * p.n_geo + (j < p.n_geo ? j : p.n_geo - 1)];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jt + 4 * g + r;
          const float me = mrow[r] * kLog2e;
          const bool land_j = (lg.land_lane >> (16 * jt + r)) & 1ull;
          const bool jin = kWs8 || j < p.n_geo;
          s[il][jt][r] += ((i_geo[il] && jin) ? me : 0.f) + ((land_j && jin) ? p.mask_l2e : 0.f);
        }
      }
    }
  } else if (m.use_shift) {  // boundary windows: region test per element, plus land keys
#pragma unroll
    for (int il = 0; il < 2; ++il) {
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jt + 4 * g + r;
          const int rid_j = (int)((lg.rid_pack >> (4 * (4 * jt + r))) & 15ull);
          const bool land_j = ((lg.land_lane >> (16 * jt + r)) & 1ull) && (kWs8 || j < p.n_geo);
          const float ms = (i_geo[il] && rid_i[il] != rid_j) ? p.mask_l2e : 0.f;
          s[il][jt][r] += ms + (land_j ? p.mask_l2e : 0.f);
        }
      }
    }
  } else if (m.land != 0ull) {  // land keys only: one additive term per key column
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jt + 4 * g + r;
        const bool land_j = ((lg.land_lane >> (16 * jt + r)) & 1ull) && (kWs8 || j < p.n_geo);
        const float ml = land_j ? p.mask_l2e : 0.f;
#pragma unroll
        for (int il = 0; il < 2; ++il) s[il][jt][r] += ml;
      }
    }
  }
  // Padded keys (generic path): keys >= n_real take the pad value, keys
  // beyond the window's rows are excluded.
  if constexpr (!kWs8) {
#pragma unroll
    for (int il = 0; il < 2; ++il)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jt + 4 * g + r;
          float y = s[il][jt][r];
          y = j >= p.n_real ? p.pad_key_l2e : y;
          s[il][jt][r] = j >= p.N ? -INFINITY : y;
        }
  }
  // Row softmax: max, exp2, sum.
#pragma unroll
  for (int il = 0; il < 2; ++il) {
    float mx = s[il][0][0];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = max_nan(mx, s[il][jt][r]);
    mx = xor_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(s[il][jt][r] - mx);
        s[il][jt][r] = e;
        sum += e;
      }
    }
    inv[il] = __builtin_amdgcn_rcpf(xor_sum(sum));
  }
}

// S^T tiles of two query tiles from K fragments (4 key tiles) and the Q
// fragments of those two query tiles (bf16: one 16-byte fragment per
// 32-channel step; fp32: D/16 fragments, lane group g holding channels
// [g*D/4, (g+1)*D/4) in both operands).
template <bool kBf16, int D>
__device__ __forceinline__ void scores_pair(f32x4 (&s)[2][4], const uint4 (&kf)[4][kBf16 ? D / 32 : D / 16],
                                            const uint4 (&qp)[2][kBf16 ? D / 32 : D / 16]) {
  constexpr int kKF = kBf16 ? D / 32 : D / 16;
#pragma unroll
  for (int il = 0; il < 2; ++il) {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (kBf16) {
#pragma unroll
        for (int ks = 0; ks < kKF; ++ks)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[jt][ks]),
                                                        __builtin_bit_cast(bf16x8, qp[il][ks]), acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int ks = 0; ks < kKF; ++ks) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = __uint_as_float(reinterpret_cast<const uint32_t*>(&kf[jt][ks])[e]);
            const float b = __uint_as_float(reinterpret_cast<const uint32_t*>(&qp[il][ks])[e]);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
          }
        }
      }
      s[il][jt] = acc;
    }
  }
}

// O^T tiles (ct, il) = V^T P^T for one half.  bf16: vfrag(ct, js) returns the
// V^T operand fragment whose k-slot e (lane group g) is key
// 32*js + 16*(e/4) + 4g + e%4 and whose row is channel 16*ct + c; fp32:
// vread(j, c) returns V[j][c].
template <bool kBf16, int D, class VFrag>
__device__ __forceinline__ void pv_half(f32x4 (&o)[D / 16][2], const f32x4 (&s)[2][4], int lane, VFrag vsrc) {
  const int g = lane >> 4, c16 = lane & 15;
  constexpr int kCT = D / 16;
#pragma unroll
  for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
    for (int il = 0; il < 2; ++il) o[ct][il] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (kBf16) {
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      // P^T fragment from the accumulators, same k-slot order as vfrag.
      bf16x8 pf[2];
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        uint32_t wds[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          wds[e / 2] = pack_bf16x2(s[il][2 * js + (e >> 2)][e & 3], s[il][2 * js + (e >> 2)][(e & 3) + 1]);
        pf[il] = __builtin_bit_cast(bf16x8, wds);
      }
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct) {
        const bf16x8 vf = vsrc(ct, js);
#pragma unroll
        for (int il = 0; il < 2; ++il)
          o[ct][il] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[il], o[ct][il], 0, 0, 0);
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
          const float a = vsrc(j, 16 * ct + c16);
#pragma unroll
          for (int il = 0; il < 2; ++il)
            o[ct][il] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s[il][jt][r], o[ct][il], 0, 0, 0);
        }
      }
    }
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: within each 16-lane group, output lane l receives
// element (l & 3) of the 8-byte words addressed by lanes (l >> 2) + 4m,
// m = 0..3.  When lane s addresses V[row(s >> 2)][c0 + 4*(s & 3) ..], lane l
// receives V[row(m)][c0 + l] for m = 0..3: four keys of one channel.
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* addr) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(__attribute__((address_space(3))) uint8_t*)(const_cast<uint8_t*>(addr)));
  return __builtin_bit_cast(uint2, r);
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (s_waitcnt vmcnt(0)),
// which would drain prefetches and output stores at each barrier; this waits
// for the wave's LDS operations only.  Data loaded into LDS by global->LDS
// DMA needs its own s_waitcnt vmcnt before the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One 16-byte global -> LDS load per lane (nontemporal): lane l of the wave
// writes LDS bytes [lds_base + 16 l, +16).  Issued from inline assembly so
// that the compiler does not place an s_waitcnt vmcnt(0) before every later
// LDS read (it cannot tell which LDS bytes the load writes); the caller waits
// for it with an explicit vmcnt.  lds_base is wave-uniform (it goes to M0).
__device__ __forceinline__ void dma_to_lds16(const void* src, uint32_t lds_base) {
  // M0 is bound by the operand constraint (the compiler writes it); the
  // s_nop is the wait state between an M0 write and an LDS DMA.
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(src), "{m0}"(lds_base) : "memory");
}

// The same load without the streaming hint: the lines stay in L2 for a
// kernel that reads the rows again from global memory (its residual add).
__device__ __forceinline__ void dma_to_lds16_cached(const void* src, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds_base) : "memory");
}

// The cached load from a wave-uniform base (SGPRs) plus a 32-bit lane offset
// (a VGPR): lane l writes LDS bytes [lds_base + 16 l, + 16).  Loop-invariant
// lane offsets stay in registers and only the base moves.
__device__ __forceinline__ void dma_to_lds16_at(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

// One 4-byte global -> LDS load per lane from a wave-uniform base plus a
// 32-bit lane offset: lane l writes LDS bytes [lds_base + 4 l, + 4).
__device__ __forceinline__ void dma_to_lds4_at(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

// 16-byte slot of (key row, chunk) in a tile of cpr chunks per
// row.  256-byte rows (head dim 128) are a whole bank period, so the chunk is
// XORed with row & 15: the 16 rows of a fragment read hit 16 distinct 16-byte
// bank groups (and 8 consecutive rows 8 distinct ones).  128-byte rows take
// the 8x8 kernels' (row >> 1) & 7.
template <int cpr>
__device__ __forceinline__ int flash_slot(int row, int chunk) {
  return row * cpr + (chunk ^ (cpr >= 16 ? (row & 15) : ((row >> 1) & 7)));
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte chunk slot of (row, chunk) in a [64][cpr] tile: the chunk index is
// XOR-swizzled within its aligned group of 8 so that the 16 rows read by one
// fragment load (and the 4 row groups of a V^T read) hit distinct banks.
__device__ __forceinline__ int tile_slot(int row, int chunk, int cpr) {
  return row * cpr + (chunk ^ ((row >> 1) & 7));
}

// One wave of window-tile attention on [64][cpr]-chunk bf16 tiles in LDS
// (tile_slot layout): head `head` occupies columns [col_head*D, (col_head+1)*D)
// of the Q, K and V tiles, the wave computes query tiles 2*half and 2*half + 1
// (K and Q fragments by row, V^T fragments by transposed reads), and O
// overwrites the wave's own Q rows of that head.  `tab` is the head's bias
// column (x log2e) with kTableMax entries; `emask` (kExplicit) the window's
// [64][64] dense mask in LDS.
template <int D, int kCpr, bool kExplicit = false>
__device__ __forceinline__ void tile_attention_wave(uint8_t* qs, const uint8_t* ks, const uint8_t* vs, int col_head,
                                                    int half, const AttnParams& p, const WindowMaskState& m,
                                                    const float* tab, int lane, const float* emask = nullptr) {
  const int g = lane >> 4, c16 = lane & 15;
  LaneGeom<true> lg;
  lane_geom_init<true>(lg, p, m, tab, lane);
  constexpr int kKF = D / 32;
  uint4 kf[4][kKF], qp[2][kKF];
  const int hc = col_head * (D / 8);  // first chunk of this head
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int s = 0; s < kKF; ++s)
      kf[t][s] = *reinterpret_cast<const uint4*>(ks + tile_slot(16 * t + c16, hc + 4 * s + g, kCpr) * 16);
#pragma unroll
  for (int il = 0; il < 2; ++il)
#pragma unroll
    for (int s = 0; s < kKF; ++s)
      qp[il][s] = *reinterpret_cast<const uint4*>(
          qs + tile_slot(16 * (2 * half + il) + c16, hc + 4 * s + g, kCpr) * 16);
  // V^T fragment (ct, js): two transposed reads, keys 32*js + 16*half2 + 4g + m.
  auto vfrag = [&](int ct, int js) -> bf16x8 {
    const int cc = col_head * D + 16 * ct + 4 * (c16 & 3);  // channel of this source lane
    uint2 part[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
      part[h2] = lds_read_tr16(vs + tile_slot(row, cc >> 3, kCpr) * 16 + (cc & 7) * 2);
    }
    const uint32_t w[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
    return __builtin_bit_cast(bf16x8, w);
  };
  // This wave's Q rows are in registers; its O overwrites exactly those
  // rows of its head's columns.  Order the reads before the writes.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  f32x4 s[2][4];
  scores_pair<true, D>(s, kf, qp);
  float inv[2];
  softmax_half<true, kExplicit>(s, inv, half, p, m, lg, emask, lane);
  f32x4 o[D / 16][2];
  pv_half<true, D>(o, s, lane, vfrag);
#pragma unroll
  for (int il = 0; il < 2; ++il) {
    const int i = 16 * (2 * half + il) + c16;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) {
      const f32x4 v = o[ct][il] * inv[il];
      const int cc = col_head * D + 16 * ct + 4 * g;  // 4 channels, 8 bytes
      uint2 pk;
      pk.x = pack_bf16x2(v[0], v[1]);
      pk.y = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint2*>(qs + tile_slot(i, cc >> 3, kCpr) * 16 + (cc & 7) * 2) = pk;
    }
  }
}

// bf16 operand fragment of ones: 1^T P^T puts each query's sum over the keys
// in every row of the tile, so the row sum runs on the matrix cores (two
// MFMAs per query tile) instead of 16 adds and a cross-lane reduction.
__device__ __forceinline__ bf16x8 ones_frag() {
  const uint32_t w[4] = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  return __builtin_bit_cast(bf16x8, w);
}

// Land terms of an 8x8 window for lane group g: land_term[jt][r] = mask_term
// if key 16jt + 4g + r is land, else 0 (a sign-extended bit ANDed with the
// term's bits).
__device__ __forceinline__ void land_terms(f32x4 (&land_term)[4], uint64_t land, int g, float mask_term) {
  const uint64_t ll = land >> (4 * g);
  const uint32_t half[2] = {(uint32_t)ll, (uint32_t)(ll >> 32)};
  const uint32_t mb = __float_as_uint(mask_term);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int bit = 16 * (jt & 1) + r;
      // v_bfe_i32 sign-extends the bit (0 or all ones).  Written out, because
      // the compiler otherwise turns the shift pair into a compare and a
      // VCC-masked select, about three times the issue cost.
      uint32_t sel;
      asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(sel) : "v"(half[jt >> 1]), "s"(bit));
      land_term[jt][r] = __uint_as_float(sel & mb);
    }
}

// Bias columns read by attend_qtiles are staged reversed: slot kTableRev - i
// holds relative index i, so the four keys r = 0..3 of an accumulator lane
// (index lane_base + 30 (it - jt) - r) sit at increasing addresses and load
// straight into the accumulator registers in order.
constexpr int kTableRev = kTableMax - 1;

// This lane's pointer into a reversed column: element (it, jt, r) of an 8x8
// window is at [30 (3 - it + jt) + r].
__device__ __forceinline__ const float* lane_bias_rev(const float* tab_rev, int lane) {
  const int g = lane >> 4, c16 = lane & 15;
  const int lane_base = 15 * ((c16 >> 3) - (g >> 1) + 7) + (c16 & 7) - 4 * (g & 1) + 7;  // in [93, 134]
  return tab_rev + (kTableRev - 90 - lane_base);  // offset in [3, 44]; largest slot 227
}

// Mask modes of attend_qtiles, chosen at compile time so that the query-tile
// loop of a window holds no branch whose two sides the register allocator
// would merge with copies: kMaskNone, kMaskLand (land keys only), kMaskShift
// (shift regions, plus land keys when the window has any).
constexpr int kMaskNone = 0, kMaskLand = 1, kMaskShift = 2;

template <int V>
struct MaskMode {
  static constexpr int value = V;
};

// Scores, softmax and O^T = V^T P^T of NQ 16-query tiles it0, it0 + 1, ... of
// an 8x8 window against its 64 keys.  The relative-position bias (tabr from
// lane_bias_rev) is the accumulator init of the S^T MFMA; land keys and shift
// regions are added to its result.  All terms are in the units of the
// accumulator: the base-2 logit is acc * logit_scale.  With a Q operand that
// already carries scale * log2(e), logit_scale = 1 and the terms are x log2e;
// with raw q, logit_scale = scale * log2(e) (> 0) and the terms are divided by
// scale.
// land_term[jt][r]: mask term of land key 16jt + 4g + r, else 0 (read only
// when the window has land keys); mask_term: the shift-region term.
// kf[jt][c]: K operand of key tile jt, k-step c (KF = head dim / 32 steps);
// vfrag(ct, js): V^T operand of column tile ct (CT = head dim / 16 tiles;
// keys 32js + 16(e/4) + 4g + e%4); qf[q][c], rid_q[q]: Q operand and query
// region id of tile it0 + q.  Returns per tile the unnormalised O^T tiles and
// 1 / (sum over keys of the bf16 probabilities that enter P V), so that the
// normalised weights sum to 1.
template <int kMask, int NQ, int KF, int CT, class VFrag>
__device__ __forceinline__ void attend_qtiles(f32x4 (&o)[NQ][CT], float (&inv)[NQ], int it0,
                                              const uint4 (&kf)[4][KF], const uint4 (&qf)[NQ][KF], const float* tabr,
                                              const WindowMaskState& m, const f32x4 (&land_term)[4],
                                              uint64_t rid_pack, const int (&rid_q)[NQ], float mask_term,
                                              float logit_scale, VFrag vfrag) {
  // The NQ query tiles advance through each stage together, which gives the
  // scheduler independent MFMA / VALU chains to interleave.
  f32x4 s[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[q][jt][r] = tabr[30 * (3 - it0 - q + jt) + r];
#pragma unroll
  for (int c = 0; c < KF; ++c)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        s[q][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[jt][c]),
                                                           __builtin_bit_cast(bf16x8, qf[q][c]), s[q][jt], 0, 0, 0);
  // Mask terms after the MFMA, on its result.
  if constexpr (kMask == kMaskShift) {  // boundary windows: region test per element, plus land keys
    const bool land = m.land != 0ull;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rid_j = (int)((rid_pack >> (4 * (4 * jt + r))) & 15ull);
          s[q][jt][r] += (rid_j != rid_q[q] ? mask_term : 0.f) + (land ? land_term[jt][r] : 0.f);
        }
  } else if constexpr (kMask == kMaskLand) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) s[q][jt] += land_term[jt];
  }
  float mx[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    mx[q] = s[q][0][0];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx[q] = max_nan(mx[q], s[q][jt][r]);
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) mx[q] = xor_max(mx[q]);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const float neg_mx = -mx[q] * logit_scale;  // logit_scale > 0: the max commutes with the scaling
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        s[q][jt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[q][jt][r], logit_scale, neg_mx));
  }
  const bf16x8 ones = ones_frag();
  f32x4 rs[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[q][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    rs[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int js = 0; js < 2; ++js) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      uint32_t wds[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        wds[e / 2] = pack_bf16x2(s[q][2 * js + (e >> 2)][e & 3], s[q][2 * js + (e >> 2)][(e & 3) + 1]);
      const bf16x8 pf = __builtin_bit_cast(bf16x8, wds);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        o[q][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag(ct, js), pf, o[q][ct], 0, 0, 0);
      rs[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, rs[q], 0, 0, 0);
    }
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) inv[q] = __builtin_amdgcn_rcpf(rs[q][0]);
}

// Head dim 32: one k-step, two column tiles (K and Q operands as plain arrays).
template <int kMask, int NQ, class VFrag>
__device__ __forceinline__ void attend_qtiles(f32x4 (&o)[NQ][2], float (&inv)[NQ], int it0, const uint4 (&kf)[4],
                                              const uint4 (&qf)[NQ], const float* tabr, const WindowMaskState& m,
                                              const f32x4 (&land_term)[4], uint64_t rid_pack, const int (&rid_q)[NQ],
                                              float mask_term, float logit_scale, VFrag vfrag) {
  attend_qtiles<kMask, NQ, 1, 2>(o, inv, it0, reinterpret_cast<const uint4(&)[4][1]>(kf),
                                 reinterpret_cast<const uint4(&)[NQ][1]>(qf), tabr, m, land_term, rid_pack, rid_q,
                                 mask_term, logit_scale, vfrag);
}

}  // namespace

// The backward of windows of more than 64 tokens (window_attention.hip), for
// terra_swin_attn_bwd: the same arguments, validated there for that path.
__attribute__((visibility("hidden"))) int flash_attention_backward(
    const void* q, const void* k, const void* v, const void* dout, void* dq, void* dk, void* dv, int dtype,
    const terra_swin_attn_bwd_desc* desc, const float* bias_table, float* dbias_table, const float* explicit_mask,
    const uint64_t* land_bits, void* stream);

}  // namespace terra
