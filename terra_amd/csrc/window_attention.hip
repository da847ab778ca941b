// Fused per-window multi-head attention forward for gfx950.
//
// Math per (window, head), window padded to 64 tokens (4 tiles of 16), head
// dim D:
//
//   S^T = K Q^T      v_mfma_f32_16x16x32_bf16 (bf16) / 16x16x4_f32 (fp32)
//   softmax          fp32 in the log2 domain: y = s*scale*log2e + bias*log2e
//                    (+ mask*log2e), p = exp2(y - max); a query row lives in
//                    4 lanes x 16 registers (in-lane reduction + 2 shuffles)
//   O^T = V^T P^T    P^T comes out of the S^T accumulators already in MFMA
//                    operand order; V is read from LDS as the transposed
//                    operand; 1/sum is applied to O, not to P.
//
// Accumulator layout of a 16x16 tile (lane l, g = l/16, c = l%16): element
// (row 4g + r, col c), r = 0..3.  In S^T rows are keys and columns queries,
// so lane l holds queries i = 16*it + c and keys j = 16*jt + 4g + r.  Query
// tiles are processed in two halves (it = 0,1 then 2,3): at most 32 score
// registers are live and a wave fits in 128 VGPRs.
//
// Two kernels share that core:
//
//   window_attn_tile_kernel   bf16, 8x8 windows, no padded tokens, analytic
//       masks.  A persistent workgroup loops over (window, group of G heads)
//       units, two waves per head (one per query half).  The group's q, k, v
//       rows (a contiguous slice of G*D channels, whole 128-byte lines) are
//       streamed into LDS with nontemporal loads while the previous unit is
//       computed; O is staged in LDS over Q and streamed out as whole lines.
//       The relative-position index of lane element (it, jt, r) is
//       lane_base + 30*(it - jt) - r, so the bias comes from LDS with
//       compile-time offsets.
//
//   window_attn_wave_kernel   everything else (fp32, any window up to 8x8,
//       padded tokens and keys, explicit dense masks): one wavefront per
//       (window, head), K and Q fragments loaded straight from global memory,
//       V staged in the wave's LDS.
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

// Reductions over the 4 lanes l, l^16, l^32, l^48 that share a query row.
// v_permlane16_swap / v_permlane32_swap with both operands = v return the
// value of the own 16-lane (32-lane) half and of the partner half, so one
// VALU op per step replaces an LDS-crossbar shuffle.
__device__ __forceinline__ float xor_max(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto p16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
  const uint32_t c = __float_as_uint(v);
  const auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
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

// Mask state of one window (uniform across the wave).
struct WindowMaskState {
  bool use_shift;     // window touches the last window row / column of the frame
  bool use_mask;      // shift boundary or any land key
  int wr, wc;         // window row / column in the frame
  uint64_t land;      // land bit per key
};

__device__ __forceinline__ WindowMaskState window_mask_state(const AttnParams& p, int w, bool analytic) {
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
  m.land = p.land_bits != nullptr ? p.land_bits[w % p.mask_windows] : 0ull;
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
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jt + 4 * g + r;
          const int jg = j < p.n_geo ? j : p.n_geo - 1;
          const float me = emask[ig * p.n_geo + jg] * kLog2e;
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
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[il][jt][r]);
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

// ============================================================================
// window-tile kernel: bf16, 8x8 windows, one workgroup per (window, head group)
// ============================================================================

constexpr int kTileMaxRowBytes = 384;  // G*D*2 <= 384 (<= 192 bf16 channels)

// 16-byte chunk slot of (row, chunk) in a [64][cpr] tile: the chunk index is
// XOR-swizzled within its aligned group of 8 so that the 16 rows read by one
// fragment load (and the 4 row groups of a V^T read) hit distinct banks.
__device__ __forceinline__ int tile_slot(int row, int chunk, int cpr) {
  return row * cpr + (chunk ^ ((row >> 1) & 7));
}

template <int D, int G>
__global__ __launch_bounds__(G * 128) void window_attn_tile_kernel(const AttnParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int nthreads = G * 128;              // two waves per head
  constexpr int cpr = G * D / 8;                 // chunks per row (multiple of 8)
  constexpr int tile_bytes = kNPad * cpr * 16;
  static_assert(cpr % 8 == 0 && G * D * 2 <= kTileMaxRowBytes, "head group must be whole 128-byte lines");
  uint8_t* qs = smem;                            // Q, later O
  uint8_t* ks = smem + tile_bytes;
  uint8_t* vs = smem + 2 * tile_bytes;
  float* tables = reinterpret_cast<float*>(smem + 3 * tile_bytes);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = wave >> 1;                    // head of the group
  const int half = wave & 1;                     // query tiles 2*half, 2*half + 1
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int units = (p.items / p.heads) * p.groups;  // (window, head group) pairs

  // A workgroup streams whole rows: each thread keeps one 16-byte chunk column
  // of the group's row slice and steps down rows row0 + kRowStep*u.
  constexpr int kPer = kNPad * cpr / nthreads;   // chunks per thread per tensor (D/16)
  constexpr int kRowStep = nthreads / cpr;
  static_assert(kRowStep * cpr == nthreads && kRowStep * kPer == kNPad, "row tiling");
  const int row0 = tid / cpr, chunk0 = tid % cpr;

  // q, k, v of one unit -> registers (nontemporal: every byte is read once).
  uint4 buf[3][kPer];
  auto fetch = [&](int unit) {
    const int w = unit / p.groups, hg = unit - w * p.groups;
    const int64_t row_base = (int64_t)w * kNPad + row0;
    const int col = hg * G * D + chunk0 * 8;
    const uint16_t* src[3] = {reinterpret_cast<const uint16_t*>(p.q) + row_base * p.q_stride + col,
                              reinterpret_cast<const uint16_t*>(p.k) + row_base * p.k_stride + col,
                              reinterpret_cast<const uint16_t*>(p.v) + row_base * p.v_stride + col};
    const int64_t step[3] = {kRowStep * p.q_stride, kRowStep * p.k_stride, kRowStep * p.v_stride};
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int u = 0; u < kPer; ++u)
        buf[t][u] = __builtin_bit_cast(
            uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src[t] + u * step[t])));
  };

  int unit = blockIdx.x;
  if (unit >= units) return;  // uniform across the workgroup
  fetch(unit);
  int table_group = -1;
  float* tab = tables + head * kTableMax;

  // Persistent loop, software-pipelined: while unit n is computed from LDS,
  // the loads of unit n + gridDim.x are in flight into `buf`.
  for (;;) {
    const int w = unit / p.groups, hg = unit - w * p.groups;
    __syncthreads();  // the previous unit's O has been read out of LDS
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int off = tile_slot(row0 + kRowStep * u, chunk0, cpr) * 16;
      *reinterpret_cast<uint4*>(qs + off) = buf[0][u];
      *reinterpret_cast<uint4*>(ks + off) = buf[1][u];
      *reinterpret_cast<uint4*>(vs + off) = buf[2][u];
    }
    if (hg != table_group) {  // bias column of this head (x log2e); the two waves split it
      table_group = hg;
      const int h = hg * G + head;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = lane + 64 * (2 * u + half);
        if (e < kTableMax)
          tab[e] = (p.bias_table != nullptr && e < p.table_size) ? p.bias_table[(int64_t)e * p.heads + h] * kLog2e
                                                                : 0.f;
      }
    }
    __syncthreads();
    const int next = unit + (int)gridDim.x;
    if (next < units) fetch(next);

    // ---- this wave: one head, query tiles 2*half, 2*half + 1 ---------------
    const WindowMaskState m = window_mask_state(p, w, true);
    LaneGeom<true> lg;
    lane_geom_init<true>(lg, p, m, tab, lane);
    constexpr int kKF = D / 32;
    uint4 kf[4][kKF], qp[2][kKF];
    const int hc = head * (D / 8);               // first chunk of this head
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < kKF; ++s)
        kf[t][s] = *reinterpret_cast<const uint4*>(ks + tile_slot(16 * t + c16, hc + 4 * s + g, cpr) * 16);
#pragma unroll
    for (int il = 0; il < 2; ++il)
#pragma unroll
      for (int s = 0; s < kKF; ++s)
        qp[il][s] = *reinterpret_cast<const uint4*>(
            qs + tile_slot(16 * (2 * half + il) + c16, hc + 4 * s + g, cpr) * 16);
    // V^T fragment (ct, js): two transposed reads, keys 32*js + 16*half2 + 4g + m.
    auto vfrag = [&](int ct, int js) -> bf16x8 {
      const int cc = head * D + 16 * ct + 4 * (c16 & 3);  // channel of this source lane
      uint2 part[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
        part[h2] = lds_read_tr16(vs + tile_slot(row, cc >> 3, cpr) * 16 + (cc & 7) * 2);
      }
      const uint32_t w[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
      return __builtin_bit_cast(bf16x8, w);
    };
    // This wave's Q rows are in registers; its O overwrites exactly those
    // rows of its head's columns.  Order the reads before the writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    {
      f32x4 s[2][4];
      scores_pair<true, D>(s, kf, qp);
      float inv[2];
      softmax_half<true, false>(s, inv, half, p, m, lg, nullptr, lane);
      f32x4 o[D / 16][2];
      pv_half<true, D>(o, s, lane, vfrag);
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        const int i = 16 * (2 * half + il) + c16;
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          const f32x4 v = o[ct][il] * inv[il];
          const int cc = head * D + 16 * ct + 4 * g;  // 4 channels, 8 bytes
          uint2 pk;
          pk.x = pack_bf16x2(v[0], v[1]);
          pk.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2*>(qs + tile_slot(i, cc >> 3, cpr) * 16 + (cc & 7) * 2) = pk;
        }
      }
    }
    __syncthreads();

    // ---- stream O out (whole lines) ------------------------------------------
    {
      const int64_t row_base = (int64_t)w * kNPad + row0;
      uint16_t* dst = reinterpret_cast<uint16_t*>(p.o) + row_base * p.o_stride + hg * G * D + chunk0 * 8;
      const int64_t ostep = kRowStep * p.o_stride;
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int off = tile_slot(row0 + kRowStep * u, chunk0, cpr) * 16;
        const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(qs + off));
        __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(dst + u * ostep));
      }
    }
    if (next >= units) break;
    unit = next;
  }
}

// ============================================================================
// per-wave kernel (generic path)
// ============================================================================

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <bool kBf16> struct EltTraits;
template <> struct EltTraits<true> { using T = uint16_t; };
template <> struct EltTraits<false> { using T = float; };

template <bool kBf16, int D>
struct alignas(16) WaveLds {
  using T = typename EltTraits<kBf16>::T;
  // Row pitch of the per-wave V tile: 16 extra bytes put the 4 row groups
  // read by one instruction into disjoint LDS bank ranges.
  static constexpr int kPitch = D + 16 / (int)sizeof(T);
  T v[kWaves][kNPad * kPitch];
  float table[kWaves][kTableMax];
};

template <bool kBf16, int D, bool kExplicit>
__global__ __launch_bounds__(kThreads) void window_attn_wave_kernel(const AttnParams p) {
  using T = typename EltTraits<kBf16>::T;
  using L = WaveLds<kBf16, D>;
  __shared__ L lds;
  constexpr int kPitch = L::kPitch;

  // The wave index is uniform across the wave; saying so keeps the item,
  // window, head and base pointers in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;

  const int item_raw = blockIdx.x * kWaves + wave;
  const bool live = item_raw < p.items;
  const int item = live ? item_raw : p.items - 1;
  const int w = item / p.heads;
  const int h = item - w * p.heads;
  const int N = p.N;

  const T* qw = reinterpret_cast<const T*>(p.q) + (int64_t)w * N * p.q_stride + (int64_t)h * D;
  const T* kw = reinterpret_cast<const T*>(p.k) + (int64_t)w * N * p.k_stride + (int64_t)h * D;
  const T* vw = reinterpret_cast<const T*>(p.v) + (int64_t)w * N * p.v_stride + (int64_t)h * D;

  // Bias-table column of head h (L2-resident; 4 loads per lane cover 256 >= 225).
  float tabv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = lane + 64 * u;
    tabv[u] = (p.bias_table != nullptr && e < p.table_size) ? p.bias_table[(int64_t)e * p.heads + h] : 0.f;
  }
  // K and Q fragments straight from global memory.
  constexpr int kKF = kBf16 ? D / 32 : D / 16;
  uint4 kf[4][kKF];
  uint4 qf[4][kKF];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 16 * t + c16;
#pragma unroll
    for (int s = 0; s < kKF; ++s) {
      const int col = kBf16 ? 32 * s + 8 * g : g * (D / 4) + 4 * s;
      kf[t][s] = row < N ? *reinterpret_cast<const uint4*>(kw + (int64_t)row * p.k_stride + col) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 16 * t + c16;
#pragma unroll
    for (int s = 0; s < kKF; ++s) {
      const int col = kBf16 ? 32 * s + 8 * g : g * (D / 4) + 4 * s;
      qf[t][s] = row < N ? *reinterpret_cast<const uint4*>(qw + (int64_t)row * p.q_stride + col) : make_uint4(0, 0, 0, 0);
    }
  }
  // V tile as 16-byte chunks (rows beyond N are zero).
  constexpr int kChunksPerRow = D * (int)sizeof(T) / 16;
  constexpr int kVLoads = kNPad * kChunksPerRow / 64;
  uint4 vr[kVLoads];
#pragma unroll
  for (int u = 0; u < kVLoads; ++u) {
    const int chunk = lane + 64 * u;
    const int row = chunk / kChunksPerRow;
    const int col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
    vr[u] = row < N ? *reinterpret_cast<const uint4*>(vw + (int64_t)row * p.v_stride + col) : make_uint4(0, 0, 0, 0);
  }

  const WindowMaskState m = window_mask_state(p, w, !kExplicit);

  // Stage the bias column (x log2e) and V in this wave's LDS.
  float* tab = lds.table[wave];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = lane + 64 * u;
    if (e < kTableMax) tab[e] = tabv[u] * kLog2e;
  }
  T* vt = lds.v[wave];
#pragma unroll
  for (int u = 0; u < kVLoads; ++u) {
    const int chunk = lane + 64 * u;
    const int row = chunk / kChunksPerRow;
    const int col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
    *reinterpret_cast<uint4*>(vt + row * kPitch + col) = vr[u];
  }
  // Order this wave's LDS writes before its later LDS reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  LaneGeom<false> lg;
  lane_geom_init<false>(lg, p, m, tab, lane);
  const float* emask = nullptr;
  if constexpr (kExplicit) emask = p.explicit_mask + (int64_t)(w % p.mask_windows) * p.n_geo * p.n_geo;
  // V^T source: bf16 fragments gathered element by element from the padded
  // row-major tile; fp32 element reads.
  auto vsrc = [&](int a, int b) {
    if constexpr (kBf16) {
      uint16_t bits[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) bits[e] = vt[(32 * b + 16 * (e >> 2) + 4 * g + (e & 3)) * kPitch + 16 * a + c16];
      return __builtin_bit_cast(bf16x8, bits);
    } else {
      return vt[a * kPitch + b];
    }
  };

  T* ow = reinterpret_cast<T*>(p.o) + (int64_t)w * N * p.o_stride + (int64_t)h * D;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    f32x4 s[2][4];
    const uint4 (&qp)[2][kKF] = *reinterpret_cast<const uint4(*)[2][kKF]>(&qf[2 * half]);
    scores_pair<kBf16, D>(s, kf, qp);
    float inv[2];
    softmax_half<false, kExplicit>(s, inv, half, p, m, lg, emask, lane);
    f32x4 o[D / 16][2];
    pv_half<kBf16, D>(o, s, lane, vsrc);
    // Store: lane holds O[i = 16*it + c16][16*ct + 4g .. +4].
    if (live) {
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        const int i = 16 * (2 * half + il) + c16;
        if (i < N) {
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) {
            T* dst = ow + (int64_t)i * p.o_stride + 16 * ct + 4 * g;
            const f32x4 v = o[ct][il] * inv[il];
            if constexpr (kBf16) {
              uint2 pk;
              pk.x = pack_bf16x2(v[0], v[1]);
              pk.y = pack_bf16x2(v[2], v[3]);
              *reinterpret_cast<uint2*>(dst) = pk;
            } else {
              *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            }
          }
        }
      }
    }
  }
}

template <bool kBf16, int D, bool kExplicit>
void launch_wave(const AttnParams& p, hipStream_t s) {
  const int blocks = (p.items + kWaves - 1) / kWaves;
  window_attn_wave_kernel<kBf16, D, kExplicit><<<blocks, kThreads, 0, s>>>(p);
}

// Resident workgroups of the persistent tile kernel: as many as the device's
// CUs hold at once (LDS and VGPR limited), queried per device once.
template <int D, int G>
int tile_grid(int lds) {
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, window_attn_tile_kernel<D, G>, G * 128, lds) !=
        hipSuccess)
      return 0;
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  return cache[dev];
}

template <int D, int G>
int launch_tile(const AttnParams& p, hipStream_t s) {
  constexpr int lds = 3 * kNPad * G * D * 2 + G * kTableMax * (int)sizeof(float);
  // The >64 KiB dynamic-LDS opt-in is a per-kernel attribute: set it once.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&window_attn_tile_kernel<D, G>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  const int resident = tile_grid<D, G>(lds);
  if (resident <= 0) return fail(TERRA_ERR_LAUNCH, "cannot size the tile kernel grid for this device");
  const int units = (p.items / p.heads) * p.groups;
  const int blocks = units < resident ? units : resident;
  window_attn_tile_kernel<D, G><<<blocks, G * 128, lds, s>>>(p);
  return TERRA_OK;
}

// Heads per workgroup of the tile kernel: the smallest divisor G of `heads`
// among the instantiated group widths whose row slice is a whole number of
// 128-byte lines (128, 256 or 384 bytes); 0 if there is none.  Small groups
// mean small workgroups (2*G waves, ~26 KB of LDS for G*D = 64), so three
// independent pipelines share a CU and their load and compute phases
// interleave (c3: 145 us with G = 2 against 166 us with G = 6).
int tile_group(int heads, int D) {
  static const int kG32[] = {2, 4, 6};  // head dim 32
  static const int kG64[] = {1, 2, 3};  // head dim 64
  const int* cand = D == 32 ? kG32 : kG64;
  for (int i = 0; i < 3; ++i)
    if (heads % cand[i] == 0) return cand[i];
  return 0;
}

int dispatch_tile(const AttnParams& p, int D, hipStream_t s) {
  if (D == 32) {
    switch (p.group) {
      case 6: return launch_tile<32, 6>(p, s);
      case 4: return launch_tile<32, 4>(p, s);
      default: return launch_tile<32, 2>(p, s);
    }
  }
  switch (p.group) {
    case 3: return launch_tile<64, 3>(p, s);
    case 2: return launch_tile<64, 2>(p, s);
    default: return launch_tile<64, 1>(p, s);
  }
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
  p.scale_l2e = d.scale * kLog2e;
  p.mask_l2e = d.mask_value * kLog2e;
  p.pad_key_l2e = d.pad_key_value * kLog2e;
  p.mask_mode = d.mask_mode; p.mask_windows = d.mask_windows > 0 ? d.mask_windows : 1;
  p.frame_h = d.frame_h; p.frame_w = d.frame_w; p.shift_h = d.shift_h; p.shift_w = d.shift_w;
  p.win_row_begin = d.win_row_begin; p.win_rows = d.win_rows; p.win_cols = d.win_cols;

  hipStream_t s = (hipStream_t)stream;
  // bf16 8x8 windows without padded tokens or a dense mask: window-tile kernel.
  const int G = tile_group(d.heads, D);
  const bool tile = dtype == TERRA_DTYPE_BF16 && d.window_h == 8 && d.window_w == 8 && d.tokens == 64 &&
                    d.n_real == 64 && d.mask_mode != TERRA_MASK_EXPLICIT && G > 0;
  if (tile) {
    p.group = G;
    p.groups = d.heads / G;
    const int st = dispatch_tile(p, D, s);
    if (st != TERRA_OK) return st;
  } else {
    p.group = p.groups = 0;
    const bool expl = d.mask_mode == TERRA_MASK_EXPLICIT;
    if (dtype == TERRA_DTYPE_BF16) {
      if (D == 32) expl ? launch_wave<true, 32, true>(p, s) : launch_wave<true, 32, false>(p, s);
      else expl ? launch_wave<true, 64, true>(p, s) : launch_wave<true, 64, false>(p, s);
    } else {
      if (D == 32) expl ? launch_wave<false, 32, true>(p, s) : launch_wave<false, 32, false>(p, s);
      else expl ? launch_wave<false, 64, true>(p, s) : launch_wave<false, 64, false>(p, s);
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
