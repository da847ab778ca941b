// Fused per-window multi-head attention forward for gfx950.
//
// One wavefront computes one (window, head) item.  With the window padded to
// 64 tokens (4 tiles of 16) and head dim D:
//
//   S^T = K Q^T      v_mfma_f32_16x16x32_bf16 (bf16) / 16x16x4_f32 (fp32).
//                    Both operands come straight from global memory: lane
//                    (c, g) of a 16-row tile loads row 16t + c, channels
//                    [8g, 8g + 8) of a 32-channel step as one 16-byte load.
//   softmax          fp32, in the log2 domain: y = s*scale*log2e + bias*log2e
//                    (+ mask*log2e), p = exp2(y - max).  A query row lives in
//                    4 lanes x 16 registers: in-lane reduction + 2 shuffles.
//   O^T = V^T P^T    P^T comes out of the S^T accumulators already in MFMA
//                    operand order; V is staged in LDS (row-major, padded
//                    pitch) and read as the transposed operand.  1/sum is
//                    applied to O, not to P.
//
// Accumulator layout of a 16x16 tile (lane l, g = l/16, c = l%16): element
// (row 4g + r, col c), r = 0..3.  In S^T rows are keys and columns queries,
// so lane l holds queries i = 16*it + c and keys j = 16*jt + 4g + r.
//
// The query tiles are processed in two halves (it = 0,1 then 2,3) so that at
// most 32 score registers are live; the wave stays within 128 VGPRs (4 waves
// per SIMD).
//
// kWs8 specialises 8x8 windows (N = 64): the relative-position index of lane
// element (it, jt, r) is lane_base + 30*(it - jt) - r, so the bias comes from
// LDS with compile-time offsets and no index arithmetic.  Other windows
// (N <= 64, any Wh x Ww <= 8 x 8, padded tokens) take the generic path.
#include "common.h"

#include <math.h>

namespace terra {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
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
  // Row pitch of the per-wave V tile: 16 extra bytes put the 4 row groups
  // read by one instruction into disjoint LDS bank ranges.
  static constexpr int kPitch = D + 16 / (int)sizeof(T);
  T v[kWaves][kNPad * kPitch];
  float table[kWaves][kTableMax];
};

// Orders this wave's LDS writes before its later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float xor_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

__device__ __forceinline__ float xor_sum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

template <bool kBf16, int D, bool kWs8, bool kExplicit>
__global__ __launch_bounds__(kThreads) void window_attn_kernel(const AttnParams p) {
  using T = typename EltTraits<kBf16>::T;
  using L = LdsLayout<kBf16, D>;
  __shared__ L lds;
  constexpr int kPitch = L::kPitch;
  static_assert(!kWs8 || kBf16, "the 8x8 specialisation is the bf16 path");

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
  const int N = kWs8 ? 64 : p.N;

  const T* qw = reinterpret_cast<const T*>(p.q) + (int64_t)w * N * p.q_stride + (int64_t)h * D;
  const T* kw = reinterpret_cast<const T*>(p.k) + (int64_t)w * N * p.k_stride + (int64_t)h * D;
  const T* vw = reinterpret_cast<const T*>(p.v) + (int64_t)w * N * p.v_stride + (int64_t)h * D;

  // ---- global loads --------------------------------------------------------
  // Bias-table column of head h (L2-resident; 4 loads per lane cover 256 >= 225).
  float tabv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = lane + 64 * u;
    tabv[u] = (p.bias_table != nullptr && e < p.table_size) ? p.bias_table[(int64_t)e * p.heads + h] : 0.f;
  }
  // K and Q fragments.  bf16: one 16-byte load per 32-channel step.  fp32:
  // lane holds channels [g*D/4, (g+1)*D/4), the k order being permuted the
  // same way in both operands (the dot products are unchanged).
  constexpr int kKF = kBf16 ? D / 32 : D / 16;
  uint4 kf[4][kKF];
  uint4 qf[4][kKF];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 16 * t + c16;
    const bool ok = kWs8 || row < N;
#pragma unroll
    for (int s = 0; s < kKF; ++s) {
      const int col = kBf16 ? 32 * s + 8 * g : g * (D / 4) + 4 * s;
      kf[t][s] = ok ? *reinterpret_cast<const uint4*>(kw + (int64_t)row * p.k_stride + col) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 16 * t + c16;
    const bool ok = kWs8 || row < N;
#pragma unroll
    for (int s = 0; s < kKF; ++s) {
      const int col = kBf16 ? 32 * s + 8 * g : g * (D / 4) + 4 * s;
      qf[t][s] = ok ? *reinterpret_cast<const uint4*>(qw + (int64_t)row * p.q_stride + col) : make_uint4(0, 0, 0, 0);
    }
  }
  // V tile as 16-byte chunks.
  constexpr int kChunksPerRow = D * (int)sizeof(T) / 16;
  constexpr int kVLoads = kNPad * kChunksPerRow / 64;
  uint4 vr[kVLoads];
#pragma unroll
  for (int u = 0; u < kVLoads; ++u) {
    const int chunk = lane + 64 * u;
    const int row = chunk / kChunksPerRow;
    const int col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
    vr[u] = (kWs8 || row < N) ? *reinterpret_cast<const uint4*>(vw + (int64_t)row * p.v_stride + col)
                              : make_uint4(0, 0, 0, 0);
  }

  // ---- per-window mask state (wave-uniform) ---------------------------------
  bool use_shift = false;
  int wr = 0, wc = 0;
  if (!kExplicit && p.mask_mode == TERRA_MASK_SHIFT) {
    const int per_img = p.win_rows * p.win_cols;
    const int wl = w % per_img;
    const int rr = wl / p.win_cols;
    wr = rr + p.win_row_begin;
    wc = wl - rr * p.win_cols;
    use_shift = (wr + 2) * p.window_h > p.frame_h || (wc + 2) * p.window_w > p.frame_w;
  }
  const uint64_t land = p.land_bits != nullptr ? p.land_bits[w % p.mask_windows] : 0ull;
  const bool use_mask = use_shift || land != 0ull;

  // ---- per-lane token geometry ----------------------------------------------
  // Generic path: lane t computes token t's bias-index terms and region id;
  // other lanes fetch them with shuffles.  idx(i, j) = base(i) - off(j).
  int g_base = 0, g_off = 0, g_rid = 0;
  if constexpr (!kWs8) {
    const int t = lane < p.n_geo ? lane : p.n_geo - 1;
    const int ti = t / p.window_w;
    const int tj = t - ti * p.window_w;
    const int rel_w = 2 * p.window_w - 1;
    g_base = (ti + p.window_h - 1) * rel_w + tj + p.window_w - 1;
    g_off = ti * rel_w + tj;
    if (use_shift)
      g_rid = 3 * region(wr * p.window_h + ti, p.frame_h, p.window_h, p.shift_h) +
              region(wc * p.window_w + tj, p.frame_w, p.window_w, p.shift_w);
  }
  // Key-side terms, lane (c, g) holding keys j = 16*jt + 4g + r:
  //   rid_pack  4-bit region id of key (jt, r) at bit 4*(4*jt + r)
  //   land_lane land bit of key (jt, r) at bit 16*jt + r
  int off_j[kWs8 ? 1 : 4][4];  // generic path: bias offset of key (jt, r)
  uint64_t rid_pack = 0;
  const uint64_t land_lane = land >> (4 * g);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jt + 4 * g + r;
      int rid;
      if constexpr (kWs8) {
        rid = use_shift ? 3 * region(wr * 8 + 2 * jt + (g >> 1), p.frame_h, 8, p.shift_h) +
                              region(wc * 8 + 4 * (g & 1) + r, p.frame_w, 8, p.shift_w)
                        : 0;
      } else {
        const int jg = j < p.n_geo ? j : p.n_geo - 1;
        off_j[jt][r] = __shfl(g_off, jg);
        rid = __shfl(g_rid, jg);
      }
      rid_pack |= (uint64_t)rid << (4 * (4 * jt + r));
    }
  }

  // ---- stage bias column (x log2e) and V in this wave's LDS -----------------
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
  wave_lds_sync();

  constexpr int kCT = D / 16;

  // ws = 8: lane part of the relative-position index (see header comment).
  const int lane_base8 = 15 * ((c16 >> 3) - (g >> 1) + 7) + (c16 & 7) - 4 * (g & 1) + 7;
  const float* tab8 = tab + (lane_base8 - 93);  // offsets 30*(it-jt) - r + 93 lie in [0, 183]

  T* ow = reinterpret_cast<T*>(p.o) + (int64_t)w * N * p.o_stride + (int64_t)h * D;
  const float* emask = nullptr;
  if constexpr (kExplicit) emask = p.explicit_mask + (int64_t)(w % p.mask_windows) * p.n_geo * p.n_geo;

#pragma unroll
  for (int half = 0; half < 2; ++half) {
    // ---- S^T tiles of queries it = 2*half, 2*half + 1 -----------------------
    f32x4 s[2][4];
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int it = 2 * half + il;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if constexpr (kBf16) {
#pragma unroll
          for (int ks = 0; ks < kKF; ++ks)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[jt][ks]),
                                                          __builtin_bit_cast(bf16x8, qf[it][ks]), acc, 0, 0, 0);
        } else {
#pragma unroll
          for (int ks = 0; ks < kKF; ++ks) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = __uint_as_float(reinterpret_cast<const uint32_t*>(&kf[jt][ks])[e]);
              const float b = __uint_as_float(reinterpret_cast<const uint32_t*>(&qf[it][ks])[e]);
              acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
            }
          }
        }
        s[il][jt] = acc;
      }
    }

    // ---- logits (log2 domain) ----------------------------------------------
    // Pass 1, branch-free: y = s * scale * log2e + bias * log2e.
    int base_i[2] = {0, 0}, rid_i[2] = {0, 0};
    bool i_geo[2] = {true, true};
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int it = 2 * half + il;
      const int i = 16 * it + c16;
      if constexpr (kWs8) {
        if (use_shift)
          rid_i[il] = 3 * region(wr * 8 + 2 * it + (c16 >> 3), p.frame_h, 8, p.shift_h) +
                      region(wc * 8 + (c16 & 7), p.frame_w, 8, p.shift_w);
      } else {
        const int ig = i < p.n_geo ? i : p.n_geo - 1;
        i_geo[il] = i < p.n_geo;
        base_i[il] = __shfl(g_base, ig);
        rid_i[il] = __shfl(g_rid, ig);
      }
    }
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int it = 2 * half + il;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float b;
          if constexpr (kWs8) {
            b = tab8[30 * (it - jt) - r + 93];
          } else {
            const int j = 16 * jt + 4 * g + r;
            b = tab[base_i[il] - off_j[jt][r]];  // clamped indices: always in range
            b = (i_geo[il] && j < p.n_geo) ? b : 0.f;
          }
          s[il][jt][r] = __builtin_fmaf(s[il][jt][r], p.scale_l2e, b);
        }
      }
    }
    // Pass 2 (windows with a shift boundary or land keys only): + mask.
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
            const float m = emask[ig * p.n_geo + jg] * kLog2e;
            const bool land_j = (land_lane >> (16 * jt + r)) & 1ull;
            const bool jin = kWs8 || j < p.n_geo;
            s[il][jt][r] += ((i_geo[il] && jin) ? m : 0.f) + ((land_j && jin) ? p.mask_l2e : 0.f);
          }
        }
      }
    } else if (use_mask) {
#pragma unroll
      for (int il = 0; il < 2; ++il) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = 16 * jt + 4 * g + r;
            const int rid_j = (int)((rid_pack >> (4 * (4 * jt + r))) & 15ull);
            const bool land_j = ((land_lane >> (16 * jt + r)) & 1ull) && (kWs8 || j < p.n_geo);
            const float ms = (i_geo[il] && rid_i[il] != rid_j) ? p.mask_l2e : 0.f;
            s[il][jt][r] += ms + (land_j ? p.mask_l2e : 0.f);
          }
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
            s[il][jt][r] = j >= N ? -INFINITY : y;
          }
    }

    // ---- row softmax: max, exp2, sum ------------------------------------------
    float inv[2];
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

    // ---- O^T = V^T P^T for this half ----------------------------------------
    f32x4 o[kCT][2];
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
      for (int il = 0; il < 2; ++il) o[ct][il] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kBf16) {
#pragma unroll
      for (int js = 0; js < 2; ++js) {
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
          // V^T operand fragment from LDS: k-slot e of lane group g is key
          // 32*js + 16*(e/4) + 4g + e%4, the order of the P^T fragment.
          uint16_t bits[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int j = 32 * js + 16 * (e >> 2) + 4 * g + (e & 3);
            bits[e] = vt[j * kPitch + 16 * ct + c16];
          }
          const bf16x8 vfrag = __builtin_bit_cast(bf16x8, bits);
#pragma unroll
          for (int il = 0; il < 2; ++il)
            o[ct][il] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag, pf[il], o[ct][il], 0, 0, 0);
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
            for (int il = 0; il < 2; ++il)
              o[ct][il] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s[il][jt][r], o[ct][il], 0, 0, 0);
          }
        }
      }
    }

    // ---- store: lane holds O[i = 16*it + c16][16*ct + 4g .. +4] -------------
    if (live) {
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        const int i = 16 * (2 * half + il) + c16;
        if (kWs8 || i < N) {
#pragma unroll
          for (int ct = 0; ct < kCT; ++ct) {
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

template <bool kBf16, int D, bool kWs8, bool kExplicit>
void launch(const AttnParams& p, hipStream_t s) {
  const int blocks = (p.items + kWaves - 1) / kWaves;
  window_attn_kernel<kBf16, D, kWs8, kExplicit><<<blocks, kThreads, 0, s>>>(p);
}

template <bool kBf16, int D>
void dispatch(const AttnParams& p, bool ws8, bool expl, hipStream_t s) {
  if constexpr (kBf16) {
    if (ws8 && !expl) return launch<true, D, true, false>(p, s);
    if (ws8 && expl) return launch<true, D, true, true>(p, s);
  }
  if (expl) launch<kBf16, D, false, true>(p, s);
  else launch<kBf16, D, false, false>(p, s);
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

  // 8x8 windows without padded tokens take the closed-form bias path.
  const bool ws8 = dtype == TERRA_DTYPE_BF16 && d.window_h == 8 && d.window_w == 8 && d.tokens == 64 &&
                   d.n_real == 64;
  const bool expl = d.mask_mode == TERRA_MASK_EXPLICIT;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TERRA_DTYPE_BF16) {
    if (D == 32) dispatch<true, 32>(p, ws8, expl, s);
    else dispatch<true, 64>(p, ws8, expl, s);
  } else {
    if (D == 32) dispatch<false, 32>(p, false, expl, s);
    else dispatch<false, 64>(p, false, expl, s);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
