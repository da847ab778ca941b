// Backward of the window-attention core (bf16, windows up to 8x8 in rows of
// up to 64 tokens, head dim 32/64/128).
//
// Per window w and head h, with z = (q k^T) * scale + bias + M the natural
// logits and P = softmax(z) (recomputed here from q, k and the masks, the
// same way the forward computes it):
//
//   dP  = dO V^T
//   dz  = P * (dP - rowsum(P * dP))        (rowsum(P * dP) = rowsum(dO * O))
//   dV  = P^T dO,   dQ = scale * dz K,   dK = scale * dz^T Q
//   dbias[idx(i, j), h] += sum over windows of dz[i, j]
//
// One workgroup per (window, head group), persistent, with a fixed head group
// per workgroup (the grid is a multiple of the number of head groups), so
// each lane keeps its share of the bias gradient in registers across all its
// windows and flushes it once.  Two waves per head:
//   phase 1 (wave = query tiles 2*half, 2*half + 1): S^T and dP^T on MFMA in
//     the forward's layout (lane = one query, 16 keys), softmax, dz; P and dz
//     go to LDS as [query][key] bf16 tiles; dQ^T = K^T dz^T straight from the
//     dz accumulators (the forward's P^T-operand trick).
//   phase 2 (wave = keys [32*half, 32*half + 32)): dV^T = dO^T P and
//     dK^T = Q^T dz with both operands read across rows of the LDS tiles
//     (transposing LDS reads), contraction over all 64 queries.
// dQ, dK and dV are staged in the V, K and dout tiles once those are dead and
// leave as whole 128-byte row slices (8-byte accumulator stores straight to
// memory made the kernel twice as slow).
//
// Windows other than 8x8 in 64-token rows (7x7: 49 tokens) run the same
// tiles with rows N..63 zero-filled: their keys take -inf (P = 0, dz = 0),
// their dout rows are zero (dz = 0 for those query rows), and they are never
// stored.  Keys >= n_real take the pad value in the softmax and get no
// gradient (the forward's masked_fill).
#include "common.h"
#include "attn_core.h"

namespace terra {
namespace {

struct BwdParams {
  AttnParams a;         // forward call; a.o / a.o_stride carry dout
  void* dq;
  void* dk;
  void* dv;
  int64_t dq_stride, dk_stride, dv_stride;
  float* dbias;         // fp32 [table_size, heads], accumulated; NULL: not wanted
  float* dsum[3];       // fp32 [C] column sums of dq, dk, dv, accumulated; NULL: not wanted
  float scale;          // natural q k^T scale
  float mask_value;     // natural-unit mask and padded-key values (generic kernel)
  float pad_key_value;
};

constexpr int kBwdTile = kNPad * 8 * 16;  // one [64][64] bf16 P or dz tile: 8 KB

// Slot of chunk `chunk` of row `row` in a [64][8]-chunk P or dz tile: chunk
// XOR (row & 7).  Those tiles are only written by 8-byte stores and read by
// transposing reads of 4 consecutive rows per 16 lanes, which the pairwise
// tile_slot swizzle ((row >> 1) & 7) maps onto the same banks two by two.
__device__ __forceinline__ int pz_slot(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

// 16x16x32 bf16 operand fragment read across the rows of a [64][cpr]-chunk
// tile (kPz: a P or dz tile in pz_slot layout, else tile_slot layout): lane
// (c, g) receives column col0 + c at rows 32*js + 16*(e/4) + 4g + e%4 for k
// slot e (col0 a multiple of 16).  As an A operand the column is the output
// row; as a B operand it is the output column.
template <bool kPz>
__device__ __forceinline__ bf16x8 rows_frag(const uint8_t* tile, int cpr, int col0, int js, int lane) {
  const int g = lane >> 4, c16 = lane & 15;
  const int cc = col0 + 4 * (c16 & 3);  // column addressed by this source lane
  uint2 part[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
    const int slot = kPz ? pz_slot(row, cc >> 3) : tile_slot(row, cc >> 3, cpr);
    part[h2] = lds_read_tr16(tile + slot * 16 + (cc & 7) * 2);
  }
  const uint32_t w[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
  return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ uint2 pack4_bf16(const f32x4& v) {
  uint2 r;
  r.x = pack_bf16x2(v[0], v[1]);
  r.y = pack_bf16x2(v[2], v[3]);
  return r;
}

// LDS row pitch of the q / k / v / dout tiles in 16-byte chunks: the
// tile_slot swizzle permutes chunks within aligned groups of 8, so rows
// narrower than 8 chunks (one head of dim 32) are padded to 8.
constexpr int bwd_tile_cpr(int G, int D) { return G * D / 8 < 8 ? 8 : G * D / 8; }

template <int D, int G, bool kExplicit, bool kWs8>
__global__ __launch_bounds__(G * 128) void window_attn_bwd_kernel(const BwdParams bp) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const AttnParams& p = bp.a;
  constexpr int nthreads = G * 128;
  constexpr int cpr = G * D / 8;                 // chunks per row of the head group
  constexpr int lcpr = bwd_tile_cpr(G, D);       // LDS row pitch in chunks
  constexpr int tile_bytes = kNPad * lcpr * 16;
  static_assert(lcpr % 8 == 0, "LDS rows must be whole groups of 8 chunks (swizzle)");
  constexpr int kKF = D / 32;
  uint8_t* qs = smem;
  uint8_t* ks = smem + tile_bytes;
  uint8_t* vs = smem + 2 * tile_bytes;
  uint8_t* dos = smem + 3 * tile_bytes;
  uint8_t* pz = smem + 4 * tile_bytes;           // per head: P tile, then dz tile
  float* tables = reinterpret_cast<float*>(pz + 2 * G * kBwdTile);  // G bias columns (x log2e)
  float* dtab = tables + G * kTableMax;          // G bias-gradient columns
  float* csum = dtab + G * kTableMax;            // column sums of dq | dk | dv (G * D each)
  const bool sums = bp.dsum[0] != nullptr || bp.dsum[1] != nullptr || bp.dsum[2] != nullptr;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = wave >> 1;
  const int half = wave & 1;
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int units = (p.items / p.heads) * p.groups;
  const int hg = blockIdx.x % p.groups;          // fixed: gridDim.x is a multiple of groups
  const int h = hg * G + head;
  uint8_t* ptile = pz + head * 2 * kBwdTile;
  uint8_t* ztile = ptile + kBwdTile;

  // Bias column of this head (x log2e, for the softmax) and a zeroed
  // gradient column.
  float* tab = tables + head * kTableMax;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = lane + 64 * (2 * u + half);
    if (e < kTableMax) {
      tab[e] = (p.bias_table != nullptr && e < p.table_size) ? p.bias_table[(int64_t)e * p.heads + h] * kLog2e : 0.f;
      dtab[head * kTableMax + e] = 0.f;
    }
  }
  for (int e = tid; e < 3 * G * D; e += nthreads) csum[e] = 0.f;  // read after the loop's first barrier

  constexpr int kPer = kNPad * cpr / nthreads;   // chunks per thread per tensor
  constexpr int kRowStep = nthreads / cpr;
  static_assert(kRowStep * cpr == nthreads && kRowStep * kPer == kNPad, "row tiling");
  const int row0 = tid / cpr, chunk0 = tid % cpr;
  const int n_rows = kWs8 ? kNPad : p.N;         // token rows per window in memory

  f32x4 gz[2][4];  // this lane's bias-gradient share: dz summed over the windows
#pragma unroll
  for (int il = 0; il < 2; ++il)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) gz[il][jt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // q, k, v, dout rows of one unit's head group -> registers (nontemporal);
  // rows >= n_rows are zeros.
  uint4 buf[4][kPer];
  auto fetch = [&](int unit) {
    const int64_t row_base = (int64_t)(unit / p.groups) * n_rows + row0;
    const int col = hg * G * D + chunk0 * 8;
    const uint16_t* src[4] = {reinterpret_cast<const uint16_t*>(p.q) + row_base * p.q_stride + col,
                              reinterpret_cast<const uint16_t*>(p.k) + row_base * p.k_stride + col,
                              reinterpret_cast<const uint16_t*>(p.v) + row_base * p.v_stride + col,
                              reinterpret_cast<const uint16_t*>(p.o) + row_base * p.o_stride + col};
    const int64_t step[4] = {kRowStep * p.q_stride, kRowStep * p.k_stride, kRowStep * p.v_stride,
                             kRowStep * p.o_stride};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < kPer; ++u)
        buf[t][u] = (kWs8 || row0 + kRowStep * u < n_rows)
                        ? __builtin_bit_cast(uint4, __builtin_nontemporal_load(
                                                        reinterpret_cast<const u32x4*>(src[t] + u * step[t])))
                        : uint4{0u, 0u, 0u, 0u};
  };

  // Persistent loop, software-pipelined: the loads of unit n + gridDim.x are
  // issued once unit n's phase 1 is done and land during its phase 2.  Head
  // dim 128 loads each unit at its start instead: its 32 chunks per thread
  // held through phase 2 beside the 128 dK / dV accumulator registers would
  // not fit the register file.
  constexpr bool kPrefetch = D <= 64;
  int unit = blockIdx.x;  // < units: the grid is never larger than the work
  if constexpr (kPrefetch) fetch(unit);
  for (;;) {
    const int w = unit / p.groups;
    // ---- q, k, v, dout rows of the head group -> LDS --------------------------
    {
      if constexpr (!kPrefetch) fetch(unit);
      lds_barrier();  // the previous unit is done with every tile
      uint8_t* dst[4] = {qs, ks, vs, dos};
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < kPer; ++u)
          *reinterpret_cast<uint4*>(dst[t] + tile_slot(row0 + kRowStep * u, chunk0, lcpr) * 16) = buf[t][u];
      lds_barrier();
    }

    // ---- phase 1: query tiles 2*half, 2*half + 1 of head `head` ---------------
    const WindowMaskState m = window_mask_state(p, w, true);
    const float* emask = nullptr;
    if constexpr (kExplicit) emask = p.explicit_mask + (int64_t)(w % p.mask_windows) * p.n_geo * p.n_geo;
    LaneGeom<kWs8> lg;
    lane_geom_init<kWs8>(lg, p, m, tab, lane);
    const int hc = head * (D / 8);  // first chunk of this head in the tiles
    f32x4 s[2][4];
    float inv[2];
    {
      uint4 kf[4][kKF], qp[2][kKF];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < kKF; ++c)
          kf[t][c] = *reinterpret_cast<const uint4*>(ks + tile_slot(16 * t + c16, hc + 4 * c + g, lcpr) * 16);
#pragma unroll
      for (int il = 0; il < 2; ++il)
#pragma unroll
        for (int c = 0; c < kKF; ++c)
          qp[il][c] = *reinterpret_cast<const uint4*>(
              qs + tile_slot(16 * (2 * half + il) + c16, hc + 4 * c + g, lcpr) * 16);
      scores_pair<true, D>(s, kf, qp);
    }
    softmax_half<kWs8, kExplicit>(s, inv, half, p, m, lg, emask, lane);
    f32x4 dp[2][4];
    {
      uint4 vf[4][kKF], df[2][kKF];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < kKF; ++c)
          vf[t][c] = *reinterpret_cast<const uint4*>(vs + tile_slot(16 * t + c16, hc + 4 * c + g, lcpr) * 16);
#pragma unroll
      for (int il = 0; il < 2; ++il)
#pragma unroll
        for (int c = 0; c < kKF; ++c)
          df[il][c] = *reinterpret_cast<const uint4*>(
              dos + tile_slot(16 * (2 * half + il) + c16, hc + 4 * c + g, lcpr) * 16);
      scores_pair<true, D>(dp, vf, df);  // dP^T: keys 16jt + 4g + r, query c16
    }
    // P = e * (1 / rowsum); dz = P * (dP - sum_j P dP).  P is rounded to bf16
    // for the tile the dV product reads, as the forward rounds it for P V.
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      float dsum = 0.f;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        s[il][jt] *= inv[il];
#pragma unroll
        for (int r = 0; r < 4; ++r) dsum += s[il][jt][r] * dp[il][jt][r];
      }
      dsum = xor_sum(dsum);
      const int i = 16 * (2 * half + il) + c16;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        f32x4 z = s[il][jt] * (dp[il][jt] - dsum);
        if constexpr (!kWs8) {
#pragma unroll
          for (int r = 0; r < 4; ++r) z[r] = 16 * jt + 4 * g + r < p.n_real ? z[r] : 0.f;
        }
        gz[il][jt] += z;
        // [query][key] tiles: this lane's keys 16jt + 4g .. + 3 are 8 bytes.
        const int off = pz_slot(i, 2 * jt + (g >> 1)) * 16 + (g & 1) * 8;
        *reinterpret_cast<uint2*>(ptile + off) = pack4_bf16(s[il][jt]);
        *reinterpret_cast<uint2*>(ztile + off) = pack4_bf16(z);
        dp[il][jt] = z;
      }
    }
    // dQ^T = K^T dz^T (dz accumulators as the P^T operand), times scale.
    f32x4 dqa[D / 16][2];
    {
      auto kfrag = [&](int ct, int js) -> bf16x8 { return rows_frag<false>(ks, lcpr, head * D + 16 * ct, js, lane); };
      pv_half<true, D>(dqa, dp, lane, kfrag);
    }
    lds_barrier();  // P and dz tiles of both halves are in LDS; K and V are no longer read
    // dQ rows of this wave -> the V tile (lane: 4 channels of query row i).
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int i = 16 * (2 * half + il) + c16;
#pragma unroll
      for (int ct = 0; ct < D / 16; ++ct) {
        const int cc = head * D + 16 * ct + 4 * g;
        *reinterpret_cast<uint2*>(vs + tile_slot(i, cc >> 3, lcpr) * 16 + (cc & 7) * 2) =
            pack4_bf16(dqa[ct][il] * bp.scale);
      }
    }
    const int next = unit + (int)gridDim.x;
    if (kPrefetch && next < units) fetch(next);

    // ---- phase 2: keys [32*half, 32*half + 32) of head `head` -----------------
    // Phase 2 (the dK / dV MFMAs) at raised wave priority, so that a wave of
    // the other workgroup in its softmax fills the gaps (276-279 against
    // 281-283 us at c3, A/B).
    __builtin_amdgcn_s_setprio(1);
    {
      f32x4 av[D / 16][2], ak[D / 16][2];
#pragma unroll
      for (int ct = 0; ct < D / 16; ++ct)
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) av[ct][jt] = ak[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int js = 0; js < 2; ++js) {  // 32 queries per MFMA step
        bf16x8 pf[2], zf[2];
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) {
          pf[jt] = rows_frag<true>(ptile, 8, 32 * half + 16 * jt, js, lane);
          zf[jt] = rows_frag<true>(ztile, 8, 32 * half + 16 * jt, js, lane);
        }
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          const bf16x8 dof = rows_frag<false>(dos, lcpr, head * D + 16 * ct, js, lane);
          const bf16x8 qf = rows_frag<false>(qs, lcpr, head * D + 16 * ct, js, lane);
#pragma unroll
          for (int jt = 0; jt < 2; ++jt) {
            av[ct][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dof, pf[jt], av[ct][jt], 0, 0, 0);
            ak[ct][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf, zf[jt], ak[ct][jt], 0, 0, 0);
          }
        }
      }
      // lane (c16, g) of tile (ct, jt): channels 16ct + 4g .. + 3 of key 32half + 16jt + c16.
      // dK -> the K tile (not read since phase 1); dV -> the dout tile once
      // every wave is done reading it.
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const int j = 32 * half + 16 * jt + c16;
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          const int cc = head * D + 16 * ct + 4 * g;
          *reinterpret_cast<uint2*>(ks + tile_slot(j, cc >> 3, lcpr) * 16 + (cc & 7) * 2) =
              pack4_bf16(ak[ct][jt] * bp.scale);
        }
      }
      lds_barrier();
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const int j = 32 * half + 16 * jt + c16;
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          const int cc = head * D + 16 * ct + 4 * g;
          *reinterpret_cast<uint2*>(dos + tile_slot(j, cc >> 3, lcpr) * 16 + (cc & 7) * 2) = pack4_bf16(av[ct][jt]);
        }
      }
    }
    lds_barrier();
    __builtin_amdgcn_s_setprio(0);
    // ---- dq (V tile), dk (K tile), dv (dout tile) -> memory, whole rows -------
    {
      const int col = hg * G * D + chunk0 * 8;
      const uint8_t* src[3] = {vs, ks, dos};
      void* const dst[3] = {bp.dq, bp.dk, bp.dv};
      const int64_t stride[3] = {bp.dq_stride, bp.dk_stride, bp.dv_stride};
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const uint16_t* base = reinterpret_cast<const uint16_t*>(dst[t]) + (int64_t)w * n_rows * stride[t];
        const __amdgpu_buffer_rsrc_t out =
            buffer_rsrc(base, (uint32_t)(((int64_t)(n_rows - 1) * stride[t] + p.heads * D) * 2));
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int row = row0 + kRowStep * u;
          if (!kWs8 && row >= n_rows) continue;
          const uint4 val = *reinterpret_cast<const uint4*>(src[t] + tile_slot(row, chunk0, lcpr) * 16);
          stream_store_nt(val, out, (uint32_t)(row * stride[t] + col) * 2);
        }
      }
      // The unit's column sums of the bf16 values stored (the q / k / v
      // Linear's bias gradient), as MFMAs of a ones operand with 16-column
      // tiles read across the rows: every output row of ones^T T is the
      // column sum.  Rows the window does not store are zeros in the tiles.
      // Each wave takes whole column tiles, so its 16 sums go to LDS words no
      // other wave adds to in this unit.
      if (sums) {
        constexpr int kColTiles = G * D / 16;
        bf16x8 ones;
#pragma unroll
        for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
        for (int ti = wave; ti < 3 * kColTiles; ti += nthreads / 64) {
          const int t = ti / kColTiles, col0 = 16 * (ti - t * kColTiles);
          if (bp.dsum[t] == nullptr) continue;  // uniform
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int js = 0; js < 2; ++js)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, rows_frag<false>(src[t], lcpr, col0, js, lane), acc,
                                                          0, 0, 0);
          if (g == 0) atomicAdd(&csum[t * G * D + col0 + c16], acc[0]);
        }
      }
    }
    if (next >= units) break;
    unit = next;
  }

  // ---- bias gradient: registers -> LDS column -> global table ----------------
  if (bp.dbias == nullptr && !sums) return;  // uniform
  // Lane element (il, jt, r) is the pair (query 16(2half+il) + c16, key 16jt + 4g + r).
  float* dcol = dtab + head * kTableMax;
  if (bp.dbias == nullptr) {
    // column sums only
  } else if constexpr (kWs8) {
    // relative index lane_base + 30*(it - jt) - r
    const int lane_base = 15 * ((c16 >> 3) - (g >> 1) + 7) + (c16 & 7) - 4 * (g & 1) + 7;
#pragma unroll
    for (int il = 0; il < 2; ++il)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          atomicAdd(dcol + lane_base + 30 * (2 * half + il - jt) - r, gz[il][jt][r]);
  } else {
    // pairs of window tokens only: idx = (hi - hj + wh - 1) (2 ww - 1) + wi - wj + ww - 1
    const int ww = p.window_w, rel = 2 * p.window_w - 1;
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const int i = 16 * (2 * half + il) + c16;
      if (i >= p.n_geo) continue;
      const int base_i = (i / ww + p.window_h - 1) * rel + i % ww + ww - 1;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jt + 4 * g + r;
          if (j < p.n_geo) atomicAdd(dcol + base_i - (j / ww) * rel - j % ww, gz[il][jt][r]);
        }
    }
  }
  lds_barrier();
  if (bp.dbias != nullptr) {
    for (int e = tid; e < G * p.table_size; e += nthreads) {
      const int hh = e / p.table_size, idx = e - hh * p.table_size;
      unsafeAtomicAdd(bp.dbias + (int64_t)idx * p.heads + hg * G + hh, dtab[hh * kTableMax + idx]);
    }
  }
  if (sums) {
    for (int e = tid; e < 3 * G * D; e += nthreads) {
      const int t = e / (G * D);
      if (bp.dsum[t] != nullptr) unsafeAtomicAdd(bp.dsum[t] + hg * G * D + (e - t * G * D), csum[e]);
    }
  }
}

template <int D, int G>
constexpr int bwd_lds_bytes() {
  return 4 * kNPad * bwd_tile_cpr(G, D) * 16 + 2 * G * kBwdTile + 2 * G * kTableMax * (int)sizeof(float) +
         3 * G * D * (int)sizeof(float);
}

template <int D, int G, bool kExplicit, bool kWs8>
int launch_bwd(const BwdParams& bp, hipStream_t s) {
  constexpr int lds = bwd_lds_bytes<D, G>();
  auto kern = window_attn_bwd_kernel<D, G, kExplicit, kWs8>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  constexpr int kMaxDevices = 64;
  static int resident_cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (resident_cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, G * 128, lds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the backward grid for this device");
    resident_cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  const int groups = bp.a.groups;
  const int units = (bp.a.items / bp.a.heads) * groups;
  int blocks = units < resident_cache[dev] ? units : resident_cache[dev];
  blocks -= blocks % groups;  // every workgroup keeps one head group
  if (blocks < groups) blocks = groups;
  kern<<<blocks, G * 128, lds, s>>>(bp);
  return TERRA_OK;
}

template <bool kWs8>
int launch_bwd_tiles(const BwdParams& bp, hipStream_t s, int D, int G, bool expl) {
  if (D == 32)
    return G == 2 ? (expl ? launch_bwd<32, 2, true, kWs8>(bp, s) : launch_bwd<32, 2, false, kWs8>(bp, s))
                  : (expl ? launch_bwd<32, 1, true, kWs8>(bp, s) : launch_bwd<32, 1, false, kWs8>(bp, s));
  if (D == 64) return expl ? launch_bwd<64, 1, true, kWs8>(bp, s) : launch_bwd<64, 1, false, kWs8>(bp, s);
  return expl ? launch_bwd<128, 1, true, kWs8>(bp, s) : launch_bwd<128, 1, false, kWs8>(bp, s);
}

// ============================================================================
// fp32 backward: any window up to 8x8, padded tokens / keys
// ============================================================================
//
// One workgroup per (window, head), plain fp32 arithmetic on LDS copies of
// q, k, v and dout (no MFMA): the shapes it serves (fp32 activations) are
// small configurations.  The logits follow the forward:
// z = q k^T * scale + bias + mask for tokens of the window geometry, keys
// >= n_real replaced by pad_key_value (their gradient is zero: masked_fill),
// keys >= tokens excluded.

// The P and dz tiles overlay the V rows (dead once phase 1 has formed dP)
// where separate tiles would not fit the 160 KB of LDS (D = 128).
template <int D>
constexpr bool generic_bwd_overlay() {
  return (4 * kNPad * (D + 1) + 2 * kNPad * (kNPad + 1) + kTableMax) * (int)sizeof(float) > 160 * 1024;
}

template <int D>
constexpr int generic_bwd_pz_floats() {
  return generic_bwd_overlay<D>() && kNPad * (D + 1) > 2 * kNPad * (kNPad + 1) ? kNPad * (D + 1)
                                                                             : 2 * kNPad * (kNPad + 1);
}

template <int D>
constexpr int generic_bwd_lds_bytes() {
  return ((generic_bwd_overlay<D>() ? 3 : 4) * kNPad * (D + 1) + generic_bwd_pz_floats<D>() + kTableMax) *
         (int)sizeof(float);
}

template <int D, bool kExplicit>
__global__ __launch_bounds__(256) void window_attn_bwd_generic_kernel(const BwdParams bp) {
  extern __shared__ __attribute__((aligned(16))) float smf[];
  const AttnParams& p = bp.a;
  constexpr int PD = D + 1;                     // odd row pitches: conflict-free column walks
  constexpr int PP = kNPad + 1;
  // q, k, v, dout rows, then the P and dz tiles; with the overlay q, k, dout,
  // then V in the region that P and dz take over.
  constexpr bool kOverlay = generic_bwd_overlay<D>();
  float* qs = smf;
  float* ks = qs + kNPad * PD;
  float* vs = ks + (kOverlay ? 2 : 1) * kNPad * PD;
  float* ds = kOverlay ? ks + kNPad * PD : vs + kNPad * PD;  // dout
  float* ps = kOverlay ? vs : ds + kNPad * PD;               // P
  float* zs = ps + kNPad * PP;                               // dz
  float* dtab = ps + generic_bwd_pz_floats<D>();             // this window-head's bias gradient
  const int tid = threadIdx.x;
  const int w = blockIdx.x / p.heads, h = blockIdx.x - (blockIdx.x / p.heads) * p.heads;
  const int N = p.N, ng = p.n_geo, ww = p.window_w, wh = p.window_h;

  auto load_rows = [&](const void* base, int64_t stride, float* dst) {
    for (int e = tid; e < N * D; e += 256) {
      const int r = e / D, c = e - r * D;
      dst[r * PD + c] = reinterpret_cast<const float*>(base)[((int64_t)w * N + r) * stride + h * D + c];
    }
  };
  load_rows(p.q, p.q_stride, qs);
  load_rows(p.k, p.k_stride, ks);
  load_rows(p.v, p.v_stride, vs);
  load_rows(p.o, p.o_stride, ds);
  for (int e = tid; e < kTableMax; e += 256) dtab[e] = 0.f;
  __syncthreads();

  const WindowMaskState m = window_mask_state(p, w, true);
  const float* emask = nullptr;
  if constexpr (kExplicit) emask = p.explicit_mask + (int64_t)(w % p.mask_windows) * ng * ng;
  auto rid = [&](int t) {                       // shift-mask region id of window token t < ng
    const int ti = t / ww, tj = t - (t / ww) * ww;
    return 3 * region(m.wr * wh + ti, p.frame_h, wh, p.shift_h) + region(m.wc * ww + tj, p.frame_w, ww, p.shift_w);
  };

  // Phase 1: four threads per query row i, keys j = jq + 4k.
  const int i = tid >> 2, jq = tid & 3;
  const bool row = i < N;
  const int rid_i = (row && i < ng && m.use_shift) ? rid(i) : 0;
  float z[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int j = jq + 4 * k;
    float val = -INFINITY;
    if (row && j < N) {
      float dot = 0.f;
#pragma unroll 8
      for (int c = 0; c < D; ++c) dot = __builtin_fmaf(qs[i * PD + c], ks[j * PD + c], dot);
      val = dot * bp.scale;
      if (i < ng && j < ng) {
        if (p.bias_table != nullptr) {
          const int hi = i / ww, wi = i - hi * ww, hj = j / ww, wj = j - hj * ww;
          val += p.bias_table[(int64_t)((hi - hj + wh - 1) * (2 * ww - 1) + (wi - wj + ww - 1)) * p.heads + h];
        }
        if constexpr (kExplicit) val += emask[i * ng + j];
        else if (m.use_shift && rid(j) != rid_i) val += bp.mask_value;
      }
      if (j < ng && ((m.land >> j) & 1ull)) val += bp.mask_value;  // land keys, every query row
      if (j >= p.n_real) val = bp.pad_key_value;
    }
    z[k] = val;
  }
  float mx = z[0];
#pragma unroll
  for (int k = 1; k < 16; ++k) mx = max_nan(mx, z[k]);
  mx = max_nan(mx, __shfl_xor(mx, 1));
  mx = max_nan(mx, __shfl_xor(mx, 2));
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    z[k] = z[k] == -INFINITY ? 0.f : expf(z[k] - mx);
    sum += z[k];
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  const float inv = row ? 1.f / sum : 0.f;
  float dp[16], dsum = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int j = jq + 4 * k;
    z[k] *= inv;                                // P
    float acc = 0.f;
    if (row && j < N) {
#pragma unroll 8
      for (int c = 0; c < D; ++c) acc = __builtin_fmaf(ds[i * PD + c], vs[j * PD + c], acc);
    }
    dp[k] = acc;
    dsum = __builtin_fmaf(z[k], acc, dsum);
  }
  dsum += __shfl_xor(dsum, 1);
  dsum += __shfl_xor(dsum, 2);
  if constexpr (kOverlay) __syncthreads();  // every thread has read V: P and dz overwrite it
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int j = jq + 4 * k;
    if (row && j < N) {
      const float dz = j < p.n_real ? z[k] * (dp[k] - dsum) : 0.f;
      ps[i * PP + j] = z[k];
      zs[i * PP + j] = dz;
      if (bp.dbias != nullptr && i < ng && j < ng) {
        const int hi = i / ww, wi = i - hi * ww, hj = j / ww, wj = j - hj * ww;
        atomicAdd(dtab + (hi - hj + wh - 1) * (2 * ww - 1) + (wi - wj + ww - 1), dz);
      }
    }
  }
  __syncthreads();

  // Phase 2: dq[r] = scale * sum_j dz[r][j] k[j],  dk[r] = scale * sum_i dz[i][r] q[i],
  //          dv[r] = sum_i P[i][r] dout[i].
  for (int e = tid; e < N * D; e += 256) {
    const int r = e / D, c = e - r * D;
    float aq = 0.f, ak = 0.f, av = 0.f;
    for (int t = 0; t < N; ++t) {
      aq = __builtin_fmaf(zs[r * PP + t], ks[t * PD + c], aq);
      ak = __builtin_fmaf(zs[t * PP + r], qs[t * PD + c], ak);
      av = __builtin_fmaf(ps[t * PP + r], ds[t * PD + c], av);
    }
    const int64_t row_g = (int64_t)w * N + r;
    reinterpret_cast<float*>(bp.dq)[row_g * bp.dq_stride + h * D + c] = aq * bp.scale;
    reinterpret_cast<float*>(bp.dk)[row_g * bp.dk_stride + h * D + c] = ak * bp.scale;
    reinterpret_cast<float*>(bp.dv)[row_g * bp.dv_stride + h * D + c] = av;
  }
  if (bp.dbias == nullptr) return;  // uniform
  __syncthreads();
  for (int e = tid; e < p.table_size; e += 256) {
    const float v = dtab[e];
    if (v != 0.f) unsafeAtomicAdd(bp.dbias + (int64_t)e * p.heads + h, v);
  }
}

template <int D, bool kExplicit>
int launch_bwd_generic(const BwdParams& bp, hipStream_t s) {
  constexpr int lds = generic_bwd_lds_bytes<D>();
  auto kern = window_attn_bwd_generic_kernel<D, kExplicit>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  kern<<<bp.a.items, 256, lds, s>>>(bp);
  return TERRA_OK;
}

}  // namespace
}  // namespace terra

using namespace terra;

namespace {

// terra_swin_attn_bwd, with the column sums of dq / dk / dv (dsum[t], C
// floats each, accumulated; NULL: not wanted) from the bf16 tile kernel.
int attn_bwd_impl(const void* q, const void* k, const void* v, const void* dout, void* dq, void* dk, void* dv,
                  int dtype, const terra_swin_attn_bwd_desc* desc, const float* bias_table, float* dbias_table,
                  const float* explicit_mask, const uint64_t* land_bits, float* const dsum[3], void* stream) {
  const bool sums = dsum[0] != nullptr || dsum[1] != nullptr || dsum[2] != nullptr;
  for (int t = 0; t < 3; ++t)
    if (((uintptr_t)dsum[t] & 3u) != 0) return fail(TERRA_ERR_ALIGN, "column sums must be 4-byte aligned");
  if (desc == nullptr) return fail(TERRA_ERR_NULL, "desc is NULL");
  if (q == nullptr || k == nullptr || v == nullptr || dout == nullptr || dq == nullptr || dk == nullptr ||
      dv == nullptr)
    return fail(TERRA_ERR_NULL, "q, k, v, dout, dq, dk and dv must be non-NULL");
  if (dtype != TERRA_DTYPE_BF16 && dtype != TERRA_DTYPE_F32)
    return fail(TERRA_ERR_DTYPE, "attention backward supports bf16 and f32 activations (got dtype %d)", dtype);
  const terra_swin_attn_desc& d = desc->fwd;
  if (d.num_windows <= 0 || d.tokens <= 0 || d.heads <= 0 || d.channels <= 0)
    return fail(TERRA_ERR_SHAPE, "num_windows/tokens/channels/heads must be positive");
  if (sums && (dtype != TERRA_DTYPE_BF16 || d.tokens > kNPad))
    return fail(TERRA_ERR_UNSUPPORTED,
                "column sums of dq / dk / dv come from the bf16 kernel for windows of at most %d tokens", kNPad);
  if (d.tokens > kNPad)
    return flash_attention_backward(q, k, v, dout, dq, dk, dv, dtype, desc, bias_table, dbias_table, explicit_mask,
                                    land_bits, stream);
  if (d.window_h <= 0 || d.window_w <= 0 || d.window_h > 8 || d.window_w > 8)
    return fail(TERRA_ERR_UNSUPPORTED, "window %dx%d outside 1..8", d.window_h, d.window_w);
  if (d.window_h * d.window_w > d.tokens)
    return fail(TERRA_ERR_SHAPE, "window %dx%d has more than %d tokens", d.window_h, d.window_w, d.tokens);
  if (d.n_real <= 0 || d.n_real > d.tokens) return fail(TERRA_ERR_SHAPE, "n_real %d outside [1, %d]", d.n_real, d.tokens);
  if (d.channels % d.heads != 0)
    return fail(TERRA_ERR_SHAPE, "channels %d not divisible by heads %d", d.channels, d.heads);
  const int D = d.channels / d.heads;
  if (D != 32 && D != 64 && D != 128) return fail(TERRA_ERR_UNSUPPORTED, "head dim %d not in {32, 64, 128}", D);
  const int elt = dtype == TERRA_DTYPE_BF16 ? 2 : 4;
  const int32_t strides[7] = {d.q_stride, d.k_stride, d.v_stride, desc->dout_stride,
                              desc->dq_stride, desc->dk_stride, desc->dv_stride};
  for (int i = 0; i < 7; ++i) {
    if (strides[i] < d.channels) return fail(TERRA_ERR_SHAPE, "row strides must be >= channels");
    if (strides[i] % (16 / elt) != 0)
      return fail(TERRA_ERR_ALIGN, "row strides must be multiples of %d elements", 16 / elt);
    if ((int64_t)strides[i] * d.tokens * elt >= (1ll << 32))
      return fail(TERRA_ERR_SHAPE, "one window must span under 4 GiB");
  }
  for (const void* ptr : {q, k, v, dout, (const void*)dq, (const void*)dk, (const void*)dv})
    if ((uintptr_t)ptr % 16 != 0) return fail(TERRA_ERR_ALIGN, "q/k/v/dout/dq/dk/dv must be 16-byte aligned");
  if ((bias_table != nullptr && (uintptr_t)bias_table % 4 != 0) ||
      (dbias_table != nullptr && (uintptr_t)dbias_table % 4 != 0))
    return fail(TERRA_ERR_ALIGN, "bias tables must be 4-byte aligned");
  if (dbias_table != nullptr && bias_table == nullptr)
    return fail(TERRA_ERR_SHAPE, "dbias_table without bias_table");
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
  const int64_t items = (int64_t)d.num_windows * d.heads;
  if (items >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "too many window-heads for one launch");

  BwdParams bp;
  memset(&bp, 0, sizeof(bp));
  AttnParams& p = bp.a;
  p.q = q; p.k = k; p.v = v; p.o = const_cast<void*>(dout);
  p.q_stride = d.q_stride; p.k_stride = d.k_stride; p.v_stride = d.v_stride; p.o_stride = desc->dout_stride;
  p.bias_table = bias_table;
  p.explicit_mask = explicit_mask;
  p.land_bits = land_bits;
  p.items = (int32_t)items;
  p.heads = d.heads;
  p.N = d.tokens;
  p.n_geo = d.window_h * d.window_w;
  p.window_h = d.window_h;
  p.window_w = d.window_w;
  p.table_size = (2 * d.window_h - 1) * (2 * d.window_w - 1);
  p.n_real = d.n_real;
  p.scale_l2e = d.scale * kLog2e;
  p.mask_l2e = d.mask_value * kLog2e;
  p.pad_key_l2e = d.pad_key_value * kLog2e;
  p.mask_mode = d.mask_mode; p.mask_windows = d.mask_windows > 0 ? d.mask_windows : 1;
  p.frame_h = d.frame_h; p.frame_w = d.frame_w; p.shift_h = d.shift_h; p.shift_w = d.shift_w;
  p.win_row_begin = d.win_row_begin; p.win_rows = d.win_rows; p.win_cols = d.win_cols;
  bp.dq = dq; bp.dk = dk; bp.dv = dv;
  bp.dq_stride = desc->dq_stride; bp.dk_stride = desc->dk_stride; bp.dv_stride = desc->dv_stride;
  bp.dbias = dbias_table;
  for (int t = 0; t < 3; ++t) bp.dsum[t] = dsum[t];
  bp.scale = d.scale;
  bp.mask_value = d.mask_value;
  bp.pad_key_value = d.pad_key_value;

  const bool expl = d.mask_mode == TERRA_MASK_EXPLICIT;
  hipStream_t s = (hipStream_t)stream;
  int st;
  if (dtype == TERRA_DTYPE_BF16) {
    // MFMA tiles for every bf16 window; the 8x8 closed-form geometry where it
    // applies (with a dense mask, only a 16-byte aligned one: that geometry
    // reads four mask entries per load).  Two heads per workgroup for head
    // dim 32 (128-byte row slices), else one.
    const bool ws8 = d.window_h == 8 && d.window_w == 8 && d.tokens == 64 && d.n_real == 64 &&
                     (!expl || (reinterpret_cast<uintptr_t>(explicit_mask) & 15) == 0);
    const int G = (D == 32 && d.heads % 2 == 0) ? 2 : 1;
    p.group = G;
    p.groups = d.heads / G;
    st = ws8 ? launch_bwd_tiles<true>(bp, s, D, G, expl) : launch_bwd_tiles<false>(bp, s, D, G, expl);
  } else {
    p.group = p.groups = 0;
    st = D == 32   ? (expl ? launch_bwd_generic<32, true>(bp, s) : launch_bwd_generic<32, false>(bp, s))
         : D == 64 ? (expl ? launch_bwd_generic<64, true>(bp, s) : launch_bwd_generic<64, false>(bp, s))
                   : (expl ? launch_bwd_generic<128, true>(bp, s) : launch_bwd_generic<128, false>(bp, s));
  }
  if (st != TERRA_OK) return st;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_bwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}

}  // namespace

extern "C" int terra_swin_attn_bwd(const void* q, const void* k, const void* v, const void* dout, void* dq,
                                   void* dk, void* dv, int dtype, const terra_swin_attn_bwd_desc* desc,
                                   const float* bias_table, float* dbias_table, const float* explicit_mask,
                                   const uint64_t* land_bits, void* stream) {
  clear_error();
  float* const none[3] = {nullptr, nullptr, nullptr};
  return attn_bwd_impl(q, k, v, dout, dq, dk, dv, dtype, desc, bias_table, dbias_table, explicit_mask, land_bits,
                       none, stream);
}

extern "C" int terra_swin_attn_bwd_sums(const void* q, const void* k, const void* v, const void* dout, void* dq,
                                        void* dk, void* dv, int dtype, const terra_swin_attn_bwd_desc* desc,
                                        const float* bias_table, float* dbias_table, const float* explicit_mask,
                                        const uint64_t* land_bits, float* dq_sums, float* dk_sums, float* dv_sums,
                                        void* stream) {
  clear_error();
  float* const sums[3] = {dq_sums, dk_sums, dv_sums};
  return attn_bwd_impl(q, k, v, dout, dq, dk, dv, dtype, desc, bias_table, dbias_table, explicit_mask, land_bits,
                       sums, stream);
}
