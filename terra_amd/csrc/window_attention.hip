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
// Three kernels share that core:
//
//   window_attn_ring_kernel   bf16, 8x8 windows, no padded tokens, analytic
//       masks, head dim 32 with an even head count (two heads per workgroup)
//       or head dim 64 (one head per workgroup): 128-byte row slices loaded
//       straight into two LDS buffers, one unit ahead (below).
//
//   window_attn_tile_kernel   the same bf16 8x8 shapes when the scale is
//       below 2^-20 (zero included): the ring kernel divides the bias and
//       mask terms by the scale, and as it goes to zero they would swamp the
//       raw scores' low bits, then overflow.  This kernel adds them after
//       scaling.  It also takes a dense [nW, 64, 64] mask (16-byte aligned),
//       staged into LDS with each unit's rows.  (An odd head count of dim 32 has no 128-byte group and
//       runs the wave kernel.)  A persistent workgroup loops over (window,
//       group of G heads) units, two waves per head (one per query half).
//       The group's q, k, v rows (a contiguous slice of G*D channels, whole
//       128-byte lines) are streamed into LDS with nontemporal loads while
//       the previous unit is computed; O is staged in LDS over Q and streamed
//       out as whole lines.
//       The relative-position index of lane element (it, jt, r) is
//       lane_base + 30*(it - jt) - r, so the bias comes from LDS with
//       compile-time offsets.
//
//   window_attn_wave_kernel   everything else (fp32, any window up to 8x8,
//       padded tokens and keys, dense masks not taken above): one wavefront per
//       (window, head), K and Q fragments loaded straight from global memory,
//       V staged in the wave's LDS.
#include "common.h"
#include "attn_core.h"

#include <cmath>
#include <utility>

namespace terra {
namespace {

// ============================================================================
// window-tile kernel: bf16, 8x8 windows, one workgroup per (window, head group)
// ============================================================================

constexpr int kTileMaxRowBytes = 384;  // G*D*2 <= 384 (<= 192 bf16 channels)

// Dense-mask bytes per unit in LDS (kExplicit): the window's [64][64] fp32 mask.
constexpr int kMaskTileBytes = kNPad * kNPad * (int)sizeof(float);

template <int D, int G, bool kExplicit>
__global__ __launch_bounds__(G * 128) void window_attn_tile_kernel(const AttnParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int nthreads = G * 128;              // two waves per head
  constexpr int cpr = G * D / 8;                 // chunks per row (multiple of 8)
  constexpr int tile_bytes = kNPad * cpr * 16;
  static_assert(cpr % 8 == 0 && G * D * 2 <= kTileMaxRowBytes, "head group must be whole 128-byte lines");
  uint8_t* qs = smem;                            // Q, later O
  uint8_t* ks = smem + tile_bytes;
  uint8_t* vs = smem + 2 * tile_bytes;
  float* mtile = reinterpret_cast<float*>(smem + 3 * tile_bytes);  // dense mask (kExplicit)
  float* tables = reinterpret_cast<float*>(smem + 3 * tile_bytes + (kExplicit ? kMaskTileBytes : 0));

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = wave >> 1;                    // head of the group
  const int half = wave & 1;                     // query tiles 2*half, 2*half + 1
  const int lane = tid & 63;
  const int units = (p.items / p.heads) * p.groups;  // (window, head group) pairs

  // A workgroup streams whole rows: each thread keeps one 16-byte chunk column
  // of the group's row slice and steps down rows row0 + kRowStep*u.
  constexpr int kPer = kNPad * cpr / nthreads;   // chunks per thread per tensor (D/16)
  constexpr int kRowStep = nthreads / cpr;
  static_assert(kRowStep * cpr == nthreads && kRowStep * kPer == kNPad, "row tiling");
  const int row0 = tid / cpr, chunk0 = tid % cpr;

  // q, k, v of one unit -> registers (nontemporal: every byte is read once);
  // with a dense mask also the window's mask (cached: windows share it).
  constexpr int kMPer = (kMaskTileBytes / 16 + nthreads - 1) / nthreads;  // 16-byte pieces per thread
  uint4 buf[3][kPer];
  float4 mbuf[kExplicit ? kMPer : 1];
  auto fetch = [&](int unit) {
    const int w = unit / p.groups, hg = unit - w * p.groups;
    if constexpr (kExplicit) {
      const float* mw = p.explicit_mask + (int64_t)(w % p.mask_windows) * kNPad * kNPad;
#pragma unroll
      for (int u = 0; u < kMPer; ++u) {
        const int e = tid + u * nthreads;
        if (e < kMaskTileBytes / 16) mbuf[u] = *reinterpret_cast<const float4*>(mw + 4 * e);
      }
    }
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
    if constexpr (kExplicit) {
#pragma unroll
      for (int u = 0; u < kMPer; ++u) {
        const int e = tid + u * nthreads;
        if (e < kMaskTileBytes / 16) *reinterpret_cast<float4*>(mtile + 4 * e) = mbuf[u];
      }
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
    tile_attention_wave<D, cpr, kExplicit>(qs, ks, vs, head, half, p, m, tab, lane, mtile);
    __syncthreads();

    // ---- stream O out (whole lines) ------------------------------------------
    {
      // The unit's slice of o: kNPad rows of G*D elements at row stride o_stride.
      const uint16_t* slice = reinterpret_cast<const uint16_t*>(p.o) + (int64_t)w * kNPad * p.o_stride + hg * G * D;
      const __amdgpu_buffer_rsrc_t out =
          buffer_rsrc(slice, (uint32_t)(((int64_t)(kNPad - 1) * p.o_stride + G * D) * 2));
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int row = row0 + kRowStep * u;
        const int off = tile_slot(row, chunk0, cpr) * 16;
        const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(qs + off));
        // nt: 128-byte slices of a strided tensor (40.7-41.0 against 41.4-41.5 us at c4 with sc1)
        stream_store_nt(val, out, (uint32_t)(row * p.o_stride + chunk0 * 8) * 2);
      }
    }
    if (next >= units) break;
    unit = next;
  }
}

// ============================================================================
// ring kernel: head dim 32, one query tile per wave, loads two windows ahead
// ============================================================================
//
// One workgroup per (window, head group of G heads), persistent, and a fixed
// head group per workgroup (the grid is a multiple of the number of groups).
// Four waves per head, one 16-query tile each.  q, k, v of a unit go straight
// from memory into one of two LDS buffers by direct global->LDS loads,
// issued one unit ahead, so a workgroup never holds loads in registers.  Two
// buffers rather than three (two units ahead): at head dim 64 a third
// four-wave workgroup then fits per CU, with more bytes in flight per CU
// than the deeper ring kept (c4's core 38.8-39.1 -> 37.4-37.9 us); c3's core
// measured 127-128 -> 124-127 us, g1's the same.  The additive terms are in
// raw-score units (bias / scale), added as the accumulator init of S^T
// (attend_qtiles).

constexpr int kRingBufs = 2;

template <int D, int G>
constexpr int ring_lds_bytes() {
  return kRingBufs * 3 * kNPad * (G * D / 8) * 16 + G * kTableMax * (int)sizeof(float);
}

template <int D, int G>
__global__ __launch_bounds__(G * 256) void window_attn_ring_kernel(const AttnParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int KF = D / 32;                      // k-steps of the score MFMA
  constexpr int CT = D / 16;                      // output column tiles of P V
  constexpr int nthreads = G * 256;
  constexpr int cpr = G * D / 8;                  // chunks per row (multiple of 8)
  constexpr int tile_bytes = kNPad * cpr * 16;
  constexpr int unit_bytes = 3 * tile_bytes;
  constexpr int kRounds = unit_bytes / (nthreads * 16);  // 16-byte loads per thread per unit
  constexpr int kBlocksPerTile = tile_bytes / 1024;
  constexpr int kOPer = kNPad * cpr / nthreads;   // O chunks per thread
  static_assert(cpr % 8 == 0 && kRounds * nthreads * 16 == unit_bytes, "whole 1 KB blocks per wave");
  static_assert(kOPer * nthreads == kNPad * cpr, "whole O chunks per thread");
  float* tables = reinterpret_cast<float*>(smem + kRingBufs * unit_bytes);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = wave >> 2;                     // head of the group
  const int it = wave & 3;                        // query tile
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int windows = p.items / p.heads;
  // Units are (window, head group) pairs, unit = window * groups + hg; the
  // grid is a multiple of groups, so this workgroup keeps head group hg and
  // steps through windows w0, w0 + wstride, ...
  const int hg = blockIdx.x % p.groups;
  const int w0 = blockIdx.x / p.groups;
  const int wstride = gridDim.x / p.groups;
  const int h = hg * G + head;

  // Bias column of this head in raw-score units; the head's four waves split it.
  float* tab = tables + head * kTableMax;
  const float tab_mul = kLog2e / p.scale_l2e;     // = 1 / scale
  for (int e = lane + 64 * it; e < kTableMax; e += 256) {
    const int ri = kTableRev - e;  // reversed column (lane_bias_rev)
    tab[e] = (p.bias_table != nullptr && ri < p.table_size) ? p.bias_table[(int64_t)ri * p.heads + h] * tab_mul : 0.f;
  }
  const float mask_term = p.mask_l2e / p.scale_l2e;  // mask_value / scale

  // This thread's part of a unit's loads: one 1 KB block of one tensor per
  // wave and round, LDS slot s of the block holding (row, chunk) with
  // flash_slot(row, chunk) = block * 64 + s.  Per round: the tensor, its row
  // stride, the element offset inside the window's rows and the LDS block.
  const uint16_t* src_base[kRounds];
  int64_t src_stride[kRounds];
  int32_t src_off[kRounds];
  int32_t lds_blk[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * (nthreads / 64) + wave;   // 0 .. 3 * kBlocksPerTile - 1
    const int t = blk / kBlocksPerTile;           // 0 q, 1 k, 2 v
    const int sl = (blk - t * kBlocksPerTile) * 64 + lane;
    const int row = sl / cpr;
    const int ch = flash_slot<cpr>(row, sl - row * cpr) - row * cpr;  // the XOR is its own inverse
    src_base[r] = t == 0 ? reinterpret_cast<const uint16_t*>(p.q)
                         : t == 1 ? reinterpret_cast<const uint16_t*>(p.k) : reinterpret_cast<const uint16_t*>(p.v);
    src_stride[r] = t == 0 ? p.q_stride : t == 1 ? p.k_stride : p.v_stride;
    src_off[r] = (int32_t)(row * src_stride[r]) + hg * G * D + ch * 8;
    lds_blk[r] = blk * 1024;
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  auto issue = [&](int w, int buf) {
#pragma unroll
    for (int r = 0; r < kRounds; ++r)
      dma_to_lds16(src_base[r] + (int64_t)w * kNPad * src_stride[r] + src_off[r],
                   lds0 + buf * unit_bytes + lds_blk[r]);
  };

  int w = w0;                                     // < windows: the grid is never larger than the work
  issue(w, 0);
  const float* tabr = lane_bias_rev(tab, lane);  // bias of element (it, jt, r) at tabr[30 (3 - it + jt) + r]
  const int hc = head * (D / 8);                  // first chunk of this head
  const int orow = tid / cpr, ochunk = tid - (tid / cpr) * cpr;  // this thread's first O chunk
  for (int n = 0;; ++n) {
    const int buf = n % kRingBufs;
    const bool more = w + wstride < windows;
    // This unit's loads were the last loads issued; the previous unit's O
    // stores came after them, and loads and stores do not complete in order
    // with each other, so the wait is for everything.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();                                // every wave's part of the unit is in LDS
    // Unit n + 1 goes into the buffer of unit n - 1, whose O every thread has
    // read out before the barrier above.
    if (more) issue(w + wstride, (n + 1) % kRingBufs);
    uint8_t* qs = smem + buf * unit_bytes;
    const uint8_t* ks = qs + tile_bytes;
    const uint8_t* vs = qs + 2 * tile_bytes;
    // Mask state of the window.  The land word is read through the scalar
    // (constant) path: a vector load here would be waited for together with
    // the loads in flight for the next units.
    WindowMaskState m = window_mask_state(p, w, true, /*land=*/false);
    if (p.land_bits != nullptr) {
      const int li = __builtin_amdgcn_readfirstlane(w % p.mask_windows);
      m.land = ((const __attribute__((address_space(4))) uint64_t*)p.land_bits)[li];
      m.use_mask = m.use_shift || m.land != 0ull;
    }
    {
      uint4 kf[4][KF], qp[1][KF];
#pragma unroll
      for (int c = 0; c < KF; ++c) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          kf[t][c] = *reinterpret_cast<const uint4*>(ks + flash_slot<cpr>(16 * t + c16, hc + 4 * c + g) * 16);
        qp[0][c] = *reinterpret_cast<const uint4*>(qs + flash_slot<cpr>(16 * it + c16, hc + 4 * c + g) * 16);
      }
      auto vfrag = [&](int ct, int js) -> bf16x8 {
        const int cc = head * D + 16 * ct + 4 * (c16 & 3);  // channel of this source lane
        uint2 part[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
          part[h2] = lds_read_tr16(vs + flash_slot<cpr>(row, cc >> 3) * 16 + (cc & 7) * 2);
        }
        const uint32_t wd[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
        return __builtin_bit_cast(bf16x8, wd);
      };
      f32x4 o[1][CT];
      float inv[1];
      f32x4 land_term[4];                          // read by attend_qtiles only for windows with land keys
      if (m.use_shift) {                           // wave-uniform mask mode of the window
        uint64_t rid_pack = 0;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            rid_pack |= (uint64_t)(3 * region(m.wr * 8 + 2 * jt + (g >> 1), p.frame_h, 8, p.shift_h) +
                                   region(m.wc * 8 + 4 * (g & 1) + r, p.frame_w, 8, p.shift_w))
                        << (4 * (4 * jt + r));
        const int rid_q[1] = {3 * region(m.wr * 8 + 2 * it + (c16 >> 3), p.frame_h, 8, p.shift_h) +
                              region(m.wc * 8 + (c16 & 7), p.frame_w, 8, p.shift_w)};
        if (m.land != 0ull) land_terms(land_term, m.land, g, mask_term);
        attend_qtiles<kMaskShift, 1>(o, inv, it, kf, qp, tabr, m, land_term, rid_pack, rid_q, mask_term,
                                     p.scale_l2e, vfrag);
      } else {
        const int rid_q[1] = {0};
        if (m.land != 0ull) {
          land_terms(land_term, m.land, g, mask_term);
          attend_qtiles<kMaskLand, 1>(o, inv, it, kf, qp, tabr, m, land_term, 0ull, rid_q, mask_term, p.scale_l2e,
                                      vfrag);
        } else {
          attend_qtiles<kMaskNone, 1>(o, inv, it, kf, qp, tabr, m, land_term, 0ull, rid_q, mask_term, p.scale_l2e,
                                      vfrag);
        }
      }
      // O over this wave's own Q rows (read above, before any write).
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      const int i = 16 * it + c16;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const f32x4 v = o[0][ct] * inv[0];
        const int cc = head * D + 16 * ct + 4 * g;  // 4 channels, 8 bytes
        uint2 pk;
        pk.x = pack_bf16x2(v[0], v[1]);
        pk.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(qs + flash_slot<cpr>(i, cc >> 3) * 16 + (cc & 7) * 2) = pk;
      }
    }
    lds_barrier();                                // O complete
    {
      // Whole-line stores, kOPer chunks per thread (rows orow + u nthreads / cpr).
      const uint16_t* slice = reinterpret_cast<const uint16_t*>(p.o) + (int64_t)w * kNPad * p.o_stride + hg * G * D;
      const __amdgpu_buffer_rsrc_t out =
          buffer_rsrc(slice, (uint32_t)(((int64_t)(kNPad - 1) * p.o_stride + G * D) * 2));
#pragma unroll
      for (int u = 0; u < kOPer; ++u) {
        const int row = orow + u * (nthreads / cpr);
        const u32x4 val =
            __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(qs + flash_slot<cpr>(row, ochunk) * 16));
        stream_store_sc1(val, out, (uint32_t)(row * p.o_stride + ochunk * 8) * 2);
      }
    }
    if (!more) break;
    w += wstride;
  }
}

// ============================================================================
// flash kernel: windows of more than 64 tokens (TERRA's ws-32 configuration:
// 1024 tokens per window), bf16, no bias and no mask
// ============================================================================
//
// One workgroup per (window, head, block of 32 W queries), W = 4 waves of 32
// queries (two 16-query tiles); the window's keys stream through LDS in tiles of 64
// (K and V straight from memory by global->LDS loads, two buffers each).  A
// wave holds its Q^T fragments in registers for the whole loop; per key tile
// it forms S^T = K Q^T one tile ahead, exponentiates the scores of the
// current tile against a lazily updated row offset (online softmax in
// raw-score units times scale * log2(e)), adds V^T P^T with P packed from the
// S^T accumulators (the same k-slot order and transposed V reads as the 8x8
// kernels), and sums P per row in fp32.  The query blocks of one (window,
// head) are workgroups b = 8 i + x, i consecutive, so they run together on
// XCD x and share the window's K and V from that XCD's L2.  The global->LDS
// loads cost issue time on the waves that make them, whatever their latency,
// so they go out spread over the score MFMAs.  Eight-wave workgroups (256
// queries, half the loads per MFMA) measured slower: one workgroup per CU
// then keeps both waves of a SIMD in the same phase between barriers, where
// two four-wave workgroups drift apart and fill each other's gaps.
constexpr int kFlashQ = 128;  // queries per workgroup (W = 4)
constexpr int kFlashK = 64;   // keys per LDS tile


template <int D>
constexpr int flash_lds_bytes() {
  return 2 * 2 * kFlashK * D * 2;  // two K and two V tiles
}

// Extra arguments of the flash kernel's statistics mode (the first pass of
// the backward): per query row i and head h it writes LSE'_i = log2 of the
// softmax denominator in the log2-domain logit units (so that P = 2^(s c -
// LSE'), c = scale log2 e) and D_i = sum_d dout[i, d] o[i, d], as two floats
// at the start of row i's head-h slice of `stats` (bf16 elements, row stride
// stats_stride: the caller's dq, which the last pass overwrites).
struct FlashStatsArgs {
  const void* dout;
  int64_t dout_stride;
  void* stats;
  int64_t stats_stride;
};

template <int D, int W, bool kStats>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void window_attn_flash_kernel(
    const AttnParams p, const FlashStatsArgs sa) {
  constexpr int KF = D / 32;                 // k-steps of S^T = K Q^T
  constexpr int CT = D / 16;                 // column tiles of O^T
  constexpr int cpr = D / 8;                 // 16-byte chunks per key row of one head
  constexpr int kTile = kFlashK * D * 2;     // one K (or V) tile
  constexpr int kBlocks = kTile / 1024;      // its 1 KB blocks
  constexpr int kHalf = kBlocks / W;         // loads per thread per K (or V) tile
  static_assert(cpr % 8 == 0 && kHalf * W == kBlocks, "whole 1 KB blocks per wave");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  // Block b -> (unit, query block): within each run of 8 * qblocks blocks,
  // unit (b / (8 qblocks)) * 8 + b % 8 takes query blocks (b / 8) % qblocks,
  // all on XCD b % 8; units past the last whole group of 8 map linearly.
  const int qblocks = p.N / (32 * W);
  const int b = (int)blockIdx.x;
  const int full = (p.items / 8) * 8 * qblocks;
  int unit, qb;
  if (b < full) {
    unit = (b / (8 * qblocks)) * 8 + (b & 7);
    qb = (b >> 3) % qblocks;
  } else {
    unit = (p.items / 8) * 8 + (b - full) / qblocks;
    qb = (b - full) % qblocks;
  }
  const int w = unit / p.heads, h = unit - w * p.heads;
  const int q0 = qb * 32 * W + wave * 32;     // this wave's first query
  const uint16_t* qbase = reinterpret_cast<const uint16_t*>(p.q) + (int64_t)w * p.N * p.q_stride + h * D;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(p.k) + (int64_t)w * p.N * p.k_stride + h * D;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(p.v) + (int64_t)w * p.N * p.v_stride + h * D;

  // Q^T operand fragments: qf[t][c] = Q[q0 + 16 t + c16][32 c + 8 g .. + 8].
  uint4 qf[2][KF];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < KF; ++c)
      qf[t][c] = *reinterpret_cast<const uint4*>(qbase + (int64_t)(q0 + 16 * t + c16) * p.q_stride + 32 * c + 8 * g);

  // LDS holds K tiles in buffers 0 and 1 and V tiles in buffers 2 and 3
  // (kTile bytes each).  K runs one key tile ahead of V: iteration kt
  // computes the scores of tile kt + 1, whose MFMAs interleave with the
  // softmax of tile kt, and O^T += V^T P^T of tile kt.  It reads K buffer
  // (kt + 1) & 1 and V buffer 2 + (kt & 1) while the DMA fills K buffer kt & 1
  // (tile kt + 2) and V buffer 2 + ((kt + 1) & 1) (tile kt + 1).
  // Round r of a K (or V) tile moves 1 KB block blk = W r + wave; its lane
  // holds slot blk * 64 + lane, which is flash_slot(row, chunk) of key row
  // row.  The lane's byte offset from the tile's first row is the same for
  // every key tile (at most 63 row strides, below 2^31 by the host's check).
  uint32_t koff[kHalf], voff[kHalf];
#pragma unroll
  for (int r = 0; r < kHalf; ++r) {
    const int sl = (r * W + wave) * 64 + lane;
    const int row = sl / cpr;
    const int ch = flash_slot<cpr>(row, sl - row * cpr) - row * cpr;  // the XOR is its own inverse
    koff[r] = (uint32_t)(row * p.k_stride * 2 + ch * 16);
    voff[r] = (uint32_t)(row * p.v_stride * 2 + ch * 16);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  // Round r of K tile kt into K buffer b (V tile kt into V buffer 2 + b).
  auto issue_k = [&](int kt, int b, int r) {
    dma_to_lds16_at(kbase + (int64_t)kt * kFlashK * p.k_stride, koff[r], lds0 + b * kTile + (r * W + wave) * 1024);
  };
  auto issue_v = [&](int kt, int b, int r) {
    dma_to_lds16_at(vbase + (int64_t)kt * kFlashK * p.v_stride, voff[r], lds0 + (2 + b) * kTile + (r * W + wave) * 1024);
  };
  // S^T = K Q^T of key tile kt: lane (c16, g) of s[t][jt] holds keys
  // 16 jt + 4 g + r of query 16 t + c16.
  auto scores = [&](int kt, f32x4 (&s)[2][4], auto&& after_kstep) {
    const uint8_t* ks = smem + (kt & 1) * kTile;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) s[t][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KF; ++c) {
      uint4 kf[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        kf[jt] = *reinterpret_cast<const uint4*>(ks + flash_slot<cpr>(16 * jt + c16, 4 * c + g) * 16);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          s[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[jt]),
                                                             __builtin_bit_cast(bf16x8, qf[t][c]), s[t][jt], 0, 0, 0);
      after_kstep(c);
    }
  };

  f32x4 o[2][CT];
  // Each lane's share of its query row's sum of P (its 16 keys of every
  // tile, fp32, before the bf16 rounding of the O update); the four lanes of
  // a row add their shares at the end.
  float rs[2] = {0.f, 0.f};
  // mu: each row's exponent offset, in log2 units (score * scale * log2 e).
  // It follows the row max lazily: P = 2^(score * scale * log2 e - mu) may
  // reach 2^kSlack before mu moves up (and O and the row sum are rescaled),
  // which keeps the same relative bf16 precision and skips the rescale of
  // most key tiles.
  constexpr float kSlack = 8.f;
  float mu[2] = {-__builtin_inff(), -__builtin_inff()};
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[t][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float c_l2e = p.scale_l2e;
  const int nk = p.N / kFlashK;  // >= 2: the host asks for a multiple of kFlashQ tokens

  // Iteration kt: softmax and O update of key tile kt (scores sc), with the
  // scores of tile kt + 1 computed into sn on the way when kNext.
  auto step = [&](int kt, f32x4 (&sc)[2][4], f32x4 (&sn)[2][4], auto next) {
    constexpr bool kNext = decltype(next)::value;
    float mt[2];
    bool grow = false;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float mx = sc[t][0][0];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = max_nan(mx, sc[t][jt][r]);
      mt[t] = xor_max(mx) * c_l2e;
      grow |= mt[t] > mu[t] + kSlack;  // always on the first tile (mu = -inf)
    }
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float mn = max_nan(mu[t], mt[t]);
        const float corr = __builtin_amdgcn_exp2f(mu[t] - mn);  // 0 on the first tile, 1 where mu stays
        mu[t] = mn;
        rs[t] *= corr;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o[t][ct] *= corr;
      }
    }
    // P = 2^(score * scale * log2 e - mu), a share of it after each k-step of
    // the next tile's score MFMAs (in program order, so that the exponentials
    // issue between the MFMAs).
    auto exps = [&](int c, int of) {
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        if (e * of / 32 != c) continue;
        const int t = e >> 4, jt = (e >> 2) & 3, r = e & 3;
        sc[t][jt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][jt][r], c_l2e, -mu[t]));
        rs[t] += sc[t][jt][r];
      }
    };
    // The loads of K tile kt + 2 and V tile kt + 1 (rounds j < kHalf of K,
    // then of V) go out spread over the k-steps of the score MFMAs, not in
    // one burst.  Past the last K tile the rounds reload tile nk - 1 into
    // the free buffer (nothing reads it), which keeps this block branch-free.
    constexpr int kPer = 2 * kHalf / KF;  // load rounds per k-step
    static_assert(kPer * KF == 2 * kHalf, "whole load rounds per k-step");
    // The MFMA phases at raised wave priority: the SIMD's other wave (of the
    // other workgroup) fills their gaps (711-713 -> 697-701 us at w32).
    __builtin_amdgcn_s_setprio(1);
    if constexpr (kNext)
      scores(kt + 1, sn, [&](int c) {
        exps(c, KF);
#pragma unroll
        for (int j = c * kPer; j < (c + 1) * kPer; ++j) {
          if (j < kHalf) issue_k(min(kt + 2, nk - 1), kt & 1, j);
          else issue_v(kt + 1, (kt + 1) & 1, j - kHalf);
        }
      });
    else exps(0, 1);
    // The V reads below stay after the score MFMAs (their registers would
    // otherwise be live across them).
    __builtin_amdgcn_sched_barrier(0);
    // O^T += V^T P^T; V^T fragments by transposed reads (keys 32 js + 16 (e/4) + 4 g + e % 4).
    const uint8_t* vs = smem + (2 + (kt & 1)) * kTile;
    auto vfrag = [&](int ct, int js) -> bf16x8 {
      const int cc = 16 * ct + 4 * (c16 & 3);
      uint2 part[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
        part[h2] = lds_read_tr16(vs + flash_slot<cpr>(row, cc >> 3) * 16 + (cc & 7) * 2);
      }
      const uint32_t wd[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
      return __builtin_bit_cast(bf16x8, wd);
    };
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      bf16x8 pf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t wds[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          wds[e / 2] = pack_bf16x2(sc[t][2 * js + (e >> 2)][e & 3], sc[t][2 * js + (e >> 2)][(e & 3) + 1]);
        pf[t] = __builtin_bit_cast(bf16x8, wds);
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const bf16x8 vf = vfrag(ct, js);
#pragma unroll
        for (int t = 0; t < 2; ++t) o[t][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[t], o[t][ct], 0, 0, 0);
      }
    }
    // Schedule the V fragment reads two column tiles ahead of their MFMAs,
    // so that the LDS latency hides behind the MFMAs in flight.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads: column tiles 0 and 1
#pragma unroll
    for (int i = 0; i < 2 * CT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA: column tile i, both query tiles
      if (i + 2 < 2 * CT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads: column tile i + 2
    }
    __builtin_amdgcn_s_setprio(0);
  };

#pragma unroll
  for (int r = 0; r < kHalf; ++r) issue_k(0, 0, r);
#pragma unroll
  for (int r = 0; r < kHalf; ++r) issue_v(0, 0, r);
#pragma unroll
  for (int r = 0; r < kHalf; ++r) issue_k(1, 1, r);
  // The Q loads and K tile 0 have landed when at most the V tile 0 and K tile
  // 1 loads are outstanding (loads complete in order).
  if constexpr (kHalf == 4) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (kHalf == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  static_assert(kHalf == 4 || kHalf == 2 || kHalf == 1, "head dim 128 or 64, 4 or 8 waves");
  lds_barrier();
  f32x4 sc[2][4], sn[2][4];
  scores(0, sc, [](int) {});
  for (int kt = 0; kt + 1 < nk; ++kt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's parts of V tile kt and K tile kt + 1
    lds_barrier();  // all of them are in LDS; every wave is done with iteration kt - 1
    step(kt, sc, sn, std::true_type{});
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) sc[t][jt] = sn[t][jt];
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // V tile nk - 1
  lds_barrier();
  step(nk - 1, sc, sn, std::false_type{});
  // O^T lane (c16, g) of (t, ct): channels 16 ct + 4 g .. + 3 of query q0 + 16 t + c16.
  if constexpr (kStats) {
    const uint16_t* dobase = reinterpret_cast<const uint16_t*>(sa.dout) + (int64_t)w * p.N * sa.dout_stride + h * D;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float l = xor_sum(rs[t]);
      const float inv = __builtin_amdgcn_rcpf(l);
      const int64_t row = q0 + 16 * t + c16;
      float dsum = 0.f;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const uint2 dv = *reinterpret_cast<const uint2*>(dobase + row * sa.dout_stride + 16 * ct + 4 * g);
        dsum = __builtin_fmaf(o[t][ct][0], __uint_as_float(dv.x << 16), dsum);
        dsum = __builtin_fmaf(o[t][ct][1], __uint_as_float(dv.x & 0xffff0000u), dsum);
        dsum = __builtin_fmaf(o[t][ct][2], __uint_as_float(dv.y << 16), dsum);
        dsum = __builtin_fmaf(o[t][ct][3], __uint_as_float(dv.y & 0xffff0000u), dsum);
      }
      const float dd = xor_sum(dsum) * inv;
      const float lse = mu[t] + __builtin_amdgcn_logf(l);  // log2
      if (g == 0) {
        float2* dst = reinterpret_cast<float2*>(reinterpret_cast<uint16_t*>(sa.stats) +
                                                ((int64_t)w * p.N + row) * sa.stats_stride + h * D);
        *dst = make_float2(lse, dd);
      }
    }
    return;
  }
  uint16_t* obase = reinterpret_cast<uint16_t*>(p.o) + (int64_t)w * p.N * p.o_stride + h * D;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float inv = __builtin_amdgcn_rcpf(xor_sum(rs[t]));
    uint16_t* orow = obase + (int64_t)(q0 + 16 * t + c16) * p.o_stride;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const f32x4 v = o[t][ct] * inv;
      uint2 pk;
      pk.x = pack_bf16x2(v[0], v[1]);
      pk.y = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint2*>(orow + 16 * ct + 4 * g) = pk;
    }
  }
}

template <int D, int W, bool kStats = false>
int launch_flash(const AttnParams& p, hipStream_t s, const FlashStatsArgs& sa = FlashStatsArgs{}) {
  constexpr int lds = flash_lds_bytes<D>();
  auto kern = window_attn_flash_kernel<D, W, kStats>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  const int64_t blocks = (int64_t)p.items * (p.N / (32 * W));
  if (blocks >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "too many query blocks for one launch");
  kern<<<(int)blocks, 64 * W, lds, s>>>(p, sa);
  return TERRA_OK;
}

// ============================================================================
// flash backward: windows of more than 64 tokens
// ============================================================================
//
// Per (window, head), after the statistics pass (the kernel above with
// kStats: LSE'_i and D_i = rowsum(dout * o) per query, kept in dq):
//   dK/dV pass, one workgroup per 64 keys (16 per wave, K and V fragments in
//     registers), the window's queries streaming through LDS in tiles of 64
//     (q, dout and their statistics, direct global->LDS, two buffers):
//       S = Q K^T, dP = dO V^T (row reads of the tiles), P = 2^(S c - LSE'),
//       dS = P (dP - D), dV^T += dO^T P, dK^T += Q^T dS (transposed reads);
//   dQ pass, one workgroup per 128 queries (32 per wave, Q and dO fragments
//     in registers), the keys streaming through LDS in tiles of 64 (K and V):
//       S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - D),
//       dQ^T += K^T dS^T, then dq = scale dQ (over the statistics).
// dK = scale dS^T Q and dV = P^T dO are the autograd of o = softmax(scale
// q k^T) v (models/attention.py:256-278 without bias and mask); P and dS
// enter the MFMAs in bf16, as the module's bf16 matmuls do.

struct FlashBwdPtrs {
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  int64_t dout_stride, dq_stride, dk_stride, dv_stride;
  float scale;
};

constexpr int kBwdKeys = 64;  // keys per dK/dV workgroup (16 per wave)
constexpr int kBwdQ = 64;     // queries per LDS tile of the dK/dV pass

template <int D>
constexpr int flash_dkv_lds_bytes() {
  return 2 * (2 * kBwdQ * D * 2 + kBwdQ * 8);  // two stages of q, dout and LSE' / D
}

// Block b -> (unit, block of the unit): blocks of one (window, head) are
// b = 8 i + x with i consecutive, on XCD x, so they share the unit's rows in
// that XCD's L2; units past the last whole group of 8 map linearly.
__device__ __forceinline__ void flash_block_map(int b, int items, int per_unit, int& unit, int& blk) {
  const int full = (items / 8) * 8 * per_unit;
  if (b < full) {
    unit = (b / (8 * per_unit)) * 8 + (b & 7);
    blk = (b >> 3) % per_unit;
  } else {
    unit = (items / 8) * 8 + (b - full) / per_unit;
    blk = (b - full) % per_unit;
  }
}

// The A operand of a transposed product from a row-major [rows][D] tile of
// 256- or 128-byte rows: M = columns 16 mt .. + 15, k = rows 32 js + 16 (e/4)
// + 4 g + e % 4 (the order the accumulators of the row products pack in).
template <int cpr>
__device__ __forceinline__ bf16x8 flash_tr_frag(const uint8_t* tile, int mt, int js, int g, int c16) {
  const int cc = 16 * mt + 4 * (c16 & 3);
  uint2 part[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    const int row = 32 * js + 16 * h2 + 4 * g + (c16 >> 2);
    part[h2] = lds_read_tr16(tile + flash_slot<cpr>(row, cc >> 3) * 16 + (cc & 7) * 2);
  }
  const uint32_t wd[4] = {part[0].x, part[0].y, part[1].x, part[1].y};
  return __builtin_bit_cast(bf16x8, wd);
}

__device__ __forceinline__ bf16x8 pack_frag8(const f32x4& a, const f32x4& b) {
  const uint32_t wd[4] = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                          pack_bf16x2(b[2], b[3])};
  return __builtin_bit_cast(bf16x8, wd);
}

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void window_attn_flash_dkv_kernel(
    const AttnParams p, const FlashBwdPtrs bp) {
  constexpr int KF = D / 32, CT = D / 16, cpr = D / 8;
  constexpr int kTile = kBwdQ * D * 2;           // one q (or dout) tile
  constexpr int kPer = kTile / 1024 / 4;         // its 1 KB loads per wave
  constexpr int kStage = 2 * kTile + kBwdQ * 8;  // q, dout, LSE' [64], D [64]
  static_assert(kPer * 4 * 1024 == kTile, "whole 1 KB blocks per wave");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int unit, kb;
  flash_block_map((int)blockIdx.x, p.items, p.N / kBwdKeys, unit, kb);
  const int w = unit / p.heads, h = unit - w * p.heads;
  const int k0 = kb * kBwdKeys + 16 * wave;  // this wave's first key
  const int64_t wrow = (int64_t)w * p.N;
  const uint16_t* qbase = reinterpret_cast<const uint16_t*>(p.q) + wrow * p.q_stride + h * D;
  const uint16_t* dobase = reinterpret_cast<const uint16_t*>(bp.dout) + wrow * bp.dout_stride + h * D;
  const uint16_t* stbase = reinterpret_cast<const uint16_t*>(bp.dq) + wrow * bp.dq_stride + h * D;

  // B operands of the wave's 16 keys: kfr[c] = K[k0 + c16][32 c + 8 g .. + 8], vfr the same of V.
  uint4 kfr[KF], vfr[KF];
#pragma unroll
  for (int c = 0; c < KF; ++c) {
    kfr[c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.k) + (wrow + k0 + c16) * p.k_stride +
                                             h * D + 32 * c + 8 * g);
    vfr[c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.v) + (wrow + k0 + c16) * p.v_stride +
                                             h * D + 32 * c + 8 * g);
  }
  // Loads of query tile qt: round r of the q (dout) tile moves 1 KB block 4 r
  // + wave, lane slot (4 r + wave) * 64 + lane = flash_slot(row, chunk);
  // waves 0 and 1 move the 64 LSE' and D values (4 bytes per lane).
  uint32_t qoff[kPer], dooff[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int sl = (r * 4 + wave) * 64 + lane;
    const int row = sl / cpr;
    const int ch = flash_slot<cpr>(row, sl - row * cpr) - row * cpr;  // the XOR is its own inverse
    qoff[r] = (uint32_t)(row * p.q_stride * 2 + ch * 16);
    dooff[r] = (uint32_t)(row * bp.dout_stride * 2 + ch * 16);
  }
  const uint32_t soff = (uint32_t)(lane * bp.dq_stride * 2 + (wave & 1) * 4);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  auto issue = [&](int qt, int buf) {
    const uint32_t st = lds0 + buf * kStage;
    const int64_t r0 = (int64_t)qt * kBwdQ;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      dma_to_lds16_at(qbase + r0 * p.q_stride, qoff[r], st + (r * 4 + wave) * 1024);
      dma_to_lds16_at(dobase + r0 * bp.dout_stride, dooff[r], st + kTile + (r * 4 + wave) * 1024);
    }
    if (wave < 2) dma_to_lds4_at(stbase + r0 * bp.dq_stride, soff, st + 2 * kTile + wave * 256);
  };

  f32x4 dka[CT], dva[CT];
#pragma unroll
  for (int mt = 0; mt < CT; ++mt) {
    dka[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    dva[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float c_l2e = p.scale_l2e;
  const int nq = p.N / kBwdQ;
  issue(0, 0);
  for (int qt = 0; qt < nq; ++qt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's part of tile qt (and the K / V loads)
    lds_barrier();  // the whole tile is in LDS; every wave is done with tile qt - 1
    if (qt + 1 < nq) issue(qt + 1, (qt + 1) & 1);
    const uint8_t* qs = smem + (qt & 1) * kStage;
    const uint8_t* dos = qs + kTile;
    const float* lse = reinterpret_cast<const float*>(qs + 2 * kTile);
    const float* dd = lse + kBwdQ;
    // S = Q K^T and dP = dO V^T: lane (c16, g) of tile i holds key k0 + c16
    // against queries 16 i + 4 g + r.
    f32x4 sa[4], dp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sa[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      dp[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int c = 0; c < KF; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 qa = *reinterpret_cast<const uint4*>(qs + flash_slot<cpr>(16 * i + c16, 4 * c + g) * 16);
        const uint4 da = *reinterpret_cast<const uint4*>(dos + flash_slot<cpr>(16 * i + c16, 4 * c + g) * 16);
        sa[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qa),
                                                        __builtin_bit_cast(bf16x8, kfr[c]), sa[i], 0, 0, 0);
        dp[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, da),
                                                        __builtin_bit_cast(bf16x8, vfr[c]), dp[i], 0, 0, 0);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse + 16 * i + 4 * g);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(dd + 16 * i + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[i][r], c_l2e, -l4[r]));
        sa[i][r] = pv;
        dp[i][r] = pv * (dp[i][r] - d4[r]);
      }
    }
    // dV^T += dO^T P and dK^T += Q^T dS, 32 queries per k-step.
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      const bf16x8 pf = pack_frag8(sa[2 * js], sa[2 * js + 1]);
      const bf16x8 sf = pack_frag8(dp[2 * js], dp[2 * js + 1]);
#pragma unroll
      for (int mt = 0; mt < CT; ++mt) {
        dva[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(flash_tr_frag<cpr>(dos, mt, js, g, c16), pf, dva[mt], 0, 0, 0);
        dka[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(flash_tr_frag<cpr>(qs, mt, js, g, c16), sf, dka[mt], 0, 0, 0);
      }
    }
  }
  // dK^T / dV^T lane (c16, g) of tile mt: channels 16 mt + 4 g .. + 3 of key k0 + c16.
  uint16_t* dkrow = reinterpret_cast<uint16_t*>(bp.dk) + (wrow + k0 + c16) * bp.dk_stride + h * D;
  uint16_t* dvrow = reinterpret_cast<uint16_t*>(bp.dv) + (wrow + k0 + c16) * bp.dv_stride + h * D;
#pragma unroll
  for (int mt = 0; mt < CT; ++mt) {
    const f32x4 kv = dka[mt] * bp.scale;
    uint2 pk;
    pk.x = pack_bf16x2(kv[0], kv[1]);
    pk.y = pack_bf16x2(kv[2], kv[3]);
    *reinterpret_cast<uint2*>(dkrow + 16 * mt + 4 * g) = pk;
    pk.x = pack_bf16x2(dva[mt][0], dva[mt][1]);
    pk.y = pack_bf16x2(dva[mt][2], dva[mt][3]);
    *reinterpret_cast<uint2*>(dvrow + 16 * mt + 4 * g) = pk;
  }
}

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void window_attn_flash_dq_kernel(
    const AttnParams p, const FlashBwdPtrs bp) {
  constexpr int KF = D / 32, CT = D / 16, cpr = D / 8;
  constexpr int kTile = kFlashK * D * 2;  // one K (or V) tile
  constexpr int kHalf = kTile / 1024 / 4;
  static_assert(kHalf * 4 * 1024 == kTile, "whole 1 KB blocks per wave");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int unit, qb;
  flash_block_map((int)blockIdx.x, p.items, p.N / kFlashQ, unit, qb);
  const int w = unit / p.heads, h = unit - w * p.heads;
  const int q0 = qb * kFlashQ + wave * 32;  // this wave's first query
  const int64_t wrow = (int64_t)w * p.N;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(p.k) + wrow * p.k_stride + h * D;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(p.v) + wrow * p.v_stride + h * D;

  // B operands of the wave's queries: qf[t][c] = Q[q0 + 16 t + c16][32 c + 8 g ..], df the same of dO;
  // each lane's query row statistics (LSE', D) from dq, which this wave
  // overwrites at the end.
  uint4 qf[2][KF], df[2][KF];
  float lse[2], dd[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = wrow + q0 + 16 * t + c16;
#pragma unroll
    for (int c = 0; c < KF; ++c) {
      qf[t][c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.q) + row * p.q_stride + h * D +
                                                 32 * c + 8 * g);
      df[t][c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(bp.dout) + row * bp.dout_stride +
                                                 h * D + 32 * c + 8 * g);
    }
    const float2 st =
        *reinterpret_cast<const float2*>(reinterpret_cast<const uint16_t*>(bp.dq) + row * bp.dq_stride + h * D);
    lse[t] = st.x;
    dd[t] = st.y;
  }
  // Key tile kt -> K buffer 2 (kt & 1), V buffer 2 (kt & 1) + 1: round r
  // moves block 4 r + wave of each.
  uint32_t koff[kHalf], voff[kHalf];
#pragma unroll
  for (int r = 0; r < kHalf; ++r) {
    const int sl = (r * 4 + wave) * 64 + lane;
    const int row = sl / cpr;
    const int ch = flash_slot<cpr>(row, sl - row * cpr) - row * cpr;
    koff[r] = (uint32_t)(row * p.k_stride * 2 + ch * 16);
    voff[r] = (uint32_t)(row * p.v_stride * 2 + ch * 16);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  auto issue = [&](int kt, int buf) {
    const uint32_t st = lds0 + buf * 2 * kTile;
#pragma unroll
    for (int r = 0; r < kHalf; ++r) {
      dma_to_lds16_at(kbase + (int64_t)kt * kFlashK * p.k_stride, koff[r], st + (r * 4 + wave) * 1024);
      dma_to_lds16_at(vbase + (int64_t)kt * kFlashK * p.v_stride, voff[r], st + kTile + (r * 4 + wave) * 1024);
    }
  };

  f32x4 o[2][CT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[t][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float c_l2e = p.scale_l2e;
  const int nk = p.N / kFlashK;
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's part of tile kt (and the Q / dO loads)
    lds_barrier();  // the whole tile is in LDS; every wave is done with tile kt - 1
    if (kt + 1 < nk) issue(kt + 1, (kt + 1) & 1);
    const uint8_t* ks = smem + (kt & 1) * 2 * kTile;
    const uint8_t* vs = ks + kTile;
    // S^T = K Q^T, dP^T = V dO^T: lane (c16, g) holds keys 16 jt + 4 g + r of query 16 t + c16.
    f32x4 s[2][4], dp[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        s[t][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[t][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int c = 0; c < KF; ++c) {
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint4 kf = *reinterpret_cast<const uint4*>(ks + flash_slot<cpr>(16 * jt + c16, 4 * c + g) * 16);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          s[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf),
                                                             __builtin_bit_cast(bf16x8, qf[t][c]), s[t][jt], 0, 0, 0);
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint4 vf = *reinterpret_cast<const uint4*>(vs + flash_slot<cpr>(16 * jt + c16, 4 * c + g) * 16);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          dp[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vf),
                                                              __builtin_bit_cast(bf16x8, df[t][c]), dp[t][jt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][jt][r], c_l2e, -lse[t]));
          dp[t][jt][r] = pv * (dp[t][jt][r] - dd[t]);
        }
    // dQ^T += K^T dS^T, 32 keys per k-step.
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      bf16x8 sf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) sf[t] = pack_frag8(dp[t][2 * js], dp[t][2 * js + 1]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const bf16x8 kt_frag = flash_tr_frag<cpr>(ks, ct, js, g, c16);
#pragma unroll
        for (int t = 0; t < 2; ++t) o[t][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt_frag, sf[t], o[t][ct], 0, 0, 0);
      }
    }
  }
  // dQ^T lane (c16, g) of (t, ct): channels 16 ct + 4 g .. + 3 of query q0 + 16 t + c16.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    uint16_t* row = reinterpret_cast<uint16_t*>(bp.dq) + (wrow + q0 + 16 * t + c16) * bp.dq_stride + h * D;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const f32x4 v = o[t][ct] * bp.scale;
      uint2 pk;
      pk.x = pack_bf16x2(v[0], v[1]);
      pk.y = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint2*>(row + 16 * ct + 4 * g) = pk;
    }
  }
}

template <int D>
int launch_flash_bwd(const AttnParams& p, const FlashBwdPtrs& bp, hipStream_t s) {
  // pass 1: row statistics into dq
  const FlashStatsArgs sa{bp.dout, bp.dout_stride, bp.dq, bp.dq_stride};
  int st = launch_flash<D, 4, true>(p, s, sa);
  if (st != TERRA_OK) return st;
  // pass 2: dK, dV
  {
    constexpr int lds = flash_dkv_lds_bytes<D>();
    auto kern = window_attn_flash_dkv_kernel<D>;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
    const int64_t blocks = (int64_t)p.items * (p.N / kBwdKeys);
    if (blocks >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "too many key blocks for one launch");
    kern<<<(int)blocks, 256, lds, s>>>(p, bp);
  }
  // pass 3: dQ over the statistics
  {
    constexpr int lds = flash_lds_bytes<D>();
    auto kern = window_attn_flash_dq_kernel<D>;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
    const int64_t blocks = (int64_t)p.items * (p.N / kFlashQ);
    kern<<<(int)blocks, 256, lds, s>>>(p, bp);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "flash backward launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
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
  // K and Q fragments straight from global memory.  Heads of more than 128
  // bytes per row (bf16 D = 128, fp32 D = 64 and 128) load them per query
  // half instead, K again for the second half (from cache), so that one
  // half's fragments, scores and O accumulators fit the register file.
  constexpr int kKF = kBf16 ? D / 32 : D / 16;
  constexpr bool kPerHalf = D * (int)sizeof(T) > 128;
  auto load_frags = [&](const T* base, int64_t stride, int t0, int nt, uint4(*dst)[kKF]) {
#pragma unroll
    for (int t = 0; t < nt; ++t) {
      const int row = 16 * (t0 + t) + c16;
#pragma unroll
      for (int s = 0; s < kKF; ++s) {
        const int col = kBf16 ? 32 * s + 8 * g : g * (D / 4) + 4 * s;
        dst[t][s] = row < N ? *reinterpret_cast<const uint4*>(base + (int64_t)row * stride + col)
                            : make_uint4(0, 0, 0, 0);
      }
    }
  };
  uint4 kf[4][kKF];
  uint4 qf[kPerHalf ? 2 : 4][kKF];
  if constexpr (!kPerHalf) {
    load_frags(kw, p.k_stride, 0, 4, kf);
    load_frags(qw, p.q_stride, 0, 4, qf);
  }
  // V tile as 16-byte chunks (rows beyond N are zero), moved to LDS in
  // batches of at most 16 chunks per lane.
  constexpr int kChunksPerRow = D * (int)sizeof(T) / 16;
  constexpr int kVLoads = kNPad * kChunksPerRow / 64;
  constexpr int kVBatch = kVLoads < 16 ? kVLoads : 16;
  static_assert(kVLoads % kVBatch == 0, "whole V batches");
  auto v_chunk = [&](int u, int& row, int& col) {
    const int chunk = lane + 64 * u;
    row = chunk / kChunksPerRow;
    col = (chunk % kChunksPerRow) * (16 / (int)sizeof(T));
  };
  uint4 vr[kVBatch];
#pragma unroll
  for (int u = 0; u < kVBatch; ++u) {
    int row, col;
    v_chunk(u, row, col);
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
  for (int u0 = 0; u0 < kVLoads; u0 += kVBatch) {
    if (u0 > 0) {
#pragma unroll
      for (int u = 0; u < kVBatch; ++u) {
        int row, col;
        v_chunk(u0 + u, row, col);
        vr[u] = row < N ? *reinterpret_cast<const uint4*>(vw + (int64_t)row * p.v_stride + col)
                        : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < kVBatch; ++u) {
      int row, col;
      v_chunk(u0 + u, row, col);
      *reinterpret_cast<uint4*>(vt + row * kPitch + col) = vr[u];
    }
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
    if constexpr (kPerHalf) {
      load_frags(kw, p.k_stride, 0, 4, kf);
      load_frags(qw, p.q_stride, 2 * half, 2, qf);
      scores_pair<kBf16, D>(s, kf, *reinterpret_cast<const uint4(*)[2][kKF]>(&qf[0]));
    } else {
      scores_pair<kBf16, D>(s, kf, *reinterpret_cast<const uint4(*)[2][kKF]>(&qf[2 * half]));
    }
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
template <int D, int G, bool kExplicit>
int tile_grid(int lds) {
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, window_attn_tile_kernel<D, G, kExplicit>, G * 128, lds) !=
        hipSuccess)
      return 0;
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  return cache[dev];
}

template <int D, int G, bool kExplicit>
int launch_tile(const AttnParams& p, hipStream_t s) {
  constexpr int lds = 3 * kNPad * G * D * 2 + G * kTableMax * (int)sizeof(float) + (kExplicit ? kMaskTileBytes : 0);
  // The >64 KiB dynamic-LDS opt-in is a per-kernel attribute: set it once.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&window_attn_tile_kernel<D, G, kExplicit>), hipFuncAttributeMaxDynamicSharedMemorySize,
      lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  const int resident = tile_grid<D, G, kExplicit>(lds);
  if (resident <= 0) return fail(TERRA_ERR_LAUNCH, "cannot size the tile kernel grid for this device");
  const int units = (p.items / p.heads) * p.groups;
  const int blocks = units < resident ? units : resident;
  window_attn_tile_kernel<D, G, kExplicit><<<blocks, G * 128, lds, s>>>(p);
  return TERRA_OK;
}

// Persistent grid of the ring kernel: as many workgroups as the device holds
// at once, rounded down to a multiple of the head groups (each workgroup keeps
// one head group), never more than the work.
template <int D, int G>
int launch_ring(const AttnParams& p, hipStream_t s) {
  constexpr int lds = ring_lds_bytes<D, G>();
  auto kern = window_attn_ring_kernel<D, G>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, G * 256, lds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the ring kernel grid for this device");
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  const int units = (p.items / p.heads) * p.groups;
  int blocks = units < cache[dev] ? units : cache[dev];
  blocks -= blocks % p.groups;
  if (blocks < p.groups) blocks = p.groups;
  kern<<<blocks, G * 256, lds, s>>>(p);
  return TERRA_OK;
}

// Heads per workgroup of the tile kernel: the smallest divisor G of `heads`
// among the instantiated group widths whose row slice is a whole number of
// 128-byte lines (128, 256 or 384 bytes); 0 if there is none.  Small groups
// mean small workgroups (2*G waves, ~26 KB of LDS for G*D = 64), so three
// independent pipelines share a CU and their load and compute phases
// interleave (c3: 145 us with G = 2 against 166 us with G = 6).  With a
// dense mask, which every unit stages whole, the largest such divisor: the
// mask is then staged once per window (c3: 179-180 us with G = 6 against
// 217-219 us with G = 2).
int tile_group(int heads, int D, bool largest) {
  static const int kG32[] = {2, 4, 6};  // head dim 32
  static const int kG64[] = {1, 2, 3};  // head dim 64
  const int* cand = D == 32 ? kG32 : kG64;
  for (int n = 0; n < 3; ++n) {
    const int i = largest ? 2 - n : n;
    if (heads % cand[i] == 0) return cand[i];
  }
  return 0;
}

template <bool kExplicit>
int dispatch_tile(const AttnParams& p, int D, hipStream_t s) {
  if (D == 32) {
    switch (p.group) {
      case 6: return launch_tile<32, 6, kExplicit>(p, s);
      case 4: return launch_tile<32, 4, kExplicit>(p, s);
      default: return launch_tile<32, 2, kExplicit>(p, s);
    }
  }
  switch (p.group) {
    case 3: return launch_tile<64, 3, kExplicit>(p, s);
    case 2: return launch_tile<64, 2, kExplicit>(p, s);
    default: return launch_tile<64, 1, kExplicit>(p, s);
  }
}

}  // namespace
}  // namespace terra

namespace terra {
namespace {

// The checks shared by the forward and the backward of windows of more than
// 64 tokens: bf16, a multiple of 128 tokens per window up to 4096 (any
// window_h x window_w with that product), head dim 64 or 128, a positive
// finite scale (the row max commutes with the scaling), no relative-position
// bias, masks or padded keys (TERRA's ws-32 configuration sets
// use_relative_position_bias and use_attn_mask off).
int flash_checks(int dtype, const terra_swin_attn_desc& d, int D, const float* bias_table,
                 const float* explicit_mask, const uint64_t* land_bits) {
  if (dtype != TERRA_DTYPE_BF16)
    return fail(TERRA_ERR_UNSUPPORTED, "windows of more than %d tokens run in bf16 only", kNPad);
  if (d.tokens % kFlashQ != 0 || d.tokens > 4096)
    return fail(TERRA_ERR_UNSUPPORTED, "windows of more than %d tokens need a multiple of %d tokens up to 4096 (got %d)",
                kNPad, kFlashQ, d.tokens);
  if (D != 64 && D != 128)
    return fail(TERRA_ERR_UNSUPPORTED, "windows of more than %d tokens need head dim 64 or 128 (got %d)", kNPad, D);
  if (d.window_h <= 0 || d.window_w <= 0 || d.window_h * d.window_w != d.tokens)
    return fail(TERRA_ERR_SHAPE, "window %dx%d does not have %d tokens", d.window_h, d.window_w, d.tokens);
  if (d.n_real != d.tokens)
    return fail(TERRA_ERR_UNSUPPORTED, "windows of more than %d tokens take no padded keys", kNPad);
  if (bias_table != nullptr || explicit_mask != nullptr || land_bits != nullptr || d.mask_mode != TERRA_MASK_NONE)
    return fail(TERRA_ERR_UNSUPPORTED,
                "windows of more than %d tokens take no relative-position bias and no mask", kNPad);
  if (!(d.scale > 0.f) || !std::isfinite(d.scale))
    return fail(TERRA_ERR_UNSUPPORTED, "windows of more than %d tokens need a positive finite scale", kNPad);
  const int64_t items = (int64_t)d.num_windows * d.heads;
  if (items * (d.tokens / kFlashQ) * 2 >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "too many window-heads for one launch");
  return TERRA_OK;
}

// Windows of more than 64 tokens: the flash kernel.
int flash_fwd(const void* q, const void* k, const void* v, void* o, int dtype, const terra_swin_attn_desc& d, int D,
              const float* bias_table, const float* explicit_mask, const uint64_t* land_bits, void* stream) {
  const int chk = flash_checks(dtype, d, D, bias_table, explicit_mask, land_bits);
  if (chk != TERRA_OK) return chk;
  if (d.q_stride < d.channels || d.k_stride < d.channels || d.v_stride < d.channels || d.o_stride < d.channels)
    return fail(TERRA_ERR_SHAPE, "row strides must be >= channels");
  if (d.q_stride % 8 || d.k_stride % 8 || d.v_stride % 8 || d.o_stride % 8)
    return fail(TERRA_ERR_ALIGN, "row strides must be multiples of 8 elements");
  for (const void* ptr : {q, k, v, (const void*)o})
    if ((uintptr_t)ptr % 16 != 0) return fail(TERRA_ERR_ALIGN, "q/k/v/o must be 16-byte aligned");
  const int64_t items = (int64_t)d.num_windows * d.heads;
  if ((int64_t)(kFlashK - 1) * std::max(d.k_stride, d.v_stride) * 2 + D * 2 >= (1ll << 31))
    return fail(TERRA_ERR_SHAPE, "k/v row strides too large for windows of more than %d tokens", kNPad);
  AttnParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_stride = d.q_stride; p.k_stride = d.k_stride; p.v_stride = d.v_stride; p.o_stride = d.o_stride;
  p.items = (int32_t)items;
  p.heads = d.heads;
  p.N = d.tokens;
  p.n_geo = d.tokens;
  p.n_real = d.tokens;
  p.window_h = d.window_h; p.window_w = d.window_w;
  p.scale_l2e = d.scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const int st = D == 64 ? launch_flash<64, 4>(p, s) : launch_flash<128, 4>(p, s);
  if (st != TERRA_OK) return st;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}

}  // namespace

int flash_attention_backward(const void* q, const void* k, const void* v, const void* dout, void* dq, void* dk,
                             void* dv, int dtype, const terra_swin_attn_bwd_desc* desc, const float* bias_table,
                             float* dbias_table, const float* explicit_mask, const uint64_t* land_bits,
                             void* stream) {
  const terra_swin_attn_desc& d = desc->fwd;
  if (d.channels % d.heads != 0)
    return fail(TERRA_ERR_SHAPE, "channels %d not divisible by heads %d", d.channels, d.heads);
  const int D = d.channels / d.heads;
  const int chk = flash_checks(dtype, d, D, bias_table, explicit_mask, land_bits);
  if (chk != TERRA_OK) return chk;
  if (dbias_table != nullptr) return fail(TERRA_ERR_SHAPE, "dbias_table without bias_table");
  const int64_t strides[7] = {d.q_stride, d.k_stride, d.v_stride, desc->dout_stride,
                              desc->dq_stride, desc->dk_stride, desc->dv_stride};
  for (int i = 0; i < 7; ++i) {
    if (strides[i] < d.channels) return fail(TERRA_ERR_SHAPE, "row strides must be >= channels");
    if (strides[i] % 8 != 0) return fail(TERRA_ERR_ALIGN, "row strides must be multiples of 8 elements");
    // 32-bit lane offsets of the global->LDS loads: 63 rows of a tile
    if (63 * strides[i] * 2 + D * 2 >= (1ll << 31))
      return fail(TERRA_ERR_SHAPE, "row strides too large for windows of more than %d tokens", kNPad);
  }
  for (const void* ptr : {q, k, v, dout, (const void*)dq, (const void*)dk, (const void*)dv})
    if ((uintptr_t)ptr % 16 != 0) return fail(TERRA_ERR_ALIGN, "q/k/v/dout/dq/dk/dv must be 16-byte aligned");
  // dq holds the row statistics between the passes, so it must not share
  // memory with what the passes read.
  const int64_t rows = (int64_t)d.num_windows * d.tokens;
  auto span = [&](const void* ptr, int64_t stride) {
    const uintptr_t b = (uintptr_t)ptr;
    return std::make_pair(b, b + (uintptr_t)(((rows - 1) * stride + d.channels) * 2));
  };
  const auto sq = span(dq, desc->dq_stride);
  const std::pair<uintptr_t, uintptr_t> inputs[4] = {span(q, d.q_stride), span(k, d.k_stride), span(v, d.v_stride),
                                                     span(dout, desc->dout_stride)};
  for (const auto& in : inputs)
    if (sq.first < in.second && in.first < sq.second)
      return fail(TERRA_ERR_SHAPE, "dq must not overlap q, k, v or dout for windows of more than %d tokens", kNPad);
  AttnParams p{};
  p.q = q; p.k = k; p.v = v; p.o = nullptr;
  p.q_stride = d.q_stride; p.k_stride = d.k_stride; p.v_stride = d.v_stride;
  p.items = (int32_t)((int64_t)d.num_windows * d.heads);
  p.heads = d.heads;
  p.N = d.tokens;
  p.n_geo = d.tokens;
  p.n_real = d.tokens;
  p.window_h = d.window_h; p.window_w = d.window_w;
  p.scale_l2e = d.scale * kLog2e;
  FlashBwdPtrs bp{};
  bp.dout = dout; bp.dq = dq; bp.dk = dk; bp.dv = dv;
  bp.dout_stride = desc->dout_stride; bp.dq_stride = desc->dq_stride;
  bp.dk_stride = desc->dk_stride; bp.dv_stride = desc->dv_stride;
  bp.scale = d.scale;
  hipStream_t s = (hipStream_t)stream;
  return D == 64 ? launch_flash_bwd<64>(p, bp, s) : launch_flash_bwd<128>(p, bp, s);
}

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
  if (d.channels % d.heads != 0)
    return fail(TERRA_ERR_SHAPE, "channels %d not divisible by heads %d", d.channels, d.heads);
  const int D = d.channels / d.heads;
  if (d.tokens > kNPad) return flash_fwd(q, k, v, o, dtype, d, D, bias_table, explicit_mask, land_bits, stream);
  if (D != 32 && D != 64 && D != 128) return fail(TERRA_ERR_UNSUPPORTED, "head dim %d not in {32, 64, 128}", D);
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
  if ((int64_t)d.o_stride * d.tokens * elt >= (1ll << 32))
    return fail(TERRA_ERR_SHAPE, "one window of o must span under 4 GiB");

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
  // bf16 8x8 windows without padded tokens: window-tile kernel (a dense mask
  // only when 16-byte aligned: it is staged in 16-byte pieces).
  const bool expl = d.mask_mode == TERRA_MASK_EXPLICIT;
  const bool ws8 = dtype == TERRA_DTYPE_BF16 && d.window_h == 8 && d.window_w == 8 && d.tokens == 64 &&
                   d.n_real == 64;
  // Head dim 128 has no window-tile instance (its head slice alone is 256
  // bytes per row): a small scale or a dense mask runs the wave kernel.
  const int G = D <= 64 ? tile_group(d.heads, D, expl) : 0;
  const bool tile = ws8 && G > 0 && (!expl || (reinterpret_cast<uintptr_t>(explicit_mask) & 15) == 0);
  // The ring kernel: head dim 32 with an even head count (two heads per
  // workgroup), head dim 64 or 128 (one head per workgroup), row slices of
  // 128 or 256 bytes.  It adds bias and masks in raw-score units (divided by
  // the scale), so it takes scales of 2^-20 and above.
  const bool ring = ws8 && !expl && ((D == 32 && d.heads % 2 == 0) || D == 64 || D == 128) && d.scale >= 0x1p-20f;
  if (ring) {
    p.group = D == 32 ? 2 : 1;
    p.groups = d.heads / p.group;
    const int st = D == 32 ? launch_ring<32, 2>(p, s) : D == 64 ? launch_ring<64, 1>(p, s) : launch_ring<128, 1>(p, s);
    if (st != TERRA_OK) return st;
  } else if (tile) {
    p.group = G;
    p.groups = d.heads / G;
    const int st = expl ? dispatch_tile<true>(p, D, s) : dispatch_tile<false>(p, D, s);
    if (st != TERRA_OK) return st;
  } else {
    p.group = p.groups = 0;
    if (dtype == TERRA_DTYPE_BF16) {
      if (D == 32) expl ? launch_wave<true, 32, true>(p, s) : launch_wave<true, 32, false>(p, s);
      else if (D == 64) expl ? launch_wave<true, 64, true>(p, s) : launch_wave<true, 64, false>(p, s);
      else expl ? launch_wave<true, 128, true>(p, s) : launch_wave<true, 128, false>(p, s);
    } else {
      if (D == 32) expl ? launch_wave<false, 32, true>(p, s) : launch_wave<false, 32, false>(p, s);
      else if (D == 64) expl ? launch_wave<false, 64, true>(p, s) : launch_wave<false, 64, false>(p, s);
      else expl ? launch_wave<false, 128, true>(p, s) : launch_wave<false, 128, false>(p, s);
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_attn_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
