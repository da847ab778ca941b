// Fused Swin attention half-block forward for gfx950: bf16 activations,
// 8x8 windows, head dim 32 (C = 32 * heads).
//
// One kernel computes, for every window of the (padded, shifted) frame,
//
//   x_w   = gather of the window's 64 tokens (pad + cyclic shift + partition)
//   xn    = LayerNorm(x_w)                      fp32 statistics, bf16 output
//   q,k,v = xn W_qkv^T + b_qkv                  MFMA, fp32 accumulate, bf16
//   o     = softmax(q k^T * scale + bias + mask) v     per head
//   y_w   = x_w + (o W_proj^T + b_proj)         bf16 projection, fp32 add
//
// and scatters y_w back to the tokens it was gathered from (inverse shift,
// crop).  Only x is read from and y written to HBM (2 * B*H*W*C*2 bytes);
// the weights (4*C*C*2 bytes) are re-read from L2 by every window.
//
// Both kernels are persistent over windows and keep every [64][C] bf16 tile
// in LDS with 16-byte chunks XOR-swizzled per row (tile_slot).  A window's
// raw rows arrive by direct global -> LDS loads issued while the previous
// window is computed; they stay in LDS for the residual add and are
// overwritten by the output rows, which are streamed back to the grid.
//
// swin_block_tile_kernel (6 heads, C = 192): one 12-wave workgroup per CU.
//   Each wave loads its whole weight slice (48 q|k|v features, 16 proj
//   features) into registers ahead of use, so the GEMM phases never wait on
//   L2.  q|k|v go to LDS tiles; attention runs two waves per head (query
//   halves) on those tiles; O overwrites Q and feeds the projection.  LDS:
//   2 row tiles (raw / LayerNorm, roles alternating per window) + Q, K, V.
//
// swin_block_kernel (12 heads, C = 384; the tiles of the variant above do not
// fit): one wave per head.  Wave h computes, for all 64 tokens,
//
//   Q^T = W_q,h xn^T, K^T = W_k,h xn^T   (A = weight rows, B = xn rows)
//   V   = xn W_v,h^T                     (A = xn rows,     B = weight rows)
//
// whose accumulators are already the MFMA operands of the attention core:
// lane (c, g) of the Q^T / K^T accumulators holds head channels 4g+r and
// 16+4g+r of token c, which packed as one 8-slot fragment is the operand of
// S^T = K Q^T under the k-slot permutation (g, e) -> 16(e/4) + 4g + e%4 on
// both sides; V's accumulators give the V^T operand of O^T = V^T P^T under
// the key permutation that P^T inherits from the S^T accumulators.  So q, k
// and v never leave registers.  Wave h then computes output features
// [32h, 32h + 32) of the projection as Y^T = W_p O^T.
//
// Windows that the frame does not emit (outside the slab's window rows, or
// outside the valid-window range) pass x through unchanged, which is what
// partition -> attention -> reverse(residual) gives for their tokens.
#include "attn_core.h"

namespace terra {
namespace {

struct BlockParams {
  AttnParams a;              // scale_l2e, mask_l2e and frame/shift fields of the attention core
  const uint8_t* x;          // [B, H, W, C] bf16
  uint8_t* y;                // [B, H, W, C] bf16 (may equal x)
  const float* gamma;        // [C] or NULL (1)
  const float* beta;         // [C] or NULL (0)
  const uint16_t* w_qkv;     // [3C, C] bf16
  const float* b_qkv;        // [3C] or NULL
  const uint16_t* w_proj;    // [C, C] bf16
  const float* b_proj;       // [C] or NULL
  const float* bias_table;   // [(2*8-1)^2, heads] or NULL
  const uint64_t* land_bits; // [land_windows] or NULL
  int32_t land_windows;
  int32_t packed;            // weights in MFMA fragment order (terra_swin_pack_linear)
  int32_t layernorm;         // 0: xn = x
  int32_t shift_mask;        // analytic shift mask on/off
  float eps, inv_c;
  int32_t H, W, Hp, Wp, shift_h, shift_w, pad_top, pad_left;
  int32_t nWw, win_row_begin, win_rows, valid_begin, valid_end, nWe;
  int32_t units;             // batch * frame windows
  FastDiv fd_frame;          // frame windows per image
  FastDiv fd_nWw;
};

// Frame window of a unit and whether the frame emits it (computed) or
// passes its tokens through.
struct UnitLoc {
  int b, wr, wc;
  int computed;  // 1: emitted window, 0: pass-through
  int w_slab;    // emitted-window index b * nWe + local index (land bits)
};

__device__ __forceinline__ UnitLoc locate(const BlockParams& p, int unit) {
  UnitLoc u;
  uint32_t b, rest, wr, wc;
  p.fd_frame.divmod((uint32_t)unit, b, rest);
  p.fd_nWw.divmod(rest, wr, wc);
  u.b = (int)b;
  u.wr = (int)wr;
  u.wc = (int)wc;
  const int wr_l = u.wr - p.win_row_begin;
  const int wl = wr_l * p.nWw + u.wc;
  u.computed = ((unsigned)wr_l < (unsigned)p.win_rows &&
                (p.valid_end <= 0 || (wl >= p.valid_begin && wl < p.valid_end))) ? 1 : 0;
  u.w_slab = u.b * p.nWe + wl;
  return u;
}

// Grid token index (b*H + sh)*W + sw of window token (ti, tj), or -1 for a
// frame-padding token.
__device__ __forceinline__ int grid_token(const BlockParams& p, const UnitLoc u, int ti, int tj) {
  int ph = u.wr * 8 + ti + p.shift_h;
  int pw = u.wc * 8 + tj + p.shift_w;
  if (ph >= p.Hp) ph -= p.Hp;
  if (pw >= p.Wp) pw -= p.Wp;
  const int sh = ph - p.pad_top, sw = pw - p.pad_left;
  if ((unsigned)sh >= (unsigned)p.H || (unsigned)sw >= (unsigned)p.W) return -1;
  return (u.b * p.H + sh) * p.W + sw;
}

__device__ __forceinline__ uint4 pack_frag(const f32x4& lo, const f32x4& hi) {
  uint4 r;
  r.x = pack_bf16x2(lo[0], lo[1]);
  r.y = pack_bf16x2(lo[2], lo[3]);
  r.z = pack_bf16x2(hi[0], hi[1]);
  r.w = pack_bf16x2(hi[2], hi[3]);
  return r;
}

__device__ __forceinline__ f32x4 load_f32x4(const float* p) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  return f32x4{v.x, v.y, v.z, v.w};
}

// The 16-byte A/B-operand fragment of weight rows [16*rt, 16*rt + 16),
// input channels [32*ks, 32*ks + 32) for this lane (row rt*16 + lane%16,
// channels 32ks + 8*(lane/16) ..): strided rows of the nn.Linear layout, or
// one contiguous 1 KB block per (rt, ks) in the packed layout.
template <int kC>
__device__ __forceinline__ uint4 weight_frag(const uint16_t* w, int packed, int rt, int ks, int lane) {
  const uint4* src = packed ? reinterpret_cast<const uint4*>(w) + ((rt * (kC / 32) + ks) * 64 + lane)
                            : reinterpret_cast<const uint4*>(w + (int64_t)(16 * rt + (lane & 15)) * kC + 32 * ks +
                                                             8 * (lane >> 4));
  return *src;
}

// Cache-policy bits of the global -> LDS loads: nontemporal (every x byte is
// read once; the weights should keep L2).
constexpr int kNtAux = 2;

// Mask terms of an emitted window (shift regions over the padded frame, land
// keys of the slab window).
__device__ __forceinline__ WindowMaskState block_mask_state(const BlockParams& p, const UnitLoc u) {
  WindowMaskState m;
  m.wr = u.wr;
  m.wc = u.wc;
  m.use_shift = p.shift_mask && ((u.wr + 2) * 8 > p.Hp || (u.wc + 2) * 8 > p.Wp);
  m.land = p.land_bits != nullptr ? p.land_bits[u.w_slab % p.land_windows] : 0ull;
  m.use_mask = m.use_shift || m.land != 0ull;
  return m;
}

// The 64 x C window rows of `u` -> LDS tile `dst`, direct global -> LDS:
// instruction r of wave w fills the 64 consecutive slots (r*kWaves + w)*64 +
// lane, and the lane of slot s = row*cpr + c' loads chunk c' ^ ((row >> 1) & 7)
// of that row, the chunk tile_slot places there.  Frame-padding tokens load
// token 0 of the grid instead; their rows are never used (LayerNorm writes
// zeros for them and they are not stored).
template <int kCpr, int kWaves>
__device__ __forceinline__ void fetch_window(const BlockParams& p, const UnitLoc u, uint8_t* dst, int wave,
                                             int lane) {
  constexpr int kRounds = 64 * kCpr / (64 * kWaves);
  static_assert(kRounds * 64 * kWaves == 64 * kCpr, "whole wave-rounds of 64 slots");
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * kWaves + wave;
    const int sl = blk * 64 + lane;
    const int row = sl / kCpr;
    const int ch = (sl - row * kCpr) ^ ((row >> 1) & 7);
    const int t = grid_token(p, u, row >> 3, row & 7);
    const uint8_t* src = p.x + (int64_t)(t >= 0 ? t : 0) * (kCpr * 16) + ch * 16;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(dst + blk * 1024), 16, 0, kNtAux);
  }
}

// LayerNorm of the window rows xr -> xn (bf16).  Eight lanes own a token;
// lane `sub` holds chunks sub + 8k, k < cpr/8.  Statistics are two-pass fp32
// over the values in registers (reduced over the 8 lanes), y = (x - mean) *
// rsqrt(var + eps) * gamma + beta rounded once: the arithmetic of
// terra_swin_partition_ln.  Frame-padding tokens get zeros.  With
// p.layernorm == 0 the rows are copied.
template <int kCpr, int kThreads>
__device__ __forceinline__ void layernorm_window(const BlockParams& p, const UnitLoc u, const uint8_t* xr,
                                                 uint8_t* xn, const float* s_gamma, const float* s_beta, int tid) {
  constexpr int kTokPass = kThreads / 8;
  constexpr int kCPL = kCpr / 8;
  const int sub = tid & 7;
  for (int t = tid >> 3; t < 64; t += kTokPass) {  // uniform per wave
    const bool in = grid_token(p, u, t >> 3, t & 7) >= 0;
    float v[kCPL][8];
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + tile_slot(t, sub + 8 * k, kCpr) * 16);
      const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[k][2 * i] = bf16_bits_to_f32((uint16_t)(w4[i] & 0xffffu));
        v[k][2 * i + 1] = bf16_bits_to_f32((uint16_t)(w4[i] >> 16));
      }
    }
    uint4 outc[kCPL];
    if (p.layernorm) {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[k][e];
      const float mean = group8_sum(sum) * p.inv_c;
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[k][e] - mean;
          sq += d * d;
        }
      const float rstd = rsqrtf(group8_sum(sq) * p.inv_c + p.eps);
#pragma unroll
      for (int k = 0; k < kCPL; ++k) {
        const int c0 = (sub + 8 * k) * 8;
        float yv[8];
#pragma unroll
        for (int q = 0; q < 8; q += 4) {
          const float4 gm = *reinterpret_cast<const float4*>(s_gamma + c0 + q);
          const float4 bt = *reinterpret_cast<const float4*>(s_beta + c0 + q);
          yv[q + 0] = (v[k][q + 0] - mean) * rstd * gm.x + bt.x;
          yv[q + 1] = (v[k][q + 1] - mean) * rstd * gm.y + bt.y;
          yv[q + 2] = (v[k][q + 2] - mean) * rstd * gm.z + bt.z;
          yv[q + 3] = (v[k][q + 3] - mean) * rstd * gm.w + bt.w;
        }
        outc[k] = make_uint4(pack_bf16x2(yv[0], yv[1]), pack_bf16x2(yv[2], yv[3]),
                             pack_bf16x2(yv[4], yv[5]), pack_bf16x2(yv[6], yv[7]));
      }
    } else {
#pragma unroll
      for (int k = 0; k < kCPL; ++k)
        outc[k] = *reinterpret_cast<const uint4*>(xr + tile_slot(t, sub + 8 * k, kCpr) * 16);
    }
#pragma unroll
    for (int k = 0; k < kCPL; ++k)
      *reinterpret_cast<uint4*>(xn + tile_slot(t, sub + 8 * k, kCpr) * 16) =
          in ? outc[k] : make_uint4(0u, 0u, 0u, 0u);
  }
}

// y_w rows (xr) -> the grid tokens they were gathered from; consecutive
// lanes store consecutive chunks of a row.  Frame-padding rows are dropped.
template <int kCpr, int kThreads>
__device__ __forceinline__ void store_window(const BlockParams& p, const UnitLoc u, const uint8_t* xr, int tid) {
  constexpr int kRowStep = kThreads / kCpr;
  static_assert(kRowStep * kCpr == kThreads && 64 % kRowStep == 0, "whole rows per pass");
  const int row0 = tid / kCpr, ch0 = tid - row0 * kCpr;
#pragma unroll
  for (int r = 0; r < 64 / kRowStep; ++r) {
    const int row = row0 + kRowStep * r;
    const int t = grid_token(p, u, row >> 3, row & 7);
    if (t >= 0) {
      const u32x4 val =
          __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(xr + tile_slot(row, ch0, kCpr) * 16));
      __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(p.y + (int64_t)t * (kCpr * 16) + ch0 * 16));
    }
  }
}

// out = bf16(x + bf16(y)) for the 4 channels of a Y^T accumulator lane, in
// place over the raw row chunk at `addr` (8 bytes): the proj output rounded
// to bf16, then the residual add rounded once.
__device__ __forceinline__ void residual_add4(uint8_t* addr, const f32x4& yv) {
  const uint2 xv = *reinterpret_cast<const uint2*>(addr);
  const float x0 = bf16_bits_to_f32((uint16_t)(xv.x & 0xffffu));
  const float x1 = bf16_bits_to_f32((uint16_t)(xv.x >> 16));
  const float x2 = bf16_bits_to_f32((uint16_t)(xv.y & 0xffffu));
  const float x3 = bf16_bits_to_f32((uint16_t)(xv.y >> 16));
  uint2 out;
  out.x = pack_bf16x2(x0 + (float)(__bf16)yv[0], x1 + (float)(__bf16)yv[1]);
  out.y = pack_bf16x2(x2 + (float)(__bf16)yv[2], x3 + (float)(__bf16)yv[3]);
  *reinterpret_cast<uint2*>(addr) = out;
}

// Bias columns (x log2e) of all heads and the LayerNorm affine -> LDS.
template <int kH, int kThreads>
__device__ __forceinline__ void stage_tables(const BlockParams& p, float* tabs, float* s_gamma, float* s_beta,
                                             int tid) {
  constexpr int C = 32 * kH;
  for (int e = tid; e < kH * kTableMax; e += kThreads) {
    const int h = e / kTableMax, i = e - h * kTableMax;
    tabs[e] = (p.bias_table != nullptr && i < 225) ? p.bias_table[i * kH + h] * kLog2e : 0.f;
  }
  for (int c = tid; c < C; c += kThreads) {
    s_gamma[c] = p.gamma != nullptr ? p.gamma[c] : 1.f;
    s_beta[c] = p.beta != nullptr ? p.beta[c] : 0.f;
  }
}

// ============================================================================
// swin_block_tile_kernel: 6 heads (C = 192), 12 waves, one workgroup per CU
// ============================================================================

template <int kH>
constexpr int block_tile_lds_bytes() {
  return 5 * 64 * 32 * kH * 2 + kH * kTableMax * 4 + 2 * 32 * kH * 4;
}

template <int kH>
__global__ __launch_bounds__(128 * kH) void swin_block_tile_kernel(const BlockParams p) {
  constexpr int C = 32 * kH;
  constexpr int cpr = C / 8;
  constexpr int kWaves = 2 * kH;
  constexpr int nthreads = 64 * kWaves;
  constexpr int tile = 64 * C * 2;
  constexpr int kKS = C / 32;                      // 32-channel MFMA k-steps
  constexpr int kQkvTiles = 3 * C / 16 / kWaves;   // 16-feature q|k|v tiles per wave
  constexpr int kFeat = 16 * kQkvTiles;            // q|k|v features per wave
  constexpr int kWavesPerTensor = C / kFeat;
  static_assert(kQkvTiles * 16 * kWaves == 3 * C && kWavesPerTensor * kFeat == C, "q|k|v split");
  static_assert(C / 16 == kWaves, "one 16-feature projection tile per wave");
  static_assert(cpr % 8 == 0, "rows must be whole groups of 8 chunks (swizzle)");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* xbuf = smem;                            // 2 row tiles: raw / LayerNorm, roles alternate
  uint8_t* qs = smem + 2 * tile;                   // Q, later O
  uint8_t* ks = smem + 3 * tile;
  uint8_t* vs = smem + 4 * tile;
  float* tabs = reinterpret_cast<float*>(smem + 5 * tile);
  float* s_gamma = tabs + kH * kTableMax;
  float* s_beta = s_gamma + C;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  int unit = blockIdx.x;
  if (unit >= p.units) return;  // uniform across the workgroup
  stage_tables<kH, nthreads>(p, tabs, s_gamma, s_beta, tid);

  UnitLoc cur = locate(p, unit);
  int par = 0;
  fetch_window<cpr, kWaves>(p, cur, xbuf, wave, lane);

  for (;;) {
    // This window's rows have landed (nothing else is in flight); the
    // barrier also orders the previous window's output reads before anything
    // overwrites that tile.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint8_t* xr = xbuf + par * tile;        // raw rows, later the output rows
    uint8_t* xn = xbuf + (par ^ 1) * tile;  // LayerNorm output, then the next window's rows
    const int next = unit + (int)gridDim.x;
    UnitLoc nxt = cur;
    if (next < p.units) nxt = locate(p, next);

    if (cur.computed) {  // uniform across the workgroup
      // Lane-derived addresses are recomputed per window rather than held in
      // registers across the persistent loop.
      int lane_i = lane;
      asm volatile("" : "+v"(lane_i));
      const int g = lane_i >> 4, c16 = lane_i & 15;
      const int tid_i = wave * 64 + lane_i;
      const int sw = (c16 >> 1) & 7;  // tile_slot swizzle of rows 16t + c16

      // ---- this wave's q|k|v weight rows [f0, f0 + kFeat), all k-steps ------
      const int f0 = kFeat * wave;
      uint4 wf[kKS][kQkvTiles];
#pragma unroll
      for (int ks = 0; ks < kKS; ++ks)
#pragma unroll
        for (int ft = 0; ft < kQkvTiles; ++ft)
          wf[ks][ft] = weight_frag<C>(p.w_qkv, p.packed, f0 / 16 + ft, ks, lane_i);

      layernorm_window<cpr, nthreads>(p, cur, xr, xn, s_gamma, s_beta, tid_i);
      __syncthreads();

      // ---- q|k|v features [f0, f0 + kFeat) of the 64 tokens: Y^T = W xn^T --
      {
        f32x4 acc[kQkvTiles][4];
#pragma unroll
        for (int ft = 0; ft < kQkvTiles; ++ft) {
          const f32x4 b = p.b_qkv != nullptr ? load_f32x4(p.b_qkv + f0 + 16 * ft + 4 * g)
                                             : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) acc[ft][tt] = b;
        }
#pragma unroll
        for (int ks = 0; ks < kKS; ++ks) {
          uint4 xf[4];
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            xf[tt] = *reinterpret_cast<const uint4*>(xn + ((16 * tt + c16) * cpr + ((4 * ks + g) ^ sw)) * 16);
#pragma unroll
          for (int ft = 0; ft < kQkvTiles; ++ft)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              acc[ft][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[ks][ft]),
                                                                    __builtin_bit_cast(bf16x8, xf[tt]),
                                                                    acc[ft][tt], 0, 0, 0);
        }
        // lane (c, g) element r: feature f0 + 16ft + 4g + r of token 16tt + c
        const int tensor = wave / kWavesPerTensor;  // 0 q, 1 k, 2 v (wave-uniform)
        uint8_t* dst = tensor == 0 ? qs : (tensor == 1 ? ks : vs);
#pragma unroll
        for (int ft = 0; ft < kQkvTiles; ++ft) {
          const int fl = kFeat * (wave - tensor * kWavesPerTensor) + 16 * ft + 4 * g;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            uint2 pk;
            pk.x = pack_bf16x2(acc[ft][tt][0], acc[ft][tt][1]);
            pk.y = pack_bf16x2(acc[ft][tt][2], acc[ft][tt][3]);
            *reinterpret_cast<uint2*>(dst + tile_slot(16 * tt + c16, fl >> 3, cpr) * 16 + (fl & 7) * 2) = pk;
          }
        }
      }

      // ---- this wave's proj weight rows [16w, 16w + 16), all k-steps ---------
      // (issued before the next window's loads, so waiting for them never
      // waits for those)
      uint4 wp[kKS];
#pragma unroll
      for (int ks = 0; ks < kKS; ++ks) wp[ks] = weight_frag<C>(p.w_proj, p.packed, wave, ks, lane_i);
      __syncthreads();  // q, k, v complete; xn is dead
      if (next < p.units) fetch_window<cpr, kWaves>(p, nxt, xn, wave, lane_i);

      // ---- attention: head wave/2, query half wave%2; O over Q ---------------
      {
        const int head = wave >> 1;
        const WindowMaskState m = block_mask_state(p, cur);
        tile_attention_wave<32, cpr>(qs, ks, vs, head, wave & 1, p.a, m, tabs + head * kTableMax, lane_i);
      }
      __syncthreads();  // O complete

      // ---- proj features [16w, 16w + 16) + residual, in place over xr ----------
      {
        f32x4 acc[4];
        const f32x4 b = p.b_proj != nullptr ? load_f32x4(p.b_proj + 16 * wave + 4 * g)
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt] = b;
#pragma unroll
        for (int ks = 0; ks < kKS; ++ks) {
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const uint4 of =
                *reinterpret_cast<const uint4*>(qs + ((16 * tt + c16) * cpr + ((4 * ks + g) ^ sw)) * 16);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wp[ks]),
                                                              __builtin_bit_cast(bf16x8, of), acc[tt], 0, 0, 0);
          }
        }
        const int fb = 16 * wave + 4 * g;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          residual_add4(xr + tile_slot(16 * tt + c16, fb >> 3, cpr) * 16 + (fb & 7) * 2, acc[tt]);
      }
      __syncthreads();  // output rows complete in xr
    } else if (next < p.units) {
      fetch_window<cpr, kWaves>(p, nxt, xn, wave, lane);
    }

    store_window<cpr, nthreads>(p, cur, xr, tid);
    if (next >= p.units) break;
    unit = next;
    cur = nxt;
    par ^= 1;
  }
}

// ============================================================================
// swin_block_kernel: one wave per head (12 heads, C = 384)
// ============================================================================

template <int kH>
constexpr int block_lds_bytes() {
  return 3 * 64 * 32 * kH * 2 + kH * kTableMax * 4 + 2 * 32 * kH * 4;
}

template <int kH>
__global__ __launch_bounds__(64 * kH) __attribute__((amdgpu_waves_per_eu(3, 3)))
void swin_block_kernel(const BlockParams p) {
  constexpr int C = 32 * kH;
  constexpr int cpr = C / 8;                 // 16-byte chunks per token row
  constexpr int nthreads = 64 * kH;
  constexpr int tile = 64 * C * 2;
  constexpr int kKS = C / 32;                // 32-channel MFMA k-steps
  static_assert(cpr % 8 == 0, "rows must be whole groups of 8 chunks (swizzle)");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* xbuf = smem;                      // 2 x [64][C]: raw rows of this and the next window
  uint8_t* xn = smem + 2 * tile;
  float* tabs = reinterpret_cast<float*>(smem + 3 * tile);
  float* s_gamma = tabs + kH * kTableMax;
  float* s_beta = s_gamma + C;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  int unit = blockIdx.x;
  if (unit >= p.units) return;  // uniform across the workgroup
  stage_tables<kH, nthreads>(p, tabs, s_gamma, s_beta, tid);

  UnitLoc cur = locate(p, unit);
  int par = 0;
  fetch_window<cpr, kH>(p, cur, xbuf, wave, lane);

  for (;;) {
    // This window's rows have landed (nothing else is in flight); the
    // barrier also orders the previous window's output reads of the other
    // buffer before the next fetch overwrites it.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint8_t* xr = xbuf + par * tile;
    uint8_t* xr_next = xbuf + (par ^ 1) * tile;
    const int next = unit + (int)gridDim.x;
    UnitLoc nxt = cur;
    if (next < p.units) nxt = locate(p, next);

    if (cur.computed) {  // uniform across the workgroup
      // Lane-derived addresses are recomputed per window rather than held in
      // registers across the persistent loop.
      int lane_i = lane;
      asm volatile("" : "+v"(lane_i));
      const int g = lane_i >> 4, c16 = lane_i & 15;
      const int tid_i = wave * 64 + lane_i;
      layernorm_window<cpr, nthreads>(p, cur, xr, xn, s_gamma, s_beta, tid_i);
      __syncthreads();
      // ---- q, k, v of head `wave` for the 64 tokens ------------------------
      const int h = wave;
      f32x4 qa[2][4], ka[2][4], va[4][2];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const int fq = 32 * h + 16 * dt + 4 * g;
        const f32x4 bq = p.b_qkv != nullptr ? load_f32x4(p.b_qkv + fq) : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 bk = p.b_qkv != nullptr ? load_f32x4(p.b_qkv + C + fq) : f32x4{0.f, 0.f, 0.f, 0.f};
        const float bv = p.b_qkv != nullptr ? p.b_qkv[2 * C + 32 * h + 16 * dt + c16] : 0.f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          qa[dt][tt] = bq;
          ka[dt][tt] = bk;
          va[tt][dt] = f32x4{bv, bv, bv, bv};
        }
      }
      {
        const int sw = (c16 >> 1) & 7;
#pragma unroll 1
        for (int ks = 0; ks < kKS; ++ks) {
          uint4 fq[2], fk[2], fv[2], xf[4];
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            fq[dt] = weight_frag<C>(p.w_qkv, p.packed, 2 * h + dt, ks, lane_i);
            fk[dt] = weight_frag<C>(p.w_qkv, p.packed, C / 16 + 2 * h + dt, ks, lane_i);
            fv[dt] = weight_frag<C>(p.w_qkv, p.packed, C / 8 + 2 * h + dt, ks, lane_i);
          }
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            xf[tt] = *reinterpret_cast<const uint4*>(
                xn + ((16 * tt + c16) * cpr + ((4 * ks + g) ^ sw)) * 16);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const bf16x8 x8 = __builtin_bit_cast(bf16x8, xf[tt]);
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
              qa[dt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fq[dt]), x8,
                                                                   qa[dt][tt], 0, 0, 0);
              ka[dt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fk[dt]), x8,
                                                                   ka[dt][tt], 0, 0, 0);
              va[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, __builtin_bit_cast(bf16x8, fv[dt]),
                                                                   va[tt][dt], 0, 0, 0);
            }
          }
        }
      }
      // Next window's rows stream in behind the q/k/v loads (the attention
      // phase issues no vector-memory loads of its own).
      if (next < p.units) fetch_window<cpr, kH>(p, nxt, xr_next, wave, lane_i);
      uint4 kf[4][1], qf[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        kf[tt][0] = pack_frag(ka[0][tt], ka[1][tt]);
        qf[tt] = pack_frag(qa[0][tt], qa[1][tt]);
      }
      uint4 vf[2][2];  // [ct][js]
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int js = 0; js < 2; ++js) vf[ct][js] = pack_frag(va[2 * js][ct], va[2 * js + 1][ct]);
      // Materialise the packed fragments here so that the fp32 accumulators die.
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        asm volatile("" : "+v"(kf[tt][0].x), "+v"(kf[tt][0].y), "+v"(kf[tt][0].z), "+v"(kf[tt][0].w));
        asm volatile("" : "+v"(qf[tt].x), "+v"(qf[tt].y), "+v"(qf[tt].z), "+v"(qf[tt].w));
      }
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int js = 0; js < 2; ++js)
          asm volatile("" : "+v"(vf[ct][js].x), "+v"(vf[ct][js].y), "+v"(vf[ct][js].z), "+v"(vf[ct][js].w));
      __syncthreads();  // every wave has read xn; O overwrites it

      // ---- attention of head h ----------------------------------------------
      {
        const WindowMaskState m = block_mask_state(p, cur);
        LaneGeom<true> lg;
        lane_geom_init<true>(lg, p.a, m, tabs + h * kTableMax, lane);
        auto vsrc = [&](int ct, int js) -> bf16x8 { return __builtin_bit_cast(bf16x8, vf[ct][js]); };
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const uint4 qp[2][1] = {{qf[2 * half]}, {qf[2 * half + 1]}};
          f32x4 s[2][4];
          scores_pair<true, 32>(s, kf, qp);
          float inv[2];
          softmax_half<true, false>(s, inv, half, p.a, m, lg, nullptr, lane);
          f32x4 o[2][2];
          pv_half<true, 32>(o, s, lane, vsrc);
#pragma unroll
          for (int il = 0; il < 2; ++il) {
            const int i = 16 * (2 * half + il) + c16;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
              const f32x4 v = o[ct][il] * inv[il];
              const int cc = 32 * h + 16 * ct + 4 * g;
              uint2 pk;
              pk.x = pack_bf16x2(v[0], v[1]);
              pk.y = pack_bf16x2(v[2], v[3]);
              *reinterpret_cast<uint2*>(xn + tile_slot(i, cc >> 3, cpr) * 16 + (cc & 7) * 2) = pk;
            }
          }
        }
      }
      __syncthreads();  // O complete

      // ---- projection features [32h, 32h+32) + residual ----------------------
      {
        const int f0 = 32 * h;
        f32x4 ya[2][4];
#pragma unroll
        for (int ft = 0; ft < 2; ++ft) {
          const f32x4 bp = p.b_proj != nullptr ? load_f32x4(p.b_proj + f0 + 16 * ft + 4 * g)
                                               : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) ya[ft][tt] = bp;
        }
        const int sw = (c16 >> 1) & 7;
#pragma unroll 2
        for (int ks = 0; ks < kKS; ++ks) {
          uint4 fp[2], of[4];
#pragma unroll
          for (int ft = 0; ft < 2; ++ft) fp[ft] = weight_frag<C>(p.w_proj, p.packed, f0 / 16 + ft, ks, lane_i);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            of[tt] = *reinterpret_cast<const uint4*>(
                xn + ((16 * tt + c16) * cpr + ((4 * ks + g) ^ sw)) * 16);
#pragma unroll
          for (int ft = 0; ft < 2; ++ft)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              ya[ft][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fp[ft]),
                                                                   __builtin_bit_cast(bf16x8, of[tt]),
                                                                   ya[ft][tt], 0, 0, 0);
        }
        // Y^T lane (c, g) element r: feature f0 + 16ft + 4g + r of token 16tt + c.
#pragma unroll
        for (int ft = 0; ft < 2; ++ft) {
          const int fb = f0 + 16 * ft + 4 * g;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            residual_add4(xr + tile_slot(16 * tt + c16, fb >> 3, cpr) * 16 + (fb & 7) * 2, ya[ft][tt]);
          }
        }
      }
      __syncthreads();  // output rows complete in xr
    } else if (next < p.units) {
      fetch_window<cpr, kH>(p, nxt, xr_next, wave, lane);
    }


    store_window<cpr, nthreads>(p, cur, xr, tid);
    if (next >= p.units) break;
    unit = next;
    cur = nxt;
    par ^= 1;
  }
}

template <class K>
int launch_persistent(K kernel, int threads, int lds, int units, const BlockParams& p, hipStream_t s,
                      int* resident) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(TERRA_ERR_LAUNCH, "no current HIP device");
  if (resident[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the block kernel grid for this device");
    resident[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  const int blocks = units < resident[dev] ? units : resident[dev];
  kernel<<<blocks, threads, lds, s>>>(p);
  return TERRA_OK;
}

// The >64 KiB dynamic-LDS opt-in is a per-kernel attribute: set once each.
template <int kH>
int launch_block(const BlockParams& p, hipStream_t s) {
  static int resident[64] = {0};
  if constexpr (kH == 6) {
    constexpr int lds = block_tile_lds_bytes<kH>();
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&swin_block_tile_kernel<kH>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
    return launch_persistent(swin_block_tile_kernel<kH>, 128 * kH, lds, p.units, p, s, resident);
  } else {
    constexpr int lds = block_lds_bytes<kH>();
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&swin_block_kernel<kH>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
    return launch_persistent(swin_block_kernel<kH>, 64 * kH, lds, p.units, p, s, resident);
  }
}

// packed[(rt * K/32 + ks) * 64 + lane] (16 bytes) = w[16 rt + lane%16][32 ks
// + 8 (lane/16) .. + 8]: one thread per 16-byte fragment chunk.
__global__ __launch_bounds__(256) void pack_linear_kernel(const uint4* __restrict__ w, uint4* __restrict__ packed,
                                                          uint32_t chunks, int k_chunks) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= chunks) return;
  const uint32_t lane = i & 63u, blk = i >> 6;
  const uint32_t ksteps = (uint32_t)k_chunks / 4u;
  const uint32_t rt = blk / ksteps, ks = blk - rt * ksteps;
  const uint32_t row = 16u * rt + (lane & 15u), col_chunk = 4u * ks + (lane >> 4);
  packed[i] = w[(uint64_t)row * (uint32_t)k_chunks + col_chunk];
}

bool ranges_overlap(const void* a, const void* b, int64_t bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)bytes && y < x + (uintptr_t)bytes;
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_block_fwd(const void* x, void* y, int dtype, const terra_swin_block_desc* desc,
                                    const float* ln_gamma, const float* ln_beta, const void* qkv_weight,
                                    const float* qkv_bias, const void* proj_weight, const float* proj_bias,
                                    const float* bias_table, const uint64_t* land_bits, void* stream) {
  clear_error();
  if (desc == nullptr) return fail(TERRA_ERR_NULL, "desc is NULL");
  if (x == nullptr || y == nullptr || qkv_weight == nullptr || proj_weight == nullptr)
    return fail(TERRA_ERR_NULL, "x, y, qkv_weight and proj_weight must be non-NULL");
  if (dtype_size(dtype) == 0) return fail(TERRA_ERR_DTYPE, "unknown dtype %d", dtype);
  if (dtype != TERRA_DTYPE_BF16) return fail(TERRA_ERR_UNSUPPORTED, "the fused block kernel is bf16 only");
  const terra_swin_block_desc& d = *desc;
  GeomDims dims;
  const int st = validate_geom(&d.geom, &dims);
  if (st != TERRA_OK) return st;
  const terra_swin_geom& q = d.geom;
  if (q.window != 8) return fail(TERRA_ERR_UNSUPPORTED, "the fused block kernel needs 8x8 windows (got %d)", q.window);
  if (d.heads != 6 && d.heads != 12)
    return fail(TERRA_ERR_UNSUPPORTED, "the fused block kernel supports 6 or 12 heads (got %d)", d.heads);
  if (q.channels != 32 * d.heads)
    return fail(TERRA_ERR_UNSUPPORTED, "the fused block kernel needs head dim 32 (channels %d, heads %d)",
                q.channels, d.heads);
  if (d.layernorm != 0 && !(d.ln_eps >= 0.f))
    return fail(TERRA_ERR_SHAPE, "ln_eps must be a non-negative number");
  if (land_bits != nullptr && d.land_windows <= 0)
    return fail(TERRA_ERR_SHAPE, "land_windows must be positive when land_bits is given");
  for (const void* ptr : {x, (const void*)y, qkv_weight, proj_weight, (const void*)ln_gamma, (const void*)ln_beta,
                          (const void*)qkv_bias, (const void*)proj_bias}) {
    if (((uintptr_t)ptr & 15u) != 0) return fail(TERRA_ERR_ALIGN, "tensors must be 16-byte aligned");
  }
  if (((uintptr_t)bias_table & 3u) != 0 || ((uintptr_t)land_bits & 7u) != 0)
    return fail(TERRA_ERR_ALIGN, "bias_table / land_bits misaligned");
  const int64_t tokens = (int64_t)q.batch * q.height * q.width;
  const int64_t bytes = tokens * q.channels * 2;
  if (x != y && ranges_overlap(x, y, bytes)) return fail(TERRA_ERR_SHAPE, "y overlaps x without being x");
  const int64_t frame_windows = dims.nWh * dims.nWw;
  const int64_t units = (int64_t)q.batch * frame_windows;
  if (units >= (1ll << 31) || tokens >= (1ll << 31) || (int64_t)q.batch * dims.nWe >= (1ll << 31))
    return fail(TERRA_ERR_SHAPE, "grid too large for one launch; split the batch");

  BlockParams p;
  memset(&p, 0, sizeof(p));
  p.a.scale_l2e = d.scale * kLog2e;
  p.a.mask_l2e = d.mask_value * kLog2e;
  p.a.frame_h = (int32_t)dims.Hp;
  p.a.frame_w = (int32_t)dims.Wp;
  p.a.shift_h = q.shift_h;
  p.a.shift_w = q.shift_w;
  p.a.window_h = p.a.window_w = 8;
  p.a.N = p.a.n_geo = p.a.n_real = 64;
  p.x = static_cast<const uint8_t*>(x);
  p.y = static_cast<uint8_t*>(y);
  p.gamma = ln_gamma;
  p.beta = ln_beta;
  p.w_qkv = static_cast<const uint16_t*>(qkv_weight);
  p.b_qkv = qkv_bias;
  p.w_proj = static_cast<const uint16_t*>(proj_weight);
  p.b_proj = proj_bias;
  p.bias_table = bias_table;
  p.land_bits = land_bits;
  p.land_windows = land_bits != nullptr ? d.land_windows : 1;
  p.packed = d.packed_weights != 0;
  p.layernorm = d.layernorm != 0;
  p.shift_mask = d.shift_mask != 0;
  p.eps = d.ln_eps;
  p.inv_c = 1.f / (float)q.channels;
  p.H = q.height;
  p.W = q.width;
  p.Hp = (int32_t)dims.Hp;
  p.Wp = (int32_t)dims.Wp;
  p.shift_h = q.shift_h;
  p.shift_w = q.shift_w;
  p.pad_top = q.pad_top;
  p.pad_left = q.pad_left;
  p.nWw = (int32_t)dims.nWw;
  p.win_row_begin = q.win_row_begin;
  p.win_rows = (int32_t)dims.rows;
  p.valid_begin = q.valid_end > 0 ? q.valid_begin : 0;
  p.valid_end = q.valid_end > 0 ? q.valid_end : 0;
  p.nWe = (int32_t)dims.nWe;
  p.units = (int32_t)units;
  p.fd_frame = FastDiv((uint32_t)frame_windows);
  p.fd_nWw = FastDiv((uint32_t)dims.nWw);

  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int ls = d.heads == 6 ? launch_block<6>(p, s) : launch_block<12>(p, s);
  if (ls != TERRA_OK) return ls;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "block kernel launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}

extern "C" int terra_swin_pack_linear(const void* weight, void* packed, int dtype, int out_features,
                                      int in_features, void* stream) {
  clear_error();
  if (weight == nullptr || packed == nullptr) return fail(TERRA_ERR_NULL, "weight and packed must be non-NULL");
  if (dtype_size(dtype) == 0) return fail(TERRA_ERR_DTYPE, "unknown dtype %d", dtype);
  if (dtype != TERRA_DTYPE_BF16) return fail(TERRA_ERR_UNSUPPORTED, "fragment packing is bf16 only");
  if (out_features <= 0 || in_features <= 0 || out_features % 16 != 0 || in_features % 32 != 0)
    return fail(TERRA_ERR_SHAPE, "weight [%d, %d] must be a multiple of [16, 32]", out_features, in_features);
  if ((((uintptr_t)weight) & 15u) != 0 || (((uintptr_t)packed) & 15u) != 0)
    return fail(TERRA_ERR_ALIGN, "weight and packed must be 16-byte aligned");
  const int64_t bytes = (int64_t)out_features * in_features * 2;
  if (bytes / 16 >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "weight too large");
  if (ranges_overlap(weight, packed, bytes)) return fail(TERRA_ERR_SHAPE, "packed overlaps weight");
  const uint32_t chunks = (uint32_t)(bytes / 16);
  pack_linear_kernel<<<(chunks + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(weight), static_cast<uint4*>(packed), chunks, in_features / 8);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "pack launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
