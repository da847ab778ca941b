// Fused Swin attention half-block forward for gfx950: bf16 activations,
// 8x8 windows; 6 or 12 heads of dim 32 (C = 192, 384) or 12 heads of dim 64
// (C = 768).
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
// The kernels are persistent over windows and keep every [64][C] bf16 tile in
// LDS with 16-byte chunks XOR-swizzled per row.  A window's raw rows arrive by
// direct global -> LDS loads issued while earlier windows are computed; at
// C <= 384 they stay in LDS for the residual add and are overwritten by the
// output rows, which are streamed back to the grid.
//
// A wave computes a (window, head) unit: for all 64 tokens,
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
// and v never leave registers.  O goes through LDS (all heads of a token are
// the proj input), and the projection runs as Y^T = W_p O^T over row tiles of
// output features.
//
// swin_block_dw_kernel (6 heads, C = 192, the benchmark shape): a pair of
// windows at a time, eight waves, three (window, head) units per SIMD.
//
// swin_block_kernel (12 heads, C = 384): one wave per head, one window at a
// time.
//
// swin_block_hd64_kernel (12 heads of dim 64, C = 768): one window at a time,
// eight waves, three heads per SIMD.
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
  int32_t land_shortcut;     // all-land windows may run unmasked (finite, moderate mask_value)
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

// This lane's index in its wave, computed where it is used: a volatile asm
// is neither hoisted out of a loop nor merged with another call, so a
// persistent loop does not hold the value (or spill it) across its body.
__device__ __forceinline__ int lane_index() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// The 16-byte A/B-operand fragment of weight rows [16*rt, 16*rt + 16),
// input channels [32*ks, 32*ks + 32) for this lane (row rt*16 + lane%16,
// channels 32ks + 8*(lane/16) ..): strided rows of the nn.Linear layout, or
// one contiguous 1 KB block per (rt, ks) in the packed layout.  The packed
// form is a buffer load: the wave-uniform block offset in an SGPR (the low two
// k-step bits in the lane offset), so no per-lane 64-bit address is formed or
// held per fragment (that alone took the c3 kernel from 284 to 268 us).
template <int kC, bool kPacked>
__device__ __forceinline__ uint4 weight_frag(const uint16_t* w, int rt, int ks, int lane) {
  if constexpr (kPacked) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(w, 0xffffffffu);  // offsets are in range by construction
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)lane * 16u + (uint32_t)(ks & 3) * 1024u,
                                                          (rt * (kC / 32) + (ks & ~3)) * 1024, 0);
    return __builtin_bit_cast(uint4, v);
  }
  else
    return *reinterpret_cast<const uint4*>(w + (int64_t)(16 * rt + (lane & 15)) * kC + 32 * ks + 8 * (lane >> 4));
}

// Mask terms of an emitted window (shift regions over the padded frame, land
// keys of the slab window).
__device__ __forceinline__ WindowMaskState block_mask_state(const BlockParams& p, const UnitLoc u) {
  WindowMaskState m;
  m.wr = u.wr;
  m.wc = u.wc;
  m.use_shift = p.shift_mask && ((u.wr + 2) * p.a.window_h > p.Hp || (u.wc + 2) * p.a.window_w > p.Wp);
  // The land word through the scalar (constant) path: a vector load would be
  // waited for together with the next window's rows in flight.
  m.land = p.land_bits != nullptr
               ? ((const __attribute__((address_space(4))) uint64_t*)
                      p.land_bits)[__builtin_amdgcn_readfirstlane(u.w_slab % p.land_windows)]
               : 0ull;
  // Every key of a window on land, and no shift boundary: the mask adds the
  // same constant to every score, which the softmax cancels, so the window
  // runs unmasked (22 % of c3's windows).  Only for a finite mask value of
  // at most 2^12 in magnitude (land_shortcut, set on the host): a larger one
  // swamps the fp32 scores it is added to (the reference then gives uniform
  // weights), and -inf gives NaN rows.
  const uint64_t keys = p.a.n_geo >= 64 ? ~0ull : (1ull << p.a.n_geo) - 1ull;
  if (p.land_shortcut && !m.use_shift && (m.land & keys) == keys) m.land = 0ull;
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
    dma_to_lds16(src, __builtin_amdgcn_readfirstlane(lds_address(dst + blk * 1024)));
  }
}

// LayerNorm of the window rows xr -> xn (bf16).  Eight lanes own a token;
// lane `sub` holds chunks sub + 8k, k < cpr/8.  fp32 statistics from bf16 dot
// products over the packed rows (Bf16Moments, token_stats8; the variance is
// recomputed from centred values where the mean is large against the
// spread), then y = (x rstd - mean rstd) gamma + beta (two FMAs per value,
// rstd = rsqrt(var + eps)) rounded once; the rows are read from LDS once for
// the statistics and once for the output.  Frame-padding tokens get zeros.
// With p.layernorm == 0 the rows are copied.
template <int kCpr, int kThreads>
__device__ __forceinline__ void layernorm_window(const BlockParams& p, const UnitLoc u, const uint8_t* xr,
                                                 uint8_t* xn, const float* s_gamma, const float* s_beta, int tid) {
  constexpr int kTokPass = kThreads / 8;
  constexpr int kCPL = kCpr / 8;
  const int sub = tid & 7;
  auto raw = [&](int t, int k) { return *reinterpret_cast<const uint4*>(xr + tile_slot(t, sub + 8 * k, kCpr) * 16); };
  for (int t = tid >> 3; t < 64; t += kTokPass) {  // uniform per wave
    const bool in = grid_token(p, u, t >> 3, t & 7) >= 0;
    if (!p.layernorm) {
#pragma unroll
      for (int k = 0; k < kCPL; ++k)
        *reinterpret_cast<uint4*>(xn + tile_slot(t, sub + 8 * k, kCpr) * 16) =
            in ? raw(t, k) : make_uint4(0u, 0u, 0u, 0u);
      continue;
    }
    Bf16Moments m;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) m.add4(raw(t, k));
    float mean, var;
    token_stats8(m, p.inv_c, mean, var);
    if (token_stats_recheck(mean, var)) {  // uniform per wave
      asm volatile("" : "+v"(mean));  // keeps this rare pass a branch, not computed on every path
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) sq = centred_sq4(raw(t, k), mean, sq);
      var = group8_sum(sq) * p.inv_c;
    }
    const float rstd = rsqrtf(fmaxf(var, 0.f) + p.eps);
    const float nmr = -mean * rstd;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const int c0 = (sub + 8 * k) * 8;
      const float4 gm0 = *reinterpret_cast<const float4*>(s_gamma + c0);
      const float4 gm1 = *reinterpret_cast<const float4*>(s_gamma + c0 + 4);
      const float4 bt0 = *reinterpret_cast<const float4*>(s_beta + c0);
      const float4 bt1 = *reinterpret_cast<const float4*>(s_beta + c0 + 4);
      const float gm[8] = {gm0.x, gm0.y, gm0.z, gm0.w, gm1.x, gm1.y, gm1.z, gm1.w};
      const float bt[8] = {bt0.x, bt0.y, bt0.z, bt0.w, bt1.x, bt1.y, bt1.z, bt1.w};
      const uint4 o = normalize_chunk(raw(t, k), rstd, nmr, gm, bt);
      *reinterpret_cast<uint4*>(xn + tile_slot(t, sub + 8 * k, kCpr) * 16) = in ? o : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// y_w rows (xr) -> the grid tokens they were gathered from; consecutive
// lanes store consecutive chunks of a row.  Frame-padding rows are dropped.
template <int kCpr, int kThreads>
__device__ __forceinline__ void store_window(const BlockParams& p, const UnitLoc u, const uint8_t* xr, int tid) {
  constexpr int kRowStep = kThreads / kCpr;
  static_assert(kRowStep * kCpr == kThreads && 64 % kRowStep == 0, "whole rows per pass");
  const int row0 = tid / kCpr, ch0 = tid - row0 * kCpr;
  // Token offsets are image-relative (grid_token), and an image is < 4 GiB.
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(p.y + (int64_t)u.b * p.H * p.W * (kCpr * 16), (uint32_t)((int64_t)p.H * p.W * (kCpr * 16)));
#pragma unroll
  for (int r = 0; r < 64 / kRowStep; ++r) {
    const int row = row0 + kRowStep * r;
    const int t = grid_token(p, u, row >> 3, row & 7);
    if (t >= 0) {
      const u32x4 val =
          __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(xr + tile_slot(row, ch0, kCpr) * 16));
      stream_store_sc1(val, out, (uint32_t)(t - u.b * p.H * p.W) * (kCpr * 16) + ch0 * 16);
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
                                             int tid, float* s_bqkv = nullptr, float* s_bproj = nullptr) {
  constexpr int C = 32 * kH;
  if (s_bqkv != nullptr) {  // linear biases (zeros when absent)
    for (int c = tid; c < 3 * C; c += kThreads) s_bqkv[c] = p.b_qkv != nullptr ? p.b_qkv[c] : 0.f;
    for (int c = tid; c < C; c += kThreads) s_bproj[c] = p.b_proj != nullptr ? p.b_proj[c] : 0.f;
  }
  for (int e = tid; e < kH * kTableMax; e += kThreads) {
    const int h = e / kTableMax, i = e - h * kTableMax;
    const int ri = kTableRev - i;  // reversed column (lane_bias_rev)
    tabs[e] = (p.bias_table != nullptr && ri < 225) ? p.bias_table[ri * kH + h] * kLog2e : 0.f;
  }
  for (int c = tid; c < C; c += kThreads) {
    s_gamma[c] = p.gamma != nullptr ? p.gamma[c] : 1.f;
    s_beta[c] = p.beta != nullptr ? p.beta[c] : 0.f;
  }
}

// ============================================================================
// Per-head phases: one wave owns head h (features [32h, 32h + 32)) of a window
// whose LayerNorm output is in `xn`.
// ============================================================================

// q, k, v of head h for the 64 tokens, straight into MFMA operand fragments:
// kf4[jt] (K rows of key tile jt), vf[ct][js] (V^T operand), qf[it] (Q^T
// operand, carrying scale * log2e).  The three projections run one after the
// other (32 accumulators live) as one stream of 3 * C/32 k-steps whose weight
// fragments flow through a ring kDepth steps deep, so each load has kDepth - 1
// steps of MFMA work to arrive; the compiler barrier at each step keeps the
// scheduler from hoisting further loads (register pressure).  `bqkv` is the
// bias (NULL: none).  From LDS it costs no wait on the weight loads in flight;
// from global memory the first MFMA of each pass waits for it, and with it
// for every weight fragment already requested (vmcnt counts in order).
template <int C, bool kPacked>
__device__ __forceinline__ void head_qkv(const BlockParams& p, const uint8_t* xn, int h, int lane, uint4 (&kf4)[4],
                                         uint4 (&vf)[2][2], uint4 (&qf)[4], const float* bqkv) {
  constexpr int cpr = C / 8, kKS = C / 32;
  constexpr int kSteps = 3 * kKS;
  constexpr int kDepth = C <= 192 ? 3 : 2;  // weight ring depth (registers)
  const int g = lane >> 4, c16 = lane & 15;
  const int sw = (c16 >> 1) & 7;
  // Pass 0: K^T (rows = features), pass 1: V (rows = tokens), pass 2: Q^T.
  auto row_tile0 = [&](int pass) { return pass == 0 ? C / 16 + 2 * h : (pass == 1 ? C / 8 + 2 * h : 2 * h); };
  auto bias0 = [&](int pass) { return pass == 0 ? C + 32 * h : (pass == 1 ? 2 * C + 32 * h : 32 * h); };
  // xn row address of token tile tt, k-step ks (tile_slot swizzle): the XOR
  // only touches the low 3 bits, so even / odd k-steps share a base.
  // For C > 192 the offsets are 32-bit LDS addresses, so that the k-step part
  // folds into the instruction's immediate offset: at 12 k-steps per pass the
  // per-k-step addresses were otherwise kept in (spilled) registers (c5
  // 547 -> 456 us).  At C = 192 the generic form is faster (274 against 354 us).
  constexpr bool kLds32 = C > 192;
  uint32_t xoff[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      xoff[e][tt] = (kLds32 ? lds_address(xn) : 0u) + ((16 * tt + c16) * cpr + ((4 * e + g) ^ sw)) * 16;
  auto xn_frag = [&](int tt, int ks) -> uint4 {
    if constexpr (kLds32)
      return __builtin_bit_cast(uint4, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                                           (uintptr_t)(xoff[ks & 1][tt] + (ks >> 1) * 128)));
    else
      return *reinterpret_cast<const uint4*>(xn + xoff[ks & 1][tt] + (ks >> 1) * 128);
  };
  uint4 ring[kDepth][2];
#pragma unroll
  for (int st = 0; st < kDepth - 1; ++st)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
      ring[st][dt] = weight_frag<C, kPacked>(p.w_qkv, row_tile0(st / kKS) + dt, st % kKS, lane);
  uint4 xf[2][4];  // xn fragments of this and the next k-step
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) xf[0][tt] = xn_frag(tt, 0);
  f32x4 acc[2][4];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const int pass = st / kKS, ks = st % kKS;
    // Loads of later steps first (weights kDepth - 1 ahead, xn one ahead),
    // then this step's MFMAs; the compiler barrier keeps further loads from
    // being hoisted above this step (register pressure).
    if (st + kDepth - 1 < kSteps) {
      const int nst = st + kDepth - 1;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
        ring[nst % kDepth][dt] = weight_frag<C, kPacked>(p.w_qkv, row_tile0(nst / kKS) + dt, nst % kKS, lane);
    }
    if (st + 1 < kSteps) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) xf[(st + 1) & 1][tt] = xn_frag(tt, (st + 1) % kKS);
    }
    asm volatile("" ::: "memory");
    if (ks == 0) {  // accumulators start at the bias
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        f32x4 b = f32x4{0.f, 0.f, 0.f, 0.f};
        if (bqkv != nullptr) {
          // Buffer loads (a 32-bit lane offset against a scalar descriptor):
          // 64-bit per-lane bias addresses held across the passes spilled.
          const __amdgpu_buffer_rsrc_t br = buffer_rsrc(bqkv, 3 * C * 4);
          if (pass != 1) {
            b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              br, (uint32_t)(16 * dt + 4 * g) * 4, bias0(pass) * 4, 0));
          } else {
            const float bv = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(br, (uint32_t)(16 * dt + c16) * 4, bias0(pass) * 4, 0));
            b = f32x4{bv, bv, bv, bv};
          }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[dt][tt] = b;
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 x8 = __builtin_bit_cast(bf16x8, xf[st & 1][tt]);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x8 w8 = __builtin_bit_cast(bf16x8, ring[st % kDepth][dt]);
        acc[dt][tt] = pass != 1 ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(w8, x8, acc[dt][tt], 0, 0, 0)
                                : __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, w8, acc[dt][tt], 0, 0, 0);
      }
    }
    if (ks == kKS - 1) {  // pass done: pack into operand fragments
      if (pass == 0) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) kf4[tt] = pack_frag(acc[0][tt], acc[1][tt]);
      } else if (pass == 1) {  // acc[ct][token tile]
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int js = 0; js < 2; ++js) vf[ct][js] = pack_frag(acc[ct][2 * js], acc[ct][2 * js + 1]);
      } else {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) qf[tt] = pack_frag(acc[0][tt] * p.a.scale_l2e, acc[1][tt] * p.a.scale_l2e);
      }
    }
  }
  // Materialise the packed fragments here so that the fp32 accumulators die.
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    asm volatile("" : "+v"(kf4[tt].x), "+v"(kf4[tt].y), "+v"(kf4[tt].z), "+v"(kf4[tt].w));
    asm volatile("" : "+v"(qf[tt].x), "+v"(qf[tt].y), "+v"(qf[tt].z), "+v"(qf[tt].w));
  }
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int js = 0; js < 2; ++js)
      asm volatile("" : "+v"(vf[ct][js].x), "+v"(vf[ct][js].y), "+v"(vf[ct][js].z), "+v"(vf[ct][js].w));
}

// Attention of head h from the register fragments, one query tile at a time;
// O (bf16) goes to columns [32h, 32h + 32) of `o_tile`, or with kHold to
// hold[it][ct] (channels 32h + 16ct + 4g .. + 3 of query 16 it + c).
template <int C, bool kHold = false, int kNQt = 4>
__device__ __forceinline__ void head_attention(const BlockParams& p, const UnitLoc cur, const float* tab, int h,
                                               int lane, const uint4 (&kf4)[4], const uint4 (&vf)[2][2],
                                               const uint4 (&qf)[4], uint8_t* o_tile, uint2 (*hold)[2] = nullptr) {
  constexpr int cpr = C / 8;
  const int g = lane >> 4, c16 = lane & 15;
  const WindowMaskState m = block_mask_state(p, cur);
  const float* tabr = lane_bias_rev(tab, lane);
  auto vsrc = [&](int ct, int js) -> bf16x8 { return __builtin_bit_cast(bf16x8, vf[ct][js]); };
  // The four query tiles under one mask mode (a wave-uniform choice per
  // window, outside the loop), kNQt of them through each stage together: the
  // more, the more independent work to overlap the MFMA, exp and cross-lane
  // latencies of a tile (four measured faster than two in the six-head
  // kernel; in the twelve-head kernel two leave its 168 registers unspilled
  // at the same speed).
  auto run = [&](auto mode, const f32x4 (&land_term)[4], uint64_t rid_pack) {
    constexpr int kMask = decltype(mode)::value;
    constexpr int kNQ = kNQt;
#pragma unroll
    for (int it0 = 0; it0 < 4; it0 += kNQ) {
      __builtin_amdgcn_sched_barrier(0);  // kNQ query tiles at a time (register pressure)
      int rid_q[kNQ];
#pragma unroll
      for (int q = 0; q < kNQ; ++q)
        rid_q[q] = kMask == kMaskShift ? 3 * region(cur.wr * 8 + 2 * (it0 + q) + (c16 >> 3), p.Hp, 8, p.shift_h) +
                                             region(cur.wc * 8 + (c16 & 7), p.Wp, 8, p.shift_w)
                                       : 0;
      uint4 qp[kNQ];
#pragma unroll
      for (int q = 0; q < kNQ; ++q) qp[q] = qf[it0 + q];
      f32x4 o[kNQ][2];
      float inv[kNQ];
      attend_qtiles<kMask, kNQ>(o, inv, it0, kf4, qp, tabr, m, land_term, rid_pack, rid_q, p.a.mask_l2e, 1.0f,
                                vsrc);
#pragma unroll
      for (int q = 0; q < kNQ; ++q) {
        const int i = 16 * (it0 + q) + c16;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const f32x4 v = o[q][ct] * inv[q];
          const int cc = 32 * h + 16 * ct + 4 * g;
          uint2 pk;
          pk.x = pack_bf16x2(v[0], v[1]);
          pk.y = pack_bf16x2(v[2], v[3]);
          if constexpr (kHold)
            hold[it0 + q][ct] = pk;
          else
            *reinterpret_cast<uint2*>(o_tile + tile_slot(i, cc >> 3, cpr) * 16 + (cc & 7) * 2) = pk;
        }
      }
    }
  };
  f32x4 land_term[4];  // read by attend_qtiles only when the window has land keys
  if (m.use_shift) {
    uint64_t rid_pack = 0;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        rid_pack |= (uint64_t)(3 * region(cur.wr * 8 + 2 * jt + (g >> 1), p.Hp, 8, p.shift_h) +
                               region(cur.wc * 8 + 4 * (g & 1) + r, p.Wp, 8, p.shift_w))
                    << (4 * (4 * jt + r));
    if (m.land != 0ull) land_terms(land_term, m.land, g, p.a.mask_l2e);
    run(MaskMode<kMaskShift>{}, land_term, rid_pack);
  } else if (m.land != 0ull) {
    land_terms(land_term, m.land, g, p.a.mask_l2e);
    run(MaskMode<kMaskLand>{}, land_term, 0ull);
  } else {
    run(MaskMode<kMaskNone>{}, land_term, 0ull);
  }
}

// Output features [32h, 32h + 32) = O W_p^T + b_p for the 64 tokens
// (Y^T = W_p O^T), rounded to bf16 and added to the raw rows in `xr`.
template <int C, bool kPacked>
__device__ __forceinline__ void head_proj(const BlockParams& p, const uint8_t* o_tile, uint8_t* xr, int h,
                                          int lane, const float* bproj) {
  constexpr int cpr = C / 8, kKS = C / 32;
  const int g = lane >> 4, c16 = lane & 15;
  const int sw = (c16 >> 1) & 7;
  const int f0 = 32 * h;
  f32x4 ya[2][4];
#pragma unroll
  for (int ft = 0; ft < 2; ++ft) {
    const f32x4 bp = bproj != nullptr ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            buffer_rsrc(bproj, C * 4), (uint32_t)(16 * ft + 4 * g) * 4, f0 * 4, 0))
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) ya[ft][tt] = bp;
  }
  constexpr int kDepth = C <= 192 ? 4 : 2;  // weight ring depth (registers)
  constexpr bool kLds32 = C > 192;  // as in head_qkv
  uint32_t ooff[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      ooff[e][tt] = (kLds32 ? lds_address(o_tile) : 0u) + ((16 * tt + c16) * cpr + ((4 * e + g) ^ sw)) * 16;
  auto o_frag = [&](int tt, int ks) -> uint4 {
    if constexpr (kLds32)
      return __builtin_bit_cast(uint4, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                                           (uintptr_t)(ooff[ks & 1][tt] + (ks >> 1) * 128)));
    else
      return *reinterpret_cast<const uint4*>(o_tile + ooff[ks & 1][tt] + (ks >> 1) * 128);
  };
  uint4 fp[kDepth][2];  // [ring slot][ft]
#pragma unroll
  for (int st = 0; st < kDepth - 1 && st < kKS; ++st)
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) fp[st][ft] = weight_frag<C, kPacked>(p.w_proj, f0 / 16 + ft, st, lane);
  uint4 of[2][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) of[0][tt] = o_frag(tt, 0);
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) {
    if (ks + kDepth - 1 < kKS) {
#pragma unroll
      for (int ft = 0; ft < 2; ++ft)
        fp[(ks + kDepth - 1) % kDepth][ft] = weight_frag<C, kPacked>(p.w_proj, f0 / 16 + ft, ks + kDepth - 1, lane);
    }
    if (ks + 1 < kKS) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) of[(ks + 1) & 1][tt] = o_frag(tt, ks + 1);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
      for (int ft = 0; ft < 2; ++ft)
        ya[ft][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fp[ks % kDepth][ft]),
                                                             __builtin_bit_cast(bf16x8, of[ks & 1][tt]), ya[ft][tt],
                                                             0, 0, 0);
    }
  }
  // Y^T lane (c, g) element r: feature f0 + 16ft + 4g + r of token 16tt + c.
#pragma unroll
  for (int ft = 0; ft < 2; ++ft) {
    const int fb = f0 + 16 * ft + 4 * g;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      residual_add4(xr + tile_slot(16 * tt + c16, fb >> 3, cpr) * 16 + (fb & 7) * 2, ya[ft][tt]);
  }
}

// ============================================================================
// swin_block_kernel: one wave per head, one window at a time (12 heads,
// C = 384, whose doubled buffers of the variant below do not fit LDS)
// ============================================================================

template <int kH>
constexpr int block_lds_bytes() {
  return 3 * 64 * 32 * kH * 2 + kH * kTableMax * 4 + 2 * 32 * kH * 4;
}

template <int kH, bool kPacked>
__global__ __launch_bounds__(64 * kH) __attribute__((amdgpu_waves_per_eu(3, 3)))
void swin_block_kernel(const BlockParams p) {
  constexpr int C = 32 * kH;
  constexpr int cpr = C / 8;                 // 16-byte chunks per token row
  constexpr int nthreads = 64 * kH;
  constexpr int tile = 64 * C * 2;
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
  UnitLoc prev = cur;
  bool have_prev = false;
  int par = 0;
  fetch_window<cpr, kH>(p, cur, xbuf, wave, lane);

  // Barriers are LDS-only (lds_barrier): the next window's rows stay in
  // flight from the q/k/v phase to the top of the next iteration, and a
  // window's output rows are stored at the start of the next iteration, so
  // the wait for the rows does not also wait for those stores.
  for (;;) {
    // This window's rows have landed; the barrier also orders the previous
    // window's proj writes before its store below.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    uint8_t* xr = xbuf + par * tile;
    uint8_t* xr_next = xbuf + (par ^ 1) * tile;
    const int next = unit + (int)gridDim.x;
    UnitLoc nxt = cur;
    if (next < p.units) nxt = locate(p, next);
    nxt.computed = __builtin_amdgcn_readfirstlane(nxt.computed);  // a scalar, not a lane register
    // Lane-derived addresses are recomputed per window rather than held in
    // registers across the persistent loop (the lane index itself included).
    const int lane_i = lane_index();
    const int tid_i = wave * 64 + lane_i;
    if (have_prev) store_window<cpr, nthreads>(p, prev, xr_next, tid_i);  // the previous window's rows

    if (cur.computed) {  // uniform across the workgroup
      layernorm_window<cpr, nthreads>(p, cur, xr, xn, s_gamma, s_beta, tid_i);
      lds_barrier();     // also: the previous window's rows are read out of xr_next
      uint4 kf4[4], vf[2][2], qf[4];
      head_qkv<C, kPacked>(p, xn, wave, lane_i, kf4, vf, qf, p.b_qkv);
      // Next window's rows stream in behind the q/k/v loads (the attention
      // phase issues no vector-memory loads of its own).
      if (next < p.units) fetch_window<cpr, kH>(p, nxt, xr_next, wave, lane_index());
      lds_barrier();     // every wave has read xn; O overwrites it
      // Two query tiles at a time: four spilled one VGPR at three waves per
      // SIMD (168 registers); two leave none (c5 411-420 -> 410-411 us A/B).
      head_attention<C, false, 2>(p, cur, tabs + wave * kTableMax, wave, lane_i, kf4, vf, qf, xn);
      lds_barrier();     // O complete
      head_proj<C, kPacked>(p, xn, xr, wave, lane_i, p.b_proj);
    } else if (next < p.units) {
      lds_barrier();     // the previous window's rows are read out of xr_next
      fetch_window<cpr, kH>(p, nxt, xr_next, wave, lane_i);
    }
    prev = cur;
    have_prev = true;
    if (next >= p.units) break;
    unit = next;
    cur = nxt;
    par ^= 1;
  }
  lds_barrier();         // output rows complete in the last window's buffer
  store_window<cpr, nthreads>(p, prev, xbuf + par * tile, wave * 64 + lane_index());
}

// ============================================================================
// swin_block_dw_kernel: 6 heads (C = 192, c3), a pair of windows at a time.
// Eight waves, two per SIMD, up to 256 VGPRs each; the 12 (window, head)
// units of a pair split three per SIMD: wave s < 4 owns units 3s and 3s + 1,
// wave s + 4 unit 3s + 2 (unit u = window u / 6, head u % 6).
// ============================================================================
//
// LDS: two row buffers for a pair (pair k's rows, which become its output
// rows; the other buffer holds pair k - 1's output rows, then receives pair
// k + 1's), one LayerNorm buffer that later holds the pair's attention
// output O, and the tables.  Per pair k:
//
//   wait for the pair's rows; LayerNorm -> the LayerNorm buffer (waves
//           4wi .. 4wi + 3 take window wi)
//   barrier
//   wave s < 4: q/k/v of unit 3s (one pass over the window's LayerNorm
//           rows: six row tiles x four token tiles, so each LayerNorm
//           fragment feeds six MFMAs and each weight fragment four), its
//           attention (O kept in registers), q/k/v of unit 3s + 1
//   wave s + 4: pair k - 1's output rows out of the other buffer, then q/k/v
//           and attention of unit 3s + 2 (O kept in registers);
//           pair k - 1's output rows out of the other buffer
//   barrier (every LayerNorm row has been read)
//   pair k + 1's rows into the other buffer (all waves); the held O and unit
//           3s + 1's attention -> the O buffer
//   barrier
//   wave w: output features [48 (w & 3), + 48) of window w >> 2 = O W_p^T +
//           b_p, plus the residual, in place over the window's rows
//
// The tiles use the 384-byte-row swizzle (tile_slot).
namespace dw {
constexpr int kH = 6, kC = 192, kCpr = kC / 8, kKS = kC / 32;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kTile = 64 * kC * 2;  // one window's rows
constexpr int kPair = 2 * kTile;
constexpr int kOffO = 2 * kPair;    // two row buffers, then the LayerNorm / O buffer
constexpr int kOffTabs = kOffO + kPair;
constexpr int kLds = kOffTabs + (kH * kTableMax + kC + kC + 3 * kC + kC) * 4;
static_assert(kLds <= 160 * 1024, "LDS");

// q, k, v of head h for the window's 64 tokens in one pass: accumulator j
// (row tiles: Q^T 2h + j, K^T C/16 + 2h + j - 2, V C/8 + 2h + j - 4) starts
// at the bias; the V tiles are computed as xn W^T (lane holds tokens 4g + r
// of feature c), the others as W xn^T.  The results are packed into the
// operand fragments of head_attention.
template <bool kPacked>
__device__ __forceinline__ void unit_qkv(const BlockParams& p, const uint8_t* xn, int h, int lane, uint4 (&kf4)[4],
                                         uint4 (&vf)[2][2], uint4 (&qf)[4], const float* bqkv) {
  constexpr int kDepth = 4;  // weight ring (registers): loads three k-steps ahead
  const int g = lane >> 4, c16 = lane & 15;
  const int sw = (c16 >> 1) & 7;
  auto rt = [&](int j) { return (j >> 1) * (kC / 16) + 2 * h + (j & 1); };
  f32x4 acc[6][4];
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    f32x4 b;
    if (j < 4) {
      b = load_f32x4(bqkv + (j >> 1) * kC + 32 * h + 16 * (j & 1) + 4 * g);
    } else {
      const float bv = bqkv[2 * kC + 32 * h + 16 * (j & 1) + c16];
      b = f32x4{bv, bv, bv, bv};
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[j][tt] = b;
  }
  uint32_t xoff[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) xoff[e][tt] = ((16 * tt + c16) * kCpr + ((4 * e + g) ^ sw)) * 16;
  auto xn_frag = [&](int tt, int ks) -> uint4 {
    return *reinterpret_cast<const uint4*>(xn + xoff[ks & 1][tt] + (ks >> 1) * 128);
  };
  uint4 ring[kDepth][6];
#pragma unroll
  for (int st = 0; st < kDepth - 1; ++st)
#pragma unroll
    for (int j = 0; j < 6; ++j) ring[st][j] = weight_frag<kC, kPacked>(p.w_qkv, rt(j), st, lane);
  uint4 xf[2][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) xf[0][tt] = xn_frag(tt, 0);
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) {
    if (ks + kDepth - 1 < kKS) {
#pragma unroll
      for (int j = 0; j < 6; ++j)
        ring[(ks + kDepth - 1) % kDepth][j] = weight_frag<kC, kPacked>(p.w_qkv, rt(j), ks + kDepth - 1, lane);
    }
    if (ks + 1 < kKS) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) xf[(ks + 1) & 1][tt] = xn_frag(tt, ks + 1);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 x8 = __builtin_bit_cast(bf16x8, xf[ks & 1][tt]);
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        const bf16x8 w8 = __builtin_bit_cast(bf16x8, ring[ks % kDepth][j]);
        acc[j][tt] = j < 4 ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(w8, x8, acc[j][tt], 0, 0, 0)
                           : __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, w8, acc[j][tt], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    kf4[tt] = pack_frag(acc[2][tt], acc[3][tt]);
    qf[tt] = pack_frag(acc[0][tt] * p.a.scale_l2e, acc[1][tt] * p.a.scale_l2e);
  }
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int js = 0; js < 2; ++js) vf[ct][js] = pack_frag(acc[4 + ct][2 * js], acc[4 + ct][2 * js + 1]);
}

// The weight fragments of proj_rows (row tiles 3 q4 .. 3 q4 + 2, all k-steps).
template <bool kPacked>
__device__ __forceinline__ void proj_weights(const BlockParams& p, int q4, int lane, uint4 (&wf)[kKS][3]) {
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks)
#pragma unroll
    for (int ft = 0; ft < 3; ++ft) wf[ks][ft] = weight_frag<kC, kPacked>(p.w_proj, 3 * q4 + ft, ks, lane);
}

// Output features [48 q4, 48 q4 + 48) of a window = O W_p^T + b_p (Y^T =
// W_p O^T, three row tiles x four token tiles; weights wf from proj_weights),
// then y = bf16(x + bf16(Y)) in place over the window's raw rows.
__device__ __forceinline__ void proj_rows(const uint8_t* o_tile, uint8_t* tile, int q4, int lane,
                                          const float* bproj, const uint4 (&wf)[kKS][3]) {
  const int g = lane >> 4, c16 = lane & 15;
  const int sw = (c16 >> 1) & 7;
  f32x4 ya[3][4];
#pragma unroll
  for (int ft = 0; ft < 3; ++ft) {
    const f32x4 b = load_f32x4(bproj + 48 * q4 + 16 * ft + 4 * g);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) ya[ft][tt] = b;
  }
  uint32_t ooff[2][4];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) ooff[e][tt] = ((16 * tt + c16) * kCpr + ((4 * e + g) ^ sw)) * 16;
  auto o_frag = [&](int tt, int ks) -> uint4 {
    return *reinterpret_cast<const uint4*>(o_tile + ooff[ks & 1][tt] + (ks >> 1) * 128);
  };
  uint4 of[2][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) of[0][tt] = o_frag(tt, 0);
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) {
    if (ks + 1 < kKS) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) of[(ks + 1) & 1][tt] = o_frag(tt, ks + 1);
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int ft = 0; ft < 3; ++ft)
        ya[ft][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[ks][ft]),
                                                             __builtin_bit_cast(bf16x8, of[ks & 1][tt]), ya[ft][tt],
                                                             0, 0, 0);
  }
  // Y^T lane (c, g) element r: feature 48 q4 + 16 ft + 4g + r of token 16 tt + c.
#pragma unroll
  for (int ft = 0; ft < 3; ++ft) {
    const int fb = 48 * q4 + 16 * ft + 4 * g;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      residual_add4(tile + tile_slot(16 * tt + c16, fb >> 3, kCpr) * 16 + (fb & 7) * 2, ya[ft][tt]);
  }
}

// Whether window u's 64 tokens are eight whole 8-token runs of the grid that
// neither wrap nor touch frame padding; base: the grid index of its first
// token (then token r of the window is base + (r >> 3) W + (r & 7)).
__device__ __forceinline__ bool interior(const BlockParams& p, const UnitLoc u, int& base) {
  const int sh0 = u.wr * 8 + p.shift_h - p.pad_top, sw0 = u.wc * 8 + p.shift_w - p.pad_left;
  base = sh0 * p.W + sw0;
  return u.wr * 8 + p.shift_h + 8 <= p.Hp && u.wc * 8 + p.shift_w + 8 <= p.Wp && sh0 >= 0 && sh0 + 8 <= p.H &&
         sw0 >= 0 && sw0 + 8 <= p.W;
}

// (x rstd - mean rstd) gamma + beta of a lane's three chunks of tokens t0 and
// t0 + 32 (w), rounded once, to xn; zeros for a frame-padding token (kAllIn:
// the window has none).
template <bool kAllIn>
__device__ __forceinline__ void layernorm_store(const uint4 (&w)[2][kCpr / 8], const float (&mean)[2],
                                                const float (&rstd)[2], const bool (&in)[2], uint8_t* xn,
                                                const float* s_gamma, const float* s_beta, int t0, int sub) {
#pragma unroll
  for (int k = 0; k < kCpr / 8; ++k) {
    const int c0 = (sub + 8 * k) * 8;
    const float4 gm0 = *reinterpret_cast<const float4*>(s_gamma + c0);
    const float4 gm1 = *reinterpret_cast<const float4*>(s_gamma + c0 + 4);
    const float4 bt0 = *reinterpret_cast<const float4*>(s_beta + c0);
    const float4 bt1 = *reinterpret_cast<const float4*>(s_beta + c0 + 4);
    const float gm[8] = {gm0.x, gm0.y, gm0.z, gm0.w, gm1.x, gm1.y, gm1.z, gm1.w};
    const float bt[8] = {bt0.x, bt0.y, bt0.z, bt0.w, bt1.x, bt1.y, bt1.z, bt1.w};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      uint4 o = normalize_chunk(w[q][k], rstd[q], -mean[q] * rstd[q], gm, bt);
      if (!kAllIn && !in[q]) o = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(xn + tile_slot(t0 + 32 * q, sub + 8 * k, kCpr) * 16) = o;
    }
  }
}

// LayerNorm of a window's rows xr -> xn by 256 threads: eight lanes per token,
// each lane group taking tokens t and t + 32 side by side (two independent
// reduction chains in flight), the values held in registers.  fp32 statistics
// from bf16 dot products (Bf16Moments, token_stats8), recomputed from centred
// values where the mean is large against the spread; y = (x rstd - mean rstd)
// gamma + beta rounded once; frame-padding tokens become zeros; without
// LayerNorm the rows are copied.
__device__ __forceinline__ void layernorm_pair_rows(const BlockParams& p, const UnitLoc u, const uint8_t* xr,
                                                    uint8_t* xn, const float* s_gamma, const float* s_beta,
                                                    int tid) {
  constexpr int kCPL = kCpr / 8;  // 3 chunks per lane
  const int sub = tid & 7, t0 = tid >> 3;
  if (!p.layernorm) {  // rows copied bit for bit, frame padding zeroed
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int t = t0 + 32 * q;
      const bool in = grid_token(p, u, t >> 3, t & 7) >= 0;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) {
        const uint4 raw = *reinterpret_cast<const uint4*>(xr + tile_slot(t, sub + 8 * k, kCpr) * 16);
        *reinterpret_cast<uint4*>(xn + tile_slot(t, sub + 8 * k, kCpr) * 16) = in ? raw : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    return;
  }
  uint4 w[2][kCPL];
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int k = 0; k < kCPL; ++k)
      w[q][k] = *reinterpret_cast<const uint4*>(xr + tile_slot(t0 + 32 * q, sub + 8 * k, kCpr) * 16);
  float mean[2], var[2], rstd[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    Bf16Moments m;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) m.add4(w[q][k]);
    token_stats8(m, p.inv_c, mean[q], var[q]);
  }
  // Both ballots, no short circuit: one uniform branch.
  if ((int)token_stats_recheck(mean[0], var[0]) | (int)token_stats_recheck(mean[1], var[1])) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      asm volatile("" : "+v"(mean[q]));  // keeps this rare pass a branch, not computed on every path
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) sq = centred_sq4(w[q][k], mean[q], sq);
      var[q] = group8_sum(sq) * p.inv_c;
    }
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) rstd[q] = rsqrtf(fmaxf(var[q], 0.f) + p.eps);
  int base;
  bool in[2] = {true, true};
  if (interior(p, u, base)) {  // uniform per wave: no frame padding in the window
    layernorm_store<true>(w, mean, rstd, in, xn, s_gamma, s_beta, t0, sub);
  } else {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int t = t0 + 32 * q;
      in[q] = grid_token(p, u, t >> 3, t & 7) >= 0;
    }
    layernorm_store<false>(w, mean, rstd, in, xn, s_gamma, s_beta, t0, sub);
  }
}

// The 64 rows of window u -> tile, as fetch_window<kCpr, kW> (the same slots
// from the same wave), with the interior fast path.
template <int kW>
__device__ __forceinline__ void fetch_rows(const BlockParams& p, const UnitLoc u, uint8_t* tile, int wv, int lane) {
  int base;
  if (!interior(p, u, base)) {  // uniform per wave
    fetch_window<kCpr, kW>(p, u, tile, wv, lane);
    return;
  }
  constexpr int kRounds = 64 * kCpr / (64 * kW);
  const uint8_t* img = p.x + ((int64_t)u.b * p.H * p.W + base) * (kCpr * 16);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * kW + wv;
    const int sl = blk * 64 + lane;
    const int row = sl / kCpr;
    const int ch = (sl - row * kCpr) ^ ((row >> 1) & 7);
    dma_to_lds16(img + ((row >> 3) * p.W + (row & 7)) * (kCpr * 16) + ch * 16,
                 __builtin_amdgcn_readfirstlane(lds_address(tile + blk * 1024)));
  }
}

// The output rows of a pair's windows (u0, u0 + 1; those < p.units) -> the
// grid tokens they came from, by kW waves (wave index wv); frame-padding rows
// are dropped.  Wave wv reads exactly the LDS slots that fetch_window<kCpr,
// kW> fills from wave wv, so once its own reads have completed a wave may
// load new rows over them with no wait on the other waves.
template <int kW>
__device__ __forceinline__ void store_pair(const BlockParams& p, int u0, const uint8_t* buf, int wv, int lane) {
  constexpr int kRounds = 64 * kCpr / (64 * kW);
  static_assert(kRounds * 64 * kW == 64 * kCpr, "whole wave-rounds of 64 slots");
#pragma unroll
  for (int wi = 0; wi < 2; ++wi) {
    if (u0 + wi >= p.units) continue;
    const UnitLoc u = locate(p, u0 + wi);
    const __amdgpu_buffer_rsrc_t out =
        buffer_rsrc(p.y + (int64_t)u.b * p.H * p.W * (kCpr * 16), (uint32_t)((int64_t)p.H * p.W * (kCpr * 16)));
    int base;
    if (interior(p, u, base)) {  // uniform per wave
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int sl = (r * kW + wv) * 64 + lane;
        const int row = sl / kCpr;
        const int ch = (sl - row * kCpr) ^ ((row >> 1) & 7);
        const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(buf + wi * kTile + sl * 16));
        stream_store_sc1(val, out, (uint32_t)(base + (row >> 3) * p.W + (row & 7)) * (kCpr * 16) + ch * 16);
      }
      continue;
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int sl = (r * kW + wv) * 64 + lane;
      const int row = sl / kCpr;
      const int ch = (sl - row * kCpr) ^ ((row >> 1) & 7);  // the chunk tile_slot places in slot sl
      const int t = grid_token(p, u, row >> 3, row & 7);
      const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(buf + wi * kTile + sl * 16));
      // Frame-padding rows store at the out-of-range marker 0xfffffff0
      // (chosen per element, so no offset wraps back into range) and are dropped.
      stream_store_sc1(val, out, t >= 0 ? (uint32_t)(t - u.b * p.H * p.W) * (kCpr * 16) + ch * 16 : 0xfffffff0u);
    }
  }
}

}  // namespace dw

template <bool kPacked>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void swin_block_dw_kernel(const BlockParams p) {
  using namespace dw;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* obuf = smem + kOffO;
  float* tabs = reinterpret_cast<float*>(smem + kOffTabs);
  float* s_gamma = tabs + kH * kTableMax;
  float* s_beta = s_gamma + kC;
  float* s_bqkv = s_beta + kC;
  float* s_bproj = s_bqkv + 3 * kC;
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int s4 = wave & 3, wwin = wave >> 2;
  const bool two = wave < 4;  // waves 0..3: units 3s, 3s + 1; waves 4..7: unit 3s + 2
  const int pairs = (p.units + 1) >> 1;
  if ((int)blockIdx.x >= pairs) return;  // uniform across the workgroup
  stage_tables<kH, kThreads>(p, tabs, s_gamma, s_beta, tid0, s_bqkv, s_bproj);
  const int n = (pairs - 1 - (int)blockIdx.x) / (int)gridDim.x + 1;
  auto first_unit = [&](int k) { return 2 * ((int)blockIdx.x + k * (int)gridDim.x); };
  {  // the first pair's rows
    const int u0 = first_unit(0);
#pragma unroll
    for (int wi = 0; wi < 2; ++wi)
      if (u0 + wi < p.units) fetch_rows<kWaves>(p, locate(p, u0 + wi), smem + wi * kTile, wave, tid0 & 63);
  }

  for (int k = 0; k < n; ++k) {
    // Lane-derived addresses are recomputed per pair (the thread id passes
    // through an empty asm) rather than hoisted and held across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    uint8_t* rows = smem + (k & 1) * kPair;          // pair k's rows, later its output rows
    uint8_t* other = smem + ((k + 1) & 1) * kPair;   // pair k - 1's output rows, then pair k + 1's rows
    const int u0 = first_unit(k);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the pair's rows
    lds_barrier();
    {
      const int u = u0 + wwin;
      if (u < p.units) {
        const UnitLoc cur = locate(p, u);
        if (cur.computed)
          layernorm_pair_rows(p, cur, rows + wwin * kTile, obuf + wwin * kTile, s_gamma, s_beta,
                              tid & (kThreads / 2 - 1));
      }
    }
    lds_barrier();  // LayerNorm rows ready
    const int ub = 3 * s4 + 1;  // waves 0..3: the unit whose attention follows the barrier
    const int wib = ub >= kH ? 1 : 0, hb = ub - wib * kH;
    const UnitLoc curb = locate(p, u0 + wib);
    const bool onb = two && u0 + wib < p.units && curb.computed;
    uint4 kf4[4], vf[2][2], qf[4];
    // O of the unit whose attention runs before the barrier (unit 3s for
    // waves 0..3, 3s + 2 for waves 4..7), held until the LayerNorm rows are
    // free.
    uint2 oa[4][2];
    const int ua = 3 * s4 + (two ? 0 : 2), wia = ua >= kH ? 1 : 0, ha = ua - wia * kH;
    const UnitLoc cura = locate(p, u0 + wia);
    const bool ona = u0 + wia < p.units && cura.computed;
    // Waves 4..7 store pair k - 1's output rows first, so that on each SIMD
    // their q/k/v overlaps the other wave's attention and their attention
    // the other wave's second q/k/v.
    if (!two && k > 0) store_pair<4>(p, first_unit(k - 1), other, wave - 4, lane);
    if (ona) {
      unit_qkv<kPacked>(p, obuf + wia * kTile, ha, lane, kf4, vf, qf, s_bqkv);
      // The attention at raised wave priority: its dependent MFMA / exp /
      // shuffle chain sets the pace, and the other wave on the SIMD fills the
      // gaps with its q/k/v MFMAs (c3 248-250 -> 245-248 us A/B).
      __builtin_amdgcn_s_setprio(1);
      head_attention<kC, true>(p, cura, tabs + ha * kTableMax, ha, lane, kf4, vf, qf, nullptr, oa);
      __builtin_amdgcn_s_setprio(0);
    }
    if (onb) unit_qkv<kPacked>(p, obuf + wib * kTile, hb, lane, kf4, vf, qf, s_bqkv);
    lds_barrier();  // every LayerNorm row has been read: O may replace them
    const bool onp = u0 + wwin < p.units && locate(p, u0 + wwin).computed;  // this wave's proj
    auto write_held_o = [&]() {
      if (!ona) return;
      uint8_t* ot = obuf + wia * kTile;
#pragma unroll
      for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int cc = 32 * ha + 16 * ct + 4 * g;
          *reinterpret_cast<uint2*>(ot + tile_slot(16 * it + c16, cc >> 3, kCpr) * 16 + (cc & 7) * 2) = oa[it][ct];
        }
    };
    if (!two) {
      // Waves 4..7, whose unit is done: pair k + 1's rows into the other
      // buffer (the slots each of them stored from), in flight while waves
      // 0..3 run the second attention.  Waves 0..3 then request their proj
      // weights with no row loads queued ahead of them.
      if (k + 1 < n) {
        const int u1 = first_unit(k + 1);
#pragma unroll
        for (int wi = 0; wi < 2; ++wi)
          if (u1 + wi < p.units) fetch_rows<4>(p, locate(p, u1 + wi), other + wi * kTile, wave - 4, lane);
      }
      write_held_o();
    } else {
      write_held_o();
      if (onb) {
        __builtin_amdgcn_s_setprio(1);
        head_attention<kC>(p, curb, tabs + hb * kTableMax, hb, lane, kf4, vf, qf, obuf + wib * kTile);
        __builtin_amdgcn_s_setprio(0);
      }
    }
    lds_barrier();  // O complete
    if (onp) {
      uint4 wproj[kKS][3];  // all of them up front: one wait
      proj_weights<kPacked>(p, s4, lane, wproj);
      proj_rows(obuf + wwin * kTile, rows + wwin * kTile, s4, lane, s_bproj, wproj);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  store_pair<kWaves>(p, first_unit(n - 1), smem + ((n - 1) & 1) * kPair, wave, tid0 & 63);
}

// ============================================================================
// swin_block_w7_kernel: 7x7 windows, 4 heads of dim 32, C = 128 (c2), a pair
// of windows at a time.  Eight waves, one (window, head) unit each (unit w:
// window w / 4, head w % 4).
// ============================================================================
//
// A window's 49 tokens occupy rows 0..48 of a 64-row tile (rows 49..63 are
// zero after the LayerNorm; their q / k / v are computed and never used:
// keys >= 49 are excluded from the softmax, queries >= 49 are not stored).
// The attention runs on the generic-geometry softmax of the attention core
// (bias by relative index base(i) - off(j), shift regions and land keys per
// token).  LDS: two row buffers for a pair (pair k's rows, overwritten by its
// output rows; the other holds pair k - 1's output rows, then receives pair
// k + 1's), one LayerNorm buffer that later holds O, and the tables.  Per pair:
//
//   wait for the pair's rows; LayerNorm (waves 4wi .. 4wi + 3 take window wi)
//   barrier
//   every wave: q/k/v of its unit (one pass: six row tiles x four token
//           tiles, four k-steps) and its attention, O kept in registers; its
//           share of pair k - 1's output rows out of the other buffer
//   barrier (every LayerNorm row has been read)
//   its share of pair k + 1's rows into the other buffer; O -> the O buffer
//   barrier
//   wave w: output features [32 (w & 3), + 32) of window w >> 2 = O W_p^T +
//           b_p, plus the residual, in place over the window's rows
//
// Rows are 256 bytes (16 chunks): chunk c of row r sits in slot r * 16 +
// (c ^ (r & 15)), so the 16 rows of a fragment read hit 16 different 16-byte
// bank groups.
namespace w7 {
constexpr int kWs = 7, kN = kWs * kWs, kH = 4, kC = 128, kCpr = kC / 8, kKS = kC / 32;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kTile = 64 * kC * 2;
constexpr int kPair = 2 * kTile;
constexpr int kOffO = 2 * kPair;
constexpr int kOffTabs = kOffO + kPair;
constexpr int kTab = 172;  // >= (2 * 7 - 1)^2 = 169, multiple of 4
constexpr int kLds = kOffTabs + (kH * kTab + kC + kC + 3 * kC + kC) * 4;
static_assert(kLds <= 160 * 1024, "LDS");

__device__ __forceinline__ int slot(int row, int chunk) { return row * kCpr + (chunk ^ (row & 15)); }

// Grid token of row `row` of window u (token (row / 7, row % 7)), or -1 for a
// frame-padding token or a row past the window's 49.
__device__ __forceinline__ int token(const BlockParams& p, const UnitLoc u, int row) {
  if (row >= kN) return -1;
  const int ti = row / kWs, tj = row - ti * kWs;
  int ph = u.wr * kWs + ti + p.shift_h;
  int pw = u.wc * kWs + tj + p.shift_w;
  if (ph >= p.Hp) ph -= p.Hp;
  if (pw >= p.Wp) pw -= p.Wp;
  const int sh = ph - p.pad_top, sw = pw - p.pad_left;
  if ((unsigned)sh >= (unsigned)p.H || (unsigned)sw >= (unsigned)p.W) return -1;
  return (u.b * p.H + sh) * p.W + sw;
}

// The window's rows -> tile by kW waves (wave index wv), direct global -> LDS:
// instruction r of wave wv fills slots (r * kW + wv) * 64 + lane.  Rows that
// are not grid tokens load token 0 (never used).
template <int kW>
__device__ __forceinline__ void fetch(const BlockParams& p, const UnitLoc u, uint8_t* tile, int wv, int lane) {
  constexpr int kRounds = 64 * kCpr / (64 * kW);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * kW + wv;
    const int sl = blk * 64 + lane;
    const int row = sl / kCpr;
    const int ch = (sl - row * kCpr) ^ (row & 15);
    const int t = token(p, u, row);
    const uint8_t* src = p.x + (int64_t)(t >= 0 ? t : 0) * (kCpr * 16) + ch * 16;
    dma_to_lds16(src, __builtin_amdgcn_readfirstlane(lds_address(tile + blk * 1024)));
  }
}

// The window's rows (tile) -> the grid tokens they came from, by kW waves;
// wave wv reads exactly the slots fetch<kW> fills from wave wv.
template <int kW>
__device__ __forceinline__ void store(const BlockParams& p, const UnitLoc u, const uint8_t* tile, int wv, int lane) {
  constexpr int kRounds = 64 * kCpr / (64 * kW);
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(p.y + (int64_t)u.b * p.H * p.W * (kCpr * 16), (uint32_t)((int64_t)p.H * p.W * (kCpr * 16)));
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int sl = (r * kW + wv) * 64 + lane;
    const int row = sl / kCpr;
    const int ch = (sl - row * kCpr) ^ (row & 15);
    const int t = token(p, u, row);
    const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(tile + sl * 16));
    // Rows that are not grid tokens fall outside the range.
    stream_store_sc1(val, out, t >= 0 ? (uint32_t)(t - u.b * p.H * p.W) * (kCpr * 16) + ch * 16 : 0xfffffff0u);
  }
}

// LayerNorm of the raw rows xr -> xn (bf16), 8 lanes per token, the values
// held in registers: fp32 statistics from bf16 dot products (Bf16Moments,
// token_stats8; the variance recomputed from centred values where the mean is
// large against the spread), y = (x rstd - mean rstd) gamma + beta rounded
// once; rows that are not grid tokens become zeros; without LayerNorm the rows
// are copied.
template <int kT>
__device__ __forceinline__ void layernorm(const BlockParams& p, const UnitLoc u, const uint8_t* xr, uint8_t* xn,
                                          const float* s_gamma, const float* s_beta, int tid) {
  constexpr int kCPL = kCpr / 8;  // 2 chunks per lane
  const int sub = tid & 7;
  for (int t = tid >> 3; t < 64; t += kT / 8) {  // uniform per wave
    const bool in = token(p, u, t) >= 0;
    uint4 w[kCPL];
#pragma unroll
    for (int k = 0; k < kCPL; ++k) w[k] = *reinterpret_cast<const uint4*>(xr + slot(t, sub + 8 * k) * 16);
    if (!p.layernorm) {
#pragma unroll
      for (int k = 0; k < kCPL; ++k)
        *reinterpret_cast<uint4*>(xn + slot(t, sub + 8 * k) * 16) = in ? w[k] : make_uint4(0u, 0u, 0u, 0u);
      continue;
    }
    Bf16Moments m;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) m.add4(w[k]);
    float mean, var;
    token_stats8(m, p.inv_c, mean, var);
    if (token_stats_recheck(mean, var)) {  // uniform per wave
      asm volatile("" : "+v"(mean));  // keeps this rare pass a branch, not computed on every path
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) sq = centred_sq4(w[k], mean, sq);
      var = group8_sum(sq) * p.inv_c;
    }
    const float rstd = rsqrtf(fmaxf(var, 0.f) + p.eps);
    const float nmr = -mean * rstd;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const int c0 = (sub + 8 * k) * 8;
      const float4 gm0 = *reinterpret_cast<const float4*>(s_gamma + c0);
      const float4 gm1 = *reinterpret_cast<const float4*>(s_gamma + c0 + 4);
      const float4 bt0 = *reinterpret_cast<const float4*>(s_beta + c0);
      const float4 bt1 = *reinterpret_cast<const float4*>(s_beta + c0 + 4);
      const float gm[8] = {gm0.x, gm0.y, gm0.z, gm0.w, gm1.x, gm1.y, gm1.z, gm1.w};
      const float bt[8] = {bt0.x, bt0.y, bt0.z, bt0.w, bt1.x, bt1.y, bt1.z, bt1.w};
      const uint4 o = normalize_chunk(w[k], rstd, nmr, gm, bt);
      *reinterpret_cast<uint4*>(xn + slot(t, sub + 8 * k) * 16) = in ? o : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// q, k, v of head h for the tile's 64 rows in one pass (accumulator j: Q^T
// row tiles 2h + j, K^T C/16 + 2h + j - 2, V C/8 + 2h + j - 4, the V tiles
// as xn W^T), packed into attention operand fragments; Q unscaled (the
// softmax applies scale * log2e).
template <bool kPacked>
__device__ __forceinline__ void unit_qkv(const BlockParams& p, const uint8_t* xn, int h, int lane, uint4 (&kf)[4][1],
                                         uint4 (&vf)[2][2], uint4 (&qf)[4][1], const float* bqkv) {
  const int g = lane >> 4, c16 = lane & 15;
  auto rt = [&](int j) { return (j >> 1) * (kC / 16) + 2 * h + (j & 1); };
  f32x4 acc[6][4];
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    f32x4 b;
    if (j < 4) {
      b = load_f32x4(bqkv + (j >> 1) * kC + 32 * h + 16 * (j & 1) + 4 * g);
    } else {
      const float bv = bqkv[2 * kC + 32 * h + 16 * (j & 1) + c16];
      b = f32x4{bv, bv, bv, bv};
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[j][tt] = b;
  }
  auto xn_frag = [&](int tt, int ks) -> uint4 {
    const int row = 16 * tt + c16;
    return *reinterpret_cast<const uint4*>(xn + slot(row, 4 * ks + g) * 16);
  };
  constexpr int kDepth = 2;  // weight ring (registers): loads one k-step ahead (deeper measured the same)
  uint4 ring[kDepth][6];
#pragma unroll
  for (int st = 0; st < kDepth - 1; ++st)
#pragma unroll
    for (int j = 0; j < 6; ++j) ring[st][j] = weight_frag<kC, kPacked>(p.w_qkv, rt(j), st, lane);
  uint4 xf[2][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) xf[0][tt] = xn_frag(tt, 0);
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) {
    if (ks + kDepth - 1 < kKS) {
#pragma unroll
      for (int j = 0; j < 6; ++j)
        ring[(ks + kDepth - 1) % kDepth][j] = weight_frag<kC, kPacked>(p.w_qkv, rt(j), ks + kDepth - 1, lane);
    }
    if (ks + 1 < kKS) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) xf[(ks + 1) & 1][tt] = xn_frag(tt, ks + 1);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 x8 = __builtin_bit_cast(bf16x8, xf[ks & 1][tt]);
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        const bf16x8 w8 = __builtin_bit_cast(bf16x8, ring[ks % kDepth][j]);
        acc[j][tt] = j < 4 ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(w8, x8, acc[j][tt], 0, 0, 0)
                           : __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, w8, acc[j][tt], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    kf[tt][0] = pack_frag(acc[2][tt], acc[3][tt]);
    qf[tt][0] = pack_frag(acc[0][tt], acc[1][tt]);
  }
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int js = 0; js < 2; ++js) vf[ct][js] = pack_frag(acc[4 + ct][2 * js], acc[4 + ct][2 * js + 1]);
}

// Attention of head h of window u from the unit's fragments; O (bf16) held in
// opk[it][ct] (channels 32h + 16 ct + 4g .. + 3 of query 16 it + c).
__device__ __forceinline__ void unit_attention(const BlockParams& p, const UnitLoc u, const float* tab, int lane,
                                               const uint4 (&kf)[4][1], const uint4 (&vf)[2][2],
                                               const uint4 (&qf)[4][1], uint2 (&opk)[4][2]) {
  const WindowMaskState m = block_mask_state(p, u);
  LaneGeom<false> lg;
  lane_geom_init<false>(lg, p.a, m, tab, lane);
  auto vsrc = [&](int ct, int js) -> bf16x8 { return __builtin_bit_cast(bf16x8, vf[ct][js]); };
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    f32x4 sc[2][4];
    const uint4 (&qp)[2][1] = *reinterpret_cast<const uint4(*)[2][1]>(&qf[2 * half]);
    scores_pair<true, 32>(sc, kf, qp);
    float inv[2];
    softmax_half<false, false>(sc, inv, half, p.a, m, lg, nullptr, lane);
    f32x4 o[2][2];
    pv_half<true, 32>(o, sc, lane, vsrc);
#pragma unroll
    for (int il = 0; il < 2; ++il)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const f32x4 v = o[ct][il] * inv[il];
        opk[2 * half + il][ct] = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
  }
}

// Output features [32 q4, 32 q4 + 32) of a window = O W_p^T + b_p (two row
// tiles x four token tiles), then y = bf16(x + bf16(Y)) in place over the
// window's raw rows.
template <bool kPacked>
__device__ __forceinline__ void proj_rows(const BlockParams& p, const uint8_t* o_tile, uint8_t* tile, int q4,
                                          int lane, const float* bproj) {
  const int g = lane >> 4, c16 = lane & 15;
  f32x4 ya[2][4];
#pragma unroll
  for (int ft = 0; ft < 2; ++ft) {
    const f32x4 b = load_f32x4(bproj + 32 * q4 + 16 * ft + 4 * g);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) ya[ft][tt] = b;
  }
  uint4 wf[kKS][2];
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks)
#pragma unroll
    for (int ft = 0; ft < 2; ++ft) wf[ks][ft] = weight_frag<kC, kPacked>(p.w_proj, 2 * q4 + ft, ks, lane);
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) {
    uint4 of[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      of[tt] = *reinterpret_cast<const uint4*>(o_tile + slot(16 * tt + c16, 4 * ks + g) * 16);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int ft = 0; ft < 2; ++ft)
        ya[ft][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[ks][ft]),
                                                             __builtin_bit_cast(bf16x8, of[tt]), ya[ft][tt], 0, 0, 0);
  }
#pragma unroll
  for (int ft = 0; ft < 2; ++ft) {
    const int fb = 32 * q4 + 16 * ft + 4 * g;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      residual_add4(tile + slot(16 * tt + c16, fb >> 3) * 16 + (fb & 7) * 2, ya[ft][tt]);
  }
}

}  // namespace w7

template <bool kPacked>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void swin_block_w7_kernel(const BlockParams p) {
  using namespace w7;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* obuf = smem + kOffO;
  float* tabs = reinterpret_cast<float*>(smem + kOffTabs);
  float* s_gamma = tabs + kH * kTab;
  float* s_beta = s_gamma + kC;
  float* s_bqkv = s_beta + kC;
  float* s_bproj = s_bqkv + 3 * kC;
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int wwin = wave >> 2, h = wave & 3;  // this wave's unit: window wwin of the pair, head h
  const int pairs = (p.units + 1) >> 1;
  if ((int)blockIdx.x >= pairs) return;  // uniform across the workgroup
  // Bias columns (x log2e, index e = relative index) and the small parameters.
  for (int e = tid0; e < kH * kTab; e += kThreads) {
    const int hh = e / kTab, i = e - hh * kTab;
    tabs[e] = (p.bias_table != nullptr && i < (2 * kWs - 1) * (2 * kWs - 1)) ? p.bias_table[i * kH + hh] * kLog2e
                                                                             : 0.f;
  }
  for (int c = tid0; c < kC; c += kThreads) {
    s_gamma[c] = p.gamma != nullptr ? p.gamma[c] : 1.f;
    s_beta[c] = p.beta != nullptr ? p.beta[c] : 0.f;
    s_bproj[c] = p.b_proj != nullptr ? p.b_proj[c] : 0.f;
  }
  for (int c = tid0; c < 3 * kC; c += kThreads) s_bqkv[c] = p.b_qkv != nullptr ? p.b_qkv[c] : 0.f;
  __syncthreads();
  const int n = (pairs - 1 - (int)blockIdx.x) / (int)gridDim.x + 1;
  auto first_unit = [&](int k) { return 2 * ((int)blockIdx.x + k * (int)gridDim.x); };
  {  // the first pair's rows
    const int u0 = first_unit(0);
#pragma unroll
    for (int wi = 0; wi < 2; ++wi)
      if (u0 + wi < p.units) fetch<kWaves>(p, locate(p, u0 + wi), smem + wi * kTile, wave, tid0 & 63);
  }

  for (int k = 0; k < n; ++k) {
    // Lane-derived addresses are recomputed per pair (the thread id passes
    // through an empty asm) rather than hoisted and held across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    uint8_t* rows = smem + (k & 1) * kPair;         // pair k's rows, later its output rows
    uint8_t* other = smem + ((k + 1) & 1) * kPair;  // pair k - 1's output rows, then pair k + 1's rows
    const int u0 = first_unit(k);
    const UnitLoc cur = locate(p, u0 + wwin);
    const bool live = u0 + wwin < p.units;
    const bool on = live && cur.computed;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the pair's rows
    lds_barrier();
    if (on)
      layernorm<kThreads / 2>(p, cur, rows + wwin * kTile, obuf + wwin * kTile, s_gamma, s_beta,
                              tid & (kThreads / 2 - 1));
    lds_barrier();  // LayerNorm rows ready
    uint2 opk[4][2];
    if (on) {
      uint4 kf[4][1], vf[2][2], qf[4][1];
      unit_qkv<kPacked>(p, obuf + wwin * kTile, h, lane, kf, vf, qf, s_bqkv);
      __builtin_amdgcn_s_setprio(1);  // as in the six-head kernel (c2 34.0-34.3 -> 33.1-33.8 us A/B)
      unit_attention(p, cur, tabs + h * kTab, lane, kf, vf, qf, opk);
      __builtin_amdgcn_s_setprio(0);
    }
    if (k > 0) {  // pair k - 1's output rows
      const int up = first_unit(k - 1);
#pragma unroll
      for (int wi = 0; wi < 2; ++wi)
        if (up + wi < p.units) store<kWaves>(p, locate(p, up + wi), other + wi * kTile, wave, lane);
    }
    lds_barrier();  // every LayerNorm row has been read: O may replace them
    if (k + 1 < n) {  // pair k + 1's rows, over the slots this wave has just stored
      const int u1 = first_unit(k + 1);
#pragma unroll
      for (int wi = 0; wi < 2; ++wi)
        if (u1 + wi < p.units) fetch<kWaves>(p, locate(p, u1 + wi), other + wi * kTile, wave, lane);
    }
    if (on) {
      uint8_t* ot = obuf + wwin * kTile;
#pragma unroll
      for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int cc = 32 * h + 16 * ct + 4 * g;
          *reinterpret_cast<uint2*>(ot + slot(16 * it + c16, cc >> 3) * 16 + (cc & 7) * 2) = opk[it][ct];
        }
    }
    lds_barrier();  // O complete
    if (on) proj_rows<kPacked>(p, obuf + wwin * kTile, rows + wwin * kTile, h, lane, s_bproj);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  {  // the last pair's output rows
    const int u0 = first_unit(n - 1);
#pragma unroll
    for (int wi = 0; wi < 2; ++wi)
      if (u0 + wi < p.units) store<kWaves>(p, locate(p, u0 + wi), smem + ((n - 1) & 1) * kPair + wi * kTile, wave,
                                           tid0 & 63);
  }
}

// ============================================================================
// swin_block_hd64_kernel: 12 heads of dim 64, C = 768 (the reference model's
// block, c4).  Eight waves, one window at a time: wave s < 4 owns heads 3s and
// 3s + 1, wave s + 4 head 3s + 2, so each SIMD (holding waves s and s + 4)
// does three heads.
// ============================================================================
//
// At C = 768 one [64][C] bf16 tile is 96 KB, so the workgroup keeps a single
// tile that holds, in turn, the window's raw rows, their LayerNorm (computed
// in place), the attention output O and the output rows:
//
//   rows -> tile (direct global -> LDS), LayerNorm in place      (all waves)
//   per head: K^T, V, then Q^T from the tile into MFMA operand fragments
//           (three passes over the 24 k-steps); a two-head wave runs its
//           first head's attention before its second head's projections
//           and writes that O to an LDS staging area
//   barrier (every wave has read the LayerNorm tile)
//   the staged O and the last head's O into columns [64h, 64h + 64) of the
//           tile
//   barrier
//   wave w: output features [96w, 96w + 96) = O W_p^T + b_p
//   barrier (every wave has read O)
//   y = x + proj (the residual x read back from global memory) into the
//   tile, rows scattered back to the grid.
//
// Tiles with 96-chunk (1536-byte) rows use the 256-byte-pitch swizzle: chunk
// c of row r at slot r * 96 + (c ^ (r & 15)).
namespace hd64 {
constexpr int kH = 12, kD = 64, kC = kH * kD, kCpr = kC / 8, kKS = kC / 32;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kTile = 64 * kC * 2;
constexpr int kStage = 4 * 64 * kD * 2;  // O of the four first heads of the two-head waves
constexpr int kLds = kTile + kStage + kH * kTableMax * 4;
static_assert(kLds <= 160 * 1024, "LDS");

__device__ __forceinline__ int slot(int row, int chunk) { return row * kCpr + (chunk ^ (row & 15)); }

// Byte offset of the 16-byte operand chunk 4 ks + g of row 16 tt + c16.
__device__ __forceinline__ uint32_t frag_off(int tt, int ks, int lane) {
  const int g = lane >> 4, c16 = lane & 15;
  return (uint32_t)(((16 * tt + c16) * kCpr + 16 * (ks >> 2) + ((4 * (ks & 3) + g) ^ c16)) * 16);
}

// The window's 64 rows -> the tile (frame-padding rows load grid token 0 and
// are never used), without the streaming hint: the residual add reads the
// rows again from global memory, so they stay in L2.
__device__ __forceinline__ void fetch(const BlockParams& p, const UnitLoc u, uint8_t* tile, int wave, int lane) {
  constexpr int kRounds = kCpr * 64 / (64 * kWaves);  // 12
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * kWaves + wave;
    const int sl = blk * 64 + lane;
    const int row = sl / kCpr;
    const int ch = (sl - row * kCpr) ^ (row & 15);
    const int t = grid_token(p, u, row >> 3, row & 7);
    const uint8_t* src = p.x + (int64_t)(t >= 0 ? t : 0) * (kCpr * 16) + ch * 16;
    dma_to_lds16_cached(src, __builtin_amdgcn_readfirstlane(lds_address(tile + blk * 1024)));
  }
}

// LayerNorm of the raw rows in place (eight lanes per token; fp32 statistics
// from bf16 dot products over the packed rows, Bf16Moments / token_stats8,
// the variance recomputed from centred values where the mean is large against
// the spread; the rows are read from LDS once for the statistics and once for
// the output; frame-padding tokens become zeros; without LayerNorm the rows
// are kept, padding zeroed).
__device__ __forceinline__ void layernorm_in_place(const BlockParams& p, const UnitLoc u, uint8_t* tile, int tid) {
  constexpr int kCPL = kCpr / 8;  // 12 chunks per lane
  const int sub = tid & 7;
  auto raw = [&](int t, int k) { return *reinterpret_cast<const uint4*>(tile + slot(t, sub + 8 * k) * 16); };
  const float* gptr = p.gamma;
  const float* bptr = p.beta;
  asm volatile("" : "+s"(gptr), "+s"(bptr));  // read per window, not held in registers
  for (int t = tid >> 3; t < 64; t += kThreads / 8) {  // uniform per wave
    const bool in = grid_token(p, u, t >> 3, t & 7) >= 0;
    if (!in || !p.layernorm) {
      if (!in) {
#pragma unroll
        for (int k = 0; k < kCPL; ++k)
          *reinterpret_cast<uint4*>(tile + slot(t, sub + 8 * k) * 16) = make_uint4(0u, 0u, 0u, 0u);
      }
      continue;
    }
    Bf16Moments m;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) m.add4(raw(t, k));
    float mean, var;
    token_stats8(m, p.inv_c, mean, var);
    if (token_stats_recheck(mean, var)) {  // uniform over the active lanes
      asm volatile("" : "+v"(mean));  // keeps this rare pass a branch, not computed on every path
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) sq = centred_sq4(raw(t, k), mean, sq);
      var = group8_sum(sq) * p.inv_c;
    }
    const float rstd = rsqrtf(fmaxf(var, 0.f) + p.eps);
    const float nmr = -mean * rstd;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const int c0 = (sub + 8 * k) * 8;
      float gm[8], bt[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 gq = gptr != nullptr ? *reinterpret_cast<const f32x4*>(gptr + c0 + 4 * h) : f32x4{1.f, 1.f, 1.f, 1.f};
        const f32x4 bq = bptr != nullptr ? *reinterpret_cast<const f32x4*>(bptr + c0 + 4 * h) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gm[4 * h + e] = gq[e];
          bt[4 * h + e] = bq[e];
        }
      }
      *reinterpret_cast<uint4*>(tile + slot(t, sub + 8 * k) * 16) = normalize_chunk(raw(t, k), rstd, nmr, gm, bt);
    }
  }
}

// One projection pass over the 24 k-steps: NF feature tiles (row tiles
// rt0 .. rt0 + NF - 1 of the packed weight) for NT token tiles from tt0,
// with the bias as the accumulator init.  kV: computed as xn W^T (A = xn
// rows; lane holds tokens 4g + r of feature c, the V^T operand layout);
// otherwise W xn^T (lane holds features 4g + r of token c).  The weights of
// the next k-step are requested before this step's MFMAs, then this step's
// xn fragments are read: a deeper ring does not fit next to the K and V
// fragments a wave holds while it computes Q.
template <int NF, int NT, bool kV, bool kPacked, int kDepth = 2>
__device__ __forceinline__ void pass(const BlockParams& p, const uint16_t* w, const float* bias, int rt0, int tt0,
                                     const uint8_t* tile, int lane, f32x4 (&acc)[NF][NT]) {
  const int g = lane >> 4, c16 = lane & 15;
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    f32x4 b = f32x4{0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr) {
      if constexpr (kV) {
        const float bv = bias[16 * (rt0 + f) + c16];
        b = f32x4{bv, bv, bv, bv};
      } else {
        b = load_f32x4(bias + 16 * (rt0 + f) + 4 * g);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[f][t] = b;
  }
  // kDepth: weight ring depth (registers), loads kDepth - 1 k-steps ahead.
  static_assert(kKS % kDepth == 0, "whole ring turns");
  uint4 ring[kDepth][NF];
#pragma unroll
  for (int st = 0; st < kDepth - 1; ++st)
#pragma unroll
    for (int f = 0; f < NF; ++f) ring[st][f] = weight_frag<kC, kPacked>(w, rt0 + f, st, lane);
  for (int ks0 = 0; ks0 < kKS; ks0 += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const int ks = ks0 + j;
      if (ks + kDepth - 1 < kKS) {
#pragma unroll
        for (int f = 0; f < NF; ++f)
          ring[(j + kDepth - 1) % kDepth][f] = weight_frag<kC, kPacked>(w, rt0 + f, ks + kDepth - 1, lane);
      }
      asm volatile("" ::: "memory");
      uint4 xf[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) xf[t] = *reinterpret_cast<const uint4*>(tile + frag_off(tt0 + t, ks, lane));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bf16x8 x8 = __builtin_bit_cast(bf16x8, xf[t]);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const bf16x8 w8 = __builtin_bit_cast(bf16x8, ring[j][f]);
          acc[f][t] = kV ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(x8, w8, acc[f][t], 0, 0, 0)
                         : __builtin_amdgcn_mfma_f32_16x16x32_bf16(w8, x8, acc[f][t], 0, 0, 0);
        }
      }
    }
  }
}

// Scores, softmax and O^T = V^T P^T of query tile `it` of an 8x8 window
// against its 64 keys, head dim 64 (two 32-channel k-steps).  As
// attend_qtiles: the relative-position bias (tabr) is the accumulator init,
// mask terms are added to the MFMA result, the row sum runs on the matrix
// cores, the Q operand carries scale * log2(e).
template <int kMask, class VFrag>
__device__ __forceinline__ void attend_tile(f32x4 (&o)[4], float& inv, int it, const uint4 (&kf)[4][2],
                                            const uint4 (&qf)[2], const float* tabr, const WindowMaskState& m,
                                            const f32x4 (&land_term)[4], uint64_t rid_pack, int rid_q,
                                            float mask_term, VFrag vfrag) {
  f32x4 s[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) s[jt][r] = tabr[30 * (3 - it + jt) + r];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
      s[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[jt][kk]),
                                                      __builtin_bit_cast(bf16x8, qf[kk]), s[jt], 0, 0, 0);
  if constexpr (kMask == kMaskShift) {
    const bool land = m.land != 0ull;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rid_j = (int)((rid_pack >> (4 * (4 * jt + r))) & 15ull);
        s[jt][r] += (rid_j != rid_q ? mask_term : 0.f) + (land ? land_term[jt][r] : 0.f);
      }
  } else if constexpr (kMask == kMaskLand) {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) s[jt] += land_term[jt];
  }
  float mx = s[0][0];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = max_nan(mx, s[jt][r]);
  mx = xor_max(mx);
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) s[jt][r] = __builtin_amdgcn_exp2f(s[jt][r] - mx);
  const bf16x8 ones = ones_frag();
  f32x4 rs = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) o[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int js = 0; js < 2; ++js) {
    uint32_t wds[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      wds[e / 2] = pack_bf16x2(s[2 * js + (e >> 2)][e & 3], s[2 * js + (e >> 2)][(e & 3) + 1]);
    const bf16x8 pf = __builtin_bit_cast(bf16x8, wds);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      o[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag(ct, js), pf, o[ct], 0, 0, 0);
    rs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, rs, 0, 0, 0);
  }
  inv = __builtin_amdgcn_rcpf(rs[0]);
}

// y rows of the window (in the tile) -> the grid tokens they came from;
// frame-padding rows are dropped.
__device__ __forceinline__ void store(const BlockParams& p, const UnitLoc u, const uint8_t* tile, int tid) {
  constexpr int kPasses = 64 * kCpr / kThreads;  // 12
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(p.y + (int64_t)u.b * p.H * p.W * (kCpr * 16), (uint32_t)((int64_t)p.H * p.W * (kCpr * 16)));
#pragma unroll
  for (int r = 0; r < kPasses; ++r) {
    const int q = r * kThreads + tid;
    const int row = q / kCpr, ch = q - row * kCpr;
    const int t = grid_token(p, u, row >> 3, row & 7);
    const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(tile + slot(row, ch) * 16));
    const uint32_t off = t >= 0 ? (uint32_t)(t - u.b * p.H * p.W) * (kCpr * 16) + ch * 16 : 0xfffffff0u;
    stream_store_sc1(val, out, off);  // padding rows fall outside the range
  }
}

}  // namespace hd64

namespace hd64 {

// K, V and Q^T (times scale * log2 e) of head h as MFMA operand fragments:
// kf[tt][kk] (K rows of key tile tt, channels 32 kk ..), vf[ct][js] (V^T
// operand), qf[it][kk] (Q operand of query tile it).  The K and V passes
// run their weights two k-steps ahead (each window streams 4.7 MB of weights
// from L2: c4 202-204 -> 193-196 us); the Q pass, which runs beside the first
// head's K and V fragments, keeps one step so that nothing spills.
template <bool kPacked>
__device__ __forceinline__ void head_qkv64(const BlockParams& p, const uint8_t* tile, int h, int lane,
                                           uint4 (&kf)[4][2], uint4 (&vf)[4][2], uint4 (&qf)[4][2]) {
  {
    f32x4 acc[4][4];
    pass<4, 4, false, kPacked, 3>(p, p.w_qkv, p.b_qkv, kC / 16 + 4 * h, 0, tile, lane, acc);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) kf[tt][kk] = pack_frag(acc[2 * kk][tt], acc[2 * kk + 1][tt]);
  }
  {
    f32x4 acc[4][4];
    pass<4, 4, true, kPacked, 3>(p, p.w_qkv, p.b_qkv, kC / 8 + 4 * h, 0, tile, lane, acc);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int js = 0; js < 2; ++js) vf[ct][js] = pack_frag(acc[ct][2 * js], acc[ct][2 * js + 1]);
  }
  {
    f32x4 acc[4][4];
    pass<4, 4, false, kPacked, 2>(p, p.w_qkv, p.b_qkv, 4 * h, 0, tile, lane, acc);
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        qf[it][kk] = pack_frag(acc[2 * kk][it] * p.a.scale_l2e, acc[2 * kk + 1][it] * p.a.scale_l2e);
  }
}

// Byte offset of channels cc .. cc + 3 (cc a multiple of 4, < 64) of row
// `row` in a head's 8 KB staging slice (128-byte rows, chunk ^ (row & 7)).
__device__ __forceinline__ uint32_t stage_off(int row, int cc) {
  return (uint32_t)(row * 128 + (((cc >> 3) ^ (row & 7)) << 4) + (cc & 7) * 2);
}

// Attention of head h (all four query tiles) from its fragments.  O goes to
// columns [64h, 64h + 64) of the tile, or with kStage to the head's staging
// slice `stage` (the tile still holds the LayerNorm rows other waves read).
template <bool kStage>
__device__ __forceinline__ void head_attention64(const BlockParams& p, const UnitLoc cur, const float* tabs, int h,
                                                 int lane, const uint4 (&kf)[4][2], const uint4 (&vf)[4][2],
                                                 const uint4 (&qf)[4][2], uint8_t* tile, uint8_t* stage) {
  // A fresh lane id: the mask terms are computed here, not hoisted.
  asm volatile("" : "+v"(lane));
  const int g = lane >> 4, c16 = lane & 15;
  const WindowMaskState m = block_mask_state(p, cur);
  const float* tabr = lane_bias_rev(tabs + h * kTableMax, lane);
  auto vsrc = [&](int ct, int js) -> bf16x8 { return __builtin_bit_cast(bf16x8, vf[ct][js]); };
  auto run = [&](auto mode, const f32x4 (&land_term)[4], uint64_t rid_pack) {
    constexpr int kMask = decltype(mode)::value;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rid_q = kMask == kMaskShift ? 3 * region(cur.wr * 8 + 2 * it + (c16 >> 3), p.Hp, 8, p.shift_h) +
                                                  region(cur.wc * 8 + (c16 & 7), p.Wp, 8, p.shift_w)
                                            : 0;
      f32x4 o[4];
      float inv;
      attend_tile<kMask>(o, inv, it, kf, qf[it], tabr, m, land_term, rid_pack, rid_q, p.a.mask_l2e, vsrc);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const f32x4 v = o[ct] * inv;
        uint2 pk;
        pk.x = pack_bf16x2(v[0], v[1]);
        pk.y = pack_bf16x2(v[2], v[3]);
        if constexpr (kStage) {
          *reinterpret_cast<uint2*>(stage + stage_off(16 * it + c16, 16 * ct + 4 * g)) = pk;
        } else {
          const int cc = kD * h + 16 * ct + 4 * g;
          *reinterpret_cast<uint2*>(tile + slot(16 * it + c16, cc >> 3) * 16 + (cc & 7) * 2) = pk;
        }
      }
    }
  };
  f32x4 land_term[4];
  if (m.use_shift) {
    uint64_t rid_pack = 0;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        rid_pack |= (uint64_t)(3 * region(cur.wr * 8 + 2 * jt + (g >> 1), p.Hp, 8, p.shift_h) +
                               region(cur.wc * 8 + 4 * (g & 1) + r, p.Wp, 8, p.shift_w))
                    << (4 * (4 * jt + r));
    if (m.land != 0ull) land_terms(land_term, m.land, g, p.a.mask_l2e);
    run(MaskMode<kMaskShift>{}, land_term, rid_pack);
  } else if (m.land != 0ull) {
    land_terms(land_term, m.land, g, p.a.mask_l2e);
    run(MaskMode<kMaskLand>{}, land_term, 0ull);
  } else {
    run(MaskMode<kMaskNone>{}, land_term, 0ull);
  }
}

}  // namespace hd64

template <bool kPacked>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void swin_block_hd64_kernel(const BlockParams p) {
  using namespace hd64;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* tile = smem;
  float* tabs = reinterpret_cast<float*>(smem + kTile + kStage);
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int s4 = wave & 3;
  const bool two = wave < 4;                 // waves 0..3: heads 3s, 3s + 1; waves 4..7: head 3s + 2
  const int h_first = two ? 3 * s4 : 3 * s4 + 2;
  if ((int)blockIdx.x >= p.units) return;  // uniform across the workgroup
  for (int e = tid0; e < kH * kTableMax; e += kThreads) {
    const int hh = e / kTableMax, i = e - hh * kTableMax;
    const int ri = kTableRev - i;  // reversed column (lane_bias_rev)
    tabs[e] = (p.bias_table != nullptr && ri < 225) ? p.bias_table[ri * kH + hh] * kLog2e : 0.f;
  }
  __syncthreads();

  for (int unit = blockIdx.x; unit < p.units; unit += gridDim.x) {
    // Lane-derived addresses are recomputed per window (the thread id passes
    // through an empty asm) rather than hoisted and held across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const UnitLoc cur = locate(p, unit);
    fetch(p, cur, tile, wave, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    if (cur.computed) {  // uniform across the workgroup
      layernorm_in_place(p, cur, tile, tid);
      lds_barrier();
      uint8_t* stage = smem + kTile + s4 * (64 * kD * 2);  // a two-head wave's first O
      if (two) {
        uint4 kf[4][2], vf[4][2], qf[4][2];
        head_qkv64<kPacked>(p, tile, h_first, lane, kf, vf, qf);
        head_attention64<true>(p, cur, tabs, h_first, lane, kf, vf, qf, tile, stage);
      }
      {
        const int h = two ? h_first + 1 : h_first;
        uint4 kf[4][2], vf[4][2], qf[4][2];
        head_qkv64<kPacked>(p, tile, h, lane, kf, vf, qf);
        lds_barrier();  // every wave has read the LayerNorm tile; O overwrites it
        if (two) {  // the staged O (written by this wave) -> its tile columns
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const int i = 64 * r + lane, row = i >> 3, ch = i & 7;
            const uint4 v = *reinterpret_cast<const uint4*>(stage + row * 128 + ((ch ^ (row & 7)) << 4));
            *reinterpret_cast<uint4*>(tile + slot(row, 8 * h_first + ch) * 16) = v;
          }
        }
        head_attention64<false>(p, cur, tabs, h, lane, kf, vf, qf, tile, stage);
      }
      lds_barrier();  // O complete
      // ---- proj: output features [96 w, 96 w + 96), then the residual ------
      f32x4 ya[6][4];
      pass<6, 4, false, kPacked>(p, p.w_proj, p.b_proj, 6 * wave, 0, tile, lane, ya);
      lds_barrier();  // every wave has read O; the output rows overwrite it
      const __amdgpu_buffer_rsrc_t xin =
          buffer_rsrc(p.x + (int64_t)cur.b * p.H * p.W * (kCpr * 16), (uint32_t)((int64_t)p.H * p.W * (kCpr * 16)));
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int row = 16 * tt + c16;
        const int t = grid_token(p, cur, row >> 3, row & 7);
        const uint32_t base = (uint32_t)(t - cur.b * p.H * p.W) * (kCpr * 16);
#pragma unroll
        for (int ft = 0; ft < 6; ++ft) {
          const int fb = 96 * wave + 16 * ft + 4 * g;
          // Frame-padding rows (t < 0) read at the out-of-range marker
          // 0xfffffff0 (+ 8 bytes does not wrap), which the buffer range
          // check turns into zeros; those rows are not stored.
          const stream_u32x2 xv = __builtin_amdgcn_raw_buffer_load_b64(xin, t >= 0 ? base + fb * 2 : 0xfffffff0u, 0, 0);
          const f32x4& a = ya[ft][tt];
          uint2 out;
          out.x = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv[0] & 0xffffu)) + (float)(__bf16)a[0],
                              bf16_bits_to_f32((uint16_t)(xv[0] >> 16)) + (float)(__bf16)a[1]);
          out.y = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv[1] & 0xffffu)) + (float)(__bf16)a[2],
                              bf16_bits_to_f32((uint16_t)(xv[1] >> 16)) + (float)(__bf16)a[3]);
          *reinterpret_cast<uint2*>(tile + slot(row, fb >> 3) * 16 + (fb & 7) * 2) = out;
        }
      }
    }
    // Rows of a window the frame does not emit pass through unchanged (they
    // were fetched into the tile as they are).
    lds_barrier();  // output rows complete
    store(p, cur, tile, tid);
    lds_barrier();  // the rows are read out before the next window's load
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
template <int kH, bool kPacked>
int launch_block_layout(const BlockParams& p, hipStream_t s) {
  static int resident[64] = {0};
  constexpr int lds = block_lds_bytes<kH>();
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&swin_block_kernel<kH, kPacked>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  return launch_persistent(swin_block_kernel<kH, kPacked>, 64 * kH, lds, p.units, p, s, resident);
}

template <int kH>
int launch_block(const BlockParams& p, hipStream_t s) {
  return p.packed ? launch_block_layout<kH, true>(p, s) : launch_block_layout<kH, false>(p, s);
}

template <bool kPacked>
int launch_block_hd64_layout(const BlockParams& p, hipStream_t s) {
  static int resident[64] = {0};
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&swin_block_hd64_kernel<kPacked>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, hd64::kLds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  return launch_persistent(swin_block_hd64_kernel<kPacked>, hd64::kThreads, hd64::kLds, p.units, p, s, resident);
}

template <bool kPacked>
int launch_block_dw_layout(const BlockParams& p, hipStream_t s) {
  static int resident[64] = {0};
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&swin_block_dw_kernel<kPacked>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, dw::kLds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  return launch_persistent(swin_block_dw_kernel<kPacked>, dw::kThreads, dw::kLds, (p.units + 1) / 2, p, s, resident);
}

int launch_block_dw(const BlockParams& p, hipStream_t s) {
  return p.packed ? launch_block_dw_layout<true>(p, s) : launch_block_dw_layout<false>(p, s);
}

template <bool kPacked>
int launch_block_w7_layout(const BlockParams& p, hipStream_t s) {
  static int resident[64] = {0};
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&swin_block_w7_kernel<kPacked>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, w7::kLds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  return launch_persistent(swin_block_w7_kernel<kPacked>, w7::kThreads, w7::kLds, (p.units + 1) / 2, p, s, resident);
}

int launch_block_w7(const BlockParams& p, hipStream_t s) {
  return p.packed ? launch_block_w7_layout<true>(p, s) : launch_block_w7_layout<false>(p, s);
}

int launch_block_hd64(const BlockParams& p, hipStream_t s) {
  return p.packed ? launch_block_hd64_layout<true>(p, s) : launch_block_hd64_layout<false>(p, s);
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
  const bool w7 = q.window == 7 && d.heads == 4 && q.channels == 128;
  if (q.window != 8 && !w7)
    return fail(TERRA_ERR_UNSUPPORTED,
                "the fused block kernel needs 8x8 windows, or 7x7 windows with 4 heads of dim 32 (window %d, heads %d, "
                "channels %d)", q.window, d.heads, q.channels);
  const bool hd64 = d.heads == 12 && q.channels == 768;
  if (!hd64 && !w7 && d.heads != 6 && d.heads != 12)
    return fail(TERRA_ERR_UNSUPPORTED, "the fused block kernel supports 6 or 12 heads (got %d)", d.heads);
  if (!hd64 && !w7 && q.channels != 32 * d.heads)
    return fail(TERRA_ERR_UNSUPPORTED,
                "the fused block kernel needs head dim 32, or 12 heads of dim 64 (channels %d, heads %d)",
                q.channels, d.heads);
  if (d.layernorm != 0 && !(d.ln_eps >= 0.f))
    return fail(TERRA_ERR_SHAPE, "ln_eps must be a non-negative number");
  // land_bits[w % land_windows]: bits built for another frame would wrap onto
  // the wrong windows, so the period must be whole images of emitted windows.
  if (land_bits != nullptr &&
      (d.land_windows <= 0 || ((int64_t)q.batch * dims.nWe) % d.land_windows != 0 || d.land_windows % dims.nWe != 0))
    return fail(TERRA_ERR_SHAPE,
                "land_windows (%d) must be a multiple of the emitted windows per image (%lld) dividing the batch's "
                "(%lld)", d.land_windows, (long long)dims.nWe, (long long)((int64_t)q.batch * dims.nWe));
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
  if ((int64_t)q.height * q.width * q.channels * 2 >= (1ll << 32))
    return fail(TERRA_ERR_SHAPE, "one image of the grid must be under 4 GiB");

  BlockParams p;
  memset(&p, 0, sizeof(p));
  p.a.scale_l2e = d.scale * kLog2e;
  p.a.mask_l2e = d.mask_value * kLog2e;
  p.a.frame_h = (int32_t)dims.Hp;
  p.a.frame_w = (int32_t)dims.Wp;
  p.a.shift_h = q.shift_h;
  p.a.shift_w = q.shift_w;
  p.a.window_h = p.a.window_w = q.window;
  p.a.N = p.a.n_geo = p.a.n_real = q.window * q.window;
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
  // The all-land shortcut cancels a constant mask term exactly only while
  // that term is finite and small enough not to swamp the fp32 scores.
  p.land_shortcut = fabsf(d.mask_value) <= 4096.f;
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
  const int ls = w7 ? launch_block_w7(p, s)
                 : hd64 ? launch_block_hd64(p, s) : (d.heads == 6 ? launch_block_dw(p, s) : launch_block<12>(p, s));
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
