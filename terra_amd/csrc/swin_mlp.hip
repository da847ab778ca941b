// Fused MLP half of a Swin block (SequentialMlp.forward, models/mlp.py:152-172):
//
//   y = x + fc2(GELU(fc1(LayerNorm(x))))        per token, bf16 activations
//
// One persistent workgroup per CU (12 waves) walks 64-token tiles.  A tile's
// rows arrive by direct global->LDS loads (double-buffered for C = 192: the
// next tile streams in while this one computes), LayerNorm writes the bf16
// operand tile, and the hidden layer never leaves the CU: it is produced in
// chunks of 384 features (fc1 on MFMA, bias as the accumulator init, then
// bf16 -> exact GELU -> bf16 into LDS) and consumed by fc2 right away, whose
// accumulators persist across the chunks.  The output is added to the raw
// rows in LDS (bf16(x + bf16(y))) and the rows are stored as whole lines at
// the start of the next tile.  Weights are in the fragment-packed layout of
// terra_swin_pack_linear and stream from L2 once per tile.
//
// Rounding follows the bf16 module: LayerNorm output, fc1 output, GELU output
// and fc2 output are rounded to bf16 (fp32 accumulation and epilogues), and
// the residual add is fp32 rounded once.
#include "common.h"
#include "attn_core.h"
#include "gelu.h"

namespace terra {
namespace {

struct MlpParams {
  const uint8_t* x;
  uint8_t* y;
  const float* gamma;  // C floats or NULL (1)
  const float* beta;   // C floats or NULL (0)
  const uint16_t* w1;  // fc1.weight [H, C], fragment-packed
  const float* b1;     // H floats or NULL
  const uint16_t* w2;  // fc2.weight [C, H], fragment-packed
  const float* b2;     // C floats or NULL
  float eps;
  float inv_c;
  int32_t tokens;
  int32_t tiles;       // ceil(tokens / 64)
  int32_t layernorm;
};

constexpr int kMlpWaves = 12;
constexpr int kMlpThreads = 64 * kMlpWaves;
constexpr int kHC = 32 * kMlpWaves;  // hidden features per chunk: 32 per wave


// LDS: GELU table, b2, LayerNorm gamma and beta (C = 192; for C = 384 the
// LayerNorm reads them from global memory), raw rows (two tiles when double-
// buffered), LayerNorm tile, hidden chunk (reused for the fc2 k-split
// reduction).  b1 is read from global memory as the fc1 accumulator init.
template <int C>
constexpr bool mlp_affine_in_lds() {
  return C <= 192;
}
template <int C>
constexpr int mlp_rows_offset() {
  return kGeluBytes + (mlp_affine_in_lds<C>() ? 3 : 1) * C * 4;
}
template <int C, bool kDB>
constexpr int mlp_lds_bytes() {
  return mlp_rows_offset<C>() + (kDB ? 3 : 2) * 64 * C * 2 + 64 * kHC * 2;
}

__device__ __forceinline__ f32x4 load_f32x4_lds(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

// Packed weight fragment (row tile rt, k-step ks) of a [rows, kIn] weight,
// by buffer load: the wave-uniform 1 KB block offset in an SGPR, the lane's
// 16-byte offset in a VGPR (no per-lane 64-bit address per fragment).
// The low two bits of the k-step go to the instruction's immediate offset
// (k-steps 4 apart share one SGPR offset).
template <int kIn>
__device__ __forceinline__ uint4 packed_frag(__amdgpu_buffer_rsrc_t w, int rt, int ks, int lane) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(w, (uint32_t)lane * 16u + (uint32_t)(ks & 3) * 1024u,
                                                        (rt * (kIn / 32) + (ks & ~3)) * 1024, 0);
  return __builtin_bit_cast(uint4, v);
}

// Tiles in LDS: 64 rows of 16-byte chunks, stored as column blocks of kBlk =
// 24 chunks (384-byte rows): one block for a C = 192 tile, two for C = 384
// and for a hidden chunk.  Within a block, chunk b of row r sits in slot
// r * 24 + (b ^ ((r >> 1) & 7)): the 384-byte pitch puts odd rows half a
// bank period after even ones and the XOR spreads the row pairs over the 8
// 16-byte columns, so the 16 rows of a fragment read (and the 32 lanes of an
// 8-byte write) hit distinct banks.
constexpr int kBlk = 24;
constexpr int kBlkBytes = 64 * kBlk * 16;

__device__ __forceinline__ int mlp_slot(int row, int chunk) {
  const int b = chunk >= kBlk ? 1 : 0;  // chunk < 2 kBlk
  return b * (64 * kBlk) + row * kBlk + ((chunk - b * kBlk) ^ ((row >> 1) & 7));
}

// Byte offset of chunk c0 + g of row 16 tt + c16 (c0 a multiple of 4, g < 4)
// relative to the lane's base for parity (c0 >> 2) & 1, which is
// (c16 * kBlk + ((4 * parity + g) ^ sw)) * 16 with sw = (c16 >> 1) & 7.
constexpr int frag_off(int c0, int tt) {
  return (c0 / kBlk) * kBlkBytes + ((c0 % kBlk) >> 3) * 128 + tt * (16 * kBlk * 16);
}

// Rows [64 t, 64 t + 64) of x -> LDS (mlp_slot layout), direct global->LDS.
// Rows past the end load row 0 (never stored).
template <int kCpr>
__device__ __forceinline__ void mlp_fetch(const MlpParams& p, int t, uint8_t* dst, int wave, int lane) {
  constexpr int kRounds = kCpr / kMlpWaves;
  static_assert(kRounds * kMlpWaves == kCpr, "whole wave-rounds of 64 slots");
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * kMlpWaves + wave;
    const int sl = blk * 64 + lane;
    const int cb = sl >= 64 * kBlk ? 1 : 0;  // column block
    const int rem = sl - cb * (64 * kBlk);
    const int row = rem / kBlk;
    const int ch = cb * kBlk + ((rem - row * kBlk) ^ ((row >> 1) & 7));
    const int tok = t * 64 + row;
    const uint8_t* src = p.x + ((int64_t)(tok < p.tokens ? tok : 0) * kCpr + ch) * 16;
    dma_to_lds16(src, __builtin_amdgcn_readfirstlane(lds_address(dst + blk * 1024)));
  }
}

// The tile's rows -> y, whole lines; rows past the end are skipped.
template <int kCpr>
__device__ __forceinline__ void mlp_store(const MlpParams& p, int t, const uint8_t* xr, int tid) {
  constexpr int kRowStep = kMlpThreads / kCpr;
  static_assert(kRowStep * kCpr == kMlpThreads && 64 % kRowStep == 0, "whole rows per pass");
  const int row0 = tid / kCpr, ch = tid - row0 * kCpr;
  const int64_t first = (int64_t)t * 64;
  const int rows = p.tokens - (int)first < 64 ? p.tokens - (int)first : 64;
  const __amdgpu_buffer_rsrc_t out = buffer_rsrc(p.y + first * kCpr * 16, (uint32_t)(rows * kCpr * 16));
#pragma unroll
  for (int r = 0; r < 64 / kRowStep; ++r) {
    const int row = row0 + kRowStep * r;
    const u32x4 val = __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(xr + mlp_slot(row, ch) * 16));
    stream_store_sc1(val, out, (uint32_t)(row * kCpr + ch) * 16);  // rows past the end fall outside the range
  }
}

// LayerNorm of the 64 raw rows -> xn (bf16).  Eight lanes per token, the
// values held in registers; fp32 statistics from bf16 dot products
// (Bf16Moments, token_stats8; the variance recomputed from centred values
// where the mean is large against the spread); y = (x rstd - mean rstd)
// gamma + beta rounded once.  With layernorm == 0 the identity (mean 0,
// rstd 1, gamma 1, beta 0: the bits are copied).
template <int C, bool kAffineLds>
__device__ __forceinline__ void mlp_layernorm(const MlpParams& p, const uint8_t* xr, uint8_t* xn, const float* s_gamma,
                                              const float* s_beta, int tid) {
  // gamma and beta from LDS, or from global memory (then NULL means 1 / 0,
  // and without LayerNorm both are the identity)
  const float* gptr = kAffineLds ? s_gamma : (p.layernorm ? p.gamma : nullptr);
  const float* bptr = kAffineLds ? s_beta : (p.layernorm ? p.beta : nullptr);
  if constexpr (!kAffineLds) {
    // read per tile (not hoisted into registers for the whole kernel)
    asm volatile("" : "+s"(gptr), "+s"(bptr));
  }
  constexpr int kCpr = C / 8, kCPL = kCpr / 8;
  const int sub = tid & 7;
  for (int t = tid >> 3; t < 64; t += kMlpThreads / 8) {  // uniform per wave
    uint4 w[kCPL];
#pragma unroll
    for (int k = 0; k < kCPL; ++k) w[k] = *reinterpret_cast<const uint4*>(xr + mlp_slot(t, sub + 8 * k) * 16);
    float mean = 0.f, rstd = 1.f;
    if (p.layernorm) {
      Bf16Moments m;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) m.add4(w[k]);
      float var;
      token_stats8(m, p.inv_c, mean, var);
      if (token_stats_recheck(mean, var)) {  // uniform per wave
        asm volatile("" : "+v"(mean));  // keeps this rare pass a branch, not computed on every path
        float sq = 0.f;
#pragma unroll
        for (int k = 0; k < kCPL; ++k) sq = centred_sq4(w[k], mean, sq);
        var = group8_sum(sq) * p.inv_c;
      }
      rstd = rsqrtf(fmaxf(var, 0.f) + p.eps);
    }
    const float nmr = -mean * rstd;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const int c0 = (sub + 8 * k) * 8;
      float gv[8], bv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 gq = gptr != nullptr ? *reinterpret_cast<const f32x4*>(gptr + c0 + 4 * h) : f32x4{1.f, 1.f, 1.f, 1.f};
        const f32x4 bq = bptr != nullptr ? *reinterpret_cast<const f32x4*>(bptr + c0 + 4 * h) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gv[4 * h + e] = gq[e];
          bv[4 * h + e] = bq[e];
        }
      }
      *reinterpret_cast<uint4*>(xn + mlp_slot(t, sub + 8 * k) * 16) = normalize_chunk(w[k], rstd, nmr, gv, bv);
    }
  }
}

template <int C, bool kDB>
__global__ __launch_bounds__(kMlpThreads) void swin_mlp_kernel(const MlpParams p) {
  constexpr int H = 4 * C;
  constexpr int kCpr = C / 8;
  constexpr int kTile = 64 * C * 2;
  constexpr int kChunks = H / kHC;
  constexpr int kNF = C / 32;                  // fc2 feature groups of 32
  constexpr int kKS = kMlpWaves / kNF;         // fc2 k-split (2 for C = 192, 1 for C = 384)
  constexpr int kKR = kHC / kKS;               // fc2 k range per wave and chunk
  constexpr int kSteps1 = C / 32;              // fc1 k-steps
  constexpr int kSteps2 = kKR / 32;            // fc2 k-steps per chunk
  static_assert(kNF * kKS == kMlpWaves && kCpr % kBlk == 0 && kCpr <= 2 * kBlk && (kKR / 8) % kBlk == 0, "shapes");
  static_assert(kKS <= 2 && (kKS == 1 || 64 * C * 4 <= 64 * kHC * 2), "the fc2 reduction reuses the hidden chunk");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* s_gelu = reinterpret_cast<uint16_t*>(smem);
  float* s_b2 = reinterpret_cast<float*>(smem + kGeluBytes);
  float* s_gamma = s_b2 + C;  // C = 192 only
  float* s_beta = s_gamma + C;
  uint8_t* xbuf = smem + mlp_rows_offset<C>();            // raw rows: 1 or 2 tiles
  uint8_t* xn = xbuf + (kDB ? 2 : 1) * kTile;
  uint8_t* hb = xn + kTile;                               // hidden chunk [64][kHC] bf16

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  if ((int)blockIdx.x >= p.tiles) return;  // uniform
  for (int i = tid; i < C; i += kMlpThreads) {
    // Without LayerNorm the normalisation below is the identity (mean 0, rstd 1, gamma 1, beta 0).
    if constexpr (mlp_affine_in_lds<C>()) {
      s_gamma[i] = p.layernorm && p.gamma != nullptr ? p.gamma[i] : 1.f;
      s_beta[i] = p.layernorm && p.beta != nullptr ? p.beta[i] : 0.f;
    }
    s_b2[i] = p.b2 != nullptr ? p.b2[i] : 0.f;
  }
  gelu_table_fill(s_gelu, tid, kMlpThreads);

  const int fr = wave % kNF, kh = wave / kNF;
  const __amdgpu_buffer_rsrc_t w1r = buffer_rsrc(p.w1, (uint32_t)(H * C * 2));
  const __amdgpu_buffer_rsrc_t w2r = buffer_rsrc(p.w2, (uint32_t)(H * C * 2));  // fc2: features [32 fr, +32), k part kh
  // Per-lane LDS byte offsets (see frag_off): every fragment address below
  // is one of two bases plus a constant.
  const int sw = (c16 >> 1) & 7;
  uint32_t fa[2], hw[2], rw[2];
  const int wl = wave % 6, fl = fr % 6;  // 4-chunk column groups within a block
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    fa[q] = (c16 * kBlk + ((4 * q + g) ^ sw)) * 16;  // MFMA B operand reads
    // GELU output: hidden columns 32 wave + 16 q + 4 g .. +3 (chunk 4 wave + 2 q + g / 2)
    hw[q] = (wave / 6) * kBlkBytes + (c16 * kBlk + 8 * (wl >> 1) + ((4 * (wl & 1) + 2 * q + (g >> 1)) ^ sw)) * 16 +
            (g & 1) * 8;
    // residual: features 32 fr + 16 q + 4 g .. +3
    rw[q] = (fr / 6) * kBlkBytes + (c16 * kBlk + 8 * (fl >> 1) + ((4 * (fl & 1) + 2 * q + (g >> 1)) ^ sw)) * 16 +
            (g & 1) * 8;
  }

  int t = blockIdx.x, prev = -1, par = 0;
  mlp_fetch<kCpr>(p, t, xbuf, wave, lane);
  for (;;) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile's rows have landed
    lds_barrier();
    uint8_t* xr = xbuf + (kDB ? par * kTile : 0);
    const int next = t + (int)gridDim.x;
    if constexpr (kDB) {
      if (prev >= 0) mlp_store<kCpr>(p, prev, xbuf + (par ^ 1) * kTile, tid);  // the previous tile's rows
    }
    mlp_layernorm<C, mlp_affine_in_lds<C>()>(p, xr, xn, s_gamma, s_beta, tid);
    lds_barrier();  // xn complete; the previous tile's rows are read out of the other buffer

    f32x4 acc2[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x4 b = kh == 0 ? load_f32x4_lds(s_b2 + 32 * fr + 16 * i + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc2[i][tt] = b;
    }
    for (int chk = 0; chk < kChunks; ++chk) {
      // ---- fc1 + bias: hidden [chk*kHC + 32 wave, +32) x 64 tokens ----------
      const int rt1 = chk * (kHC / 16) + 2 * wave;
      f32x4 acc1[2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f32x4 b = p.b1 != nullptr ? *reinterpret_cast<const f32x4*>(p.b1 + 16 * (rt1 + i) + 4 * g)
                                         : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc1[i][tt] = b;
      }
      {
        uint4 wf[3][2];  // weight ring: step ks in slot ks % 3, loaded two steps ahead
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0)
#pragma unroll
          for (int i = 0; i < 2; ++i) wf[s0][i] = packed_frag<C>(w1r, rt1 + i, s0, lane);
#pragma unroll
        for (int ks = 0; ks < kSteps1; ++ks) {
          if (ks + 2 < kSteps1) {
#pragma unroll
            for (int i = 0; i < 2; ++i) wf[(ks + 2) % 3][i] = packed_frag<C>(w1r, rt1 + i, ks + 2, lane);
          }
          // Compiler barrier: without it the scheduler sinks each weight load
          // to just before its MFMA (least register pressure), which exposes
          // the whole L2 latency of every fragment.
          asm volatile("" ::: "memory");
          uint4 xf[4];
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            xf[tt] = *reinterpret_cast<const uint4*>(xn + fa[ks & 1] + frag_off(4 * ks, tt));
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              acc1[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[ks % 3][i]),
                                                                    __builtin_bit_cast(bf16x8, xf[tt]), acc1[i][tt],
                                                                    0, 0, 0);
        }
      }
      if constexpr (kDB) {
        // The next tile's rows stream in under the GELU epilogue (the first
        // later wait on a global load also waits for them).
        if (chk == 0 && next < p.tiles) mlp_fetch<kCpr>(p, next, xbuf + (par ^ 1) * kTile, wave, lane);
      }
      // ---- bf16 -> GELU -> bf16 into the hidden chunk -------------------------
      // lane (c16, g) of (i, tt): hidden 16 i + 4 g + r of token 16 tt + c16.
      // Table lookups for all values; if any lane holds a value outside the
      // table (|x| < 2^-22 or >= 32: rare), the wave redoes the chunk exactly.
      {
        uint32_t hp[2][4][2], gp[2][4][2];
        u16x2 dmax = {0, 0};
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            hp[i][tt][0] = pack_bf16x2(acc1[i][tt][0], acc1[i][tt][1]);
            hp[i][tt][1] = pack_bf16x2(acc1[i][tt][2], acc1[i][tt][3]);
            // the packed pairs are the operands from here on (no per-half re-conversion)
            asm volatile("" : "+v"(hp[i][tt][0]), "+v"(hp[i][tt][1]));
            gp[i][tt][0] = gelu_pair_table(hp[i][tt][0], s_gelu, dmax);
            gp[i][tt][1] = gelu_pair_table(hp[i][tt][1], s_gelu, dmax);
          }
        const uint32_t dm = dmax.x > dmax.y ? dmax.x : dmax.y;
        if (__builtin_amdgcn_ballot_w64(dm >= (uint32_t)kGeluSpan) != 0) {
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
              for (int q = 0; q < 2; ++q)
                gp[i][tt][q] = gelu_bf16(hp[i][tt][q] & 0xffffu, s_gelu) | (gelu_bf16(hp[i][tt][q] >> 16, s_gelu) << 16);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            *reinterpret_cast<uint2*>(hb + hw[i] + tt * (16 * kBlk * 16)) = make_uint2(gp[i][tt][0], gp[i][tt][1]);
      }
      lds_barrier();  // hidden chunk complete
      // ---- fc2 partial: features [32 fr, +32), hidden [kh*kKR, +kKR) of the chunk ----
      {
        const int ks0 = (chk * kHC + kh * kKR) / 32;  // k-step of this wave's first hidden column
        uint4 wf[3][2];
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0)
#pragma unroll
          for (int i = 0; i < 2; ++i) wf[s0][i] = packed_frag<H>(w2r, 2 * fr + i, ks0 + s0, lane);
#pragma unroll
        for (int s = 0; s < kSteps2; ++s) {
          if (s + 2 < kSteps2) {
#pragma unroll
            for (int i = 0; i < 2; ++i) wf[(s + 2) % 3][i] = packed_frag<H>(w2r, 2 * fr + i, ks0 + s + 2, lane);
          }
          asm volatile("" ::: "memory");  // keeps the weight loads two steps ahead (see fc1)
          uint4 hf[4];
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            hf[tt] = *reinterpret_cast<const uint4*>(hb + fa[s & 1] + kh * (kKR / 8 / kBlk) * kBlkBytes +
                                                     frag_off(4 * s, tt));
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              acc2[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[s % 3][i]),
                                                                    __builtin_bit_cast(bf16x8, hf[tt]), acc2[i][tt],
                                                                    0, 0, 0);
        }
      }
      lds_barrier();  // the chunk is consumed before the next one overwrites it
    }

    // ---- fc2 k-split reduction, + bias, residual ---------------------------
    // lane (c16, g) of (i, tt): features 32 fr + 16 i + 4 g + r of token 16 tt + c16.
    // With the k-split, part kh finishes token tiles tt in [2 kh, 2 kh + 2)
    // and hands the other two to its partner through the idle hidden chunk
    // (fp32, 16-byte chunks XOR-swizzled by c16 against bank conflicts).
    if constexpr (kKS == 2) {
      float* red = reinterpret_cast<float*>(hb);  // [64][C] fp32
      const int rc = ((8 * fr + g) ^ c16);  // 16-byte chunk of 32 fr + 4 g (+ 16 i: chunk ^ 4 i)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          if ((tt >> 1) != kh) *reinterpret_cast<f32x4*>(red + (16 * tt + c16) * C + 4 * (rc ^ (4 * i))) = acc2[i][tt];
      lds_barrier();
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          if ((tt >> 1) == kh) acc2[i][tt] += *reinterpret_cast<const f32x4*>(red + (16 * tt + c16) * C + 4 * (rc ^ (4 * i)));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        if (kKS == 2 && (tt >> 1) != kh) continue;
        uint8_t* addr = xr + rw[i] + tt * (16 * kBlk * 16);
        const uint2 xv = *reinterpret_cast<const uint2*>(addr);
        uint2 out;
        out.x = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv.x & 0xffffu)) + (float)(__bf16)acc2[i][tt][0],
                            bf16_bits_to_f32((uint16_t)(xv.x >> 16)) + (float)(__bf16)acc2[i][tt][1]);
        out.y = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv.y & 0xffffu)) + (float)(__bf16)acc2[i][tt][2],
                            bf16_bits_to_f32((uint16_t)(xv.y >> 16)) + (float)(__bf16)acc2[i][tt][3]);
        *reinterpret_cast<uint2*>(addr) = out;
      }
    if constexpr (!kDB) {
      lds_barrier();                                 // output rows complete
      mlp_store<kCpr>(p, t, xr, tid);
      if (next >= p.tiles) break;
      lds_barrier();                                 // the rows are read out before the next load
      mlp_fetch<kCpr>(p, next, xbuf, wave, lane);
      t = next;
    } else {
      prev = t;
      if (next >= p.tiles) {
        lds_barrier();                               // output rows complete
        mlp_store<kCpr>(p, t, xr, tid);
        break;
      }
      t = next;
      par ^= 1;
    }
  }
}

// ============================================================================
// swin_mlp_wide_kernel: the same MLP half for C = 128 (c2) and C = 768 (the
// reference model's C, c4).
// ============================================================================
//
// The same per-tile scheme as swin_mlp_kernel (64-token tiles, LayerNorm
// tile, hidden chunks of 32 features per wave on chip, fc2 accumulators
// across the chunks), sized for these widths:
//   C = 128: 8 waves, hidden chunks of 256 (two per tile), fc2 split in two
//            along k (as C = 192), raw rows double-buffered in LDS;
//   C = 768: 8 waves, hidden chunks of 256 (twelve per tile), each wave owns
//            96 fc2 output features (no k split).  The raw rows land in the
//            LayerNorm tile and are normalised in place (a 96 KB tile; a
//            second one does not fit beside the hidden chunk), the residual
//            is read back from global memory in the epilogue, and the output
//            rows are staged in the same tile for whole-line stores.
// Row pitches here are multiples of 256 bytes (a whole bank period), so a
// 16-byte chunk c of row r sits in slot r * pitch + (c ^ (r & 15)) (XOR
// within aligned groups of 16 chunks): the 16 rows of a fragment read land
// on 16 different 16-byte bank groups.  The affine parameters and biases are
// read from global memory (L1-resident).

template <int C>
struct WideShape {
  static constexpr int kWaves = 8;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int H = 4 * C;
  static constexpr int kCpr = C / 8;                  // 16-byte chunks per x row
  static constexpr int kHC = 32 * kWaves;             // hidden features per chunk
  static constexpr int kHCpr = kHC / 8;               // chunks per hidden row
  static constexpr int kChunks = H / kHC;
  static constexpr int kNF = C / 32;                  // fc2 feature groups of 32
  static constexpr int kFPW = kNF >= kWaves ? kNF / kWaves : 1;  // groups per wave
  static constexpr int kKS = kNF >= kWaves ? 1 : kWaves / kNF;   // fc2 k split
  static constexpr int kKR = kHC / kKS;               // fc2 k range per wave and chunk
  static constexpr bool kRaw = C <= 384;              // raw rows in LDS (double-buffered)
  static constexpr int kTile = 64 * C * 2;
  static constexpr int kHid = 64 * kHC * 2;
  static constexpr int kLds = kGeluBytes + (kRaw ? 3 : 1) * kTile + kHid;
  static_assert(kChunks * kHC == H && kKS * kKR == kHC && kKS <= 2, "chunking");
  static_assert(kFPW * kWaves * (kKS == 1 ? 1 : 0) + (kKS == 2 ? kNF * 2 : 0) == (kKS == 1 ? kNF : kWaves),
                "fc2 split");
  static_assert(kCpr % 16 == 0 && kHCpr % 16 == 0, "256-byte row pitches");
  static_assert(kKS == 1 || 64 * C * 4 <= kHid, "the fc2 reduction reuses the hidden chunk");
  static_assert(kLds <= 160 * 1024, "LDS");
};

template <int kPitch>
__device__ __forceinline__ int wide_slot(int row, int chunk) {
  return row * kPitch + (chunk ^ (row & 15));
}

// Rows [64 t, +64) of x -> LDS tile (wide_slot layout), direct global->LDS;
// rows past the end load row 0 (never stored).
template <int C>
__device__ __forceinline__ void wide_fetch(const MlpParams& p, int t, uint8_t* dst, int wave, int lane) {
  using S = WideShape<C>;
  constexpr int kRounds = S::kCpr * 64 / (64 * S::kWaves);
  static_assert(kRounds * S::kWaves == S::kCpr, "whole wave-rounds");
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int blk = r * S::kWaves + wave;
    const int sl = blk * 64 + lane;
    const int row = sl / S::kCpr;
    const int ch = (sl - row * S::kCpr) ^ (row & 15);
    const int tok = t * 64 + row;
    const uint8_t* src = p.x + ((int64_t)(tok < p.tokens ? tok : 0) * S::kCpr + ch) * 16;
    // At C = 768 the epilogue reads the rows again from global memory for
    // the residual: no streaming hint, so they stay in L2.
    if constexpr (S::kRaw)
      dma_to_lds16(src, __builtin_amdgcn_readfirstlane(lds_address(dst + blk * 1024)));
    else
      dma_to_lds16_cached(src, __builtin_amdgcn_readfirstlane(lds_address(dst + blk * 1024)));
  }
}

template <int C>
__device__ __forceinline__ void wide_store(const MlpParams& p, int t, const uint8_t* xr, int tid) {
  using S = WideShape<C>;
  constexpr int kPasses = 64 * S::kCpr / S::kThreads;
  static_assert(kPasses * S::kThreads == 64 * S::kCpr, "whole passes");
  const int64_t first = (int64_t)t * 64;
  const int rows = p.tokens - (int)first < 64 ? p.tokens - (int)first : 64;
  const __amdgpu_buffer_rsrc_t out = buffer_rsrc(p.y + first * S::kCpr * 16, (uint32_t)(rows * S::kCpr * 16));
#pragma unroll
  for (int r = 0; r < kPasses; ++r) {
    const int q = r * S::kThreads + tid;  // consecutive lanes, consecutive chunks of the tile's rows
    const int row = q / S::kCpr, ch = q - row * S::kCpr;
    const u32x4 val =
        __builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(xr + wide_slot<S::kCpr>(row, ch) * 16));
    stream_store_sc1(val, out, (uint32_t)q * 16);  // rows past the end fall outside the range
  }
}

// LayerNorm of the tile's raw rows (xr) into xn (may be xr: in place, each
// lane rewriting only the chunks it read).  Eight lanes per token; fp32
// statistics from bf16 dot products (Bf16Moments, token_stats8; the variance
// recomputed from centred values where the mean is large against the
// spread), the rows read from LDS once for the statistics and once for the
// output; without LayerNorm the identity.
template <int C>
__device__ __forceinline__ void wide_layernorm(const MlpParams& p, const uint8_t* xr, uint8_t* xn, int tid) {
  using S = WideShape<C>;
  constexpr int kCPL = S::kCpr / 8;
  const int sub = tid & 7;
  const float* gptr = p.layernorm ? p.gamma : nullptr;
  const float* bptr = p.layernorm ? p.beta : nullptr;
  asm volatile("" : "+s"(gptr), "+s"(bptr));  // read per tile, not held in registers
  auto raw = [&](int t, int k) {
    return *reinterpret_cast<const uint4*>(xr + wide_slot<S::kCpr>(t, sub + 8 * k) * 16);
  };
  for (int t = tid >> 3; t < 64; t += S::kThreads / 8) {  // uniform per wave
    float mean = 0.f, rstd = 1.f;
    if (p.layernorm) {
      Bf16Moments m;
#pragma unroll
      for (int k = 0; k < kCPL; ++k) m.add4(raw(t, k));
      float var;
      token_stats8(m, p.inv_c, mean, var);
      if (token_stats_recheck(mean, var)) {  // uniform per wave
        asm volatile("" : "+v"(mean));  // keeps this rare pass a branch, not computed on every path
        float sq = 0.f;
#pragma unroll
        for (int k = 0; k < kCPL; ++k) sq = centred_sq4(raw(t, k), mean, sq);
        var = group8_sum(sq) * p.inv_c;
      }
      rstd = rsqrtf(fmaxf(var, 0.f) + p.eps);
    }
    const float nmr = -mean * rstd;
#pragma unroll
    for (int k = 0; k < kCPL; ++k) {
      const int c0 = (sub + 8 * k) * 8;
      float gv[8], bv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 gq = gptr != nullptr ? *reinterpret_cast<const f32x4*>(gptr + c0 + 4 * h) : f32x4{1.f, 1.f, 1.f, 1.f};
        const f32x4 bq = bptr != nullptr ? *reinterpret_cast<const f32x4*>(bptr + c0 + 4 * h) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gv[4 * h + e] = gq[e];
          bv[4 * h + e] = bq[e];
        }
      }
      *reinterpret_cast<uint4*>(xn + wide_slot<S::kCpr>(t, sub + 8 * k) * 16) =
          normalize_chunk(raw(t, k), rstd, nmr, gv, bv);
    }
  }
}

template <int C>
__global__ __launch_bounds__(WideShape<C>::kThreads) void swin_mlp_wide_kernel(const MlpParams p) {
  using S = WideShape<C>;
  constexpr int H = S::H, kCpr = S::kCpr, kHCpr = S::kHCpr;
  constexpr int kSteps1 = C / 32;          // fc1 k-steps
  constexpr int kSteps2 = S::kKR / 32;     // fc2 k-steps per chunk
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* s_gelu = reinterpret_cast<uint16_t*>(smem);
  uint8_t* tiles = smem + kGeluBytes;
  uint8_t* xbuf = tiles;                                        // raw rows (kRaw: two tiles)
  uint8_t* xn = S::kRaw ? tiles + 2 * S::kTile : tiles;         // LayerNorm tile (kRaw off: also the raw rows)
  uint8_t* hb = xn + S::kTile;                                  // hidden chunk [64][kHC] bf16

  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  if ((int)blockIdx.x >= p.tiles) return;  // uniform
  for (int e = tid0; e < 2 * kGeluSpan; e += S::kThreads) {
    const uint32_t sign = e >= kGeluSpan ? 0x8000u : 0u;
    const uint32_t bits = sign | (kGeluLo + (uint32_t)(e - (sign ? kGeluSpan : 0)));
    const float xv = bf16_bits_to_f32((uint16_t)bits);
    s_gelu[e] = f32_to_bf16_bits(xv * 0.5f * (1.f + erff(xv * 0.70710678118654752f)));
  }
  const int fr = S::kKS == 1 ? wave : wave % S::kNF;  // fc2 feature groups fr * kFPW + f
  const int kh = S::kKS == 1 ? 0 : wave / S::kNF;     // fc2 k part
  const __amdgpu_buffer_rsrc_t w1r = buffer_rsrc(p.w1, (uint32_t)(H * C * 2));
  const __amdgpu_buffer_rsrc_t w2r = buffer_rsrc(p.w2, (uint32_t)(H * C * 2));

  int t = blockIdx.x, prev = -1, par = 0;
  wide_fetch<C>(p, t, S::kRaw ? xbuf : xn, wave, tid0 & 63);
  for (;;) {
    // Lane-derived addresses are recomputed per tile (the thread id passes
    // through an empty asm) rather than hoisted and held across the loop.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    // Per-lane bases of fragment reads: chunk 16 a + 4 b + g of row 16 tt + c16
    // is at fa(b) + 256 a + tt * 16 * pitch * 16 (wide_slot with row & 15 = c16).
    auto fa = [&](int pitch, int b) { return (uint32_t)((c16 * pitch + ((4 * b + g) ^ c16)) * 16); };
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile's rows have landed
    lds_barrier();
    uint8_t* xr = S::kRaw ? xbuf + par * S::kTile : xn;
    const int next = t + (int)gridDim.x;
    if constexpr (S::kRaw) {
      if (prev >= 0) wide_store<C>(p, prev, xbuf + (par ^ 1) * S::kTile, tid);  // the previous tile's rows
    }
    wide_layernorm<C>(p, xr, xn, tid);
    lds_barrier();  // xn complete

    f32x4 acc2[S::kFPW][2][4];
#pragma unroll
    for (int f = 0; f < S::kFPW; ++f)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int fb = 32 * (fr * S::kFPW + f) + 16 * i + 4 * g;
        const f32x4 b = (kh == 0 && p.b2 != nullptr) ? *reinterpret_cast<const f32x4*>(p.b2 + fb)
                                                      : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc2[f][i][tt] = b;
      }
    for (int chk = 0; chk < S::kChunks; ++chk) {
      // ---- fc1 + bias: hidden [chk kHC + 32 wave, +32) x 64 tokens ----------
      const int rt1 = chk * (S::kHC / 16) + 2 * wave;
      f32x4 acc1[2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f32x4 b = p.b1 != nullptr ? *reinterpret_cast<const f32x4*>(p.b1 + 16 * (rt1 + i) + 4 * g)
                                         : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc1[i][tt] = b;
      }
      {
        uint4 wf[3][2];  // weight ring: step ks in slot ks % 3, loaded two steps ahead
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0)
#pragma unroll
          for (int i = 0; i < 2; ++i) wf[s0][i] = packed_frag<C>(w1r, rt1 + i, s0, lane);
#pragma unroll
        for (int ks = 0; ks < kSteps1; ++ks) {
          if (ks + 2 < kSteps1) {
#pragma unroll
            for (int i = 0; i < 2; ++i) wf[(ks + 2) % 3][i] = packed_frag<C>(w1r, rt1 + i, ks + 2, lane);
          }
          asm volatile("" ::: "memory");  // keeps the weight loads two steps ahead
          uint4 xf[4];
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            xf[tt] = *reinterpret_cast<const uint4*>(xn + fa(kCpr, ks & 3) + (ks >> 2) * 256 + tt * (16 * kCpr * 16));
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              acc1[i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[ks % 3][i]),
                                                                    __builtin_bit_cast(bf16x8, xf[tt]), acc1[i][tt],
                                                                    0, 0, 0);
        }
      }
      if constexpr (S::kRaw) {
        // The next tile's rows stream in under the GELU epilogue.
        if (chk == 0 && next < p.tiles) wide_fetch<C>(p, next, xbuf + (par ^ 1) * S::kTile, wave, lane);
      }
      // ---- bf16 -> GELU -> bf16 into the hidden chunk -------------------------
      {
        uint32_t hp[2][4][2], gp[2][4][2];
        u16x2 dmax = {0, 0};
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            hp[i][tt][0] = pack_bf16x2(acc1[i][tt][0], acc1[i][tt][1]);
            hp[i][tt][1] = pack_bf16x2(acc1[i][tt][2], acc1[i][tt][3]);
            asm volatile("" : "+v"(hp[i][tt][0]), "+v"(hp[i][tt][1]));
            gp[i][tt][0] = gelu_pair_table(hp[i][tt][0], s_gelu, dmax);
            gp[i][tt][1] = gelu_pair_table(hp[i][tt][1], s_gelu, dmax);
          }
        const uint32_t dm = dmax.x > dmax.y ? dmax.x : dmax.y;
        if (__builtin_amdgcn_ballot_w64(dm >= (uint32_t)kGeluSpan) != 0) {
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
              for (int q = 0; q < 2; ++q)
                gp[i][tt][q] = gelu_bf16(hp[i][tt][q] & 0xffffu, s_gelu) | (gelu_bf16(hp[i][tt][q] >> 16, s_gelu) << 16);
        }
        // lane (c16, g) of (i, tt): hidden 32 wave + 16 i + 4 g .. + 3 of token 16 tt + c16
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const int row = 16 * tt + c16;
            const int ch = (32 * wave + 16 * i + 4 * g) >> 3;
            *reinterpret_cast<uint2*>(hb + wide_slot<kHCpr>(row, ch) * 16 + (g & 1) * 8) =
                make_uint2(gp[i][tt][0], gp[i][tt][1]);
          }
      }
      lds_barrier();  // hidden chunk complete
      // ---- fc2 partial: feature groups fr kFPW + f, hidden [kh kKR, +kKR) of the chunk ----
      {
        const int ks0 = (chk * S::kHC + kh * S::kKR) / 32;
        uint4 wf[3][S::kFPW][2];
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0)
#pragma unroll
          for (int f = 0; f < S::kFPW; ++f)
#pragma unroll
            for (int i = 0; i < 2; ++i) wf[s0][f][i] = packed_frag<H>(w2r, 2 * (fr * S::kFPW + f) + i, ks0 + s0, lane);
#pragma unroll
        for (int s = 0; s < kSteps2; ++s) {
          if (s + 2 < kSteps2) {
#pragma unroll
            for (int f = 0; f < S::kFPW; ++f)
#pragma unroll
              for (int i = 0; i < 2; ++i)
                wf[(s + 2) % 3][f][i] = packed_frag<H>(w2r, 2 * (fr * S::kFPW + f) + i, ks0 + s + 2, lane);
          }
          asm volatile("" ::: "memory");
          const int kc = (kh * S::kKR) / 8 + 4 * s;  // first chunk of this k-step within the hidden row
          uint4 hf[4];
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            hf[tt] = *reinterpret_cast<const uint4*>(hb + fa(kHCpr, (kc >> 2) & 3) + (kc >> 4) * 256 +
                                                     tt * (16 * kHCpr * 16));
#pragma unroll
          for (int f = 0; f < S::kFPW; ++f)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
              for (int tt = 0; tt < 4; ++tt)
                acc2[f][i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, wf[s % 3][f][i]), __builtin_bit_cast(bf16x8, hf[tt]), acc2[f][i][tt],
                    0, 0, 0);
        }
      }
      lds_barrier();  // the chunk is consumed before the next one overwrites it
    }

    // ---- fc2 k-split reduction (C = 128), + residual -------------------------
    // lane (c16, g) of (f, i, tt): features 32 (fr kFPW + f) + 16 i + 4 g + r of token 16 tt + c16.
    if constexpr (S::kKS == 2) {
      float* red = reinterpret_cast<float*>(hb);  // [64][C] fp32, 16-byte chunks XOR-swizzled by c16
      const int rc = ((8 * fr + g) ^ c16);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          if ((tt >> 1) != kh) *reinterpret_cast<f32x4*>(red + (16 * tt + c16) * C + 4 * (rc ^ (4 * i))) = acc2[0][i][tt];
      lds_barrier();
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          if ((tt >> 1) == kh)
            acc2[0][i][tt] += *reinterpret_cast<const f32x4*>(red + (16 * tt + c16) * C + 4 * (rc ^ (4 * i)));
    }
    const __amdgpu_buffer_rsrc_t xres =
        buffer_rsrc(p.x + (int64_t)t * 64 * C * 2,
                    (uint32_t)((p.tokens - t * 64 < 64 ? p.tokens - t * 64 : 64) * C * 2));
#pragma unroll
    for (int f = 0; f < S::kFPW; ++f)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          if (S::kKS == 2 && (tt >> 1) != kh) continue;
          const int row = 16 * tt + c16;
          const int fb = 32 * (fr * S::kFPW + f) + 16 * i + 4 * g;
          uint8_t* addr = xr + wide_slot<kCpr>(row, fb >> 3) * 16 + (fb & 7) * 2;
          uint2 xv;
          if constexpr (S::kRaw) {
            xv = *reinterpret_cast<const uint2*>(addr);
          } else {  // from global memory (rows past the end read 0 and are not stored)
            const stream_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(xres, (uint32_t)(row * C + fb) * 2, 0, 0);
            xv = make_uint2(v[0], v[1]);
          }
          const f32x4& a = acc2[f][i][tt];
          uint2 out;
          out.x = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv.x & 0xffffu)) + (float)(__bf16)a[0],
                              bf16_bits_to_f32((uint16_t)(xv.x >> 16)) + (float)(__bf16)a[1]);
          out.y = pack_bf16x2(bf16_bits_to_f32((uint16_t)(xv.y & 0xffffu)) + (float)(__bf16)a[2],
                              bf16_bits_to_f32((uint16_t)(xv.y >> 16)) + (float)(__bf16)a[3]);
          *reinterpret_cast<uint2*>(addr) = out;
        }
    if constexpr (!S::kRaw) {
      lds_barrier();                                 // output rows complete
      wide_store<C>(p, t, xr, tid);
      if (next >= p.tiles) break;
      lds_barrier();                                 // the rows are read out before the next load
      wide_fetch<C>(p, next, xn, wave, lane);
      t = next;
    } else {
      prev = t;
      if (next >= p.tiles) {
        lds_barrier();                               // output rows complete
        wide_store<C>(p, t, xr, tid);
        break;
      }
      t = next;
      par ^= 1;
    }
  }
}

template <int C>
int launch_mlp_wide(const MlpParams& p, hipStream_t s) {
  using S = WideShape<C>;
  auto kern = swin_mlp_wide_kernel<C>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, S::kLds);
  if (attr != hipSuccess) return fail(TERRA_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, S::kThreads, S::kLds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the MLP grid for this device");
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  const int blocks = p.tiles < cache[dev] ? p.tiles : cache[dev];
  kern<<<blocks, S::kThreads, S::kLds, s>>>(p);
  return TERRA_OK;
}

template <int C, bool kDB>
int launch_mlp(const MlpParams& p, hipStream_t s) {
  constexpr int lds = mlp_lds_bytes<C, kDB>();
  static_assert(lds <= 160 * 1024, "LDS");
  auto kern = swin_mlp_kernel<C, kDB>;
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
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kMlpThreads, lds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the MLP grid for this device");
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  const int blocks = p.tiles < cache[dev] ? p.tiles : cache[dev];
  kern<<<blocks, kMlpThreads, lds, s>>>(p);
  return TERRA_OK;
}

bool mlp_ranges_overlap(const void* a, const void* b, int64_t bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)bytes && y < x + (uintptr_t)bytes;
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_mlp_fwd(const void* x, void* y, int dtype, const terra_swin_mlp_desc* desc,
                                  const float* ln_gamma, const float* ln_beta, const void* fc1_weight,
                                  const float* fc1_bias, const void* fc2_weight, const float* fc2_bias,
                                  void* stream) {
  clear_error();
  if (desc == nullptr) return fail(TERRA_ERR_NULL, "desc is NULL");
  if (x == nullptr || y == nullptr || fc1_weight == nullptr || fc2_weight == nullptr)
    return fail(TERRA_ERR_NULL, "x, y and the packed fc1 / fc2 weights must be non-NULL");
  if (dtype_size(dtype) == 0) return fail(TERRA_ERR_DTYPE, "unknown dtype %d", dtype);
  if (dtype != TERRA_DTYPE_BF16) return fail(TERRA_ERR_UNSUPPORTED, "the fused MLP is built for bf16 activations");
  const terra_swin_mlp_desc& d = *desc;
  if (d.tokens <= 0) return fail(TERRA_ERR_SHAPE, "tokens must be positive");
  if (d.channels != 128 && d.channels != 192 && d.channels != 384 && d.channels != 768)
    return fail(TERRA_ERR_UNSUPPORTED, "channels %d not in {128, 192, 384, 768}", d.channels);
  if (d.hidden != 4 * d.channels)
    return fail(TERRA_ERR_UNSUPPORTED, "hidden %d != 4 * channels (%d)", d.hidden, 4 * d.channels);
  if (!(d.ln_eps >= 0.f)) return fail(TERRA_ERR_SHAPE, "ln_eps must be >= 0");
  for (const void* ptr : {x, (const void*)y, fc1_weight, fc2_weight, (const void*)ln_gamma, (const void*)ln_beta,
                          (const void*)fc1_bias, (const void*)fc2_bias})
    if (((uintptr_t)ptr & 15u) != 0) return fail(TERRA_ERR_ALIGN, "tensors must be 16-byte aligned");
  const int64_t bytes = (int64_t)d.tokens * d.channels * 2;
  if (bytes >= (1ll << 32)) return fail(TERRA_ERR_SHAPE, "x must be under 4 GiB; split the tokens");
  if (x != y && mlp_ranges_overlap(x, y, bytes)) return fail(TERRA_ERR_SHAPE, "y overlaps x without being x");

  MlpParams p;
  memset(&p, 0, sizeof(p));
  p.x = static_cast<const uint8_t*>(x);
  p.y = static_cast<uint8_t*>(y);
  p.gamma = ln_gamma;
  p.beta = ln_beta;
  p.w1 = static_cast<const uint16_t*>(fc1_weight);
  p.b1 = fc1_bias;
  p.w2 = static_cast<const uint16_t*>(fc2_weight);
  p.b2 = fc2_bias;
  p.eps = d.ln_eps;
  p.inv_c = 1.f / (float)d.channels;
  p.tokens = d.tokens;
  p.tiles = (d.tokens + 63) / 64;
  p.layernorm = d.layernorm != 0;
  hipStream_t s = (hipStream_t)stream;
  int st;
  switch (d.channels) {
    case 128: st = launch_mlp_wide<128>(p, s); break;
    case 192: st = launch_mlp<192, true>(p, s); break;
    case 384: st = launch_mlp<384, false>(p, s); break;
    default: st = launch_mlp_wide<768>(p, s); break;
  }
  if (st != TERRA_OK) return st;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_mlp_fwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
