// Token-row linear layers with fused epilogues for gfx950 (bf16), the GEMM
// side of the C = 1024 half-blocks:
//
//   acc[m][f] = b[f] + sum_k x[m][k] W[f][k]      fp32 accumulation on MFMA
//
// followed by one of
//
//   store     y[m]    = bf16(acc)                              (nn.Linear)
//   gelu      y[m]    = GELU(bf16(acc))                        (fc1 + nn.GELU)
//   residual  y[m]    = bf16(r[m] + bf16(acc))                 (fc2 + shortcut)
//   scatter   y[t(m)] = bf16(r[t(m)] + bf16(acc))              (proj + window
//             reverse + inverse roll + shortcut: row m of window-order x goes
//             back to the grid token t(m) it was gathered from; frame-padding
//             rows are dropped)
//
// so that the activation, the residual add and the permutation back to the
// grid ride on the GEMM's output instead of making their own HBM passes.
//
// Shape: Y^T = W X^T on v_mfma_f32_16x16x32_bf16 (A = weight rows from the
// fragment-packed layout of terra_swin_pack_linear, B = token rows), so an
// accumulator lane holds four consecutive output features of one token and
// stores 8 contiguous bytes.  A workgroup (8 waves, one per CU) computes a
// 256-feature x 256-token tile; wave w owns features 64 (w & 3) .. + 64 of
// tokens 128 (w >> 2) .. + 128: 4 x 8 accumulator tiles, each weight fragment
// feeding 8 MFMAs and each token fragment 4.  Per 64-wide stage (two
// k-steps) the tile's weights (32 packed 1 KB blocks) and token rows (256
// whole 128-byte lines) stream straight into LDS by global->LDS loads, two
// 64 KB buffers, one stage ahead, as one stream across a workgroup's tiles;
// a k-step's fragments are read out of LDS while the previous k-step's MFMAs
// run.  Measured (MI355X, 156672 rows): 1024 -> 1024 at 34 % of the bf16
// MFMA peak, 4096 -> 1024 at 40 %, about hipBLASLt's rate for the plain
// product; the fused epilogues are what it adds.
//
// Tiles are walked persistently and XCD-aware: workgroup b runs on XCD b % 8
// (the hardware's round-robin), XCD x takes token blocks x, x + 8, ... and
// its workgroups sweep all feature tiles of one token block before the next,
// so a token block is read from HBM once and re-read by its feature tiles
// from that XCD's L2, while the weight stream (2 MB for a 1024 x 1024 layer)
// stays L2-resident.
#include "common.h"
#include "attn_core.h"
#include "gelu.h"

#include <type_traits>

namespace terra {
namespace {

constexpr int kLinF = 256;                         // output features per tile
constexpr int kLinT = 256;                         // token rows per tile
constexpr int kLinKS = 64;                         // input features per stage (two k-steps)
constexpr int kLinStages = 2;
constexpr int kLinThreads = 512;
constexpr int kLinWBytes = kLinF * kLinKS * 2;     // 16 feature tiles x 2 packed 1 KB blocks
constexpr int kLinXBytes = kLinT * kLinKS * 2;     // 256 rows x 128 bytes
constexpr int kLinStage = kLinWBytes + kLinXBytes;
constexpr int kLinMaxN = 4096;                     // output features (bias staged in LDS)
constexpr int kLinBiasOff = kLinStages * kLinStage;
constexpr int kLinGeluOff = kLinBiasOff + kLinMaxN * 4;
static_assert(kLinGeluOff + kGeluBytes <= 160 * 1024, "LDS");

enum { kEpiStore = 0, kEpiGelu = 1, kEpiResidual = 2, kEpiScatter = 3 };

struct LinParams {
  const uint8_t* x;       // [M rows] x K bf16, row stride x_ld bytes
  const uint8_t* w;       // packed [N, K] bf16
  const float* bias;      // [N] or NULL
  const uint8_t* res;     // residual (kEpiResidual / kEpiScatter), row stride y_ld
  uint8_t* y;             // output rows, row stride y_ld bytes
  int64_t x_ld, y_ld;
  int32_t M, N, K;
  int32_t tiles_m, tiles_n;
  // kEpiScatter: window-order rows of 8x8 windows -> grid tokens
  int32_t H, W, Hp, Wp, shift_h, shift_w, pad_top, pad_left;
  FastDiv fd_nWe, fd_nWw;  // emitted windows per image, windows per frame row
};

// This lane's index in its wave, computed where it is used (a volatile asm
// is not hoisted out of the tile loop and held in a register across it).
__device__ __forceinline__ int lin_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// 16-byte slot of (row, chunk c < 8) in a stage's token rows: 128-byte rows,
// the chunk XOR-swizzled by (row ^ (row >> 3)) & 7, so that the rows of a
// fragment read hit distinct banks whether the LDS serves 8 lanes from 128
// bytes of banks or 16 lanes from 256 bytes per cycle.
__device__ __forceinline__ int lin_swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lin_slot(int row, int c) { return row * 8 + (c ^ lin_swz(row)); }

// Grid token of window-order row m (window m / 64, token m % 64 of an 8x8
// window), or -1 for a frame-padding token: the position the partition read
// the row from (pad, then a cyclic shift by (shift_h, shift_w)).
__device__ __forceinline__ int64_t lin_grid_row(const LinParams& p, int m) {
  const uint32_t w = (uint32_t)m >> 6, s = (uint32_t)m & 63u;
  uint32_t b, wl, wr, wc;
  p.fd_nWe.divmod(w, b, wl);
  p.fd_nWw.divmod(wl, wr, wc);
  int ph = (int)(wr * 8u + (s >> 3)) + p.shift_h;
  int pw = (int)(wc * 8u + (s & 7u)) + p.shift_w;
  if (ph >= p.Hp) ph -= p.Hp;
  if (pw >= p.Wp) pw -= p.Wp;
  const int sh = ph - p.pad_top, sw = pw - p.pad_left;
  if ((unsigned)sh >= (unsigned)p.H || (unsigned)sw >= (unsigned)p.W) return -1;
  return ((int64_t)b * p.H + sh) * p.W + sw;
}

// bf16(r + o) per element of four packed bf16 pairs' worth (fp32 add, one rounding).
__device__ __forceinline__ uint2 add_bf16x4(uint2 r, uint2 o) {
  const uint32_t rw[2] = {r.x, r.y}, ow[2] = {o.x, o.y};
  uint32_t out[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float lo = __uint_as_float(rw[q] << 16) + __uint_as_float(ow[q] << 16);
    const float hi = __uint_as_float(rw[q] & 0xffff0000u) + __uint_as_float(ow[q] & 0xffff0000u);
    out[q] = pack_bf16x2(lo, hi);
  }
  return make_uint2(out[0], out[1]);
}

template <int kEpi>
__global__ __launch_bounds__(kLinThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void linear_kernel(const LinParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wave & 3, wt = wave >> 2;
  float* s_bias = reinterpret_cast<float*>(smem + kLinBiasOff);
  const uint16_t* s_gelu = reinterpret_cast<const uint16_t*>(smem + kLinGeluOff);
  // Bias (and the GELU table) in LDS: a global load at a tile's start would
  // complete only behind the loads already in flight for the next stage.
  for (int e = tid; e < p.N; e += kLinThreads) s_bias[e] = p.bias != nullptr ? p.bias[e] : 0.f;
  if constexpr (kEpi == kEpiGelu) gelu_table_fill(reinterpret_cast<uint16_t*>(smem + kLinGeluOff), tid, kLinThreads);
  __syncthreads();
  const int xcd = (int)blockIdx.x & 7;
  const int nx = ((int)gridDim.x - xcd + 7) >> 3;  // workgroups with this blockIdx % 8
  const int ksteps = p.K / 32;
  const int nst = p.K / kLinKS;                     // stages per tile
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));

  // Tile t of this workgroup: slot (blockIdx.x >> 3) + t nx of its XCD's list.
  auto tile_of = [&](int t, int& m0, int& f0) -> bool {
    const int s = ((int)blockIdx.x >> 3) + t * nx;
    const int tq = s / p.tiles_n;
    const int tb = tq * 8 + xcd;
    m0 = tb * kLinT;
    f0 = (s - tq * p.tiles_n) * kLinF;
    return tb < p.tiles_m;
  };

  // One stream of stages over all of this workgroup's tiles (stage g in LDS
  // buffer g % 2), issued one stage ahead, so the loads run on across tile
  // boundaries.  A stage is 64 input features: every token row contributes
  // one whole 128-byte line (a 64-byte half line per request halves what the
  // L2 delivers), and each feature tile its two adjacent packed blocks.
  // This thread's part: 1 KB blocks wave + 8q (q < 4) of the weights (tile
  // blk / 2, k-step 2 st + blk % 2) and of the token rows (rows 8 blk .. + 8,
  // lane l taking slot l of the block).
  const uint8_t* xbase = nullptr;  // token row m0 of the issue tile (wave-uniform)
  const uint8_t* wbase = nullptr;  // first packed block of the issue tile's features (wave-uniform)
  uint32_t xoff[4];
  int issue_tile = 0, issue_st = 0;
  auto set_sources = [&](int t) -> bool {
    int m0, f0;
    if (!tile_of(t, m0, f0)) return false;
    const int lane = lin_lane();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 8 * (wave + 8 * q) + (lane >> 3);
      const int c = (lane & 7) ^ lin_swz(row);
      const int r = m0 + row < p.M ? row : p.M - 1 - m0;  // rows past the end: a valid row, never stored
      xoff[q] = (uint32_t)r * (uint32_t)p.x_ld + (uint32_t)c * 16u;
    }
    xbase = p.x + (int64_t)m0 * p.x_ld;
    wbase = p.w + (int64_t)(f0 / 16) * ksteps * 1024;
    return true;
  };
  bool issue_valid = set_sources(0);
  auto issue_next = [&](int buf) {
    if (!issue_valid) return;  // uniform: the stream has ended
    const uint32_t base = lds0 + buf * kLinStage;
    const uint32_t woff = (uint32_t)lin_lane() * 16u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int blk = wave + 8 * q;
      dma_to_lds16_at(wbase + ((int64_t)(blk >> 1) * ksteps + 2 * issue_st + (blk & 1)) * 1024, woff, base + blk * 1024);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) dma_to_lds16_at(xbase + issue_st * 128, xoff[q], base + kLinWBytes + (wave + 8 * q) * 1024);
    if (++issue_st == nst) {
      issue_st = 0;
      issue_valid = set_sources(++issue_tile);
    }
  };

  // Fragments of k-step kk of the stage in buffer buf.
  auto read_frags = [&](int buf, int kk, uint4 (&wfr)[4], uint4 (&xfr)[8]) {
    const int lane = lin_lane();
    const int g = lane >> 4, c16 = lane & 15;
    const uint8_t* stg = smem + buf * kLinStage;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      wfr[i] = *reinterpret_cast<const uint4*>(stg + (2 * (4 * wf + i) + kk) * 1024 + lane * 16);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      xfr[jj] = *reinterpret_cast<const uint4*>(stg + kLinWBytes + lin_slot(128 * wt + 16 * jj + c16, 4 * kk + g) * 16);
  };
  auto mfmas = [&](f32x4 (&acc)[4][8], const uint4 (&wfr)[4], const uint4 (&xfr)[8]) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wfr[i]),
                                                             __builtin_bit_cast(bf16x8, xfr[jj]), acc[i][jj], 0, 0, 0);
  };

  // Stage g + 1 is issued right after the barrier that ends the reads of
  // stage g - 1 (its buffer), so the only loads outstanding at the wait for a
  // stage are its own (and an epilogue's, which the wait then also covers).
  issue_next(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  issue_next(1);
  uint4 wa[4], xa[8], wb[4], xb[8];  // fragments of k-steps 2 st (a) and 2 st + 1 (b)
  read_frags(0, 0, wa, xa);
  int sg = 0;  // stream index of the stage being computed
  for (int t = 0;; ++t) {
    int m0, f0;
    if (!tile_of(t, m0, f0)) break;  // uniform
    int m1, f1;
    const bool next_tile = tile_of(t + 1, m1, f1);
    f32x4 acc[4][8];
    {
      const int g = lin_lane() >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(s_bias + f0 + 64 * wf + 16 * i + 4 * g);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc[i][jj] = b;
      }
    }
    for (int st = 0; st < nst; ++st, ++sg) {
      read_frags(sg & 1, 1, wb, xb);
      mfmas(acc, wa, xa);
      if (st + 1 < nst || next_tile) {  // uniform: stage sg + 1 exists
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();  // stage sg + 1 is in LDS; every wave has read stage sg out
        issue_next(sg & 1);
        read_frags((sg + 1) & 1, 0, wa, xa);
      }
      mfmas(acc, wb, xb);
    }
    const int lane = lin_lane();
    const int g = lane >> 4, c16 = lane & 15;

    // Epilogue: lane (c16, g) of tile (i, jj) holds features f0 + 64 wf +
    // 16 i + 4 g .. + 3 of token row m0 + 128 wt + 16 jj + c16.
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      uint2 o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = make_uint2(pack_bf16x2(acc[i][jj][0], acc[i][jj][1]),
                                                    pack_bf16x2(acc[i][jj][2], acc[i][jj][3]));
      if constexpr (kEpi == kEpiGelu) {
        // Table lookups; a wave holding a value outside the table (|x| < 2^-22
        // or >= 32) redoes the row exactly.
        u16x2 dmax = {0, 0};
        uint2 gv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          asm volatile("" : "+v"(o[i].x), "+v"(o[i].y));
          gv[i].x = gelu_pair_table(o[i].x, s_gelu, dmax);
          gv[i].y = gelu_pair_table(o[i].y, s_gelu, dmax);
        }
        const uint32_t dm = dmax.x > dmax.y ? dmax.x : dmax.y;
        if (__builtin_amdgcn_ballot_w64(dm >= (uint32_t)kGeluSpan) != 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            gv[i].x = gelu_bf16(o[i].x & 0xffffu, s_gelu) | (gelu_bf16(o[i].x >> 16, s_gelu) << 16);
            gv[i].y = gelu_bf16(o[i].y & 0xffffu, s_gelu) | (gelu_bf16(o[i].y >> 16, s_gelu) << 16);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = gv[i];
      }
      const int m = m0 + 128 * wt + 16 * jj + c16;
      if (m >= p.M) continue;
      int64_t orow = m;
      if constexpr (kEpi == kEpiScatter) {
        orow = lin_grid_row(p, m);
        if (orow < 0) continue;  // frame padding
      }
      uint8_t* yr = p.y + orow * p.y_ld + (f0 + 64 * wf + 4 * g) * 2;
      if constexpr (kEpi == kEpiResidual || kEpi == kEpiScatter) {
        const uint8_t* rr = p.res + orow * p.y_ld + (f0 + 64 * wf + 4 * g) * 2;
        uint2 r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const uint2*>(rr + 32 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = add_bf16x4(r[i], o[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint2*>(yr + 32 * i) = o[i];
    }
  }
}

template <int kEpi>
int launch_linear(const LinParams& p, hipStream_t s) {
  constexpr int lds = kEpi == kEpiGelu ? kLinGeluOff + kGeluBytes : kLinGeluOff;
  auto kern = linear_kernel<kEpi>;
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
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kLinThreads, lds) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the linear kernel grid for this device");
    const int resident = cus * (per_cu > 0 ? per_cu : 1);
    cache[dev] = resident >= 16 ? resident - resident % 8 : 8;  // whole XCD rounds
  }
  kern<<<cache[dev], kLinThreads, lds, s>>>(p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "linear kernel launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}

bool lin_overlap(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)bbytes && y < x + (uintptr_t)abytes;
}

// Shared checks of both entry points; fills the GEMM fields of `p`.
int lin_validate(const void* x, const void* w, const float* bias, const void* y, int dtype, int64_t rows,
                 int in_features, int out_features, int64_t x_stride, int64_t y_stride, LinParams* p) {
  if (x == nullptr || w == nullptr || y == nullptr) return fail(TERRA_ERR_NULL, "x, weight and y must be non-NULL");
  if (dtype_size(dtype) == 0) return fail(TERRA_ERR_DTYPE, "unknown dtype %d", dtype);
  if (dtype != TERRA_DTYPE_BF16) return fail(TERRA_ERR_UNSUPPORTED, "the linear kernels are bf16 only");
  if (rows < 0 || rows >= (1ll << 31)) return fail(TERRA_ERR_SHAPE, "rows must be in [0, 2^31) (got %lld)",
                                                   (long long)rows);
  if (in_features <= 0 || in_features % kLinKS != 0 || out_features <= 0 || out_features % kLinF != 0 ||
      out_features > kLinMaxN)
    return fail(TERRA_ERR_SHAPE,
                "in_features must be a positive multiple of 64 and out_features a multiple of 256 up to %d (got %d, %d)",
                kLinMaxN, in_features, out_features);
  if (x_stride < in_features || y_stride < out_features || x_stride % 8 != 0 || y_stride % 4 != 0 ||
      x_stride * 2 * kLinT >= (1ll << 32))
    return fail(TERRA_ERR_SHAPE,
                "row strides must cover the rows (x_stride >= %d, a multiple of 8; y_stride >= %d, a multiple of 4)",
                in_features, out_features);
  if (((uintptr_t)x & 15u) != 0 || ((uintptr_t)w & 15u) != 0 || ((uintptr_t)bias & 15u) != 0 ||
      ((uintptr_t)y & 7u) != 0)
    return fail(TERRA_ERR_ALIGN, "x, weight and bias must be 16-byte aligned and y 8-byte aligned");
  if ((int64_t)out_features * in_features * 2 >= (1ll << 31))
    return fail(TERRA_ERR_SHAPE, "weight of %d x %d exceeds 2 GB", out_features, in_features);
  p->x = static_cast<const uint8_t*>(x);
  p->w = static_cast<const uint8_t*>(w);
  p->bias = bias;
  p->y = static_cast<uint8_t*>(const_cast<void*>(y));
  p->res = nullptr;
  p->x_ld = x_stride * 2;
  p->y_ld = y_stride * 2;
  p->M = (int32_t)rows;
  p->N = out_features;
  p->K = in_features;
  p->tiles_m = (int32_t)((rows + kLinT - 1) / kLinT);
  p->tiles_n = out_features / kLinF;
  return TERRA_OK;
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_linear(const void* x, void* y, int dtype, int64_t rows, int in_features,
                                 int out_features, int64_t x_stride, int64_t y_stride, const void* weight_packed,
                                 const float* bias, int epilogue, void* stream) {
  clear_error();
  LinParams p{};
  const int st =
      lin_validate(x, weight_packed, bias, y, dtype, rows, in_features, out_features, x_stride, y_stride, &p);
  if (st != TERRA_OK) return st;
  if (epilogue != TERRA_LINEAR_STORE && epilogue != TERRA_LINEAR_GELU)
    return fail(TERRA_ERR_SHAPE, "unknown epilogue %d", epilogue);
  const int64_t xb = (rows - 1) * p.x_ld + (int64_t)in_features * 2, yb = (rows - 1) * p.y_ld + (int64_t)out_features * 2;
  if (rows > 0 && lin_overlap(x, xb, y, yb)) return fail(TERRA_ERR_SHAPE, "y overlaps x");
  if (rows == 0) return TERRA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return epilogue == TERRA_LINEAR_GELU ? launch_linear<kEpiGelu>(p, s) : launch_linear<kEpiStore>(p, s);
}

extern "C" int terra_swin_linear_residual(const void* x, const void* residual, void* y, int dtype, int64_t rows,
                                          int in_features, int out_features, const void* weight_packed,
                                          const float* bias, const terra_swin_geom* geom, void* stream) {
  clear_error();
  LinParams p{};
  const int st = lin_validate(x, weight_packed, bias, y, dtype, rows, in_features, out_features, in_features,
                              out_features, &p);
  if (st != TERRA_OK) return st;
  if (residual == nullptr) return fail(TERRA_ERR_NULL, "residual must be non-NULL");
  if (((uintptr_t)residual & 7u) != 0) return fail(TERRA_ERR_ALIGN, "residual must be 8-byte aligned");
  p.res = static_cast<const uint8_t*>(residual);
  int64_t out_rows = rows;  // rows of residual / y
  if (geom != nullptr) {
    GeomDims dims;
    const int gs = validate_geom(geom, &dims);
    if (gs != TERRA_OK) return gs;
    const terra_swin_geom& q = *geom;
    if (q.window != 8) return fail(TERRA_ERR_UNSUPPORTED, "the scatter epilogue needs 8x8 windows (got %d)", q.window);
    if (q.channels != out_features)
      return fail(TERRA_ERR_SHAPE, "geom channels (%d) must equal out_features (%d)", q.channels, out_features);
    // Every grid token must come from exactly one emitted window, so that the
    // scatter writes all of y: the whole frame emitted, no valid-window range.
    if (q.win_row_begin != 0 || dims.rows != dims.nWh || q.valid_end > 0)
      return fail(TERRA_ERR_UNSUPPORTED,
                  "the scatter epilogue needs every window of the frame emitted (no window-row or valid-window range)");
    if (rows != (int64_t)q.batch * dims.nWe * 64)
      return fail(TERRA_ERR_SHAPE, "rows (%lld) must be the window tokens of the frame (%lld)", (long long)rows,
                  (long long)((int64_t)q.batch * dims.nWe * 64));
    out_rows = (int64_t)q.batch * q.height * q.width;
    p.H = q.height; p.W = q.width; p.Hp = (int32_t)dims.Hp; p.Wp = (int32_t)dims.Wp;
    p.shift_h = q.shift_h; p.shift_w = q.shift_w; p.pad_top = q.pad_top; p.pad_left = q.pad_left;
    p.fd_nWe = FastDiv((uint32_t)dims.nWe);
    p.fd_nWw = FastDiv((uint32_t)dims.nWw);
  }
  const int64_t xb = rows * (int64_t)in_features * 2, yb = out_rows * (int64_t)out_features * 2;
  if (rows > 0 && lin_overlap(x, xb, y, yb)) return fail(TERRA_ERR_SHAPE, "y overlaps x");
  if (y != residual && lin_overlap(residual, yb, y, yb))
    return fail(TERRA_ERR_SHAPE, "y overlaps residual without being residual");
  if (rows == 0) return TERRA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return geom != nullptr ? launch_linear<kEpiScatter>(p, s) : launch_linear<kEpiResidual>(p, s);
}
