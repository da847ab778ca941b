// Fused pad + cyclic shift + window partition, and its inverse
// (window reverse + inverse shift + crop + optional residual add).
//
// Both kernels are pure permutations at token granularity: a token is a
// contiguous C-vector in the [B, H, W, C] grid and in the [B_, N, C] window
// tensor alike, so every 16-byte chunk a lane moves is read from and written
// to contiguous memory, and consecutive lanes touch consecutive chunks of the
// same token row.  Each kernel iterates over its *destination* (gather form),
// so writes are perfectly sequential and each destination byte is written
// exactly once; reads are contiguous runs of C*elt bytes.  Nothing is staged
// through LDS: with >= 192-byte contiguous runs on both sides there is no
// uncoalesced access for LDS to fix.
#include "common.h"

namespace terra {

int validate_geom(const terra_swin_geom* geom, GeomDims* dims) {
  if (geom == nullptr) return fail(TERRA_ERR_NULL, "geom is NULL");
  const terra_swin_geom& q = *geom;
  if (q.batch <= 0 || q.height <= 0 || q.width <= 0 || q.channels <= 0 || q.window <= 0)
    return fail(TERRA_ERR_SHAPE, "batch/height/width/channels/window must be positive (got %d/%d/%d/%d/%d)",
                q.batch, q.height, q.width, q.channels, q.window);
  if (q.pad_top < 0 || q.pad_bottom < 0 || q.pad_left < 0 || q.pad_right < 0)
    return fail(TERRA_ERR_SHAPE, "padding must be non-negative");
  const int64_t Hp = (int64_t)q.height + q.pad_top + q.pad_bottom;
  const int64_t Wp = (int64_t)q.width + q.pad_left + q.pad_right;
  if (Hp % q.window != 0 || Wp % q.window != 0)
    return fail(TERRA_ERR_SHAPE, "padded grid %lldx%lld is not a multiple of window %d",
                (long long)Hp, (long long)Wp, q.window);
  if (q.shift_h < 0 || q.shift_h >= Hp || q.shift_w < 0 || q.shift_w >= Wp)
    return fail(TERRA_ERR_SHAPE, "shift (%d, %d) outside [0, padded extent)", q.shift_h, q.shift_w);
  const int64_t nWh = Hp / q.window, nWw = Wp / q.window;
  const int64_t rows = q.win_rows <= 0 ? nWh - q.win_row_begin : q.win_rows;
  if (q.win_row_begin < 0 || rows <= 0 || q.win_row_begin + rows > nWh)
    return fail(TERRA_ERR_SHAPE, "window rows [%d, %lld) outside the %lld-row window grid",
                q.win_row_begin, (long long)(q.win_row_begin + rows), (long long)nWh);
  const int64_t nWe = rows * nWw;
  if (q.valid_end > 0 && (q.valid_begin < 0 || q.valid_begin >= q.valid_end || q.valid_end > nWe))
    return fail(TERRA_ERR_SHAPE, "valid window range [%d, %d) outside [0, %lld)", q.valid_begin,
                q.valid_end, (long long)nWe);
  dims->Hp = Hp; dims->Wp = Wp; dims->nWh = nWh; dims->nWw = nWw; dims->rows = rows; dims->nWe = nWe;
  return TERRA_OK;
}

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int VB> struct Chunk;
template <> struct Chunk<16> { using T = u32x4; };
template <> struct Chunk<8> { using T = u32x2; };
template <> struct Chunk<4> { using T = uint32_t; };
template <> struct Chunk<2> { using T = uint16_t; };
template <> struct Chunk<1> { using T = uint8_t; };

template <int VB>
__device__ __forceinline__ typename Chunk<VB>::T fill_chunk(uint32_t pat) {
  using T = typename Chunk<VB>::T;
  if constexpr (VB >= 8) return T(pat);  // splat
  else return (T)pat;
}

// Every byte is touched once per launch: loads carry the nontemporal hint and
// stores go out as sc1 buffer stores (stream_store_sc1).
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) { return __builtin_nontemporal_load(p); }

struct CopyGeom {
  int32_t H, W, ws, Hp, Wp;
  int32_t shift_h, shift_w, pad_top, pad_left;
  int32_t win_row_begin, win_rows, nWw;
  int32_t valid_begin, valid_end;  // valid_end <= 0: all valid
  int32_t N;
  int64_t row_bytes;               // C * elt
  int64_t win_row_bytes;           // C * elt of the windows (the LayerNorm kernels' mixed-dtype forms)
  FastDiv fd_cv, fd_N, fd_nWe, fd_nWw, fd_ws, fd_W, fd_H;
  uint32_t total;                  // chunks in the destination
  uint32_t pad_pattern;
};

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

template <int VB>
__global__ __launch_bounds__(kThreads) void partition_kernel(const uint8_t* __restrict__ x,
                                                             uint8_t* __restrict__ win,
                                                             const CopyGeom g) {
  using T = typename Chunk<VB>::T;
  const uint32_t first = blockIdx.x * (kThreads * kUnroll);
  const uint32_t base = first + threadIdx.x;
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(win + (int64_t)first * VB, min(g.total - first, (uint32_t)(kThreads * kUnroll)) * VB);
  // Loads are unconditional (lanes without a source read chunk 0 and take the
  // pad value afterwards): a load under a branch gets its own wait at the
  // branch join, which would leave one load in flight per lane.
  int64_t src[kUnroll];
  bool have[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t c = base + u * kThreads;
    uint32_t rest, cv, rest2, t, b, wl, wr, wc, ti, tj;
    g.fd_cv.divmod(c, rest, cv);
    g.fd_N.divmod(rest, rest2, t);
    g.fd_nWe.divmod(rest2, b, wl);
    g.fd_nWw.divmod(wl, wr, wc);
    g.fd_ws.divmod(t, ti, tj);
    const bool valid = g.valid_end <= 0 || ((int)wl >= g.valid_begin && (int)wl < g.valid_end);
    int ph = (int)((wr + g.win_row_begin) * g.ws + ti) + g.shift_h;
    int pw = (int)(wc * g.ws + tj) + g.shift_w;
    if (ph >= g.Hp) ph -= g.Hp;
    if (pw >= g.Wp) pw -= g.Wp;
    const int sh = ph - g.pad_top;
    const int sw = pw - g.pad_left;
    have[u] = c < g.total && valid && (unsigned)sh < (unsigned)g.H && (unsigned)sw < (unsigned)g.W;
    src[u] = have[u] ? (((int64_t)b * g.H + sh) * g.W + sw) * g.row_bytes + (int64_t)cv * VB : 0;
  }
  T vals[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) vals[u] = stream_load(reinterpret_cast<const T*>(x + src[u]));
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (!have[u]) vals[u] = fill_chunk<VB>(g.pad_pattern);
    if (base + u * kThreads < g.total) stream_store_sc1(vals[u], out, (threadIdx.x + u * kThreads) * VB);
  }
}

// ---- fused LayerNorm + pad + roll + partition ------------------------------
// Eight lanes own one destination token; lane `sub` of the group holds the
// 16-byte chunks sub, sub + 8, ... of the token's C-vector, so each load /
// store instruction of the group covers 128 contiguous bytes.  Mean and
// variance are two-pass fp32 statistics over the values held in registers
// (reduced over the 8 lanes with xor shuffles); y = (x - mean) * rstd *
// gamma + beta in fp32, rounded once to the activation type.  Tokens that
// partition would pad (frame padding, pad windows) are written as pad_value.
// Rows of more than 48 chunks (C > 384 in bf16) take 16 lanes per token, so
// that a lane holds at most 6 chunks: at 12 chunks per lane (C = 768) the
// register footprint left too few waves to cover the load latency (43 % of
// the HBM peak on c4).
constexpr int kLnLanes = 8;

// Sum over the kL lanes of a token (DPP; the 16-lane step adds the row
// mirror of the 8-lane sums).
template <int kL>
__device__ __forceinline__ float group_sum(float v) {
  v = group8_sum(v);
  if constexpr (kL == 16) v += dpp_move<0x140>(v);
  return v;
}

template <int DT> struct LnElt;
template <> struct LnElt<TERRA_DTYPE_F32> { static constexpr int kPerChunk = 4; };
template <> struct LnElt<TERRA_DTYPE_BF16> { static constexpr int kPerChunk = 8; };
template <> struct LnElt<TERRA_DTYPE_F16> { static constexpr int kPerChunk = 8; };

template <int DT>
__device__ __forceinline__ void unpack_chunk(const u32x4& c, float* f) {
  if constexpr (DT == TERRA_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(c[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = (uint16_t)(c[i] & 0xffffu), hi = (uint16_t)(c[i] >> 16);
      if constexpr (DT == TERRA_DTYPE_BF16) {
        f[2 * i] = bf16_bits_to_f32(lo);
        f[2 * i + 1] = bf16_bits_to_f32(hi);
      } else {
        f[2 * i] = __half2float(__ushort_as_half(lo));
        f[2 * i + 1] = __half2float(__ushort_as_half(hi));
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ u32x4 pack_chunk(const float* f) {
  u32x4 c;
  if constexpr (DT == TERRA_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __float_as_uint(f[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo, hi;
      if constexpr (DT == TERRA_DTYPE_BF16) {
        lo = f32_to_bf16_bits(f[2 * i]);
        hi = f32_to_bf16_bits(f[2 * i + 1]);
      } else {
        lo = __half_as_ushort(__float2half_rn(f[2 * i]));
        hi = __half_as_ushort(__float2half_rn(f[2 * i + 1]));
      }
      c[i] = lo | (hi << 16);
    }
  }
  return c;
}

struct LnParams {
  const float* gamma;  // C floats or NULL (1)
  const float* beta;   // C floats or NULL (0)
  float eps;
  float inv_c;         // 1 / C
  int32_t chunks;      // 16-byte chunks per token row
  uint32_t tokens;     // destination tokens
};

// Widest fused LayerNorm row: C <= 1024 channels (gamma / beta staged whole)
// and at most 256 chunks of 16 bytes (fp32 C = 1024: 4096 bytes).
constexpr int kLnMaxChannels = 1024;
constexpr int kLnMaxChunks = 256;

// DTO: the windows' dtype, DT's or (DT = f32) bf16: each fp32 chunk of four
// values then leaves as eight bytes, the LayerNorm output rounded once to
// bf16 (what bf16 autocast casts the fp32 output to before the next Linear).
template <int DT, int CPL, int kL, int DTO = DT>
__global__ __launch_bounds__(kThreads) void partition_ln_kernel(const uint8_t* __restrict__ x,
                                                                uint8_t* __restrict__ win,
                                                                const CopyGeom g, const LnParams ln) {
  static_assert(DTO == DT || (DT == TERRA_DTYPE_F32 && DTO == TERRA_DTYPE_BF16), "output dtype");
  constexpr bool kCast = DTO != DT;
  constexpr int kTokensPerBlock = kThreads / kL;
  constexpr int E = LnElt<DT>::kPerChunk;
  // gamma / beta of all C channels, staged once per workgroup.  Their loads
  // are issued first and the row loads right after (vector memory completes
  // in order, so the staging waits for gamma / beta only); the barrier is
  // LDS-only, and the rows stay in flight across it.
  // Sized for the widest row this instance serves (CPL chunks on each of kL
  // lanes), so narrow rows stage and hold no more than they use.
  constexpr int kMaxC = CPL * kL * E;
  __shared__ __attribute__((aligned(16))) float s_gamma[kMaxC];
  __shared__ __attribute__((aligned(16))) float s_beta[kMaxC];
  constexpr int kGB = (kMaxC + kThreads - 1) / kThreads;
  const int C = ln.chunks * E;
  float gv[kGB], bv[kGB];
#pragma unroll
  for (int i = 0; i < kGB; ++i) {
    const int c = threadIdx.x + i * kThreads;
    gv[i] = (ln.gamma != nullptr && c < C) ? ln.gamma[c] : 1.f;
    bv[i] = (ln.beta != nullptr && c < C) ? ln.beta[c] : 0.f;
  }
  asm volatile("" ::: "memory");  // the gamma / beta loads before the row loads

  const uint32_t tok_raw = blockIdx.x * kTokensPerBlock + threadIdx.x / kL;
  const bool live = tok_raw < ln.tokens;  // whole lane groups share it
  const uint32_t tok = live ? tok_raw : 0u;
  const int sub = threadIdx.x & (kL - 1);
  uint32_t w, t, b, wl, wr, wc, ti, tj;
  g.fd_N.divmod(tok, w, t);
  g.fd_nWe.divmod(w, b, wl);
  g.fd_nWw.divmod(wl, wr, wc);
  g.fd_ws.divmod(t, ti, tj);
  const bool valid = g.valid_end <= 0 || ((int)wl >= g.valid_begin && (int)wl < g.valid_end);
  int ph = (int)((wr + g.win_row_begin) * g.ws + ti) + g.shift_h;
  int pw = (int)(wc * g.ws + tj) + g.shift_w;
  if (ph >= g.Hp) ph -= g.Hp;
  if (pw >= g.Wp) pw -= g.Wp;
  const int sh = ph - g.pad_top;
  const int sw = pw - g.pad_left;
  const bool in = valid && (unsigned)sh < (unsigned)g.H && (unsigned)sw < (unsigned)g.W;

  const u32x4* src = reinterpret_cast<const u32x4*>(x + (((int64_t)b * g.H + sh) * g.W + sw) * g.row_bytes);
  float v[CPL][E];
  // Unconditional loads (absent chunks read chunk 0 of x, then count as
  // zeros): a load under a branch gets its own wait at the branch join.
  u32x4 raw[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = sub + kL * k;
    raw[k] = __builtin_nontemporal_load((in && c < ln.chunks) ? src + c : reinterpret_cast<const u32x4*>(x));
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < kGB; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < C) {
      s_gamma[c] = gv[i];
      s_beta[c] = bv[i];
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (!live) return;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = sub + kL * k;
    unpack_chunk<DT>((in && c < ln.chunks) ? raw[k] : u32x4(0u), v[k]);
  }
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < E; ++e) sum += v[k][e];  // absent chunks hold zeros
  const float mean = group_sum<kL>(sum) * ln.inv_c;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const bool present = sub + kL * k < ln.chunks;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float d = v[k][e] - mean;
      sq += present ? d * d : 0.f;
    }
  }
  const float rstd = rsqrtf(group_sum<kL>(sq) * ln.inv_c + ln.eps);

  const uint32_t first = blockIdx.x * kTokensPerBlock;
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(win + (int64_t)first * g.win_row_bytes,
                  (uint32_t)(min(ln.tokens - first, (uint32_t)kTokensPerBlock) * g.win_row_bytes));
  const uint32_t row_off = (tok - first) * (uint32_t)g.win_row_bytes;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = sub + kL * k;
    if (c < ln.chunks) {
      float y[E];
      if (in) {
#pragma unroll
        for (int q = 0; q < E; q += 4) {
          const float4 gm = *reinterpret_cast<const float4*>(s_gamma + c * E + q);
          const float4 bt = *reinterpret_cast<const float4*>(s_beta + c * E + q);
          y[q + 0] = (v[k][q + 0] - mean) * rstd * gm.x + bt.x;
          y[q + 1] = (v[k][q + 1] - mean) * rstd * gm.y + bt.y;
          y[q + 2] = (v[k][q + 2] - mean) * rstd * gm.z + bt.z;
          y[q + 3] = (v[k][q + 3] - mean) * rstd * gm.w + bt.w;
        }
      }
      if constexpr (kCast) {  // four fp32 values -> four bf16, eight bytes
        u32x2 val = u32x2(g.pad_pattern);
        if (in) {
          val[0] = f32_to_bf16_bits(y[0]) | ((uint32_t)f32_to_bf16_bits(y[1]) << 16);
          val[1] = f32_to_bf16_bits(y[2]) | ((uint32_t)f32_to_bf16_bits(y[3]) << 16);
        }
        stream_store_sc1(val, out, row_off + c * 8);
      } else {
        const u32x4 val = in ? pack_chunk<DT>(y) : u32x4(g.pad_pattern);
        stream_store_sc1(val, out, row_off + c * 16);
      }
    }
  }
}

// ---- backward of the fused LayerNorm + pad + roll + partition ---------------
// Gather form over the grid tokens, like reverse_kernel: token (b, h, w) reads
// the gradient g of the window slot partition wrote it to (zero when the
// frame does not emit it or emits a pad window there), recomputes the
// forward's statistics from its row of x (two-pass fp32, as
// partition_ln_kernel), and writes
//   dx = rstd (gamma g - mean_c(gamma g) - xhat mean_c(gamma g xhat)) (+ dres)
// rounded once to the activation dtype, xhat = (x - mean) rstd.  The kL lanes
// of a token hold its chunks as in the forward.  Workgroups loop over the
// tokens (grid-stride) and keep per-lane sums of g xhat and g for the
// channels they hold; at the end each workgroup reduces them in LDS and adds
// them to dgamma / dbeta with one float atomic per channel.
struct LnBwdParams {
  const float* gamma;  // C floats or NULL (1)
  float* dgamma;       // C floats, accumulated, or NULL
  float* dbeta;        // C floats, accumulated, or NULL
  float eps;
  float inv_c;
  int32_t chunks;      // 16-byte chunks per token row
  uint32_t tokens;     // grid tokens B * H * W
};

// DTG: the windows' gradient dtype, DT's or (DT = f32) bf16 (the gradient
// of the bf16 windows partition_ln_kernel<f32, .., bf16> writes): each chunk
// of four values is read as eight bytes.
template <int DT, int CPL, int kL, bool kRes, int DTG = DT>
__global__ __launch_bounds__(kThreads) void partition_ln_bwd_kernel(const uint8_t* __restrict__ dwin,
                                                                    const uint8_t* __restrict__ x, uint8_t* dx,
                                                                    const uint8_t* dres, const CopyGeom g,
                                                                    const LnBwdParams ln) {
  static_assert(DTG == DT || (DT == TERRA_DTYPE_F32 && DTG == TERRA_DTYPE_BF16), "gradient dtype");
  constexpr bool kCast = DTG != DT;
  constexpr int kTokensPerPass = kThreads / kL;
  constexpr int E = LnElt<DT>::kPerChunk;
  constexpr int kMaxC = CPL * kL * E;
  __shared__ __attribute__((aligned(16))) float s_gamma[kMaxC];
  __shared__ float s_dg[kMaxC];
  __shared__ float s_db[kMaxC];
  const int C = ln.chunks * E;
  for (int c = threadIdx.x; c < kMaxC; c += kThreads) {
    s_gamma[c] = (ln.gamma != nullptr && c < C) ? ln.gamma[c] : 1.f;
    s_dg[c] = 0.f;
    s_db[c] = 0.f;
  }
  __syncthreads();
  const int sub = threadIdx.x & (kL - 1);
  float acc_g[CPL][E], acc_b[CPL][E];  // this lane's sums of g xhat and g over its tokens
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < E; ++e) acc_g[k][e] = acc_b[k][e] = 0.f;

  // Passes of kTokensPerPass tokens: `first` is uniform over the workgroup,
  // so dx's buffer descriptor is one scalar value per pass (a descriptor
  // built from each lane group's own token is not, and every store then
  // became a loop over the wave's distinct descriptors).
  for (uint32_t first = blockIdx.x * kTokensPerPass; first < ln.tokens; first += gridDim.x * kTokensPerPass) {
    const uint32_t tok = first + threadIdx.x / kL;
    if (tok >= ln.tokens) continue;  // uniform per lane group
    uint32_t rest, sw, b, sh;
    g.fd_W.divmod(tok, rest, sw);
    g.fd_H.divmod(rest, b, sh);
    int fi = (int)sh + g.pad_top - g.shift_h;
    int fj = (int)sw + g.pad_left - g.shift_w;
    if (fi < 0) fi += g.Hp;
    if (fj < 0) fj += g.Wp;
    uint32_t wr, ti, wc, tj;
    g.fd_ws.divmod((uint32_t)fi, wr, ti);
    g.fd_ws.divmod((uint32_t)fj, wc, tj);
    const int wr_l = (int)wr - g.win_row_begin;
    const int wl = wr_l * g.nWw + (int)wc;
    const bool have = (unsigned)wr_l < (unsigned)g.win_rows &&
                      (g.valid_end <= 0 || (wl >= g.valid_begin && wl < g.valid_end));
    const int64_t slot = have ? ((int64_t)b * g.win_rows * g.nWw + wl) * g.N + (int64_t)(ti * g.ws + tj) : 0;
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + (int64_t)tok * g.row_bytes);
    const u32x4* gs = reinterpret_cast<const u32x4*>(dwin + slot * g.win_row_bytes);
    const u32x2* gs2 = reinterpret_cast<const u32x2*>(dwin + slot * g.win_row_bytes);
    const u32x4* rs = reinterpret_cast<const u32x4*>(dres + (kRes ? (int64_t)tok * g.row_bytes : 0));
    // Unconditional loads: chunks past the row read chunk 0 and count as zeros.
    u32x4 xr[CPL], gr[kCast ? 1 : CPL], rr[kRes ? CPL : 1];
    u32x2 gr2[kCast ? CPL : 1];
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k < ln.chunks ? sub + kL * k : 0;
      xr[k] = __builtin_nontemporal_load(xs + c);
      if constexpr (kCast)
        gr2[k] = __builtin_nontemporal_load(gs2 + c);
      else
        gr[k] = __builtin_nontemporal_load(gs + c);
      if constexpr (kRes) rr[k] = __builtin_nontemporal_load(rs + c);
    }
    float v[CPL][E], gv[CPL][E];
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const bool pc = sub + kL * k < ln.chunks;
      unpack_chunk<DT>(pc ? xr[k] : u32x4(0u), v[k]);
      if constexpr (kCast) {
        const u32x2 w = (pc && have) ? gr2[k] : u32x2(0u);
        gv[k][0] = __uint_as_float(w[0] << 16);
        gv[k][1] = __uint_as_float(w[0] & 0xffff0000u);
        gv[k][2] = __uint_as_float(w[1] << 16);
        gv[k][3] = __uint_as_float(w[1] & 0xffff0000u);
      } else {
        unpack_chunk<DT>((pc && have) ? gr[k] : u32x4(0u), gv[k]);
      }
    }
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k)
#pragma unroll
      for (int e = 0; e < E; ++e) sum += v[k][e];  // absent chunks hold zeros
    const float mean = group_sum<kL>(sum) * ln.inv_c;
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const bool pc = sub + kL * k < ln.chunks;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float d = v[k][e] - mean;
        sq += pc ? d * d : 0.f;
      }
    }
    const float rstd = rsqrtf(group_sum<kL>(sq) * ln.inv_c + ln.eps);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float xh = (v[k][e] - mean) * rstd;
        const float gm = c < ln.chunks ? s_gamma[c * E + e] : 0.f;
        acc_g[k][e] += gv[k][e] * xh;
        acc_b[k][e] += gv[k][e];
        const float dxh = gv[k][e] * gm;
        v[k][e] = xh;    // from here on: xhat
        gv[k][e] = dxh;  // from here on: gamma g
        s1 += dxh;
        s2 += dxh * xh;
      }
    }
    s1 = group_sum<kL>(s1) * ln.inv_c;
    s2 = group_sum<kL>(s2) * ln.inv_c;
    const __amdgpu_buffer_rsrc_t out =
        buffer_rsrc(dx + (int64_t)first * g.row_bytes,
                    (uint32_t)(min(ln.tokens - first, (uint32_t)kTokensPerPass) * g.row_bytes));
    const uint32_t row_off = (tok - first) * (uint32_t)g.row_bytes;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k;
      if (c >= ln.chunks) continue;
      float y[E];
#pragma unroll
      for (int e = 0; e < E; ++e) y[e] = rstd * (gv[k][e] - s1 - v[k][e] * s2);
      if constexpr (kRes) {
        float r[E];
        unpack_chunk<DT>(rr[k], r);
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] += r[e];
      }
      stream_store_sc1(pack_chunk<DT>(y), out, row_off + (uint32_t)c * 16);
    }
  }
  if (ln.dgamma == nullptr && ln.dbeta == nullptr) return;  // uniform
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = sub + kL * k;
    if (c >= ln.chunks) continue;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      atomicAdd(&s_dg[c * E + e], acc_g[k][e]);
      atomicAdd(&s_db[c * E + e], acc_b[k][e]);
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += kThreads) {
    if (ln.dgamma != nullptr) unsafeAtomicAdd(ln.dgamma + c, s_dg[c]);
    if (ln.dbeta != nullptr) unsafeAtomicAdd(ln.dbeta + c, s_db[c]);
  }
}

// ---- fp32 rows -> bf16 windows: pad + roll + partition + cast --------------
// The backward of reverse under bf16 autocast: the fp32 gradient of the grid
// gathered into windows and rounded once to bf16 (bit-identical to
// partition_kernel in fp32 followed by a cast), with (kSum) the column sums of
// the bf16 values written, i.e. the bias gradient of the Linear whose output
// the windows are.  kL lanes own one destination token, lane `sub` holding
// chunks sub, sub + kL, ... of its fp32 row, as in partition_ln_kernel.
// Workgroups loop over the tokens in passes (grid-stride, the resident
// count), so each lane keeps its channels' sums in registers; at the end each
// workgroup reduces them in LDS and adds them to the output with one float
// atomic per channel.
struct CastParams {
  float* colsum;    // C floats, accumulated (kSum)
  int32_t chunks;   // 16-byte fp32 chunks per token row
  uint32_t tokens;  // destination (window) tokens
};

template <int CPL, int kL, bool kSum>
__global__ __launch_bounds__(kThreads) void partition_cast_kernel(const uint8_t* __restrict__ x,
                                                                  uint8_t* __restrict__ win, const CopyGeom g,
                                                                  const CastParams cp) {
  constexpr int kTokensPerPass = kThreads / kL;
  constexpr int kMaxC = CPL * kL * 4;
  __shared__ float s_sum[kSum ? kMaxC : 1];
  if constexpr (kSum) {
    for (int c = threadIdx.x; c < kMaxC; c += kThreads) s_sum[c] = 0.f;
    __syncthreads();
  }
  const int sub = threadIdx.x & (kL - 1);
  float acc[CPL][4];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[k][e] = 0.f;

  for (uint32_t first = blockIdx.x * kTokensPerPass; first < cp.tokens; first += gridDim.x * kTokensPerPass) {
    const uint32_t tok = first + threadIdx.x / kL;
    if (tok >= cp.tokens) continue;  // uniform per lane group
    uint32_t w, t, b, wl, wr, wc, ti, tj;
    g.fd_N.divmod(tok, w, t);
    g.fd_nWe.divmod(w, b, wl);
    g.fd_nWw.divmod(wl, wr, wc);
    g.fd_ws.divmod(t, ti, tj);
    const bool valid = g.valid_end <= 0 || ((int)wl >= g.valid_begin && (int)wl < g.valid_end);
    int ph = (int)((wr + g.win_row_begin) * g.ws + ti) + g.shift_h;
    int pw = (int)(wc * g.ws + tj) + g.shift_w;
    if (ph >= g.Hp) ph -= g.Hp;
    if (pw >= g.Wp) pw -= g.Wp;
    const int sh = ph - g.pad_top;
    const int sw = pw - g.pad_left;
    const bool in = valid && (unsigned)sh < (unsigned)g.H && (unsigned)sw < (unsigned)g.W;
    const u32x4* src =
        reinterpret_cast<const u32x4*>(x + (in ? (((int64_t)b * g.H + sh) * g.W + sw) * g.row_bytes : 0));
    // Unconditional loads: absent chunks read chunk 0 of x and are not used.
    u32x4 raw[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k;
      raw[k] = __builtin_nontemporal_load((in && c < cp.chunks) ? src + c : reinterpret_cast<const u32x4*>(x));
    }
    // One descriptor per pass (uniform over the workgroup).
    const __amdgpu_buffer_rsrc_t out =
        buffer_rsrc(win + (int64_t)first * g.win_row_bytes,
                    (uint32_t)(min(cp.tokens - first, (uint32_t)kTokensPerPass) * g.win_row_bytes));
    const uint32_t row_off = (tok - first) * (uint32_t)g.win_row_bytes;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k;
      if (c >= cp.chunks) continue;
      u32x2 val = u32x2(g.pad_pattern);
      if (in) {
        val[0] = f32_to_bf16_bits(__uint_as_float(raw[k][0])) |
                 ((uint32_t)f32_to_bf16_bits(__uint_as_float(raw[k][1])) << 16);
        val[1] = f32_to_bf16_bits(__uint_as_float(raw[k][2])) |
                 ((uint32_t)f32_to_bf16_bits(__uint_as_float(raw[k][3])) << 16);
      }
      stream_store_sc1(val, out, row_off + (uint32_t)c * 8);
      if constexpr (kSum) {  // the values as written
        acc[k][0] += __uint_as_float(val[0] << 16);
        acc[k][1] += __uint_as_float(val[0] & 0xffff0000u);
        acc[k][2] += __uint_as_float(val[1] << 16);
        acc[k][3] += __uint_as_float(val[1] & 0xffff0000u);
      }
    }
  }
  if constexpr (kSum) {
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = sub + kL * k;
      if (c >= cp.chunks) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) atomicAdd(&s_sum[c * 4 + e], acc[k][e]);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < cp.chunks * 4; c += kThreads) unsafeAtomicAdd(cp.colsum + c, s_sum[c]);
  }
}

// Element-wise residual add of one chunk, rounding like the torch op
// (fp32 add; bf16 / fp16: add in fp32, round to nearest even).
template <int VB, int DT>
__device__ __forceinline__ typename Chunk<VB>::T add_chunk(typename Chunk<VB>::T a,
                                                           typename Chunk<VB>::T b) {
  using T = typename Chunk<VB>::T;
  T r;
  if constexpr (DT == TERRA_DTYPE_F32) {
    static_assert(VB % 4 == 0, "fp32 chunks hold whole elements");
    const float* pa = reinterpret_cast<const float*>(&a);
    const float* pb = reinterpret_cast<const float*>(&b);
    float* pr = reinterpret_cast<float*>(&r);
#pragma unroll
    for (int i = 0; i < VB / 4; ++i) pr[i] = pa[i] + pb[i];
  } else {
    static_assert(VB % 2 == 0, "16-bit chunks hold whole elements");
    const uint16_t* pa = reinterpret_cast<const uint16_t*>(&a);
    const uint16_t* pb = reinterpret_cast<const uint16_t*>(&b);
    uint16_t* pr = reinterpret_cast<uint16_t*>(&r);
#pragma unroll
    for (int i = 0; i < VB / 2; ++i) {
      if constexpr (DT == TERRA_DTYPE_BF16) {
        pr[i] = f32_to_bf16_bits(bf16_bits_to_f32(pa[i]) + bf16_bits_to_f32(pb[i]));
      } else {
        const __half ha = __ushort_as_half(pa[i]);
        const __half hb = __ushort_as_half(pb[i]);
        pr[i] = __half_as_ushort(__float2half_rn(__half2float(ha) + __half2float(hb)));
      }
    }
  }
  return r;
}

// DTW: the windows' dtype, DT's or (DT = f32) bf16: each fp32 chunk of four
// values is then read as eight bytes of bf16 and widened exactly, so the sum
// is the fp32 add torch's type promotion gives `shortcut + x` for an fp32
// shortcut and autocast's bf16 proj output.
template <int VB, int DT, bool kResidual, int DTW = DT>
__global__ __launch_bounds__(kThreads) void reverse_kernel(const uint8_t* __restrict__ win,
                                                           uint8_t* y,
                                                           const uint8_t* residual,
                                                           const CopyGeom g) {
  static_assert(DTW == DT || (DT == TERRA_DTYPE_F32 && DTW == TERRA_DTYPE_BF16 && VB == 16), "windows dtype");
  constexpr bool kWiden = DTW != DT;
  constexpr int kWinVB = kWiden ? VB / 2 : VB;
  using T = typename Chunk<VB>::T;
  using TW = typename Chunk<kWinVB>::T;
  const uint32_t first = blockIdx.x * (kThreads * kUnroll);
  const uint32_t base = first + threadIdx.x;
  const __amdgpu_buffer_rsrc_t out =
      buffer_rsrc(y + (int64_t)first * VB, min(g.total - first, (uint32_t)(kThreads * kUnroll)) * VB);
  // Unconditional loads, as in partition_kernel: lanes without a source
  // window token read chunk 0 and take zero afterwards.
  int64_t src[kUnroll];
  bool have[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t c = base + u * kThreads;
    uint32_t rest, cv, rest2, sw, b, sh;
    g.fd_cv.divmod(c, rest, cv);
    g.fd_W.divmod(rest, rest2, sw);
    g.fd_H.divmod(rest2, b, sh);
    int fi = (int)sh + g.pad_top - g.shift_h;
    int fj = (int)sw + g.pad_left - g.shift_w;
    if (fi < 0) fi += g.Hp;
    if (fj < 0) fj += g.Wp;
    uint32_t wr, ti, wc, tj;
    g.fd_ws.divmod((uint32_t)fi, wr, ti);
    g.fd_ws.divmod((uint32_t)fj, wc, tj);
    const int wr_l = (int)wr - g.win_row_begin;
    const int wl = wr_l * g.nWw + (int)wc;
    const bool valid = g.valid_end <= 0 || (wl >= g.valid_begin && wl < g.valid_end);
    have[u] = c < g.total && (unsigned)wr_l < (unsigned)g.win_rows && valid;
    const int64_t w = (int64_t)b * g.win_rows * g.nWw + wl;
    src[u] = have[u] ? (w * g.N + (int64_t)(ti * g.ws + tj)) * g.win_row_bytes + (int64_t)cv * kWinVB : 0;
  }
  TW wv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) wv[u] = stream_load(reinterpret_cast<const TW*>(win + src[u]));
  T vals[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if constexpr (kWiden) {  // bf16 -> fp32 is exact: the bits move up 16 places
      TW w = wv[u];
      if (!have[u]) w = TW(0u);
      vals[u] = T{w[0] << 16, w[0] & 0xffff0000u, w[1] << 16, w[1] & 0xffff0000u};
    } else {
      vals[u] = wv[u];
      if (!have[u]) vals[u] = fill_chunk<VB>(0u);
    }
  }
  if constexpr (kResidual) {
    T r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t c = base + u * kThreads;
      r[u] = stream_load(reinterpret_cast<const T*>(residual) + (c < g.total ? c : 0u));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) vals[u] = add_chunk<VB, DT>(r[u], vals[u]);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (base + u * kThreads < g.total) stream_store_sc1(vals[u], out, (threadIdx.x + u * kThreads) * VB);
}

uint32_t pad_pattern(int dtype, float v) {
  switch (dtype) {
    case TERRA_DTYPE_F32: {
      uint32_t u;
      memcpy(&u, &v, 4);
      return u;
    }
    case TERRA_DTYPE_BF16: {
      uint32_t u;
      memcpy(&u, &v, 4);
      uint32_t b;
      if ((u & 0x7fffffffu) > 0x7f800000u) b = (u >> 16) | 0x40;
      else b = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
      return (b & 0xffff) | (b << 16);
    }
    case TERRA_DTYPE_F16: {
      const __half h = __float2half(v);
      uint16_t b;
      memcpy(&b, &h, 2);
      return (uint32_t)b | ((uint32_t)b << 16);
    }
    default: {
      const uint32_t b = (uint32_t)((int)v) & 0xff;
      return b | (b << 8) | (b << 16) | (b << 24);
    }
  }
}

// Validates `geom` and fills the kernel-side geometry.  `total_dst_tokens`
// selects which side is the destination (window tokens or grid tokens).
int prepare(const terra_swin_geom* geom, int dtype, bool dest_is_windows, CopyGeom* g, int* vb,
            const void* p0, const void* p1, const void* p2) {
  if (geom == nullptr) return fail(TERRA_ERR_NULL, "geom is NULL");
  const int elt = dtype_size(dtype);
  if (elt == 0) return fail(TERRA_ERR_DTYPE, "unknown dtype %d", dtype);
  GeomDims dims;
  const int st = validate_geom(geom, &dims);
  if (st != TERRA_OK) return st;
  const terra_swin_geom& q = *geom;
  const int64_t Hp = dims.Hp, Wp = dims.Wp, nWw = dims.nWw, rows = dims.rows, nWe = dims.nWe;
  const int64_t row_bytes = (int64_t)q.channels * elt;
  int v = 16;
  while (v > 1 && (row_bytes % v) != 0) v >>= 1;
  for (const void* p : {p0, p1, p2}) {
    while (v > 1 && p != nullptr && ((uintptr_t)p % v) != 0) v >>= 1;
  }
  if (v < elt) return fail(TERRA_ERR_ALIGN, "pointer not aligned to its element size");
  const int64_t N = (int64_t)q.window * q.window;
  const int64_t tokens = dest_is_windows ? (int64_t)q.batch * nWe * N
                                         : (int64_t)q.batch * q.height * q.width;
  const int64_t chunks = tokens * (row_bytes / v);
  if (chunks >= (1ll << 31))
    return fail(TERRA_ERR_SHAPE, "%lld chunks exceed one launch (2^31); split the batch", (long long)chunks);
  g->H = q.height; g->W = q.width; g->ws = q.window; g->Hp = (int32_t)Hp; g->Wp = (int32_t)Wp;
  g->shift_h = q.shift_h; g->shift_w = q.shift_w; g->pad_top = q.pad_top; g->pad_left = q.pad_left;
  g->win_row_begin = q.win_row_begin; g->win_rows = (int32_t)rows; g->nWw = (int32_t)nWw;
  g->valid_begin = q.valid_end > 0 ? q.valid_begin : 0;
  g->valid_end = q.valid_end > 0 ? q.valid_end : 0;
  g->N = (int32_t)N;
  g->row_bytes = row_bytes;
  g->win_row_bytes = row_bytes;
  g->fd_cv = FastDiv((uint32_t)(row_bytes / v));
  g->fd_N = FastDiv((uint32_t)N);
  g->fd_nWe = FastDiv((uint32_t)nWe);
  g->fd_nWw = FastDiv((uint32_t)nWw);
  g->fd_ws = FastDiv((uint32_t)q.window);
  g->fd_W = FastDiv((uint32_t)q.width);
  g->fd_H = FastDiv((uint32_t)q.height);
  g->total = (uint32_t)chunks;
  *vb = v;
  return TERRA_OK;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return TERRA_OK;
}

template <int VB>
void launch_partition(const void* x, void* win, const CopyGeom& g, hipStream_t s) {
  const uint32_t blocks = (g.total + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  partition_kernel<VB><<<blocks, kThreads, 0, s>>>((const uint8_t*)x, (uint8_t*)win, g);
}

template <int DT, int CPL, int kL = kLnLanes, int DTO = DT>
void launch_partition_ln(const void* x, void* win, const CopyGeom& g, const LnParams& ln, hipStream_t s) {
  constexpr uint32_t kTokensPerBlock = kThreads / kL;
  const uint32_t blocks = (ln.tokens + kTokensPerBlock - 1) / kTokensPerBlock;
  partition_ln_kernel<DT, CPL, kL, DTO><<<blocks, kThreads, 0, s>>>((const uint8_t*)x, (uint8_t*)win, g, ln);
}

template <int DT, int DTO = DT>
void dispatch_partition_ln(int cpl, const void* x, void* win, const CopyGeom& g, const LnParams& ln,
                           hipStream_t s) {
  if (cpl <= 1) launch_partition_ln<DT, 1, kLnLanes, DTO>(x, win, g, ln, s);
  else if (cpl <= 2) launch_partition_ln<DT, 2, kLnLanes, DTO>(x, win, g, ln, s);
  else if (cpl <= 3) launch_partition_ln<DT, 3, kLnLanes, DTO>(x, win, g, ln, s);
  else if (cpl <= 4) launch_partition_ln<DT, 4, kLnLanes, DTO>(x, win, g, ln, s);
  else if (cpl <= 6) launch_partition_ln<DT, 6, kLnLanes, DTO>(x, win, g, ln, s);
  else if (cpl <= 8) launch_partition_ln<DT, 4, 16, DTO>(x, win, g, ln, s);  // 16 lanes per token
  else if (cpl <= 12) launch_partition_ln<DT, 6, 16, DTO>(x, win, g, ln, s);
  else if (cpl <= 16) launch_partition_ln<DT, 8, 16, DTO>(x, win, g, ln, s);  // bf16 C = 1024
  else if (cpl <= 24) launch_partition_ln<DT, 12, 16, DTO>(x, win, g, ln, s);
  else launch_partition_ln<DT, 16, 16, DTO>(x, win, g, ln, s);                // fp32 C = 1024
}

// Resident workgroups of the LayerNorm backward (grid-stride over the
// tokens), queried per device and instance once.
template <int DT, int CPL, int kL, bool kRes, int DTG = DT>
int launch_partition_ln_bwd(const void* dwin, const void* x, void* dx, const void* dres, const CopyGeom& g,
                            const LnBwdParams& ln, hipStream_t s) {
  auto kern = partition_ln_bwd_kernel<DT, CPL, kL, kRes, DTG>;
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, 0) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the LayerNorm backward grid for this device");
    cache[dev] = cus * (per_cu > 0 ? per_cu : 1);
  }
  constexpr uint32_t kTokensPerPass = kThreads / kL;
  const uint32_t need = (ln.tokens + kTokensPerPass - 1) / kTokensPerPass;
  const uint32_t blocks = need < (uint32_t)cache[dev] ? need : (uint32_t)cache[dev];
  kern<<<blocks, kThreads, 0, s>>>((const uint8_t*)dwin, (const uint8_t*)x, (uint8_t*)dx, (const uint8_t*)dres, g,
                                   ln);
  return TERRA_OK;
}

template <int DT, bool kRes, int DTG = DT>
int dispatch_partition_ln_bwd(int cpl, const void* dwin, const void* x, void* dx, const void* dres,
                              const CopyGeom& g, const LnBwdParams& ln, hipStream_t s) {
  if (cpl <= 1) return launch_partition_ln_bwd<DT, 1, 8, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 2) return launch_partition_ln_bwd<DT, 2, 8, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 3) return launch_partition_ln_bwd<DT, 3, 8, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 4) return launch_partition_ln_bwd<DT, 4, 8, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 8) return launch_partition_ln_bwd<DT, 4, 16, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 12) return launch_partition_ln_bwd<DT, 6, 16, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  if (cpl <= 16 || DT != TERRA_DTYPE_F32)
    return launch_partition_ln_bwd<DT, 8, 16, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  // fp32 rows of more than 512 channels (16-bit rows of at most 1024 channels
  // never get here)
  if constexpr (DT == TERRA_DTYPE_F32) {
    if (cpl <= 24) return launch_partition_ln_bwd<DT, 12, 16, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
    return launch_partition_ln_bwd<DT, 16, 16, kRes, DTG>(dwin, x, dx, dres, g, ln, s);
  }
  return fail(TERRA_ERR_UNSUPPORTED, "fused LayerNorm backward: row too wide");
}

template <int VB, int DT>
void launch_reverse(const void* win, void* y, const void* res, const CopyGeom& g, hipStream_t s) {
  const uint32_t blocks = (g.total + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  if constexpr (DT != TERRA_DTYPE_U8 && (DT != TERRA_DTYPE_F32 || VB >= 4)) {
    if (res != nullptr) {
      reverse_kernel<VB, DT, true><<<blocks, kThreads, 0, s>>>((const uint8_t*)win, (uint8_t*)y,
                                                              (const uint8_t*)res, g);
      return;
    }
  }
  reverse_kernel<VB, DT, false><<<blocks, kThreads, 0, s>>>((const uint8_t*)win, (uint8_t*)y, nullptr, g);
}

// Resident workgroups of a grid-stride kernel on the current device, at most
// max_per_cu per CU, queried once per device and kernel instance.
template <typename Kernel>
int resident_blocks(Kernel kern, int max_per_cu, int* cache, int* out) {
  constexpr int kMaxDevices = 64;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, 0) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size a grid-stride launch for this device");
    per_cu = per_cu < 1 ? 1 : (per_cu > max_per_cu ? max_per_cu : per_cu);
    cache[dev] = cus * per_cu;
  }
  *out = cache[dev];
  return TERRA_OK;
}

template <int CPL, int kL, bool kSum>
int launch_partition_cast(const void* x, void* win, const CopyGeom& g, const CastParams& cp, hipStream_t s) {
  auto kern = partition_cast_kernel<CPL, kL, kSum>;
  static int cache[64] = {0};
  int resident = 0;
  // With column sums every workgroup ends with one float atomic per channel
  // into the same C addresses: four workgroups per CU measured 129 us at c3
  // (fp32 -> bf16 with sums; 117 us without), against 137 with two, 205 with
  // one and 144 with all seven resident.
  const int st = resident_blocks(kern, kSum ? 4 : 64, cache, &resident);
  if (st != TERRA_OK) return st;
  constexpr uint32_t kTokensPerPass = kThreads / kL;
  const uint32_t need = (cp.tokens + kTokensPerPass - 1) / kTokensPerPass;
  const uint32_t blocks = need < (uint32_t)resident ? need : (uint32_t)resident;
  kern<<<blocks, kThreads, 0, s>>>((const uint8_t*)x, (uint8_t*)win, g, cp);
  return TERRA_OK;
}

template <bool kSum>
int dispatch_partition_cast(int cpl, const void* x, void* win, const CopyGeom& g, const CastParams& cp,
                            hipStream_t s) {
  if (cpl <= 1) return launch_partition_cast<1, 8, kSum>(x, win, g, cp, s);
  if (cpl <= 2) return launch_partition_cast<2, 8, kSum>(x, win, g, cp, s);
  if (cpl <= 3) return launch_partition_cast<3, 8, kSum>(x, win, g, cp, s);
  if (cpl <= 4) return launch_partition_cast<4, 8, kSum>(x, win, g, cp, s);
  if (cpl <= 6) return launch_partition_cast<6, 8, kSum>(x, win, g, cp, s);
  if (cpl <= 8) return launch_partition_cast<4, 16, kSum>(x, win, g, cp, s);
  if (cpl <= 12) return launch_partition_cast<6, 16, kSum>(x, win, g, cp, s);
  if (cpl <= 16) return launch_partition_cast<8, 16, kSum>(x, win, g, cp, s);
  if (cpl <= 24) return launch_partition_cast<12, 16, kSum>(x, win, g, cp, s);
  return launch_partition_cast<16, 16, kSum>(x, win, g, cp, s);  // fp32 C = 1024
}

// bf16 windows into fp32 y (reverse_kernel's DTW); 16-byte fp32 chunks.
void launch_reverse_widen(const void* win, void* y, const void* res, const CopyGeom& g, hipStream_t s) {
  const uint32_t blocks = (g.total + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  if (res != nullptr)
    reverse_kernel<16, TERRA_DTYPE_F32, true, TERRA_DTYPE_BF16><<<blocks, kThreads, 0, s>>>(
        (const uint8_t*)win, (uint8_t*)y, (const uint8_t*)res, g);
  else
    reverse_kernel<16, TERRA_DTYPE_F32, false, TERRA_DTYPE_BF16><<<blocks, kThreads, 0, s>>>(
        (const uint8_t*)win, (uint8_t*)y, nullptr, g);
}

template <int VB>
void dispatch_reverse(int dtype, const void* win, void* y, const void* res, const CopyGeom& g,
                      hipStream_t s) {
  switch (dtype) {
    case TERRA_DTYPE_F32: launch_reverse<VB, TERRA_DTYPE_F32>(win, y, res, g, s); break;
    case TERRA_DTYPE_F16: launch_reverse<VB, TERRA_DTYPE_F16>(win, y, res, g, s); break;
    case TERRA_DTYPE_BF16: launch_reverse<VB, TERRA_DTYPE_BF16>(win, y, res, g, s); break;
    default: launch_reverse<VB, TERRA_DTYPE_U8>(win, y, res, g, s); break;
  }
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_partition(const void* x, void* windows, int dtype,
                                    const terra_swin_geom* geom, float pad_value, void* stream) {
  clear_error();
  if (x == nullptr || windows == nullptr) return fail(TERRA_ERR_NULL, "x or windows is NULL");
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, dtype, true, &g, &vb, x, windows, nullptr);
  if (st != TERRA_OK) return st;
  g.pad_pattern = pad_pattern(dtype, pad_value);
  hipStream_t s = (hipStream_t)stream;
  switch (vb) {
    case 16: launch_partition<16>(x, windows, g, s); break;
    case 8: launch_partition<8>(x, windows, g, s); break;
    case 4: launch_partition<4>(x, windows, g, s); break;
    case 2: launch_partition<2>(x, windows, g, s); break;
    default: launch_partition<1>(x, windows, g, s); break;
  }
  return launch_status("terra_swin_partition");
}

namespace terra {
namespace {

// terra_swin_partition_ln with windows of dtype wdt: x's dtype, or bf16 for
// fp32 x (partition_ln_kernel's DTO).
int partition_ln_impl(const void* x, int dtype, void* windows, int wdt, const terra_swin_geom* geom,
                      const float* gamma, const float* beta, float eps, float pad_value, void* stream) {
  if (x == nullptr || windows == nullptr) return fail(TERRA_ERR_NULL, "x or windows is NULL");
  if (dtype != TERRA_DTYPE_F32 && dtype != TERRA_DTYPE_BF16 && dtype != TERRA_DTYPE_F16)
    return fail(TERRA_ERR_DTYPE, "fused LayerNorm supports f32, f16 and bf16 (got dtype %d)", dtype);
  const bool cast = wdt != dtype;
  if (cast && !(dtype == TERRA_DTYPE_F32 && wdt == TERRA_DTYPE_BF16))
    return fail(TERRA_ERR_DTYPE, "fused LayerNorm: windows of dtype %d from x of dtype %d (mixed: f32 x, bf16 windows)",
                wdt, dtype);
  if (!(eps >= 0.f)) return fail(TERRA_ERR_SHAPE, "eps must be non-negative");
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, dtype, true, &g, &vb, x, windows, nullptr);
  if (st != TERRA_OK) return st;
  if (vb != 16)
    return fail(TERRA_ERR_ALIGN, "fused LayerNorm needs 16-byte aligned rows (C * element size %% 16 == 0)");
  for (const float* p : {gamma, beta})
    if (p != nullptr && (uintptr_t)p % 4 != 0) return fail(TERRA_ERR_ALIGN, "gamma / beta must be 4-byte aligned");
  const int chunks = (int)(g.row_bytes / 16);
  const int cpl = (chunks + kLnLanes - 1) / kLnLanes;
  if (chunks > kLnMaxChunks || geom->channels > kLnMaxChannels)
    return fail(TERRA_ERR_UNSUPPORTED, "fused LayerNorm handles up to %d channels in rows of up to %d bytes (got %d "
                "channels, %lld bytes)", kLnMaxChannels, kLnMaxChunks * 16, geom->channels, (long long)g.row_bytes);
  g.win_row_bytes = (int64_t)geom->channels * dtype_size(wdt);
  g.pad_pattern = pad_pattern(wdt, pad_value);
  LnParams ln;
  ln.gamma = gamma;
  ln.beta = beta;
  ln.eps = eps;
  ln.inv_c = 1.0f / (float)geom->channels;
  ln.chunks = chunks;
  ln.tokens = g.total / (uint32_t)chunks;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TERRA_DTYPE_F32:
      if (cast)
        dispatch_partition_ln<TERRA_DTYPE_F32, TERRA_DTYPE_BF16>(cpl, x, windows, g, ln, s);
      else
        dispatch_partition_ln<TERRA_DTYPE_F32>(cpl, x, windows, g, ln, s);
      break;
    case TERRA_DTYPE_F16: dispatch_partition_ln<TERRA_DTYPE_F16>(cpl, x, windows, g, ln, s); break;
    default: dispatch_partition_ln<TERRA_DTYPE_BF16>(cpl, x, windows, g, ln, s); break;
  }
  return launch_status("terra_swin_partition_ln");
}

}  // namespace
}  // namespace terra

extern "C" int terra_swin_partition_ln(const void* x, void* windows, int dtype, const terra_swin_geom* geom,
                                       const float* gamma, const float* beta, float eps, float pad_value,
                                       void* stream) {
  clear_error();
  return partition_ln_impl(x, dtype, windows, dtype, geom, gamma, beta, eps, pad_value, stream);
}

extern "C" int terra_swin_partition_ln_mixed(const void* x, int x_dtype, void* windows, int windows_dtype,
                                             const terra_swin_geom* geom, const float* gamma, const float* beta,
                                             float eps, float pad_value, void* stream) {
  clear_error();
  return partition_ln_impl(x, x_dtype, windows, windows_dtype, geom, gamma, beta, eps, pad_value, stream);
}

extern "C" int terra_swin_reverse(const void* windows, void* y, const void* residual, int dtype,
                                  const terra_swin_geom* geom, void* stream) {
  clear_error();
  if (windows == nullptr || y == nullptr) return fail(TERRA_ERR_NULL, "windows or y is NULL");
  if (residual != nullptr && dtype == TERRA_DTYPE_U8)
    return fail(TERRA_ERR_DTYPE, "residual add is not defined for u8");
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, dtype, false, &g, &vb, windows, y, residual);
  if (st != TERRA_OK) return st;
  g.pad_pattern = 0;
  hipStream_t s = (hipStream_t)stream;
  switch (vb) {
    case 16: dispatch_reverse<16>(dtype, windows, y, residual, g, s); break;
    case 8: dispatch_reverse<8>(dtype, windows, y, residual, g, s); break;
    case 4: dispatch_reverse<4>(dtype, windows, y, residual, g, s); break;
    case 2:
      if (dtype == TERRA_DTYPE_F16) launch_reverse<2, TERRA_DTYPE_F16>(windows, y, residual, g, s);
      else if (dtype == TERRA_DTYPE_BF16) launch_reverse<2, TERRA_DTYPE_BF16>(windows, y, residual, g, s);
      else launch_reverse<2, TERRA_DTYPE_U8>(windows, y, nullptr, g, s);
      break;
    default: launch_reverse<1, TERRA_DTYPE_U8>(windows, y, nullptr, g, s); break;
  }
  return launch_status("terra_swin_reverse");
}

namespace terra {
namespace {

// terra_swin_partition_ln_bwd with a windows gradient of dtype gdt: x's, or
// bf16 for fp32 x (partition_ln_bwd_kernel's DTG).
int partition_ln_bwd_impl(const void* dwindows, int gdt, const void* x, const void* dresidual, void* dx, int dtype,
                          const terra_swin_geom* geom, const float* gamma, float eps, float* dgamma, float* dbeta,
                          void* stream) {
  if (dwindows == nullptr || x == nullptr || dx == nullptr) return fail(TERRA_ERR_NULL, "dwindows, x or dx is NULL");
  if (dtype != TERRA_DTYPE_F32 && dtype != TERRA_DTYPE_BF16 && dtype != TERRA_DTYPE_F16)
    return fail(TERRA_ERR_DTYPE, "fused LayerNorm backward supports f32, f16 and bf16 (got dtype %d)", dtype);
  const bool cast = gdt != dtype;
  if (cast && !(dtype == TERRA_DTYPE_F32 && gdt == TERRA_DTYPE_BF16))
    return fail(TERRA_ERR_DTYPE,
                "fused LayerNorm backward: a windows gradient of dtype %d for x of dtype %d (mixed: f32 x, bf16 gradient)",
                gdt, dtype);
  if (!(eps >= 0.f)) return fail(TERRA_ERR_SHAPE, "eps must be non-negative");
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, dtype, false, &g, &vb, dwindows, x, dx);
  if (st != TERRA_OK) return st;
  if (vb != 16 || (dresidual != nullptr && ((uintptr_t)dresidual & 15u) != 0))
    return fail(TERRA_ERR_ALIGN, "fused LayerNorm backward needs 16-byte aligned rows and tensors");
  for (const float* p : {gamma, (const float*)dgamma, (const float*)dbeta})
    if (p != nullptr && (uintptr_t)p % 4 != 0) return fail(TERRA_ERR_ALIGN, "gamma / dgamma / dbeta must be 4-byte aligned");
  const int chunks = (int)(g.row_bytes / 16);
  if (chunks > kLnMaxChunks || geom->channels > kLnMaxChannels)
    return fail(TERRA_ERR_UNSUPPORTED, "fused LayerNorm backward handles up to %d channels in rows of up to %d bytes",
                kLnMaxChannels, kLnMaxChunks * 16);
  const int64_t grid_bytes = (int64_t)geom->batch * geom->height * geom->width * g.row_bytes;
  const uintptr_t xa = (uintptr_t)x, da = (uintptr_t)dx;
  if (xa < da + (uintptr_t)grid_bytes && da < xa + (uintptr_t)grid_bytes)
    return fail(TERRA_ERR_SHAPE, "dx must not overlap x");
  g.win_row_bytes = (int64_t)geom->channels * dtype_size(gdt);
  LnBwdParams ln;
  ln.gamma = gamma;
  ln.dgamma = dgamma;
  ln.dbeta = dbeta;
  ln.eps = eps;
  ln.inv_c = 1.0f / (float)geom->channels;
  ln.chunks = chunks;
  ln.tokens = (uint32_t)((int64_t)geom->batch * geom->height * geom->width);
  const int cpl = (chunks + kLnLanes - 1) / kLnLanes;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  const bool res = dresidual != nullptr;
  switch (dtype) {
    case TERRA_DTYPE_F32:
      if (cast)
        rc = res ? dispatch_partition_ln_bwd<TERRA_DTYPE_F32, true, TERRA_DTYPE_BF16>(cpl, dwindows, x, dx, dresidual,
                                                                                    g, ln, s)
                 : dispatch_partition_ln_bwd<TERRA_DTYPE_F32, false, TERRA_DTYPE_BF16>(cpl, dwindows, x, dx, nullptr,
                                                                                     g, ln, s);
      else
        rc = res ? dispatch_partition_ln_bwd<TERRA_DTYPE_F32, true>(cpl, dwindows, x, dx, dresidual, g, ln, s)
                 : dispatch_partition_ln_bwd<TERRA_DTYPE_F32, false>(cpl, dwindows, x, dx, nullptr, g, ln, s);
      break;
    case TERRA_DTYPE_F16:
      rc = res ? dispatch_partition_ln_bwd<TERRA_DTYPE_F16, true>(cpl, dwindows, x, dx, dresidual, g, ln, s)
               : dispatch_partition_ln_bwd<TERRA_DTYPE_F16, false>(cpl, dwindows, x, dx, nullptr, g, ln, s);
      break;
    default:
      rc = res ? dispatch_partition_ln_bwd<TERRA_DTYPE_BF16, true>(cpl, dwindows, x, dx, dresidual, g, ln, s)
               : dispatch_partition_ln_bwd<TERRA_DTYPE_BF16, false>(cpl, dwindows, x, dx, nullptr, g, ln, s);
      break;
  }
  if (rc != TERRA_OK) return rc;
  return launch_status("terra_swin_partition_ln_bwd");
}

}  // namespace
}  // namespace terra

extern "C" int terra_swin_partition_ln_bwd(const void* dwindows, const void* x, const void* dresidual, void* dx,
                                           int dtype, const terra_swin_geom* geom, const float* gamma, float eps,
                                           float* dgamma, float* dbeta, void* stream) {
  clear_error();
  return partition_ln_bwd_impl(dwindows, dtype, x, dresidual, dx, dtype, geom, gamma, eps, dgamma, dbeta, stream);
}

extern "C" int terra_swin_partition_ln_bwd_mixed(const void* dwindows, int dwindows_dtype, const void* x,
                                                 const void* dresidual, void* dx, int x_dtype,
                                                 const terra_swin_geom* geom, const float* gamma, float eps,
                                                 float* dgamma, float* dbeta, void* stream) {
  clear_error();
  return partition_ln_bwd_impl(dwindows, dwindows_dtype, x, dresidual, dx, x_dtype, geom, gamma, eps, dgamma, dbeta,
                               stream);
}

extern "C" int terra_swin_partition_mixed(const void* x, int x_dtype, void* windows, int windows_dtype,
                                          const terra_swin_geom* geom, float pad_value, float* column_sums,
                                          void* stream) {
  clear_error();
  if (x == nullptr || windows == nullptr) return fail(TERRA_ERR_NULL, "x or windows is NULL");
  if (x_dtype != TERRA_DTYPE_F32 || windows_dtype != TERRA_DTYPE_BF16)
    return fail(TERRA_ERR_DTYPE, "mixed partition: f32 x into bf16 windows only (got dtype %d into %d)", x_dtype,
                windows_dtype);
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, TERRA_DTYPE_F32, true, &g, &vb, x, nullptr, nullptr);
  if (st != TERRA_OK) return st;
  if (vb != 16 || ((uintptr_t)windows & 7u) != 0 || ((uintptr_t)column_sums & 3u) != 0)
    return fail(TERRA_ERR_ALIGN, "mixed partition needs C %% 4 == 0, 16-byte aligned x, 8-byte aligned windows and "
                "4-byte aligned column sums");
  const int chunks = (int)(g.row_bytes / 16);
  if (chunks > kLnMaxChunks)
    return fail(TERRA_ERR_UNSUPPORTED, "mixed partition handles up to %d channels (got %d)", kLnMaxChunks * 4,
                geom->channels);
  g.win_row_bytes = (int64_t)geom->channels * 2;
  g.pad_pattern = pad_pattern(TERRA_DTYPE_BF16, pad_value);
  CastParams cp;
  cp.colsum = column_sums;
  cp.chunks = chunks;
  cp.tokens = g.total / (uint32_t)chunks;
  if (cp.tokens == 0) return TERRA_OK;
  const int cpl = (chunks + kLnLanes - 1) / kLnLanes;
  hipStream_t s = (hipStream_t)stream;
  const int rc = column_sums != nullptr ? dispatch_partition_cast<true>(cpl, x, windows, g, cp, s)
                                        : dispatch_partition_cast<false>(cpl, x, windows, g, cp, s);
  if (rc != TERRA_OK) return rc;
  return launch_status("terra_swin_partition_mixed");
}

extern "C" int terra_swin_reverse_mixed(const void* windows, int windows_dtype, void* y, const void* residual,
                                        int dtype, const terra_swin_geom* geom, void* stream) {
  clear_error();
  if (windows == nullptr || y == nullptr) return fail(TERRA_ERR_NULL, "windows or y is NULL");
  if (dtype != TERRA_DTYPE_F32 || windows_dtype != TERRA_DTYPE_BF16)
    return fail(TERRA_ERR_DTYPE, "mixed reverse: bf16 windows into f32 y only (got dtype %d into %d)", windows_dtype,
                dtype);
  CopyGeom g;
  int vb = 0;
  const int st = prepare(geom, TERRA_DTYPE_F32, false, &g, &vb, y, residual, nullptr);
  if (st != TERRA_OK) return st;
  if (vb != 16 || ((uintptr_t)windows & 7u) != 0)
    return fail(TERRA_ERR_ALIGN, "mixed reverse needs C %% 4 == 0, 16-byte aligned y / residual and 8-byte aligned "
                "windows");
  g.win_row_bytes = (int64_t)geom->channels * 2;
  g.pad_pattern = 0;
  if (g.total == 0) return TERRA_OK;
  launch_reverse_widen(windows, y, residual, g, (hipStream_t)stream);
  return launch_status("terra_swin_reverse_mixed");
}
