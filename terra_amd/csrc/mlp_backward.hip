// The MLP half's GELU backward for training, with the column sums of its
// result (fc1's bias gradient) in the same pass.
//
//   dh[t, f] = dout[t, f] * (Phi(h) + h phi(h)),  h = h[t, f]
//   Phi(h) = 0.5 (1 + erf(h / sqrt 2)),  phi(h) = exp(-h^2 / 2) / sqrt(2 pi)
//
// the derivative of nn.GELU() (erf form, models/mlp.py:165) applied to the
// gradient fc2's backward gives, computed in fp32 and rounded once to the
// activation dtype, and optionally  colsum[f] += sum_t dh[t, f]  over the
// rounded values (fc1's bias gradient, models/mlp.py:162).
#include "common.h"

namespace terra {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGeluThreads = 512;
constexpr int kGeluWaves = kGeluThreads / 64;
constexpr int kGeluMaxChunks = 512;  // 16-byte chunks per row: bf16 F <= 4096, fp32 F <= 2048

// Rows per wave per pass, their loads in flight together: about 8 chunks of
// each input per lane.
template <int CPL>
constexpr int gelu_rows() { return CPL >= 8 ? 1 : 8 / CPL; }

// d/dh GELU(h) in fp32 (the erf form's exact derivative, before the
// multiplication by the incoming gradient).
__device__ __forceinline__ float gelu_slope(float h) {
  constexpr float kAlpha = 0.70710678118654752f;  // 1 / sqrt(2)
  constexpr float kBeta = 0.39894228040143268f;   // 1 / sqrt(2 pi)
  const float cdf = 0.5f * (1.f + erff(h * kAlpha));
  const float pdf = expf(-0.5f * h * h) * kBeta;
  return cdf + h * pdf;
}

// The slope of a bf16 input by table.  fc1's output is rounded to bf16
// before the activation, so the slope takes one of 2^16 values; for
// 2^-26 <= |h| < 32 it is read from an fp32 table each workgroup fills at
// start with gelu_slope itself (so the product g * slope is bit for bit the
// one computed directly).  Outside that range it has a closed form in fp32:
// 0.5 for |h| < 2^-26 (erf(h / sqrt 2) and h phi(h) are then below half an
// ulp of 1 and of 0.5), 1 for 32 <= h < inf and 0 for -inf < h <= -32 (erf
// is +-1 and phi(h) underflows to 0), NaN for +-inf (inf * 0) and NaN.
constexpr uint32_t kSlopeLo = 0x3280;  // bf16 bits of 2^-26
constexpr uint32_t kSlopeHi = 0x4200;  // bf16 bits of 32
constexpr int kSlopeSpan = (int)(kSlopeHi - kSlopeLo);  // 3968 entries per sign
constexpr int kSlopeEntries = 2 * kSlopeSpan;

__device__ __forceinline__ void slope_table_fill(float* table) {
  for (int e = threadIdx.x; e < kSlopeEntries; e += blockDim.x) {
    const uint32_t sign = e >= kSlopeSpan ? 0x8000u : 0u;
    const uint32_t bits = sign | (kSlopeLo + (uint32_t)(e - (sign ? kSlopeSpan : 0)));
    table[e] = gelu_slope(__uint_as_float(bits << 16));
  }
}

// g * slope(h) for the bf16 bits hb of h (in the low 16 bits).
__device__ __forceinline__ float gelu_grad_bf16(float g, uint32_t hb, const float* table) {
  const uint32_t mag = hb & 0x7fffu;
  const uint32_t sign = (hb >> 15) & 1u;
  const uint32_t d = mag - kSlopeLo;  // wraps below kSlopeLo
  const float tab = table[(d < (uint32_t)kSlopeSpan ? d : 0u) + (sign ? kSlopeSpan : 0u)];
  const float outer = mag >= 0x7f80u ? __uint_as_float(0x7fc00000u) : (sign ? 0.f : 1.f);
  const float slope = d < (uint32_t)kSlopeSpan ? tab : (mag < kSlopeLo ? 0.5f : outer);
  return g * slope;
}

template <int DT> struct GeluElt;
template <> struct GeluElt<TERRA_DTYPE_F32> { static constexpr int kPerChunk = 4; };
template <> struct GeluElt<TERRA_DTYPE_BF16> { static constexpr int kPerChunk = 8; };

// kL lanes per row (64: one wave; 32: two rows side by side, for rows of
// 32 * odd chunks that would leave half a wave idle on their last chunk),
// kGeluRows rows per lane group and pass, lane l of a group holding the
// 16-byte chunks l, l + kL, ... of its rows, so its columns stay fixed and
// their sums stay in registers.  Workgroups loop over the rows grid-stride
// (the resident count, capped); at the end each workgroup reduces its lanes'
// sums in LDS and adds them to colsum with one float atomic per column.
template <int DT, int CPL, bool kSum, int kL = 64>
__global__ __launch_bounds__(kGeluThreads) void gelu_bwd_kernel(const uint8_t* __restrict__ dout,
                                                                const uint8_t* __restrict__ h,
                                                                uint8_t* __restrict__ dh, float* colsum,
                                                                int64_t rows, int chunks) {
  constexpr int E = GeluElt<DT>::kPerChunk;
  constexpr int kMaxCols = CPL * 64 * E;
  constexpr int kGeluRows = gelu_rows<CPL>();
  constexpr int kSub = 64 / kL;                 // rows side by side in a wave
  constexpr int kWaveRows = kGeluRows * kSub;   // rows per wave and pass
  static_assert(kL == 64 || kL == 32, "lanes per row");
  constexpr bool kTable = DT == TERRA_DTYPE_BF16;
  __shared__ float s_sum[kSum ? kMaxCols : 1];
  __shared__ float s_slope[kTable ? kSlopeEntries : 1];
  if constexpr (kSum)
    for (int c = threadIdx.x; c < kMaxCols; c += kGeluThreads) s_sum[c] = 0.f;
  if constexpr (kTable) slope_table_fill(s_slope);
  if constexpr (kSum || kTable) __syncthreads();
  const int lane = threadIdx.x & (kL - 1);      // lane within its row group
  const int sub = kSub == 1 ? 0 : (int)((threadIdx.x & 63) / kL);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row_bytes = (int64_t)chunks * 16;
  float acc[CPL][E];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[k][e] = 0.f;

  const int64_t stride = (int64_t)gridDim.x * kGeluWaves * kWaveRows;
  for (int64_t r0 = ((int64_t)blockIdx.x * kGeluWaves + wave) * kWaveRows; r0 < rows; r0 += stride) {
    u32x4 gv[kGeluRows][CPL], hv[kGeluRows][CPL];
#pragma unroll
    for (int i = 0; i < kGeluRows; ++i) {
      const int64_t ri = r0 + kSub * i + sub;
      const int64_t r = ri < rows ? ri : r0;  // a missing row re-reads row r0 and stores nothing
      const u32x4* gs = reinterpret_cast<const u32x4*>(dout + r * row_bytes);
      const u32x4* hs = reinterpret_cast<const u32x4*>(h + r * row_bytes);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const int c = lane + kL * k < chunks ? lane + kL * k : 0;
        gv[i][k] = __builtin_nontemporal_load(gs + c);
        hv[i][k] = __builtin_nontemporal_load(hs + c);
      }
    }
#pragma unroll
    for (int i = 0; i < kGeluRows; ++i) {
      if (r0 + kSub * i >= rows) break;  // uniform per wave
      // One descriptor over the wave's kSub rows of this step (uniform).
      const int64_t left = rows - (r0 + kSub * i);
      const __amdgpu_buffer_rsrc_t out =
          buffer_rsrc(dh + (r0 + kSub * i) * row_bytes, (uint32_t)((left < kSub ? left : kSub) * row_bytes));
      const bool live = r0 + kSub * i + sub < rows;
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        const int c = lane + kL * k;
        if (c >= chunks || !live) continue;
        u32x4 res;
        if constexpr (DT == TERRA_DTYPE_BF16) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t g2 = gv[i][k][q], h2 = hv[i][k][q];
            const uint32_t lo = f32_to_bf16_bits(gelu_grad_bf16(__uint_as_float(g2 << 16), h2, s_slope));
            const uint32_t hi =
                f32_to_bf16_bits(gelu_grad_bf16(__uint_as_float(g2 & 0xffff0000u), h2 >> 16, s_slope));
            res[q] = lo | (hi << 16);
            if constexpr (kSum) {  // the values as written
              acc[k][2 * q] += __uint_as_float(lo << 16);
              acc[k][2 * q + 1] += __uint_as_float(hi << 16);
            }
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float v = __uint_as_float(gv[i][k][q]) * gelu_slope(__uint_as_float(hv[i][k][q]));
            res[q] = __float_as_uint(v);
            if constexpr (kSum) acc[k][q] += v;
          }
        }
        stream_store_sc1(res, out, (uint32_t)(sub * row_bytes) + (uint32_t)c * 16);
      }
    }
  }
  if constexpr (kSum) {
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = lane + kL * k;
      if (c >= chunks) continue;
#pragma unroll
      for (int e = 0; e < E; ++e) atomicAdd(&s_sum[c * E + e], acc[k][e]);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < chunks * E; c += kGeluThreads) unsafeAtomicAdd(colsum + c, s_sum[c]);
  }
}

// Resident workgroups, capped at two per CU (four waves per SIMD): every
// workgroup adds one float atomic per column at its end, so the cap bounds
// those to 2 * CUs * F per launch.
constexpr int kGeluMaxBlocksPerCu = 2;

template <int DT, int CPL, bool kSum, int kL = 64>
int launch_gelu_bwd(const void* dout, const void* h, void* dh, float* colsum, int64_t rows, int chunks,
                    hipStream_t s) {
  auto kern = gelu_bwd_kernel<DT, CPL, kSum, kL>;
  constexpr int kMaxDevices = 64;
  static int cache[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TERRA_ERR_LAUNCH, "cannot query the current device");
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kGeluThreads, 0) != hipSuccess)
      return fail(TERRA_ERR_LAUNCH, "cannot size the GELU backward grid for this device");
    per_cu = per_cu < 1 ? 1 : (per_cu > kGeluMaxBlocksPerCu ? kGeluMaxBlocksPerCu : per_cu);
    cache[dev] = cus * per_cu;
  }
  const int64_t per_block = (int64_t)kGeluWaves * gelu_rows<CPL>() * (64 / kL);
  const int64_t need = (rows + per_block - 1) / per_block;
  const int blocks = need < cache[dev] ? (int)need : cache[dev];
  kern<<<blocks, kGeluThreads, 0, s>>>((const uint8_t*)dout, (const uint8_t*)h, (uint8_t*)dh, colsum, rows, chunks);
  return TERRA_OK;
}

template <int DT, bool kSum>
int dispatch_gelu_bwd(const void* dout, const void* h, void* dh, float* colsum, int64_t rows, int chunks,
                      hipStream_t s) {
  if (chunks <= 32) return launch_gelu_bwd<DT, 1, kSum, 32>(dout, h, dh, colsum, rows, chunks, s);
  if (chunks <= 64) return launch_gelu_bwd<DT, 1, kSum>(dout, h, dh, colsum, rows, chunks, s);
  if (chunks <= 96) return launch_gelu_bwd<DT, 3, kSum, 32>(dout, h, dh, colsum, rows, chunks, s);  // c3: 768 bf16
  if (chunks <= 128) return launch_gelu_bwd<DT, 2, kSum>(dout, h, dh, colsum, rows, chunks, s);
  if (chunks <= 192) return launch_gelu_bwd<DT, 3, kSum>(dout, h, dh, colsum, rows, chunks, s);
  if (chunks <= 256) return launch_gelu_bwd<DT, 4, kSum>(dout, h, dh, colsum, rows, chunks, s);
  if (chunks <= 384) return launch_gelu_bwd<DT, 6, kSum>(dout, h, dh, colsum, rows, chunks, s);
  return launch_gelu_bwd<DT, 8, kSum>(dout, h, dh, colsum, rows, chunks, s);
}

}  // namespace
}  // namespace terra

using namespace terra;

extern "C" int terra_swin_gelu_bwd(const void* dout, const void* h, void* dh, int dtype, int64_t rows,
                                   int features, float* column_sums, void* stream) {
  clear_error();
  if (dout == nullptr || h == nullptr || dh == nullptr) return fail(TERRA_ERR_NULL, "dout, h or dh is NULL");
  if (dtype != TERRA_DTYPE_BF16 && dtype != TERRA_DTYPE_F32)
    return fail(TERRA_ERR_DTYPE, "GELU backward supports bf16 and f32 (got dtype %d)", dtype);
  if (rows < 0 || features <= 0) return fail(TERRA_ERR_SHAPE, "rows must be >= 0 and features > 0");
  const int elt = dtype_size(dtype);
  if (((int64_t)features * elt) % 16 != 0)
    return fail(TERRA_ERR_ALIGN, "GELU backward needs rows of whole 16-byte chunks (features * element size %% 16 == 0)");
  const int chunks = (int)((int64_t)features * elt / 16);
  if (chunks > kGeluMaxChunks)
    return fail(TERRA_ERR_UNSUPPORTED, "GELU backward handles rows of up to %d bytes (got %d features)",
                kGeluMaxChunks * 16, features);
  for (const void* p : {dout, h, (const void*)dh})
    if (((uintptr_t)p & 15u) != 0) return fail(TERRA_ERR_ALIGN, "dout, h and dh must be 16-byte aligned");
  if (((uintptr_t)column_sums & 3u) != 0) return fail(TERRA_ERR_ALIGN, "column_sums must be 4-byte aligned");
  const uintptr_t bytes = (uintptr_t)(rows * (int64_t)chunks * 16);
  for (const void* p : {dout, h}) {
    const uintptr_t a = (uintptr_t)p, d = (uintptr_t)dh;
    if (rows > 0 && a < d + bytes && d < a + bytes) return fail(TERRA_ERR_SHAPE, "dh must not overlap dout or h");
  }
  if (rows * (int64_t)chunks * 16 >= (1ll << 40)) return fail(TERRA_ERR_SHAPE, "tensor too large");
  if (rows == 0) return TERRA_OK;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (dtype == TERRA_DTYPE_BF16)
    rc = column_sums != nullptr ? dispatch_gelu_bwd<TERRA_DTYPE_BF16, true>(dout, h, dh, column_sums, rows, chunks, s)
                                : dispatch_gelu_bwd<TERRA_DTYPE_BF16, false>(dout, h, dh, nullptr, rows, chunks, s);
  else
    rc = column_sums != nullptr ? dispatch_gelu_bwd<TERRA_DTYPE_F32, true>(dout, h, dh, column_sums, rows, chunks, s)
                                : dispatch_gelu_bwd<TERRA_DTYPE_F32, false>(dout, h, dh, nullptr, rows, chunks, s);
  if (rc != TERRA_OK) return rc;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TERRA_ERR_LAUNCH, "terra_swin_gelu_bwd launch failed: %s", hipGetErrorString(e));
  return TERRA_OK;
}
