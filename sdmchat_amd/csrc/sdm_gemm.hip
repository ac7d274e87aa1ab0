// sdm_gemm.hip -- sdm_rt_gemm_rows: y = x W^T (+ bias) for a few rows of x, in bfloat16 with float32 sums (the
// projections of a decode step: the mixer's fused wk/wq/wv/wg map and wo, experiments/track4/sdmllm/
// track4_onesdm_models.py:199-207, :247, and TrainedSdm's wq and wo, :443-455, for one token per stream).  A GEMM
// library tiles for many rows; with 64 rows the work is reading W once, so this kernel gives every workgroup a
// 64-row x 32-column tile and splits K over its four waves, and the waves' partial tiles are added in a fixed order
// (the result does not depend on timing).
#include "sdm_common.h"

namespace sdmrt {

constexpr int kGemmRows = 64;   // rows per workgroup tile
constexpr int kGemmCols = 32;   // columns per workgroup tile

// one 16-deep step of a wave: rows m0 .. m0 + 63 (two 32 x 32 accumulators) times columns n0 .. n0 + 31
__device__ __forceinline__ void gemm_step(const bf16_t* a0, const bf16_t* a1, const bf16_t* b, floatx16& acc0,
                                          floatx16& acc1) {
  const uint4 x0 = *reinterpret_cast<const uint4*>(a0);
  const uint4 x1 = *reinterpret_cast<const uint4*>(a1);
  const uint4 w = *reinterpret_cast<const uint4*>(b);
  acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x0), __builtin_bit_cast(bf16x8, w), acc0,
                                                 0, 0, 0);
  acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x1), __builtin_bit_cast(bf16x8, w), acc1,
                                                 0, 0, 0);
}

// Block (32-column tile, 64-row tile), 256 threads.  Wave w sums k in [w K/4, (w + 1) K/4): lane l feeds row
// m0 + l % 32 (and m0 + 32 + l % 32) of x and row n0 + l % 32 of W, k-elements 8 (l / 32) .. + 7 of each 16-deep
// step; the accumulators hold column n0 + l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 (r < 16) of each 32-row half.
// The four partial tiles meet in LDS; thread (g, l) adds registers 8 g .. 8 g + 7 of lane l over the waves in order,
// adds the bias and rounds to bfloat16.  STEPS: 16-deep steps per wave (K / 64) when unrolled, 0 for a loop.
// Rows of the x tile staged in LDS (STAGE: k = 768): 64 rows of 768 bfloat16 plus 16 bytes, so that the 32 rows a
// matrix-core operand load reads fall on different banks
constexpr int kStageK = 768;
constexpr int kStageRow = kStageK * 2 + 16;   // bytes

template <int STEPS, bool STAGE>
__global__ void __launch_bounds__(256) gemm_rows_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                        const bf16_t* __restrict__ w, int64_t ws,
                                                        const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                        int64_t ys, int rows, int k) {
  __shared__ float part[4][32][64];   // [wave][accumulator register][lane]
  extern __shared__ __attribute__((aligned(16))) unsigned char xs_lds[];   // STAGE: the x tile [64][kStageRow]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kGemmCols, m0 = blockIdx.y * kGemmRows;
  const int kq = k / 4;
  const int kb = wave * kq + 8 * (lane >> 5);
  const int r = lane & 31;
  const bf16_t* a0 = x + static_cast<int64_t>(min(m0 + r, rows - 1)) * xs + kb;        // rows past the end: clamped,
  const bf16_t* a1 = x + static_cast<int64_t>(min(m0 + 32 + r, rows - 1)) * xs + kb;   // their sums unused
  const bf16_t* b = w + static_cast<int64_t>(n0 + r) * ws + kb;
  floatx16 acc0 = {}, acc1 = {};
  if constexpr (STAGE) {
    // The x tile is the same for every column tile, and the operand layout (lane l: row l % 32) makes each direct
    // load touch 32 rows; staged, each load instruction reads 1 KB of consecutive row bytes (thread t: the 16-byte
    // pieces t, t + 256, ...), and the operands come from LDS.  The weights' loads are issued first.  (Staging the
    // weight tile the same way gains under 0.1 us.)
    static_assert(STEPS == kStageK / 64, "the staged tile holds k = 768");
    uint4 wv[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) wv[s] = *reinterpret_cast<const uint4*>(b + 16 * s);
    constexpr int kPieces = kGemmRows * kStageK / 8;   // 16-byte pieces of the tile: 6,144
    uint4 xv[kPieces / 256];
#pragma unroll
    for (int j = 0; j < kPieces / 256; ++j) {
      const int i = threadIdx.x + 256 * j;
      const int row = i / (kStageK / 8), col8 = i - row * (kStageK / 8);
      xv[j] = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(min(m0 + row, rows - 1)) * xs + 8 * col8);
    }
#pragma unroll
    for (int j = 0; j < kPieces / 256; ++j) {
      const int i = threadIdx.x + 256 * j;
      const int row = i / (kStageK / 8), col8 = i - row * (kStageK / 8);
      *reinterpret_cast<uint4*>(xs_lds + row * kStageRow + 16 * col8) = xv[j];
    }
    __syncthreads();
    const unsigned char* l0 = xs_lds + r * kStageRow + 2 * kb;
    const unsigned char* l1 = xs_lds + (32 + r) * kStageRow + 2 * kb;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const uint4 x0 = *reinterpret_cast<const uint4*>(l0 + 32 * s);
      const uint4 x1 = *reinterpret_cast<const uint4*>(l1 + 32 * s);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x0), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x1), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc1, 0, 0, 0);
    }
  } else if constexpr (STEPS > 0) {   // every operand of the wave loaded before the first product: one round trip
    uint4 x0[STEPS], x1[STEPS], wv[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      wv[s] = *reinterpret_cast<const uint4*>(b + 16 * s);
      x0[s] = *reinterpret_cast<const uint4*>(a0 + 16 * s);
      x1[s] = *reinterpret_cast<const uint4*>(a1 + 16 * s);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the scheduler from moving loads below the products
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x0[s]), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x1[s]), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc1, 0, 0, 0);
    }
  } else {
    for (int s = 0; s < kq / 16; ++s) gemm_step(a0 + 16 * s, a1 + 16 * s, b + 16 * s, acc0, acc1);
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    part[wave][q][lane] = acc0[q];
    part[wave][16 + q][lane] = acc1[q];
  }
  __syncthreads();
  const int g = wave;   // this thread finishes registers 8 g .. 8 g + 7 of lane `lane`
  const int n = n0 + r;
  const float bv = bias ? to_f32(bias[n]) : 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int reg = 8 * g + q;                                   // 0..15: rows 0..31, 16..31: rows 32..63
    const int rr = reg & 15;
    const int m = m0 + 32 * (reg >> 4) + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
    float v = part[0][reg][lane];
    v += part[1][reg][lane];
    v += part[2][reg][lane];
    v += part[3][reg][lane];
    if (m < rows) reinterpret_cast<uint16_t*>(y)[static_cast<int64_t>(m) * ys + n] = static_cast<uint16_t>(pack_bf16(v + bv, 0.f));
  }
}

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

int sdm_rt_gemm_rows(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, const void* bias,
                     void* y, int64_t y_row_stride, int64_t rows, int32_t n, int32_t k, void* stream) {
  g_err[0] = 0;
  if (rows < 0 || n < 0 || k < 0) return set_err(SDM_RT_EINVAL, "rows, n and k must be >= 0");
  if (n % kGemmCols != 0) return set_err(SDM_RT_EUNSUPPORTED, "n = %d must be a multiple of %d", n, kGemmCols);
  if (k % 64 != 0 || k == 0) return set_err(SDM_RT_EUNSUPPORTED, "k = %d must be a positive multiple of 64", k);
  if (rows > (1 << 20)) return set_err(SDM_RT_EUNSUPPORTED, "rows = %lld: too many for this kernel", (long long)rows);
  if (rows == 0 || n == 0) return SDM_RT_OK;
  if (!x || !w || !y) return set_err(SDM_RT_EINVAL, "x, w and y must not be NULL");
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n) return set_err(SDM_RT_EINVAL, "row strides too small");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 || (x_row_stride * 2) % 16 ||
      (w_row_stride * 2) % 16)
    return set_err(SDM_RT_EINVAL, "x and w rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(n / kGemmCols), static_cast<unsigned>((rows + kGemmRows - 1) / kGemmRows));
  const bf16_t* xb = static_cast<const bf16_t*>(x);
  const bf16_t* wb = static_cast<const bf16_t*>(w);
  const bf16_t* bb = static_cast<const bf16_t*>(bias);
  bf16_t* yb = static_cast<bf16_t*>(y);
  // k = 768 with few column tiles (the maps of a decode step's layers): the x tile staged in LDS; the wide maps (the
  // tied head) keep the direct loads, with several workgroups per compute unit
  if (k == kStageK && grid.x * grid.y <= 256) {
    constexpr int kStageBytes = kGemmRows * kStageRow;   // 99,328
    static const bool lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_rows_kernel<12, true>),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   kStageBytes) == hipSuccess;
    if (!lds_ok) return set_err(SDM_RT_ELAUNCH, "gemm_rows: cannot enable %d bytes of LDS", kStageBytes);
    hipLaunchKernelGGL((gemm_rows_kernel<12, true>), grid, dim3(256), kStageBytes, st, xb, x_row_stride, wb,
                       w_row_stride, bb, yb, y_row_stride, static_cast<int>(rows), k);
  } else if (k == kStageK) {
    hipLaunchKernelGGL((gemm_rows_kernel<12, false>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb,
                       yb, y_row_stride, static_cast<int>(rows), k);
  } else {
    hipLaunchKernelGGL((gemm_rows_kernel<0, false>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb,
                       yb, y_row_stride, static_cast<int>(rows), k);
  }
  return check_launch("gemm_rows");
}

}  // extern "C"
