// sdm_gemm.hip -- sdm_rt_gemm_rows: y = x W^T (+ bias) for a few rows of x, in bfloat16 with float32 sums (the
// projections of a decode step: the mixer's fused wk/wq/wv/wg map and wo, experiments/track4/sdmllm/
// track4_onesdm_models.py:199-207, :247, and TrainedSdm's wq and wo, :443-455, for one token per stream).  A GEMM
// library tiles for many rows; with 64 rows the work is reading W once, so these kernels give every workgroup a
// tile of 32 columns (64 or 32 rows) and split K over its four waves, and the waves' partial tiles are added in a
// fixed order (the result does not depend on timing, and the three kernels give the same bits).
#include "sdm_norm.h"

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
// adds the bias and rounds to bfloat16.  Every kernel below keeps this per-element order (the same 16-deep steps of
// one wave in sequence, then the waves' partial sums added in wave order), so all give the same bits.
__global__ void __launch_bounds__(256) gemm_rows_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                        const bf16_t* __restrict__ w, int64_t ws,
                                                        const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                        int64_t ys, int rows, int k) {
  __shared__ float part[4][32][64];   // [wave][accumulator register][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kGemmCols, m0 = blockIdx.y * kGemmRows;
  const int kq = k / 4;
  const int kb = wave * kq + 8 * (lane >> 5);
  const int r = lane & 31;
  const bf16_t* a0 = x + static_cast<int64_t>(min(m0 + r, rows - 1)) * xs + kb;        // rows past the end: clamped,
  const bf16_t* a1 = x + static_cast<int64_t>(min(m0 + 32 + r, rows - 1)) * xs + kb;   // their sums unused
  const bf16_t* b = w + static_cast<int64_t>(n0 + r) * ws + kb;
  floatx16 acc0 = {}, acc1 = {};
  for (int s = 0; s < kq / 16; ++s) gemm_step(a0 + 16 * s, a1 + 16 * s, b + 16 * s, acc0, acc1);
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

// k = 768, few column tiles (a decode step's layer maps): blocks of TR = 32 or 16 rows x 32 columns, two or four
// times the blocks of the 64-row tiling for the same map, each loading a half or a quarter of the rows of x (the
// launcher takes the smaller tile while the blocks still fit the compute units at once); every operand of a wave
// (12 16-deep steps) is loaded before its first product (one round trip).  Wave w's sums are those of
// gemm_rows_kernel's first accumulator (with TR = 16 the operand rows past the tile repeat its last row, unused).
// FOLD kFoldAdd: x is rms_norm(x + y) (OneSdmLM's residual add and the next layer's input norm in front of its map):
// the block computes its TR rows' sums and norms with the norm kernel's own code (norm_rows: the same bits as
// sdm_rt_add_rms_norm, TR / 8 rows per half-wave, every load first) into LDS, column tile 0's blocks write the sums,
// and the operands come from LDS (rows padded by 16 bytes, so the 32 rows an operand load reads spread over the banks).
// FOLD kFoldEmbed: the same with x's rows gathered from a table by token (OneSdmLM's embedding in front of the first
// layer's norm and map) and no add: column tile 0's blocks write the gathered rows, the residual stream.
constexpr int kRowsK = 768;
constexpr int kRowsSteps = kRowsK / 64;   // 16-deep steps per wave
constexpr int kFoldRow = kRowsK + 8;      // bfloat16 per LDS row of the normed tile

constexpr int kFoldNone = 0, kFoldAdd = 1, kFoldEmbed = 2;

struct RowsFold {   // what runs in front of the map (FOLD): the residual add or the embedding gather, then the norm
  const bf16_t* y;
  int64_t ys;
  const float* w;
  float eps;
  bf16_t* sum;        // the sums (kFoldAdd) or the gathered rows (kFoldEmbed)
  int64_t ss;
  const int64_t* idx; // kFoldEmbed: the token of each row, clamped to [0, vocab)
  int64_t vocab;
};

template <int TR, int FOLD>
__global__ void __launch_bounds__(256) gemm_rows_tile_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                          const bf16_t* __restrict__ w, int64_t ws,
                                                          const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                          int64_t ys, int rows, RowsFold fold) {
  __shared__ float part[4][16][64];   // [wave][accumulator register][lane]
  static_assert(TR == 16 || TR == 32, "tiles of 16 or 32 rows");
  __shared__ __attribute__((aligned(16))) bf16_t s_hx[FOLD != kFoldNone ? TR : 1][FOLD != kFoldNone ? kFoldRow : 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kGemmCols, m0 = blockIdx.y * TR;
  const int kb = wave * (kRowsK / 4) + 8 * (lane >> 5);
  const int r = lane & 31;
  const int ra = min(min(r, TR - 1), rows - 1 - m0);   // the operand row in the tile: past it or past the end clamped
  const bf16_t* b = w + static_cast<int64_t>(n0 + r) * ws + kb;
  uint4 av[kRowsSteps], bv[kRowsSteps];
  if constexpr (FOLD != kFoldNone) {
#pragma unroll
    for (int s = 0; s < kRowsSteps; ++s) bv[s] = *reinterpret_cast<const uint4*>(b + 16 * s);
    constexpr int R = TR / 8;   // rows 8 j + 2 wave + lane / 32 of the tile, j < R, for half-wave (wave, lane / 32)
    const bf16_t* xr[R];
    const bf16_t* yr[R];
    bf16_t* sr[R];
    bf16_t* dr[R];
    bool live[R], keep[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int i = 8 * j + 2 * wave + (lane >> 5);
      live[j] = m0 + i < rows;
      keep[j] = live[j] && blockIdx.x == 0;
      const int64_t rr = live[j] ? m0 + i : m0;   // rows past the end: an in-bounds stand-in, nothing written
      if constexpr (FOLD == kFoldEmbed) {
        const int64_t t = min(max(fold.idx[rr], static_cast<int64_t>(0)), fold.vocab - 1);
        xr[j] = x + t * xs;
        yr[j] = x;   // unused
      } else {
        xr[j] = x + rr * xs;
        yr[j] = fold.y + rr * fold.ys;
      }
      sr[j] = fold.sum + rr * fold.ss;
      dr[j] = &s_hx[i][0];
    }
    norm_rows<bf16_t, bf16_t, FOLD == kFoldAdd, kRowsK / 256, R>(xr, yr, sr, dr, fold.w, kRowsK, fold.eps, lane, live,
                                                                 keep);
    __syncthreads();
    const bf16_t* a = &s_hx[ra][kb];
#pragma unroll
    for (int s = 0; s < kRowsSteps; ++s) av[s] = *reinterpret_cast<const uint4*>(a + 16 * s);
  } else {
    const bf16_t* a = x + static_cast<int64_t>(m0 + ra) * xs + kb;
#pragma unroll
    for (int s = 0; s < kRowsSteps; ++s) {
      bv[s] = *reinterpret_cast<const uint4*>(b + 16 * s);
      av[s] = *reinterpret_cast<const uint4*>(a + 16 * s);
    }
  }
  __builtin_amdgcn_sched_barrier(0);   // keep the scheduler from moving loads below the products
  floatx16 acc = {};
#pragma unroll
  for (int s = 0; s < kRowsSteps; ++s)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[s]), __builtin_bit_cast(bf16x8, bv[s]),
                                                  acc, 0, 0, 0);
#pragma unroll
  for (int q = 0; q < 16; ++q) part[wave][q][lane] = acc[q];
  __syncthreads();
  const int n = n0 + r;
  const float bb = bias ? to_f32(bias[n]) : 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {   // this thread finishes registers 4 wave .. 4 wave + 3 of lane `lane`
    const int reg = 4 * wave + q;
    const int m = m0 + 8 * (reg >> 2) + 4 * (lane >> 5) + (reg & 3);
    float v = part[0][reg][lane];
    v += part[1][reg][lane];
    v += part[2][reg][lane];
    v += part[3][reg][lane];
    if (m < rows && m - m0 < TR)
      reinterpret_cast<uint16_t*>(y)[static_cast<int64_t>(m) * ys + n] = static_cast<uint16_t>(pack_bf16(v + bb, 0.f));
  }
}

// the row tile of a few-rows map: 16 rows while the blocks fit the compute units at once, else 32
inline int map_tile_rows(int ntiles, int64_t rows) { return static_cast<int64_t>(ntiles) * ((rows + 15) / 16) <= 256 ? 16 : 32; }

// k = 768, many column tiles (the tied head over the vocabulary): a block per 64-row tile and 256 / (row tiles)
// column positions; its waves load their x operands once and walk the column tiles blockIdx.x, blockIdx.x +
// gridDim.x, ..., loading the next tile's weights while the current tile's partial sums meet in LDS.  Each tile's
// sums are gemm_rows_kernel's.
__global__ void __launch_bounds__(256) gemm_rows_wide_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                             const bf16_t* __restrict__ w, int64_t ws,
                                                             const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                             int64_t ys, int rows, int ntiles) {
  __shared__ float part[4][32][64];   // [wave][accumulator register][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * kGemmRows;
  const int kb = wave * (kRowsK / 4) + 8 * (lane >> 5);
  const int r = lane & 31;
  const bf16_t* a0 = x + static_cast<int64_t>(min(m0 + r, rows - 1)) * xs + kb;        // rows past the end: clamped
  const bf16_t* a1 = x + static_cast<int64_t>(min(m0 + 32 + r, rows - 1)) * xs + kb;
  uint4 x0[kRowsSteps], x1[kRowsSteps], wv[kRowsSteps];
  int ct = blockIdx.x;   // < ntiles: the grid has at most ntiles columns
#pragma unroll
  for (int s = 0; s < kRowsSteps; ++s) {
    wv[s] = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(ct * kGemmCols + r) * ws + kb + 16 * s);
    x0[s] = *reinterpret_cast<const uint4*>(a0 + 16 * s);
    x1[s] = *reinterpret_cast<const uint4*>(a1 + 16 * s);
  }
  for (; ct < ntiles; ct += gridDim.x) {
    floatx16 acc0 = {}, acc1 = {};
#pragma unroll
    for (int s = 0; s < kRowsSteps; ++s) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x0[s]), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x1[s]), __builtin_bit_cast(bf16x8, wv[s]),
                                                     acc1, 0, 0, 0);
    }
    const int cn = min(ct + static_cast<int>(gridDim.x), ntiles - 1);   // the last tile loads itself again
#pragma unroll
    for (int s = 0; s < kRowsSteps; ++s)
      wv[s] = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(cn * kGemmCols + r) * ws + kb + 16 * s);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      part[wave][q][lane] = acc0[q];
      part[wave][16 + q][lane] = acc1[q];
    }
    __syncthreads();
    const int n = ct * kGemmCols + r;
    const float bb = bias ? to_f32(bias[n]) : 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int reg = 8 * wave + q;
      const int rr = reg & 15;
      const int m = m0 + 32 * (reg >> 4) + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
      float v = part[0][reg][lane];
      v += part[1][reg][lane];
      v += part[2][reg][lane];
      v += part[3][reg][lane];
      if (m < rows) reinterpret_cast<uint16_t*>(y)[static_cast<int64_t>(m) * ys + n] = static_cast<uint16_t>(pack_bf16(v + bb, 0.f));
    }
    __syncthreads();   // part is written again by the next tile
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
  const bf16_t* xb = static_cast<const bf16_t*>(x);
  const bf16_t* wb = static_cast<const bf16_t*>(w);
  const bf16_t* bb = static_cast<const bf16_t*>(bias);
  bf16_t* yb = static_cast<bf16_t*>(y);
  const int ntiles = n / kGemmCols;
  const int row_tiles = static_cast<int>((rows + kGemmRows - 1) / kGemmRows);
  if (k == kRowsK && static_cast<int64_t>(ntiles) * row_tiles <= 256) {
    // a decode step's layer maps: 16- or 32-row tiles
    const int tr = map_tile_rows(ntiles, rows);
    const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>((rows + tr - 1) / tr));
    if (tr == 16)
      hipLaunchKernelGGL((gemm_rows_tile_kernel<16, kFoldNone>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride,
                         bb, yb, y_row_stride, static_cast<int>(rows), RowsFold{});
    else
      hipLaunchKernelGGL((gemm_rows_tile_kernel<32, kFoldNone>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride,
                         bb, yb, y_row_stride, static_cast<int>(rows), RowsFold{});
  } else if (k == kRowsK && row_tiles <= 256) {
    // wide maps: about one block per compute unit, each walking its column tiles
    const int cols = min(ntiles, max(1, 256 / row_tiles));
    hipLaunchKernelGGL(gemm_rows_wide_kernel, dim3(static_cast<unsigned>(cols), static_cast<unsigned>(row_tiles)),
                       dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb, yb, y_row_stride, static_cast<int>(rows),
                       ntiles);
  } else {
    hipLaunchKernelGGL(gemm_rows_kernel, dim3(static_cast<unsigned>(ntiles), static_cast<unsigned>(row_tiles)),
                       dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb, yb, y_row_stride, static_cast<int>(rows),
                       k);
  }
  return check_launch("gemm_rows");
}

int sdm_rt_gemm_rows_residual(const void* x, int64_t x_row_stride, const void* y, int64_t y_row_stride,
                              const float* norm_w, float norm_eps, void* sum_out, int64_t sum_row_stride,
                              const void* w, int64_t w_row_stride, const void* bias, void* out,
                              int64_t out_row_stride, int64_t rows, int32_t n, int32_t k, void* stream) {
  g_err[0] = 0;
  if (rows < 0 || n < 0 || k < 0) return set_err(SDM_RT_EINVAL, "rows, n and k must be >= 0");
  if (k != kRowsK) return set_err(SDM_RT_EUNSUPPORTED, "gemm_rows_residual: k = %d, must be %d", k, kRowsK);
  if (n == 0 || n % kGemmCols != 0)
    return set_err(SDM_RT_EUNSUPPORTED, "gemm_rows_residual: n = %d must be a positive multiple of %d", n, kGemmCols);
  if (rows == 0) return SDM_RT_OK;
  const int ntiles = n / kGemmCols;
  if (static_cast<int64_t>(ntiles) * ((rows + kGemmRows - 1) / kGemmRows) > 256)
    return set_err(SDM_RT_EUNSUPPORTED,
                   "gemm_rows_residual: %lld rows x %d columns: more than 256 tiles of 64 x 32 (call "
                   "sdm_rt_add_rms_norm, then sdm_rt_gemm_rows)", (long long)rows, n);
  if (!x || !y || !norm_w || !sum_out || !w || !out)
    return set_err(SDM_RT_EINVAL, "x, y, norm_w, sum_out, w and out must not be NULL");
  if (x_row_stride < k || y_row_stride < k || sum_row_stride < k || w_row_stride < k || out_row_stride < n)
    return set_err(SDM_RT_EINVAL, "row strides too small");
  auto al16 = [](const void* p, int64_t stride) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (stride * 2) % 16 == 0;
  };
  if (!al16(x, x_row_stride) || !al16(y, y_row_stride) || !al16(sum_out, sum_row_stride) || !al16(w, w_row_stride) ||
      reinterpret_cast<uintptr_t>(norm_w) % 16)
    return set_err(SDM_RT_EINVAL, "x, y, sum_out and w rows and norm_w must be 16-byte aligned");
  // every column tile's blocks read x and y while column tile 0's write the sums, and all write out
  if (sum_out == x || sum_out == y || out == x || out == y || out == sum_out)
    return set_err(SDM_RT_EINVAL, "gemm_rows_residual: sum_out and out must not alias x, y or each other");
  const RowsFold fold{static_cast<const bf16_t*>(y), y_row_stride, norm_w, norm_eps, static_cast<bf16_t*>(sum_out),
                      sum_row_stride, nullptr, 0};
  const int tr = map_tile_rows(ntiles, rows);
  const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>((rows + tr - 1) / tr));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t* xb = static_cast<const bf16_t*>(x);
  const bf16_t* wb = static_cast<const bf16_t*>(w);
  const bf16_t* bb = static_cast<const bf16_t*>(bias);
  bf16_t* ob = static_cast<bf16_t*>(out);
  if (tr == 16)
    hipLaunchKernelGGL((gemm_rows_tile_kernel<16, kFoldAdd>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb,
                       ob, out_row_stride, static_cast<int>(rows), fold);
  else
    hipLaunchKernelGGL((gemm_rows_tile_kernel<32, kFoldAdd>), grid, dim3(256), 0, st, xb, x_row_stride, wb, w_row_stride, bb,
                       ob, out_row_stride, static_cast<int>(rows), fold);
  return check_launch("gemm_rows_residual");
}

int sdm_rt_gemm_rows_embed(const int64_t* tokens, const void* table, int64_t table_row_stride, int64_t vocab,
                           const float* norm_w, float norm_eps, void* x_out, int64_t x_row_stride, const void* w,
                           int64_t w_row_stride, const void* bias, void* out, int64_t out_row_stride, int64_t rows,
                           int32_t n, int32_t k, void* stream) {
  g_err[0] = 0;
  if (rows < 0 || n < 0 || k < 0) return set_err(SDM_RT_EINVAL, "rows, n and k must be >= 0");
  if (k != kRowsK) return set_err(SDM_RT_EUNSUPPORTED, "gemm_rows_embed: k = %d, must be %d", k, kRowsK);
  if (n == 0 || n % kGemmCols != 0)
    return set_err(SDM_RT_EUNSUPPORTED, "gemm_rows_embed: n = %d must be a positive multiple of %d", n, kGemmCols);
  if (vocab < 1) return set_err(SDM_RT_EINVAL, "gemm_rows_embed: vocab must be >= 1");
  if (rows == 0) return SDM_RT_OK;
  const int ntiles = n / kGemmCols;
  if (static_cast<int64_t>(ntiles) * ((rows + kGemmRows - 1) / kGemmRows) > 256)
    return set_err(SDM_RT_EUNSUPPORTED,
                   "gemm_rows_embed: %lld rows x %d columns: more than 256 tiles of 64 x 32 (gather, call "
                   "sdm_rt_rms_norm, then sdm_rt_gemm_rows)", (long long)rows, n);
  if (!tokens || !table || !norm_w || !x_out || !w || !out)
    return set_err(SDM_RT_EINVAL, "tokens, table, norm_w, x_out, w and out must not be NULL");
  if (table_row_stride < k || x_row_stride < k || w_row_stride < k || out_row_stride < n)
    return set_err(SDM_RT_EINVAL, "row strides too small");
  auto al16 = [](const void* p, int64_t stride) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (stride * 2) % 16 == 0;
  };
  if (!al16(table, table_row_stride) || !al16(x_out, x_row_stride) || !al16(w, w_row_stride) ||
      reinterpret_cast<uintptr_t>(norm_w) % 16)
    return set_err(SDM_RT_EINVAL, "table, x_out and w rows and norm_w must be 16-byte aligned");
  if (out == x_out || x_out == table || out == table)
    return set_err(SDM_RT_EINVAL, "gemm_rows_embed: x_out and out must not alias the table or each other");
  const RowsFold fold{nullptr, 0, norm_w, norm_eps, static_cast<bf16_t*>(x_out), x_row_stride, tokens, vocab};
  const int tr = map_tile_rows(ntiles, rows);
  const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>((rows + tr - 1) / tr));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t* tb = static_cast<const bf16_t*>(table);
  const bf16_t* wb = static_cast<const bf16_t*>(w);
  const bf16_t* bb = static_cast<const bf16_t*>(bias);
  bf16_t* ob = static_cast<bf16_t*>(out);
  if (tr == 16)
    hipLaunchKernelGGL((gemm_rows_tile_kernel<16, kFoldEmbed>), grid, dim3(256), 0, st, tb, table_row_stride, wb,
                       w_row_stride, bb, ob, out_row_stride, static_cast<int>(rows), fold);
  else
    hipLaunchKernelGGL((gemm_rows_tile_kernel<32, kFoldEmbed>), grid, dim3(256), 0, st, tb, table_row_stride, wb,
                       w_row_stride, bb, ob, out_row_stride, static_cast<int>(rows), fold);
  return check_launch("gemm_rows_embed");
}

}  // extern "C"
