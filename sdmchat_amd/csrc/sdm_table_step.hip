// sdm_table_step.hip -- sdm_rt_table_step: TrainedSdm's read for a few tokens (a decode step) in one launch: the
// query map q = hx Wq^T, the product-key addressing of q and the weighted read of the picked table rows
// (TrainedSdm.forward, experiments/track4/sdmllm/track4_onesdm_models.py:438-455: F.linear, pk_address :134-148 with
// the softmax weights, embedding_bag).  Each stage is computed as its own entry point computes it (the query map as
// sdm_rt_gemm_rows sums it, the addressing as sdm_rt_address, the read as sdm_rt_table_read), so the three calls and
// this one give the same bits; between the stages the data stay in LDS and registers.
#include "sdm_norm.h"

namespace sdmrt {

struct TableStepArgs {
  AddrGeom g;
  const bf16_t* hx;        // [N][d] normed inputs
  int64_t hx_stride;
  int d;
  const bf16_t* wq;        // [H * d_a][d]
  int64_t wq_stride;
  const bf16_t* values;    // [H][M][dh]
  int M, dh, pitch, B, T;
  bf16_t* q_out;           // [N][H * d_a] or nullptr
  int64_t q_stride;
  int32_t* slot_out;       // [B][H][T][pitch]
  float* w_out;            // same layout or nullptr
  float* s_out;            // same layout or nullptr
  bf16_t* r_out;           // [N][H * dh]
  int64_t r_stride;
  // the residual add and the input norm folded in front (FOLD): hx = rms_norm(rx + ry), rsum = rx + ry
  const bf16_t* rx;        // [N][d]
  int64_t rx_stride;
  const bf16_t* ry;        // [N][d]
  int64_t ry_stride;
  bf16_t* rsum;            // [N][d], written by head 0's blocks
  int64_t rsum_stride;
  const float* rw;         // [d] the norm's weight
  float reps;
  bf16_t* hx_out;          // [N][d] the normed rows (head 0's blocks), or nullptr
  int64_t hx_out_stride;
};

constexpr int kTableStepTokens = 256;  // at most this many tokens (sdm_rt_gemm_rows' row range, whose sums it repeats)
constexpr int kStepK = 12;             // 16-deep steps per wave of the query map when d = 768
constexpr int kFoldD = 768;            // the layer width of the folded residual add and norm (FOLD)
constexpr int kMaxHeadDim = 1024;      // the read's 16-byte pieces of a head's row: at most 32 per wave

// Block (token, head), 4 waves.
//  1. the head's d_a query columns of the token's row: wave w sums k in [w d/4, (w + 1) d/4) on the matrix cores
//     with the operand layout of gemm_rows_kernel (row 0 of a 32-row tile: accumulator register 0 of lanes 0..31),
//     the four partial sums are added in wave order and rounded to bfloat16 once;
//  2. wave q < 2 NS / 32 scores half q / (NS / 32) of the query against sub-key tile q % (NS / 32) (half_scores,
//     reading the query from LDS), and wave 0 selects the picks across its lanes (select_lanes);
//  3. the picks pass through LDS; wave w reads its quarter of the 16-byte pieces of the picked rows, every pick's
//     piece in flight at once, and sums them in pick order over the pitch (pads: slot 0, weight 0) in float32, as the
//     table read does.  (A block per token spreads the read over as many compute units as there are tokens.)
// FOLD (d = 768): before 1., the first half of wave 0 computes the token's residual sum rx + ry and its norm with the
// norm kernel's own code (norm_row: the same bits as sdm_rt_add_rms_norm), writes the sum (head 0's block only) and
// leaves the normed row in LDS, from which the query map reads it.
template <int HALF, int CAP, int MODE, bool FOLD>
__global__ void __launch_bounds__(256) table_step_kernel(TableStepArgs a) {
  constexpr int NS = MODE >= 3 ? 64 : 32;
  constexpr int NT = NS / 32;
  constexpr bool FULL = MODE == 2 || MODE == 4;
  constexpr int DA = 2 * HALF;   // query columns of a head
  constexpr int NCT = DA / 32;   // 32-column tiles of the query map per head
  static_assert(DA % 32 == 0, "the query map runs on 32-column tiles");
  __shared__ float s_part[4][NCT][32];   // [wave][column tile][column]
  __shared__ __attribute__((aligned(16))) uint16_t s_q[DA];
  __shared__ float s_sc[2][NS];
  __shared__ float s_inv[2];
  __shared__ int s_slot[CAP];
  __shared__ float s_w[CAP];
  __shared__ __attribute__((aligned(16))) bf16_t s_hx[FOLD ? kFoldD : 8];
  const int h = blockIdx.y;
  const int64_t n = blockIdx.x;   // the token
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // the loads that do not depend on the token's row, issued first: the wave's query-map weights (FOLD: d = 768)
  // and its sub-key piece for the scoring
  uint4 wpre[FOLD ? NCT : 1][kStepK];
  if constexpr (FOLD) {
    const int kb = wave * (kFoldD / 4) + 8 * (lane >> 5);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const bf16_t* wr = a.wq + static_cast<int64_t>(h * DA + 32 * ct + (lane & 31)) * a.wq_stride + kb;
#pragma unroll
      for (int s = 0; s < kStepK; ++s) wpre[ct][s] = *reinterpret_cast<const uint4*>(wr + 16 * s);
    }
  }
  SubKeyPiece<HALF> kpre;
  if (wave < 2 * NT) load_sub_key_piece<HALF>(a.g, h, wave / NT, 32 * (wave % NT), kpre);
  if constexpr (FOLD) {
    if (wave == 0) {   // both halves take part in the norm's sums; the second passes the same row, not live
      const bool live = lane < 32;
      norm_row<bf16_t, bf16_t, true, kFoldD / 256>(a.rx + n * a.rx_stride, a.ry + n * a.ry_stride,
                                                   a.rsum + n * a.rsum_stride, s_hx, a.rw, kFoldD, a.reps, lane, live,
                                                   live && h == 0);
      if (a.hx_out && live && h == 0) {   // the lane's own pieces, as norm_row stored them
#pragma unroll
        for (int k = 0; k < kFoldD / 256; ++k) {
          const int c = 8 * (lane + 32 * k);
          *reinterpret_cast<uint4*>(a.hx_out + n * a.hx_out_stride + c) = *reinterpret_cast<const uint4*>(&s_hx[c]);
        }
      }
    }
    __syncthreads();
  }
  {
    const int kq = a.d / 4;
    const int kb = wave * kq + 8 * (lane >> 5);
    // every row of the tile is the token's (the rows past the first are unused); FOLD: the normed row in LDS
    const bf16_t* xr = FOLD ? s_hx + kb : a.hx + n * a.hx_stride + kb;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const bf16_t* wr = a.wq + static_cast<int64_t>(h * DA + 32 * ct + (lane & 31)) * a.wq_stride + kb;
      floatx16 acc = {};
      if (kq == 16 * kStepK) {   // d = 768: every operand of the wave loaded before the first product
        uint4 xv[kStepK], wv[kStepK];
#pragma unroll
        for (int s = 0; s < kStepK; ++s) {
          xv[s] = *reinterpret_cast<const uint4*>(xr + 16 * s);
          wv[s] = FOLD ? wpre[ct][s] : *reinterpret_cast<const uint4*>(wr + 16 * s);
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the scheduler from moving loads below the products
#pragma unroll
        for (int s = 0; s < kStepK; ++s)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv[s]),
                                                        __builtin_bit_cast(bf16x8, wv[s]), acc, 0, 0, 0);
      } else {
        for (int s = 0; s < kq / 16; ++s) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xr + 16 * s);
          const uint4 wv = *reinterpret_cast<const uint4*>(wr + 16 * s);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv), __builtin_bit_cast(bf16x8, wv),
                                                        acc, 0, 0, 0);
        }
      }
      if (lane < 32) s_part[wave][ct][lane] = acc[0];   // row 0, column lane
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < DA; c += 256) {
    const int ct = c >> 5, cl = c & 31;
    float v = s_part[0][ct][cl];
    v += s_part[1][ct][cl];
    v += s_part[2][ct][cl];
    v += s_part[3][ct][cl];
    const uint16_t bits = static_cast<uint16_t>(pack_bf16(v + 0.f, 0.f));   // as gemm_rows adds a zero bias
    s_q[c] = bits;
    if (a.q_out) reinterpret_cast<uint16_t*>(a.q_out)[n * a.q_stride + h * DA + c] = bits;
  }
  __syncthreads();
  if (wave < 2 * NT) {
    const int hf = wave / NT, tile = wave % NT;
    floatx16 acc[2];
    float inv[2];
    half_scores_bf16_with<HALF, FULL>(a.g, h, hf, reinterpret_cast<const bf16_t*>(s_q), DA, 1, acc, inv, 0, kpre);
    // lane l < 32 of the address row 0: sub-keys 32 tile + 8 (r / 4) + 4 (l / 32) + r % 4
    if ((lane & 31) == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s_sc[hf][32 * tile + 8 * (r / 4) + 4 * (lane >> 5) + (r & 3)] = acc[0][r];
      if (lane == 0 && tile == 0) s_inv[hf] = inv[0];
    }
  }
  __syncthreads();
  if (wave == 0) {
    int slot;
    float w, sc;
    select_lanes<CAP, FULL, NS>(a.g, a.g.log_scale[h], &s_sc[0][0], s_inv, 1.f, slot, w, sc);
    if (lane < CAP) {   // lanes past kk: slot 0, weight 0
      s_slot[lane] = slot;
      s_w[lane] = w;
    }
    const int b = static_cast<int>(n / a.T);
    const int t = static_cast<int>(n - static_cast<int64_t>(b) * a.T);
    const int64_t base = ((static_cast<int64_t>(b) * a.g.H + h) * a.T + t) * a.pitch;
    if (lane < CAP && lane < a.pitch) {
      const bool live = lane < a.g.kk;
      a.slot_out[base + lane] = live ? slot : -1;
      if (a.w_out) a.w_out[base + lane] = w;
      if (a.s_out) a.s_out[base + lane] = sc;
    }
  }
  __syncthreads();
  const int pieces = a.dh / 8;
  const int per_wave = (pieces + 3) / 4;
  const int pc = wave * per_wave + lane;
  if (lane >= per_wave || pc >= pieces) return;
  const bf16_t* tab = a.values + static_cast<int64_t>(h) * a.M * a.dh + 8 * pc;
  uint4 raw[CAP];
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    raw[j] = j < a.pitch ? *reinterpret_cast<const uint4*>(tab + static_cast<int64_t>(s_slot[j]) * a.dh)
                         : make_uint4(0u, 0u, 0u, 0u);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    if (j < a.pitch) {
      const float wj = s_w[j];
      const uint32_t wd[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] = fmaf(wj, __uint_as_float(wd[q] << 16), acc[2 * q]);
        acc[2 * q + 1] = fmaf(wj, __uint_as_float(wd[q] & 0xffff0000u), acc[2 * q + 1]);
      }
    }
  }
  store_vals<8, bf16_t>(a.r_out + n * a.r_stride + static_cast<int64_t>(h) * a.dh + 8 * pc, acc);
}

template <int HALF>
struct TableStepLaunch {
  template <int CAP, int MODE>
  static int go(const Plan& p, const TableStepArgs& a, hipStream_t st) {
    const int64_t N = static_cast<int64_t>(p.B) * p.T;
    const dim3 grid(static_cast<unsigned>(N), p.H);
    if (a.rx)
      hipLaunchKernelGGL((table_step_kernel<HALF, CAP, MODE, true>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((table_step_kernel<HALF, CAP, MODE, false>), grid, dim3(256), 0, st, a);
    return check_launch("table_step");
  }
  // the addressing mode of sdm_rt_address for this shape (AddressLaunch::run)
  static int run(const Plan& p, const TableStepArgs& a, hipStream_t st) {
    if (use_mf(p)) {
      if (full_grid(p)) return go<8, 2>(p, a, st);
      return p.cap == 8 ? go<8, 1>(p, a, st) : go<16, 1>(p, a, st);
    }
    if (use_mf64(p)) {
      const bool full = p.n_sub == 64 && p.c1 == p.cap && p.kk == p.cap;
      if (p.cap == 8) return full ? go<8, 4>(p, a, st) : go<8, 3>(p, a, st);
      return full ? go<16, 4>(p, a, st) : go<16, 3>(p, a, st);
    }
    return set_err(SDM_RT_EUNSUPPORTED, "table_step: n_sub = %d: at most 64 sub-keys per half", p.n_sub);
  }
};

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

namespace {

struct Residual {   // the folded residual add and norm of sdm_rt_table_step_residual
  const void* x;
  int64_t x_stride;
  const void* y;
  int64_t y_stride;
  const float* w;
  float eps;
  void* sum;
  int64_t sum_stride;
  void* hx;
  int64_t hx_stride;
};

int table_step_impl(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* hx, int64_t hx_row_stride,
                    int32_t d, const void* wq, int64_t wq_row_stride, const void* values, void* q_out,
                    int64_t q_row_stride, int32_t* slot_out, float* score_out, float* weight_out, void* out,
                    int64_t out_row_stride, const Residual* res, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if ((rc = check_params(params, false, false))) return rc;
  const int64_t N = static_cast<int64_t>(p.B) * p.T;
  if (N == 0) return SDM_RT_OK;
  if (N > kTableStepTokens)
    return set_err(SDM_RT_EUNSUPPORTED, "table_step: %lld tokens, at most %d", (long long)N, kTableStepTokens);
  if (d <= 0 || d % 64 != 0) return set_err(SDM_RT_EUNSUPPORTED, "table_step: d = %d must be a positive multiple of 64", d);
  if (p.d_a % 32 != 0 || p.d_a > 64)
    return set_err(SDM_RT_EUNSUPPORTED, "table_step: addr_dim = %d must be 32 or 64", p.d_a);
  if (p.dh % 8 != 0 || p.dh > kMaxHeadDim)
    return set_err(SDM_RT_EUNSUPPORTED, "table_step: head_dim = %d must be a multiple of 8 up to %d", p.dh,
                   kMaxHeadDim);
  if (p.pitch != p.cap) return set_err(SDM_RT_EUNSUPPORTED, "table_step: pick pitch %d", p.pitch);
  if ((!res && !hx) || !wq || !values || !slot_out || !out)
    return set_err(SDM_RT_EINVAL, "hx, wq, values, slot_out and out must not be NULL");
  if ((!res && hx_row_stride < d) || wq_row_stride < d || out_row_stride < static_cast<int64_t>(p.H) * p.dh ||
      (q_out && q_row_stride < static_cast<int64_t>(p.H) * p.d_a))
    return set_err(SDM_RT_EINVAL, "table_step: a row stride is smaller than its row");
  auto al16 = [](const void* ptr, int64_t stride) {
    return reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && (stride * 2) % 16 == 0;
  };
  if ((!res && !al16(hx, hx_row_stride)) || !al16(wq, wq_row_stride) || !al16(values, p.dh) ||
      !al16(out, out_row_stride))
    return set_err(SDM_RT_EINVAL, "table_step: hx, wq, values and out rows must be 16-byte aligned");
  if (res) {
    if (d != kFoldD) return set_err(SDM_RT_EUNSUPPORTED, "table_step_residual: d = %d, must be %d", d, kFoldD);
    if (!res->x || !res->y || !res->w || !res->sum)
      return set_err(SDM_RT_EINVAL, "table_step_residual: x, y, norm_w and sum_out must not be NULL");
    if (res->x_stride < d || res->y_stride < d || res->sum_stride < d)
      return set_err(SDM_RT_EINVAL, "table_step_residual: a row stride is smaller than its row");
    if (!al16(res->x, res->x_stride) || !al16(res->y, res->y_stride) || !al16(res->sum, res->sum_stride) ||
        reinterpret_cast<uintptr_t>(res->w) % 16)
      return set_err(SDM_RT_EINVAL, "table_step_residual: x, y, sum_out rows and norm_w must be 16-byte aligned");
    // every head's blocks read x and y; head 0's write the sum: in place only with one head
    if (p.H > 1 && (res->sum == res->x || res->sum == res->y))
      return set_err(SDM_RT_EINVAL, "table_step_residual: sum_out may alias x only with one head");
    if (res->sum == res->y) return set_err(SDM_RT_EINVAL, "table_step_residual: sum_out must not alias y");
    if (res->hx && (res->hx_stride < d || !al16(res->hx, res->hx_stride)))
      return set_err(SDM_RT_EINVAL, "table_step_residual: hx_out rows must be 16-byte aligned and >= d long");
  }
  TableStepArgs a{};
  a.g = addr_geom(p, params);
  a.hx = static_cast<const bf16_t*>(hx);
  a.hx_stride = hx_row_stride;
  a.d = d;
  a.wq = static_cast<const bf16_t*>(wq);
  a.wq_stride = wq_row_stride;
  a.values = static_cast<const bf16_t*>(values);
  a.M = p.M;
  a.dh = p.dh;
  a.pitch = p.pitch;
  a.B = p.B;
  a.T = p.T;
  a.q_out = static_cast<bf16_t*>(q_out);
  a.q_stride = q_row_stride;
  a.slot_out = slot_out;
  a.w_out = weight_out;
  a.s_out = score_out;
  a.r_out = static_cast<bf16_t*>(out);
  a.r_stride = out_row_stride;
  if (res) {
    a.rx = static_cast<const bf16_t*>(res->x);
    a.rx_stride = res->x_stride;
    a.ry = static_cast<const bf16_t*>(res->y);
    a.ry_stride = res->y_stride;
    a.rsum = static_cast<bf16_t*>(res->sum);
    a.rsum_stride = res->sum_stride;
    a.rw = res->w;
    a.reps = res->eps;
    a.hx_out = static_cast<bf16_t*>(res->hx);
    a.hx_out_stride = res->hx_stride;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return p.d_a == 32 ? TableStepLaunch<16>::run(p, a, st) : TableStepLaunch<32>::run(p, a, st);
}

}  // namespace

int sdm_rt_table_step(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* hx, int64_t hx_row_stride,
                      int32_t d, const void* wq, int64_t wq_row_stride, const void* values, void* q_out,
                      int64_t q_row_stride, int32_t* slot_out, float* score_out, float* weight_out, void* out,
                      int64_t out_row_stride, void* stream) {
  return table_step_impl(dims, params, hx, hx_row_stride, d, wq, wq_row_stride, values, q_out, q_row_stride, slot_out,
                         score_out, weight_out, out, out_row_stride, nullptr, stream);
}

int sdm_rt_table_step_residual(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* x,
                               int64_t x_row_stride, const void* y, int64_t y_row_stride, const float* norm_w,
                               float norm_eps, void* sum_out, int64_t sum_row_stride, void* hx_out,
                               int64_t hx_row_stride, int32_t d, const void* wq, int64_t wq_row_stride,
                               const void* values, void* q_out, int64_t q_row_stride, int32_t* slot_out,
                               float* score_out, float* weight_out, void* out, int64_t out_row_stride, void* stream) {
  const Residual res{x, x_row_stride, y, y_row_stride, norm_w, norm_eps, sum_out, sum_row_stride, hx_out, hx_row_stride};
  return table_step_impl(dims, params, nullptr, 0, d, wq, wq_row_stride, values, q_out, q_row_stride, slot_out,
                         score_out, weight_out, out, out_row_stride, &res, stream);
}

}  // extern "C"
