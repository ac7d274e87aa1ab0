// sdm_misc.hip -- the input norm (sdm_rt_rms_norm, and with the residual add before it sdm_rt_add_rms_norm),
// SwiGLU's gate (sdm_rt_silu_mul), the table read of TrainedSdm (sdm_rt_table_read) and the addressing entry point
// (sdm_rt_address).
#include "sdm_norm.h"

namespace sdmrt {

// rms_norm: two rows per wave, 32 lanes per row, each lane taking 8 consecutive values at a time (KC pieces of 8
// per lane, KC = ceil(d / 256)); the row, the residual and the weights are all loaded before any use.  ADD: the row
// is x + y rounded to the input type (a residual add), which is also written to sum (in place over x is allowed:
// each value is read and written by the same lane).
template <typename InT, typename OutT, bool ADD, int KC>
__global__ void __launch_bounds__(256) rms_norm_kernel(const InT* x, int64_t x_stride, const InT* y, int64_t y_stride,
                                                       InT* sum, int64_t sum_stride, OutT* __restrict__ out,
                                                       int64_t out_stride, const float* __restrict__ w, int64_t rows,
                                                       int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 6) * 2 + (lane >> 5);
  const bool live = row < rows;   // both halves of a wave take part in the sums
  const int64_t r = live ? row : 0;
  norm_row<InT, OutT, ADD, KC>(x + r * x_stride, ADD ? y + r * y_stride : nullptr, ADD ? sum + r * sum_stride : nullptr,
                               out + r * out_stride, w, d, eps, lane, live, ADD && live);
}

// SwiGLU's gate: out = silu(g) * u with g, u the two halves of a row of the fused [gate | up] projection, each
// product rounded as torch rounds silu(g) and then the product (x / (1 + exp(-x)) in float32, then the cast)
template <typename T>
__global__ void __launch_bounds__(256) silu_mul_kernel(const T* __restrict__ gu, int64_t gu_stride, T* __restrict__ out,
                                                       int64_t out_stride, int64_t rows, int f) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;   // 8 values per thread
  const int64_t per_row = f;
  const int64_t row = i / per_row;
  const int c = static_cast<int>(i - row * per_row);
  if (row >= rows) return;
  float g[8], u[8], o[8];
  load8<T>(gu + row * gu_stride + c, g);
  load8<T>(gu + row * gu_stride + f + c, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] = round_to<T>(g[e] / (1.f + expf(-g[e]))) * u[e];
  }
  store8<T>(out + row * out_stride + c, o);
}

// ---------------------------------------------------------------------------------------------------------------
// The KP picks of one (token, head) of a table read: slots clamped into the table (pads, -1, and stray ids stay
// inside it) and weights (0 past kk), in 16-byte loads when both arrays are 16-byte aligned (the pick rows are
// KP * 4 bytes at multiples of KP * 4 bytes, so the base pointers decide)
template <int KP>
__device__ __forceinline__ void load_picks(const int32_t* sp, const float* wp, int M, int kk, int (&sl)[KP],
                                           float (&w)[KP]) {
  if ((reinterpret_cast<uintptr_t>(sp) | reinterpret_cast<uintptr_t>(wp)) & 15u) {
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      sl[j] = min(max(sp[j], 0), M - 1);
      w[j] = j < kk ? wp[j] : 0.f;
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < KP / 4; ++q) {
    const int4 s4 = reinterpret_cast<const int4*>(sp)[q];
    const float4 w4 = reinterpret_cast<const float4*>(wp)[q];
    const int sv[4] = {s4.x, s4.y, s4.z, s4.w};
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sl[4 * q + e] = min(max(sv[e], 0), M - 1);
      w[4 * q + e] = 4 * q + e < kk ? wv[e] : 0.f;
    }
  }
}

// table read: the weighted sum of the picked rows of per-head value tables (TrainedSdm.forward's embedding_bag,
// track4_onesdm_models.py:448-455): out[n][h * dh + c] = sum_j w[n][h][j] * values[h][slot[n][h][j]][c] in float32,
// picks in order.  One workgroup of 256 threads per (token, head); thread i takes columns 4i ... 4i + 3 of every
// 1,024 (dh a multiple of 4), with the loads of all picks issued before any use: one round trip for the picks, one
// for the rows.
template <int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(256) table_read_kernel(const int32_t* __restrict__ slots,
                                                         const float* __restrict__ wts,
                                                         const VT* __restrict__ values, OutT* __restrict__ out,
                                                         int64_t out_stride, int B, int T, int H, int M, int dh,
                                                         int kk) {
  const int64_t item = blockIdx.x;   // (token, head)
  const int64_t n = item / H;
  const int h = static_cast<int>(item - n * H);
  const int b = static_cast<int>(n / T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * T);
  const int64_t pb = ((static_cast<int64_t>(b) * H + h) * T + t) * KP;
  int sl[KP];
  float w[KP];
  load_picks<KP>(slots + pb, wts + pb, M, kk, sl, w);
  const VT* tab = values + static_cast<int64_t>(h) * M * dh;
  for (int c0 = 4 * static_cast<int>(threadIdx.x); c0 < dh; c0 += 1024) {
    float v[KP][4];
#pragma unroll
    for (int j = 0; j < KP; ++j) load_vals<4, VT>(tab + static_cast<int64_t>(sl[j]) * dh + c0, v[j]);   // weight 0 past kk
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KP; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(w[j], v[j][e], acc[e]);
    }
    store_vals<4, OutT>(out + n * out_stride + static_cast<int64_t>(h) * dh + c0, acc);
  }
}

// The same read with the columns split eighth by eighth over the XCDs.  A launch deals its workgroups to the 8 XCDs
// in turn (workgroup i to XCD i mod 8), so with slice = blockIdx % 8 each XCD reads only its eighth of every row and
// its L2 holds H * M * dh / 8 values of the tables, where the read above makes every XCD's L2 cycle through whole
// tables larger than it.  A thread owns 16 bytes of a row slice for one (token, head): dh / (8 * kVec) threads per
// token, `tok` tokens per workgroup; the sums run over the picks in the same order as above (the same results).
template <int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(256) table_read_sliced_kernel(const int32_t* __restrict__ slots,
                                                                const float* __restrict__ wts,
                                                                const VT* __restrict__ values, OutT* __restrict__ out,
                                                                int64_t out_stride, int B, int T, int H, int M, int dh,
                                                                int kk, int tpt, int tok) {
  constexpr int kVec = 16 / static_cast<int>(sizeof(VT));
  const int slice = static_cast<int>(blockIdx.x & 7u);
  const int64_t rest = blockIdx.x >> 3;   // (token group, head)
  const int h = static_cast<int>(rest % H);
  const int64_t n = (rest / H) * tok + threadIdx.x / tpt;
  const int part = static_cast<int>(threadIdx.x % tpt);
  if (static_cast<int>(threadIdx.x) >= tok * tpt || n >= static_cast<int64_t>(B) * T) return;
  const int b = static_cast<int>(n / T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * T);
  const int64_t pb = ((static_cast<int64_t>(b) * H + h) * T + t) * KP;
  int sl[KP];
  float w[KP];
  load_picks<KP>(slots + pb, wts + pb, M, kk, sl, w);
  const int c0 = slice * (dh >> 3) + part * kVec;
  const VT* tab = values + static_cast<int64_t>(h) * M * dh + c0;
  float acc[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) acc[e] = 0.f;
  if ((reinterpret_cast<uintptr_t>(values) & 15u) == 0) {
    // 16-byte rows pieces kept raw until their turn (4 registers a pick; bfloat16 unpacked by shifts)
    uint4 raw[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) raw[j] = *reinterpret_cast<const uint4*>(tab + static_cast<int64_t>(sl[j]) * dh);
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      const uint32_t wd[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (sizeof(VT) == 2) {
          acc[2 * q] = fmaf(w[j], __uint_as_float(wd[q] << 16), acc[2 * q]);
          acc[2 * q + 1] = fmaf(w[j], __uint_as_float(wd[q] & 0xffff0000u), acc[2 * q + 1]);
        } else {
          acc[q] = fmaf(w[j], __uint_as_float(wd[q]), acc[q]);
        }
      }
    }
  } else {   // a table not 16-byte aligned: element loads, one pick at a time
    for (int j = 0; j < KP; ++j) {
      float v[kVec];
      load_vals<kVec, VT>(tab + static_cast<int64_t>(sl[j]) * dh, v);
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[e] = fmaf(w[j], v[e], acc[e]);
    }
  }
  store_vals<kVec, OutT>(out + n * out_stride + static_cast<int64_t>(h) * dh + c0, acc);
}

// a row-major array whose rows all start 16-byte aligned (the norm and silu kernels load 16 bytes at a time)
inline bool aligned16(const void* p, int64_t row_stride, sdm_rt_dtype dt) {
  const int64_t es = dt == SDM_RT_BF16 ? 2 : 4;
  return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (row_stride * es) % 16 == 0;
}

// rms_norm_kernel with kc pieces of 8 values per lane (d <= 256 kc)
template <typename IT, typename OT, bool ADD, typename... Args>
int norm_launch(int kc, unsigned blocks, hipStream_t st, Args... args) {
  switch (kc) {
    case 1: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 1>), dim3(blocks), dim3(256), 0, st, args...); break;
    case 2: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 2>), dim3(blocks), dim3(256), 0, st, args...); break;
    case 3: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 3>), dim3(blocks), dim3(256), 0, st, args...); break;
    case 4: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 4>), dim3(blocks), dim3(256), 0, st, args...); break;
    case 5: case 6: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 6>), dim3(blocks), dim3(256), 0, st, args...); break;
    default: hipLaunchKernelGGL((rms_norm_kernel<IT, OT, ADD, 8>), dim3(blocks), dim3(256), 0, st, args...); break;
  }
  return SDM_RT_OK;
}

// sdm_rt_prepare_key_pieces: block (head, half, sub-key tile of 32 rows), one wave; each lane computes its piece as
// the scoring does (load_sub_key_piece) and stores it in the KeyPieces layout
template <int HALF>
__global__ void __launch_bounds__(64) key_pieces_kernel(AddrGeom g, uint32_t* __restrict__ out) {
  constexpr int Q = SubKeyPiece<HALF>::Q;
  const int h = blockIdx.x, hf = blockIdx.y, tile = blockIdx.z;
  g.kpieces = nullptr;
  SubKeyPiece<HALF> kp;
  load_sub_key_piece<HALF>(g, h, hf, 32 * tile, kp);
  const int l = threadIdx.x & 63, kb = l >> 5;
  const int nsp = key_piece_rows(g.n_sub);
  const int64_t row = (static_cast<int64_t>(h) * 2 + hf) * nsp + 32 * tile + (l & 31);
  uint4* dst = reinterpret_cast<uint4*>(out + (row * 2 + kb) * KeyPieces<HALF>::kWords);
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int q = 0; q < Q; ++q) dst[t * Q + q] = make_uint4(kp.kt[t][q][0], kp.kt[t][q][1], kp.kt[t][q][2], kp.kt[t][q][3]);
  if (kb == 0) reinterpret_cast<float*>(out + KeyPieces<HALF>::term_words(g.H, nsp))[row] = kp.c;
}

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

size_t sdm_rt_key_pieces_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (!dims || make_plan(dims, &p, false)) return 0;
  return static_cast<size_t>(key_pieces_bytes(p));
}

int sdm_rt_prepare_key_pieces(const sdm_rt_dims* dims, const sdm_rt_params* params, void* out, size_t out_bytes,
                              void* stream) {
  g_err[0] = 0;
  if (!dims || !params) return set_err(SDM_RT_EINVAL, "dims and params must not be NULL");
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if (!params->keys1 || !params->keys2) return set_err(SDM_RT_EINVAL, "keys1 and keys2 must not be NULL");
  const int64_t need = key_pieces_bytes(p);
  if (need == 0) return set_err(SDM_RT_EUNSUPPORTED, "key pieces: no bfloat16 matrix-core scoring for this shape");
  if (!out || static_cast<int64_t>(out_bytes) < need)
    return set_err(SDM_RT_ENOSPACE, "key pieces: %zu bytes given, %lld needed", out_bytes, (long long)need);
  if (reinterpret_cast<uintptr_t>(out) % 16) return set_err(SDM_RT_EINVAL, "key pieces: out must be 16-byte aligned");
  AddrGeom g = addr_geom(p, params);
  const dim3 grid(static_cast<unsigned>(p.H), 2, static_cast<unsigned>(key_piece_rows(p.n_sub) / 32));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* o = static_cast<uint32_t*>(out);
  switch (p.half) {
    case 8: hipLaunchKernelGGL(key_pieces_kernel<8>, grid, dim3(64), 0, st, g, o); break;
    case 16: hipLaunchKernelGGL(key_pieces_kernel<16>, grid, dim3(64), 0, st, g, o); break;
    default: hipLaunchKernelGGL(key_pieces_kernel<32>, grid, dim3(64), 0, st, g, o); break;
  }
  return check_launch("prepare_key_pieces");
}

int sdm_rt_rms_norm(const void* x, int64_t x_row_stride, sdm_rt_dtype in_dtype, int64_t rows, int32_t d,
                    const float* w, float eps, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                    void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (rows < 0 || d < 1) return set_err(SDM_RT_EINVAL, "rows must be >= 0 and d >= 1");
  if (d % 8 != 0 || d > 2048) return set_err(SDM_RT_EUNSUPPORTED, "d = %d must be a multiple of 8 up to 2048", d);
  if (rows == 0) return SDM_RT_OK;
  if (!x || !w || !out) return set_err(SDM_RT_EINVAL, "x, w and out must not be NULL");
  if (x_row_stride < d || out_row_stride < d) return set_err(SDM_RT_EINVAL, "row strides must be >= d");
  if (!aligned16(x, x_row_stride, in_dtype) || !aligned16(out, out_row_stride, out_dtype) || !aligned16(w, 0, SDM_RT_F32))
    return set_err(SDM_RT_EINVAL, "x, out and w rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>((rows + 7) / 8);
  const int kc = (d + 255) / 256;
#define SDM_RT_NORM(IT, OT)                                                                                       \
  rc = norm_launch<IT, OT, false>(kc, blocks, st, static_cast<const IT*>(x), x_row_stride, nullptr, 0, nullptr, 0, \
                                  static_cast<OT*>(out), out_row_stride, w, rows, d, eps)
  if (in_dtype == SDM_RT_BF16) {
    if (out_dtype == SDM_RT_BF16) SDM_RT_NORM(bf16_t, bf16_t);
    else SDM_RT_NORM(bf16_t, float);
  } else {
    if (out_dtype == SDM_RT_BF16) SDM_RT_NORM(float, bf16_t);
    else SDM_RT_NORM(float, float);
  }
#undef SDM_RT_NORM
  if (rc) return rc;
  return check_launch("rms_norm");
}

int sdm_rt_add_rms_norm(const void* x, int64_t x_row_stride, const void* y, int64_t y_row_stride,
                        sdm_rt_dtype in_dtype, int64_t rows, int32_t d, const float* w, float eps, void* sum_out,
                        int64_t sum_row_stride, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                        void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (rows < 0 || d < 1) return set_err(SDM_RT_EINVAL, "rows must be >= 0 and d >= 1");
  if (d % 8 != 0 || d > 2048) return set_err(SDM_RT_EUNSUPPORTED, "d = %d must be a multiple of 8 up to 2048", d);
  if (rows == 0) return SDM_RT_OK;
  if (!x || !y || !w || !sum_out || !out) return set_err(SDM_RT_EINVAL, "x, y, w, sum_out and out must not be NULL");
  if (x_row_stride < d || y_row_stride < d || sum_row_stride < d || out_row_stride < d)
    return set_err(SDM_RT_EINVAL, "row strides must be >= d");
  if (!aligned16(x, x_row_stride, in_dtype) || !aligned16(y, y_row_stride, in_dtype) ||
      !aligned16(sum_out, sum_row_stride, in_dtype) || !aligned16(out, out_row_stride, out_dtype) ||
      !aligned16(w, 0, SDM_RT_F32))
    return set_err(SDM_RT_EINVAL, "x, y, sum_out, out and w rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>((rows + 7) / 8);
  const int kc = (d + 255) / 256;
#define SDM_RT_ADD_NORM(IT, OT)                                                                                \
  rc = norm_launch<IT, OT, true>(kc, blocks, st, static_cast<const IT*>(x), x_row_stride,                       \
                                 static_cast<const IT*>(y), y_row_stride, static_cast<IT*>(sum_out), sum_row_stride, \
                                 static_cast<OT*>(out), out_row_stride, w, rows, d, eps)
  if (in_dtype == SDM_RT_BF16) {
    if (out_dtype == SDM_RT_BF16) SDM_RT_ADD_NORM(bf16_t, bf16_t);
    else SDM_RT_ADD_NORM(bf16_t, float);
  } else {
    if (out_dtype == SDM_RT_BF16) SDM_RT_ADD_NORM(float, bf16_t);
    else SDM_RT_ADD_NORM(float, float);
  }
#undef SDM_RT_ADD_NORM
  if (rc) return rc;
  return check_launch("add_rms_norm");
}

int sdm_rt_silu_mul(const void* gate_up, int64_t gate_up_row_stride, sdm_rt_dtype dtype, int64_t rows, int32_t f,
                    void* out, int64_t out_row_stride, void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype(dtype, "dtype"))) return rc;
  if (rows < 0 || f < 1) return set_err(SDM_RT_EINVAL, "rows must be >= 0 and f >= 1");
  if (f % 8 != 0) return set_err(SDM_RT_EUNSUPPORTED, "f = %d must be a multiple of 8", f);
  if (rows == 0) return SDM_RT_OK;
  if (!gate_up || !out) return set_err(SDM_RT_EINVAL, "gate_up and out must not be NULL");
  if (gate_up_row_stride < 2 * static_cast<int64_t>(f) || out_row_stride < f)
    return set_err(SDM_RT_EINVAL, "gate_up_row_stride must be >= 2 f and out_row_stride >= f");
  if (!aligned16(gate_up, gate_up_row_stride, dtype) || !aligned16(out, out_row_stride, dtype))
    return set_err(SDM_RT_EINVAL, "gate_up and out rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t threads = rows * (f / 8);
  const unsigned blocks = static_cast<unsigned>((threads + 255) / 256);
  if (dtype == SDM_RT_BF16)
    hipLaunchKernelGGL((silu_mul_kernel<bf16_t>), dim3(blocks), dim3(256), 0, st, static_cast<const bf16_t*>(gate_up),
                       gate_up_row_stride, static_cast<bf16_t*>(out), out_row_stride, rows, f);
  else
    hipLaunchKernelGGL((silu_mul_kernel<float>), dim3(blocks), dim3(256), 0, st, static_cast<const float*>(gate_up),
                       gate_up_row_stride, static_cast<float*>(out), out_row_stride, rows, f);
  return check_launch("silu_mul");
}
int sdm_rt_address(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* z, int64_t z_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, int32_t* slot_out,
                   float* score_out, float* weight_out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if ((rc = check_params(params, false, false))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!z || !slot_out) return set_err(SDM_RT_EINVAL, "z and slot_out must not be NULL");
  if (z_row_stride < static_cast<int64_t>(p.H) * p.d_a)
    return set_err(SDM_RT_EINVAL, "z_row_stride %lld < heads * addr_dim", (long long)z_row_stride);
  if (gate_logits && gate_row_stride < p.H)
    return set_err(SDM_RT_EINVAL, "gate_row_stride %lld < heads", (long long)gate_row_stride);
  (void)workspace;   // the addressing alone needs no workspace
  (void)workspace_bytes;
  hipStream_t st = static_cast<hipStream_t>(stream);
  AddrArgs a{};
  a.g = addr_geom(p, params);
  a.z = z;
  a.z_stride = z_row_stride;
  a.gl = gate_logits;
  a.g_stride = gate_row_stride;
  a.B = p.B;
  a.T = p.T;
  a.pitch = p.pitch;
  a.slot_out = slot_out;
  a.w_out = weight_out;
  a.s_out = score_out;
  return launch_address(p, a, in_dtype, st);
}

int sdm_rt_table_read(const sdm_rt_dims* dims, const int32_t* slots, const float* weights, const void* values,
                      sdm_rt_dtype values_dtype, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                      void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if ((rc = check_dtype(values_dtype, "values_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (p.dh < 4 || p.dh % 4 != 0) return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d must be a positive multiple of 4", p.dh);
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!slots || !weights || !values || !out) return set_err(SDM_RT_EINVAL, "slots, weights, values and out must not be NULL");
  if (out_row_stride < static_cast<int64_t>(p.H) * p.dh)
    return set_err(SDM_RT_EINVAL, "out_row_stride %lld < heads * head_dim", (long long)out_row_stride);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n_tok = static_cast<int64_t>(p.B) * p.T;
  // the XCD-sliced read when a slice is whole 16-byte pieces and the tables outgrow an XCD's L2 share (1 MiB)
  const int vb = values_dtype == SDM_RT_BF16 ? 2 : 4;
  const int kvec = 16 / vb;
  const bool sliced = p.dh % (8 * kvec) == 0 && p.dh / (8 * kvec) <= 256 &&
                      static_cast<int64_t>(p.H) * p.M * p.dh * vb >= (int64_t{1} << 20);
  const int tpt = p.dh / (8 * kvec);
  const int tok = sliced ? 256 / tpt : 1;
  const int64_t groups = (n_tok + tok - 1) / tok;
  if (sliced && groups * p.H * 8 > 0x7fffffff) return set_err(SDM_RT_EUNSUPPORTED, "too many tokens for one launch");
  const unsigned blocks = static_cast<unsigned>(sliced ? groups * p.H * 8 : n_tok * p.H);
#define SDM_RT_TABLE(KP, VT, OT)                                                                                   \
  do {                                                                                                             \
    if (sliced)                                                                                                    \
      hipLaunchKernelGGL((table_read_sliced_kernel<KP, VT, OT>), dim3(blocks), dim3(tok * tpt), 0, st, slots,     \
                         weights, static_cast<const VT*>(values), static_cast<OT*>(out), out_row_stride, p.B, p.T, \
                         p.H, p.M, p.dh, p.kk, tpt, tok);                                                          \
    else                                                                                                           \
      hipLaunchKernelGGL((table_read_kernel<KP, VT, OT>), dim3(blocks), dim3(256), 0, st, slots, weights,         \
                         static_cast<const VT*>(values), static_cast<OT*>(out), out_row_stride, p.B, p.T, p.H,     \
                         p.M, p.dh, p.kk);                                                                         \
  } while (0)
#define SDM_RT_TABLE_KP(VT, OT) \
  if (p.pitch == 8) SDM_RT_TABLE(8, VT, OT); else SDM_RT_TABLE(16, VT, OT)
  if (values_dtype == SDM_RT_BF16) {
    if (out_dtype == SDM_RT_BF16) { SDM_RT_TABLE_KP(bf16_t, bf16_t); } else { SDM_RT_TABLE_KP(bf16_t, float); }
  } else {
    if (out_dtype == SDM_RT_BF16) { SDM_RT_TABLE_KP(float, bf16_t); } else { SDM_RT_TABLE_KP(float, float); }
  }
#undef SDM_RT_TABLE_KP
#undef SDM_RT_TABLE
  return check_launch("table_read");
}
}  // extern "C"
