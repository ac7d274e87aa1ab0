// sdm_norm.h -- the RMS norm of one row, with the residual add before it (RMSNorm, experiments/track4/sdmllm/
// track4_sdmllm_models.py:69-71, after OneSdmLM's x = x + layer(x), track4_onesdm_models.py:540-547), shared by the
// norm kernels and the table step's folded prologue so that both give the same bits.
#pragma once
#include "sdm_common.h"

namespace sdmrt {

// x rounded to T and back (bfloat16: the hardware conversion, nearest even)
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (sizeof(T) == 2) return __uint_as_float(pack_bf16(x, 0.f) << 16);
  else return x;
}
// 8 values from / to T (16-byte pieces: p is 16-byte aligned, as the launchers check)
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __uint_as_float(w[e] << 16);
      v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  } else {
    const float4 q0 = reinterpret_cast<const float4*>(p)[0], q1 = reinterpret_cast<const float4*>(p)[1];
    v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
    v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
  }
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                                              pack_bf16(v[6], v[7]));
  } else {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}
// the sum over the 32 lanes of each half of the wave, in every lane of the half (DPP within rows of 16, then
// rows 0 + 1 and 2 + 3, read back from lanes 31 and 63)
__device__ __forceinline__ float half_wave_sum(float v, int lane) {
  v += dpp_f<0xb1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);    // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror: every lane of a row holds the row's sum
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));   // row_bcast:15
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return lane < 32 ? lo : hi;
}

// 8 values of T as one load brings them (bfloat16: one 16-byte piece; float32: two), unpacked when used
template <typename T>
struct Piece8 {
  uint4 q[sizeof(T) == 2 ? 1 : 2];
};
template <typename T>
__device__ __forceinline__ Piece8<T> load_piece8(const T* p) {
  Piece8<T> r;
#pragma unroll
  for (int i = 0; i < (sizeof(T) == 2 ? 1 : 2); ++i) r.q[i] = reinterpret_cast<const uint4*>(p)[i];
  return r;
}
template <typename T>
__device__ __forceinline__ void unpack8(const Piece8<T>& pc, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w[4] = {pc.q[0].x, pc.q[0].y, pc.q[0].z, pc.q[0].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __uint_as_float(w[e] << 16);
      v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      v[4 * i] = __uint_as_float(pc.q[i].x);
      v[4 * i + 1] = __uint_as_float(pc.q[i].y);
      v[4 * i + 2] = __uint_as_float(pc.q[i].z);
      v[4 * i + 3] = __uint_as_float(pc.q[i].w);
    }
  }
}

// R rows of the norm per half-wave: the 32 lanes of a half-wave (l % 32) each hold KC pieces of 8 consecutive values
// of every row, c = 8 (l % 32 + 32 k), d <= 256 KC; the rows, the residuals and the weights are all loaded before
// any use.  ADD: a row is x + y rounded to InT (a residual add); the row (the sum, or x unchanged without ADD) is
// written to sum when keep_sum (in place over x is allowed: each value is read and written by the same lane).  out = (s * rsqrt(mean(s^2) + eps) rounded to InT)
// * w, written when live.  Both halves of the wave take part (the sums cross lanes): a half without a row passes
// in-bounds pointers and live = keep_sum = false.  Each row's arithmetic does not depend on R.
template <typename InT, typename OutT, bool ADD, int KC, int R>
__device__ __forceinline__ void norm_rows(const InT* const (&xr)[R], const InT* const (&yr)[R], InT* const (&sr)[R],
                                          OutT* const (&dst)[R], const float* __restrict__ w, int d, float eps,
                                          int lane, const bool (&live)[R], const bool (&keep_sum)[R]) {
  const int hl = lane & 31;
  Piece8<InT> xp[R][KC], yp[R][ADD ? KC : 1];
  Piece8<float> wp[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = 8 * (hl + 32 * k);
    if (c < d) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        xp[r][k] = load_piece8<InT>(xr[r] + c);
        if constexpr (ADD) yp[r][k] = load_piece8<InT>(yr[r] + c);
      }
      wp[k] = load_piece8<float>(w + c);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float v[KC][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int c = 8 * (hl + 32 * k);
      if (c < d) {
        unpack8<InT>(xp[r][k], v[k]);
        if constexpr (ADD) {
          float u[8];
          unpack8<InT>(yp[r][k], u);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[k][e] = round_to<InT>(v[k][e] + u[e]);   // x + y in the input type
        }
        if (keep_sum[r]) store8<InT>(sr[r] + c, v[k]);   // the sum (ADD), or x itself (a gathered row's copy)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
      }
    }
    ss = half_wave_sum(ss, lane);
    const float rs = rsqrtf(ss / static_cast<float>(d) + eps);
    if (live[r]) {
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int c = 8 * (hl + 32 * k);
        if (c < d) {
          float wv[8], o[8];
          unpack8<float>(wp[k], wv);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = round_to<InT>(v[k][e] * rs) * wv[e];   // .to(x.dtype) * w
          store8<OutT>(dst[r] + c, o);
        }
      }
    }
  }
}

// One row of the norm per half-wave (norm_rows with R = 1)
template <typename InT, typename OutT, bool ADD, int KC>
__device__ __forceinline__ void norm_row(const InT* xr, const InT* yr, InT* sr, OutT* dst, const float* __restrict__ w,
                                         int d, float eps, int lane, bool live, bool keep_sum) {
  const InT* const xa[1] = {xr};
  const InT* const ya[1] = {yr};
  InT* const sa[1] = {sr};
  OutT* const da[1] = {dst};
  const bool la[1] = {live}, ka[1] = {keep_sum};
  norm_rows<InT, OutT, ADD, KC, 1>(xa, ya, sa, da, w, d, eps, lane, la, ka);
}

}  // namespace sdmrt
