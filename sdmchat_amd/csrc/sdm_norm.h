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

// One row of the norm: the 32 lanes of a half-wave (l % 32) each hold KC pieces of 8 consecutive values,
// c = 8 (l % 32 + 32 k), d <= 256 KC; the row, the residual and the weights are all loaded before any use.  ADD: the
// row is x + y rounded to InT (a residual add), also written to sum when keep_sum (in place over x is allowed: each
// value is read and written by the same lane).  out = (s * rsqrt(mean(s^2) + eps) rounded to InT) * w, written
// when live.  Both halves of the wave take part (the sum crosses lanes): a half without a row passes in-bounds
// pointers and live = keep_sum = false.
template <typename InT, typename OutT, bool ADD, int KC>
__device__ __forceinline__ void norm_row(const InT* xr, const InT* yr, InT* sr, OutT* dst, const float* __restrict__ w,
                                         int d, float eps, int lane, bool live, bool keep_sum) {
  const int hl = lane & 31;
  float v[KC][8], wv[KC][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = 8 * (hl + 32 * k);
    if (c < d) {
      load8<InT>(xr + c, v[k]);
      load8<float>(w + c, wv[k]);
      if constexpr (ADD) {
        float u[8];
        load8<InT>(yr + c, u);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = round_to<InT>(v[k][e] + u[e]);   // x + y in the input type
        if (keep_sum) store8<InT>(sr + c, v[k]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
  ss = half_wave_sum(ss, lane);
  const float rs = rsqrtf(ss / static_cast<float>(d) + eps);
  if (!live) return;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = 8 * (hl + 32 * k);
    if (c < d) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = round_to<InT>(v[k][e] * rs) * wv[k][e];   // .to(x.dtype) * w
      store8<OutT>(dst + c, o);
    }
  }
}

}  // namespace sdmrt
