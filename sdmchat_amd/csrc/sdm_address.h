// sdm_address.h -- product-key addressing kernels (pk_address, experiments/track4/sdmllm/track4_onesdm_models.py:134-148,
// with the softmax weights and gate of prepare :203-207) and their launcher.  Included by sdm_address_bf16.hip and
// sdm_address_f32.hip, which instantiate them per input type in their own translation units (the builds run in
// parallel).
#pragma once

#include "sdm_common.h"

namespace sdmrt {


// sdm_rt_address: one thread per (token, head).  Grid: x = token tiles of 64, y = head.  MODE 1 and 2: the tile is
// addressed by the wave on the matrix cores (address_wave; 2 = no masked candidate), MODE 3 and 4 likewise with 64
// sub-keys per half (two sub-key tiles; 4 = no masked candidate), MODE 0: per thread with the sub-keys staged in
// LDS (address_one).
template <int HALF, int CAP, typename InT, int MODE>
__global__ void __launch_bounds__(64) address_kernel(AddrArgs a) {
  extern __shared__ float kn[];   // [2][n_sub][HALF] (per-thread path)
  const int h = blockIdx.y;
  const int64_t N = static_cast<int64_t>(a.B) * a.T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t n = n0 + threadIdx.x;
  if (blockIdx.z == 1) {   // the second address set
    a.z = a.z2;
    a.z_stride = a.z2_stride;
    a.gl = nullptr;
    a.slot_out = a.slot_out2;
    a.w_out = a.w_out2;
    a.s_out = a.s_out2;
  }
  const float gate =
      (a.gl && n < N) ? gate_of(static_cast<const InT*>(a.gl) + n * a.g_stride, h, a.g.gate_bias) : 1.f;
  int slot[CAP];
  float w[CAP], sc[CAP];
  if constexpr (MODE > 0) {
    address_wave<HALF, CAP, InT, MODE == 2 || MODE == 4, (MODE >= 3 ? 64 : 32)>(
        a.g, h, static_cast<const InT*>(a.z) + n0 * a.z_stride, a.z_stride,
                                     static_cast<int>(min<int64_t>(64, N - n0)), gate, slot, w, sc);
    if (n >= N) return;
  } else {
    stage_keys<HALF>(a.g, h, kn, threadIdx.x, 64);
    __syncthreads();
    if (n >= N) return;
    const InT* zrow = static_cast<const InT*>(a.z) + n * a.z_stride + static_cast<int64_t>(h) * 2 * HALF;
    address_one<HALF, CAP, InT>(a.g, h, kn, zrow, gate, slot, w, sc);
  }
  const int b = static_cast<int>(n / a.T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * a.T);
  const int64_t base = ((static_cast<int64_t>(b) * a.g.H + h) * a.T + t) * a.pitch;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    if (p < a.pitch) {
      const bool live = p < a.g.kk;
      a.slot_out[base + p] = live ? slot[p] : -1;
      if (a.w_out) a.w_out[base + p] = w[p];
      if (a.s_out) a.s_out[base + p] = sc[p];
    }
  }
}


// sdm_rt_address for few tokens (a decode step), where one wave per 64 addresses leaves the GPU idle and the
// selection of an address is the longest chain: block (4 addresses, head, set), 4 waves.  Wave q < 2 NS / 32 scores
// half q / (NS / 32) of the block's addresses against sub-key tile q % (NS / 32) on the matrix cores (half_scores, the
// scoring of address_wave); through LDS, wave j then selects address j across its lanes (select_lanes: the same keys,
// so the same picks, order, weights and scores as address_wave) and its lanes p < pitch store pick p.
template <int HALF, int CAP, typename InT, int MODE>
__global__ void __launch_bounds__(256) address_lanes_kernel(AddrArgs a) {
  constexpr int NS = MODE >= 3 ? 64 : 32;
  constexpr int NT = NS / 32;          // sub-key tiles per half
  constexpr bool FULL = MODE == 2 || MODE == 4;
  constexpr int kGroup = 4;
  __shared__ float s_sc[kGroup][2][NS];   // [address][half][sub-key] raw scores
  __shared__ float s_inv[kGroup][2];
  const int h = blockIdx.y;
  const int64_t N = static_cast<int64_t>(a.B) * a.T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kGroup;
  const int nb = static_cast<int>(min<int64_t>(kGroup, N - n0));
  const int lane = threadIdx.x & 63;
  const int q = threadIdx.x >> 6;
  if (blockIdx.z == 1) {   // the second address set
    a.z = a.z2;
    a.z_stride = a.z2_stride;
    a.gl = nullptr;
    a.slot_out = a.slot_out2;
    a.w_out = a.w_out2;
    a.s_out = a.s_out2;
  }
  if (q < 2 * NT) {
    const int hf = q / NT, tile = q % NT;
    const InT* z0 = static_cast<const InT*>(a.z) + n0 * a.z_stride;
    floatx16 acc[2];
    float inv[2];
    if constexpr (sizeof(InT) == 2) half_scores_bf16<HALF, FULL>(a.g, h, hf, z0, a.z_stride, nb, acc, inv, 32 * tile);
    else half_scores_f32<HALF, InT, FULL>(a.g, h, hf, z0, a.z_stride, nb, acc, inv, 32 * tile);
    // lane l: address l % 32 of tile 0, sub-keys 32 tile + 8 (r / 4) + 4 (l / 32) + r % 4
    const int row = lane & 31;
    if (row < nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s_sc[row][hf][32 * tile + 8 * (r / 4) + 4 * (lane >> 5) + (r & 3)] = acc[0][r];
      if (lane < 32 && tile == 0) s_inv[row][hf] = inv[0];
    }
  }
  __syncthreads();
  if (q >= nb) return;
  const int64_t n = n0 + q;
  const float gate = a.gl ? gate_of(static_cast<const InT*>(a.gl) + n * a.g_stride, h, a.g.gate_bias) : 1.f;
  int slot;
  float w, sc;
  select_lanes<CAP, FULL, NS>(a.g, a.g.log_scale[h], &s_sc[q][0][0], &s_inv[q][0], gate, slot, w, sc);
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

// token counts up to this take address_lanes_kernel (a block per 4 addresses pays when few blocks fill the GPU)
constexpr int64_t kSplitAddressTokens = 1024;

template <int HALF, typename InT>
struct AddressLaunch {
  template <int CAP, int MODE>
  static void go(const Plan& p, const AddrArgs& a, hipStream_t st) {
    const int64_t N = static_cast<int64_t>(p.B) * p.T;
    dim3 grid(static_cast<unsigned>((N + 63) / 64), p.H, a.z2 ? 2 : 1);
    if constexpr (MODE > 0) {
      if (N <= kSplitAddressTokens) {   // few tokens: a block per 4 addresses, each selected across a wave
        hipLaunchKernelGGL((address_lanes_kernel<HALF, CAP, InT, MODE>), dim3(static_cast<unsigned>((N + 3) / 4), p.H,
                           a.z2 ? 2 : 1), dim3(256), 0, st, a);
        return;
      }
    }
    const size_t lds = MODE > 0 ? 0 : sizeof(float) * 2 * p.n_sub * HALF;
    hipLaunchKernelGGL((address_kernel<HALF, CAP, InT, MODE>), grid, dim3(64), lds, st, a);
  }
  static int run(const Plan& p, const AddrArgs& a, hipStream_t st) {
    if constexpr (mf_half(HALF)) {
      if (use_mf(p)) {
        if (full_grid(p)) go<8, 2>(p, a, st);
        else if (p.cap == 8) go<8, 1>(p, a, st);
        else go<16, 1>(p, a, st);
        return check_launch("address");
      }
      if (use_mf64(p)) {   // 64 sub-keys per half: no masked candidate when n_sub = 64 and c1 = kk = CAP
        const bool full = p.n_sub == 64 && p.c1 == p.cap && p.kk == p.cap;
        if (p.cap == 8) full ? go<8, 4>(p, a, st) : go<8, 3>(p, a, st);
        else full ? go<16, 4>(p, a, st) : go<16, 3>(p, a, st);
        return check_launch("address");
      }
    }
    if (p.cap == 8) go<8, 0>(p, a, st);
    else go<16, 0>(p, a, st);
    return check_launch("address");
  }
};

}  // namespace sdmrt
