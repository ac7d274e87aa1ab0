// sdm_decode.h -- the decode step's kernels: the recurrence of RunTimeSdm.forward_sequential
// (experiments/track4/sdmllm/track4_onesdm_models.py:276-300) for one token per stream, the state carried in place.
// decode_fused_kernel (one launch: the addressing of both address sets on the matrix cores, then the step) is
// instantiated per value type by sdm_decode_bf16.hip and sdm_decode_f32.hip; decode_kernel (after a separate
// addressing launch, for the shapes the matrix-core addressing does not take) by sdm_decode.hip.
#pragma once

#include "sdm_common.h"

namespace sdmrt {

// The state of stream b, head h is kept as (mem, cnt, scale): the true memory is scale * mem and the true counts
// scale * cnt.  A step (after an optional reset, which empties the memory) reads first, then fades the state by lam
// in O(1) (scale <- lam * scale) and adds its writes divided by the new scale; when the scale falls below 2^-60 the
// slab is multiplied by it once and the scale reset to 1.  A head with decay 0 keeps nothing but the last step's
// writes: with the slots of those writes kept (last), the next step zeroes those rows only.  So the cost of a step
// does not grow with the position.  One wave per (stream, head); lane l takes columns l, l + 64, ...
constexpr int32_t kLastUnknown = -2;   // last[0]: the slab may hold other rows (clear it whole when decay is 0)

struct DecodeArgs {
  const int32_t* wslot;   // [B][H][pitch] write picks of this token (from a separate addressing launch)
  const float* wwt;       //   and their weights (gate included)
  const int32_t* rslot;   // read picks
  const float* rwt;
  const void* v;          // value rows (one per stream)
  int64_t v_stride;
  const float* decay;     // [H]
  const float* onorm_w;   // [H][dh]
  const uint8_t* reset;   // [B] or nullptr: 1 empties the stream's memory before it reads
  float* mem;             // [B][H][M][dh]
  float* cnt;             // [B][H][M]
  float* scale;           // [B][H]
  int32_t* last;          // [B][H][pitch] slots of the last step's writes (-1 unused; kLastUnknown), or nullptr
  void* r_out;            // rows of H * dh (one per stream)
  int64_t r_stride;
  int out_bf16, B, H, dh, M, kk, pitch, read_mean, out_norm;
  float read_eps, out_norm_eps;
  // the fused kernel's addressing: write keys (gated) and read queries, one row per stream
  AddrGeom g;
  const void* kz;
  int64_t kz_stride;
  const void* qz;
  int64_t qz_stride;
  const void* gl;
  int64_t g_stride;
};

// a wave's global stores complete and visible to its own later loads (one wave owns a (stream, head) slab)
__device__ __forceinline__ void wave_fence() {
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
}

// the slab of one (stream, head) times f (0 empties it), float4 at a time; the caller fences
__device__ __forceinline__ void scale_slab(float* mem, float* cnt, int M, int dh, float f, int lane) {
  float4* m4 = reinterpret_cast<float4*>(mem);
  const int n4 = M * dh / 4;
  for (int i = lane; i < n4; i += 4 * 64) {
    float4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = i + 64 * u < n4 ? m4[i + 64 * u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i + 64 * u < n4) m4[i + 64 * u] = make_float4(x[u].x * f, x[u].y * f, x[u].z * f, x[u].w * f);
    }
  }
  for (int m = lane; m < M; m += 64) cnt[m] *= f;
}

// what a step of stream b, head h loads independently of its picks and of the state: the value row, the out-norm
// weights, the scale, the fade, the reset flag and the last-write slots (columns lane + 64 q, q < C; past dh
// clamped, unused).  Loads stay unconditional (null arrays read a stand-in word of the scales), so they issue together.
template <typename VT, int KP, int C>
struct DecodePre {
  float vv[C], onw[C];
  float mu, lam;
  bool rst;
  int32_t last[KP];
};
template <typename VT, int KP, int C>
__device__ __forceinline__ DecodePre<VT, KP, C> decode_pre(const DecodeArgs& a, int b, int h, int lane) {
  DecodePre<VT, KP, C> d;
  const int64_t sl = static_cast<int64_t>(b) * a.H + h;
  const VT* vrow = static_cast<const VT*>(a.v) + static_cast<int64_t>(b) * a.v_stride + static_cast<int64_t>(h) * a.dh;
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int cc = min(lane + 64 * q, a.dh - 1);
    d.vv[q] = to_f32(vrow[cc]);
    const float w0 = *(a.out_norm ? a.onorm_w + h * a.dh + cc : a.scale + sl);
    d.onw[q] = a.out_norm ? w0 : 1.f;
  }
  d.mu = a.scale[sl];
  d.lam = a.decay[h];
  d.rst = a.reset && *(a.reset + b);
#pragma unroll
  for (int j = 0; j < KP; ++j) d.last[j] = a.last ? a.last[sl * a.pitch + j] : kLastUnknown;
  return d;
}

// The step of stream b, head h by one wave, given the token's picks (pads: slot 0 with weight 0): every state
// value it uses (the read rows and counts, and the old values of the written rows and counts) is loaded at once,
// then the read-out is finished and stored, the state faded (the old values scaled as the slab is) and the writes
// stored.
template <typename VT, int KP, int C>
__device__ __forceinline__ void decode_one(const DecodeArgs& a, int b, int h, int lane,
                                           const DecodePre<VT, KP, C>& pre, const int (&rsl)[KP],
                                           const float (&rwv)[KP], const int (&wsl)[KP], const float (&wwv)[KP]) {
  const int64_t sl = static_cast<int64_t>(b) * a.H + h;
  float* mem = a.mem + sl * a.M * a.dh;
  float* cnt = a.cnt + sl * a.M;
  const int kk = a.kk;
  float row[KP][C], old[KP][C], cr[KP], oc[KP];
  if (!pre.rst) {
#pragma unroll
    for (int q = 0; q < C; ++q) {
      const int cc = min(lane + 64 * q, a.dh - 1);
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        row[j][q] = mem[static_cast<int64_t>(rsl[j]) * a.dh + cc];
        old[j][q] = mem[static_cast<int64_t>(wsl[j]) * a.dh + cc];
      }
    }
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      cr[j] = cnt[rsl[j]];
      oc[j] = cnt[wsl[j]];
    }
  } else {   // a document starts here: the memory is emptied before the read, which then reads zeros
#pragma unroll
    for (int j = 0; j < KP; ++j) {
#pragma unroll
      for (int q = 0; q < C; ++q) row[j][q] = old[j][q] = 0.f;
      cr[j] = oc[j] = 0.f;
    }
    scale_slab(mem, cnt, a.M, a.dh, 0.f, lane);
    wave_fence();
  }
  const float mu = pre.rst ? 1.f : pre.mu;
  // read: mu * sum_j wr_j * mem[sir_j], mu * sum_j wr_j * cnt[sir_j] (track4_onesdm_models.py:290-293)
  float acc[C];
#pragma unroll
  for (int q = 0; q < C; ++q) {
    acc[q] = 0.f;
#pragma unroll
    for (int j = 0; j < KP; ++j) acc[q] = fmaf(rwv[j], row[j][q], acc[q]);   // weight 0 past kk
  }
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < KP; ++j) den = fmaf(rwv[j], cr[j], den);
  // finish (:243-246, without wo): mean read, then the per-head output norm
  const float dn = mu * den;
  const float rinv = a.read_mean ? 1.f / (dn + a.read_eps) : 1.f;
  float r[C];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < C; ++q) {
    r[q] = lane + 64 * q < a.dh ? (a.read_mean ? (mu * acc[q]) * rinv : mu * acc[q]) : 0.f;
    ss = fmaf(r[q], r[q], ss);
  }
  float on = 1.f;
  if (a.out_norm) {   // the wave sum: rows of 16 lanes by DPP, then the four row sums
    float s16 = sum8(ss);
    s16 += dpp_f<0x140>(s16);   // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 48));
    ss = (r0 + r1) + (r2 + r3);
    on = rsqrtf(ss / static_cast<float>(a.dh) + a.out_norm_eps);
  }
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float o = r[q];
      if (a.out_norm) o = o * on * pre.onw[q];
      const int64_t at = static_cast<int64_t>(b) * a.r_stride + static_cast<int64_t>(h) * a.dh + c;
      if (a.out_bf16) static_cast<bf16_t*>(a.r_out)[at] = from_f32<bf16_t>(o);
      else static_cast<float*>(a.r_out)[at] = o;
    }
  }
  // fade (O(1) through the scale; rescale the slab when the scale gets small), then write (:294-298)
  float mu2 = mu * pre.lam;
  const bool cleared = mu2 == 0.f;   // decay 0: nothing but this step's writes remains
  if (!(mu2 >= kMuFloor)) {
    if (cleared) {
      if (!pre.rst) {
        if (pre.last[0] != kLastUnknown) {   // only the last step's rows are nonzero: zero them
#pragma unroll
          for (int j = 0; j < KP; ++j) {
            const int32_t s0 = pre.last[j];
            if (s0 >= 0) {
#pragma unroll
              for (int q = 0; q < C; ++q) {
                const int c = lane + 64 * q;
                if (c < a.dh) mem[static_cast<int64_t>(s0) * a.dh + c] = 0.f;
              }
              if (lane == 0) cnt[s0] = 0.f;
            }
          }
        } else {
          scale_slab(mem, cnt, a.M, a.dh, 0.f, lane);
        }
      }
#pragma unroll
      for (int j = 0; j < KP; ++j) {   // the whole slab is zero now
#pragma unroll
        for (int q = 0; q < C; ++q) old[j][q] = 0.f;
        oc[j] = 0.f;
      }
    } else {
      scale_slab(mem, cnt, a.M, a.dh, mu2, lane);
#pragma unroll
      for (int j = 0; j < KP; ++j) {   // as the slab scales
#pragma unroll
        for (int q = 0; q < C; ++q) old[j][q] *= mu2;
        oc[j] *= mu2;
      }
    }
    mu2 = 1.f;
    wave_fence();
  }
  const float inv = 1.f / mu2;
#pragma unroll
  for (int q = 0; q < C; ++q) {   // the picks of one token are distinct slots
    const int c = lane + 64 * q;
    if (c < a.dh) {
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) mem[static_cast<int64_t>(wsl[j]) * a.dh + c] = fmaf(wwv[j] * inv, pre.vv[q], old[j][q]);
      }
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j < kk) cnt[wsl[j]] = oc[j] + wwv[j] * inv;
    }
    a.scale[sl] = mu2;
    if (a.last) {
#pragma unroll
      for (int j = 0; j < KP; ++j)
        a.last[sl * a.pitch + j] = cleared ? (j < kk ? wsl[j] : -1) : (j == 0 ? kLastUnknown : -1);
    }
  }
}

// columns per lane of a step: head_dim <= 64, else <= 512
inline int decode_cols(int dh) { return dh <= 64 ? 1 : 8; }

// after a separate addressing launch: one wave per (head, stream), the picks from global memory
template <typename VT, int KP, int C>
__global__ void __launch_bounds__(64) decode_kernel(DecodeArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t sl = static_cast<int64_t>(b) * a.H + h;
  const DecodePre<VT, KP, C> pre = decode_pre<VT, KP, C>(a, b, h, threadIdx.x);
  int rsl[KP], wsl[KP];
  float rwv[KP], wwv[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {   // pads (slot -1) read row 0 with weight 0
    rsl[j] = max(a.rslot[sl * KP + j], 0);
    const float rw = a.rwt[sl * KP + j];
    rwv[j] = j < a.kk ? rw : 0.f;
    wsl[j] = max(a.wslot[sl * KP + j], 0);
    const float ww = a.wwt[sl * KP + j];
    wwv[j] = j < a.kk ? ww : 0.f;
  }
  decode_one<VT, KP, C>(a, b, h, threadIdx.x, pre, rsl, rwv, wsl, wwv);
}

// One launch: block (head, group of 4 streams), 8 waves.  Wave 2 s + hf scores half hf of the group's addresses of
// set s (0: write keys, 1: read queries) against the head's sub-keys on the matrix cores (half_scores, the forward's
// scoring); through LDS, wave 4 s + j then selects address j of set s across its lanes (select_lanes), so the picks
// equal the forward's; the picks pass through LDS again and wave j steps stream b0 + j.
template <int HALF, int CAP, typename VT, bool FULL, int C>
__global__ void __launch_bounds__(512) decode_fused_kernel(DecodeArgs a) {
  constexpr int kGroup = 4;
  __shared__ float s_sc[2][kGroup][2][32];   // [set][stream][half][sub-key] raw scores
  __shared__ float s_inv[2][kGroup][2];
  __shared__ int s_slot[2][kGroup][CAP];
  __shared__ float s_w[2][kGroup][CAP];
  const int h = blockIdx.x;
  const int b0 = blockIdx.y * kGroup;
  const int nb = min(kGroup, a.B - b0);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the loads that depend on nothing else first: the stepping waves' value rows, scales, ..., and the gate
  const DecodePre<VT, CAP, C> pre = decode_pre<VT, CAP, C>(a, b0 + min(wave, nb - 1), h, lane);   // unused past nb
  const int set = wave / kGroup, jg = wave % kGroup;
  // the raw gate logit now, its sigmoid after the scoring (a use here would wait for every load above)
  const bool gated = set == 0 && a.gl && jg < nb;
  const float glog = gated ? to_f32(static_cast<const VT*>(a.gl)[(b0 + jg) * a.g_stride + h]) : 0.f;
  const float gbias = gated && a.g.gate_bias ? a.g.gate_bias[h] : 0.f;
  const float log_scale = a.g.log_scale[h];
  if (wave < 4) {
    const int ss = wave >> 1, hf = wave & 1;
    const VT* z = static_cast<const VT*>(ss == 0 ? a.kz : a.qz) + b0 * (ss == 0 ? a.kz_stride : a.qz_stride);
    const int64_t zs = ss == 0 ? a.kz_stride : a.qz_stride;
    floatx16 acc[2];
    float inv[2];
    if constexpr (sizeof(VT) == 2) half_scores_bf16<HALF, FULL>(a.g, h, hf, z, zs, nb, acc, inv);
    else half_scores_f32<HALF, VT, FULL>(a.g, h, hf, z, zs, nb, acc, inv);
    // lane l: address l % 32 of tile 0, sub-keys 8 (r / 4) + 4 (l / 32) + r % 4
    const int row = lane & 31;
    if (row < nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s_sc[ss][row][hf][8 * (r / 4) + 4 * (lane >> 5) + (r & 3)] = acc[0][r];
      if (lane < 32) s_inv[ss][row][hf] = inv[0];
    }
  }
  __syncthreads();
  if (jg < nb) {
    const float gate = gated ? 1.f / (1.f + expf(-(glog + gbias))) : 1.f;   // gate_of
    int slot;
    float w, score;
    select_lanes<CAP, FULL>(a.g, log_scale, &s_sc[set][jg][0][0], &s_inv[set][jg][0], gate, slot, w, score);
    if (lane < CAP) {
      s_slot[set][jg][lane] = slot;
      s_w[set][jg][lane] = w;
    }
  }
  __syncthreads();
  if (wave >= nb) return;
  int rsl[CAP], wsl[CAP];
  float rwv[CAP], wwv[CAP];
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    wsl[j] = s_slot[0][wave][j];
    wwv[j] = s_w[0][wave][j];
    rsl[j] = s_slot[1][wave][j];
    rwv[j] = s_w[1][wave][j];
  }
  decode_one<VT, CAP, C>(a, b0 + wave, h, lane, pre, rsl, rwv, wsl, wwv);
}

template <int HALF, typename VT>
struct DecodeFusedLaunch {
  template <int CAP, bool FULL>
  static int go(const Plan& p, const DecodeArgs& a, hipStream_t st) {
    dim3 grid(p.H, (p.B + 3) / 4);
    if (decode_cols(p.dh) == 1) hipLaunchKernelGGL((decode_fused_kernel<HALF, CAP, VT, FULL, 1>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((decode_fused_kernel<HALF, CAP, VT, FULL, 8>), grid, dim3(512), 0, st, a);
    return check_launch("decode");
  }
  static int run(const Plan& p, const DecodeArgs& a, hipStream_t st) {
    if constexpr (mf_half(HALF)) {
      if (full_grid(p)) return go<8, true>(p, a, st);
      return p.cap == 8 ? go<8, false>(p, a, st) : go<16, false>(p, a, st);
    }
    return set_err(SDM_RT_EUNSUPPORTED, "decode: no matrix-core addressing for addr_dim %d", 2 * HALF);
  }
};

// defined in sdm_decode_bf16.hip and sdm_decode_f32.hip: the fused step for shapes with use_mf(p)
int launch_decode_fused_bf16(const Plan& p, const DecodeArgs& a, hipStream_t st);
int launch_decode_fused_f32(const Plan& p, const DecodeArgs& a, hipStream_t st);

}  // namespace sdmrt
