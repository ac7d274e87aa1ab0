// sdm_decode.hip -- one decode step (sdm_rt_decode_step): the recurrence of RunTimeSdm.forward_sequential
// (experiments/track4/sdmllm/track4_onesdm_models.py:276-300) for one token per stream, the state carried in place.
#include "sdm_common.h"

namespace sdmrt {

// ---------------------------------------------------------------------------------------------------------------
// decode step: one token per stream (the recurrence of forward_sequential, track4_onesdm_models.py:276-300)
//
// The state of stream b, head h is kept as (mem, cnt, scale): the true memory is scale * mem and the true counts
// scale * cnt.  A step (after an optional reset, which empties the memory) reads first, then fades the state by lam
// in O(1) (scale <- lam * scale) and adds its writes divided by the new scale; when the scale falls below 2^-60 (or
// to 0) the slab is multiplied by it once and the scale reset to 1.  So the cost of a step does not grow with the
// position.  One wave per (head, stream); lane l takes columns l, l + 64, ...
struct DecodeArgs {
  const int32_t* wslot;   // [B][H][pitch] write picks of this token (from the addressing)
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
  void* r_out;            // rows of H * dh (one per stream)
  int64_t r_stride;
  int out_bf16, H, dh, M, kk, pitch, read_mean, out_norm;
  float read_eps, out_norm_eps;
};

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

template <typename VT, int KP>
__global__ void __launch_bounds__(64) decode_kernel(DecodeArgs a) {
  constexpr int kCols = 8;   // columns per lane: head_dim <= 512
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t sl = static_cast<int64_t>(b) * a.H + h;
  float* mem = a.mem + sl * a.M * a.dh;
  float* cnt = a.cnt + sl * a.M;
  const int kk = a.kk;
  // every load that does not depend on the state first, all issued together: the picks (pads: slot -1 read as
  // row 0 with weight 0; the weights of picks past kk are masked after the load), the value row, the scale, the
  // fade, the reset flag and the out-norm weights.  Loads stay unconditional (indexes clamped, null arrays read a
  // stand-in word of the scales): a load under a branch would be waited for on its own.
  int rsl[KP], wsl[KP];
  float rwv[KP], wwv[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    rsl[j] = max(a.rslot[sl * KP + j], 0);
    const float rw = a.rwt[sl * KP + j];
    rwv[j] = j < kk ? rw : 0.f;
    wsl[j] = max(a.wslot[sl * KP + j], 0);
    const float ww = a.wwt[sl * KP + j];
    wwv[j] = j < kk ? ww : 0.f;
  }
  const VT* vrow = static_cast<const VT*>(a.v) + static_cast<int64_t>(b) * a.v_stride + static_cast<int64_t>(h) * a.dh;
  float vv[kCols], onw[kCols];
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    const int cc = min(c, a.dh - 1);
    const float v0 = to_f32(vrow[cc]);
    vv[q] = c < a.dh ? v0 : 0.f;
    const float w0 = *(a.out_norm ? a.onorm_w + h * a.dh + cc : a.scale + sl);
    onw[q] = a.out_norm ? w0 : 1.f;
  }
  float mu = a.scale[sl];
  const float lam = a.decay[h];
  const uint8_t rst = *(a.reset ? a.reset + b : reinterpret_cast<const uint8_t*>(a.scale + sl));
  if (a.reset && rst) {   // a document starts here: the memory is emptied before the read
    scale_slab(mem, cnt, a.M, a.dh, 0.f, lane);
    mu = 1.f;
    __threadfence_block();
    __syncthreads();
  }
  // read: mu * sum_j wr_j * mem[sir_j], mu * sum_j wr_j * cnt[sir_j] (track4_onesdm_models.py:290-293); the rows
  // of all picks are loaded at once
  float acc[kCols];
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    acc[q] = 0.f;
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float row[KP];
#pragma unroll
      for (int j = 0; j < KP; ++j) row[j] = mem[static_cast<int64_t>(rsl[j]) * a.dh + c];   // weight 0 past kk
#pragma unroll
      for (int j = 0; j < KP; ++j) acc[q] = fmaf(rwv[j], row[j], acc[q]);
    }
  }
  float cr[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) cr[j] = cnt[rsl[j]];
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < KP; ++j) den = fmaf(rwv[j], cr[j], den);
  // finish (:243-246, without wo): mean read, then the per-head output norm
  const float dn = mu * den;
  const float rinv = a.read_mean ? 1.f / (dn + a.read_eps) : 1.f;
  float r[kCols];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    r[q] = c < a.dh ? (a.read_mean ? (mu * acc[q]) * rinv : mu * acc[q]) : 0.f;
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
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float o = r[q];
      if (a.out_norm) o = o * on * onw[q];
      const int64_t at = static_cast<int64_t>(b) * a.r_stride + static_cast<int64_t>(h) * a.dh + c;
      if (a.out_bf16) static_cast<bf16_t*>(a.r_out)[at] = from_f32<bf16_t>(o);
      else static_cast<float*>(a.r_out)[at] = o;
    }
  }
  // fade (O(1) through the scale; rescale the slab when the scale gets small), then write (:294-298)
  float mu2 = mu * lam;
  if (!(mu2 >= kMuFloor)) {
    scale_slab(mem, cnt, a.M, a.dh, mu2, lane);
    mu2 = 1.f;
    __threadfence_block();
    __syncthreads();
  }
  const float inv = 1.f / mu2;
#pragma unroll
  for (int q = 0; q < kCols; ++q) {   // the picks of one token are distinct slots
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float old[KP];
#pragma unroll
      for (int j = 0; j < KP; ++j) old[j] = mem[static_cast<int64_t>(wsl[j]) * a.dh + c];   // stored only below kk
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) mem[static_cast<int64_t>(wsl[j]) * a.dh + c] = fmaf(wwv[j] * inv, vv[q], old[j]);
      }
    }
  }
  if (lane == 0) {
    float oc[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) oc[j] = cnt[wsl[j]];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j < kk) cnt[wsl[j]] = oc[j] + wwv[j] * inv;
    }
    a.scale[sl] = mu2;
  }
}

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

size_t sdm_rt_decode_workspace_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  return 2 * align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256) +
         2 * align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
}

int sdm_rt_decode_step(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                       const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                       const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype,
                       const uint8_t* reset, float* state_mem, float* state_cnt, float* state_scale, void* r_out,
                       int64_t out_row_stride, sdm_rt_dtype out_dtype, void* workspace, size_t workspace_bytes,
                       void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if (p.T != 1) return set_err(SDM_RT_EINVAL, "a decode step takes one token per stream: seq_len must be 1, not %d", p.T);
  if ((rc = check_params(params, dims->out_norm != 0))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (p.B == 0) return SDM_RT_OK;
  if (!kz || !qz || !v || !r_out) return set_err(SDM_RT_EINVAL, "kz, qz, v and r_out must not be NULL");
  if (!state_mem || !state_cnt || !state_scale)
    return set_err(SDM_RT_EINVAL, "state_mem, state_cnt and state_scale must not be NULL");
  if (reinterpret_cast<uintptr_t>(state_mem) % 16 != 0) return set_err(SDM_RT_EINVAL, "state_mem must be 16-byte aligned");
  if (dims->write_gate && !gate_logits) return set_err(SDM_RT_EINVAL, "write_gate is set but gate_logits is NULL");
  const int64_t wa = static_cast<int64_t>(p.H) * p.d_a;
  const int64_t wv = static_cast<int64_t>(p.H) * p.dh;
  if (kz_row_stride < wa || qz_row_stride < wa)
    return set_err(SDM_RT_EINVAL, "kz/qz row stride (%lld, %lld) < heads * addr_dim", (long long)kz_row_stride,
                   (long long)qz_row_stride);
  if (v_row_stride < wv) return set_err(SDM_RT_EINVAL, "v_row_stride %lld < heads * head_dim", (long long)v_row_stride);
  if (gate_logits && gate_row_stride < p.H)
    return set_err(SDM_RT_EINVAL, "gate_row_stride %lld < heads", (long long)gate_row_stride);
  if (out_row_stride < wv)
    return set_err(SDM_RT_EINVAL, "out_row_stride %lld < heads * head_dim", (long long)out_row_stride);
  const size_t need = sdm_rt_decode_workspace_bytes(dims);
  if (!workspace || workspace_bytes < need)
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const size_t si = align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  const size_t sf = align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  int32_t* wslot = reinterpret_cast<int32_t*>(ws);
  int32_t* rslot = reinterpret_cast<int32_t*>(ws + si);
  float* wwt = reinterpret_cast<float*>(ws + 2 * si);
  float* rwt = reinterpret_cast<float*>(ws + 2 * si + sf);
  // the picks of this token, [B][H][1][pitch]: write keys (gated) and read queries, in one launch
  AddrArgs aa{};
  aa.g = addr_geom(p, params);
  aa.B = p.B;
  aa.T = 1;
  aa.pitch = p.pitch;
  aa.z = kz;
  aa.z_stride = kz_row_stride;
  aa.gl = dims->write_gate ? gate_logits : nullptr;
  aa.g_stride = gate_row_stride;
  aa.slot_out = wslot;
  aa.w_out = wwt;
  aa.z2 = qz;
  aa.z2_stride = qz_row_stride;
  aa.slot_out2 = rslot;
  aa.w_out2 = rwt;
  rc = launch_address(p, aa, in_dtype, st);
  if (rc) return rc;
  DecodeArgs da{};
  da.wslot = wslot;
  da.wwt = wwt;
  da.rslot = rslot;
  da.rwt = rwt;
  da.v = v;
  da.v_stride = v_row_stride;
  da.decay = params->decay;
  da.onorm_w = params->onorm_w;
  da.reset = reset;
  da.mem = state_mem;
  da.cnt = state_cnt;
  da.scale = state_scale;
  da.r_out = r_out;
  da.r_stride = out_row_stride;
  da.out_bf16 = out_dtype == SDM_RT_BF16;
  da.H = p.H;
  da.dh = p.dh;
  da.M = p.M;
  da.kk = p.kk;
  da.pitch = p.pitch;
  da.read_mean = dims->read_mean;
  da.out_norm = dims->out_norm;
  da.read_eps = dims->read_eps;
  da.out_norm_eps = dims->out_norm_eps;
  dim3 grid(p.H, p.B);
#define SDM_RT_DECODE(VT, KP) hipLaunchKernelGGL((decode_kernel<VT, KP>), grid, dim3(64), 0, st, da)
  if (in_dtype == SDM_RT_BF16) {
    if (p.pitch == 8) SDM_RT_DECODE(bf16_t, 8);
    else SDM_RT_DECODE(bf16_t, 16);
  } else {
    if (p.pitch == 8) SDM_RT_DECODE(float, 8);
    else SDM_RT_DECODE(float, 16);
  }
#undef SDM_RT_DECODE
  return check_launch("decode");
}
}  // extern "C"
