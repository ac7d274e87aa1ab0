// sdm_decode.hip -- one decode step (sdm_rt_decode_step): the recurrence of RunTimeSdm.forward_sequential
// (experiments/track4/sdmllm/track4_onesdm_models.py:276-300) for one token per stream, the state carried in place.
// Shapes whose addressing runs on the matrix cores take one launch (decode_fused_kernel); the others an addressing
// launch and decode_kernel.
#include "sdm_decode.h"

using namespace sdmrt;

extern "C" {

size_t sdm_rt_decode_workspace_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  if (use_mf(p)) return 256;   // one launch: the picks stay on chip
  return 2 * align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256) +
         2 * align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
}

int sdm_rt_decode_step(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                       const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                       const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype,
                       const uint8_t* reset, float* state_mem, float* state_cnt, float* state_scale,
                       int32_t* state_last, void* r_out,
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
  DecodeArgs da{};
  da.v = v;
  da.v_stride = v_row_stride;
  da.decay = params->decay;
  da.onorm_w = params->onorm_w;
  da.reset = reset;
  da.mem = state_mem;
  da.cnt = state_cnt;
  da.scale = state_scale;
  da.last = state_last;
  da.r_out = r_out;
  da.r_stride = out_row_stride;
  da.out_bf16 = out_dtype == SDM_RT_BF16;
  da.B = p.B;
  da.H = p.H;
  da.dh = p.dh;
  da.M = p.M;
  da.kk = p.kk;
  da.pitch = p.pitch;
  da.read_mean = dims->read_mean;
  da.out_norm = dims->out_norm;
  da.read_eps = dims->read_eps;
  da.out_norm_eps = dims->out_norm_eps;
  da.g = addr_geom(p, params);
  da.kz = kz;
  da.kz_stride = kz_row_stride;
  da.qz = qz;
  da.qz_stride = qz_row_stride;
  da.gl = dims->write_gate ? gate_logits : nullptr;
  da.g_stride = gate_row_stride;
  if (use_mf(p))   // one launch: addressing on the matrix cores, then the step
    return in_dtype == SDM_RT_BF16 ? launch_decode_fused_bf16(p, da, st) : launch_decode_fused_f32(p, da, st);
  // other shapes: the picks of this token, [B][H][1][pitch] (write keys, gated, and read queries) in one launch,
  // then the step
  char* ws = static_cast<char*>(workspace);
  const size_t si = align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  const size_t sf = align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  int32_t* wslot = reinterpret_cast<int32_t*>(ws);
  int32_t* rslot = reinterpret_cast<int32_t*>(ws + si);
  float* wwt = reinterpret_cast<float*>(ws + 2 * si);
  float* rwt = reinterpret_cast<float*>(ws + 2 * si + sf);
  AddrArgs aa{};
  aa.g = da.g;
  aa.B = p.B;
  aa.T = 1;
  aa.pitch = p.pitch;
  aa.z = kz;
  aa.z_stride = kz_row_stride;
  aa.gl = da.gl;
  aa.g_stride = gate_row_stride;
  aa.slot_out = wslot;
  aa.w_out = wwt;
  aa.z2 = qz;
  aa.z2_stride = qz_row_stride;
  aa.slot_out2 = rslot;
  aa.w_out2 = rwt;
  rc = launch_address(p, aa, in_dtype, st);
  if (rc) return rc;
  da.wslot = wslot;
  da.wwt = wwt;
  da.rslot = rslot;
  da.rwt = rwt;
  dim3 grid(p.H, p.B);
#define SDM_RT_DECODE(VT, KP)                                                                 \
  do {                                                                                        \
    if (decode_cols(p.dh) == 1) hipLaunchKernelGGL((decode_kernel<VT, KP, 1>), grid, dim3(64), 0, st, da); \
    else hipLaunchKernelGGL((decode_kernel<VT, KP, 8>), grid, dim3(64), 0, st, da);          \
  } while (0)
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
