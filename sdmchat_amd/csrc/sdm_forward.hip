// sdm_forward.hip -- the forward of the SDM core (sdm_rt_forward): plan_kernel, then the scan with the read-out
// finished in place (pick_scan_kernel where its shape fits, else scan_kernel).  Replaces RunTimeSdm.forward between
// the projections and wo (experiments/track4/sdmllm/track4_onesdm_models.py:195-274, finish :243-246 without wo).
#include <atomic>
#include <cstdlib>

#include "sdm_pick.h"

namespace sdmrt {

static std::atomic<uint32_t> g_wait_limit{kSpinLimit};
uint32_t wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }
static std::atomic<int> g_crowded_bytes{kVarStage};
int crowded_threshold() { return g_crowded_bytes.load(std::memory_order_relaxed); }

// the status word a forward's scan leaves in its workspace (after the progress counters)
static size_t status_offset(const Plan& p) {
  return p.off_sync + sizeof(uint32_t) * static_cast<size_t>(p.B) * p.H * p.groups;
}

// SDM_RT_SCAN=chunk in the environment keeps every shape on scan_kernel (read once per process)
static bool pick_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("SDM_RT_SCAN");
    return !(e && std::strcmp(e, "chunk") == 0);
  }();
  return on;
}

// dst[i] = src ? src[i] : 0 for n floats: the state of a call with no positions (a kernel, not a memset or copy
// node, so that it may be captured in a graph)
__global__ void __launch_bounds__(256) state_copy_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                         int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[i] = src ? src[i] : 0.f;
}

static int state_copy(float* dst, const float* src, int64_t n, hipStream_t st) {
  if (n <= 0) return SDM_RT_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(state_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, dst, src, n);
  return check_launch("state copy");
}

int run_core(const Plan& p, const sdm_rt_dims* dims, const sdm_rt_params* prm, const CoreIO& io, void* workspace,
             hipStream_t st) {
  char* ws = static_cast<char*>(workspace);
  int32_t* sizes = reinterpret_cast<int32_t*>(ws + p.off_sizes);
  unsigned char* plans = reinterpret_cast<unsigned char*>(ws + p.off_plans);
  uint32_t* sync = reinterpret_cast<uint32_t*>(ws + p.off_sync);
  float* xch = reinterpret_cast<float*>(ws + p.off_xch);
  const size_t vb = io.in_dtype == SDM_RT_BF16 ? 2 : 4;
  const bool pick = pick_enabled() && pick_path(p);
  const int cw = pick ? kPickCols : scan_cw(p, io.in_dtype);
  if (!cw) return SDM_RT_EUNSUPPORTED;

  PlanArgs pa{};
  pa.g = addr_geom(p, prm);
  pa.kz = io.kz;
  pa.kz_stride = io.kz_stride;
  pa.qz = io.qz;
  pa.qz_stride = io.qz_stride;
  pa.gl = dims->write_gate ? io.gate_logits : nullptr;
  pa.gate_copy = pa.gl ? ws + p.off_gate : nullptr;
  pa.g_stride = io.g_stride;
  pa.decay = prm->decay;
  pa.reset = io.reset;
  pa.plans = plans;
  pa.sizes = sizes;
  pa.sync = sync;
  pa.groups = p.groups;
  pa.xch = pick && dims->out_norm && p.dh / cw > 1 ? reinterpret_cast<unsigned long long*>(xch) : nullptr;
  pa.xgroups = p.dh / cw;
  pa.row_bytes = cw * static_cast<int>(sizeof(float));
  pa.B = p.B;
  pa.T = p.T;
  pa.M = p.M;
  pa.n_chunks = p.n_chunks;
  int rc = io.in_dtype == SDM_RT_BF16 ? launch_plan_bf16(p, pa, st, pick) : launch_plan_f32(p, pa, st, pick);
  if (rc) return rc;

  ScanArgs s{};
  s.plans = plans;
  s.sizes = sizes;
  s.v = io.v;
  s.v_stride = io.v_stride;
  s.decay = prm->decay;
  s.onorm_w = dims->out_norm ? prm->onorm_w : nullptr;
  s.state_in_mem = io.state_in_mem;
  s.state_in_cnt = io.state_in_cnt;
  s.state_out_mem = io.state_out_mem;
  s.state_out_cnt = io.state_out_cnt;
  s.r_out = io.r_out;
  s.r_stride = io.r_stride;
  s.read_out = io.read_out;
  s.den_out = dims->read_mean ? io.den_out : nullptr;
  s.sync = sync;
  s.xch = xch;
  s.S = p.B * p.H;
  s.T = p.T;
  s.H = p.H;
  s.dh = p.dh;
  s.M = p.M;
  s.n_chunks = p.n_chunks;
  s.groups = p.dh / cw;
  s.sync_stride = p.groups;
  // direct copies of the value rows into LDS move 16-byte pieces: rows and the column groups in them aligned to 16
  s.v_direct = reinterpret_cast<uintptr_t>(io.v) % 16 == 0 && (static_cast<size_t>(io.v_stride) * vb) % 16 == 0 &&
               (static_cast<size_t>(p.dh) * vb) % 16 == 0 && (cw * vb) % 16 == 0;
  if (pick)   // the pick scan loads four values at a time
    s.v_direct = reinterpret_cast<uintptr_t>(io.v) % (4 * vb) == 0 && io.v_stride % 4 == 0;
  s.spin_limit = wait_limit();
  s.crowded_bytes = crowded_threshold();
  s.read_mean = dims->read_mean;
  s.read_eps = dims->read_eps;
  s.out_eps = dims->out_norm_eps;
  if (pick)
    return io.in_dtype == SDM_RT_BF16 ? launch_pick_scan_bf16(p, s, io.out_dtype, st)
                                      : launch_pick_scan_f32(p, s, io.out_dtype, st);
  return io.in_dtype == SDM_RT_BF16 ? launch_scan_bf16(p, s, io.out_dtype, st) : launch_scan_f32(p, s, io.out_dtype, st);
}

}  // namespace sdmrt

using namespace sdmrt;

extern "C" {

size_t sdm_rt_workspace_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  return p.total;
}

size_t sdm_rt_gate_copy_offset(const sdm_rt_dims* dims) {
  Plan p;
  if (!dims || !dims->write_gate || make_plan(dims, &p) != SDM_RT_OK) return 0;
  return p.off_gate;
}

void sdm_rt_set_wait_limit(int64_t polls) {
  g_wait_limit.store(polls < 0 ? kSpinLimit : static_cast<uint32_t>(std::min<int64_t>(polls, 0xffffffffll)),
                     std::memory_order_relaxed);
}

void sdm_rt_set_crowded_threshold(int32_t bytes) {
  g_crowded_bytes.store(bytes < 0 ? kVarStage : bytes, std::memory_order_relaxed);
}

int sdm_rt_status(const sdm_rt_dims* dims, const void* workspace, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hipStreamSynchronize(st) != hipSuccess) return set_err(SDM_RT_ELAUNCH, "stream synchronisation failed");
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  const unsigned char* ws = static_cast<const unsigned char*>(workspace);
  if (!ws && (rc = scratch_ptr(reinterpret_cast<void**>(const_cast<unsigned char**>(&ws))))) return rc;
  uint32_t word = 0;
  if (hipMemcpy(&word, ws + status_offset(p), sizeof(word), hipMemcpyDeviceToHost) != hipSuccess)
    return set_err(SDM_RT_ELAUNCH, "reading the status word failed");
  if (word)
    return set_err(SDM_RT_ETIMEOUT,
                   "the scan's wait for the other column groups of a slab gave up: the read-outs of that chunk are "
                   "NaN (were the slab's workgroups not all resident, e.g. beside another call filling the GPU?)");
  return SDM_RT_OK;
}

int32_t sdm_rt_pick_pitch(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p, false) != SDM_RT_OK) return 0;
  return p.pitch;
}

int sdm_rt_forward(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                   const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, const uint8_t* reset,
                   void* r_out, int64_t out_row_stride, sdm_rt_dtype out_dtype, const float* state_in_mem,
                   const float* state_in_cnt, float* state_out_mem, float* state_out_cnt, void* workspace,
                   size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if ((rc = check_params(params, dims->out_norm != 0))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  const bool empty = p.B == 0 || p.T == 0;
  if (!empty && (!kz || !qz || !v || !r_out))
    return set_err(SDM_RT_EINVAL, "kz, qz, v and r_out must not be NULL");
  if (!empty && dims->write_gate && !gate_logits)
    return set_err(SDM_RT_EINVAL, "write_gate is set but gate_logits is NULL");
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
  if ((state_in_mem == nullptr) != (state_in_cnt == nullptr))
    return set_err(SDM_RT_EINVAL, "state_in_mem and state_in_cnt must both be given or both be NULL");
  if ((state_out_mem == nullptr) != (state_out_cnt == nullptr))
    return set_err(SDM_RT_EINVAL, "state_out_mem and state_out_cnt must both be given or both be NULL");
  if (!empty && (!workspace || workspace_bytes < p.total))
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, p.total);
  if (p.B == 0) return SDM_RT_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.T == 0) {   // no positions: the state out is the state in (or empty)
    if (state_out_mem) {
      const int64_t n_cnt = static_cast<int64_t>(p.B) * p.H * p.M;
      if ((rc = state_copy(state_out_mem, state_in_mem, n_cnt * p.dh, st))) return rc;
      if ((rc = state_copy(state_out_cnt, state_in_cnt, n_cnt, st))) return rc;
    }
    return SDM_RT_OK;
  }
  CoreIO io{};
  io.kz = kz;
  io.kz_stride = kz_row_stride;
  io.qz = qz;
  io.qz_stride = qz_row_stride;
  io.v = v;
  io.v_stride = v_row_stride;
  io.gate_logits = gate_logits;
  io.g_stride = gate_row_stride;
  io.in_dtype = in_dtype;
  io.reset = reset;
  io.r_out = r_out;
  io.r_stride = out_row_stride;
  io.out_dtype = out_dtype;
  io.state_in_mem = state_in_mem;
  io.state_in_cnt = state_in_cnt;
  io.state_out_mem = state_out_mem;
  io.state_out_cnt = state_out_cnt;
  return run_core(p, dims, params, io, workspace, st);
}

}  // extern "C"
