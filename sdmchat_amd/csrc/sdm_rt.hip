// sdm_rt.hip -- HIP kernels for gfx950 and the C ABI declared in include/sdm_rt.h.
//
// Kernels (one forward = keynorm, address x2 address sets, scan, finish):
//   keynorm_kernel   unit-normalise every sub-key once per call (F.normalize of keys, track4_onesdm_models.py:137-140)
//   address_kernel   per (token, head, address set): unit halves, scores against the n_sub unit sub-keys, exact
//                    top-c1 per half, exact top-kk of the dominance-pruned c1 x c1 grid, softmax weights, gate
//                    (pk_address :134-148, prepare :203-207)
//   scan_kernel      per (batch row, head, group of 8 value columns): the memory slab of M x 8 float32 columns
//                    plus the M write counts lives in LDS for the whole sequence; positions are processed 64 at
//                    a time (one per lane): read the carried state, add the in-chunk earlier writes found through
//                    per-location lists, then fold the chunk's faded writes into the slab (_chunk :215-241)
//   finish_kernel    per (token, head): r * rsqrt(mean(r^2) + eps) * onorm_w (finish :243-246)
//
// Decay bookkeeping in scan_kernel: the slab holds A with the true state S = mu * A (mu a per-slab scalar).  A chunk
// of L positions reads mu * lam^p * A[slot] at offset p, then mu <- mu * lam^L and each write at offset q adds
// lam^(L-1-q) / mu * w * v.  When mu falls below 2^-60 the slab is multiplied by mu once and mu reset to 1, so the
// slab is only rescaled about once every 60 / -log2(lam^64) chunks (never, at T = 2048, for lam >= 0.97) and
// lam = 0 (keep only the previous write) and lam = 1 (never fade) are exact.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "sdm_rt.h"

namespace {

// ---------------------------------------------------------------------------------------------------------------
// error reporting
thread_local char g_err[512] = "";

int set_err(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// ---------------------------------------------------------------------------------------------------------------
// element types: bfloat16 is carried as its 16 raw bits
struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(static_cast<uint32_t>(x.bits) << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  // round to nearest even, quiet NaN preserved
  uint32_t u = __float_as_uint(x);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
  }
  return r;
}

constexpr float kMuFloor = 8.673617379884035e-19f;  // 2^-60

// ---------------------------------------------------------------------------------------------------------------
// keynorm: out[s][:] = keys[s][:] / max(||keys[s]||, 1e-12) for the 2 * H * n_sub sub-keys
__global__ void keynorm_kernel(const float* __restrict__ keys1, const float* __restrict__ keys2,
                               float* __restrict__ out, int rows_per_set, int half) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= 2 * rows_per_set) return;
  const float* src = (r < rows_per_set ? keys1 + static_cast<int64_t>(r) * half
                                       : keys2 + static_cast<int64_t>(r - rows_per_set) * half);
  float ss = 0.f;
  for (int d = 0; d < half; ++d) ss = fmaf(src[d], src[d], ss);
  const float n = fmaxf(sqrtf(ss), 1e-12f);
  for (int d = 0; d < half; ++d) out[static_cast<int64_t>(r) * half + d] = src[d] / n;
}

// ---------------------------------------------------------------------------------------------------------------
// sorted top list in registers: v[0] >= v[1] >= ...; an incoming value moves ahead of an entry only when strictly
// greater, so among equal values the one inserted first (the lower index, as candidates arrive in index order)
// stays ahead.  Only the first `cnt` entries are live.
template <int CAP>
__device__ __forceinline__ void top_insert(float (&v)[CAP], int (&ix)[CAP], float x, int xi, int cnt) {
  bool gt[CAP];
#pragma unroll
  for (int p = 0; p < CAP; ++p) gt[p] = (p < cnt) && (x > v[p]);
#pragma unroll
  for (int p = CAP - 1; p >= 1; --p) {
    if (gt[p]) {
      v[p] = gt[p - 1] ? v[p - 1] : x;
      ix[p] = gt[p - 1] ? ix[p - 1] : xi;
    }
  }
  if (gt[0]) {
    v[0] = x;
    ix[0] = xi;
  }
}

struct AddrArgs {
  const void* z[2];           // address rows of the two sets (0: write keys, 1: read queries)
  int64_t z_stride[2];
  const void* g;              // gate logit rows or nullptr (applies to set 0 only)
  int64_t g_stride;
  const float* gate_bias;     // [H] or nullptr
  const float* knorm;         // [2][H][n_sub][half] unit sub-keys
  const float* addr_b;        // [H][d_a] or nullptr
  const float* log_scale;     // [H]
  int B, T, H, n_sub, c1, kk, pitch;
  // outputs, layout [B][H][T][pitch] per set
  uint16_t* idx16[2];
  int32_t* idx32[2];
  float* w_out[2];
  float* s_out[2];
};

// One thread per (token, head, set).  Grid: x = token tiles of 64, y = head, z = set.  Block = one wave, so the
// head and set are uniform and the sub-key reads are scalar loads.
template <int HALF, int CAP, typename InT>
__global__ void __launch_bounds__(64) address_kernel(AddrArgs a) {
  const int set = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t N = static_cast<int64_t>(a.B) * a.T;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  if (a.z[set] == nullptr || n >= N) return;
  constexpr int DA = 2 * HALF;

  const InT* zrow = static_cast<const InT*>(a.z[set]) + n * a.z_stride[set] + static_cast<int64_t>(h) * DA;
  float z[DA];
#pragma unroll
  for (int d = 0; d < DA; ++d) {
    const float bias = a.addr_b ? a.addr_b[h * DA + d] : 0.f;
    z[d] = to_f32(zrow[d]) + bias;
  }

  float hv[2][CAP];
  int hi[2][CAP];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    float u[HALF];
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < HALF; ++d) ss = fmaf(z[part * HALF + d], z[part * HALF + d], ss);
    const float nrm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int d = 0; d < HALF; ++d) u[d] = z[part * HALF + d] / nrm;
#pragma unroll
    for (int p = 0; p < CAP; ++p) {
      hv[part][p] = -INFINITY;
      hi[part][p] = 0;
    }
    const float* kb = a.knorm + (static_cast<int64_t>(part) * a.H + h) * a.n_sub * HALF;
    for (int s = 0; s < a.n_sub; ++s) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < HALF; ++d) acc = fmaf(u[d], kb[s * HALF + d], acc);
      top_insert<CAP>(hv[part], hi[part], acc, s, a.c1);
    }
  }

  // Combine: (a, b) can be among the kk best only when fewer than kk pairs dominate it, i.e. (a+1)(b+1) <= kk
  // (a dominating pair has a score >= and a lower flat index a * c1 + b).
  float cv[CAP];
  int ci[CAP];
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    cv[p] = -INFINITY;
    ci[p] = 0;
  }
#pragma unroll
  for (int ra = 0; ra < CAP; ++ra) {
    if (ra < a.c1) {
#pragma unroll
      for (int rb = 0; rb < CAP; ++rb) {
        if (rb < a.c1 && (ra + 1) * (rb + 1) <= a.kk) {
          const float s = (hv[0][ra] + hv[1][rb]) * 0.5f;
          top_insert<CAP>(cv, ci, s, ra * a.c1 + rb, a.kk);
        }
      }
    }
  }

  // softmax(exp(log_scale) * score) over the kk picks; the first pick holds the maximum
  const float scale = expf(a.log_scale[h]);
  float e[CAP];
  const float x0 = cv[0] * scale;
  float sum = 0.f;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    e[p] = (p < a.kk) ? expf(cv[p] * scale - x0) : 0.f;
    sum += e[p];
  }
  float gate = 1.f;
  if (set == 0 && a.g != nullptr) {
    const InT* grow = static_cast<const InT*>(a.g) + n * a.g_stride;
    const float logit = to_f32(grow[h]) + (a.gate_bias ? a.gate_bias[h] : 0.f);
    gate = 1.f / (1.f + expf(-logit));
  }

  const int b = static_cast<int>(n / a.T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * a.T);
  const int64_t base = ((static_cast<int64_t>(b) * a.H + h) * a.T + t) * a.pitch;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    if (p < a.pitch) {
      const bool live = p < a.kk;
      int slot = -1;
      if (live) {
        const int ra = ci[p] / a.c1;
        const int rb = ci[p] - ra * a.c1;
        int i1 = 0, i2 = 0;
#pragma unroll
        for (int q = 0; q < CAP; ++q) {
          if (q == ra) i1 = hi[0][q];
          if (q == rb) i2 = hi[1][q];
        }
        slot = i1 * a.n_sub + i2;
      }
      if (a.idx16[set]) a.idx16[set][base + p] = static_cast<uint16_t>(live ? slot : 0);
      if (a.idx32[set]) a.idx32[set][base + p] = slot;
      if (a.w_out[set]) a.w_out[set][base + p] = live ? e[p] / sum * gate : 0.f;
      if (a.s_out[set]) a.s_out[set][base + p] = live ? cv[p] : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// scan
struct ScanArgs {
  const uint16_t* idx_w;   // [B][H][T][KP]
  const uint16_t* idx_r;
  const float* w_w;
  const float* w_r;
  const void* v;           // value rows
  int64_t v_stride;
  const float* decay;      // [H]
  const float* state_in_mem;   // [B][H][M][dh] or nullptr
  const float* state_in_cnt;   // [B][H][M] or nullptr
  float* state_out_mem;
  float* state_out_cnt;
  void* r_out;             // rows of H * dh; OutT
  int64_t r_stride;
  int B, T, H, dh, M, kk, read_mean;
  float read_eps;
};

constexpr int kCols = 8;     // value columns per workgroup
constexpr int kChunk = 64;   // positions per chunk = lanes

// LDS layout (floats / ints): A[M][8], cnt[M], head[M], nxt[64*KP], wq[64*KP], vc[64][8]
__host__ __device__ inline size_t scan_lds_bytes(int M, int KP) {
  return sizeof(float) * (static_cast<size_t>(M) * kCols + M) + sizeof(int) * M +
         (sizeof(int) + sizeof(float)) * kChunk * KP + sizeof(float) * kChunk * kCols;
}

template <int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(64) scan_kernel(ScanArgs a) {
  extern __shared__ float lds[];
  const int M = a.M;
  float* A = lds;                                  // [M][8]
  float* cnt = A + static_cast<size_t>(M) * kCols; // [M]
  int* head = reinterpret_cast<int*>(cnt + M);     // [M]
  int* nxt = head + M;                             // [64*KP]
  float* wq = reinterpret_cast<float*>(nxt + kChunk * KP);  // [64*KP]
  float* vc = wq + kChunk * KP;                    // [64][8]

  const int cg = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x;
  const int col0 = cg * kCols;
  const int64_t slab = static_cast<int64_t>(b) * a.H + h;
  const float lam = a.decay[h];

  for (int m = lane; m < M; m += kChunk) {
#pragma unroll
    for (int c = 0; c < kCols; ++c)
      A[m * kCols + c] = a.state_in_mem ? a.state_in_mem[(slab * M + m) * a.dh + col0 + c] : 0.f;
    cnt[m] = a.state_in_cnt ? a.state_in_cnt[slab * M + m] : 0.f;
    head[m] = -1;
  }
  float mu = 1.f;
  __syncthreads();

  for (int c0 = 0; c0 < a.T; c0 += kChunk) {
    const int L = min(kChunk, a.T - c0);
    const bool active = lane < L;
    const int t = c0 + lane;

    int iw[KP], ir[KP];
    float ww[KP], wr[KP], v[kCols];
    if (active) {
      const int64_t pb = (slab * a.T + t) * KP;
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        iw[j] = a.idx_w[pb + j];
        ir[j] = a.idx_r[pb + j];
        ww[j] = a.w_w[pb + j];
        wr[j] = a.w_r[pb + j];
      }
      const VT* vrow = static_cast<const VT*>(a.v) + (static_cast<int64_t>(b) * a.T + t) * a.v_stride +
                       static_cast<int64_t>(h) * a.dh + col0;
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        v[c] = to_f32(vrow[c]);
        vc[lane * kCols + c] = v[c];
      }
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < a.kk) {
          const int e = lane * KP + j;
          nxt[e] = atomicExch(&head[iw[j]], e);
          wq[e] = ww[j];
        }
      }
    }
    __syncthreads();

    if (active) {
      float acc[kCols];
      float dacc = 0.f;
#pragma unroll
      for (int c = 0; c < kCols; ++c) acc[c] = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        if (i < a.kk) {
          const float* row = A + ir[i] * kCols;
#pragma unroll
          for (int c = 0; c < kCols; ++c) acc[c] = fmaf(wr[i], row[c], acc[c]);
          dacc = fmaf(wr[i], cnt[ir[i]], dacc);
        }
      }
      const float fin = mu * powf(lam, static_cast<float>(lane));
#pragma unroll
      for (int c = 0; c < kCols; ++c) acc[c] *= fin;
      dacc *= fin;
      // writes earlier in this chunk to the same locations, faded lam^(p-1-q)
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        if (i < a.kk) {
          int e = head[ir[i]];
          while (e >= 0) {
            const int q = e / KP;
            if (q < lane) {
              const float f = wr[i] * wq[e] * powf(lam, static_cast<float>(lane - 1 - q));
#pragma unroll
              for (int c = 0; c < kCols; ++c) acc[c] = fmaf(f, vc[q * kCols + c], acc[c]);
              dacc += f;
            }
            e = nxt[e];
          }
        }
      }
      OutT* orow = static_cast<OutT*>(a.r_out) + (static_cast<int64_t>(b) * a.T + t) * a.r_stride +
                   static_cast<int64_t>(h) * a.dh + col0;
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        const float r = a.read_mean ? acc[c] / (dacc + a.read_eps) : acc[c];
        orow[c] = from_f32<OutT>(r);
      }
    }
    __syncthreads();

    float mu_new = mu * powf(lam, static_cast<float>(L));
    if (!(mu_new >= kMuFloor)) {
      for (int m = lane; m < M; m += kChunk) {
#pragma unroll
        for (int c = 0; c < kCols; ++c) A[m * kCols + c] *= mu_new;
        cnt[m] *= mu_new;
      }
      mu_new = 1.f;
      __syncthreads();
    }
    if (active) {
      const float cw = powf(lam, static_cast<float>(L - 1 - lane)) / mu_new;
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < a.kk) {
          const float f = cw * ww[j];
          float* row = A + iw[j] * kCols;
#pragma unroll
          for (int c = 0; c < kCols; ++c) atomicAdd(&row[c], f * v[c]);
          atomicAdd(&cnt[iw[j]], f);
        }
      }
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int j = 0; j < KP; ++j)
        if (j < a.kk) head[iw[j]] = -1;
    }
    mu = mu_new;
    __syncthreads();
  }

  if (a.state_out_mem) {
    for (int m = lane; m < M; m += kChunk) {
#pragma unroll
      for (int c = 0; c < kCols; ++c) a.state_out_mem[(slab * M + m) * a.dh + col0 + c] = mu * A[m * kCols + c];
    }
  }
  if (a.state_out_cnt && cg == 0) {
    for (int m = lane; m < M; m += kChunk) a.state_out_cnt[slab * M + m] = mu * cnt[m];
  }
}

// ---------------------------------------------------------------------------------------------------------------
// finish: one wave per (token, head) row of dh float32 read-outs
template <typename OutT>
__global__ void __launch_bounds__(256) finish_kernel(const float* __restrict__ r, int64_t r_stride,
                                                     OutT* __restrict__ out, int64_t out_stride,
                                                     const float* __restrict__ onorm_w, int64_t rows, int H,
                                                     int dh, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t n = row / H;
  const int h = static_cast<int>(row - n * H);
  const float* src = r + n * r_stride + static_cast<int64_t>(h) * dh;
  float ss = 0.f;
  for (int d = lane; d < dh; d += 64) ss = fmaf(src[d], src[d], ss);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(dh) + eps);
  OutT* dst = out + n * out_stride + static_cast<int64_t>(h) * dh;
  for (int d = lane; d < dh; d += 64) dst[d] = from_f32<OutT>(src[d] * inv * onorm_w[h * dh + d]);
}

// ---------------------------------------------------------------------------------------------------------------
// host side
struct Plan {
  int B, T, H, dh, d_a, half, n_sub, M, k, c1, kk, pitch, cap;
  // workspace offsets
  size_t off_knorm, off_iw, off_ir, off_ww, off_wr, off_rtmp, total;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int make_plan(const sdm_rt_dims* d, Plan* p) {
  if (!d) return set_err(SDM_RT_EINVAL, "dims is NULL");
  if (d->batch < 0 || d->seq_len < 0) return set_err(SDM_RT_EINVAL, "negative batch or seq_len");
  if (d->heads < 1) return set_err(SDM_RT_EINVAL, "heads must be >= 1");
  if (d->head_dim < 8 || d->head_dim % 8 != 0)
    return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d must be a positive multiple of 8", d->head_dim);
  if (d->addr_dim < 2 || d->addr_dim % 2 != 0) return set_err(SDM_RT_EINVAL, "addr_dim %d must be even", d->addr_dim);
  if (d->n_sub < 1) return set_err(SDM_RT_EINVAL, "n_sub must be >= 1");
  if (d->top_k < 1) return set_err(SDM_RT_EINVAL, "top_k must be >= 1");
  p->B = d->batch;
  p->T = d->seq_len;
  p->H = d->heads;
  p->dh = d->head_dim;
  p->d_a = d->addr_dim;
  p->half = d->addr_dim / 2;
  p->n_sub = d->n_sub;
  p->M = d->n_sub * d->n_sub;
  p->k = d->top_k;
  p->c1 = d->top_k < d->n_sub ? d->top_k : d->n_sub;
  p->kk = d->top_k < p->c1 * p->c1 ? d->top_k : p->c1 * p->c1;
  if (p->c1 > 16 || p->kk > 16)
    return set_err(SDM_RT_EUNSUPPORTED, "min(k, n_sub) = %d and picks %d must be <= 16", p->c1, p->kk);
  if (p->M > 65535) return set_err(SDM_RT_EUNSUPPORTED, "n_sub^2 = %d locations exceed 65535", p->M);
  p->cap = p->c1 <= 8 && p->kk <= 8 ? 8 : 16;
  p->pitch = (p->kk + 7) / 8 * 8;
  const size_t tok = static_cast<size_t>(p->B) * p->T;
  const size_t picks = tok * p->H * p->pitch;
  size_t o = 0;
  p->off_knorm = o;
  o = align_up(o + sizeof(float) * 2 * p->H * p->n_sub * p->half, 256);
  p->off_iw = o;
  o = align_up(o + sizeof(uint16_t) * picks, 256);
  p->off_ir = o;
  o = align_up(o + sizeof(uint16_t) * picks, 256);
  p->off_ww = o;
  o = align_up(o + sizeof(float) * picks, 256);
  p->off_wr = o;
  o = align_up(o + sizeof(float) * picks, 256);
  p->off_rtmp = o;
  o = align_up(o + (d->out_norm ? sizeof(float) * tok * p->H * p->dh : 0), 256);
  p->total = o;
  return SDM_RT_OK;
}

bool aligned(const void* ptr, size_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_err(SDM_RT_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return SDM_RT_OK;
}

int launch_keynorm(const Plan& p, const sdm_rt_params* prm, float* knorm, hipStream_t st) {
  const int rows = p.H * p.n_sub;
  const int threads = 128;
  const int blocks = (2 * rows + threads - 1) / threads;
  hipLaunchKernelGGL(keynorm_kernel, dim3(blocks), dim3(threads), 0, st, prm->keys1, prm->keys2, knorm, rows, p.half);
  return check_launch("keynorm");
}

template <int HALF, int CAP, typename InT>
void launch_address_t(const Plan& p, const AddrArgs& a, int sets, hipStream_t st) {
  const int64_t N = static_cast<int64_t>(p.B) * p.T;
  dim3 grid(static_cast<unsigned>((N + 63) / 64), p.H, sets);
  hipLaunchKernelGGL((address_kernel<HALF, CAP, InT>), grid, dim3(64), 0, st, a);
}

template <int HALF, typename InT>
int launch_address_h(const Plan& p, const AddrArgs& a, int sets, hipStream_t st) {
  if (p.cap == 8)
    launch_address_t<HALF, 8, InT>(p, a, sets, st);
  else
    launch_address_t<HALF, 16, InT>(p, a, sets, st);
  return check_launch("address");
}

template <typename InT>
int launch_address_d(const Plan& p, const AddrArgs& a, int sets, hipStream_t st) {
  switch (p.half) {
    case 1: return launch_address_h<1, InT>(p, a, sets, st);
    case 2: return launch_address_h<2, InT>(p, a, sets, st);
    case 3: return launch_address_h<3, InT>(p, a, sets, st);
    case 4: return launch_address_h<4, InT>(p, a, sets, st);
    case 6: return launch_address_h<6, InT>(p, a, sets, st);
    case 8: return launch_address_h<8, InT>(p, a, sets, st);
    case 12: return launch_address_h<12, InT>(p, a, sets, st);
    case 16: return launch_address_h<16, InT>(p, a, sets, st);
    case 24: return launch_address_h<24, InT>(p, a, sets, st);
    case 32: return launch_address_h<32, InT>(p, a, sets, st);
    default:
      return set_err(SDM_RT_EUNSUPPORTED, "addr_dim %d: half width must be one of 1,2,3,4,6,8,12,16,24,32", p.d_a);
  }
}

int launch_address(const Plan& p, const AddrArgs& a, int sets, sdm_rt_dtype dt, hipStream_t st) {
  return dt == SDM_RT_BF16 ? launch_address_d<bf16_t>(p, a, sets, st) : launch_address_d<float>(p, a, sets, st);
}

template <int KP, typename VT, typename OutT>
int launch_scan_t(const Plan& p, const ScanArgs& a, hipStream_t st) {
  const size_t lds = scan_lds_bytes(p.M, KP);
  dim3 grid(p.dh / kCols, p.H, p.B);
  hipLaunchKernelGGL((scan_kernel<KP, VT, OutT>), grid, dim3(kChunk), lds, st, a);
  return check_launch("scan");
}

template <typename VT, typename OutT>
int launch_scan_v(const Plan& p, const ScanArgs& a, hipStream_t st) {
  return p.pitch == 8 ? launch_scan_t<8, VT, OutT>(p, a, st) : launch_scan_t<16, VT, OutT>(p, a, st);
}

int launch_scan(const Plan& p, const ScanArgs& a, sdm_rt_dtype vt, sdm_rt_dtype ot, hipStream_t st) {
  if (vt == SDM_RT_BF16) {
    return ot == SDM_RT_BF16 ? launch_scan_v<bf16_t, bf16_t>(p, a, st) : launch_scan_v<bf16_t, float>(p, a, st);
  }
  return ot == SDM_RT_BF16 ? launch_scan_v<float, bf16_t>(p, a, st) : launch_scan_v<float, float>(p, a, st);
}

int check_dtype(sdm_rt_dtype t, const char* what) {
  if (t != SDM_RT_F32 && t != SDM_RT_BF16) return set_err(SDM_RT_EINVAL, "%s: unknown dtype %d", what, (int)t);
  return SDM_RT_OK;
}

int check_params(const Plan& p, const sdm_rt_params* prm, bool need_onorm) {
  if (!prm) return set_err(SDM_RT_EINVAL, "params is NULL");
  if (!prm->keys1 || !prm->keys2) return set_err(SDM_RT_EINVAL, "keys1/keys2 must not be NULL");
  if (!prm->log_scale) return set_err(SDM_RT_EINVAL, "log_scale must not be NULL");
  if (!prm->decay) return set_err(SDM_RT_EINVAL, "decay must not be NULL");
  if (need_onorm && !prm->onorm_w) return set_err(SDM_RT_EINVAL, "onorm_w must not be NULL when out_norm is set");
  (void)p;
  return SDM_RT_OK;
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// C ABI
extern "C" {

size_t sdm_rt_workspace_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  return p.total;
}

int32_t sdm_rt_pick_pitch(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  return p.pitch;
}

const char* sdm_rt_last_error(void) { return g_err; }

int sdm_rt_address(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* z, int64_t z_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, int32_t* slot_out,
                   float* score_out, float* weight_out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if ((rc = check_params(p, params, false))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!z || !slot_out) return set_err(SDM_RT_EINVAL, "z and slot_out must not be NULL");
  if (z_row_stride < static_cast<int64_t>(p.H) * p.d_a)
    return set_err(SDM_RT_EINVAL, "z_row_stride %lld < heads * addr_dim", (long long)z_row_stride);
  if (gate_logits && gate_row_stride < p.H)
    return set_err(SDM_RT_EINVAL, "gate_row_stride %lld < heads", (long long)gate_row_stride);
  if (!workspace || workspace_bytes < p.total)
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, p.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* knorm = reinterpret_cast<float*>(ws + p.off_knorm);
  if ((rc = launch_keynorm(p, params, knorm, st))) return rc;
  AddrArgs a{};
  a.z[0] = z;
  a.z[1] = nullptr;
  a.z_stride[0] = z_row_stride;
  a.g = gate_logits;
  a.g_stride = gate_row_stride;
  a.gate_bias = params->gate_bias;
  a.knorm = knorm;
  a.addr_b = params->addr_b;
  a.log_scale = params->log_scale;
  a.B = p.B;
  a.T = p.T;
  a.H = p.H;
  a.n_sub = p.n_sub;
  a.c1 = p.c1;
  a.kk = p.kk;
  a.pitch = p.pitch;
  a.idx32[0] = slot_out;
  a.w_out[0] = weight_out;
  a.s_out[0] = score_out;
  return launch_address(p, a, 1, in_dtype, st);
}

int sdm_rt_forward(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                   const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, void* r_out,
                   int64_t out_row_stride, sdm_rt_dtype out_dtype, const float* state_in_mem,
                   const float* state_in_cnt, float* state_out_mem, float* state_out_cnt, void* workspace,
                   size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if ((rc = check_params(p, params, dims->out_norm != 0))) return rc;
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
  if (out_row_stride < static_cast<int64_t>(p.H) * p.dh)
    return set_err(SDM_RT_EINVAL, "out_row_stride %lld < heads * head_dim", (long long)out_row_stride);
  if ((state_in_mem == nullptr) != (state_in_cnt == nullptr))
    return set_err(SDM_RT_EINVAL, "state_in_mem and state_in_cnt must both be given or both be NULL");
  if ((state_out_mem == nullptr) != (state_out_cnt == nullptr))
    return set_err(SDM_RT_EINVAL, "state_out_mem and state_out_cnt must both be given or both be NULL");
  if (!empty && (!workspace || workspace_bytes < p.total))
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, p.total);
  const size_t lds = scan_lds_bytes(p.M, p.pitch);
  if (lds > 160 * 1024)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations need %zu bytes of LDS (> 160 KiB)", p.M, lds);
  if (p.B == 0) return SDM_RT_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.T == 0) {
    if (state_out_mem) {
      const size_t mem_b = sizeof(float) * p.B * p.H * static_cast<size_t>(p.M) * p.dh;
      const size_t cnt_b = sizeof(float) * p.B * p.H * static_cast<size_t>(p.M);
      hipError_t e1 = state_in_mem ? hipMemcpyAsync(state_out_mem, state_in_mem, mem_b, hipMemcpyDeviceToDevice, st)
                                   : hipMemsetAsync(state_out_mem, 0, mem_b, st);
      hipError_t e2 = state_in_cnt ? hipMemcpyAsync(state_out_cnt, state_in_cnt, cnt_b, hipMemcpyDeviceToDevice, st)
                                   : hipMemsetAsync(state_out_cnt, 0, cnt_b, st);
      if (e1 != hipSuccess || e2 != hipSuccess) return set_err(SDM_RT_ELAUNCH, "state copy failed");
    }
    return SDM_RT_OK;
  }
  char* ws = static_cast<char*>(workspace);
  float* knorm = reinterpret_cast<float*>(ws + p.off_knorm);
  uint16_t* iw = reinterpret_cast<uint16_t*>(ws + p.off_iw);
  uint16_t* ir = reinterpret_cast<uint16_t*>(ws + p.off_ir);
  float* w_w = reinterpret_cast<float*>(ws + p.off_ww);
  float* w_r = reinterpret_cast<float*>(ws + p.off_wr);
  float* rtmp = reinterpret_cast<float*>(ws + p.off_rtmp);

  if ((rc = launch_keynorm(p, params, knorm, st))) return rc;
  AddrArgs a{};
  a.z[0] = kz;
  a.z[1] = qz;
  a.z_stride[0] = kz_row_stride;
  a.z_stride[1] = qz_row_stride;
  a.g = dims->write_gate ? gate_logits : nullptr;
  a.g_stride = gate_row_stride;
  a.gate_bias = params->gate_bias;
  a.knorm = knorm;
  a.addr_b = params->addr_b;
  a.log_scale = params->log_scale;
  a.B = p.B;
  a.T = p.T;
  a.H = p.H;
  a.n_sub = p.n_sub;
  a.c1 = p.c1;
  a.kk = p.kk;
  a.pitch = p.pitch;
  a.idx16[0] = iw;
  a.idx16[1] = ir;
  a.w_out[0] = w_w;
  a.w_out[1] = w_r;
  if ((rc = launch_address(p, a, 2, in_dtype, st))) return rc;

  ScanArgs s{};
  s.idx_w = iw;
  s.idx_r = ir;
  s.w_w = w_w;
  s.w_r = w_r;
  s.v = v;
  s.v_stride = v_row_stride;
  s.decay = params->decay;
  s.state_in_mem = state_in_mem;
  s.state_in_cnt = state_in_cnt;
  s.state_out_mem = state_out_mem;
  s.state_out_cnt = state_out_cnt;
  s.B = p.B;
  s.T = p.T;
  s.H = p.H;
  s.dh = p.dh;
  s.M = p.M;
  s.kk = p.kk;
  s.read_mean = dims->read_mean;
  s.read_eps = dims->read_eps;
  if (dims->out_norm) {
    s.r_out = rtmp;
    s.r_stride = static_cast<int64_t>(p.H) * p.dh;
    if ((rc = launch_scan(p, s, in_dtype, SDM_RT_F32, st))) return rc;
    const int64_t rows = static_cast<int64_t>(p.B) * p.T * p.H;
    const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
    if (out_dtype == SDM_RT_BF16) {
      hipLaunchKernelGGL((finish_kernel<bf16_t>), dim3(blocks), dim3(256), 0, st, rtmp, s.r_stride,
                         static_cast<bf16_t*>(r_out), out_row_stride, params->onorm_w, rows, p.H, p.dh,
                         dims->out_norm_eps);
    } else {
      hipLaunchKernelGGL((finish_kernel<float>), dim3(blocks), dim3(256), 0, st, rtmp, s.r_stride,
                         static_cast<float*>(r_out), out_row_stride, params->onorm_w, rows, p.H, p.dh,
                         dims->out_norm_eps);
    }
    return check_launch("finish");
  }
  s.r_out = r_out;
  s.r_stride = out_row_stride;
  return launch_scan(p, s, in_dtype, out_dtype, st);
}

}  // extern "C"
