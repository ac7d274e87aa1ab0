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

constexpr int kChunk = 64;                 // positions per chunk (one bit each in the per-location writer masks)
constexpr size_t kLdsBytes = 160 * 1024;   // LDS per workgroup on gfx950
constexpr int kScanThreads = 512;          // 64 positions x 8 lanes
constexpr int kNoQ = 0x7f;                 // "no in-chunk writer" in the packed read flags

__host__ __device__ constexpr int pad4(int M) { return (M + 3) / 4 * 4; }

// LDS of one scan workgroup, in order: the slab A[M][CW] (CW value columns of every location), the write counts
// cnt[M], the writer masks of the current chunk wmask[M] (bit q: position q of the chunk writes the location);
// u16 [64][KP] arrays: picks s_iw / s_ir, packed read flags s_qf (first and second earlier in-chunk writer of the
// read pick, and a bit for "three or more"), write ranks s_rk (earlier in-chunk writers of the write pick's slot);
// f32 [64][KP]: weights s_ww / s_wr and the two in-chunk read coefficients s_c1 / s_c2; the staged values s_v[64][CW]
// (VT: bfloat16 inputs are staged exactly as bfloat16), denominators s_den[64], fade powers pw[68], and the
// largest write rank of the chunk.
__host__ __device__ constexpr size_t scan_lds_bytes(int M, int KP, int CW, int v_bytes) {
  return sizeof(float) * (static_cast<size_t>(M) * CW + pad4(M)) + sizeof(unsigned long long) * pad4(M) +
         sizeof(uint16_t) * 4 * kChunk * KP + sizeof(float) * 4 * kChunk * KP +
         static_cast<size_t>(v_bytes) * kChunk * CW + sizeof(float) * (kChunk + 68) + 16;
}

// The KP picks of one position: slot ids (16-bit) and weights, loaded with 128-bit LDS reads.
template <int KP>
__device__ __forceinline__ void load_picks(const uint16_t* sl, const float* wt, int (&m)[KP], float (&w)[KP]) {
#pragma unroll
  for (int g = 0; g < KP / 8; ++g) {
    const uint4 v = *reinterpret_cast<const uint4*>(sl + 8 * g);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m[8 * g + 2 * e] = static_cast<int>(u[e] & 0xffffu);
      m[8 * g + 2 * e + 1] = static_cast<int>(u[e] >> 16);
    }
  }
#pragma unroll
  for (int g = 0; g < KP / 4; ++g) {
    const float4 v = *reinterpret_cast<const float4*>(wt + 4 * g);
    w[4 * g] = v.x;
    w[4 * g + 1] = v.y;
    w[4 * g + 2] = v.z;
    w[4 * g + 3] = v.w;
  }
}

template <int KP>
__device__ __forceinline__ void load_u16(const uint16_t* sl, int (&m)[KP]) {
#pragma unroll
  for (int g = 0; g < KP / 8; ++g) {
    const uint4 v = *reinterpret_cast<const uint4*>(sl + 8 * g);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m[8 * g + 2 * e] = static_cast<int>(u[e] & 0xffffu);
      m[8 * g + 2 * e + 1] = static_cast<int>(u[e] >> 16);
    }
  }
}

template <int KP>
__device__ __forceinline__ void load_f32(const float* wt, float (&w)[KP]) {
#pragma unroll
  for (int g = 0; g < KP / 4; ++g) {
    const float4 v = *reinterpret_cast<const float4*>(wt + 4 * g);
    w[4 * g] = v.x;
    w[4 * g + 1] = v.y;
    w[4 * g + 2] = v.z;
    w[4 * g + 3] = v.w;
  }
}

// Weight with which position q (its KP slot ids sl and weights wt, the first kk live) wrote slot m (a position
// writes a slot at most once; 0 when it did not).
template <int KP>
__device__ __forceinline__ float writer_weight(const uint16_t* sl, const float* wt, int m, int kk) {
  int mq[KP];
  float wq[KP];
  load_picks<KP>(sl, wt, mq, wq);
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < KP; ++j) r = (j < kk && mq[j] == m) ? wq[j] : r;
  return r;
}

// CPL consecutive floats (CPL = 4, 2, 1) of LDS, one vector access; the bfloat16 variant converts.
template <int CPL>
struct Seg {
  float v[CPL];
};
template <int CPL>
__device__ __forceinline__ Seg<CPL> lds_seg(const float* p) {
  Seg<CPL> r;
  if constexpr (CPL == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
  } else if constexpr (CPL == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r.v[0] = t.x; r.v[1] = t.y;
  } else {
    r.v[0] = *p;
  }
  return r;
}
template <int CPL>
__device__ __forceinline__ Seg<CPL> lds_seg(const bf16_t* p) {
  Seg<CPL> r;
  if constexpr (CPL == 4) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    r.v[0] = __uint_as_float(t.x << 16); r.v[1] = __uint_as_float(t.x & 0xffff0000u);
    r.v[2] = __uint_as_float(t.y << 16); r.v[3] = __uint_as_float(t.y & 0xffff0000u);
  } else if constexpr (CPL == 2) {
    const uint32_t t = *reinterpret_cast<const uint32_t*>(p);
    r.v[0] = __uint_as_float(t << 16); r.v[1] = __uint_as_float(t & 0xffff0000u);
  } else {
    r.v[0] = to_f32(*p);
  }
  return r;
}
template <int CPL>
__device__ __forceinline__ void lds_seg_store(float* p, const Seg<CPL>& r) {
  if constexpr (CPL == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
  } else if constexpr (CPL == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(r.v[0], r.v[1]);
  } else {
    *p = r.v[0];
  }
}

template <typename OutT, int CPL>
__device__ __forceinline__ void store_seg(OutT* o, const float (&v)[CPL]) {
#pragma unroll
  for (int c = 0; c < CPL; ++c) o[c] = from_f32<OutT>(v[c]);
}

// Sum over the 8 consecutive lanes of a position (DPP: swap neighbours, swap pairs, mirror the halves of 8).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float sum8(float v) {
  v += dpp_f<0xb1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);    // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  return v;
}

// Workgroup barrier that orders LDS accesses only: the scan shares nothing else between its threads, so global loads
// issued ahead (the next chunk's picks) and global stores (read-outs) need not complete at every barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Scan of one (batch row, head) slab over CW of its value columns, 512 threads = 64 positions x 8 lanes.
// Per chunk of up to 64 positions, separated by barriers:
//   P1 stage   lane (position, pick): the chunk's picks and weights (loaded one chunk ahead) and CW/8 value columns
//              into LDS; first the previous chunk's writer marks made from the same entries are cleared
//   P2 mark    each write (q, j) sets bit q of wmask[slot]
//   P3 control lane (position, pick): the read pick's S_in count term, its first two earlier in-chunk writers and
//              their coefficients (a flag for more), the position's denominator (summed over its 8 lanes), and the
//              write pick's rank = number of earlier in-chunk writers of its slot
//   P4 read    lane (position, segment of CW/8 columns): mu * lam^p * S_in rows of the picks plus the in-chunk
//              writes, divided by the denominator
//   P5 write   in rounds r = 0, 1, ...: the writes of rank r add their faded value to their slot's row with one
//              128-bit read-modify-write per lane (no two writes of a round share a slot; no LDS float atomics)
// All sums are over fixed orders, so results are deterministic.
template <int CW, int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(kScanThreads) scan_kernel(ScanArgs a) {
  constexpr int CPL = CW / 8;   // value columns per data lane
  constexpr int G = KP / 8;     // picks per control lane
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int M = a.M;
  float* A = lds;
  float* cnt = A + static_cast<size_t>(M) * CW;
  unsigned long long* wmask = reinterpret_cast<unsigned long long*>(cnt + pad4(M));
  uint16_t* s_iw = reinterpret_cast<uint16_t*>(wmask + pad4(M));
  uint16_t* s_ir = s_iw + kChunk * KP;
  uint16_t* s_qf = s_ir + kChunk * KP;
  uint16_t* s_rk = s_qf + kChunk * KP;
  float* s_ww = reinterpret_cast<float*>(s_rk + kChunk * KP);
  float* s_wr = s_ww + kChunk * KP;
  float* s_c1 = s_wr + kChunk * KP;
  float* s_c2 = s_c1 + kChunk * KP;
  VT* s_v = reinterpret_cast<VT*>(s_c2 + kChunk * KP);
  float* s_den = reinterpret_cast<float*>(s_v + kChunk * CW);
  float* pw = s_den + kChunk;
  int* s_maxrank = reinterpret_cast<int*>(pw + 68);

  const int cg = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int p = tid >> 3;     // position in the chunk
  const int l8 = tid & 7;     // pick (control) or column segment (data)
  const int col0 = cg * CW;
  const int64_t slab = static_cast<int64_t>(b) * a.H + h;
  const float lam = a.decay[h];
  const int kk = a.kk;

  for (int i = tid; i < M * CW; i += kScanThreads) {
    const int m = i / CW;
    const int c = i - m * CW;
    A[i] = a.state_in_mem ? a.state_in_mem[(slab * M + m) * a.dh + col0 + c] : 0.f;
  }
  for (int m = tid; m < M; m += kScanThreads) {
    cnt[m] = a.state_in_cnt ? a.state_in_cnt[slab * M + m] : 0.f;
    wmask[m] = 0ull;
  }
  if (tid <= kChunk) {
    float v = 1.f;   // lam^tid by repeated multiplication (exact for lam = 0 and lam = 1)
    for (int e = 0; e < tid; ++e) v *= lam;
    pw[tid] = v;
  }
  float mu = 1.f;

  // this lane's picks (control role) and value columns (data role) of the next chunk, loaded one chunk ahead
  int n_iw[G], n_ir[G];
  float n_ww[G], n_wr[G];
  VT n_v[CPL];
  auto fetch = [&](int c0) {
    if (p < min(kChunk, a.T - c0)) {
      const int64_t pb = (slab * a.T + c0 + p) * KP;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int j = l8 + 8 * g;
        n_iw[g] = a.idx_w[pb + j];
        n_ir[g] = a.idx_r[pb + j];
        n_ww[g] = a.w_w[pb + j];
        n_wr[g] = a.w_r[pb + j];
      }
      const VT* vrow = static_cast<const VT*>(a.v) + (static_cast<int64_t>(b) * a.T + c0 + p) * a.v_stride +
                       static_cast<int64_t>(h) * a.dh + col0 + CPL * l8;
#pragma unroll
      for (int c = 0; c < CPL; ++c) n_v[c] = vrow[c];
    }
  };
  fetch(0);
  lds_barrier();

  for (int c0 = 0; c0 < a.T; c0 += kChunk) {
    const int L = min(kChunk, a.T - c0);
    const bool active = p < L;
    const int64_t row = static_cast<int64_t>(b) * a.T + c0 + p;
    int iw[G], ir[G];
    float ww[G], wr[G];
    float vreg[CPL];
    // P1: clear the previous chunk's marks made from this lane's entries, then stage
    if (c0 > 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int j = l8 + 8 * g;
        if (j < kk) wmask[s_iw[p * KP + j]] = 0ull;
      }
    }
    if (tid == 0) *s_maxrank = 0;
    if (active) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int j = l8 + 8 * g;
        iw[g] = n_iw[g];
        ir[g] = n_ir[g];
        ww[g] = n_ww[g];
        wr[g] = n_wr[g];
        s_iw[p * KP + j] = static_cast<uint16_t>(iw[g]);
        s_ir[p * KP + j] = static_cast<uint16_t>(ir[g]);
        s_ww[p * KP + j] = ww[g];
        s_wr[p * KP + j] = wr[g];
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        vreg[c] = to_f32(n_v[c]);
        s_v[p * CW + CPL * l8 + c] = n_v[c];
      }
    }
    lds_barrier();
    // P2: mark; then start loading the next chunk
    if (active) {
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (l8 + 8 * g < kk) atomicOr(&wmask[iw[g]], 1ull << p);
    }
    if (c0 + kChunk < a.T) fetch(c0 + kChunk);
    lds_barrier();
    // P3: control
    if (active) {
      const float fin = mu * pw[p];
      const unsigned long long below = (1ull << p) - 1ull;
      float dpart = 0.f;
      int myrank = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int i = l8 + 8 * g;
        uint32_t qf = kNoQ | (kNoQ << 7);
        uint16_t rk = 0;
        float c1 = 0.f, c2 = 0.f;
        if (i < kk) {
          const int m = ir[g];
          const float w = wr[g];
          dpart = fmaf(w * fin, cnt[m], dpart);
          unsigned long long mk = wmask[m] & below;
          if (mk) {
            const int q1 = __builtin_ctzll(mk);
            mk &= mk - 1ull;
            const int q2 = mk ? __builtin_ctzll(mk) : q1;
            const float w1 = writer_weight<KP>(s_iw + q1 * KP, s_ww + q1 * KP, m, kk);
            const float w2 = writer_weight<KP>(s_iw + q2 * KP, s_ww + q2 * KP, m, kk);
            c1 = w * w1 * pw[p - 1 - q1];
            dpart += c1;
            qf = q1 | (kNoQ << 7);
            if (mk) {
              c2 = w * w2 * pw[p - 1 - q2];
              dpart += c2;
              qf = q1 | (q2 << 7);
              mk &= mk - 1ull;
              if (mk) qf |= 1u << 14;
              while (mk) {   // three or more earlier writers: the rest only enters the denominator here
                const int q = __builtin_ctzll(mk);
                mk &= mk - 1ull;
                dpart += w * writer_weight<KP>(s_iw + q * KP, s_ww + q * KP, m, kk) * pw[p - 1 - q];
              }
            }
          }
          const unsigned long long mm = wmask[iw[g]] & below;
          rk = static_cast<uint16_t>(__builtin_popcountll(mm));
          myrank = max(myrank, static_cast<int>(rk));
        }
        s_qf[p * KP + i] = static_cast<uint16_t>(qf);
        s_c1[p * KP + i] = c1;
        s_c2[p * KP + i] = c2;
        s_rk[p * KP + i] = rk;
      }
      dpart = sum8(dpart);
      if (l8 == 0) s_den[p] = dpart;
      if (myrank > 0) atomicMax(s_maxrank, myrank);
    }
    lds_barrier();
    // P4: read
    if (active) {
      const float fin = mu * pw[p];
      int m[KP], qfl[KP];
      float w[KP], c1[KP], c2[KP];
      load_picks<KP>(s_ir + p * KP, s_wr + p * KP, m, w);
      load_u16<KP>(s_qf + p * KP, qfl);
      load_f32<KP>(s_c1 + p * KP, c1);
      load_f32<KP>(s_c2 + p * KP, c2);
      float acc[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c] = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i) {   // pad picks carry weight 0
        const Seg<CPL> x = lds_seg<CPL>(&A[m[i] * CW + CPL * l8]);
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[c] = fmaf(w[i], x.v[c], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c] *= fin;
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        const int q1 = qfl[i] & kNoQ;
        const int q2 = (qfl[i] >> 7) & kNoQ;
        if (q1 != kNoQ) {
          const Seg<CPL> v1 = lds_seg<CPL>(&s_v[q1 * CW + CPL * l8]);
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[c] = fmaf(c1[i], v1.v[c], acc[c]);
        }
        if (q2 != kNoQ) {
          const Seg<CPL> v2 = lds_seg<CPL>(&s_v[q2 * CW + CPL * l8]);
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[c] = fmaf(c2[i], v2.v[c], acc[c]);
        }
      }
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        if (!(qfl[i] & (1 << 14))) continue;   // three or more earlier writers (rare)
        unsigned long long mk = wmask[m[i]] & ((1ull << p) - 1ull);
        mk &= mk - 1ull;
        mk &= mk - 1ull;
        while (mk) {
          const int q = __builtin_ctzll(mk);
          mk &= mk - 1ull;
          const float coef = w[i] * writer_weight<KP>(s_iw + q * KP, s_ww + q * KP, m[i], kk) * pw[p - 1 - q];
          const Seg<CPL> vq = lds_seg<CPL>(&s_v[q * CW + CPL * l8]);
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[c] = fmaf(coef, vq.v[c], acc[c]);
        }
      }
      if (a.read_mean) {
        const float inv = 1.f / (s_den[p] + a.read_eps);
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[c] *= inv;
      }
      store_seg<OutT, CPL>(static_cast<OutT*>(a.r_out) + row * a.r_stride + static_cast<int64_t>(h) * a.dh + col0 +
                               CPL * l8, acc);
    }
    lds_barrier();
    // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small)
    float mu_new = mu * pw[L];
    if (!(mu_new >= kMuFloor)) {
      for (int i = tid; i < M * CW; i += kScanThreads) A[i] *= mu_new;
      for (int m = tid; m < M; m += kScanThreads) cnt[m] *= mu_new;
      mu_new = 1.f;
      lds_barrier();
    }
    // P5: write, in rounds of equal rank
    const int maxrank = *s_maxrank;
    {
      const float cpos = active ? pw[L - 1 - p] / mu_new : 0.f;
      int m[KP], rk[KP];
      float w[KP];
      if (active) {
        load_picks<KP>(s_iw + p * KP, s_ww + p * KP, m, w);
        load_u16<KP>(s_rk + p * KP, rk);
      }
      for (int r = 0; r <= maxrank; ++r) {
        if (active) {
          Seg<CPL> x[KP];
          float cc[KP];
#pragma unroll
          for (int j = 0; j < KP; ++j) {
            if (j < kk && rk[j] == r) {
              x[j] = lds_seg<CPL>(&A[m[j] * CW + CPL * l8]);
              if (l8 == 0) cc[j] = cnt[m[j]];
            }
          }
#pragma unroll
          for (int j = 0; j < KP; ++j) {
            if (j < kk && rk[j] == r) {
              const float cp = cpos * w[j];
#pragma unroll
              for (int c = 0; c < CPL; ++c) x[j].v[c] = fmaf(cp, vreg[c], x[j].v[c]);
              lds_seg_store<CPL>(&A[m[j] * CW + CPL * l8], x[j]);
              if (l8 == 0) cnt[m[j]] = cc[j] + cp;
            }
          }
        }
        lds_barrier();
      }
    }
    mu = mu_new;
  }

  if (a.state_out_mem) {
    for (int i = tid; i < M * CW; i += kScanThreads) {
      const int m = i / CW;
      const int c = i - m * CW;
      a.state_out_mem[(slab * M + m) * a.dh + col0 + c] = mu * A[i];
    }
  }
  if (a.state_out_cnt && cg == 0) {
    for (int m = tid; m < M; m += kScanThreads) a.state_out_cnt[slab * M + m] = mu * cnt[m];
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
  if (scan_lds_bytes(p->M, p->pitch, 8, sizeof(float)) > kLdsBytes)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations do not fit a slab of 8 columns in LDS", p->M);
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

template <int CW, int KP, typename VT, typename OutT>
int launch_scan_t(const Plan& p, const ScanArgs& a, hipStream_t st) {
  const size_t lds = scan_lds_bytes(p.M, KP, CW, sizeof(VT));
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<CW, KP, VT, OutT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     static_cast<int>(kLdsBytes));
  if (attr != hipSuccess) return set_err(SDM_RT_ELAUNCH, "scan: cannot enable %zu bytes of LDS", kLdsBytes);
  dim3 grid(p.dh / CW, p.H, p.B);
  hipLaunchKernelGGL((scan_kernel<CW, KP, VT, OutT>), grid, dim3(kScanThreads), lds, st, a);
  return check_launch("scan");
}

template <int CW, typename VT, typename OutT>
int launch_scan_k(const Plan& p, const ScanArgs& a, hipStream_t st) {
  return p.pitch == 8 ? launch_scan_t<CW, 8, VT, OutT>(p, a, st) : launch_scan_t<CW, 16, VT, OutT>(p, a, st);
}

// widest column group per scan workgroup (32, 16 or 8 value columns) whose slab and staging fit in LDS
template <typename VT>
int scan_columns(const Plan& p) {
  for (int cw : {32, 16, 8})
    if (p.dh % cw == 0 && scan_lds_bytes(p.M, p.pitch, cw, sizeof(VT)) <= kLdsBytes) return cw;
  return 0;
}

template <typename VT, typename OutT>
int launch_scan_v(const Plan& p, const ScanArgs& a, hipStream_t st) {
  switch (scan_columns<VT>(p)) {
    case 32: return launch_scan_k<32, VT, OutT>(p, a, st);
    case 16: return launch_scan_k<16, VT, OutT>(p, a, st);
    case 8: return launch_scan_k<8, VT, OutT>(p, a, st);
    default: return set_err(SDM_RT_EUNSUPPORTED, "no scan column group fits in LDS");
  }
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
