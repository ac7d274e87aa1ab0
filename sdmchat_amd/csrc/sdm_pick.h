// sdm_pick.h -- pick_scan_kernel: the scan of one (batch row, head) slab over a group of 32 of its value columns,
// executing pick plans (plan_kernel<..., PICK = true>), with the read-out finished in place (RunTimeSdm._chunk,
// forward and finish, experiments/track4/sdmllm/track4_onesdm_models.py:215-247 without wo).  It serves picks of at
// most 8, head_dim a multiple of 32 and slabs of at most 1,024 locations; scan_kernel (sdm_scan.h) serves the rest.
//
// Layout of the work: 1,024 threads, one per (position p, pick i, column half hh): lane u = tid % 16 of position
// p = tid / 16 holds b = u % 4, hh = (u / 4) % 2 and pick i = 2 b + u / 8.  A lane gathers the 16 columns of its
// half of its pick's slab row (four 16-byte LDS reads), scales them by the read weight, adds the in-chunk
// contribution the plan gave its record, and the eight pick lanes of the half then reduce-scatter the 16 sums
// (DPP: reverse within the quad, swap neighbours in the quad, lanes 8 apart), after which the lane holds columns
// 4 b + 2 (u / 8) and + 1 of its half.  The lane reads its four pieces (4 columns each) in the order b, b ^ 1,
// 3 - b, (3 - b) ^ 1 of its half, which the reduction consumes without any register selects above the last stage,
// and eight consecutive lanes then read eight different 16-byte pieces (all 32 banks) at every read.
// The write of a chunk is done by the owner lanes: the lane of pick j owns the slot if its position is the first
// writer of the slot the chunk keeps; it adds its faded value and those of the slot's later writers in the chunk to
// the slot's row (read, add, write back: each slot has one owner, so the sums run in a fixed order and the result
// is deterministic).
// Records, the chunk's value rows and the variable part of its plan (contributions and later writers beyond the
// first) are loaded into registers one chunk ahead; rows and variable part are stored into LDS at the end of the
// previous chunk.  Decay bookkeeping, the out-norm exchange between the column groups of a slab and the
// reset handling are those of scan_kernel (sdm_scan.h).
#pragma once

#include "sdm_scan.h"

namespace sdmrt {

constexpr int kPickThreads = 1024;   // 64 positions x 8 picks x 2 column halves
constexpr int kPickCols = 32;        // value columns per workgroup

// LDS of one pick scan workgroup: the slab A[M + 1][32] and counts cnt[M + 1], by chunk parity two buffers of the
// chunk's value rows [64][32] (float32, whatever the value type) and of its staged variable part, the fade powers
// pw[68] and the variable-part sizes of the n_chunks plans
__host__ __device__ constexpr size_t pick_lds_bytes(int M, int n_chunks) {
  return sizeof(float) * (static_cast<size_t>(M + 1) * kPickCols + pad4(M + 1)) +
         2 * sizeof(float) * kChunk * kPickCols + 2 * static_cast<size_t>(kVarStage) + sizeof(float) * 68 +
         sizeof(int32_t) * pad4(n_chunks);
}

// the pick scan serves this shape (values of vb bytes)
inline bool pick_path(const Plan& p) {
  return use_mf(p) && p.pitch == 8 && p.dh % kPickCols == 0 && p.M <= 1024 && pick_lds_bytes(p.M, p.n_chunks) <= kLdsBytes;
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
// sum over the eight pick lanes of a column half (u % 4 and u / 8); every lane gets the same value
__device__ __forceinline__ float pick_sum(float v) {
  v += dppf<0xb1>(v);    // quad_perm [1,0,3,2]
  v += dppf<0x4e>(v);    // quad_perm [2,3,0,1]
  v += dppf<0x128>(v);   // row_ror:8 (lane u ^ 8)
  return v;
}
// sum over all 16 lanes of a position
__device__ __forceinline__ float pos_sum(float v) {
  v = pick_sum(v);
  v += dppf<0x124>(v);   // row_ror:4 (the other half: lane u - 4 mod 16)
  return v;
}

// four consecutive float32 values of a value row in LDS
template <typename VT>
struct VPiece;
template <>
struct VPiece<float> {
  float4 w;
  __device__ __forceinline__ void load(const float* p) { w = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ void fma4(float c, float* acc) const {
    acc[0] = fmaf(c, w.x, acc[0]);
    acc[1] = fmaf(c, w.y, acc[1]);
    acc[2] = fmaf(c, w.z, acc[2]);
    acc[3] = fmaf(c, w.w, acc[3]);
  }
};

template <typename VT, typename OutT>
__global__ void __launch_bounds__(kPickThreads) pick_scan_kernel(ScanArgs a) {
  constexpr int CW = kPickCols;
  constexpr int VS = kVarStage;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int M = a.M;
  const int G = a.groups;
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int jr = (bid >> 3) / G;
  const int g = (bid >> 3) - jr * G;
  const int s = 8 * jr + xcd;
  if (s >= a.S) return;
  const int b_row = s / a.H;
  const int h = s - b_row * a.H;
  float* A = lds;                                                          // [M + 1][32]
  float* cnt = A + static_cast<size_t>(M + 1) * CW;                        // [M + 1]
  float* s_v = cnt + pad4(M + 1);                                          // [2][64][32]
  unsigned char* var = reinterpret_cast<unsigned char*>(s_v + 2 * kChunk * CW);   // [2][VS]
  float* pw = reinterpret_cast<float*>(var + 2 * VS);                      // [68]
  int32_t* s_sizes = reinterpret_cast<int32_t*>(pw + 68);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int p = tid >> 4;
  const int u = tid & 15;
  const int bq = u & 3;               // this lane's final piece in its half
  const int hh = (u >> 2) & 1;        // column half
  const int io = u >> 3;              // which two columns of the piece
  const int pick = 2 * bq + io;       // the pick (record) this lane reads
  const int col0 = g * CW;
  const int hcol = hh * 16;
  // the lane's pieces, in the order the reduction consumes them
  const int ord[4] = {bq, bq ^ 1, 3 - bq, (3 - bq) ^ 1};
  const int fcol = hcol + 4 * bq + 2 * io;   // the lane's two final columns (in the group)
  const float lam = a.decay[h];
  const bool norm = a.onorm_w != nullptr;
  const bool xnorm = norm && G > 1;
  const unsigned char* plans_s = a.plans + static_cast<int64_t>(s) * a.n_chunks * PickGeom::stride();
  const VT* v_b = static_cast<const VT*>(a.v) + static_cast<int64_t>(b_row) * a.T * a.v_stride +
                  static_cast<int64_t>(h) * a.dh + col0;

  for (int i = tid; i < (M + 1) * CW; i += kPickThreads) {
    const int m = i / CW;
    const int cc = i - m * CW;
    A[i] = (a.state_in_mem && m < M) ? a.state_in_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] : 0.f;
  }
  for (int m = tid; m <= M; m += kPickThreads)
    cnt[m] = (a.state_in_cnt && m < M) ? a.state_in_cnt[static_cast<int64_t>(s) * M + m] : 0.f;
  for (int i = tid; i < a.n_chunks; i += kPickThreads) s_sizes[i] = a.sizes[static_cast<int64_t>(s) * a.n_chunks + i];
  if (tid <= kChunk) {
    float v = 1.f, sq = lam;   // lam^tid by squaring (as the plan computes it; exact for lam = 0 and lam = 1)
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      v = ((tid >> bit) & 1) ? v * sq : v;
      sq *= sq;
    }
    pw[tid] = v;
  }
  float onw[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) onw[k] = norm ? a.onorm_w[h * a.dh + col0 + fcol + k] : 1.f;
  float mu = 1.f;

  // this lane's read and write records of chunk c
  auto load_recs = [&](int c, uint3& rr, uint3& wr) {
    const unsigned char* base = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(PickGeom::stride()) +
                                PickGeom::kRec * (pick * kChunk + p);
    rr = *reinterpret_cast<const uint3*>(base);
    wr = *reinterpret_cast<const uint3*>(base + PickGeom::off_w());
  };
  // chunk c's value rows and variable part, loaded into registers (two values of row p at columns 2 u, 2 u + 1;
  // dword tid of the variable part) and stored into LDS buffer c & 1 at the end of the previous chunk.  (Direct
  // global-to-LDS copies would make the compiler wait for every load in flight before the first LDS read after
  // them, the record prefetch included.)
  using VPair = typename std::conditional<sizeof(VT) == 2, uint32_t, uint2>::type;
  auto load_v = [&](int c) {
    const int row = min(c * kChunk + p, a.T - 1);
    const VT* src = v_b + static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_stride) + 2 * u;
    if (a.v_direct) return *reinterpret_cast<const VPair*>(src);
    VPair pr;
    VT* d = reinterpret_cast<VT*>(&pr);
    d[0] = src[0];
    d[1] = src[1];
    return pr;
  };
  auto load_var = [&](int c, int bytes) {
    const unsigned char* src = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(PickGeom::stride()) +
                               PickGeom::off_var() + 4 * tid;
    return 4 * tid < min(bytes, VS) ? *reinterpret_cast<const uint32_t*>(src) : 0u;
  };
  auto stage = [&](int c, const VPair& vv, uint32_t vr) {   // the values as float32
    float2 f;
    if constexpr (sizeof(VT) == 2) f = make_float2(__uint_as_float(vv << 16), __uint_as_float(vv & 0xffff0000u));
    else f = make_float2(__uint_as_float(vv.x), __uint_as_float(vv.y));
    *reinterpret_cast<float2*>(s_v + (c & 1) * kChunk * CW + p * CW + 2 * u) = f;
    reinterpret_cast<uint32_t*>(var + (c & 1) * VS)[tid] = vr;
  };
  // the lane's two read-out columns at position p of chunk 0; chunk c is c * 64 rows further (bfloat16 rounded to
  // nearest even by the hardware conversion)
  OutT* r_lane = static_cast<OutT*>(a.r_out) + (static_cast<int64_t>(b_row) * a.T + p) * a.r_stride +
                 static_cast<int64_t>(h) * a.dh + col0 + fcol;
  const bool r_vec = reinterpret_cast<uintptr_t>(r_lane) % (2 * sizeof(OutT)) == 0 &&
                     (static_cast<uint64_t>(a.r_stride) * sizeof(OutT)) % (2 * sizeof(OutT)) == 0;
  auto store_r = [&](int c, const float (&x)[2]) {
    OutT* dst = r_lane + static_cast<int64_t>(c) * kChunk * a.r_stride;
    if constexpr (sizeof(OutT) == 2) {
      const uint32_t w = pack_bf16(x[0], x[1]);
      if (r_vec) {
        *reinterpret_cast<uint32_t*>(dst) = w;
      } else {
        reinterpret_cast<uint16_t*>(dst)[0] = static_cast<uint16_t>(w);
        reinterpret_cast<uint16_t*>(dst)[1] = static_cast<uint16_t>(w >> 16);
      }
    } else {
      if (r_vec) {
        *reinterpret_cast<float2*>(dst) = make_float2(x[0], x[1]);
      } else {
        dst[0] = x[0];
        dst[1] = x[1];
      }
    }
  };
  // The out-norm exchange between the G groups of a slab: every group stores its per-position partial sum of
  // squares of chunk c as one 64-bit word {sum, 1} (the plan kernel cleared the words), and finishes chunk c's
  // read-out two chunks later with the others' words, waiting (a bounded spin that rarely runs) until they are
  // written.  With two groups the partner's word is loaded in the middle of the chunk and used at its end.
  unsigned long long* xw = reinterpret_cast<unsigned long long*>(a.xch) + static_cast<int64_t>(s) * a.n_chunks * G * kChunk + p;
  auto xget = [&](int c, int gg) {
    return __hip_atomic_load(xw + (c * G + gg) * kChunk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto partner = [&](int c, int gg, unsigned long long v) {   // group gg's sum for chunk c, once written
    if (__ballot(!(v >> 32))) {
      for (uint32_t it = 0;; ++it) {
        __builtin_amdgcn_s_sleep(2);
        if (!(v >> 32)) v = xget(c, gg);
        if (!__ballot(!(v >> 32))) break;
        if (it >= kSpinLimit) {
          if (lane == 0) store_sync(a.sync + static_cast<int64_t>(a.S) * a.sync_stride, 1u);
          break;
        }
      }
    }
    return __uint_as_float(static_cast<uint32_t>(v));
  };
  auto finish = [&](int c, const float (&x)[2], float ss, unsigned long long xo) {
    float tot;
    if (G == 2) {
      const float o = partner(c, 1 - g, xo);
      tot = g == 0 ? ss + o : o + ss;   // group order, the same sum in both groups
    } else {
      tot = 0.f;
      for (int gg = 0; gg < G; ++gg) tot += gg == g ? ss : partner(c, gg, xget(c, gg));
    }
    if (p < min(kChunk, a.T - c * kChunk)) {
      const float inv = fast_rsqrt(tot * (1.f / static_cast<float>(a.dh)) + a.out_eps);
      float o[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) o[k] = x[k] * inv * onw[k];
      store_r(c, o);
    }
  };
  float rq[3][2] = {};
  float sq[3] = {0.f, 0.f, 0.f};

  uint3 rr, wr;
  load_recs(0, rr, wr);
  stage(0, load_v(0), load_var(0, a.sizes[static_cast<int64_t>(s) * a.n_chunks]));
  lds_barrier();
  const float lam_chunk = pw[kChunk];
  const float inv_dh = 1.f / static_cast<float>(a.dh);
  const unsigned char* A_b = reinterpret_cast<const unsigned char*>(A);
  unsigned char* A_w = reinterpret_cast<unsigned char*>(A);
  int soff[4];   // byte offsets of the lane's pieces in a slab row
#pragma unroll
  for (int t = 0; t < 4; ++t) soff[t] = 4 * (hcol + 4 * ord[t]);

  for (int c = 0; c < a.n_chunks; ++c) {
    const bool fin2 = xnorm && c >= 2;
    // the next chunk's records, values and variable part are loaded into registers during this chunk (the last
    // chunk loads its own again)
    const int cn = min(c + 1, a.n_chunks - 1);
    uint3 rr_n, wr_n;
    load_recs(cn, rr_n, wr_n);
    const VPair v_n = load_v(cn);
    const uint32_t var_n = load_var(cn, s_sizes[cn]);
    const int c0 = c * kChunk;
    const int L = min(kChunk, a.T - c0);
    const unsigned char* varc = var + (c & 1) * VS;
    const float* s_vc = s_v + (c & 1) * kChunk * CW;
    const int bytes = s_sizes[c];
    const bool all_staged = bytes <= VS;
    const unsigned char* gvar =
        plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(PickGeom::stride()) + PickGeom::off_var();
    auto ent_at = [&](int e, auto st) {
      const int o = PickGeom::off_ent() + 8 * min(max(e, 0), PickGeom::max_entries() - 1);
      if constexpr (decltype(st)::value) return *reinterpret_cast<const uint2*>(varc + o);
      else return o + 8 <= VS ? *reinterpret_cast<const uint2*>(varc + o) : *reinterpret_cast<const uint2*>(gvar + o);
    };

    // ---- read: the pick's row, scaled; the in-chunk contribution of this lane's record ----
    const int rslot = static_cast<int>(rr.x & 0xffffu);
    const int n_in = static_cast<int>(rr.x >> 24);
    const float sw = __uint_as_float(rr.y) * (mu * pw[p]);
    float acc[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4 q4 = *reinterpret_cast<const float4*>(A_b + rslot * (CW * 4) + soff[t]);
      acc[4 * t] = sw * q4.x;
      acc[4 * t + 1] = sw * q4.y;
      acc[4 * t + 2] = sw * q4.z;
      acc[4 * t + 3] = sw * q4.w;
    }
    float dl = sw * cnt[rslot];
    if (pick < n_in) {   // contribution number `pick` of the position
      const float cc = __uint_as_float(rr.z);
      const float* vrow = s_vc + ((rr.x >> 16) & 63u) * CW;
      VPiece<float> vq[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) vq[t].load(vrow + soff[t] / 4);
#pragma unroll
      for (int t = 0; t < 4; ++t) vq[t].fma4(cc, acc + 4 * t);
      dl += cc;
    }
    if (n_in > 8) {   // contributions past the eight in the records (crowded chunks only)
      const int e0 = reinterpret_cast<const uint16_t*>(varc + 16)[p];   // the position's first entry
      auto over = [&](auto st) {
        for (int j = 8 + pick; j < n_in; j += 8) {
          const uint2 e = ent_at(e0 + j - 8, st);
          const float ce = __uint_as_float(e.x);
          VPiece<float> vq[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) vq[t].load(s_vc + (e.y & 63u) * CW + soff[t] / 4);
#pragma unroll
          for (int t = 0; t < 4; ++t) vq[t].fma4(ce, acc + 4 * t);
          dl += ce;
        }
      };
      if (all_staged) over(std::true_type{});
      else over(std::false_type{});
    }
    // reduce-scatter over the eight pick lanes of the half: 16 -> 8 -> 4 -> 2 columns
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] += dppf<0x1b>(acc[8 + k]);   // quad_perm [3,2,1,0]: piece 3 - b
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += dppf<0xb1>(acc[4 + k]);   // quad_perm [1,0,3,2]: piece b ^ 1
    float r[2];
    {
      const float k0 = io ? acc[2] : acc[0], k1 = io ? acc[3] : acc[1];
      const float s0 = io ? acc[0] : acc[2], s1 = io ? acc[1] : acc[3];
      r[0] = k0 + dppf<0x128>(s0);   // row_ror:8: the lane of the other two columns
      r[1] = k1 + dppf<0x128>(s1);
    }
    const float den = pick_sum(dl);
    if (a.read_mean) {
      if (a.den_out && g == 0 && u == 0 && p < L) a.den_out[(static_cast<int64_t>(b_row) * a.T + c0 + p) * a.H + h] = den;
      const float inv = fast_rcp(den + a.read_eps);
      r[0] *= inv;
      r[1] *= inv;
    }
    if (a.read_out && p < L) {
      float* dst = a.read_out + (static_cast<int64_t>(b_row) * a.T + c0 + p) * static_cast<int64_t>(a.H) * a.dh +
                   static_cast<int64_t>(h) * a.dh + col0 + fcol;
      store_vals<2, float>(dst, r);
    }
    if (norm) {
      const float ss = pos_sum(fmaf(r[1], r[1], r[0] * r[0]));
      if (xnorm) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          rq[2][k] = rq[1][k];
          rq[1][k] = rq[0][k];
          rq[0][k] = r[k];
        }
        sq[2] = sq[1];
        sq[1] = sq[0];
        sq[0] = ss;
        if (u == 0)
          __hip_atomic_store(xw + (c * G + g) * kChunk, (1ull << 32) | __float_as_uint(ss), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      } else if (p < L) {
        const float inv = fast_rsqrt(ss * inv_dh + a.out_eps);
        float o[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) o[k] = r[k] * inv * onw[k];
        store_r(c, o);
      }
    } else if (p < L) {
      store_r(c, r);
    }
    lds_barrier();
    // the partner's partial sums of chunk c - 2 (used when it finishes, at the end of this chunk)
    const unsigned long long xo = (fin2 && G == 2) ? xget(c - 2, 1 - g) : 0ull;
    // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small); a chunk with a reset empties it
    const bool chunk_reset = reinterpret_cast<const uint32_t*>(varc)[1] & 0x80000000u;
    float mu_new = mu * (L == kChunk ? lam_chunk : pw[L]);
    if (chunk_reset) {
      float4* a4 = reinterpret_cast<float4*>(A);
      for (int i = tid; i < (M + 1) * CW / 4; i += kPickThreads) a4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int i = tid; i <= M; i += kPickThreads) cnt[i] = 0.f;
      mu_new = 1.f;
      lds_barrier();
    } else if (!(mu_new >= kMuFloor)) {
      for (int i = tid; i < (M + 1) * CW; i += kPickThreads) A[i] *= mu_new;
      for (int i = tid; i <= M; i += kPickThreads) cnt[i] *= mu_new;
      mu_new = 1.f;
      lds_barrier();
    }
    // ---- write: the owner lanes add their faded values and those of the slot's later writers ----
    const float inv_mu = fast_rcp(mu_new);
    const int wslot = static_cast<int>(wr.x & 0x7ffu);
    if (wslot != M) {
      const int n_l = static_cast<int>((wr.x >> 17) & 63u);
      float y[16];
      unsigned char* row = A_w + wslot * (CW * 4);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float4 q4 = *reinterpret_cast<const float4*>(row + soff[t]);
        y[4 * t] = q4.x;
        y[4 * t + 1] = q4.y;
        y[4 * t + 2] = q4.z;
        y[4 * t + 3] = q4.w;
      }
      VPiece<float> vp[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) vp[t].load(s_vc + p * CW + soff[t] / 4);
      const float a0 = __uint_as_float(wr.y) * inv_mu;
      float cw = cnt[wslot] + a0;
#pragma unroll
      for (int t = 0; t < 4; ++t) vp[t].fma4(a0, y + 4 * t);
      if (n_l > 0) {
        const float a1 = __uint_as_float(wr.z) * inv_mu;
        VPiece<float> vl[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) vl[t].load(s_vc + ((wr.x >> 11) & 63u) * CW + soff[t] / 4);
#pragma unroll
        for (int t = 0; t < 4; ++t) vl[t].fma4(a1, y + 4 * t);
        cw += a1;
        if (n_l > 1) {   // later writers past the first, from the variable part
          const int w_e0 = static_cast<int>(wr.x >> 23);   // the first of them among the entries
          auto later = [&](auto st) {
            for (int e = 0; e < n_l - 1; ++e) {
              const uint2 en = ent_at(w_e0 + e, st);
              const float ae = __uint_as_float(en.x) * inv_mu;
              VPiece<float> ve[4];
#pragma unroll
              for (int t = 0; t < 4; ++t) ve[t].load(s_vc + (en.y & 63u) * CW + soff[t] / 4);
#pragma unroll
              for (int t = 0; t < 4; ++t) ve[t].fma4(ae, y + 4 * t);
              cw += ae;
            }
          };
          if (all_staged) later(std::true_type{});
          else later(std::false_type{});
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
        *reinterpret_cast<float4*>(row + soff[t]) = make_float4(y[4 * t], y[4 * t + 1], y[4 * t + 2], y[4 * t + 3]);
      if (hh == 0) cnt[wslot] = cw;   // one of the two half lanes of the pick
    }
    mu = mu_new;
    rr = rr_n;
    wr = wr_n;
    stage(c + 1, v_n, var_n);   // buffer (c + 1) & 1 held chunk c - 1, done before the last barrier
    if (fin2) finish(c - 2, rq[2], sq[2], xo);
    lds_barrier();
  }
  if (xnorm) {   // the last two chunks (or one)
    const int n = a.n_chunks;
    if (n >= 2) finish(n - 2, rq[1], sq[1], G == 2 ? xget(n - 2, 1 - g) : 0ull);
    finish(n - 1, rq[0], sq[0], G == 2 ? xget(n - 1, 1 - g) : 0ull);
  }

  if (a.state_out_mem) {
    for (int i = tid; i < M * CW; i += kPickThreads) {
      const int m = i / CW;
      const int cc = i - m * CW;
      a.state_out_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] = mu * A[i];
    }
  }
  if (a.state_out_cnt && g == 0) {
    for (int m = tid; m < M; m += kPickThreads) a.state_out_cnt[static_cast<int64_t>(s) * M + m] = mu * cnt[m];
  }
}

template <typename VT, typename OutT>
int launch_pick_scan_t(const Plan& p, const ScanArgs& a, hipStream_t st) {
  const size_t lds = pick_lds_bytes(p.M, p.n_chunks);
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&pick_scan_kernel<VT, OutT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     static_cast<int>(kLdsBytes));
  if (attr != hipSuccess) return set_err(SDM_RT_ELAUNCH, "pick scan: cannot enable %zu bytes of LDS", kLdsBytes);
  if (a.groups * kPickCols != p.dh || a.sync_stride < a.groups || !pick_path(p))
    return set_err(SDM_RT_EINVAL, "pick scan: %d groups for head_dim %d", a.groups, p.dh);
  const int slabs8 = (p.B * p.H + 7) / 8 * 8;
  hipLaunchKernelGGL((pick_scan_kernel<VT, OutT>), dim3(slabs8 * a.groups), dim3(kPickThreads), lds, st, a);
  return check_launch("pick scan");
}

// defined in sdm_pick_bf16.hip and sdm_pick_f32.hip (values in bfloat16 or float32), for either output type
int launch_pick_scan_bf16(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st);
int launch_pick_scan_f32(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st);

}  // namespace sdmrt
