// sdm_pick.h -- pick_scan_kernel: the scan of one (batch row, head) slab over a group of 32 of its value columns,
// executing pick plans (plan_kernel<..., PICK = true>), with the read-out finished in place (RunTimeSdm._chunk,
// forward and finish, experiments/track4/sdmllm/track4_onesdm_models.py:215-247 without wo).  It serves picks of at
// most 8, head_dim a multiple of 32 and slabs of at most 1,024 locations; scan_kernel (sdm_scan.h) serves the rest.
//
// Layout of the work: 512 threads, one lane per (position p, pick j) of the chunk, tid = 8 p + j, each over all 32
// columns of the group (eight 4-column pieces).
//   read   lane j gathers the row of its read pick (eight 16-byte LDS reads) in the order j, j^1, j^2, j^3, j^7,
//          j^6, j^5, j^4, scales it by the read weight and adds the in-chunk contribution number j the plan gave
//          its record; the position's eight lanes then reduce-scatter the sums by DPP without register selects
//          (lanes j and 7 - j exchange four pieces (row_half_mirror), then j and j^2, then j and j^1), after which
//          lane j holds piece j (columns 4 j ... 4 j + 3) summed over the picks.  At every read the eight lanes of a
//          position touch eight different pieces, i.e. all 32 banks.
//   write  the lane of write pick j owns the slot if its position is the first writer of the slot the chunk keeps;
//          it loads the slot's row and count during the read phase (no other lane writes that slot in the chunk),
//          and after the barrier adds its faded value (value row p, assembled from the pieces the position's eight
//          lanes staged, by DPP) and those of the slot's later writers in the chunk, and stores the row back: each
//          slot has one owner, so the sums run in a fixed order and the result is deterministic.
// Records, the chunk's value pieces and the variable part of its plan (contributions and later writers beyond the
// first) are loaded into registers one chunk ahead; values and variable part are stored into LDS at the end of the
// previous chunk.  Decay bookkeeping, the out-norm exchange between the column groups of a slab and the reset
// handling are those of scan_kernel (sdm_scan.h); a wait of the exchange that gives up records a time-out in the
// status word and leaves the chunk's read-outs NaN.
#pragma once

#include "sdm_scan.h"

namespace sdmrt {

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

constexpr int kPickThreads = 512;    // 64 positions x 8 picks
constexpr int kTeamWriters = 32;     // a wave with a slot of this many later writers in a chunk writes in teams
constexpr int kPrefetchContribs = 40;  // a wave with a position of more contributions loads their entries together

template <typename VT, typename OutT>
__global__ void __launch_bounds__(kPickThreads) pick_scan_kernel(ScanArgs a) {
  constexpr int CW = kPickCols;
  constexpr int VS = kVarStage;
  constexpr int NT = kPickThreads;
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
  const int lane = tid & 63;
  const int p = tid >> 3;
  const int j = tid & 7;   // the lane's pick, and its final piece
  const int col0 = g * CW;
  const int fcol = 4 * j;  // the lane's four read-out columns (in the group)
  int soff[8];             // byte offsets of the lane's pieces in a 32-column row, in read order
#pragma unroll
  for (int k = 0; k < 8; ++k) soff[k] = 16 * (j ^ (k < 4 ? k : 11 - k));
  const float lam = a.decay[h];
  const bool norm = a.onorm_w != nullptr;
  const bool xnorm = norm && G > 1;
  const unsigned char* plans_s = a.plans + static_cast<int64_t>(s) * a.n_chunks * PickGeom::stride();
  const VT* v_b = static_cast<const VT*>(a.v) + static_cast<int64_t>(b_row) * a.T * a.v_stride +
                  static_cast<int64_t>(h) * a.dh + col0;

  for (int i = tid; i < (M + 1) * CW; i += NT) {
    const int m = i / CW;
    const int cc = i - m * CW;
    A[i] = (a.state_in_mem && m < M) ? a.state_in_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] : 0.f;
  }
  for (int m = tid; m <= M; m += NT)
    cnt[m] = (a.state_in_cnt && m < M) ? a.state_in_cnt[static_cast<int64_t>(s) * M + m] : 0.f;
  for (int i = tid; i < a.n_chunks; i += NT) s_sizes[i] = a.sizes[static_cast<int64_t>(s) * a.n_chunks + i];
  if (tid <= kChunk) {
    float v = 1.f, sq = lam;   // lam^tid by squaring (as the plan computes it; exact for lam = 0 and lam = 1)
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      v = ((tid >> bit) & 1) ? v * sq : v;
      sq *= sq;
    }
    pw[tid] = v;
  }
  float onw[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) onw[k] = norm ? a.onorm_w[h * a.dh + col0 + fcol + k] : 1.f;
  float mu = 1.f;

  // this lane's read and write records of chunk c
  auto load_recs = [&](int c, uint3& rr, uint3& wr) {
    const unsigned char* base = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(PickGeom::stride()) +
                                PickGeom::kRec * (j * kChunk + p);
    rr = *reinterpret_cast<const uint3*>(base);
    wr = *reinterpret_cast<const uint3*>(base + PickGeom::off_w());
  };
  // chunk c's value rows and variable part, loaded into registers (row p, columns 4 j ... 4 j + 3; bytes 8 tid ...
  // 8 tid + 7 of the variable part) and stored into LDS buffer c & 1 at the end of the previous chunk
  using VQuad = typename std::conditional<sizeof(VT) == 2, uint2, uint4>::type;
  auto load_v = [&](int c) {
    const int row = min(c * kChunk + p, a.T - 1);
    const VT* src = v_b + static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_stride) + fcol;
    if (a.v_direct) return *reinterpret_cast<const VQuad*>(src);
    VQuad q;
    VT* d = reinterpret_cast<VT*>(&q);
#pragma unroll
    for (int k = 0; k < 4; ++k) d[k] = src[k];
    return q;
  };
  auto load_var = [&](int c, int bytes) {
    const unsigned char* src = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(PickGeom::stride()) +
                               PickGeom::off_var() + 8 * tid;
    return 8 * tid < min(bytes, VS) ? *reinterpret_cast<const uint2*>(src) : make_uint2(0u, 0u);
  };
  auto stage = [&](int c, const VQuad& vv, const uint2& vr) {   // the values as float32
    float4 f;
    if constexpr (sizeof(VT) == 2) {
      f = make_float4(__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u), __uint_as_float(vv.y << 16),
                      __uint_as_float(vv.y & 0xffff0000u));
    } else {
      f = make_float4(__uint_as_float(vv.x), __uint_as_float(vv.y), __uint_as_float(vv.z), __uint_as_float(vv.w));
    }
    *reinterpret_cast<float4*>(s_v + (c & 1) * kChunk * CW + p * CW + fcol) = f;
    reinterpret_cast<uint2*>(var + (c & 1) * VS)[tid] = vr;
  };
  // the lane's four read-out columns at position p of chunk 0; chunk c is c * 64 rows further
  OutT* r_lane = static_cast<OutT*>(a.r_out) + (static_cast<int64_t>(b_row) * a.T + p) * a.r_stride +
                 static_cast<int64_t>(h) * a.dh + col0 + fcol;
  const bool r_vec = reinterpret_cast<uintptr_t>(r_lane) % (4 * sizeof(OutT)) == 0 &&
                     (static_cast<uint64_t>(a.r_stride) * sizeof(OutT)) % (4 * sizeof(OutT)) == 0;
  auto store_r = [&](int c, const float (&x)[4]) {
    OutT* dst = r_lane + static_cast<int64_t>(c) * kChunk * a.r_stride;
    if constexpr (sizeof(OutT) == 2) {
      const uint2 w = make_uint2(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]));
      if (r_vec) {
        *reinterpret_cast<uint2*>(dst) = w;
      } else {
        uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
        d16[0] = static_cast<uint16_t>(w.x);
        d16[1] = static_cast<uint16_t>(w.x >> 16);
        d16[2] = static_cast<uint16_t>(w.y);
        d16[3] = static_cast<uint16_t>(w.y >> 16);
      }
    } else {
      if (r_vec) {
        *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = x[k];
      }
    }
  };
  // The out-norm exchange between the G groups of a slab: every group stores its per-position partial sum of
  // squares of chunk c as one 64-bit word {sum, 1} (the plan kernel cleared the words), and finishes chunk c's
  // read-out two chunks later with the others' words, waiting (a bounded spin that rarely runs) until they are
  // written.  With two groups the partner's word is loaded in the middle of the chunk and used at its end.  A wait
  // that gives up records a time-out in the status word and finishes the chunk with NaN read-outs.
  unsigned long long* xw = reinterpret_cast<unsigned long long*>(a.xch) + static_cast<int64_t>(s) * a.n_chunks * G * kChunk + p;
  auto xget = [&](int c, int gg) {
    return __hip_atomic_load(xw + (c * G + gg) * kChunk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto partner = [&](int c, int gg, unsigned long long v) {   // group gg's sum for chunk c, once written
    if (a.spin_limit == 0) v = 0ull;   // waits give up at once (the error path's test)
    if (__ballot(!(v >> 32))) {
      for (uint32_t it = 0;; ++it) {
        if (it >= a.spin_limit) {
          if (lane == 0) store_sync(a.sync + static_cast<int64_t>(a.S) * a.sync_stride, 1u);
          return __builtin_nanf("");
        }
        __builtin_amdgcn_s_sleep(2);
        if (!(v >> 32)) v = xget(c, gg);
        if (!__ballot(!(v >> 32))) break;
      }
    }
    return __uint_as_float(static_cast<uint32_t>(v));
  };
  auto finish = [&](int c, const float (&x)[4], float ss, unsigned long long xo) {
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
      float o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = x[k] * inv * onw[k];
      store_r(c, o);
    }
  };
  float rq[3][4] = {};
  float sq[3] = {0.f, 0.f, 0.f};

  // the value piece this lane staged for the current chunk (piece j of row p), as float32
  auto as_f4 = [&](const VQuad& vv) {
    if constexpr (sizeof(VT) == 2)
      return make_float4(__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u), __uint_as_float(vv.y << 16),
                         __uint_as_float(vv.y & 0xffff0000u));
    else
      return make_float4(__uint_as_float(vv.x), __uint_as_float(vv.y), __uint_as_float(vv.z), __uint_as_float(vv.w));
  };
  uint3 rr, wr;
  load_recs(0, rr, wr);
  VQuad v_cur = load_v(0);
  stage(0, v_cur, load_var(0, a.sizes[static_cast<int64_t>(s) * a.n_chunks]));
  lds_barrier();
  const float lam_chunk = pw[kChunk];
  const float inv_dh = 1.f / static_cast<float>(a.dh);
  const unsigned char* A_b = reinterpret_cast<const unsigned char*>(A);
  unsigned char* A_w = reinterpret_cast<unsigned char*>(A);

  // A slab with crowded chunks (a chunk's variable part past a.crowded_bytes, by default the LDS staging area: most
  // positions of the chunk write the same slots) runs the chunk step whose owners sum their writes before the read
  // barrier (EARLY), so a crowded wave's writes overlap the other waves' reads; the other slabs the plain step, whose
  // sums after the barrier hide the partner word's load (the early sums cost varied addresses ~5%).  Both give the
  // same bits.
  bool crowded = false;
  for (int i = lane; i < a.n_chunks; i += 64) crowded |= s_sizes[i] > a.crowded_bytes;
  crowded = __ballot(crowded) != 0ull;
  auto chunk_loop = [&](auto early_t) {
    constexpr bool EARLY = decltype(early_t)::value;
    for (int c = 0; c < a.n_chunks; ++c) {
      const bool fin2 = xnorm && c >= 2;
      // the next chunk's records, values and variable part are loaded into registers during this chunk (the last
      // chunk loads its own again)
      const int cn = min(c + 1, a.n_chunks - 1);
      uint3 rr_n, wr_n;
      load_recs(cn, rr_n, wr_n);
      const VQuad v_n = load_v(cn);
      const uint2 var_n = load_var(cn, s_sizes[cn]);
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
      // row v of the staged values, scaled by cf, added to acc (the lane's read order)
      auto add_vrow = [&](float cf, int v, float (&acc)[32]) {
        const float* vrow = s_vc + v * CW;
        VPiece<float> vq[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) vq[k].load(vrow + soff[k] / 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) vq[k].fma4(cf, acc + 4 * k);
      };

      // ---- read: the pick's row, scaled; the in-chunk contribution of this lane's record ----
      const int rslot = static_cast<int>(rr.x & 0xffffu);
      const int n_in = static_cast<int>(rr.x >> 24);
      const float sw = __uint_as_float(rr.y) * (mu * pw[p]);
      float acc[32];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 q4 = *reinterpret_cast<const float4*>(A_b + rslot * (CW * 4) + soff[k]);
        acc[4 * k] = sw * q4.x;
        acc[4 * k + 1] = sw * q4.y;
        acc[4 * k + 2] = sw * q4.z;
        acc[4 * k + 3] = sw * q4.w;
      }
      float dl = sw * cnt[rslot];
      if (j < n_in) {   // contribution number j of the position
        const float cc = __uint_as_float(rr.z);
        add_vrow(cc, static_cast<int>((rr.x >> 16) & 63u), acc);
        dl += cc;
      }
      if (n_in > 8) {   // contributions past the eight in the records (crowded chunks only)
        const int e0 = reinterpret_cast<const uint16_t*>(varc + 16)[p];   // the position's first entry
        auto over = [&](auto st) {
          if (__ballot(n_in > kPrefetchContribs)) {   // crowded: contributions 8 + j, 16 + j, ... (at most 7: n_in <
            uint2 ev[7];                                // 64), their entries loaded together first
#pragma unroll
            for (int t = 0; t < 7; ++t) ev[t] = 8 + j + 8 * t < n_in ? ent_at(e0 + j + 8 * t, st) : make_uint2(0u, 0u);
#pragma unroll
            for (int t = 0; t < 7; ++t) {
              if (8 + j + 8 * t < n_in) {
                const float ce = __uint_as_float(ev[t].x);
                add_vrow(ce, static_cast<int>(ev[t].y & 63u), acc);
                dl += ce;
              }
            }
          } else {
            for (int jj = 8 + j; jj < n_in; jj += 8) {
              const uint2 e = ent_at(e0 + jj - 8, st);
              const float ce = __uint_as_float(e.x);
              add_vrow(ce, static_cast<int>(e.y & 63u), acc);
              dl += ce;
            }
          }
        };
        if (all_staged) over(std::true_type{});
        else over(std::false_type{});
      }
      // the owned write slot's row and count, loaded now (no other lane writes the slot in this chunk; reads of it
      // by other lanes do not change it), so the write phase after the barrier only adds and stores
      const int wslot = static_cast<int>(wr.x & 0x7ffu);
      float y[32];
      float cw_old = 0.f;
      if (wslot != M) {
        const unsigned char* row = A_b + wslot * (CW * 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float4 q4 = *reinterpret_cast<const float4*>(row + soff[k]);
          y[4 * k] = q4.x;
          y[4 * k + 1] = q4.y;
          y[4 * k + 2] = q4.z;
          y[4 * k + 3] = q4.w;
        }
        cw_old = cnt[wslot];
      }
      // the eight pieces of value row p in the lane's read order, from the pieces the position's eight lanes staged
      // (lane x holds piece x): pieces j ^ 1, j ^ 2, j ^ 3 by quad permutes, j ^ 7 by the half-row mirror, and
      // j ^ 6, j ^ 5, j ^ 4 by the mirror of the first three
      float vp[32];
      {
        const float4 f = as_f4(v_cur);
        const float x[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t1 = dppf<0xb1>(x[e]), t2 = dppf<0x4e>(x[e]), t3 = dppf<0x1b>(x[e]);
          vp[e] = x[e];
          vp[4 + e] = t1;
          vp[8 + e] = t2;
          vp[12 + e] = t3;
          vp[16 + e] = dppf<0x141>(x[e]);
          vp[20 + e] = dppf<0x141>(t1);
          vp[24 + e] = dppf<0x141>(t2);
          vp[28 + e] = dppf<0x141>(t3);
        }
      }
      // reduce-scatter over the eight pick lanes of the position: 32 -> 16 -> 8 -> 4 columns
#pragma unroll
      for (int k = 0; k < 16; ++k) acc[k] += dppf<0x141>(acc[16 + k]);   // row_half_mirror: lane 7 - j
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] += dppf<0x4e>(acc[8 + k]);      // quad_perm [2,3,0,1]: lane j ^ 2
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += dppf<0xb1>(acc[4 + k]);      // quad_perm [1,0,3,2]: lane j ^ 1
      float r[4] = {acc[0], acc[1], acc[2], acc[3]};
      const float den = sum8(dl);
      if (a.read_mean) {
        if (a.den_out && g == 0 && j == 0 && p < L) a.den_out[(static_cast<int64_t>(b_row) * a.T + c0 + p) * a.H + h] = den;
        const float inv = fast_rcp(den + a.read_eps);
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] *= inv;
      }
      if (a.read_out && p < L) {
        float* dst = a.read_out + (static_cast<int64_t>(b_row) * a.T + c0 + p) * static_cast<int64_t>(a.H) * a.dh +
                     static_cast<int64_t>(h) * a.dh + col0 + fcol;
        store_vals<4, float>(dst, r);
      }
      if (norm) {
        const float ss = sum8(fmaf(r[3], r[3], fmaf(r[2], r[2], fmaf(r[1], r[1], r[0] * r[0]))));
        if (xnorm) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            rq[2][k] = rq[1][k];
            rq[1][k] = rq[0][k];
            rq[0][k] = r[k];
          }
          sq[2] = sq[1];
          sq[1] = sq[0];
          sq[0] = ss;
          if (j == 0)
            __hip_atomic_store(xw + (c * G + g) * kChunk, (1ull << 32) | __float_as_uint(ss), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else if (p < L) {
          const float inv = fast_rsqrt(ss * inv_dh + a.out_eps);
          float o[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) o[k] = r[k] * inv * onw[k];
          store_r(c, o);
        }
      } else if (p < L) {
        store_r(c, r);
      }
      float mu_new;              // the slab's scale after this chunk
      unsigned long long xo;     // the partner's word of chunk c - 2
      if constexpr (EARLY) {
      // ---- write, summed before the barrier: the slab is not written until every read of the chunk is done, but
      // the owners' sums use only their loaded rows, the staged values and the plan, so each wave adds its owned
      // rows (a crowded wave its teams' rows) while the other waves still read, and stores them after the barrier ----
      // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small); a chunk with a reset empties it
      const bool chunk_reset = reinterpret_cast<const uint32_t*>(varc)[1] & 0x80000000u;
      mu_new = mu * (L == kChunk ? lam_chunk : pw[L]);
      const bool rescale = !chunk_reset && !(mu_new >= kMuFloor);
      const float slab_scale = mu_new;
      if (chunk_reset) {   // the slab empties, the owners' loaded rows with it
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] = 0.f;
        cw_old = 0.f;
        mu_new = 1.f;
      } else if (rescale) {   // the slab is rescaled, the owners' loaded rows with it
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] *= mu_new;
        cw_old *= mu_new;
        mu_new = 1.f;
      }
      const float inv_mu = fast_rcp(mu_new);
      // every owner adds its own faded value to its loaded row
      float cw = cw_old;
      if (wslot != M) {
        const float a0 = __uint_as_float(wr.y) * inv_mu;
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] = fmaf(a0, vp[k], y[k]);
        cw += a0;
      }
      const int n_l_own = wslot != M ? static_cast<int>((wr.x >> 17) & 63u) : 0;
      const bool teams = __ballot(n_l_own >= kTeamWriters);
      // the teams of a crowded wave (as in the plain step): team j, the lanes of pick j of the wave's eight positions,
      // sums the owned slots of its members one after another and leaves each lane one four-column piece (h4) of the
      // member's row and the team the slot's count (ct)
      const unsigned long long owners = __ballot(wslot != M);
      const int mi = lane >> 3;   // the lane's member index in its team
      auto team_member = [&](int k, float (&h4)[4], float& ct, int& mslot) {
        const int src = 8 * k + j;
        const uint32_t mx = static_cast<uint32_t>(__shfl(static_cast<int>(wr.x), src));
        const uint32_t mz = static_cast<uint32_t>(__shfl(static_cast<int>(wr.z), src));
        mslot = static_cast<int>(mx & 0x7ffu);
        float part[32];
        float cwp = 0.f;
        const bool self = mi == k && mslot != M;   // the member itself: its row with its own value added
#pragma unroll
        for (int q = 0; q < 32; ++q) part[q] = self ? y[q] : 0.f;
        if (self) cwp = cw;
        if (mslot != M) {   // later writers mi, mi + 8, ...: 0 is the inline one, i > 0 entry w_e0 + i - 1
          const int n_l = static_cast<int>((mx >> 17) & 63u);
          const int w_e0 = static_cast<int>(mx >> 23);
          for (int i = mi; i < n_l; i += 8) {
            const uint2 it = i == 0 ? make_uint2(mz, (mx >> 11) & 63u) : ent_at(w_e0 + i - 1, std::false_type{});
            const float ae = __uint_as_float(it.x) * inv_mu;
            add_vrow(ae, static_cast<int>(it.y & 63u), part);
            cwp += ae;
          }
        }
        // over the team: lanes 32 apart (32 -> 16 values), 16 apart (-> 8), 8 apart (-> 4)
        float h16[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[q]), __float_as_uint(part[16 + q]),
                                                           false, false);
          h16[q] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);   // lane < 32: values q, else 16 + q
        }
        const bool b4 = lane & 16, b3 = lane & 8;
        float h8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float keep = b4 ? h16[8 + q] : h16[q];
          h8[q] = keep + __shfl_xor(b4 ? h16[q] : h16[8 + q], 16);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float keep = b3 ? h8[4 + q] : h8[q];
          h4[q] = keep + __int_as_float(__builtin_amdgcn_update_dpp(
                             0, __float_as_int(b3 ? h8[q] : h8[4 + q]), 0x128, 0xf, 0xf, false));   // row_ror:8
        }
        ct = cwp;
        ct += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ct), 0x128, 0xf, 0xf, false));
        ct += __shfl_xor(ct, 16);
        {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ct), __float_as_uint(ct), false, false);
          ct = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
      };
      // the team's store of member k's slot: the lane's piece (number mi of the read order) and the count
      auto team_store = [&](int k, const float (&h4)[4], float ct, int mslot) {
        if (mslot != M) {
          const int piece = j ^ (mi < 4 ? mi : 11 - mi);
          *reinterpret_cast<float4*>(A_w + mslot * (CW * 4) + 16 * piece) = make_float4(h4[0], h4[1], h4[2], h4[3]);
          if (mi == k) cnt[mslot] = ct;
        }
      };
      uint32_t members = 0;   // members with owned slots (bit k: member k)
#pragma unroll
      for (int k = 0; k < 8; ++k) members |= ((owners >> (8 * k)) & 0xffull) ? (1u << k) : 0u;
      // a team wave of one member (where every position of the chunk writes the same slots) sums it now
      const bool team_now = teams && __builtin_popcount(members) == 1;
      const int k1 = members ? __builtin_ctz(members) : 0;
      float h4a[4], cta;   // set and used only when team_now
      int msa;
      if (!teams) {
        if (wslot != M && n_l_own > 0) {   // the owner adds the slot's later writers
          const float a1 = __uint_as_float(wr.z) * inv_mu;
          add_vrow(a1, static_cast<int>((wr.x >> 11) & 63u), y);
          cw += a1;
          const int w_e0 = static_cast<int>(wr.x >> 23);   // the later writers past the first, among the entries
          for (int e = 0; e < n_l_own - 1; ++e) {
            const uint2 en = ent_at(w_e0 + e, std::false_type{});
            const float ae = __uint_as_float(en.x) * inv_mu;
            add_vrow(ae, static_cast<int>(en.y & 63u), y);
            cw += ae;
          }
        }
      } else if (team_now) {
        team_member(k1, h4a, cta, msa);
      }
      lds_barrier();
      // the partner's partial sums of chunk c - 2 (used when it finishes, at the end of this chunk)
      xo = (fin2 && G == 2) ? xget(c - 2, 1 - g) : 0ull;
      if (chunk_reset) {
        float4* a4 = reinterpret_cast<float4*>(A);
        for (int i = tid; i < (M + 1) * CW / 4; i += NT) a4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int i = tid; i <= M; i += NT) cnt[i] = 0.f;
        lds_barrier();
      } else if (rescale) {
        float4* a4 = reinterpret_cast<float4*>(A);
        for (int i = tid; i < (M + 1) * CW / 4; i += NT) {
          const float4 t = a4[i];
          a4[i] = make_float4(t.x * slab_scale, t.y * slab_scale, t.z * slab_scale, t.w * slab_scale);
        }
        for (int i = tid; i <= M; i += NT) cnt[i] *= slab_scale;
        lds_barrier();
      }
      // ---- write, stored: every owned slot has one owner (or one team), so the rows are written in a fixed order ----
      if (!teams) {
        if (wslot != M) {
          unsigned char* row = A_w + wslot * (CW * 4);
#pragma unroll
          for (int k = 0; k < 8; ++k)
            *reinterpret_cast<float4*>(row + soff[k]) = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
          cnt[wslot] = cw;
        }
      } else if (team_now) {
        team_store(k1, h4a, cta, msa);
      } else {
        for (int k = 0; k < 8; ++k) {   // several members: each summed and stored in turn, after the barrier
          if (!((members >> k) & 1u)) continue;
          float h4[4], ct;
          int ms;
          team_member(k, h4, ct, ms);
          team_store(k, h4, ct, ms);
        }
      }
      } else {
      lds_barrier();
      // the partner's partial sums of chunk c - 2 (used when it finishes, at the end of this chunk)
      xo = (fin2 && G == 2) ? xget(c - 2, 1 - g) : 0ull;
      // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small); a chunk with a reset empties it
      const bool chunk_reset = reinterpret_cast<const uint32_t*>(varc)[1] & 0x80000000u;
      mu_new = mu * (L == kChunk ? lam_chunk : pw[L]);
      if (chunk_reset) {   // the slab empties, the owners' loaded rows with it
        float4* a4 = reinterpret_cast<float4*>(A);
        for (int i = tid; i < (M + 1) * CW / 4; i += NT) a4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int i = tid; i <= M; i += NT) cnt[i] = 0.f;
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] = 0.f;
        cw_old = 0.f;
        mu_new = 1.f;
        lds_barrier();
      } else if (!(mu_new >= kMuFloor)) {   // the slab is rescaled, the owners' loaded rows with it
        float4* a4 = reinterpret_cast<float4*>(A);
        for (int i = tid; i < (M + 1) * CW / 4; i += NT) {
          const float4 t = a4[i];
          a4[i] = make_float4(t.x * mu_new, t.y * mu_new, t.z * mu_new, t.w * mu_new);
        }
        for (int i = tid; i <= M; i += NT) cnt[i] *= mu_new;
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] *= mu_new;
        cw_old *= mu_new;
        mu_new = 1.f;
        lds_barrier();
      }
      // ---- write: the owner lanes add their faded values and those of the slot's later writers ----
      const float inv_mu = fast_rcp(mu_new);
      // every owner adds its own faded value to its loaded row
      float cw = cw_old;
      if (wslot != M) {
        const float a0 = __uint_as_float(wr.y) * inv_mu;
#pragma unroll
        for (int k = 0; k < 32; ++k) y[k] = fmaf(a0, vp[k], y[k]);
        cw += a0;
      }
      const int n_l_own = wslot != M ? static_cast<int>((wr.x >> 17) & 63u) : 0;
      if (!__ballot(n_l_own >= kTeamWriters)) {
        if (wslot != M) {   // the owner adds the slot's later writers and stores the row
          const int n_l = n_l_own;
          unsigned char* row = A_w + wslot * (CW * 4);
          if (n_l > 0) {
            const float a1 = __uint_as_float(wr.z) * inv_mu;
            add_vrow(a1, static_cast<int>((wr.x >> 11) & 63u), y);
            cw += a1;
            if (n_l > 1) {   // later writers past the first, from the variable part
              const int w_e0 = static_cast<int>(wr.x >> 23);   // the first of them among the entries
              auto later = [&](auto st) {
                for (int e = 0; e < n_l - 1; ++e) {
                  const uint2 en = ent_at(w_e0 + e, st);
                  const float ae = __uint_as_float(en.x) * inv_mu;
                  add_vrow(ae, static_cast<int>(en.y & 63u), y);
                  cw += ae;
                }
              };
              if (all_staged) later(std::true_type{});
              else later(std::false_type{});
            }
          }
#pragma unroll
          for (int k = 0; k < 8; ++k)
            *reinterpret_cast<float4*>(row + soff[k]) = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
          cnt[wslot] = cw;
        }
      } else {
        // A wave with a slot of many later writers (crowded addresses) writes as eight teams: team j, the lanes of
        // pick j of the wave's eight positions, takes the owned slots of its members one after another; the member's
        // row (its own value added) and the slot's later writers (every eighth, from the member's index in the team)
        // are summed per lane, then over the team (lanes 8 apart) by a fixed butterfly that leaves each lane one
        // four-column piece of the row, which it stores.
        const unsigned long long owners = __ballot(wslot != M);
        const int mi = lane >> 3;   // the lane's member index in its team
        auto team = [&](auto st) {
          for (int k = 0; k < 8; ++k) {
            if (!((owners >> (8 * k)) & 0xffull)) continue;   // no owner among the teams' members k
            const int src = 8 * k + j;
            const uint32_t mx = static_cast<uint32_t>(__shfl(static_cast<int>(wr.x), src));
            const uint32_t mz = static_cast<uint32_t>(__shfl(static_cast<int>(wr.z), src));
            const int mslot = static_cast<int>(mx & 0x7ffu);
            float part[32];
            float cwp = 0.f;
            const bool self = mi == k && mslot != M;   // the member itself: its row with its own value added
#pragma unroll
            for (int q = 0; q < 32; ++q) part[q] = self ? y[q] : 0.f;
            if (self) cwp = cw;
            if (mslot != M) {   // later writers mi, mi + 8, ...: 0 is the inline one, i > 0 entry w_e0 + i - 1
              const int n_l = static_cast<int>((mx >> 17) & 63u);
              const int w_e0 = static_cast<int>(mx >> 23);
              for (int i = mi; i < n_l; i += 8) {
                const uint2 it = i == 0 ? make_uint2(mz, (mx >> 11) & 63u) : ent_at(w_e0 + i - 1, st);
                const float ae = __uint_as_float(it.x) * inv_mu;
                add_vrow(ae, static_cast<int>(it.y & 63u), part);
                cwp += ae;
              }
            }
            // over the team: lanes 32 apart (32 -> 16 values), 16 apart (-> 8), 8 apart (-> 4)
            float h16[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[q]), __float_as_uint(part[16 + q]),
                                                               false, false);
              h16[q] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);   // lane < 32: values q, else 16 + q
            }
            const bool b4 = lane & 16, b3 = lane & 8;
            float h8[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              const float keep = b4 ? h16[8 + q] : h16[q];
              h8[q] = keep + __shfl_xor(b4 ? h16[q] : h16[8 + q], 16);
            }
            float h4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float keep = b3 ? h8[4 + q] : h8[q];
              h4[q] = keep + __int_as_float(__builtin_amdgcn_update_dpp(
                                 0, __float_as_int(b3 ? h8[q] : h8[4 + q]), 0x128, 0xf, 0xf, false));   // row_ror:8
            }
            float ct = cwp;
            ct += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ct), 0x128, 0xf, 0xf, false));
            ct += __shfl_xor(ct, 16);
            {
              const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ct), __float_as_uint(ct), false, false);
              ct = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            }
            if (mslot != M) {   // the lane's piece: number mi of the read order
              const int piece = j ^ (mi < 4 ? mi : 11 - mi);
              *reinterpret_cast<float4*>(A_w + mslot * (CW * 4) + 16 * piece) = make_float4(h4[0], h4[1], h4[2], h4[3]);
              if (mi == k) cnt[mslot] = ct;
            }
          }
        };
        team(std::false_type{});   // rare: one instance, the entries staged or not
      }
      }
      mu = mu_new;
      rr = rr_n;
      wr = wr_n;
      v_cur = v_n;
      stage(c + 1, v_n, var_n);   // buffer (c + 1) & 1 held chunk c - 1, done before the last barrier
      if (fin2) finish(c - 2, rq[2], sq[2], xo);
      lds_barrier();
    }
  };
  if (crowded) chunk_loop(std::true_type{});
  else chunk_loop(std::false_type{});
  if (xnorm) {   // the last two chunks (or one)
    const int n = a.n_chunks;
    if (n >= 2) finish(n - 2, rq[1], sq[1], G == 2 ? xget(n - 2, 1 - g) : 0ull);
    finish(n - 1, rq[0], sq[0], G == 2 ? xget(n - 1, 1 - g) : 0ull);
  }

  if (a.state_out_mem) {
    for (int i = tid; i < M * CW; i += NT) {
      const int m = i / CW;
      const int cc = i - m * CW;
      a.state_out_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] = mu * A[i];
    }
  }
  if (a.state_out_cnt && g == 0) {
    for (int m = tid; m < M; m += NT) a.state_out_cnt[static_cast<int64_t>(s) * M + m] = mu * cnt[m];
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
