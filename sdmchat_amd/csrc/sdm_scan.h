// sdm_scan.h -- scan_kernel: executes the chunk plans of one (batch row, head) slab over a group of CW of its value
// columns, with the read-out finished in place (RunTimeSdm._chunk, forward and finish,
// experiments/track4/sdmllm/track4_onesdm_models.py:215-247 without wo).  Included by sdm_scan_bf16.hip and
// sdm_scan_f32.hip, which instantiate it per value type.
//
// Decay bookkeeping: the slab holds A with the true state S = mu * A (mu a per-slab scalar).  A chunk of L positions
// reads mu * lam^p * A[slot] at offset p, then mu <- mu * lam^L and each write at offset q adds lam^(L-1-q) / mu *
// w * v.  When mu falls below 2^-60 the slab is multiplied by mu once and mu reset to 1, so lam = 0 (keep only the
// previous write) and lam = 1 (never fade) are exact and the slab is rarely rescaled.
//
// The out-norm needs all dh columns of a head, which G = dh / CW workgroups share.  Each workgroup publishes the
// per-position sum of squares of its columns of a chunk (xch) and a progress counter (sync), and finishes a chunk's
// read-out two chunks later, once every other group of its slab has published that chunk; all groups add the G
// partial sums in the same order, so they scale by the same factor.  The G groups of a slab are placed on one XCD
// and next to each other in its dispatch order (workgroup w runs on XCD w % 8), so they start together and share an
// L2; a group waits only for groups of its own slab, and every wait is bounded (a status word records a time-out).
#pragma once

#include "sdm_plan.h"

namespace sdmrt {

struct ScanArgs {
  const unsigned char* plans;  // [S][n_chunks][stride]
  const int32_t* sizes;        // [S][n_chunks]
  const void* v;               // value rows
  int64_t v_stride;
  const float* decay;          // [H]
  const float* onorm_w;        // [H][dh], or nullptr: no out-norm
  const float* state_in_mem;   // [S][M][dh] or nullptr
  const float* state_in_cnt;   // [S][M] or nullptr
  float* state_out_mem;
  float* state_out_cnt;
  void* r_out;                 // rows of H * dh read-outs; OutT
  int64_t r_stride;
  float* read_out;             // rows of H * dh float32: the read before the out-norm, or nullptr
  float* den_out;              // [B*T][H] read denominators (mean read), or nullptr
  uint32_t* sync;              // [S][groups] progress counters, then a status word
  float* xch;                  // [S][n_chunks][groups][64] partial sums of squares
  int S, T, H, dh, M, n_chunks, groups, read_mean;
  int sync_stride;             // progress counters per slab in sync (at least groups)
  int v_direct;                // 1: value rows are 16-byte aligned and copied into LDS directly
  float read_eps, out_eps;
  uint32_t spin_limit;         // polls of a partner's progress before a wait gives up (0: give up at once)
  int crowded_bytes;           // pick scan: a chunk plan's variable part past this makes its slab crowded
};

constexpr uint32_t kSpinLimit = 1u << 20;   // the default polls of a partner's progress before a wait gives up

// the polls a wait makes before it gives up, process-wide (sdm_rt_set_wait_limit)
uint32_t wait_limit();
// the pick scan's crowded-slab threshold in plan bytes, process-wide (sdm_rt_set_crowded_threshold)
int crowded_threshold();

// CPL consecutive float values from LDS in one access
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

// 8 consecutive floats of a slab row, and 8 consecutive values of a value row, from LDS (16-byte accesses)
__device__ __forceinline__ void lds_row8(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void lds_row8_store(float* p, const float (&v)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void lds_vals8(const float* p, float (&v)[8]) { lds_row8(p, v); }
__device__ __forceinline__ void lds_vals8(const bf16_t* p, float (&v)[8]) {
  const uint4 t = *reinterpret_cast<const uint4*>(p);
  const uint32_t wd[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __uint_as_float(wd[q] << 16);
    v[2 * q + 1] = __uint_as_float(wd[q] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint32_t u4_word(const uint4& q, int i) {
  return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// relaxed, device-coherent accesses of the progress counters and partial sums (sc1: no stale cache line)
__device__ __forceinline__ uint32_t load_sync(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_sync(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_xch(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_xch(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 1 / sqrt(x) for positive normal x: hardware reciprocal square root and one Newton step
__device__ __forceinline__ float fast_rsqrt(float x) {
  const float y = __builtin_amdgcn_rsqf(x);
  return y * fmaf(-0.5f * x * y, y, 1.5f);
}

// direct copies of 16-byte pieces from global memory into LDS: lane l of the calling wave moves src (its own
// address) to dst_wave + 16 l (dst_wave the same in every lane); counted by vmcnt, like a load
__device__ __forceinline__ void copy_to_lds(const void* src, void* dst_wave) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                             reinterpret_cast<uintptr_t>(dst_wave)), 16, 0, 0);
}

// Scan of one slab over CW of its value columns, 512 threads = 64 positions x 8 lanes of CPL = CW / 8 columns.
// Per chunk:
//   read   mu * lam^p * the rows of the position's read picks (pads read row M, which stays zero), plus its in-chunk
//          contributions (kInline in the record, the rest from the variable part); the mean read divides by
//          mu * lam^p * sum(w * cnt) + the in-chunk coefficient sum; then the out-norm (with more than one column
//          group, its partial sum of squares: the read-out finishes two chunks later)
//   write  the position's owned picks, faded values divided by mu after the fade (picks it does not own point at
//          row M and are masked off); then the slots written more than once take their later writers, one group
//          per slot; lane l adds pick l's coefficients to its slot's count
// The next chunk's position records, values and variable part are copied from global memory into LDS by the
// waves themselves (16-byte direct copies issued after the read), so no register waits for a load in flight and
// the copies stream while the chunk writes.  Every slot has one owner, so no two groups change one row, and all sums
// run in fixed orders: the results are deterministic.
template <int CW, int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(kScanThreads) scan_kernel(ScanArgs a) {
  constexpr int CPL = CW / 8;
  constexpr PlanGeom pg{KP};
  constexpr int VS = kVarStage;
  constexpr int NR = pg.pos_bytes() / 16;                   // 16-byte words of a position record
  constexpr int REC_PIECES = kChunk * pg.pos_bytes() / 16;  // a multiple of 64 (64 (KP + 3))
  constexpr int V_ROW = CW * static_cast<int>(sizeof(VT));  // bytes of a position's values in the group
  constexpr int V_PIECES = kChunk * V_ROW / 16;             // 64, 128 or 256
  constexpr int kShift = CW == 32 ? 5 : CW == 16 ? 4 : 3;   // row offset >> kShift = slot * 4 (the count's offset)
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int M = a.M;
  const int G = a.groups;
  // workgroup -> (slab, column group): the G groups of slab 8 j + x are workgroups 8 (G j + g) + x
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int jr = (bid >> 3) / G;
  const int g = (bid >> 3) - jr * G;
  const int s = 8 * jr + xcd;
  if (s >= a.S) return;
  const int b = s / a.H;
  const int h = s - b * a.H;
  float* A = lds;                                                        // [M + 1][CW]
  float* cnt = A + static_cast<size_t>(M + 1) * CW;                      // [M + 1]
  VT* s_v = reinterpret_cast<VT*>(cnt + pad4(M + 1));                    // [2][64][CW], by chunk parity
  unsigned char* var = reinterpret_cast<unsigned char*>(s_v + 2 * kChunk * CW);   // [2][VS], by chunk parity
  unsigned char* recs = var + 2 * VS;                                    // [64][pos_bytes]
  float* pw = reinterpret_cast<float*>(recs + kChunk * pg.pos_bytes());
  int32_t* s_sizes = reinterpret_cast<int32_t*>(pw + 68);   // read from LDS: a scalar load in the loop would hold up
                                                            // every LDS wait behind a memory round trip
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int p = tid >> 3;
  const int l8 = tid & 7;
  const int col0 = g * CW;
  const int cl = CPL * l8;   // the lane's first column in the group
  const float lam = a.decay[h];
  const bool norm = a.onorm_w != nullptr;
  const bool xnorm = norm && G > 1;   // the out-norm needs the other groups' partial sums
  const unsigned char* A_lane = reinterpret_cast<const unsigned char*>(A + cl);   // + row offset = the lane's segment
  unsigned char* A_lane_w = reinterpret_cast<unsigned char*>(A + cl);
  unsigned char* cnt_b = reinterpret_cast<unsigned char*>(cnt);
  const unsigned char* plans_s = a.plans + static_cast<int64_t>(s) * a.n_chunks * pg.stride();
  const VT* v_b = static_cast<const VT*>(a.v) + static_cast<int64_t>(b) * a.T * a.v_stride +
                  static_cast<int64_t>(h) * a.dh + col0;

  for (int i = tid; i < (M + 1) * CW; i += kScanThreads) {
    const int m = i / CW;
    const int cc = i - m * CW;
    A[i] = (a.state_in_mem && m < M) ? a.state_in_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] : 0.f;
  }
  for (int m = tid; m <= M; m += kScanThreads)
    cnt[m] = (a.state_in_cnt && m < M) ? a.state_in_cnt[static_cast<int64_t>(s) * M + m] : 0.f;
  for (int i = tid; i < a.n_chunks; i += kScanThreads) s_sizes[i] = a.sizes[static_cast<int64_t>(s) * a.n_chunks + i];
  if (tid <= kChunk) {
    float v = 1.f, sq = lam;   // lam^tid by squaring (as the plan computes it; exact for lam = 0 and lam = 1)
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      v = ((tid >> bit) & 1) ? v * sq : v;
      sq *= sq;
    }
    pw[tid] = v;
  }
  float onw[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) onw[k] = norm ? a.onorm_w[h * a.dh + col0 + cl + k] : 1.f;
  float mu = 1.f;

  // chunk c's records, values and variable part into LDS (the variable part's sizes come from global memory here,
  // as the copy may run before s_sizes is written).  Every lane copies a valid source (indexes clamped); copies past
  // a part's size land in the unused rest of its buffer.
  auto copy_chunk = [&](int c, int bytes) {
    const unsigned char* base = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(pg.stride());
    for (int blk = wave; blk * 64 < REC_PIECES; blk += kScanThreads / 64)
      copy_to_lds(base + 16 * (blk * 64 + lane), recs + 1024 * blk);
    const int pieces = min((bytes + 15) >> 4, VS / 16);
    for (int blk = wave; blk * 64 < VS / 16; blk += kScanThreads / 64)
      copy_to_lds(base + pg.off_var() + 16 * min(blk * 64 + lane, max(pieces - 1, 0)),
                  var + (c & 1) * VS + 1024 * blk);
    if (a.v_direct) {
      for (int blk = wave; blk * 64 < V_PIECES; blk += kScanThreads / 64) {
        const int piece = blk * 64 + lane;
        const int pos = piece / (V_ROW / 16), part = piece - pos * (V_ROW / 16);
        const int row = min(c * kChunk + pos, a.T - 1);
        copy_to_lds(v_b + static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_stride) + part * (16 / static_cast<int>(sizeof(VT))),
                    reinterpret_cast<unsigned char*>(s_v) + (c & 1) * kChunk * V_ROW + 1024 * blk);
      }
    } else {   // values whose rows are not 16-byte aligned: through registers (a wait for the loads here)
      const int row = min(c * kChunk + p, a.T - 1);
      const VT* vr = v_b + static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_stride) + cl;
      VT* dst = s_v + (c & 1) * kChunk * CW + p * CW + cl;
#pragma unroll
      for (int k = 0; k < CPL; ++k) dst[k] = vr[k];
    }
  };
  auto store_r = [&](int c, int pos, const float (&x)[CPL]) {
    OutT* dst = static_cast<OutT*>(a.r_out) + (static_cast<int64_t>(b) * a.T + c * kChunk + pos) * a.r_stride +
                static_cast<int64_t>(h) * a.dh + col0 + cl;
    store_vals<CPL, OutT>(dst, x);
  };
  uint32_t* my_sync = a.sync + static_cast<int64_t>(s) * a.sync_stride;
  // The out-norm of chunk c finishes two chunks later, in three steps whose loads overlap other work: poll (issue
  // the load of every other group's progress counter), wait (until each has published chunk c: a bounded spin that
  // rarely runs) and gather (issue the loads of their partial sums; with two groups the one partial sum is loaded
  // into xo here, with more groups they are loaded when the chunk finishes).
  auto poll = [&]() { return (lane < G && lane != g) ? load_sync(my_sync + lane) : 0xffffffffu; };
  auto wait_published = [&](uint32_t got, int c) {
    const uint32_t need = static_cast<uint32_t>(c) + 1u;
    if (a.spin_limit == 0) got = 0u;   // waits give up at once (the error path's test)
    bool ok = true;
    if (__ballot(got < need)) {   // the first check outside the spin loop, whose own waits are for everything
      for (uint32_t it = 0;; ++it) {
        if (it >= a.spin_limit) {
          if (lane == 0) store_sync(a.sync + static_cast<int64_t>(a.S) * a.sync_stride, 1u);
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        got = poll();
        if (!__ballot(got < need)) break;
      }
    }
    asm volatile("" ::: "memory");
    return ok;
  };
  auto xch_at = [&](int c) { return a.xch + (static_cast<int64_t>(s) * a.n_chunks + c) * G * kChunk + p; };
  auto gather = [&](int c) { return G == 2 ? load_xch(xch_at(c) + (1 - g) * kChunk) : 0.f; };
  // ok = false: the wait for the other groups gave up, and the chunk's read-outs are NaN
  auto finish = [&](int c, const float (&x)[CPL], float ss, float xo, bool ok) {
    const int L = min(kChunk, a.T - c * kChunk);
    if (p < L) {
      float tot;
      if (G == 2) {
        tot = g == 0 ? ss + xo : xo + ss;   // group order, the same sum in both groups
      } else {
        tot = 0.f;
        for (int gg = 0; gg < G; ++gg) tot += gg == g ? ss : load_xch(xch_at(c) + gg * kChunk);
      }
      if (!ok) tot = __builtin_nanf("");
      const float inv = fast_rsqrt(tot * (1.f / static_cast<float>(a.dh)) + a.out_eps);
      float o[CPL];
#pragma unroll
      for (int k = 0; k < CPL; ++k) o[k] = x[k] * inv * onw[k];
      store_r(c, p, o);
    }
  };
  // the read-outs of the last three chunks and their sums of squares (rotated by copies: 5 values a chunk)
  float rq[3][CPL] = {};
  float sq[3] = {0.f, 0.f, 0.f};

  copy_chunk(0, a.sizes[static_cast<int64_t>(s) * a.n_chunks]);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the copies are in LDS
  lds_barrier();
  const float lam_chunk = pw[kChunk];   // the fade of a full chunk, kept in a register
  const float inv_dh = 1.f / static_cast<float>(a.dh);
  const uint32_t null_b = static_cast<uint32_t>(M) * static_cast<uint32_t>(CW * sizeof(float));

  for (int c = 0; c < a.n_chunks; ++c) {
    const bool fin2 = xnorm && c >= 2;   // chunk c - 2 finishes at the end of this chunk
    uint32_t got = 0u;
    if (fin2) got = poll();
    if (xnorm && c > 0 && tid == 0) store_sync(my_sync + g, static_cast<uint32_t>(c));   // chunks < c published
    const int c0 = c * kChunk;
    const int L = min(kChunk, a.T - c0);
    const unsigned char* varc = var + (c & 1) * VS;
    const VT* s_vc = s_v + (c & 1) * kChunk * CW;
    // this chunk's record (the eight lanes of a position read the same words: LDS broadcasts them)
    uint4 rr[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) rr[k] = reinterpret_cast<const uint4*>(recs + p * pg.pos_bytes())[k];
    const uint32_t* rw32 = reinterpret_cast<const uint32_t*>(recs + p * pg.pos_bytes());
    uint32_t own_roff[KP / 8], own_woff[KP / 8], own_wc[KP / 8];
    float own_rw[KP / 8];
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) {   // the lane's count entries: picks l8 (and l8 + 8)
      own_roff[k] = rw32[l8 + 8 * k];
      own_rw[k] = __uint_as_float(rw32[pg.off_rw() / 4 + l8 + 8 * k]);
      own_woff[k] = rw32[pg.off_woff() / 4 + l8 + 8 * k];
      own_wc[k] = rw32[pg.off_wc() / 4 + l8 + 8 * k];
    }
    auto rec = [&](int i) { return u4_word(rr[i / 4], i % 4); };
    constexpr int TW = pg.off_tail() / 4;
    const uint32_t t0 = rec(TW);
    const float csum = __uint_as_float(rec(TW + 1));
    const int n_in = static_cast<int>(t0 & 0xffffu), ro = static_cast<int>(t0 >> 16);
    const int bytes = s_sizes[c];
    const bool all_staged = bytes <= VS;
    const unsigned char* gvar = plans_s + static_cast<uint32_t>(c) * static_cast<uint32_t>(pg.stride()) + pg.off_var();
    // variable-part entries: from LDS within the staged bytes, else from the plan in global memory.  The two code
    // paths stay separate (st = std::true_type: LDS only): a global load on a joined path makes every later wait
    // wait for all vector-memory loads in flight.
    auto ent_at = [&](int e, auto st) {
      const int o = 16 + 8 * min(max(e, 0), pg.max_entries() - 1);   // inside the plan whatever the entry index
      if constexpr (decltype(st)::value) return *reinterpret_cast<const uint2*>(varc + o);
      else return o + 8 <= VS ? *reinterpret_cast<const uint2*>(varc + o) : *reinterpret_cast<const uint2*>(gvar + o);
    };

    // read: every load issued first
    const float fin = mu * pw[p];
    Seg<CPL> x[KP], vi[kInline];
#pragma unroll
    for (int i = 0; i < KP; ++i) x[i] = lds_seg<CPL>(reinterpret_cast<const float*>(A_lane + rec(i)));
#pragma unroll
    for (int t = 0; t < kInline; ++t) {   // only the contributions the position has (LDS bandwidth)
      if (t < n_in) vi[t] = lds_seg<CPL>(&s_vc[((rec(TW + 2 + t / 4) >> (8 * (t % 4))) & 63u) * CW + cl]);
      else
#pragma unroll
        for (int k = 0; k < CPL; ++k) vi[t].v[k] = 0.f;
    }
    float cval[KP / 8];
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) cval[k] = *reinterpret_cast<const float*>(cnt_b + (own_roff[k] >> kShift));
    float acc[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const float w = __uint_as_float(rec(pg.off_rw() / 4 + i));
#pragma unroll
      for (int k = 0; k < CPL; ++k) acc[k] = fmaf(w, x[i].v[k], acc[k]);
    }
#pragma unroll
    for (int k = 0; k < CPL; ++k) acc[k] *= fin;
#pragma unroll
    for (int t = 0; t < kInline; ++t) {
      const float cf = __uint_as_float(rec(TW + 4 + t));
#pragma unroll
      for (int k = 0; k < CPL; ++k) acc[k] = fmaf(cf, vi[t].v[k], acc[k]);
    }
    if (n_in > kInline) {   // contributions past the inline ones (rare: the branch diverges between positions)
      auto over = [&](auto st) {
        for (int e = 0; e < n_in - kInline; ++e) {
          const uint2 t = ent_at(ro + e, st);
          const Seg<CPL> vq = lds_seg<CPL>(&s_vc[(t.y & 63u) * CW + cl]);
#pragma unroll
          for (int k = 0; k < CPL; ++k) acc[k] = fmaf(__uint_as_float(t.x), vq.v[k], acc[k]);
        }
      };
      if (all_staged) over(std::true_type{});
      else over(std::false_type{});
    }
    float cp = 0.f;   // lane l8: picks l8 (and l8 + 8)
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) cp = fmaf(own_rw[k], cval[k], cp);
    float den = sum8(cp);
    if (a.read_mean) {
      den = fmaf(fin, den, csum);
      if (a.den_out && g == 0 && l8 == 0 && p < L) a.den_out[(static_cast<int64_t>(b) * a.T + c0 + p) * a.H + h] = den;
      const float inv = fast_rcp(den + a.read_eps);
#pragma unroll
      for (int k = 0; k < CPL; ++k) acc[k] *= inv;
    }
    if (a.read_out && p < L) {
      float* dst = a.read_out + (static_cast<int64_t>(b) * a.T + c0 + p) * static_cast<int64_t>(a.H) * a.dh +
                   static_cast<int64_t>(h) * a.dh + col0 + cl;
      store_vals<CPL, float>(dst, acc);
    }
    if (norm) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < CPL; ++k) ss = fmaf(acc[k], acc[k], ss);
      ss = sum8(ss);
      if (xnorm) {
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
          rq[2][k] = rq[1][k];
          rq[1][k] = rq[0][k];
          rq[0][k] = acc[k];
        }
        sq[2] = sq[1];
        sq[1] = sq[0];
        sq[0] = ss;
        if (l8 == 0) store_xch(a.xch + ((static_cast<int64_t>(s) * a.n_chunks + c) * G + g) * kChunk + p, ss);
      } else if (p < L) {
        const float inv = fast_rsqrt(ss * inv_dh + a.out_eps);
        float o[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) o[k] = acc[k] * inv * onw[k];
        store_r(c, p, o);
      }
    } else if (p < L) {
      store_r(c, p, acc);
    }
    // the values of the owner's writes, read while the records are still in LDS
    const Seg<CPL> vown = lds_seg<CPL>(&s_vc[p * CW + cl]);
    lds_barrier();
    float xo = 0.f;
    bool xok = true;
    if (fin2) {
      xok = wait_published(got, c - 2);
      xo = gather(c - 2);
    }
    // the next chunk's records, values and variable part stream into LDS while this chunk writes
    if (c + 1 < a.n_chunks) copy_chunk(c + 1, s_sizes[c + 1]);
    // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small); a chunk with a reset empties it
    const bool chunk_reset = reinterpret_cast<const uint32_t*>(varc)[1] & 0x80000000u;
    float mu_new = mu * (L == kChunk ? lam_chunk : pw[L]);
    if (chunk_reset) {
      float4* a4 = reinterpret_cast<float4*>(A);
      for (int i = tid; i < (M + 1) * CW / 4; i += kScanThreads) a4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int i = tid; i <= M; i += kScanThreads) cnt[i] = 0.f;
      mu_new = 1.f;
      lds_barrier();
    } else if (!(mu_new >= kMuFloor)) {
      for (int i = tid; i < (M + 1) * CW; i += kScanThreads) A[i] *= mu_new;
      for (int i = tid; i <= M; i += kScanThreads) cnt[i] *= mu_new;
      mu_new = 1.f;
      lds_barrier();
    }
    // write, owners: the position's owned picks (picks it does not own point at row M: their accesses are masked
    // off), every load issued first
    const float inv_mu = fast_rcp(mu_new);
    {
      Seg<CPL> y[KP];
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        if (rec(pg.off_woff() / 4 + i) != null_b) y[i] = lds_seg<CPL>(reinterpret_cast<const float*>(A_lane + rec(pg.off_woff() / 4 + i)));
        else
#pragma unroll
          for (int k = 0; k < CPL; ++k) y[i].v[k] = 0.f;
      }
      float cold[KP / 8];
#pragma unroll
      for (int k = 0; k < KP / 8; ++k) cold[k] = *reinterpret_cast<const float*>(cnt_b + (own_woff[k] >> kShift));
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        const float cf = __uint_as_float(rec(pg.off_wc() / 4 + i)) * inv_mu;
#pragma unroll
        for (int k = 0; k < CPL; ++k) y[i].v[k] = fmaf(cf, vown.v[k], y[i].v[k]);
      }
#pragma unroll
      for (int i = 0; i < KP; ++i)
        if (rec(pg.off_woff() / 4 + i) != null_b)
          lds_seg_store<CPL>(reinterpret_cast<float*>(A_lane_w + rec(pg.off_woff() / 4 + i)), y[i]);
#pragma unroll
      for (int k = 0; k < KP / 8; ++k)   // lane l8's counts: picks l8 (and l8 + 8)
        *reinterpret_cast<float*>(cnt_b + (own_woff[k] >> kShift)) = fmaf(__uint_as_float(own_wc[k]), inv_mu, cold[k]);
    }
    // write, later writers: the slots written more than once take their later writers' values (from LDS), one
    // group per slot after the owners (n_x is the same for the whole workgroup)
    const int x0 = static_cast<int>(reinterpret_cast<const uint32_t*>(varc)[2]);
    const int n_x = static_cast<int>(reinterpret_cast<const uint32_t*>(varc)[3]);
    if (n_x > 0) {
      lds_barrier();
      // CW / 8 lanes per slot, 8 columns each: 64 * 8 / CPL slots at a time (one round for the usual n_x)
      constexpr int LPS = CW / 8;
      const int l_s = tid % LPS, grp = tid / LPS;
      auto later = [&](auto st) {
        for (int r = grp; r < n_x; r += kScanThreads / LPS) {
          const uint2 xr = ent_at(x0 + r, st);
          float* row = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(A + 8 * l_s) + xr.x);
          float* crow = reinterpret_cast<float*>(cnt_b + (xr.x >> kShift));
          float z[8];
          lds_row8(row, z);
          const float cold = *crow;
          const int e0 = static_cast<int>(xr.y & 0xffffu), n = min(static_cast<int>(xr.y >> 16), kChunk);
          float csum_w = 0.f;
          for (int e = 0; e < n; e += 2) {   // two writers at a time (the second one's weight is 0 past n)
            const uint2 e_0 = ent_at(e0 + e, st);
            const uint2 e_1 = ent_at(e0 + min(e + 1, n - 1), st);
            const float c_0 = __uint_as_float(e_0.x) * inv_mu;
            const float c_1 = e + 1 < n ? __uint_as_float(e_1.x) * inv_mu : 0.f;
            float v0[8], v1[8];
            lds_vals8(&s_vc[(e_0.y & 63u) * CW + 8 * l_s], v0);
            lds_vals8(&s_vc[(e_1.y & 63u) * CW + 8 * l_s], v1);
#pragma unroll
            for (int k = 0; k < 8; ++k) z[k] = fmaf(c_1, v1[k], fmaf(c_0, v0[k], z[k]));
            csum_w += c_0 + c_1;
          }
          lds_row8_store(row, z);
          if (l_s == 0) *crow = cold + csum_w;
        }
      };
      if (all_staged) later(std::true_type{});
      else later(std::false_type{});
    }
    mu = mu_new;
    // the copies (and this chunk's partial sums, which the next chunk publishes) are complete before the barrier;
    // they were issued a whole write phase ago
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    if (fin2) finish(c - 2, rq[2], sq[2], xo, xok);
    lds_barrier();
  }
  if (xnorm) {   // the last two chunks (or one)
    const int n = a.n_chunks;
    if (tid == 0) store_sync(my_sync + g, static_cast<uint32_t>(n));
    const bool ok = wait_published(poll(), n - 1);
    if (n >= 2) finish(n - 2, rq[1], sq[1], gather(n - 2), ok);
    finish(n - 1, rq[0], sq[0], gather(n - 1), ok);
  }

  if (a.state_out_mem) {
    for (int i = tid; i < M * CW; i += kScanThreads) {
      const int m = i / CW;
      const int cc = i - m * CW;
      a.state_out_mem[(static_cast<int64_t>(s) * M + m) * a.dh + col0 + cc] = mu * A[i];
    }
  }
  if (a.state_out_cnt && g == 0) {
    for (int m = tid; m < M; m += kScanThreads) a.state_out_cnt[static_cast<int64_t>(s) * M + m] = mu * cnt[m];
  }
}

template <int CW, int KP, typename VT, typename OutT>
int launch_scan_t(const Plan& p, const ScanArgs& a, hipStream_t st) {
  const size_t lds = scan_lds_bytes(p.M, CW, p.n_chunks, KP, static_cast<int>(sizeof(VT)));
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel<CW, KP, VT, OutT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     static_cast<int>(kLdsBytes));
  if (attr != hipSuccess) return set_err(SDM_RT_ELAUNCH, "scan: cannot enable %zu bytes of LDS", kLdsBytes);
  if (a.groups * CW != p.dh || a.sync_stride < a.groups)
    return set_err(SDM_RT_EINVAL, "scan: %d groups of %d columns for head_dim %d", a.groups, CW, p.dh);
  const int slabs8 = (p.B * p.H + 7) / 8 * 8;
  hipLaunchKernelGGL((scan_kernel<CW, KP, VT, OutT>), dim3(slabs8 * a.groups), dim3(kScanThreads), lds, st, a);
  return check_launch("scan");
}

template <typename VT, typename OutT>
int launch_scan_v(const Plan& p, const ScanArgs& a, hipStream_t st) {
#define SDM_RT_SCAN_CW(CW) \
  return p.pitch == 8 ? launch_scan_t<CW, 8, VT, OutT>(p, a, st) : launch_scan_t<CW, 16, VT, OutT>(p, a, st)
  switch (sizeof(VT) == 2 ? p.cw : p.cw32) {
    case 32: SDM_RT_SCAN_CW(32);
    case 16: SDM_RT_SCAN_CW(16);
    case 8: SDM_RT_SCAN_CW(8);
    default: return set_err(SDM_RT_EUNSUPPORTED, "no scan column group fits in LDS");
  }
#undef SDM_RT_SCAN_CW
}

// defined in sdm_scan_bf16.hip and sdm_scan_f32.hip (values in bfloat16 or float32), for either output type
int launch_scan_bf16(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st);
int launch_scan_f32(const Plan& p, const ScanArgs& a, sdm_rt_dtype out_dtype, hipStream_t st);

}  // namespace sdmrt
