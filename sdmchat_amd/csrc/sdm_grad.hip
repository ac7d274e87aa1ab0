// sdm_grad.hip -- the backward of the run-time SDM core (sdm_rt_forward_train, sdm_rt_backward) and of TrainedSdm's
// table layer (sdm_rt_table_backward).
//
// The gradient of RunTimeSdm.forward (track4_onesdm_models.py:195-274, the part between the projections and wo) for
// picks held fixed (topk and the slot ids carry no gradient).  With K[t][s] = lam^(t-1-s) sum_ij wr[t,i] ww[s,j]
// [sir[t,i] = siw[s,j]] (same segment, s < t), num_t = sum_s K[t][s] V_s, den_t = sum_s K[t][s] and, from the
// read-out norm and the mean, dnum_t and dden_t:
//   X[t][s]   = <dnum_t, V_s> + dden_t
//   dwr[t,i]  = sum_{s<t} lam^(t-1-s) sum_j ww[s,j] [match] X[t][s]  = <dnum_t, mem_t[sir_i]> + dden_t cnt_t[sir_i]
//   dww[s,j]  = sum_{t>s} lam^(t-1-s) sum_i wr[t,i] [match] X[t][s]  = <V_s, B_s[siw_j]> + Bc_s[siw_j]
//   dV_s      = sum_j ww[s,j] B_s[siw_j]
// where mem/cnt is the forward memory and B/Bc the adjoint memory written by the reads (slots sir, weights wr,
// values dnum, counts dden) and read by the writes, in reverse time.  Both are one kernel, grad_scan_kernel: a strict
// causal scan whose reads return, per pick, the dot of the row read with a per-position vector (and optionally the
// weighted sum of the rows).  The forward direction gives dwr, the reverse direction dww and dV.  Then
// addr_grad_kernel takes the softmax, gate, address normalisation and sub-key products back (pk_address :134-148,
// prepare :199-207) and grad_reduce / keys_grad_kernel sum the parameter gradients in a fixed order.
//
// lam * dL/dlam (the gradient with respect to log lam) needs no extra pass: sum_{t,s} (t-1-s) K[t][s] X[t][s]
// = sum_t t P_t - sum_s (s+1) Q_s with P_t = sum_i wr[t,i] dwr[t,i] and Q_s = sum_j ww[s,j] dww[s,j].

#include <hipcub/hipcub.hpp>

#include "sdm_scan.h"

namespace sdmrt {

constexpr int kGradScanThreads = 512;   // grad scans: 64 positions x 8 lanes


// ---------------------------------------------------------------------------------------------------------------
// read-out backward: out-norm (finish :243-246) and mean read, per (token, head)
//   y = r * rho * w, rho = rsqrt(mean(r^2) + eps2)      dr = rho w dy - rho^3 r <dy w, r> / dh
//   r = num / (den + eps)                               dnum = dr / (den + eps), dden = -<dr, r> / (den + eps)
// Block (row block, head): 32 tokens at a time, 8 lanes per token; the out-norm weight gradient sum_n dy r rho is
// summed per block into part[rb][h][dh] (in a fixed order).
constexpr int kReadGradRows = 256;   // tokens per block

template <typename DyT, int STEPS>
__global__ void __launch_bounds__(256) read_grad_kernel(const DyT* __restrict__ dy, int64_t dy_stride,
                                                        const float* __restrict__ r, const float* __restrict__ den,
                                                        const float* __restrict__ onorm_w, float* __restrict__ dnum,
                                                        float* __restrict__ dden, float* __restrict__ part,
                                                        int64_t N, int H, int dh, int read_mean, float read_eps,
                                                        float out_eps) {
  __shared__ float red[32][65];
  const int h = blockIdx.y;
  const int g = threadIdx.x >> 3;
  const int l8 = threadIdx.x & 7;
  constexpr int kMaxSteps = STEPS;   // steps of 64 columns: dh <= 64 * STEPS
  float acc[kMaxSteps][8];
#pragma unroll
  for (int k = 0; k < kMaxSteps; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
  const int64_t n_begin = static_cast<int64_t>(blockIdx.x) * kReadGradRows;
  const int64_t rstride = static_cast<int64_t>(H) * dh;
  // the head's out-norm weights, the same for every token: loaded once
  float wrow[kMaxSteps][8];
#pragma unroll
  for (int k = 0; k < kMaxSteps; ++k) {
    const int c = 8 * l8 + 64 * k;
    if (onorm_w && c < dh) {
      load_vals<8, float>(onorm_w + h * dh + c, wrow[k]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) wrow[k][e] = 1.f;
    }
  }
  for (int i = 0; i < kReadGradRows / 32; ++i) {
    const int64_t n = n_begin + 32 * i + g;
    const bool live = n < N;   // every lane runs the cross-lane sums
    const int64_t nn = live ? n : 0;
    const float* rr = r + nn * rstride + static_cast<int64_t>(h) * dh;
    const DyT* dd = dy + nn * dy_stride + static_cast<int64_t>(h) * dh;
    // issued with the rows; den is null for the sum read, which reads a word of the row instead and ignores it
    const float den_n = *(den ? den + nn * H + h : rr);
    float rv[kMaxSteps][8], gv[kMaxSteps][8];
#pragma unroll
    for (int k = 0; k < kMaxSteps; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) rv[k][e] = gv[k][e] = 0.f;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxSteps; ++k) {
      const int c = 8 * l8 + 64 * k;
      if (c < dh) {
        load_vals<8, float>(rr + c, rv[k]);
        load_vals<8, DyT>(dd + c, gv[k]);
        if (!live) {
#pragma unroll
          for (int e = 0; e < 8; ++e) rv[k][e] = gv[k][e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(rv[k][e], rv[k][e], ss);
      }
    }
    float rho = 1.f;
    if (onorm_w) {
      ss = sum8(ss);
      rho = 1.f / sqrtf(ss / static_cast<float>(dh) + out_eps);
      float dot = 0.f;
#pragma unroll
      for (int k = 0; k < kMaxSteps; ++k) {
        const int c = 8 * l8 + 64 * k;
        if (c < dh) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc[k][e] = fmaf(gv[k][e] * rv[k][e], rho, acc[k][e]);
            gv[k][e] *= wrow[k][e];
            dot = fmaf(gv[k][e], rv[k][e], dot);
          }
        }
      }
      dot = sum8(dot);
      const float f = rho * rho * rho * dot / static_cast<float>(dh);
#pragma unroll
      for (int k = 0; k < kMaxSteps; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[k][e] = rho * gv[k][e] - f * rv[k][e];
    }
    float inv = 1.f, dd_sum = 0.f;
    if (read_mean) {
      inv = 1.f / ((live ? den_n : 0.f) + read_eps);
#pragma unroll
      for (int k = 0; k < kMaxSteps; ++k) {
        const int c = 8 * l8 + 64 * k;
        if (c < dh) {
#pragma unroll
          for (int e = 0; e < 8; ++e) dd_sum = fmaf(gv[k][e], rv[k][e], dd_sum);
        }
      }
      dd_sum = sum8(dd_sum);
    }
    if (live) {
      float* dst = dnum + nn * rstride + static_cast<int64_t>(h) * dh;
#pragma unroll
      for (int k = 0; k < kMaxSteps; ++k) {
        const int c = 8 * l8 + 64 * k;
        if (c < dh) {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = gv[k][e] * inv;
          store_vals<8, float>(dst + c, o);
        }
      }
      if (l8 == 0) dden[nn * H + h] = read_mean ? -dd_sum * inv : 0.f;
    }
  }
  if (!onorm_w || !part) return;
  // block sum of the out-norm weight gradient: 64 columns at a time through LDS
#pragma unroll
  for (int k = 0; k < kMaxSteps; ++k) {
    if (64 * k >= dh) break;
#pragma unroll
    for (int e = 0; e < 8; ++e) red[g][8 * l8 + e] = acc[k][e];
    __syncthreads();
    if (threadIdx.x < 64 && 64 * k + static_cast<int>(threadIdx.x) < dh) {
      float s = 0.f;
      for (int q = 0; q < 32; ++q) s += red[q][threadIdx.x];
      part[(static_cast<int64_t>(blockIdx.x) * H + h) * dh + 64 * k + threadIdx.x] = s;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------------------------
// chain plan: the write side of one chunk of a grad scan, built in parallel before the scan (the write records of the
// forward plan, for the picks the forward kept).  Per (chunk, head, batch row), stride chain_stride(KP) bytes:
//   u32 {n_rec, n_ext, 0, 0}
//   wrec[64][KP]   uint2 {slot | q0 << 16 | xo << 22, c0 | more << 31}: the distinct slots the chunk's kept writers
//                  write, record u at [u % 64][u / 64] (group g applies records g, g + 64, ...); q0 the slot's first
//                  kept writer, c0 = lam^(L-1-q0) w; with more, its later writers are ext[xo], ext[xo + 1], ... up to
//                  the one flagged last.  Unused entries are null records {M, 0}.
//   ext[64 * KP]   uint2 {c = lam^(L-1-q) w, q | last << 31}
__host__ __device__ constexpr int chain_stride(int KP) { return (16 + 2 * 64 * KP * 8 + 255) / 256 * 256; }

struct ChainArgs {
  const int32_t* w_slot;   // [B][H][T][KP] write picks
  const float* w_wt;
  const uint8_t* reset;    // [B*T] or nullptr
  const float* decay;      // [H]
  unsigned char* chains;   // [B][H][n_chunks][chain_stride]
  int B, T, H, M, kk, n_chunks;
};

// one wave per (chunk, head, batch row); lane p = position p of the chunk (in scan order: REV runs backwards)
template <int KP, bool REV>
__global__ void __launch_bounds__(64) chain_plan_kernel(ChainArgs a) {
  __shared__ __attribute__((aligned(16))) int32_t s_sl[kChunk][KP];   // pads -1
  __shared__ __attribute__((aligned(16))) float s_w[kChunk][KP];
  __shared__ float pw[kChunk + 4];
  extern __shared__ unsigned long long wm[];   // [M] writer masks
  const int c = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int p = threadIdx.x;
  const int M = a.M;
  const int kk = a.kk;
  const int T = a.T;
  const int u0 = c * kChunk;
  const int L = min(kChunk, T - u0);
  const bool valid = p < L;
  const int t = valid ? (REV ? T - 1 - (u0 + p) : u0 + p) : 0;
  const int64_t prow = ((static_cast<int64_t>(b) * a.H + h) * T + t) * KP;
  const float lam = a.decay[h];
  {
    float v = 1.f, sq = lam;   // lam^p by squaring (exact for lam = 0 and lam = 1)
#pragma unroll
    for (int bit = 0; bit < 6; ++bit) {
      v = ((p >> bit) & 1) ? v * sq : v;
      sq *= sq;
    }
    pw[p] = v;
  }
  // loads unconditional inside the row (a missing position reads row 0, no reset flags read a word of the fades),
  // masked after: all of them in flight together
  int slr[KP];
  float wr[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    slr[j] = a.w_slot[prow + j];
    wr[j] = a.w_wt[prow + j];
  }
  const int64_t ri = static_cast<int64_t>(b) * T + (REV ? (valid && u0 + p >= 1 ? T - (u0 + p) : 0) : t);
  const uint8_t rv8 = *(a.reset ? a.reset + ri : reinterpret_cast<const uint8_t*>(a.decay));
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const bool live = valid && j < kk;
    s_sl[p][j] = live ? ((slr[j] >= 0 && slr[j] < M) ? slr[j] : 0) : -1;
    s_w[p][j] = live ? wr[j] : 0.f;
  }
  const bool rf = valid && a.reset && (REV ? u0 + p >= 1 : true) && rv8 != 0;
  const unsigned long long rmask = __ballot(rf);
  const int last = rmask ? 63 - __builtin_clzll(rmask) : -1;   // writers before the chunk's last reset do not reach
  const unsigned long long keep = last >= 0 ? ~((1ull << last) - 1ull) : ~0ull;   // the state
  for (int i = p; i < M; i += 64) wm[i] = 0ull;
  __syncthreads();
  if (valid) {
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j >= kk) break;
      atomicOr(&wm[s_sl[p][j]], 1ull << p);
    }
  }
  __syncthreads();
  auto weight_of = [&](int q, int m) {   // the weight with which position q wrote slot m (pads never match)
    float r = 0.f;
#pragma unroll
    for (int j4 = 0; j4 < KP; j4 += 4) {
      const int4 s4 = *reinterpret_cast<const int4*>(&s_sl[q][j4]);
      const float4 w4 = *reinterpret_cast<const float4*>(&s_w[q][j4]);
      r = s4.x == m ? w4.x : r;
      r = s4.y == m ? w4.y : r;
      r = s4.z == m ? w4.z : r;
      r = s4.w == m ? w4.w : r;
    }
    return r;
  };

  // records owned by this position (first kept writer) and their later writers
  int n_own = 0, n_later = 0, n_chained = 0;
  if (valid) {
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j >= kk) break;
      const unsigned long long mm = wm[s_sl[p][j]] & keep;
      if (mm && __builtin_ctzll(mm) == p) {
        const int later = __builtin_popcountll(mm) - 1;
        ++n_own;
        n_later += later;
        n_chained += later > 0;
      }
    }
  }
  const int inc_own = wave_incl_scan(n_own, p);
  const int inc_later = wave_incl_scan(n_later, p);
  const int inc_chained = wave_incl_scan(n_chained, p);
  const int n_rec = __shfl(inc_own, 63);
  const int n_ext = __shfl(inc_later, 63);
  const int n_chained_all = __shfl(inc_chained, 63);
  unsigned char* plan = a.chains + ((static_cast<int64_t>(b) * a.H + h) * a.n_chunks + c) * chain_stride(KP);
  uint2* wrec = reinterpret_cast<uint2*>(plan + 16);
  uint2* ext = wrec + kChunk * KP;
  if (p == 0) *reinterpret_cast<uint4*>(plan) = make_uint4(n_rec, n_ext, 0u, 0u);
#pragma unroll
  for (int k = 0; k < KP; ++k)
    if (p + kChunk * k >= n_rec) wrec[p * KP + k] = make_uint2(static_cast<uint32_t>(M), 0u);
  if (!valid) return;
  // slots with later writers take the lowest record indexes (records k = 0, 1, ... of the groups), so the scan's
  // walks of the later writers gather in the first record batches
  int u_m = inc_chained - n_chained, u_s = n_chained_all + (inc_own - inc_chained) - (n_own - n_chained);
  int e = inc_later - n_later;
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    if (j >= kk) break;
    const int m = s_sl[p][j];
    unsigned long long mm = wm[m] & keep;
    if (!mm || __builtin_ctzll(mm) != p) continue;
    mm &= mm - 1ull;
    const uint32_t cw = __float_as_uint(pw[L - 1 - p] * s_w[p][j]) | (mm ? 0x80000000u : 0u);
    const int u = mm ? u_m++ : u_s++;
    wrec[(u & 63) * KP + (u >> 6)] =
        make_uint2(static_cast<uint32_t>(m) | (static_cast<uint32_t>(p) << 16) | (static_cast<uint32_t>(e) << 22), cw);
    while (mm) {
      const int q = __builtin_ctzll(mm);
      mm &= mm - 1ull;
      ext[e] = make_uint2(__float_as_uint(pw[L - 1 - q] * weight_of(q, m)),
                          static_cast<uint32_t>(q) | (mm ? 0u : 0x80000000u));
      ++e;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// grad_scan_kernel: the per-pick scan (see the top of this file)
struct GradScanArgs {
  const int32_t* w_slot;   // [B][H][T][KP] write picks (entries >= kk ignored)
  const float* w_wt;       //   and weights
  const int32_t* r_slot;   // [B][H][T][KP] read picks
  const float* r_wt;
  const void* wv;          // write value rows (H * dh per row), type WT
  int64_t wv_stride;
  const float* wc;         // [B*T][H] write count factors, or nullptr for 1
  const void* rv;          // read vector rows, type RT
  int64_t rv_stride;
  const float* rc;         // [B*T][H] read count factors, or nullptr for 1
  const uint8_t* reset;    // [B*T] or nullptr
  const float* decay;      // [H]
  float* dot_out;          // [dh / CW][B][H][T][KP] per-pick dots of this column group (count term in group 0)
  float* sum_out;          // rows of H * dh float32 (weighted sums of the rows read), or nullptr
  int64_t sum_stride;
  const unsigned char* chains;   // [B][H][n_chunks][chain_stride(KP)] chain plans of the writes (chain_plan_kernel)
  int B, T, H, dh, M, kk, n_chunks;
};

// chain entries a grad_scan stages in LDS (the rest are read from the chain plan in global memory); typical chunks
// hold 100-400 entries
__host__ __device__ constexpr int grad_ext_stage(int KP) { return KP <= 8 ? 64 * KP * 8 : 3072; }

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) / 16 * 16; }

// LDS of one grad_scan workgroup: writer masks wmask[M] (u64), slab A[M + 1][CW] and counts cnt[M + 1] (row M stays
// zero: null write records read it and write nothing), the chunk's write picks s_ws[64][KP] and weights
// s_ww[64][KP], write values s_wv[64][CW], count factors s_wc[64], fade powers pw[68], the chunk's reset mask and its
// staged chain entries
struct GradScanLds {
  size_t wmask, A, cnt, ws, ww, wv, wc, pw, rm, ext, total;
  __host__ __device__ constexpr GradScanLds(int M, int KP, int CW)
      : wmask(0),
        A(align16(8 * static_cast<size_t>(M))),
        cnt(A + align16(4 * static_cast<size_t>(M + 1) * CW)),
        ws(cnt + align16(4 * static_cast<size_t>(M + 1))),
        ww(ws + 4 * 64 * KP),
        wv(ww + 4 * 64 * KP),
        wc(wv + 4 * 64 * CW),
        pw(wc + 4 * 64),
        rm(pw + 4 * 68),
        ext(rm + 16),
        total(ext + grad_ext_stage(KP)) {}
};

// weight with which chunk position q wrote slot m >= 0 (0 if it did not); pad picks hold slot -1 and never match
template <int KP>
__device__ __forceinline__ float writer_weight(const int32_t* s_ws, const float* s_ww, int q, int m) {
  float r = 0.f;
#pragma unroll
  for (int j4 = 0; j4 < KP; j4 += 4) {
    const int4 s = *reinterpret_cast<const int4*>(&s_ws[q * KP + j4]);
    const float4 w = *reinterpret_cast<const float4*>(&s_ww[q * KP + j4]);
    r = s.x == m ? w.x : r;
    r = s.y == m ? w.y : r;
    r = s.z == m ? w.z : r;
    r = s.w == m ? w.w : r;
  }
  return r;
}

// The 8 lanes of a group hold partial values p[0..8); lane l8 returns the group sum of p[l8] (a butterfly that
// halves the vector at each step; fixed order).  The exchanges are DPP moves: the mirror within 8 lanes pairs the
// two halves of the group, then the quad permutes pair lanes 2 and 1 apart.
__device__ __forceinline__ float group_reduce_scatter8(const float (&p)[8], int l8) {
  float t4[4], t2[2];
  const bool b2 = l8 & 4, b1 = l8 & 2, b0 = l8 & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float mine = b2 ? p[4 + i] : p[i];
    const float other = b2 ? p[i] : p[4 + i];
    t4[i] = mine + dpp_f<0x141>(other);   // row_half_mirror
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float mine = b1 ? t4[2 + i] : t4[i];
    const float other = b1 ? t4[i] : t4[2 + i];
    t2[i] = mine + dpp_f<0x4e>(other);    // quad_perm [2,3,0,1]
  }
  const float mine = b0 ? t2[1] : t2[0];
  const float other = b0 ? t2[0] : t2[1];
  return mine + dpp_f<0xb1>(other);       // quad_perm [1,0,3,2]
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, true));
}

// OR over the aligned group of 8 lanes
__device__ __forceinline__ unsigned long long group_or8(unsigned long long v) {
  uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  lo |= dpp_u<0xb1>(lo);
  hi |= dpp_u<0xb1>(hi);
  lo |= dpp_u<0x4e>(lo);
  hi |= dpp_u<0x4e>(hi);
  lo |= dpp_u<0x141>(lo);
  hi |= dpp_u<0x141>(hi);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// One workgroup per (column group, head, batch row): 512 threads = 64 positions x 8 lanes of CW/8 columns; the
// slab A (true state mu * A) and the counts stay in LDS.  REV runs the sequence backwards (position u is t = T-1-u);
// a reset at t then separates u = T-t and later from what came before.  Per chunk of 64 positions:
//   stage   the chunk's write picks, weights, values and count factors into LDS; mark each slot's writers in wmask
//   read    group = position: the carried rows of its picks (scaled by mu lam^p; none after a reset in the chunk)
//           and the in-chunk writes of earlier positions of its segment; per pick the dot with the position's read
//           vector (+ the read count factor times the count, in column group 0) and, with sum_out, the pick-weighted
//           sum of the rows
//   write   fade (mu <- mu lam^L; a chunk with a reset empties the slab), then group g applies the chain plan's
//           write records g + 64 k: each written slot's kept writers' faded values / mu, added to the slot's row in
//           one pass (one owner per row: no atomics), lane l8 the count of record l8 + 8 b
template <int CW, int KP, bool REV, typename WT, typename RT>
__global__ void __launch_bounds__(kGradScanThreads) grad_scan_kernel(GradScanArgs a) {
  constexpr int CPL = CW / 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char glds[];
  const int M = a.M;
  const GradScanLds lay(M, KP, CW);
  unsigned long long* wmask = reinterpret_cast<unsigned long long*>(glds + lay.wmask);
  float* A = reinterpret_cast<float*>(glds + lay.A);
  float* cnt = reinterpret_cast<float*>(glds + lay.cnt);
  int32_t* s_ws = reinterpret_cast<int32_t*>(glds + lay.ws);
  float* s_ww = reinterpret_cast<float*>(glds + lay.ww);
  float* s_wv = reinterpret_cast<float*>(glds + lay.wv);
  float* s_wc = reinterpret_cast<float*>(glds + lay.wc);
  float* pw = reinterpret_cast<float*>(glds + lay.pw);
  unsigned char* s_rm = glds + lay.rm;
  unsigned char* s_ext = glds + lay.ext;
  constexpr int XS = grad_ext_stage(KP);
  constexpr int NX = (XS / 16 + kGradScanThreads - 1) / kGradScanThreads;   // staged chain pieces per thread

  const int cg = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int g = tid >> 3;
  const int l8 = tid & 7;
  const int lane = tid & 63;
  const int col0 = cg * CW;
  const int kk = a.kk;
  const int T = a.T;
  const int64_t bh = static_cast<int64_t>(b) * a.H + h;
  const float lam = a.decay[h];
  float* dot_out = a.dot_out + (static_cast<int64_t>(cg) * a.B * a.H + bh) * T * KP;

  for (int i = tid; i < (M + 1) * CW; i += kGradScanThreads) A[i] = 0.f;
  for (int i = tid; i <= M; i += kGradScanThreads) cnt[i] = 0.f;
  if (tid <= kChunk) {
    float v = 1.f;   // lam^tid by repeated multiplication (exact for lam = 0 and lam = 1)
    for (int e = 0; e < tid; ++e) v *= lam;
    pw[tid] = v;
  }
  float mu = 1.f;
  __syncthreads();

  // one chunk's global inputs, loaded a chunk ahead into registers (raw element types, converted when staged)
  struct In {
    int ws[KP / 8];
    float ww[KP / 8];
    WT wv[CPL];
    float wc;
    bool rf;
    int rs[KP];
    float rw[KP];
    RT rv[CPL];
    float rcf;
    uint4 wrec[KP / 2];   // the group's write records
    uint2 own_w[KP / 8];  // write records k = l8 + 8 b (the lane's count updates)
    uint4 xp[NX];         // chain pieces to stage
  };
  const unsigned char* chains = a.chains + bh * a.n_chunks * chain_stride(KP);
  auto fetch = [&](int c, In& x) {
    const int u0 = c * kChunk;
    const bool valid = g < min(kChunk, T - u0);
    const int t = valid ? (REV ? T - 1 - (u0 + g) : u0 + g) : 0;   // row 0 stands in for a missing position
    const int64_t n = static_cast<int64_t>(b) * T + t;
    const int64_t prow = (bh * T + t) * KP;
#pragma unroll
    for (int o = 0; o < KP / 8; ++o) {
      const bool live = valid && l8 + 8 * o < kk;
      x.ws[o] = live ? a.w_slot[prow + l8 + 8 * o] : -1;
      x.ww[o] = live ? a.w_wt[prow + l8 + 8 * o] : 0.f;
    }
    const WT* wvp = static_cast<const WT*>(a.wv) + n * a.wv_stride + static_cast<int64_t>(h) * a.dh + col0 + CPL * l8;
#pragma unroll
    for (int k = 0; k < CPL; ++k) x.wv[k] = wvp[k];
    x.wc = valid ? (a.wc ? a.wc[n * a.H + h] : 1.f) : 0.f;
    x.rf = false;
    if (valid && a.reset) {
      if constexpr (REV) {
        x.rf = (u0 + g >= 1) && a.reset[static_cast<int64_t>(b) * T + (T - (u0 + g))];
      } else {
        x.rf = a.reset[n] != 0;
      }
    }
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const bool live = valid && i < kk;
      x.rs[i] = live ? a.r_slot[prow + i] : 0;
      x.rw[i] = live ? a.r_wt[prow + i] : 0.f;
    }
    const RT* rvp = static_cast<const RT*>(a.rv) + n * a.rv_stride + static_cast<int64_t>(h) * a.dh + col0 + CPL * l8;
#pragma unroll
    for (int k = 0; k < CPL; ++k) x.rv[k] = rvp[k];
    x.rcf = (valid && a.rc) ? a.rc[n * a.H + h] : 1.f;
    const unsigned char* cp = chains + static_cast<int64_t>(c) * chain_stride(KP);
    const uint2* wrow = reinterpret_cast<const uint2*>(cp + 16) + g * KP;
#pragma unroll
    for (int k = 0; k < KP / 2; ++k) x.wrec[k] = reinterpret_cast<const uint4*>(wrow)[k];
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) x.own_w[k] = wrow[l8 + 8 * k];
    // the first chain entries (the whole staged span: loads past n_ext stay inside the plan)
    const uint4* xs = reinterpret_cast<const uint4*>(cp + 16 + 8 * kChunk * KP);
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      const int piece = tid + k * kGradScanThreads;
      x.xp[k] = piece < XS / 16 ? xs[piece] : make_uint4(0u, 0u, 0u, 0u);
    }
  };

  In cur;
  fetch(0, cur);
  for (int c = 0; c < a.n_chunks; ++c) {
    const int u0 = c * kChunk;
    const int L = min(kChunk, T - u0);
    const bool valid = g < L;
    const int t = valid ? (REV ? T - 1 - (u0 + g) : u0 + g) : 0;
    const int64_t n = static_cast<int64_t>(b) * T + t;
    // stage the writes
#pragma unroll
    for (int o = 0; o < KP / 8; ++o) {
      const int s = cur.ws[o];
      s_ws[g * KP + l8 + 8 * o] = s < 0 ? -1 : min(s, M - 1);   // pads -1
      s_ww[g * KP + l8 + 8 * o] = cur.ww[o];
    }
    {
      float vv[CPL];
#pragma unroll
      for (int k = 0; k < CPL; ++k) vv[k] = valid ? to_f32(cur.wv[k]) : 0.f;
      lds_seg_store<CPL>(&s_wv[g * CW + CPL * l8], *reinterpret_cast<const Seg<CPL>*>(vv));
    }
    if (l8 == 0) s_wc[g] = cur.wc;
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      const int piece = tid + k * kGradScanThreads;
      if (piece < XS / 16) reinterpret_cast<uint4*>(s_ext)[piece] = cur.xp[k];
    }
    {
      const unsigned long long bal = __ballot(cur.rf && l8 == 0);   // bits 0, 8, ..., 56: the wave's 8 positions
      if (lane == 0) {
        unsigned v8 = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) v8 |= static_cast<unsigned>((bal >> (8 * k)) & 1ull) << k;
        s_rm[tid >> 6] = static_cast<unsigned char>(v8);
      }
    }
    // the read side of this position, in registers: all picks (every lane), the lane's vector columns
    int rs[KP];
    float rw[KP];
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      rs[i] = (cur.rs[i] >= 0 && cur.rs[i] < M) ? cur.rs[i] : 0;
      rw[i] = cur.rw[i];
    }
    float rv[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) rv[k] = valid ? to_f32(cur.rv[k]) : 0.f;
    const float rcf = cur.rcf;
    for (int i = tid; i < M; i += kGradScanThreads) wmask[i] = 0ull;
    In nxt;
    const bool more = c + 1 < a.n_chunks;
    if (more) fetch(c + 1, nxt);   // in flight across the barriers below (they order LDS only)
    lds_barrier();
    if (valid) {
#pragma unroll
      for (int j = l8; j < KP; j += 8)
        if (j < kk) {
          const int m = s_ws[g * KP + j];
          if (m >= 0) atomicOr(&wmask[m], 1ull << g);
        }
    }
    const unsigned long long rmask = *reinterpret_cast<const unsigned long long*>(s_rm);
    lds_barrier();

    // read
    constexpr int NO = KP / 8;   // picks owned per lane: l8, l8 + 8
    float dot[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o) dot[o] = 0.f;
    float sum[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) sum[k] = 0.f;
    if (valid) {
      const int p = g;
      const unsigned long long upto = rmask & (p == 63 ? ~0ull : (2ull << p) - 1ull);
      const int seg0 = upto ? 63 - __builtin_clzll(upto) : -1;
      if (seg0 < 0) {   // the carried state
        const float fin = mu * pw[p];
        float part[KP];
#pragma unroll
        for (int i = 0; i < KP; ++i) {
          const Seg<CPL> x = lds_seg<CPL>(&A[rs[i] * CW + CPL * l8]);
          float d = 0.f;
#pragma unroll
          for (int k = 0; k < CPL; ++k) {
            d = fmaf(rv[k], x.v[k], d);
            sum[k] = fmaf(rw[i], x.v[k], sum[k]);
          }
          part[i] = d;
        }
#pragma unroll
        for (int o = 0; o < NO; ++o) {
          float p8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) p8[e] = part[8 * o + e];
          dot[o] = fin * group_reduce_scatter8(p8, l8);
        }
        if (cg == 0) {   // the count term, once per pick
#pragma unroll
          for (int o = 0; o < NO; ++o) {
            int so = 0;
#pragma unroll
            for (int i = 0; i < KP; ++i)
              if (i == l8 + 8 * o) so = rs[i];
            dot[o] = fmaf(fin * rcf, cnt[so], dot[o]);
          }
        }
#pragma unroll
        for (int k = 0; k < CPL; ++k) sum[k] *= fin;
      }
      // in-chunk writes of earlier positions of the segment
      const unsigned long long below = (1ull << p) - 1ull;
      const unsigned long long vis = below & (seg0 >= 0 ? ~((1ull << seg0) - 1ull) : ~0ull);
      int so[NO];
      float wo[NO];
      unsigned long long mk[NO];
      unsigned long long any = 0ull;
#pragma unroll
      for (int o = 0; o < NO; ++o) {
        so[o] = 0;
        wo[o] = 0.f;
#pragma unroll
        for (int i = 0; i < KP; ++i)
          if (i == l8 + 8 * o) {
            so[o] = rs[i];
            wo[o] = rw[i];
          }
        mk[o] = (l8 + 8 * o < kk) ? (wmask[so[o]] & vis) : 0ull;
        any |= mk[o];
      }
      unsigned long long U = group_or8(any);
      while (U) {
        const int q = __builtin_ctzll(U);
        U &= U - 1ull;
        const Seg<CPL> x = lds_seg<CPL>(&s_wv[q * CW + CPL * l8]);
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < CPL; ++k) d = fmaf(rv[k], x.v[k], d);
        d = sum8(d);
        const float fq = pw[p - 1 - q];
        const float wcq = s_wc[q];
        float cs = 0.f;
#pragma unroll
        for (int o = 0; o < NO; ++o) {
          const float wq = writer_weight<KP>(s_ws, s_ww, q, so[o]);   // loaded with the row: no branch
          const float co = ((mk[o] >> q) & 1ull) ? fq * wq : 0.f;
          dot[o] = fmaf(co, d, dot[o]);
          if (cg == 0) dot[o] = fmaf(co * rcf, wcq, dot[o]);
          cs = fmaf(wo[o], co, cs);
        }
        if (a.sum_out) {
          cs = sum8(cs);
#pragma unroll
          for (int k = 0; k < CPL; ++k) sum[k] = fmaf(cs, x.v[k], sum[k]);
        }
      }
      // outputs
#pragma unroll
      for (int o = 0; o < NO; ++o) {
        const int i = l8 + 8 * o;
        dot_out[static_cast<int64_t>(t) * KP + i] = i < kk ? dot[o] : 0.f;
      }
      if (a.sum_out) {
        store_vals<CPL, float>(a.sum_out + n * a.sum_stride + static_cast<int64_t>(h) * a.dh + col0 + CPL * l8, sum);
      }
    }
    lds_barrier();

    // write: fade (an emptied slab for a chunk with a reset), then the kept writers of each slot
    float mu_new = mu * pw[L];
    if (rmask) {
      for (int i = tid; i < M * CW; i += kGradScanThreads) A[i] = 0.f;
      for (int i = tid; i < M; i += kGradScanThreads) cnt[i] = 0.f;
      mu_new = 1.f;
      lds_barrier();
    } else if (!(mu_new >= kMuFloor)) {
      for (int i = tid; i < M * CW; i += kGradScanThreads) A[i] *= mu_new;
      for (int i = tid; i < M; i += kGradScanThreads) cnt[i] *= mu_new;
      mu_new = 1.f;
      lds_barrier();
    }
    // group g applies records g + 64 k of the chain plan, 8 at a time (distinct slots; null records write nothing)
    {
      const float inv_mu = fast_rcp(mu_new);
      const unsigned char* gext = chains + static_cast<int64_t>(c) * chain_stride(KP) + 16 + 8 * kChunk * KP;
      auto ext_at = [&](int e) {
        return 8 * e + 8 <= XS ? reinterpret_cast<const uint2*>(s_ext)[e] : reinterpret_cast<const uint2*>(gext)[e];
      };
      uint2 wr[KP];
#pragma unroll
      for (int k = 0; k < KP; ++k)
        wr[k] = make_uint2(u4_word(cur.wrec[k / 2], 2 * (k % 2)), u4_word(cur.wrec[k / 2], 2 * (k % 2) + 1));
#pragma unroll
      for (int k0 = 0; k0 < KP; k0 += 8) {
        Seg<CPL> x[8], vq[8];
        float dc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t rx = wr[k0 + j].x;
          dc[j] = __uint_as_float(wr[k0 + j].y & 0x7fffffffu) * inv_mu;
          x[j] = lds_seg<CPL>(&A[(rx & 0xffffu) * CW + CPL * l8]);
          vq[j] = lds_seg<CPL>(&s_wv[((rx >> 16) & 63u) * CW + CPL * l8]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
          for (int k = 0; k < CPL; ++k) x[j].v[k] = fmaf(dc[j], vq[j].v[k], x[j].v[k]);
          if (wr[k0 + j].y & 0x80000000u) {   // later writers of the slot in this chunk
            int e = wr[k0 + j].x >> 22;
            uint2 t;
            do {
              t = ext_at(e++);
              const float cf = __uint_as_float(t.x) * inv_mu;
              const Seg<CPL> vx = lds_seg<CPL>(&s_wv[(t.y & 63u) * CW + CPL * l8]);
#pragma unroll
              for (int k = 0; k < CPL; ++k) x[j].v[k] = fmaf(cf, vx.v[k], x[j].v[k]);
            } while (!(t.y & 0x80000000u));
          }
        }
        // lane l8's count update for record k0 + l8: the writers' coefficients times their count factors
        const uint2 ow = cur.own_w[k0 / 8];
        const int mc = static_cast<int>(ow.x & 0xffffu);
        float dcc = __uint_as_float(ow.y & 0x7fffffffu) * s_wc[(ow.x >> 16) & 63u];
        if (ow.y & 0x80000000u) {
          int e = ow.x >> 22;
          uint2 t;
          do {
            t = ext_at(e++);
            dcc = fmaf(__uint_as_float(t.x), s_wc[t.y & 63u], dcc);
          } while (!(t.y & 0x80000000u));
        }
        const float cold = cnt[mc];
#pragma unroll
        for (int j = 0; j < 8; ++j) {   // null records (row M) write nothing: no same-row write conflicts
          const int mj = static_cast<int>(wr[k0 + j].x & 0xffffu);
          if (mj != M) lds_seg_store<CPL>(&A[mj * CW + CPL * l8], x[j]);
        }
        if (mc != M) cnt[mc] = fmaf(dcc, inv_mu, cold);
      }
    }
    mu = mu_new;
    lds_barrier();
    if (more) cur = nxt;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// addr_grad_kernel: softmax, gate, address normalisation and sub-key products backward, one wave per (token, head,
// address set) at a time, lane e = address element e (d_a = 2 * HALF <= 64); lane j < KP also holds pick j for the
// softmax and gate math, whose per-pick results reach every lane by v_readlane.  Block (token block, head, set) of W
// waves (4 per SIMD: their memory round trips overlap); wave w takes tokens n_begin + w + W i.
//   read set:  x_j = tau sv_j, wr = softmax(x):          dx_j = wr_j (dwr_j - P), P = sum_j wr_j dwr_j
//   write set: ww = softmax(tau sv) * g:                 dp_j = g dww_j, dx_j = p_j (dp_j - sum p dp),
//                                                        dg = sum_j p_j dww_j, dlogit = dg g (1 - g)
//   both:      dsv_j = tau dx_j, dtau += sum_j sv_j dx_j; sv_j = (v1[i1_j] + v2[i2_j]) / 2 with v = <u, k^>:
//              du += dsv_j / 2 k^[i_j], dk^[i_j] += dsv_j / 2 u; u = z / max(|z|, 1e-12):
//              dz = (du - u <u, du>) / |z| (du / 1e-12 below the floor); z = kz + addr_b
// Per block: partial sums of dtau, the gate bias, addr_b, lam dL/dlam (float64) and the unit sub-key gradient (one
// copy per wave in LDS, summed in wave order: no atomics, a fixed order).
constexpr int kAddrGradWaveTokens = 16;   // tokens per wave
// waves per block at most (4 per SIMD; the kernel needs well under 128 registers)
__host__ __device__ constexpr int addr_grad_max_waves(int) { return 16; }

struct AddrGradArgs {
  const void* kz;
  int64_t kz_stride;
  const void* qz;
  int64_t qz_stride;
  const void* gl;            // gate logit rows or nullptr (no gate)
  int64_t g_stride;
  const float* keys[2];      // raw sub-keys [H][n_sub][HALF]
  const float* addr_b;       // [H][d_a] or nullptr
  const float* log_scale;    // [H]
  const float* gate_bias;    // [H] or nullptr
  const int32_t* slot[2];    // [B][H][T][KP]: write, read
  const float* wt[2];
  const float* score[2];
  const float* dot[2];       // [CG][B][H][T][KP] per-pick gradient partials: dww, dwr
  int n_cg;
  float* dz[2];              // rows of H * d_a float32: d kz, d qz
  int64_t dz_stride[2];
  float* dgl;                // rows of H float32 or nullptr
  int64_t dgl_stride;
  float* part_f;             // [n_blk][2][H][2 + d_a]: dtau, d gate bias, d addr_b
  double* part_d;            // [n_blk][2][H]: lam dL/dlam
  float* part_k;             // [n_blk][2][H][2][n_sub][HALF]: d unit sub-keys
  int B, T, H, n_sub, kk;
  int set0;                  // the first address set (grid z covers set0 .. set0 + gridDim.z - 1)
};


__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// sum over aligned groups of 16 lanes (the rows of the wave), by DPP
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  return v + dpp_f<0x140>(v);   // row_mirror: lane i and lane 15 - i hold the two 8-lane sums
}

// sum over the 64 lanes (every lane active): the rows by DPP, then the four row sums read out of lanes 0, 16, 32, 48
__device__ __forceinline__ float wave_sum(float v) {
  const float s = sum16(v);
  return (lane_f(s, 0) + lane_f(s, 16)) + (lane_f(s, 32) + lane_f(s, 48));
}

// sum over the lane's half of the address (lanes [0, HALF) or [HALF, 2 HALF))
template <int HALF>
__device__ __forceinline__ float half_sum(float v, int e) {
  if constexpr (HALF == 32) {   // rows 0 + 1 and 2 + 3
    const float s = sum16(v);
    const float s0 = lane_f(s, 0) + lane_f(s, 16);
    const float s1 = lane_f(s, 32) + lane_f(s, 48);
    return e < 32 ? s0 : s1;
  } else if constexpr (HALF == 16) {
    return sum16(v);
  } else if constexpr (HALF == 8) {
    return sum8(v);
  } else if constexpr ((HALF & (HALF - 1)) == 0) {   // aligned groups of HALF lanes
#pragma unroll
    for (int off = 1; off < HALF; off <<= 1) v += __shfl_xor(v, off);
    return v;
  } else {
    const float s1 = wave_sum(e < HALF ? v : 0.f);
    const float s2 = wave_sum(e >= HALF && e < 2 * HALF ? v : 0.f);
    return e < HALF ? s1 : s2;
  }
}

// LDS of addr_grad_kernel for W waves: wave partials of lam dL/dlam (float64), unit sub-keys, one sub-key gradient
// copy and one partial record per wave
__host__ __device__ constexpr size_t addr_grad_lds(int n_sub, int half, int W) {
  return sizeof(double) * W + sizeof(float) * (2 * static_cast<size_t>(n_sub) * half * (1 + W) + W * (2 * half + 2));
}

// sum over lanes [0, KP) (aligned groups of KP lanes; KP a power of two)
template <int KP>
__device__ __forceinline__ float pick_sum(float v) {
  if constexpr (KP == 8) {
    return sum8(v);
  } else if constexpr (KP == 16) {
    return sum16(v);
  } else {
#pragma unroll
    for (int off = 1; off < KP; off <<= 1) v += __shfl_xor(v, off);
    return v;
  }
}


template <int HALF, int KP, typename InT>
__global__ void __launch_bounds__(64 * addr_grad_max_waves(KP)) addr_grad_kernel(AddrGradArgs a) {
  constexpr int DA = 2 * HALF;
  extern __shared__ __attribute__((aligned(16))) unsigned char albuf[];
  const int W = blockDim.x >> 6;
  const int n_sub = a.n_sub;
  const int KS = 2 * n_sub * HALF;                                // sub-key values of both halves
  double* redd = reinterpret_cast<double*>(albuf);                // [W]
  float* kn = reinterpret_cast<float*>(albuf + sizeof(double) * W);   // [2][n_sub][HALF] unit sub-keys
  float* dk = kn + KS;                                            // [W][2][n_sub][HALF] their gradient per wave
  float* red = dk + W * KS;                                       // [W][DA + 2] wave partials
  const int h = blockIdx.y;
  const int set = a.set0 + blockIdx.z;   // 0: write keys, 1: read queries
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int e = tid & 63;       // address element; lanes e < KP also hold pick e
  const int kk = a.kk;
  if constexpr ((HALF & (HALF - 1)) == 0) {   // unit sub-keys: one row per aligned group of HALF lanes, all waves
    for (int i0 = w * 64; i0 < KS; i0 += blockDim.x) {   // wave-uniform bound: every lane takes the lane sums
      const int i = i0 + e;
      const int r = i / HALF;
      const int part = r >= n_sub;
      const float v = i < KS ? a.keys[part][(static_cast<int64_t>(h) * n_sub + (r - part * n_sub)) * HALF + i % HALF]
                             : 0.f;
      const float nrm = fmaxf(sqrtf(half_sum<HALF>(v * v, e)), 1e-12f);
      if (i < KS) kn[i] = v / nrm;
    }
  } else {
    for (int r = tid; r < 2 * n_sub; r += blockDim.x) {
      const int part = r >= n_sub;
      const float* src = a.keys[part] + (static_cast<int64_t>(h) * n_sub + (r - part * n_sub)) * HALF;
      float ss = 0.f;
      for (int d = 0; d < HALF; ++d) ss = fmaf(src[d], src[d], ss);
      const float nrm = fmaxf(sqrtf(ss), 1e-12f);
      for (int d = 0; d < HALF; ++d) kn[r * HALF + d] = src[d] / nrm;
    }
  }
  for (int i = tid; i < W * KS; i += blockDim.x) dk[i] = 0.f;
  __syncthreads();
  float* dkw = dk + w * KS;   // this wave's copy: within a wave the lanes of one pick touch distinct entries
  const float tau = expf(a.log_scale[h]);
  const float ab = (e < DA && a.addr_b) ? a.addr_b[h * DA + e] : 0.f;
  const float gb = a.gate_bias ? a.gate_bias[h] : 0.f;
  const int hf = e >= HALF;               // the lane's half
  const int ec = e - hf * HALF;           // column within the half
  // slot -> (i1, i2) = (s / n_sub, s % n_sub) by a multiply-high: exact for s < 2^16, n_sub <= 256
  const uint32_t magic = n_sub > 1 ? 0xFFFFFFFFu / static_cast<uint32_t>(n_sub) + 1u : 0u;
  const InT* zb = static_cast<const InT*>(set == 0 ? a.kz : a.qz);
  const int64_t zs = set == 0 ? a.kz_stride : a.qz_stride;
  const bool gated = set == 0 && a.gl;
  const int32_t* slot = a.slot[set];
  const float* wtp = a.wt[set];
  const float* scp = a.score[set];
  const float* dotp = a.dot[set];
  float* dzp = a.dz[set];
  const int64_t dzs = a.dz_stride[set];
  const bool pl = e < kk;                 // the lane holds a live pick
  float acc_tau = 0.f, acc_gb = 0.f, acc_ab = 0.f;
  double acc_lam = 0.0;
  const int64_t N = static_cast<int64_t>(a.B) * a.T;
  const int64_t cg_stride = N * a.H * KP;
  int64_t n = static_cast<int64_t>(blockIdx.x) * W * kAddrGradWaveTokens + w;
  int b = static_cast<int>(n / a.T);
  int t = static_cast<int>(n - static_cast<int64_t>(b) * a.T);
  // one token's loads, issued a token ahead: unconditional, at indexes clamped into the arrays (masked after use)
  struct TokIn {
    InT z, gl;
    int sl;
    float sv, wt, d0, d1;
  };
  const int ez = (DA == 64 || e < DA) ? e : 0;
  const int ep = pl ? e : 0;
  auto load = [&](int64_t nn, int bb, int tt) {
    TokIn x;
    const int64_t prow = ((static_cast<int64_t>(bb) * a.H + h) * a.T + tt) * KP + ep;
    x.z = zb[nn * zs + static_cast<int64_t>(h) * DA + ez];
    x.gl = gated ? static_cast<const InT*>(a.gl)[nn * a.g_stride + h] : zb[0];
    x.sl = slot[prow];
    x.sv = scp[prow];
    x.wt = wtp[prow];
    x.d0 = dotp[prow];
    x.d1 = a.n_cg > 1 ? dotp[cg_stride + prow] : 0.f;
    return x;
  };
  TokIn cur = load(n < N ? n : 0, n < N ? b : 0, n < N ? t : 0);
  for (int i = 0; i < kAddrGradWaveTokens; ++i) {
    if (n >= N) break;   // wave-uniform
    // the next token (W positions on) and its loads
    const int64_t n2 = n + W;
    int b2 = b, t2 = t + W;
    while (t2 >= a.T) {
      t2 -= a.T;
      ++b2;
    }
    TokIn nxt = cur;
    if (i + 1 < kAddrGradWaveTokens && n2 < N) nxt = load(n2, b2, t2);
    const int64_t prow = ((static_cast<int64_t>(b) * a.H + h) * a.T + t) * KP;
    const float z = (DA == 64 || e < DA) ? to_f32(cur.z) + ab : 0.f;
    const float glv = gated ? to_f32(cur.gl) : 0.f;
    int sl = pl ? cur.sl : 0;
    sl = (sl >= 0 && sl < n_sub * n_sub) ? sl : 0;
    const float sv = pl ? cur.sv : 0.f;
    const float wt = pl ? cur.wt : 0.f;
    float dw = pl ? cur.d0 + cur.d1 : 0.f;
    for (int c = 2; c < a.n_cg; ++c) dw += pl ? dotp[c * cg_stride + prow + e] : 0.f;
    // softmax (and gate) backward, pick e on lane e
    float dx;
    if (set == 1) {   // read: softmax
      const float P = pick_sum<KP>(wt * dw);
      dx = wt * (dw - P);
      acc_lam += static_cast<double>(t) * static_cast<double>(P);
    } else {          // write: gated softmax
      const float Q = pick_sum<KP>(wt * dw);
      acc_lam -= static_cast<double>(t + 1) * static_cast<double>(Q);
      const float x0 = lane_f(sv, 0) * tau;
      float pj = pl ? __expf(sv * tau - x0) : 0.f;
      pj *= fast_rcp(pick_sum<KP>(pj));
      const float gt = gated ? fast_rcp(1.f + __expf(-(glv + gb))) : 1.f;
      const float S = pick_sum<KP>(pj * gt * dw);
      const float dg = pick_sum<KP>(pj * dw);
      dx = pj * (gt * dw - S);
      if (gated) {
        const float dlogit = dg * gt * (1.f - gt);
        if (e == 0 && a.dgl) a.dgl[n * a.dgl_stride + h] = dlogit;
        acc_gb += e == 0 ? dlogit : 0.f;
      }
    }
    if (!pl) dx = 0.f;
    acc_tau = fmaf(sv, dx, acc_tau);        // per lane (pick), summed over lanes at the end
    const float hs = 0.5f * tau * dx;        // d sv / 2 of pick e
    const int i1 = n_sub > 1 ? static_cast<int>(__umulhi(static_cast<uint32_t>(sl), magic)) : sl;
    const int i2 = sl - i1 * n_sub;
    const float z2 = z * z;
    const float nz = __builtin_amdgcn_sqrtf(half_sum<HALF>(z2, e));
    const float inz = fast_rcp(fmaxf(nz, 1e-12f));
    const float u = z * inz;
    // pick j: du += hs_j k^[i_j], dk^[i_j] += hs_j u.  Both row offsets are read out of pick lane j and the lane's
    // half selects one (no branch); picks sharing a row add up in pick order
    const int off1 = i1 * HALF;
    const int off2 = (n_sub + i2) * HALF;
    float du = 0.f;
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j >= kk) break;   // uniform
      const float hj = lane_f(hs, j);
      const int o1 = __builtin_amdgcn_readlane(off1, j);
      const int o2 = __builtin_amdgcn_readlane(off2, j);
      const int o = (hf ? o2 : o1) + ec;
      if (DA == 64 || e < DA) {
        du = fmaf(hj, kn[o], du);
        dkw[o] += hj * u;
      }
    }
    const float ud = half_sum<HALF>(u * du, e);
    const float dz = nz > 1e-12f ? (du - u * ud) * inz : du * 1e12f;
    if (e < DA) dzp[n * dzs + static_cast<int64_t>(h) * DA + e] = dz;
    acc_ab += dz;
    cur = nxt;
    n = n2;
    b = b2;
    t = t2;
  }
  acc_tau = wave_sum(acc_tau);   // the picks' lanes, in a fixed order
  // block sums in a fixed order: waves -> LDS -> threads
  if (e < DA) red[w * (DA + 2) + e] = acc_ab;
  if (e == 0) {
    red[w * (DA + 2) + DA] = acc_tau;
    red[w * (DA + 2) + DA + 1] = acc_gb;
    redd[w] = acc_lam;
  }
  __syncthreads();
  const int64_t pid = (static_cast<int64_t>(blockIdx.x) * gridDim.z + blockIdx.z) * a.H + h;
  for (int c = tid; c < DA + 2; c += blockDim.x) {
    float s = 0.f;
    for (int q = 0; q < W; ++q) s += red[q * (DA + 2) + c];
    // record order: dtau, d gate bias, d addr_b[DA]
    const int f = c == DA ? 0 : c == DA + 1 ? 1 : 2 + c;
    a.part_f[pid * (2 + DA) + f] = s;
  }
  if (tid == 0) {
    double s = 0.0;
    for (int q = 0; q < W; ++q) s += redd[q];
    a.part_d[pid] = s;
  }
  for (int i = tid; i < KS; i += blockDim.x) {
    float s = 0.f;
    for (int q = 0; q < W; ++q) s += dk[q * KS + i];
    a.part_k[pid * KS + i] = s;
  }
}

// Sums over records: out[i] = sum_r part[r * rec_stride + i] (r < n_rec) in float64 for n_items items.  Block of
// 64 x 16 threads: lane i of group rg sums records rg, rg + 16, ... (loads issued together), then the 16 group sums
// are added in group order: a fixed order, so the result is deterministic.
constexpr int kRedGroups = 16;

template <typename T>
__global__ void __launch_bounds__(64 * kRedGroups) reduce_records_kernel(const T* __restrict__ part, int n_rec,
                                                                        int64_t rec_stride, int64_t n_items,
                                                                        double* __restrict__ out) {
  __shared__ double red[kRedGroups][64];
  const int l = threadIdx.x & 63;
  const int rg = threadIdx.x >> 6;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 64 + l;
  double s = 0.0;
  if (i < n_items) {
    constexpr int kBatch = 16;
    for (int r0 = rg; r0 < n_rec; r0 += kRedGroups * kBatch) {
      T v[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int r = r0 + q * kRedGroups;
        v[q] = r < n_rec ? part[static_cast<int64_t>(r) * rec_stride + i] : T(0);
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) s += static_cast<double>(v[q]);
    }
  }
  red[rg][l] = s;
  __syncthreads();
  if (rg == 0 && i < n_items) {
    double t = 0.0;
    for (int q = 0; q < kRedGroups; ++q) t += red[q][l];
    out[i] = t;
  }
}

// the per-head sums to the parameter gradients: sums[h][F] = (dtau, d gate bias, d addr_b[DA]) and lam dL/dlam
__global__ void __launch_bounds__(128) addr_post_kernel(const double* __restrict__ sums, const double* __restrict__ lam,
                                                        int DA, const float* __restrict__ log_scale, float* d_log_scale,
                                                        float* d_gate_bias, float* d_addr_b, float* d_log_decay) {
  const int h = blockIdx.x;
  const int F = 2 + DA;
  for (int f = threadIdx.x; f <= F; f += blockDim.x) {
    if (f == F) {
      if (d_log_decay) d_log_decay[h] = static_cast<float>(lam[h]);
    } else if (f == 0) {
      if (d_log_scale) d_log_scale[h] = static_cast<float>(sums[h * F] * static_cast<double>(expf(log_scale[h])));
    } else if (f == 1) {
      if (d_gate_bias) d_gate_bias[h] = static_cast<float>(sums[h * F + 1]);
    } else if (d_addr_b) {
      d_addr_b[h * DA + (f - 2)] = static_cast<float>(sums[h * F + f]);
    }
  }
}

// raw sub-key gradient from the summed unit sub-key gradient dk^ ([H][2][n_sub][half]; F.normalize backward):
// one wave per sub-key row, dK = (dk^ - k^ <k^, dk^>) / |K|   (dk^ / 1e-12 below the floor)
__global__ void __launch_bounds__(64) keys_grad_kernel(const double* __restrict__ dkn_sum, int n_sub, int half,
                                                       const float* __restrict__ keys1,
                                                       const float* __restrict__ keys2, float* d_keys1,
                                                       float* d_keys2) {
  const int row = blockIdx.x;                 // [H][2][n_sub]
  const int h = row / (2 * n_sub);
  const int part = (row / n_sub) & 1;
  const int i = row % n_sub;
  const int c = threadIdx.x;
  const bool live = c < half;
  const float* key = (part ? keys2 : keys1) + (static_cast<int64_t>(h) * n_sub + i) * half;
  float* out = (part ? d_keys2 : d_keys1);
  const float kv = live ? key[c] : 0.f;
  const float dkn = live ? static_cast<float>(dkn_sum[static_cast<int64_t>(row) * half + c]) : 0.f;
  const float nk = sqrtf(wave_sum(kv * kv));
  const float kh = kv / fmaxf(nk, 1e-12f);
  const float dot = wave_sum(kh * dkn);
  const float d = nk > 1e-12f ? (dkn - kh * dot) / nk : dkn * 1e12f;
  if (live && out) out[(static_cast<int64_t>(h) * n_sub + i) * half + c] = d;
}

__global__ void __launch_bounds__(256) to_float_kernel(const double* __restrict__ in, int64_t n, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = static_cast<float>(in[i]);
}

// ---------------------------------------------------------------------------------------------------------------
// table read backward (TrainedSdm's embedding_bag, track4_onesdm_models.py:448-455)
//   dw[n][h][j]          = <values[h][slot_j], dy[n][h]>    (table_grad_kernel: the per-pick gradient the softmax
//                                                           backward takes; one wave per (token, head), lane l takes
//                                                           columns 4l, 4l + 256, ...)
//   d_values[h][s]       = sum over the picks (n, j) of slot s of w_j dy[n][h]   (table_values_grad_kernel: the picks
//                          sorted by (head, slot) with a stable radix sort, so each row is one wave's sum in pick
//                          order -- no atomics, a fixed order)
template <int KP, typename VT, typename DyT>
__global__ void __launch_bounds__(256) table_grad_kernel(const int32_t* __restrict__ slots,
                                                         const float* __restrict__ wts,
                                                         const VT* __restrict__ values, const DyT* __restrict__ dy,
                                                         int64_t dy_stride, float* __restrict__ dw, int B, int T,
                                                         int H, int M, int dh, int kk) {
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= static_cast<int64_t>(B) * T * H) return;   // whole waves
  const int64_t n = wave / H;
  const int h = static_cast<int>(wave - n * H);
  const int b = static_cast<int>(n / T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * T);
  const int64_t pb = ((static_cast<int64_t>(b) * H + h) * T + t) * KP;
  int sl[KP];
  float d[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    sl[j] = min(max(slots[pb + j], 0), M - 1);   // pads (-1) and stray ids stay inside the table
    d[j] = 0.f;
  }
  (void)wts;
  const VT* tab = values + static_cast<int64_t>(h) * M * dh;
  for (int c0 = 4 * lane; c0 < dh; c0 += 256) {
    float g[4];
    load_vals<4, DyT>(dy + n * dy_stride + static_cast<int64_t>(h) * dh + c0, g);
    // every pick's row, pads included (their dots are dropped below): unconditional loads issue together
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      float v[4];
      load_vals<4, VT>(tab + static_cast<int64_t>(sl[j]) * dh + c0, v);
#pragma unroll
      for (int e = 0; e < 4; ++e) d[j] = fmaf(g[e], v[e], d[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const float s = wave_sum(d[j]);
    if (lane == 0) dw[pb + j] = j < kk ? s : 0.f;
  }
}

__global__ void __launch_bounds__(256) zero_i32_kernel(int32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// sort keys of the picks: entry e of the [B][H][T][KP] pick arrays gets key h * M + slot (pads: H * M, after every
// real key) and value e; count[key] counts the live picks of each (head, slot)
__global__ void __launch_bounds__(256) pick_keys_kernel(const int32_t* __restrict__ slots, int64_t n_entries, int T,
                                                        int H, int KP, int M, int kk, int32_t* __restrict__ keys,
                                                        int32_t* __restrict__ vals, int32_t* __restrict__ count) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_entries) return;
  const int j = static_cast<int>(e % KP);
  const int h = static_cast<int>((e / KP / T) % H);
  int key = H * M;
  if (j < kk) {
    const int s = min(max(slots[e], 0), M - 1);
    key = h * M + s;
    atomicAdd(&count[key], 1);   // integer counts: exact in any order
  }
  keys[e] = key;
  vals[e] = static_cast<int32_t>(e);
}

// d_values[h][s] = sum of w_e dy[n_e][h] over the picks e of (h, s), in the sorted (entry) order; one wave per row,
// lane l takes columns 4l, 4l + 256, ...; four picks' loads in flight at a time
template <typename DyT>
__global__ void __launch_bounds__(256) table_values_grad_kernel(const int32_t* __restrict__ sorted_vals,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ count,
                                                                const float* __restrict__ wts,
                                                                const DyT* __restrict__ dy, int64_t dy_stride,
                                                                float* __restrict__ d_values, int T, int H, int KP,
                                                                int M, int dh) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);   // h * M + s
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(H) * M) return;   // whole waves
  const int h = static_cast<int>(row / M);
  const int off = offsets[row];
  const int cnt = count[row];
  float* dst = d_values + row * dh;
  // up to CS column steps of 256 held in registers; the picks QS at a time: their indexes and weights, then every
  // row segment, all loads of a batch in flight together; the sum runs in pick order
  constexpr int CS = 4, QS = 8;
  for (int cb = 0; cb < dh; cb += 256 * CS) {
    float acc[CS][4];
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[s][c] = 0.f;
    for (int i0 = 0; i0 < cnt; i0 += QS) {
      int64_t ro[QS];
      float w[QS];
#pragma unroll
      for (int q = 0; q < QS; ++q) {
        const int i = min(i0 + q, cnt - 1);
        const int64_t e = sorted_vals[off + i];   // ((b * H + h) * T + t) * KP + j
        const int64_t u = e / KP;
        const int64_t b = u / (static_cast<int64_t>(H) * T);
        const int64_t t = u - (b * H + h) * T;
        w[q] = i0 + q < cnt ? wts[e] : 0.f;
        ro[q] = (b * T + t) * dy_stride + static_cast<int64_t>(h) * dh;
      }
#pragma unroll
      for (int q = 0; q < QS; ++q) {
#pragma unroll
        for (int s = 0; s < CS; ++s) {
          const int c0 = cb + 256 * s + 4 * lane;
          if (c0 < dh) {
            float g[4];
            load_vals<4, DyT>(dy + ro[q] + c0, g);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[s][c] = fmaf(w[q], g[c], acc[s][c]);
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      const int c0 = cb + 256 * s + 4 * lane;
      if (c0 < dh) store_vals<4, float>(dst + c0, acc[s]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// host side of the backward
// waves per addr_grad block: as many as LDS holds, up to addr_grad_max_waves
int addr_grad_waves(int n_sub, int half, int KP) {
  for (int w = addr_grad_max_waves(KP); w >= 1; --w)
    if (addr_grad_lds(n_sub, half, w) <= kLdsBytes) return w;
  return 0;
}

struct GradPlan {
  Plan p;
  int cw, n_cg, n_rb, n_blk, addr_waves;
  size_t off_dnum, off_dden, off_dotw, off_dotr, off_p1, off_pf, off_pd, off_pk, off_sums, off_chains, total;
};

// widest column group (32, 16, 8) whose grad_scan slab fits in LDS
int grad_columns(const Plan& p) {
  for (int cw : {32, 16, 8})
    if (p.dh % cw == 0 && GradScanLds(p.M, p.pitch, cw).total <= kLdsBytes) return cw;
  return 0;
}

int make_grad_plan(const sdm_rt_dims* d, GradPlan* g) {
  int rc = make_plan(d, &g->p);
  if (rc) return rc;
  const Plan& p = g->p;
  if (p.d_a > 64) return set_err(SDM_RT_EUNSUPPORTED, "backward: addr_dim %d exceeds 64", p.d_a);
  g->cw = grad_columns(p);
  if (!g->cw) return set_err(SDM_RT_EUNSUPPORTED, "backward: M = %d locations do not fit a slab in LDS", p.M);
  g->addr_waves = addr_grad_waves(p.n_sub, p.half, p.pitch);
  if (!g->addr_waves) return set_err(SDM_RT_EUNSUPPORTED, "backward: n_sub = %d sub-keys do not fit in LDS", p.n_sub);
  g->n_cg = p.dh / g->cw;
  const int64_t N = static_cast<int64_t>(p.B) * p.T;
  g->n_rb = static_cast<int>((N + kReadGradRows - 1) / kReadGradRows);
  const int64_t tpb = static_cast<int64_t>(g->addr_waves) * kAddrGradWaveTokens;
  g->n_blk = static_cast<int>((N + tpb - 1) / tpb);
  const size_t hd = static_cast<size_t>(p.H) * p.dh;
  const size_t picks = static_cast<size_t>(N) * p.H * p.pitch;
  size_t o = 0;
  g->off_dnum = o;
  o = align_up(o + sizeof(float) * N * hd, 256);
  g->off_dden = o;
  o = align_up(o + sizeof(float) * N * p.H, 256);
  g->off_dotw = o;
  o = align_up(o + sizeof(float) * g->n_cg * picks, 256);
  g->off_dotr = o;
  o = align_up(o + sizeof(float) * g->n_cg * picks, 256);
  g->off_p1 = o;
  o = align_up(o + sizeof(float) * g->n_rb * hd, 256);
  g->off_pf = o;
  o = align_up(o + sizeof(float) * 2 * g->n_blk * p.H * (2 + p.d_a), 256);
  g->off_pd = o;
  o = align_up(o + sizeof(double) * 2 * g->n_blk * p.H, 256);
  g->off_pk = o;
  o = align_up(o + sizeof(float) * 2 * g->n_blk * p.H * 2 * static_cast<size_t>(p.n_sub) * p.half, 256);
  g->off_sums = o;   // float64 sums: addressing fields [H][2 + d_a], lam [H], unit sub-keys [H][2][n_sub][half], onorm
  o = align_up(o + sizeof(double) * (static_cast<size_t>(p.H) * (2 + p.d_a) + p.H +
                                     static_cast<size_t>(p.H) * 2 * p.n_sub * p.half + hd), 256);
  g->off_chains = o;   // the chain plans of one scan direction at a time
  o = align_up(o + static_cast<size_t>(p.B) * p.H * p.n_chunks * chain_stride(p.pitch), 256);
  g->total = o;
  return SDM_RT_OK;
}

template <int CW, int KP, bool REV, typename WT, typename RT>
int launch_grad_scan_t(const GradPlan& g, const GradScanArgs& a, hipStream_t st) {
  {
    ChainArgs c{};
    c.w_slot = a.w_slot;
    c.w_wt = a.w_wt;
    c.reset = a.reset;
    c.decay = a.decay;
    c.chains = const_cast<unsigned char*>(a.chains);
    c.B = a.B;
    c.T = a.T;
    c.H = a.H;
    c.M = a.M;
    c.kk = a.kk;
    c.n_chunks = a.n_chunks;
    hipLaunchKernelGGL((chain_plan_kernel<KP, REV>), dim3(a.n_chunks, a.H, a.B), dim3(64),
                       sizeof(unsigned long long) * a.M, st, c);
    if (int rc = check_launch("chain plan")) return rc;
  }
  const size_t lds = GradScanLds(g.p.M, KP, CW).total;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&grad_scan_kernel<CW, KP, REV, WT, RT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
  if (attr != hipSuccess) return set_err(SDM_RT_ELAUNCH, "grad scan: cannot enable %zu bytes of LDS", kLdsBytes);
  dim3 grid(g.n_cg, g.p.H, g.p.B);
  hipLaunchKernelGGL((grad_scan_kernel<CW, KP, REV, WT, RT>), grid, dim3(kGradScanThreads), lds, st, a);
  return check_launch("grad scan");
}

template <bool REV, typename WT, typename RT>
int launch_grad_scan(const GradPlan& g, const GradScanArgs& a, hipStream_t st) {
  const bool k8 = g.p.pitch == 8;
  switch (g.cw) {
    case 32: return k8 ? launch_grad_scan_t<32, 8, REV, WT, RT>(g, a, st) : launch_grad_scan_t<32, 16, REV, WT, RT>(g, a, st);
    case 16: return k8 ? launch_grad_scan_t<16, 8, REV, WT, RT>(g, a, st) : launch_grad_scan_t<16, 16, REV, WT, RT>(g, a, st);
    default: return k8 ? launch_grad_scan_t<8, 8, REV, WT, RT>(g, a, st) : launch_grad_scan_t<8, 16, REV, WT, RT>(g, a, st);
  }
}

template <int HALF, typename InT>
struct AddrGradLaunch {
  static int run(const GradPlan& g, const AddrGradArgs& a, hipStream_t st) {
    const Plan& p = g.p;
    const size_t lds = addr_grad_lds(p.n_sub, HALF, g.addr_waves);
    dim3 grid(g.n_blk, p.H, 2 - a.set0);
    dim3 block(64 * g.addr_waves);
    if (p.pitch == 8) {
      static const bool ok = allow_lds(reinterpret_cast<const void*>(&addr_grad_kernel<HALF, 8, InT>));
      if (!ok) return lds_err("addr grad");
      hipLaunchKernelGGL((addr_grad_kernel<HALF, 8, InT>), grid, block, lds, st, a);
    } else {
      static const bool ok = allow_lds(reinterpret_cast<const void*>(&addr_grad_kernel<HALF, 16, InT>));
      if (!ok) return lds_err("addr grad");
      hipLaunchKernelGGL((addr_grad_kernel<HALF, 16, InT>), grid, block, lds, st, a);
    }
    return check_launch("addr grad");
  }
};

int check_saved(const sdm_rt_saved* s, bool need_den) {
  if (!s) return set_err(SDM_RT_EINVAL, "saved is NULL");
  if (!s->slots_w || !s->weights_w || !s->scores_w || !s->slots_r || !s->weights_r || !s->scores_r || !s->read)
    return set_err(SDM_RT_EINVAL, "saved: picks, weights, scores and read must not be NULL");
  if (need_den && !s->den) return set_err(SDM_RT_EINVAL, "saved: den must not be NULL for the mean read");
  return SDM_RT_OK;
}

// workspace of sdm_rt_table_backward: per-pick gradients, addressing partials (read set only), float64 sums
struct TablePlan {
  Plan p;
  int n_blk, addr_waves, key_bits;
  int64_t n_entries;
  size_t off_dw, off_pf, off_pd, off_pk, off_sums, off_keys, off_count, off_offsets, off_cub, cub_bytes, total;
};

int make_table_plan(const sdm_rt_dims* d, TablePlan* g) {
  int rc = make_plan(d, &g->p, false);
  if (rc) return rc;
  const Plan& p = g->p;
  if (p.d_a > 64) return set_err(SDM_RT_EUNSUPPORTED, "table backward: addr_dim %d exceeds 64", p.d_a);
  if (p.dh < 4 || p.dh % 4 != 0) return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d must be a positive multiple of 4", p.dh);
  g->addr_waves = addr_grad_waves(p.n_sub, p.half, p.pitch);
  if (!g->addr_waves) return set_err(SDM_RT_EUNSUPPORTED, "table backward: n_sub = %d sub-keys do not fit in LDS", p.n_sub);
  const int64_t N = static_cast<int64_t>(p.B) * p.T;
  const int64_t tpb = static_cast<int64_t>(g->addr_waves) * kAddrGradWaveTokens;
  g->n_blk = static_cast<int>((N + tpb - 1) / tpb);
  const size_t KSH = static_cast<size_t>(p.H) * 2 * p.n_sub * p.half;
  size_t o = 0;
  g->off_dw = o;
  o = align_up(o + sizeof(float) * N * p.H * p.pitch, 256);
  g->off_pf = o;
  o = align_up(o + sizeof(float) * g->n_blk * p.H * (2 + p.d_a), 256);
  g->off_pd = o;
  o = align_up(o + sizeof(double) * g->n_blk * p.H, 256);
  g->off_pk = o;
  o = align_up(o + sizeof(float) * g->n_blk * KSH, 256);
  g->off_sums = o;
  o = align_up(o + sizeof(double) * (static_cast<size_t>(p.H) * (2 + p.d_a) + p.H + KSH), 256);
  // the value-table gradient: sort keys and values (in and out), per-row counts and offsets, hipCUB's scratch
  g->n_entries = N * p.H * p.pitch;
  if (g->n_entries > 0x7fffffffLL) return set_err(SDM_RT_EUNSUPPORTED, "table backward: too many picks");
  const int n_keys = p.H * p.M + 1;
  g->key_bits = 1;
  while ((1LL << g->key_bits) <= n_keys) ++g->key_bits;
  g->off_keys = o;
  o = align_up(o + 4 * sizeof(int32_t) * static_cast<size_t>(g->n_entries), 256);
  g->off_count = o;
  o = align_up(o + sizeof(int32_t) * n_keys, 256);
  g->off_offsets = o;
  o = align_up(o + sizeof(int32_t) * n_keys, 256);
  size_t sort_bytes = 0, scan_bytes = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<const int32_t*>(nullptr),
                                         static_cast<int32_t*>(nullptr), static_cast<const int32_t*>(nullptr),
                                         static_cast<int32_t*>(nullptr), static_cast<int>(g->n_entries), 0,
                                         g->key_bits) != hipSuccess ||
      hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, static_cast<const int32_t*>(nullptr),
                                       static_cast<int32_t*>(nullptr), n_keys) != hipSuccess)
    return set_err(SDM_RT_ELAUNCH, "table backward: sort scratch size query failed");
  g->cub_bytes = sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
  g->off_cub = o;
  o = align_up(o + g->cub_bytes, 256);
  g->total = o;
  return SDM_RT_OK;
}

}  // namespace sdmrt

using namespace sdmrt;

// ---------------------------------------------------------------------------------------------------------------
// C ABI of the backward
extern "C" {

int sdm_rt_forward_train(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz,
                         int64_t kz_row_stride, const void* qz, int64_t qz_row_stride, const void* v,
                         int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                         sdm_rt_dtype in_dtype, const uint8_t* reset, void* r_out, int64_t out_row_stride,
                         sdm_rt_dtype out_dtype, const sdm_rt_saved* saved, void* workspace, size_t workspace_bytes,
                         void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p);
  if (rc) return rc;
  if ((rc = check_params(params, dims->out_norm != 0))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if ((rc = check_saved(saved, dims->read_mean != 0))) return rc;
  if (!kz || !qz || !v || !r_out) return set_err(SDM_RT_EINVAL, "kz, qz, v and r_out must not be NULL");
  if (dims->write_gate && !gate_logits) return set_err(SDM_RT_EINVAL, "write_gate is set but gate_logits is NULL");
  const int64_t wa = static_cast<int64_t>(p.H) * p.d_a;
  const int64_t wv = static_cast<int64_t>(p.H) * p.dh;
  if (kz_row_stride < wa || qz_row_stride < wa) return set_err(SDM_RT_EINVAL, "kz/qz row stride < heads * addr_dim");
  if (v_row_stride < wv) return set_err(SDM_RT_EINVAL, "v_row_stride < heads * head_dim");
  if (gate_logits && gate_row_stride < p.H) return set_err(SDM_RT_EINVAL, "gate_row_stride < heads");
  if (out_row_stride < wv) return set_err(SDM_RT_EINVAL, "out_row_stride < heads * head_dim");
  if (!workspace || workspace_bytes < p.total)
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, p.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const void* gl = dims->write_gate ? gate_logits : nullptr;

  // both address sets: picks, weights (gate included) and scores
  AddrArgs aa{};
  aa.g = addr_geom(p, params);
  aa.z = kz;
  aa.z_stride = kz_row_stride;
  aa.gl = gl;
  aa.g_stride = gate_row_stride;
  aa.B = p.B;
  aa.T = p.T;
  aa.pitch = p.pitch;
  aa.slot_out = saved->slots_w;
  aa.w_out = saved->weights_w;
  aa.s_out = saved->scores_w;
  aa.z2 = qz;
  aa.z2_stride = qz_row_stride;
  aa.slot_out2 = saved->slots_r;
  aa.w_out2 = saved->weights_r;
  aa.s_out2 = saved->scores_r;
  rc = launch_address(p, aa, in_dtype, st);
  if (rc) return rc;

  CoreIO io{};
  io.kz = kz;
  io.kz_stride = kz_row_stride;
  io.qz = qz;
  io.qz_stride = qz_row_stride;
  io.v = v;
  io.v_stride = v_row_stride;
  io.gate_logits = gl;
  io.g_stride = gate_row_stride;
  io.in_dtype = in_dtype;
  io.reset = reset;
  io.r_out = r_out;
  io.r_stride = out_row_stride;
  io.out_dtype = out_dtype;
  io.read_out = saved->read;
  io.den_out = dims->read_mean ? saved->den : nullptr;
  return run_core(p, dims, params, io, workspace, st);
}

size_t sdm_rt_backward_workspace_bytes(const sdm_rt_dims* dims) {
  GradPlan g;
  if (make_grad_plan(dims, &g) != SDM_RT_OK) return 0;
  return g.total;
}

int sdm_rt_backward(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                    const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                    const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, const uint8_t* reset,
                    const sdm_rt_saved* saved, const void* dy, int64_t dy_row_stride, sdm_rt_dtype dy_dtype,
                    const sdm_rt_grads* grads, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  GradPlan g;
  int rc = make_grad_plan(dims, &g);
  if (rc) return rc;
  const Plan& p = g.p;
  if ((rc = check_params(params, dims->out_norm != 0))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(dy_dtype, "dy_dtype"))) return rc;
  if (!grads) return set_err(SDM_RT_EINVAL, "grads is NULL");
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if ((rc = check_saved(saved, dims->read_mean != 0))) return rc;
  if (!kz || !qz || !v || !dy) return set_err(SDM_RT_EINVAL, "kz, qz, v and dy must not be NULL");
  if (dims->write_gate && !gate_logits) return set_err(SDM_RT_EINVAL, "write_gate is set but gate_logits is NULL");
  if (!grads->d_kz || !grads->d_qz || !grads->d_v)
    return set_err(SDM_RT_EINVAL, "grads: d_kz, d_qz and d_v must not be NULL");
  if (dims->write_gate && !grads->d_gate_logits)
    return set_err(SDM_RT_EINVAL, "grads: d_gate_logits must not be NULL when write_gate is set");
  const int64_t wa = static_cast<int64_t>(p.H) * p.d_a;
  const int64_t wv = static_cast<int64_t>(p.H) * p.dh;
  if (kz_row_stride < wa || qz_row_stride < wa) return set_err(SDM_RT_EINVAL, "kz/qz row stride < heads * addr_dim");
  if (v_row_stride < wv || dy_row_stride < wv) return set_err(SDM_RT_EINVAL, "v/dy row stride < heads * head_dim");
  if (gate_logits && gate_row_stride < p.H) return set_err(SDM_RT_EINVAL, "gate_row_stride < heads");
  if (grads->d_kz_row_stride < wa || grads->d_qz_row_stride < wa)
    return set_err(SDM_RT_EINVAL, "grads: d_kz/d_qz row stride < heads * addr_dim");
  if (grads->d_v_row_stride < wv) return set_err(SDM_RT_EINVAL, "grads: d_v row stride < heads * head_dim");
  if (dims->write_gate && grads->d_gate_row_stride < p.H)
    return set_err(SDM_RT_EINVAL, "grads: d_gate_logits row stride < heads");
  if (!workspace || workspace_bytes < g.total)
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, g.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* dnum = reinterpret_cast<float*>(ws + g.off_dnum);
  float* dden = reinterpret_cast<float*>(ws + g.off_dden);
  float* dotw = reinterpret_cast<float*>(ws + g.off_dotw);
  float* dotr = reinterpret_cast<float*>(ws + g.off_dotr);
  float* p1 = reinterpret_cast<float*>(ws + g.off_p1);
  float* pf = reinterpret_cast<float*>(ws + g.off_pf);
  double* pd = reinterpret_cast<double*>(ws + g.off_pd);
  float* pk = reinterpret_cast<float*>(ws + g.off_pk);
  const int64_t N = static_cast<int64_t>(p.B) * p.T;
  const float* onw = dims->out_norm ? params->onorm_w : nullptr;

  // 1. read-out backward
  {
    dim3 grid(g.n_rb, p.H);
    if (dy_dtype == SDM_RT_BF16) {
      hipLaunchKernelGGL((p.dh <= 64 ? read_grad_kernel<bf16_t, 1> : read_grad_kernel<bf16_t, 8>), grid, dim3(256), 0, st, static_cast<const bf16_t*>(dy),
                         dy_row_stride, saved->read, saved->den, onw, dnum, dden, p1, N, p.H, p.dh, dims->read_mean,
                         dims->read_eps, dims->out_norm_eps);
    } else {
      hipLaunchKernelGGL((p.dh <= 64 ? read_grad_kernel<float, 1> : read_grad_kernel<float, 8>), grid, dim3(256), 0, st, static_cast<const float*>(dy),
                         dy_row_stride, saved->read, saved->den, onw, dnum, dden, p1, N, p.H, p.dh, dims->read_mean,
                         dims->read_eps, dims->out_norm_eps);
    }
    if ((rc = check_launch("read grad"))) return rc;
  }
  // 2. forward replay: dwr
  {
    GradScanArgs a{};
    a.w_slot = saved->slots_w;
    a.w_wt = saved->weights_w;
    a.r_slot = saved->slots_r;
    a.r_wt = saved->weights_r;
    a.wv = v;
    a.wv_stride = v_row_stride;
    a.wc = nullptr;
    a.rv = dnum;
    a.rv_stride = wv;
    a.rc = dden;
    a.reset = reset;
    a.decay = params->decay;
    a.dot_out = dotr;
    a.sum_out = nullptr;
    a.B = p.B;
    a.T = p.T;
    a.H = p.H;
    a.dh = p.dh;
    a.M = p.M;
    a.kk = p.kk;
    a.n_chunks = p.n_chunks;
    a.chains = reinterpret_cast<const unsigned char*>(ws + g.off_chains);
    rc = in_dtype == SDM_RT_BF16 ? launch_grad_scan<false, bf16_t, float>(g, a, st)
                                 : launch_grad_scan<false, float, float>(g, a, st);
    if (rc) return rc;
  }
  // 3. reverse scan: dww and dV
  {
    GradScanArgs a{};
    a.w_slot = saved->slots_r;
    a.w_wt = saved->weights_r;
    a.r_slot = saved->slots_w;
    a.r_wt = saved->weights_w;
    a.wv = dnum;
    a.wv_stride = wv;
    a.wc = dden;
    a.rv = v;
    a.rv_stride = v_row_stride;
    a.rc = nullptr;
    a.reset = reset;
    a.decay = params->decay;
    a.dot_out = dotw;
    a.sum_out = grads->d_v;
    a.sum_stride = grads->d_v_row_stride;
    a.B = p.B;
    a.T = p.T;
    a.H = p.H;
    a.dh = p.dh;
    a.M = p.M;
    a.kk = p.kk;
    a.n_chunks = p.n_chunks;
    a.chains = reinterpret_cast<const unsigned char*>(ws + g.off_chains);
    rc = in_dtype == SDM_RT_BF16 ? launch_grad_scan<true, float, bf16_t>(g, a, st)
                                 : launch_grad_scan<true, float, float>(g, a, st);
    if (rc) return rc;
  }
  // 4. softmax, gate and address backward
  {
    AddrGradArgs a{};
    a.kz = kz;
    a.kz_stride = kz_row_stride;
    a.qz = qz;
    a.qz_stride = qz_row_stride;
    a.gl = dims->write_gate ? gate_logits : nullptr;
    a.g_stride = gate_row_stride;
    a.keys[0] = params->keys1;
    a.keys[1] = params->keys2;
    a.addr_b = params->addr_b;
    a.log_scale = params->log_scale;
    a.gate_bias = params->gate_bias;
    a.slot[0] = saved->slots_w;
    a.slot[1] = saved->slots_r;
    a.wt[0] = saved->weights_w;
    a.wt[1] = saved->weights_r;
    a.score[0] = saved->scores_w;
    a.score[1] = saved->scores_r;
    a.dot[0] = dotw;
    a.dot[1] = dotr;
    a.n_cg = g.n_cg;
    a.dz[0] = grads->d_kz;
    a.dz[1] = grads->d_qz;
    a.dz_stride[0] = grads->d_kz_row_stride;
    a.dz_stride[1] = grads->d_qz_row_stride;
    a.dgl = dims->write_gate ? grads->d_gate_logits : nullptr;
    a.dgl_stride = grads->d_gate_row_stride;
    a.part_f = pf;
    a.part_d = pd;
    a.part_k = pk;
    a.B = p.B;
    a.T = p.T;
    a.H = p.H;
    a.n_sub = p.n_sub;
    a.kk = p.kk;
    rc = in_dtype == SDM_RT_BF16 ? by_half<AddrGradLaunch, bf16_t>(p.half, g, a, st)
                                 : by_half<AddrGradLaunch, float>(p.half, g, a, st);
    if (rc) return rc;
  }
  // 5. parameter sums (fixed order, float64)
  {
    double* sums_f = reinterpret_cast<double*>(ws + g.off_sums);
    double* sums_d = sums_f + static_cast<size_t>(p.H) * (2 + p.d_a);
    double* sums_k = sums_d + p.H;
    double* sums_o = sums_k + static_cast<size_t>(p.H) * 2 * p.n_sub * p.half;
    const int n_rec = 2 * g.n_blk;
    auto reduce = [&](auto* part, int nr, int64_t items, double* out) {
      using T = std::remove_const_t<std::remove_pointer_t<decltype(part)>>;
      hipLaunchKernelGGL(reduce_records_kernel<T>, dim3(static_cast<unsigned>((items + 63) / 64)), dim3(64 * kRedGroups),
                         0, st, part, nr, items, items, out);
      return check_launch("reduce");
    };
    const int64_t F = 2 + p.d_a;
    const int64_t KSH = static_cast<int64_t>(p.H) * 2 * p.n_sub * p.half;
    if ((rc = reduce(static_cast<const float*>(pf), n_rec, p.H * F, sums_f))) return rc;
    if ((rc = reduce(static_cast<const double*>(pd), n_rec, p.H, sums_d))) return rc;
    hipLaunchKernelGGL(addr_post_kernel, dim3(p.H), dim3(128), 0, st, sums_f, sums_d, p.d_a, params->log_scale,
                       grads->d_log_scale, grads->d_gate_bias, grads->d_addr_b, grads->d_log_decay);
    if ((rc = check_launch("addr post"))) return rc;
    if (grads->d_keys1 || grads->d_keys2) {
      if (!grads->d_keys1 || !grads->d_keys2) return set_err(SDM_RT_EINVAL, "grads: give both d_keys1 and d_keys2");
      if ((rc = reduce(static_cast<const float*>(pk), n_rec, KSH, sums_k))) return rc;
      hipLaunchKernelGGL(keys_grad_kernel, dim3(p.H * 2 * p.n_sub), dim3(64), 0, st, sums_k, p.n_sub, p.half,
                         params->keys1, params->keys2, grads->d_keys1, grads->d_keys2);
      if ((rc = check_launch("keys grad"))) return rc;
    }
    if (grads->d_onorm_w && onw) {
      if ((rc = reduce(static_cast<const float*>(p1), g.n_rb, wv, sums_o))) return rc;
      hipLaunchKernelGGL(to_float_kernel, dim3(static_cast<unsigned>((wv + 255) / 256)), dim3(256), 0, st, sums_o, wv,
                         grads->d_onorm_w);
      if ((rc = check_launch("onorm"))) return rc;
    }
  }
  return SDM_RT_OK;
}

size_t sdm_rt_table_backward_workspace_bytes(const sdm_rt_dims* dims) {
  TablePlan g;
  if (make_table_plan(dims, &g) != SDM_RT_OK) return 0;
  return g.total;
}

int sdm_rt_table_backward(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* q, int64_t q_row_stride,
                          sdm_rt_dtype in_dtype, const int32_t* slots, const float* weights, const float* scores,
                          const void* values, sdm_rt_dtype values_dtype, const void* dy, int64_t dy_row_stride,
                          sdm_rt_dtype dy_dtype, float* d_q, int64_t d_q_row_stride, float* d_values,
                          float* d_keys1, float* d_keys2, float* d_log_scale, void* workspace,
                          size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  TablePlan g;
  int rc = make_table_plan(dims, &g);
  if (rc) return rc;
  const Plan& p = g.p;
  if ((rc = check_params(params, false, false))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(values_dtype, "values_dtype"))) return rc;
  if ((rc = check_dtype(dy_dtype, "dy_dtype"))) return rc;
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!q || !slots || !weights || !scores || !values || !dy || !d_q || !d_values)
    return set_err(SDM_RT_EINVAL, "q, slots, weights, scores, values, dy, d_q and d_values must not be NULL");
  if ((d_keys1 == nullptr) != (d_keys2 == nullptr)) return set_err(SDM_RT_EINVAL, "give both d_keys1 and d_keys2");
  const int64_t wa = static_cast<int64_t>(p.H) * p.d_a;
  const int64_t wv = static_cast<int64_t>(p.H) * p.dh;
  if (q_row_stride < wa || d_q_row_stride < wa) return set_err(SDM_RT_EINVAL, "q/d_q row stride < heads * addr_dim");
  if (dy_row_stride < wv) return set_err(SDM_RT_EINVAL, "dy_row_stride < heads * head_dim");
  if (!workspace || workspace_bytes < g.total)
    return set_err(SDM_RT_ENOSPACE, "workspace %zu bytes < required %zu", workspace_bytes, g.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* dw = reinterpret_cast<float*>(ws + g.off_dw);
  float* pf = reinterpret_cast<float*>(ws + g.off_pf);
  double* pd = reinterpret_cast<double*>(ws + g.off_pd);
  float* pk = reinterpret_cast<float*>(ws + g.off_pk);
  // 1. the value table gradient: picks sorted by (head, slot), then one wave per row
  {
    int32_t* kin = reinterpret_cast<int32_t*>(ws + g.off_keys);
    int32_t* kout = kin + g.n_entries;
    int32_t* vin = kout + g.n_entries;
    int32_t* vout = vin + g.n_entries;
    int32_t* count = reinterpret_cast<int32_t*>(ws + g.off_count);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + g.off_offsets);
    const int n_keys = p.H * p.M + 1;
    hipLaunchKernelGGL(zero_i32_kernel, dim3(static_cast<unsigned>((n_keys + 255) / 256)), dim3(256), 0, st, count,
                       n_keys);
    if ((rc = check_launch("zero"))) return rc;
    hipLaunchKernelGGL(pick_keys_kernel, dim3(static_cast<unsigned>((g.n_entries + 255) / 256)), dim3(256), 0, st,
                       slots, g.n_entries, p.T, p.H, p.pitch, p.M, p.kk, kin, vin, count);
    if ((rc = check_launch("pick keys"))) return rc;
    size_t cb = g.cub_bytes;
    if (hipcub::DeviceScan::ExclusiveSum(ws + g.off_cub, cb, count, offsets, n_keys, st) != hipSuccess)
      return set_err(SDM_RT_ELAUNCH, "table backward: scan failed");
    cb = g.cub_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(ws + g.off_cub, cb, kin, kout, vin, vout, static_cast<int>(g.n_entries), 0,
                                           g.key_bits, st) != hipSuccess)
      return set_err(SDM_RT_ELAUNCH, "table backward: sort failed");
    const unsigned rblocks = static_cast<unsigned>((static_cast<int64_t>(p.H) * p.M + 3) / 4);
    if (dy_dtype == SDM_RT_BF16) {
      hipLaunchKernelGGL(table_values_grad_kernel<bf16_t>, dim3(rblocks), dim3(256), 0, st, vout, offsets, count,
                         weights, static_cast<const bf16_t*>(dy), dy_row_stride, d_values, p.T, p.H, p.pitch, p.M,
                         p.dh);
    } else {
      hipLaunchKernelGGL(table_values_grad_kernel<float>, dim3(rblocks), dim3(256), 0, st, vout, offsets, count,
                         weights, static_cast<const float*>(dy), dy_row_stride, d_values, p.T, p.H, p.pitch, p.M,
                         p.dh);
    }
    if ((rc = check_launch("table values grad"))) return rc;
  }
  // 2. the per-pick gradients
  {
    const int64_t waves = static_cast<int64_t>(p.B) * p.T * p.H;
    const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
#define SDM_RT_TG(KP, VT, DT)                                                                                      \
  hipLaunchKernelGGL((table_grad_kernel<KP, VT, DT>), dim3(blocks), dim3(256), 0, st, slots, weights,              \
                     static_cast<const VT*>(values), static_cast<const DT*>(dy), dy_row_stride, dw, p.B, p.T, p.H,  \
                     p.M, p.dh, p.kk)
#define SDM_RT_TG_DT(KP, VT) \
  if (dy_dtype == SDM_RT_BF16) SDM_RT_TG(KP, VT, bf16_t); else SDM_RT_TG(KP, VT, float)
#define SDM_RT_TG_KP(VT) \
  if (p.pitch == 8) { SDM_RT_TG_DT(8, VT); } else { SDM_RT_TG_DT(16, VT); }
    if (values_dtype == SDM_RT_BF16) { SDM_RT_TG_KP(bf16_t); } else { SDM_RT_TG_KP(float); }
#undef SDM_RT_TG_KP
#undef SDM_RT_TG_DT
#undef SDM_RT_TG
    if ((rc = check_launch("table grad"))) return rc;
  }
  // 3. softmax and product-key backward of the read set (no gate, no address bias)
  {
    GradPlan gp;
    gp.p = p;
    gp.n_blk = g.n_blk;
    gp.addr_waves = g.addr_waves;
    AddrGradArgs a{};
    a.kz = q;
    a.kz_stride = q_row_stride;
    a.qz = q;
    a.qz_stride = q_row_stride;
    a.keys[0] = params->keys1;
    a.keys[1] = params->keys2;
    a.log_scale = params->log_scale;
    a.slot[1] = slots;
    a.wt[1] = weights;
    a.score[1] = scores;
    a.dot[1] = dw;
    a.n_cg = 1;
    a.dz[1] = d_q;
    a.dz_stride[1] = d_q_row_stride;
    a.part_f = pf;
    a.part_d = pd;
    a.part_k = pk;
    a.B = p.B;
    a.T = p.T;
    a.H = p.H;
    a.n_sub = p.n_sub;
    a.kk = p.kk;
    a.set0 = 1;
    rc = in_dtype == SDM_RT_BF16 ? by_half<AddrGradLaunch, bf16_t>(p.half, gp, a, st)
                                 : by_half<AddrGradLaunch, float>(p.half, gp, a, st);
    if (rc) return rc;
  }
  // 4. parameter sums (fixed order, float64)
  double* sums_f = reinterpret_cast<double*>(ws + g.off_sums);
  double* sums_d = sums_f + static_cast<size_t>(p.H) * (2 + p.d_a);
  double* sums_k = sums_d + p.H;
  const int64_t F = 2 + p.d_a;
  const int64_t KSH = static_cast<int64_t>(p.H) * 2 * p.n_sub * p.half;
  hipLaunchKernelGGL(reduce_records_kernel<float>, dim3(static_cast<unsigned>((p.H * F + 63) / 64)),
                     dim3(64 * kRedGroups), 0, st, static_cast<const float*>(pf), g.n_blk, p.H * F, p.H * F, sums_f);
  if ((rc = check_launch("reduce"))) return rc;
  hipLaunchKernelGGL(reduce_records_kernel<double>, dim3(static_cast<unsigned>((p.H + 63) / 64)),
                     dim3(64 * kRedGroups), 0, st, static_cast<const double*>(pd), g.n_blk, p.H, p.H, sums_d);
  if ((rc = check_launch("reduce"))) return rc;
  hipLaunchKernelGGL(addr_post_kernel, dim3(p.H), dim3(128), 0, st, sums_f, sums_d, p.d_a, params->log_scale,
                     d_log_scale, nullptr, nullptr, nullptr);
  if ((rc = check_launch("addr post"))) return rc;
  if (d_keys1) {
    hipLaunchKernelGGL(reduce_records_kernel<float>, dim3(static_cast<unsigned>((KSH + 63) / 64)),
                       dim3(64 * kRedGroups), 0, st, static_cast<const float*>(pk), g.n_blk, KSH, KSH, sums_k);
    if ((rc = check_launch("reduce"))) return rc;
    hipLaunchKernelGGL(keys_grad_kernel, dim3(p.H * 2 * p.n_sub), dim3(64), 0, st, sums_k, p.n_sub, p.half,
                       params->keys1, params->keys2, d_keys1, d_keys2);
    if ((rc = check_launch("keys grad"))) return rc;
  }
  return SDM_RT_OK;
}

}  // extern "C"
