// sdm_plan.h -- plan_kernel: product-key addressing of one chunk of 64 positions of one (batch row, head) and the
// plan the scan executes for it (RunTimeSdm._chunk, experiments/track4/sdmllm/track4_onesdm_models.py:215-241, with
// pk_address :134-148 and the softmax weights and gate of prepare :203-207).  Included by sdm_plan_bf16.hip and
// sdm_plan_f32.hip, which instantiate it per input type.
//
// One plan per (batch row, head, chunk) at a fixed stride (PlanGeom) in the workspace.
//   position records [64], 16 KP + 48 bytes each, for position p of the chunk:
//     u32 roff[KP]    read picks as byte offsets of their slab rows in the scan's LDS (slot * row_bytes; pads: row M,
//                     which stays zero)
//     f32 rw[KP]      read weights (0 for pads and when a reset earlier in the chunk hides the carried state)
//     u32 woff[KP]    write picks owned by p (p is the first writer of the slot among the writers the chunk keeps) as
//                     row byte offsets; picks p does not own: row M
//     f32 wc[KP]      owned pick: lam^(L-1-p) * ww, p's faded write coefficient; else 0
//     tail, 12 words:
//       t0  n_in (bits 0..15: in-chunk read contributions) | ro (bits 16..31: entry index of those past the inline)
//       t1  csum, the sum of all in-chunk read coefficients (the mean read's in-chunk denominator)
//       t2, t3  q of the first kInline contributions (u8 each; 0 when unused)
//       t4..t9  their coefficients (0 when unused)
//   variable part: a 16-byte header {bytes, flags (bit 31: the chunk holds a reset), x0, n_x}, then 8-byte entries:
//     read contributions past the inline ones {c, q}: position q < p of the chunk wrote some of p's read slots,
//       c = the sum over those slots of wr * ww * lam^(p-1-q); a position's contributions run in ascending q
//     from x0, the n_x records {row offset, e | n << 16} of the slots written more than once, then the n entries
//       {c = lam^(L-1-q) * ww, q} of each one's later writers (the owner's write is in its position record) from
//       entry e, in ascending q
//   sizes[] holds the bytes of each plan's variable part.
#pragma once

#include "sdm_common.h"

namespace sdmrt {

struct PlanArgs {
  AddrGeom g;
  const void* kz;
  int64_t kz_stride;
  const void* qz;
  int64_t qz_stride;
  const void* gl;          // gate logit rows or nullptr
  int64_t g_stride;
  const float* decay;      // [H]
  const uint8_t* reset;    // [B*T rows] or nullptr: 1 empties the memory before that position reads
  unsigned char* plans;    // [B][H][n_chunks][stride]
  int32_t* sizes;          // [B][H][n_chunks] bytes of each plan's variable part
  uint32_t* sync;          // [B*H][groups] scan progress counters, then a status word: zeroed here, or nullptr
  unsigned long long* xch; // pick plans: [B*H][n_chunks][xgroups][64] out-norm partial sums, cleared here, or nullptr
  void* gate_copy;         // [B*T][H] of the input type: the gate logits as read (rows of H), or nullptr
  int groups;
  int xgroups;             // column groups of the pick scan
  int row_bytes;           // bytes of a slab row in the scan's LDS (its column group width * 4)
  int B, T, M, n_chunks;
};

// The pick plan of one chunk (PickGeom, sdm_common.h) from the picks in registers and the writer masks in LDS:
// wave 1 (set 1) writes the read records of its position (the in-chunk read contributions in ascending q, number j
// into the record of pick j, those past the eighth into the variable part), wave 0 the write records (owned picks,
// the first later writer inline, the others into the variable part).  Every thread of the block calls it.
__device__ __forceinline__ void emit_pick_plan(const PlanArgs& a, int b, int h, int c, int set, int p, int L, int M,
                                               int kk, const int (&ms)[8], const float (&ws)[8],
                                               const unsigned long long* wmask, const uint16_t* sbase,
                                               const float* wtab, const float* pw, int* tot, int seg0,
                                               unsigned long long rmask, unsigned long long keep) {
  constexpr int KP = 8;
  auto rank_below = [&](int m, int q) {   // sbase[m] + the writes of slot m by positions before q
    return static_cast<int>(sbase[m]) + __builtin_popcountll(wmask[m] & ((1ull << q) - 1ull));
  };
  unsigned long long mk[KP];   // read side: the earlier writers (same segment) of each read slot
  int rk[KP];                  // read side: the rank in wtab of each read slot's next earlier writer
  unsigned long long touched = 0ull;
  int n_in = 0, n_e = 0;
  uint32_t own = 0u;
  int nl[KP];                  // write side: later writers of each owned slot
#pragma unroll
  for (int j = 0; j < KP; ++j) nl[j] = 0;
  if (p < L) {
    if (set == 1) {
      const unsigned long long below = ((1ull << p) - 1ull) & (seg0 >= 0 ? ~((1ull << seg0) - 1ull) : ~0ull);
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        mk[i] = i < kk ? wmask[ms[i]] & below : 0ull;
        rk[i] = i < kk ? rank_below(ms[i], seg0 >= 0 ? seg0 : 0) : 0;
        touched |= mk[i];
      }
      n_in = __builtin_popcountll(touched);
      n_e = max(n_in - KP, 0);
    } else {
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) {
          const unsigned long long mm = wmask[ms[j]] & keep;
          if (mm && __builtin_ctzll(mm) == p) {
            own |= 1u << j;
            nl[j] = __builtin_popcountll(mm) - 1;
            n_e += max(nl[j] - 1, 0);
          }
        }
      }
    }
  }
  const int inc_e = wave_incl_scan(n_e, p);
  if (p == 63) tot[set] = inc_e;
  __syncthreads();
  const int n_ro = tot[1], n_wo = tot[0];
  const int64_t plan_id = (static_cast<int64_t>(b) * a.g.H + h) * a.n_chunks + c;
  if (a.xch) {   // the chunk's out-norm partial sums: not yet written
    unsigned long long* x = a.xch + plan_id * a.xgroups * kChunk;
    for (int i = set * 64 + p; i < a.xgroups * kChunk; i += 128) x[i] = 0ull;
  }
  unsigned char* plan = a.plans + plan_id * PickGeom::stride();
  uint2* ent = reinterpret_cast<uint2*>(plan + PickGeom::off_var() + PickGeom::off_ent());
  if (set == 0 && p == 0) {
    const int bytes = PickGeom::off_ent() + 8 * (n_ro + n_wo);
    *reinterpret_cast<uint4*>(plan + PickGeom::off_var()) = make_uint4(
        static_cast<uint32_t>(bytes), rmask ? 0x80000000u : 0u, static_cast<uint32_t>(n_ro), static_cast<uint32_t>(n_wo));
    a.sizes[plan_id] = bytes;
  }
  const uint32_t mrow = static_cast<uint32_t>(M);
  if (set == 1) {
    const int e0 = n_wo + inc_e - n_e;   // the position's first entry past its eighth contribution (after the writes')
    reinterpret_cast<uint16_t*>(plan + PickGeom::off_var() + 16)[p] = static_cast<uint16_t>(e0);
    float cj[KP];
    uint32_t qj[KP];
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      cj[i] = 0.f;
      qj[i] = 0u;
    }
    int j = 0;
    while (touched) {
      const int q = __builtin_ctzll(touched);
      touched &= touched - 1ull;
      float wq[KP];
#pragma unroll
      for (int i = 0; i < KP; ++i) wq[i] = wtab[min(rk[i], kChunk * KP - 1)];
      float coef = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        const bool hit = (mk[i] >> q) & 1ull;
        coef = fmaf(ws[i], hit ? wq[i] : 0.f, coef);
        rk[i] += hit ? 1 : 0;
      }
      coef *= pw[p - 1 - q];
      if (j < KP) {
#pragma unroll
        for (int t = 0; t < KP; ++t)
          if (t == j) {
            cj[t] = coef;
            qj[t] = static_cast<uint32_t>(q);
          }
      } else {
        ent[e0 + j - KP] = make_uint2(__float_as_uint(coef), static_cast<uint32_t>(q));
      }
      ++j;
    }
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const uint32_t slot = (p < L && i < kk) ? static_cast<uint32_t>(ms[i]) : mrow;
      const float rw = (p < L && i < kk && seg0 < 0) ? ws[i] : 0.f;
      *reinterpret_cast<uint3*>(plan + PickGeom::kRec * (i * kChunk + p)) =
          make_uint3(slot | (qj[i] << 16) | (static_cast<uint32_t>(n_in) << 24), __float_as_uint(rw),
                     __float_as_uint(cj[i]));
    }
  } else {
    int e = inc_e - n_e;   // the write entries come first: the owners walk them in sequence, so they stay in LDS
#pragma unroll
    for (int jj = 0; jj < KP; ++jj) {
      uint32_t w0 = mrow;
      float wc = 0.f, l0 = 0.f;
      if ((own >> jj) & 1u) {
        const int m = ms[jj];
        // the later writers past the first start at entry e (< 511)
        w0 = static_cast<uint32_t>(m) | (static_cast<uint32_t>(nl[jj]) << 17) | (static_cast<uint32_t>(e) << 23);
        wc = pw[L - 1 - p] * ws[jj];
        if (nl[jj] > 0) {
          unsigned long long mm = (wmask[m] & keep) & ~(1ull << p);   // every writer of m after p
          int rank = rank_below(m, p) + 1;
          const int q1 = __builtin_ctzll(mm);
          mm &= mm - 1ull;
          w0 |= static_cast<uint32_t>(q1) << 11;
          l0 = pw[L - 1 - q1] * wtab[rank++];
          while (mm) {
            const int q = __builtin_ctzll(mm);
            mm &= mm - 1ull;
            ent[e++] = make_uint2(__float_as_uint(pw[L - 1 - q] * wtab[rank++]), static_cast<uint32_t>(q));
          }
        }
      }
      *reinterpret_cast<uint3*>(plan + PickGeom::off_w() + PickGeom::kRec * (jj * kChunk + p)) =
          make_uint3(w0, __float_as_uint(wc), __float_as_uint(l0));
    }
  }
}

// plan_kernel: block (chunk, head, batch row), 128 threads: wave 0 addresses the write keys of the chunk's
// positions, wave 1 the read queries (MODE 1, 2: on the matrix cores, MODE 0: per thread); the writers of every slot
// are marked in 64-bit masks; wave 1 then finds each position's in-chunk read contributions, wave 0 each position's
// owned writes and the later writers of the slots written more than once; entry counts are prefix-summed within
// each wave.  PICK: the plan is a pick plan (emit_pick_plan) for pick_scan_kernel.
template <int HALF, int KP, typename InT, int MODE, bool PICK = false>
__global__ void __launch_bounds__(128, 3) plan_kernel(PlanArgs a) {
  constexpr PlanGeom pg{KP};
  const int c = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int set = tid >> 6;     // 0: write keys, 1: read queries
  const int p = tid & 63;
  const int M = a.M;
  const int kk = a.g.kk;
  const int c0 = c * kChunk;
  const int L = min(kChunk, a.T - c0);
  const float lam = a.decay[h];

  __shared__ float pw[kChunk + 4];
  __shared__ int tot[4];
  // dynamic: the writers of every slot [M] (bit q: position q wrote it), the first rank of every slot's writes [M],
  // the write weights by slot and rank [64 KP], then (per-thread path) the head's sub-keys [2][n_sub][HALF]
  extern __shared__ unsigned long long wmask[];
  uint16_t* sbase = reinterpret_cast<uint16_t*>(wmask + M);
  float* wtab = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(sbase) + plan_rank_bytes(M));
  float* kn = wtab + kChunk * KP;

  if (c == 0 && a.sync && tid < a.groups) a.sync[(static_cast<int64_t>(b) * a.g.H + h) * a.groups + tid] = 0u;
  if (c == 0 && h == 0 && b == 0 && a.sync && tid == 0)
    a.sync[static_cast<int64_t>(a.B) * a.g.H * a.groups] = 0u;   // the status word
  if constexpr (MODE == 0) stage_keys<HALF>(a.g, h, kn, tid, 128);
  for (int i = tid; i < M; i += 128) wmask[i] = 0ull;
  if (tid <= kChunk) {
    float v = 1.f, sq = lam;   // lam^tid by squaring (exact for lam = 0 and lam = 1)
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      v = ((tid >> bit) & 1) ? v * sq : v;
      sq *= sq;
    }
    pw[tid] = v;
  }
  if constexpr (MODE == 0) __syncthreads();

  // addressing: the position's picks (slots; pads M) and weights, kept in registers
  int ms[KP];
  float ws[KP];
  {
    int slot[KP];
    float w[KP], sc[KP];
    const int64_t row0 = static_cast<int64_t>(b) * a.T + c0;
    const float gate = (set == 0 && a.gl && p < L)
                           ? gate_of(static_cast<const InT*>(a.gl) + (row0 + p) * a.g_stride, h, a.g.gate_bias)
                           : 1.f;
    if (set == 0 && a.gate_copy && p < L)   // the caller's compact copy of the logits (RunTimeSdm.last_gate)
      static_cast<InT*>(a.gate_copy)[(row0 + p) * a.g.H + h] = static_cast<const InT*>(a.gl)[(row0 + p) * a.g_stride + h];
    const InT* zb = static_cast<const InT*>(set == 0 ? a.kz : a.qz);
    const int64_t zs = set == 0 ? a.kz_stride : a.qz_stride;
    if constexpr (MODE > 0) {
      address_wave<HALF, KP, InT, MODE == 2>(a.g, h, zb + row0 * zs, zs, L, gate, slot, w, sc);
    } else if (p < L) {
      address_one<HALF, KP, InT>(a.g, h, kn, zb + (row0 + p) * zs + static_cast<int64_t>(h) * 2 * HALF, gate, slot, w,
                                 sc);
    }
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      const bool live = p < L && j < kk;
      ms[j] = live ? slot[j] : M;
      ws[j] = live ? w[j] : 0.f;
    }
  }
  // resets of the chunk (OM:229-233, 287-289): a reader sees the writers of its own segment only, no carried state
  // after a reset, and only the writers after the chunk's last reset reach the state the chunk leaves
  const unsigned long long rmask = __ballot(a.reset && p < L && a.reset[static_cast<int64_t>(b) * a.T + c0 + p]);
  const unsigned long long upto = rmask & (p == 63 ? ~0ull : (2ull << p) - 1ull);
  const int seg0 = upto ? 63 - __builtin_clzll(upto) : -1;          // this position's segment start in the chunk
  const int last = rmask ? 63 - __builtin_clzll(rmask) : -1;        // the chunk's last reset
  const unsigned long long keep = last >= 0 ? ~((1ull << last) - 1ull) : ~0ull;   // writers that reach the state
  __syncthreads();
  // mark the writers of every slot
  if (set == 0 && p < L) {
    for (int j = 0; j < kk; ++j) atomicOr(&wmask[ms[j]], 1ull << p);
  }
  __syncthreads();
  // the write weights by slot and rank: the writes of slot m, in ascending position, are wtab[sbase[m] ...]; the
  // write of position q is at rank popcount(wmask[m] below q) (a position's picks are distinct locations)
  {
    const int spt = (M + 127) / 128;   // slots per thread
    const int m0 = min(tid * spt, M), m1 = min(m0 + spt, M);
    int n = 0;
    for (int m = m0; m < m1; ++m) n += __builtin_popcountll(wmask[m]);
    const int inc = wave_incl_scan(n, p);
    if (p == 63) tot[set] = inc;
    __syncthreads();
    int run = inc - n + (set == 1 ? tot[0] : 0);
    for (int m = m0; m < m1; ++m) {
      sbase[m] = static_cast<uint16_t>(run);
      run += __builtin_popcountll(wmask[m]);
    }
  }
  __syncthreads();
  auto rank_below = [&](int m, int q) {   // sbase[m] + the writes of slot m by positions before q
    return static_cast<int>(sbase[m]) + __builtin_popcountll(wmask[m] & ((1ull << q) - 1ull));
  };
  if (set == 0 && p < L) {
    for (int j = 0; j < kk; ++j) wtab[rank_below(ms[j], p)] = ws[j];
  }
  __syncthreads();
  if constexpr (PICK) {
    emit_pick_plan(a, b, h, c, set, p, L, M, kk, ms, ws, wmask, sbase, wtab, pw, tot, seg0, rmask, keep);
    return;
  }
  unsigned long long mk[KP];           // read side: the earlier writers of each read slot
  int rk[KP];                          // read side: the rank in wtab of each read slot's next earlier writer
  unsigned long long touched = 0ull;   // read side: every earlier position contributing to this one
  int n_in = 0;                        // read side: contributions
  int n_e = 0;                         // entries in the variable part (read side: past the inline; write: later writers)
  uint32_t own = 0u, more = 0u;        // write side: picks owned, and owned with later writers
  if (p < L) {
    if (set == 1) {
      const unsigned long long below = ((1ull << p) - 1ull) & (seg0 >= 0 ? ~((1ull << seg0) - 1ull) : ~0ull);
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        mk[i] = i < kk ? wmask[ms[i]] & below : 0ull;
        rk[i] = i < kk ? rank_below(ms[i], seg0 >= 0 ? seg0 : 0) : 0;
        touched |= mk[i];
      }
      n_in = __builtin_popcountll(touched);
      n_e = max(n_in - kInline, 0);
    } else {
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) {
          const unsigned long long mm = wmask[ms[j]] & keep;
          if (mm && __builtin_ctzll(mm) == p) {
            own |= 1u << j;
            const int later = __builtin_popcountll(mm) - 1;
            if (later > 0) {
              more |= 1u << j;
              n_e += later;   // the later writers' entries
            }
          }
        }
      }
    }
  }
  const int inc_e = wave_incl_scan(n_e, p);
  const int n_rec = __builtin_popcount(more);   // write side: records of slots written more than once
  const int inc_rec = wave_incl_scan(n_rec, p);
  if (p == 63) {
    tot[set] = inc_e;
    if (set == 0) tot[2] = inc_rec;
  }
  __syncthreads();
  const int n_ro = tot[1], n_x = tot[2], n_le = tot[0];   // read overflow, then the records, then their writers
  const int64_t plan_id = (static_cast<int64_t>(b) * a.g.H + h) * a.n_chunks + c;
  unsigned char* plan = a.plans + plan_id * pg.stride();
  unsigned char* prec = plan + p * pg.pos_bytes();
  uint2* ent = reinterpret_cast<uint2*>(plan + pg.off_var() + 16);
  if (tid == 0) {
    const int bytes = 16 + 8 * (n_ro + n_x + n_le);
    *reinterpret_cast<uint4*>(plan + pg.off_var()) = make_uint4(
        static_cast<uint32_t>(bytes), rmask ? 0x80000000u : 0u, static_cast<uint32_t>(n_ro), static_cast<uint32_t>(n_x));
    a.sizes[plan_id] = bytes;
  }
  uint32_t* tail = reinterpret_cast<uint32_t*>(prec + pg.off_tail());
  const uint32_t null_row = static_cast<uint32_t>(M) * static_cast<uint32_t>(a.row_bytes);
  if (set == 1) {
    // read picks as row offsets and their weights (no carried state after a reset in this chunk)
#pragma unroll
    for (int i = 0; i < KP; i += 4) {
      *reinterpret_cast<uint4*>(prec + 4 * i) =
          make_uint4(ms[i] * a.row_bytes, ms[i + 1] * a.row_bytes, ms[i + 2] * a.row_bytes, ms[i + 3] * a.row_bytes);
      *reinterpret_cast<uint4*>(prec + pg.off_rw() + 4 * i) =
          seg0 >= 0 ? make_uint4(0u, 0u, 0u, 0u)
                    : make_uint4(__float_as_uint(ws[i]), __float_as_uint(ws[i + 1]), __float_as_uint(ws[i + 2]),
                                 __float_as_uint(ws[i + 3]));
    }
    // in-chunk contributions in ascending q: the first kInline into the tail, the rest into the variable part
    const int e0 = inc_e - n_e;
    int k = e0, j = 0;
    float csum = 0.f;
    unsigned long long qb = 0ull;
    float ic[kInline] = {};
    while (touched) {
      const int q = __builtin_ctzll(touched);
      touched &= touched - 1ull;
      // q's weight for each of p's read slots it wrote: every slot's next writer is read at once (the slots q
      // did not write add nothing)
      float wq[KP];
#pragma unroll
      for (int i = 0; i < KP; ++i) wq[i] = wtab[min(rk[i], kChunk * KP - 1)];
      float coef = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        const bool hit = (mk[i] >> q) & 1ull;
        coef = fmaf(ws[i], hit ? wq[i] : 0.f, coef);
        rk[i] += hit ? 1 : 0;
      }
      coef *= pw[p - 1 - q];
      if (j < kInline) {
        qb |= static_cast<unsigned long long>(q) << (8 * j);
#pragma unroll
        for (int t = 0; t < kInline; ++t)
          if (t == j) ic[t] = coef;
        ++j;
      } else {
        ent[k++] = make_uint2(__float_as_uint(coef), static_cast<uint32_t>(q));
      }
      csum += coef;
    }
    *reinterpret_cast<uint4*>(tail) =
        make_uint4(static_cast<uint32_t>(n_in) | (static_cast<uint32_t>(e0) << 16), __float_as_uint(csum),
                   static_cast<uint32_t>(qb), static_cast<uint32_t>(qb >> 32));
    *reinterpret_cast<uint4*>(tail + 4) =
        make_uint4(__float_as_uint(ic[0]), __float_as_uint(ic[1]), __float_as_uint(ic[2]), __float_as_uint(ic[3]));
    *reinterpret_cast<uint4*>(tail + 8) = make_uint4(__float_as_uint(ic[4]), __float_as_uint(ic[5]), 0u, 0u);
  } else {
    // owned write picks as row offsets with their coefficients; the records and later writers of the slots written
    // more than once
    int e = n_ro + n_x + inc_e - n_e;
    int r = n_ro + inc_rec - n_rec;
    uint32_t wo[KP], wcv[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      wo[j] = null_row;
      wcv[j] = 0u;
      if ((own >> j) & 1u) {
        wo[j] = static_cast<uint32_t>(ms[j]) * static_cast<uint32_t>(a.row_bytes);
        wcv[j] = __float_as_uint(pw[L - 1 - p] * ws[j]);
        if ((more >> j) & 1u) {
          const int m = ms[j];
          unsigned long long mm = (wmask[m] & keep) & ~(1ull << p);   // every writer of m after p
          const int e_first = e;
          int rank = rank_below(m, p) + 1;
          while (mm) {
            const int q = __builtin_ctzll(mm);
            mm &= mm - 1ull;
            ent[e++] = make_uint2(__float_as_uint(pw[L - 1 - q] * wtab[rank++]), static_cast<uint32_t>(q));
          }
          ent[r++] = make_uint2(wo[j], static_cast<uint32_t>(e_first) | (static_cast<uint32_t>(e - e_first) << 16));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KP; i += 4) {
      *reinterpret_cast<uint4*>(prec + pg.off_woff() + 4 * i) = make_uint4(wo[i], wo[i + 1], wo[i + 2], wo[i + 3]);
      *reinterpret_cast<uint4*>(prec + pg.off_wc() + 4 * i) = make_uint4(wcv[i], wcv[i + 1], wcv[i + 2], wcv[i + 3]);
    }
  }
}

template <int HALF, typename InT>
struct PlanLaunch {
  template <int KP, int MODE, bool PICK>
  static int go(const Plan& p, const PlanArgs& a, hipStream_t st) {
    dim3 grid(p.n_chunks, p.H, p.B);
    const size_t lds = plan_dynamic_lds(p.M, KP) + (MODE > 0 ? 0 : sizeof(float) * 2 * p.n_sub * HALF);
    static const bool ok = allow_lds(reinterpret_cast<const void*>(&plan_kernel<HALF, KP, InT, MODE, PICK>));
    if (!ok) return lds_err("plan");
    hipLaunchKernelGGL((plan_kernel<HALF, KP, InT, MODE, PICK>), grid, dim3(128), lds, st, a);
    return check_launch("plan");
  }
  // pick: write pick plans (matrix-core addressing and picks of at most 8 only)
  static int run(const Plan& p, const PlanArgs& a, hipStream_t st, bool pick) {
    if constexpr (mf_half(HALF)) {
      if (use_mf(p)) {
        if (pick) return full_grid(p) ? go<8, 2, true>(p, a, st) : go<8, 1, true>(p, a, st);
        return full_grid(p) ? go<8, 2, false>(p, a, st)
                            : p.pitch == 8 ? go<8, 1, false>(p, a, st) : go<16, 1, false>(p, a, st);
      }
    }
    if (pick) return set_err(SDM_RT_EINVAL, "pick plans need the matrix-core addressing");
    return p.pitch == 8 ? go<8, 0, false>(p, a, st) : go<16, 0, false>(p, a, st);
  }
};

// defined in sdm_plan_bf16.hip and sdm_plan_f32.hip
int launch_plan_bf16(const Plan& p, const PlanArgs& a, hipStream_t st, bool pick);
int launch_plan_f32(const Plan& p, const PlanArgs& a, hipStream_t st, bool pick);

}  // namespace sdmrt
