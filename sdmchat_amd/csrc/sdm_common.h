// sdm_common.h -- internals shared by the translation units of libsdm_rt.so (gfx950): element types, the
// product-key addressing (device), cross-lane helpers, and the host-side shape plan and launch helpers.  Everything
// here is inline or a template, in namespace sdmrt; the C ABI is declared in include/sdm_rt.h.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <type_traits>

#include "sdm_rt.h"

namespace sdmrt {

// ---------------------------------------------------------------------------------------------------------------
// error reporting (defined in sdm_errors.hip): a thread-local message, read by sdm_rt_last_error
extern thread_local char g_err[512];
int set_err(int code, const char* fmt, ...);

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
constexpr int kChunk = 64;                          // positions per chunk (one bit each in the writer masks)
constexpr size_t kLdsBytes = 160 * 1024;            // LDS per workgroup on gfx950

// ---------------------------------------------------------------------------------------------------------------
// addressing of one (token, head, address set)

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

struct AddrGeom {
  const float* keys[2];    // [H][n_sub][half] sub-keys of each half (unit-normalised where they are used,
                           // F.normalize of keys, track4_onesdm_models.py:137-140)
  const float* addr_b;     // [H][d_a] or nullptr
  const float* log_scale;  // [H]
  const float* gate_bias;  // [H] or nullptr
  // the bfloat16 scoring's sub-key pieces prepared once for these keys and addr_b (sdm_rt_prepare_key_pieces,
  // KeyPieces below), or nullptr: every scoring wave then normalises and splits its sub-keys itself
  const uint32_t* kpieces;
  int H, n_sub, c1, kk;
};

// Picks of one address (pk_address, track4_onesdm_models.py:134-148): z (2*HALF values of type InT, plus addr_b)
// split in two unit halves, each scored against the n_sub unit sub-keys of its half, exact top-c1 per half, exact
// top-kk of the dominance-pruned c1 x c1 grid of mean scores, slot = i1 * n_sub + i2; weights
// softmax(exp(log_scale) * score) (prepare :203-206) times `gate`.  Pad entries (>= kk): slot 0, weight 0, score 0.
// kn: the head's unit sub-keys, [2][n_sub][HALF] (staged in LDS by the caller).
template <int HALF, int CAP, typename InT>
__device__ __forceinline__ void address_one(const AddrGeom& g, int h, const float* kn, const InT* zrow, float gate,
                                            int (&slot)[CAP], float (&w)[CAP], float (&score)[CAP]) {
  constexpr int DA = 2 * HALF;
  float z[DA];
#pragma unroll
  for (int d = 0; d < DA; ++d) {
    const float bias = g.addr_b ? g.addr_b[h * DA + d] : 0.f;
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
    const float* kb = kn + part * g.n_sub * HALF;
    for (int s = 0; s < g.n_sub; ++s) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < HALF; ++d) acc = fmaf(u[d], kb[s * HALF + d], acc);
      top_insert<CAP>(hv[part], hi[part], acc, s, g.c1);
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
    if (ra < g.c1) {
#pragma unroll
      for (int rb = 0; rb < CAP; ++rb) {
        if (rb < g.c1 && (ra + 1) * (rb + 1) <= g.kk) {
          const float s = (hv[0][ra] + hv[1][rb]) * 0.5f;
          top_insert<CAP>(cv, ci, s, ra * g.c1 + rb, g.kk);
        }
      }
    }
  }
  // softmax over the kk picks; the first pick holds the maximum
  const float scale = expf(g.log_scale[h]);
  float e[CAP];
  const float x0 = cv[0] * scale;
  float sum = 0.f;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    e[p] = (p < g.kk) ? expf(cv[p] * scale - x0) : 0.f;
    sum += e[p];
  }
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    const bool live = p < g.kk;
    int sl = 0;
    if (live) {
      const int ra = ci[p] / g.c1;
      const int rb = ci[p] - ra * g.c1;
      int i1 = 0, i2 = 0;
#pragma unroll
      for (int q = 0; q < CAP; ++q) {
        if (q == ra) i1 = hi[0][q];
        if (q == rb) i2 = hi[1][q];
      }
      sl = i1 * g.n_sub + i2;
    }
    slot[p] = sl;
    w[p] = live ? e[p] / sum * gate : 0.f;
    score[p] = live ? cv[p] : 0.f;
  }
}

template <typename InT>
__device__ __forceinline__ float gate_of(const InT* grow, int h, const float* gate_bias) {
  const float logit = to_f32(grow[h]) + (gate_bias ? gate_bias[h] : 0.f);
  return 1.f / (1.f + expf(-logit));
}

// ---------------------------------------------------------------------------------------------------------------
// addressing of 64 addresses by one wave on the matrix cores (n_sub <= 32, half width HALF = 2 * S, S in {4, 8, 16})
//
// The scores of one half form the 32 x 64 product of the zero-padded unit sub-keys and the 64 unit address halves:
// two 32 x 32 tiles of v_mfma_f32_32x32x2f32 accumulated over S steps.  Lane l feeds sub-key row l % 32 and address
// column l % 32 of a tile, with dims (l / 32) * S + s at step s.  Lane l's output covers address l % 32 of the tile
// and sub-keys 8 * (r / 4) + 4 * (l / 32) + r % 4 (r < 16); one permlane32 swap per output register leaves lane l
// with all 32 sub-key scores of address l.  Selection then runs per lane on f64 keys with bitonic networks.

typedef float floatx16 __attribute__((ext_vector_type(16)));

// f64 selection key: plain double order = (score descending, then lower tie index first).  A float converted to
// double has 29 zero low mantissa bits; they hold a TB-bit tie field above a PB-bit payload field.  The tie field
// is the tie index for negative scores and (2^TB - 1) - tie index otherwise, so the lower index gives the larger key;
// the payload (a function of the candidate, below the tie field) never decides an order.  A zero score's key is
// built the same way and then given the smallest normal exponent (fix_zero_key): it sorts between every negative
// and every positive score, in tie order, and no key is a denormal.
template <int TB, int PB>
__device__ __forceinline__ double sel_key(float s, int tie, int payload) {
  static_assert(TB + PB <= 29, "key fields exceed the free mantissa bits");
  // (2^TB - 1) - tie == tie ^ (2^TB - 1): flip the tie field unless the sign bit is set
  const uint32_t flip = ~static_cast<uint32_t>(static_cast<int32_t>(__float_as_uint(s)) >> 31) &
                        (((1u << TB) - 1u) << PB);
  const uint32_t low = ((static_cast<uint32_t>(tie) << PB) | static_cast<uint32_t>(payload)) ^ flip;
  return __longlong_as_double(__double_as_longlong(static_cast<double>(s)) | low);
}
// A +0 score's key has a zero high word (exponent field 0); every other key's high word is at least 0x36A00000
// (positive) or has the sign bit set, so an unsigned max with 0x00100000 moves exactly the zero keys to exponent 1.
__device__ __forceinline__ double fix_zero_key(double k) {
  const unsigned long long b = __double_as_longlong(k);
  const uint32_t hi = max(static_cast<uint32_t>(b >> 32), 0x00100000u);
  return __longlong_as_double((static_cast<unsigned long long>(hi) << 32) | (b & 0xffffffffull));
}
// the most negative finite double: below every real key, and no NaN whatever the low word
__device__ __forceinline__ double lowest_key(double k) {
  return __longlong_as_double((0xffefffffull << 32) | (__double_as_longlong(k) & 0xffffffffull));
}
// the score and the payload of a key
template <int PB>
__device__ __forceinline__ void sel_decode(double k, float& s, int& payload) {
  const unsigned long long bits = __double_as_longlong(k);
  s = ((bits >> 52) & 0x7ffu) <= 1u ? 0.f : static_cast<float>(__longlong_as_double(bits & ~0x1fffffffull));
  payload = static_cast<int>(bits & ((1ull << PB) - 1));
}

// compare-exchange networks on f64 keys, descending
__device__ __forceinline__ void ce_desc(double& a, double& b) {
  const double x = a, y = b;
  a = fmax(x, y);
  b = fmin(x, y);
}
// 8 keys with the 19-comparator network of depth 6
__device__ __forceinline__ void sort8_desc(double* v) {
  ce_desc(v[0], v[2]); ce_desc(v[1], v[3]); ce_desc(v[4], v[6]); ce_desc(v[5], v[7]);
  ce_desc(v[0], v[4]); ce_desc(v[1], v[5]); ce_desc(v[2], v[6]); ce_desc(v[3], v[7]);
  ce_desc(v[0], v[1]); ce_desc(v[2], v[3]); ce_desc(v[4], v[5]); ce_desc(v[6], v[7]);
  ce_desc(v[2], v[4]); ce_desc(v[3], v[5]);
  ce_desc(v[1], v[4]); ce_desc(v[3], v[6]);
  ce_desc(v[1], v[2]); ce_desc(v[3], v[4]); ce_desc(v[5], v[6]);
}
template <int N>
__device__ __forceinline__ void bitonic_sort_desc(double* v) {
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const double x = v[i], y = v[l];
          if ((i & k) == 0) {
            v[i] = fmax(x, y);
            v[l] = fmin(x, y);
          } else {
            v[i] = fmin(x, y);
            v[l] = fmax(x, y);
          }
        }
      }
    }
  }
}
// a, b sorted descending -> a = the N largest of both, sorted descending
template <int N>
__device__ __forceinline__ void merge_top_desc(double* a, const double* b) {
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = fmax(a[i], b[N - 1 - i]);   // bitonic
#pragma unroll
  for (int j = N >> 1; j > 0; j >>= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int l = i ^ j;
      if (l > i) {
        const double x = a[i], y = a[l];
        a[i] = fmax(x, y);
        a[l] = fmin(x, y);
      }
    }
  }
}
// the K largest of c[0..N) (N a multiple of K) -> c[0..K), sorted descending
template <int K, int N>
__device__ __forceinline__ void top_k_desc(double (&c)[N]) {
#pragma unroll
  for (int g = 0; g < N / K; ++g) {
    if constexpr (K == 8) sort8_desc(c + g * K);
    else bitonic_sort_desc<K>(c + g * K);
  }
#pragma unroll
  for (int g = 1; g < N / K; ++g) merge_top_desc<K>(c, c + g * K);
}

// n values of type InT from p into floats: 16-byte (or, for 4 bfloat16, 8-byte) loads when p is aligned to them,
// element loads otherwise
template <int n, typename InT>
__device__ __forceinline__ void load_vals(const InT* p, float (&out)[n]) {
  constexpr int kBytes = n * static_cast<int>(sizeof(InT));
  if constexpr (kBytes % 16 == 0) {
    if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
#pragma unroll
      for (int q = 0; q < kBytes / 16; ++q) {
        const uint4 u = reinterpret_cast<const uint4*>(p)[q];
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (sizeof(InT) == 2) {
            out[8 * q + 2 * e] = __uint_as_float(wd[e] << 16);
            out[8 * q + 2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
          } else {
            out[4 * q + e] = __uint_as_float(wd[e]);
          }
        }
      }
      return;
    }
  }
  if constexpr (kBytes == 8 && sizeof(InT) == 2) {
    if ((reinterpret_cast<uintptr_t>(p) & 7u) == 0) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      out[0] = __uint_as_float(u.x << 16);
      out[1] = __uint_as_float(u.x & 0xffff0000u);
      out[2] = __uint_as_float(u.y << 16);
      out[3] = __uint_as_float(u.y & 0xffff0000u);
      return;
    }
  }
#pragma unroll
  for (int s = 0; s < n; ++s) out[s] = to_f32(p[s]);
}

// n floats to n values of type OutT at p: 16-byte stores when p is 16-byte aligned, element stores otherwise
template <int n, typename OutT>
__device__ __forceinline__ void store_vals(OutT* p, const float (&v)[n]) {
  constexpr int kBytes = n * static_cast<int>(sizeof(OutT));
  if constexpr (kBytes % 16 == 0) {
    if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
#pragma unroll
      for (int q = 0; q < kBytes / 16; ++q) {
        uint32_t wd[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (sizeof(OutT) == 2) {
            wd[e] = static_cast<uint32_t>(from_f32<bf16_t>(v[8 * q + 2 * e]).bits) |
                    (static_cast<uint32_t>(from_f32<bf16_t>(v[8 * q + 2 * e + 1]).bits) << 16);
          } else {
            wd[e] = __float_as_uint(v[4 * q + e]);
          }
        }
        reinterpret_cast<uint4*>(p)[q] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
      return;
    }
  }
  if constexpr (kBytes == 8 && sizeof(OutT) == 2) {
    if ((reinterpret_cast<uintptr_t>(p) & 7u) == 0) {
      *reinterpret_cast<uint2*>(p) =
          make_uint2(static_cast<uint32_t>(from_f32<bf16_t>(v[0]).bits) | (static_cast<uint32_t>(from_f32<bf16_t>(v[1]).bits) << 16),
                     static_cast<uint32_t>(from_f32<bf16_t>(v[2]).bits) | (static_cast<uint32_t>(from_f32<bf16_t>(v[3]).bits) << 16));
      return;
    }
  }
#pragma unroll
  for (int s = 0; s < n; ++s) p[s] = from_f32<OutT>(v[s]);
}

// number of grid pairs (a, b), a, b < CAP, with (a+1)(b+1) <= CAP: the candidates of the top-CAP combine
__host__ __device__ constexpr int n_pairs(int cap) {
  int n = 0;
  for (int a = 0; a < cap; ++a)
    for (int b = 0; b < cap; ++b)
      if ((a + 1) * (b + 1) <= cap) ++n;
  return n;
}

// Offset selection keys of the matrix-core addressing (address_wave).  A cosine score s (|s| < 2) is keyed by the
// double s + 6: one binade [4, 8) with a grid of 2^-50.  The low 19 mantissa bits are cleared (scores closer than
// 2^-31 then tie) and hold fields that order equal values (larger field first) and name the candidate:
//   half key        bits FS..FS+4: 31 - i (sub-key i); FS = 6 for the first half, 1 for the second
//   ranked half key plus bits 15..18 (first half) or 11..14 (second): 15 - rank within the half
// Every field bit is even, so the sum of a ranked first-half key and a ranked second-half key is exact (a multiple
// of 2^-49 in [8, 16)): its value part is the sum of the two truncated scores + 12, and its low 18 bits are
//   14..17: 15 - ra, 10..13: 15 - rb, 5..9: 31 - i1, 0..4: 31 - i2
// so plain double order is (mean score descending, then (ra, rb) ascending), and the field names the slot.  Keys
// of invalid candidates get the high word 0x00100000: a normal double below every real key.
// With 64 sub-keys per half (NS = 64) the index fields are 6 bits wide and every field sits one place higher per
// extra index bit: a half key clears its low 21 bits (scores closer than 2^-29 tie), half 2's index is at bits 1..6
// and half 1's at 7..12, the ranks at 13..16 and 17..20; a grid key's low 20 bits hold 16..19: 15 - ra,
// 12..15: 15 - rb, 6..11: 63 - i1, 0..5: 63 - i2.  KeyLayout<NS> gives the positions for either.
template <int NS>
struct KeyLayout {
  static_assert(NS == 32 || NS == 64, "32 or 64 sub-keys per half");
  static constexpr int IB = NS == 64 ? 6 : 5;       // index field width
  static constexpr int FS2 = 1, FS1 = 1 + IB;       // index fields of a half key (second half, first half)
  static constexpr int RS2 = 1 + 2 * IB, RS1 = 5 + 2 * IB;   // rank fields of a ranked half key
  static constexpr uint32_t kClear = ~((1u << (2 * IB + 9)) - 1u);   // the value part of a half key's low word
  static constexpr unsigned long long kGridFields = (1ull << (2 * IB + 8)) - 1ull;
};
template <int FS, int NS = 32>
__device__ __forceinline__ double half_key(float a, double inv, int i) {   // s = a * inv
  const unsigned long long b = __double_as_longlong(fma(static_cast<double>(a), inv, 6.0));
  const uint32_t lo = (static_cast<uint32_t>(b) & KeyLayout<NS>::kClear) | (static_cast<uint32_t>(NS - 1 - i) << FS);
  return __longlong_as_double((b & 0xffffffff00000000ull) | lo);
}
__device__ __forceinline__ double key_or(double k, uint32_t bits) {
  return __longlong_as_double(__double_as_longlong(k) | bits);
}
__device__ __forceinline__ double key_invalid(double k) {
  return __longlong_as_double((0x00100000ull << 32) | (__double_as_longlong(k) & 0xffffffffull));
}
// the mean score of a grid key, to within 2^-32 (2^-30 with 64 sub-keys)
template <int NS = 32>
__device__ __forceinline__ float grid_score(double k) {
  const double v = __longlong_as_double(__double_as_longlong(k) & ~KeyLayout<NS>::kGridFields);
  return static_cast<float>(fma(v, 0.5, -6.0));
}

// merges of sorted (descending) key lists: Batcher's odd-even merge of 2 + 2 and 4 + 4
__device__ __forceinline__ void oe_merge22(double a0, double a1, double b0, double b1, double (&c)[4]) {
  ce_desc(a0, b0);
  ce_desc(a1, b1);
  ce_desc(a1, b0);
  c[0] = a0;
  c[1] = a1;
  c[2] = b0;
  c[3] = b1;
}
__device__ __forceinline__ void oe_merge44(const double (&a)[4], const double (&b)[4], double (&c)[8]) {
  double v[4], w[4];
  oe_merge22(a[0], a[2], b[0], b[2], v);
  oe_merge22(a[1], a[3], b[1], b[3], w);
  c[0] = v[0];
  c[7] = w[3];
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    c[2 * i - 1] = fmax(w[i - 1], v[i]);
    c[2 * i] = fmin(w[i - 1], v[i]);
  }
}
// the 8 largest grid keys, sorted, of the pruned 8 x 8 grid ((ra + 1)(rb + 1) <= 8): its rows and its first column
// are already sorted runs, merged as row 0 | (row 1 | column ra >= 4) | (row 2 | row 3)
__device__ __forceinline__ void grid_top8(const double (&g0)[8], const double (&g1)[4], const double (&g2)[2],
                                          const double (&g3)[2], const double (&gc)[4], double (&out)[8]) {
  double m4[4], m8[8];
  oe_merge22(g2[0], g2[1], g3[0], g3[1], m4);
  oe_merge44(g1, gc, m8);
#pragma unroll
  for (int i = 4; i < 8; ++i) m8[i] = fmax(m8[i], m4[7 - i]);   // top 8 of m8 | m4, bitonic
#pragma unroll
  for (int j = 4; j > 0; j >>= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((i ^ j) > i) ce_desc(m8[i], m8[i ^ j]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = g0[i];
  merge_top_desc<8>(out, m8);
}

// 1 / max(sqrt(ss), 1e-12): hardware reciprocal square root and one Newton step
__device__ __forceinline__ float inv_norm(float ss) {
  const float x = fmaxf(ss, 1e-24f);
  const float y = __builtin_amdgcn_rsqf(x);
  return y * fmaf(-0.5f * x * y, y, 1.5f);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 8 consecutive bfloat16 values at p as raw bits: one 16-byte load when p is 16-byte aligned
__device__ __forceinline__ uint4 load_raw8(const bf16_t* p) {
  if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) return *reinterpret_cast<const uint4*>(p);
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = p[2 * e].bits | (static_cast<uint32_t>(p[2 * e + 1].bits) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// a and b rounded to bfloat16 (nearest even), packed a | b << 16
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// Cosine scores of one half (hf) of the wave's 64 addresses against the head's sub-keys of that half, up to one
// factor per address: lane l, tile t: acc[t][r] * inv[t] = cos(sub-key 8(r/4) + 4(l/32) + r%4, address row
// 32t + l%32), inv[t] = 1 / max(|z + addr_b|, 1e-12) of that row.  Sub-key rows past n_sub score 0.  Rows past
// `rows` are clamped.

// float32 matrix cores: lane l feeds dims (l/32) * HALF/2 ... (l/32) * HALF/2 + HALF/2 - 1 of sub-key row l%32 and
// of both address rows
template <int HALF, typename InT, bool FULL>
__device__ __forceinline__ void half_scores_f32(const AddrGeom& g, int h, int hf, const InT* z0, int64_t zstride,
                                                int rows, floatx16 (&acc)[2], float (&inv)[2], int kofs = 0) {
  constexpr int S = HALF / 2;
  const int l = threadIdx.x & 63;
  const int kb = l >> 5, jl = l & 31;
  const int kr = kofs + jl;   // this lane's sub-key row (kofs: the sub-key tile, 0 or 32)
  float ka[S], zb[2][S], ab[S];
  load_vals<S, float>(g.keys[hf] + (static_cast<int64_t>(h) * g.n_sub + min(kr, g.n_sub - 1)) * HALF + kb * S, ka);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = min(32 * t + jl, rows - 1);
    load_vals<S, InT>(z0 + row * zstride + static_cast<int64_t>(h) * 2 * HALF + hf * HALF + kb * S, zb[t]);
  }
  if (g.addr_b) {
    load_vals<S, float>(g.addr_b + h * 2 * HALF + hf * HALF + kb * S, ab);
  } else {
#pragma unroll
    for (int s = 0; s < S; ++s) ab[s] = 0.f;
  }
  {   // unit-normalised sub-key row
    float ks = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) ks = fmaf(ka[s], ka[s], ks);
    const auto kp = __builtin_amdgcn_permlane32_swap(__float_as_uint(ks), __float_as_uint(ks), false, false);
    const float kinv = (FULL || kr < g.n_sub) ? inv_norm(__uint_as_float(kp[0]) + __uint_as_float(kp[1])) : 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) ka[s] *= kinv;
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      zb[t][s] += ab[s];
      ss = fmaf(zb[t][s], zb[t][s], ss);
    }
    const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    inv[t] = inv_norm(__uint_as_float(pr[0]) + __uint_as_float(pr[1]));   // same order in both lane halves
    acc[t] = floatx16{};
#pragma unroll
    for (int s = 0; s < S; ++s) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[s], zb[t][s], acc[t], 0, 0, 0);
  }
}

// bfloat16 matrix cores (bfloat16 addresses, HALF a multiple of 8): each unit sub-key is split into three bfloat16
// terms k = k0 + k1 + k2 + r (k0 the nearest bfloat16 to k, k1 to k - k0, k2 to k - k0 - k1; |r| <= 2^-27 |k|), the
// address values are bfloat16 already, so every product is exact in the float32 accumulation.  The address bias
// enters through the accumulator's start value c_i = k_i . addr_b (one float32 matrix step: c_i x 1) and through
// inv.  Lane l feeds dims 16q + 8(l/32) + e (e < 8) of sub-key row l%32 and of both address rows (HALF = 8: lanes
// 32..63 feed zeros).  Head h's address columns start at column zcol of a row (h * 2 HALF when zcol < 0).
// The layout of the prepared sub-key pieces of the bfloat16 scoring (HALF: half width, NSP: sub-key rows per half
// rounded up to 32): per (head, half, sub-key row, lane half) the 3 Q x 4 words of the three bfloat16 terms that
// lane feeds the matrix cores, then per (head, half, sub-key row) the float32 c = k . addr_b.
template <int HALF>
struct KeyPieces {
  static constexpr int Q = (HALF + 15) / 16;
  static constexpr int kWords = 3 * Q * 4;   // per lane
  __host__ __device__ static constexpr int64_t term_words(int H, int nsp) { return static_cast<int64_t>(H) * 2 * nsp * 2 * kWords; }
  __host__ __device__ static constexpr int64_t bytes(int H, int nsp) { return 4 * (term_words(H, nsp) + static_cast<int64_t>(H) * 2 * nsp); }
};
__host__ __device__ constexpr int key_piece_rows(int n_sub) { return (n_sub + 31) / 32 * 32; }

// The lane's part of the bfloat16 scoring of half hf against sub-key tile kofs (lane l: sub-key row kofs + l % 32,
// dims 16 q + 8 (l / 32) + e): the three bfloat16 terms of its unit sub-key piece (k = k0 + k1 + k2 + r, each term
// the nearest bfloat16 to what is left), c = k . addr_b over the whole row, and its address-bias piece.
template <int HALF>
struct SubKeyPiece {
  static constexpr int Q = (HALF + 15) / 16;
  uint32_t kt[3][Q][4];   // the terms, packed in pairs
  float c;
  float ab[Q][8];
};
// computes the lane's piece from the sub-keys (sub-key rows past n_sub: zero terms; all 64 lanes take part), or
// loads it when g.kpieces holds the prepared pieces (the same values: sdm_rt_prepare_key_pieces computes them here)
template <int HALF>
__device__ __forceinline__ void load_sub_key_piece(const AddrGeom& g, int h, int hf, int kofs, SubKeyPiece<HALF>& kp) {
  constexpr int Q = SubKeyPiece<HALF>::Q;
  const int l = threadIdx.x & 63;
  const int kb = l >> 5, jl = l & 31;
  const bool has = HALF >= 16 || kb == 0;
  const int d0 = hf * HALF + 8 * kb;
  const int kr = kofs + jl;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (g.addr_b && has) {
      load_vals<8, float>(g.addr_b + h * 2 * HALF + d0 + 16 * q, kp.ab[q]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) kp.ab[q][e] = 0.f;
    }
  }
  if (g.kpieces) {
    const int nsp = key_piece_rows(g.n_sub);
    const int64_t row = (static_cast<int64_t>(h) * 2 + hf) * nsp + min(kr, nsp - 1);
    const uint4* src = reinterpret_cast<const uint4*>(g.kpieces + (row * 2 + kb) * KeyPieces<HALF>::kWords);
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const uint4 v = src[t * Q + q];
        kp.kt[t][q][0] = v.x;
        kp.kt[t][q][1] = v.y;
        kp.kt[t][q][2] = v.z;
        kp.kt[t][q][3] = v.w;
      }
    kp.c = reinterpret_cast<const float*>(g.kpieces + KeyPieces<HALF>::term_words(g.H, nsp))[row];
    return;
  }
  float ka[Q][8];
  const float* krow = g.keys[hf] + (static_cast<int64_t>(h) * g.n_sub + min(kr, g.n_sub - 1)) * HALF + 8 * kb;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (has) {
      load_vals<8, float>(krow + 16 * q, ka[q]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) ka[q][e] = 0.f;
    }
  }
  {   // unit-normalised sub-key row (rows past n_sub: zero)
    float ks = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) ks = fmaf(ka[q][e], ka[q][e], ks);
    const auto kpv = __builtin_amdgcn_permlane32_swap(__float_as_uint(ks), __float_as_uint(ks), false, false);
    const float kinv = kr < g.n_sub ? inv_norm(__uint_as_float(kpv[0]) + __uint_as_float(kpv[1])) : 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) ka[q][e] *= kinv;
  }
  {   // c = k . addr_b (the address bias enters the scores through the accumulator's start value)
    float cp = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) cp = fmaf(ka[q][e], kp.ab[q][e], cp);
    const auto cw = __builtin_amdgcn_permlane32_swap(__float_as_uint(cp), __float_as_uint(cp), false, false);
    kp.c = __uint_as_float(cw[0]) + __uint_as_float(cw[1]);
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float x0 = ka[q][2 * e2], x1 = ka[q][2 * e2 + 1];
#pragma unroll
      for (int term = 0; term < 3; ++term) {
        const uint32_t pk = pack_bf16(x0, x1);
        kp.kt[term][q][e2] = pk;
        x0 -= __uint_as_float(pk << 16);   // exact
        x1 -= __uint_as_float(pk & 0xffff0000u);
      }
    }
  }
}

// bfloat16 matrix cores (bfloat16 addresses, HALF a multiple of 8): each unit sub-key is split into three bfloat16
// terms k = k0 + k1 + k2 + r (k0 the nearest bfloat16 to k, k1 to k - k0, k2 to k - k0 - k1; |r| <= 2^-27 |k|), the
// address values are bfloat16 already, so every product is exact in the float32 accumulation.  The address bias
// enters through the accumulator's start value c_i = k_i . addr_b (one float32 matrix step: c_i x 1) and through
// inv.  Lane l feeds dims 16q + 8(l/32) + e (e < 8) of sub-key row l%32 and of both address rows (HALF = 8: lanes
// 32..63 feed zeros).  Head h's address columns start at column zcol of a row (h * 2 HALF when zcol < 0).  kp: the
// lane's sub-key piece (load_sub_key_piece with the same h, hf and sub-key tile).  Sub-key rows past n_sub score 0.
template <int HALF, bool FULL>
__device__ __forceinline__ void half_scores_bf16_with(const AddrGeom& g, int h, int hf, const bf16_t* z0,
                                                      int64_t zstride, int rows, floatx16 (&acc)[2], float (&inv)[2],
                                                      int zcol, const SubKeyPiece<HALF>& kp) {
  static_assert(HALF % 8 == 0, "bfloat16 scoring feeds 8 dims per lane");
  constexpr int Q = (HALF + 15) / 16;
  const int l = threadIdx.x & 63;
  const int kb = l >> 5, jl = l & 31;
  const bool has = HALF >= 16 || kb == 0;
  const int d0 = hf * HALF + 8 * kb;   // first dim of the address this lane feeds
  uint4 zr[2][Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = min(32 * t + jl, rows - 1);
      zr[t][q] = has ? load_raw8(z0 + row * zstride + (zcol >= 0 ? zcol : static_cast<int64_t>(h) * 2 * HALF) + d0 +
                                 16 * q)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  floatx16 init = {};
  if (g.addr_b) init = __builtin_amdgcn_mfma_f32_32x32x2f32(kb == 0 ? kp.c : 0.f, kb == 0 ? 1.f : 0.f, init, 0, 0, 0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const uint32_t wd[4] = {zr[t][q].x, zr[t][q].y, zr[t][q].z, zr[t][q].w};
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float v0 = __uint_as_float(wd[e2] << 16) + kp.ab[q][2 * e2];
        const float v1 = __uint_as_float(wd[e2] & 0xffff0000u) + kp.ab[q][2 * e2 + 1];
        ss = fmaf(v0, v0, ss);
        ss = fmaf(v1, v1, ss);
      }
    }
    const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    inv[t] = inv_norm(__uint_as_float(pr[0]) + __uint_as_float(pr[1]));
    acc[t] = init;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
#pragma unroll
      for (int term = 2; term >= 0; --term) {
        const uint4 kq = make_uint4(kp.kt[term][q][0], kp.kt[term][q][1], kp.kt[term][q][2], kp.kt[term][q][3]);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kq),
                                                         __builtin_bit_cast(bf16x8, zr[t][q]), acc[t], 0, 0, 0);
      }
    }
  }
}

// half_scores_bf16_with on the lane's sub-key piece of tile kofs, loaded here after the address loads issue
template <int HALF, bool FULL>
__device__ __forceinline__ void half_scores_bf16(const AddrGeom& g, int h, int hf, const bf16_t* z0, int64_t zstride,
                                                 int rows, floatx16 (&acc)[2], float (&inv)[2], int kofs = 0,
                                                 int zcol = -1) {
  SubKeyPiece<HALF> kp;
  load_sub_key_piece<HALF>(g, h, hf, kofs, kp);
  half_scores_bf16_with<HALF, FULL>(g, h, hf, z0, zstride, rows, acc, inv, zcol, kp);
}

// The CAP best offset keys (descending) of half hf of the wave's 64 addresses over sub-key tile `tile` (sub-keys
// 32 tile ... 32 tile + 31), lane l holding address row l of z0 (rows past `rows` are clamped).  The tile's 32 keys
// are taken CAP at a time (sub-keys 2 GR grp ... 2 GR grp + 2 GR - 1), each group sorted and merged into the best:
// the same top CAP as one 32-key selection (the keys are distinct), with a quarter of the keys live at once.
// (best is merged into when merge_into is set: the keys of an earlier tile of the same half.)
template <int HALF, int CAP, typename InT, bool FULL, int NS>
__device__ __forceinline__ void tile_best(const AddrGeom& g, int h, const InT* z0, int64_t zstride, int rows, int hf,
                                          int tile, bool merge_into, double (&best)[CAP]) {
  using KL = KeyLayout<NS>;
  const int kb = (threadIdx.x & 63) >> 5;
  floatx16 acc[2];
  float inv[2];
  if constexpr (sizeof(InT) == 2) half_scores_bf16<HALF, FULL>(g, h, hf, z0, zstride, rows, acc, inv, 32 * tile);
  else half_scores_f32<HALF, InT, FULL>(g, h, hf, z0, zstride, rows, acc, inv, 32 * tile);
  // after the swap below lane l holds every score of address row l
  const double dinv = static_cast<double>(kb ? inv[1] : inv[0]);
  constexpr int GR = CAP / 2;   // score registers per group
#pragma unroll
  for (int grp = 0; grp < 16 / GR; ++grp) {
    double c[CAP];
#pragma unroll
    for (int rr = 0; rr < GR; ++rr) {
      const int r = GR * grp + rr;
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0][r]), __float_as_uint(acc[1][r]),
                                                       false, false);
      const int i0 = 32 * tile + 8 * (r / 4) + (r % 4);
      if (hf == 0) {
        c[rr] = half_key<KL::FS1, NS>(__uint_as_float(sw[0]), dinv, i0);
        c[GR + rr] = half_key<KL::FS1, NS>(__uint_as_float(sw[1]), dinv, i0 + 4);
      } else {
        c[rr] = half_key<KL::FS2, NS>(__uint_as_float(sw[0]), dinv, i0);
        c[GR + rr] = half_key<KL::FS2, NS>(__uint_as_float(sw[1]), dinv, i0 + 4);
      }
      if (!FULL) {   // sub-keys past n_sub are never picked
        if (i0 >= g.n_sub) c[rr] = key_invalid(c[rr]);
        if (i0 + 4 >= g.n_sub) c[GR + rr] = key_invalid(c[GR + rr]);
      }
    }
    if constexpr (CAP == 8) sort8_desc(c);
    else bitonic_sort_desc<CAP>(c);
    if (!merge_into && grp == 0) {
#pragma unroll
      for (int r = 0; r < CAP; ++r) best[r] = c[r];
    } else {
      merge_top_desc<CAP>(best, c);
    }
  }
}

// the half's best keys tagged with their rank within the half (the grid key's rank fields)
template <int CAP, int NS>
__device__ __forceinline__ void rank_half(int hf, const double (&best)[CAP], double (&hk)[CAP]) {
  using KL = KeyLayout<NS>;
#pragma unroll
  for (int r = 0; r < CAP; ++r) hk[r] = key_or(best[r], static_cast<uint32_t>(15 - r) << (hf == 0 ? KL::RS1 : KL::RS2));
}

// The picks of one address from its two ranked halves: the combine over the dominance-pruned grid (see
// address_one), the slots, the mean scores and the softmax weights (times the gate).
template <int CAP, bool FULL, int NS>
__device__ __forceinline__ void grid_pick(const AddrGeom& g, int h, const double (&hk0)[CAP], const double (&hk1)[CAP],
                                          float gate, int (&slot)[CAP], float (&w)[CAP], float (&score)[CAP]) {
  using KL = KeyLayout<NS>;
  auto cell = [&](int ra, int rb) {
    const double k = hk0[ra] + hk1[rb];
    if (FULL) return k;
    return (ra < g.c1 && rb < g.c1 && (ra + 1) * (rb + 1) <= g.kk) ? k : key_invalid(k);
  };
  double pc[CAP];
  if constexpr (CAP == 8) {
    double g0[8], g1[4], g2[2], g3[2], gc[4];
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) g0[rb] = cell(0, rb);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) g1[rb] = cell(1, rb);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      g2[rb] = cell(2, rb);
      g3[rb] = cell(3, rb);
    }
#pragma unroll
    for (int ra = 4; ra < 8; ++ra) gc[ra - 4] = cell(ra, 0);
    grid_top8(g0, g1, g2, g3, gc, pc);
  } else {
    constexpr int NP = n_pairs(CAP);
    constexpr int NPAD = (NP + CAP - 1) / CAP * CAP;
    double all[NPAD];
    int n = 0;
#pragma unroll
    for (int ra = 0; ra < CAP; ++ra) {
#pragma unroll
      for (int rb = 0; rb < CAP; ++rb) {
        if ((ra + 1) * (rb + 1) <= CAP) all[n++] = cell(ra, rb);
      }
    }
#pragma unroll
    for (int i = NP; i < NPAD; ++i) all[i] = -INFINITY;
    top_k_desc<CAP, NPAD>(all);
#pragma unroll
    for (int p = 0; p < CAP; ++p) pc[p] = all[p];
  }
  float cv[CAP];
  int si[CAP];
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    cv[p] = grid_score<NS>(pc[p]);
    const uint32_t f = static_cast<uint32_t>(__double_as_longlong(pc[p]));
    if (FULL) {   // (NS - 1 - i1) * NS + (NS - 1 - i2) = NS^2 - 1 - slot
      si[p] = NS * NS - 1 - static_cast<int>(f & static_cast<uint32_t>(NS * NS - 1));
    } else {
      const int i1 = NS - 1 - static_cast<int>((f >> KL::IB) & static_cast<uint32_t>(NS - 1));
      const int i2 = NS - 1 - static_cast<int>(f & static_cast<uint32_t>(NS - 1));
      si[p] = min(i1 * g.n_sub + i2, g.n_sub * g.n_sub - 1);
    }
  }
  const float scale = expf(g.log_scale[h]);
  float e[CAP];
  const float x0 = cv[0] * scale;
  float sum = 0.f;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    e[p] = (FULL || p < g.kk) ? expf(cv[p] * scale - x0) : 0.f;
    sum += e[p];
  }
  const float wscale = gate / sum;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    const bool live = FULL || p < g.kk;
    slot[p] = live ? si[p] : 0;
    w[p] = live ? e[p] * wscale : 0.f;
    score[p] = live ? cv[p] : 0.f;
  }
}

// Picks of address l (lane l) of the 64 rows z0[r * zstride + h * 2 * HALF ...], r < rows (rows past `rows` are
// clamped; their lanes' outputs are unspecified): the selection of address_one on offset keys, scores within 2^-31
// of float rounding (2^-29 with NS = 64).  NS: 32 sub-keys per half (n_sub <= 32) or 64 (n_sub <= 64: two sub-key
// tiles scored in turn, each tile's CAP best merged into the half's).  FULL: n_sub = NS and c1 = kk = CAP (no
// candidate is masked).  All 64 lanes of the wave must call it.
template <int HALF, int CAP, typename InT, bool FULL, int NS = 32>
__device__ __forceinline__ void address_wave(const AddrGeom& g, int h, const InT* z0, int64_t zstride, int rows,
                                             float gate, int (&slot)[CAP], float (&w)[CAP], float (&score)[CAP]) {
  double hk[2][CAP];   // ranked half keys
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    double best[CAP];   // the half's CAP best keys so far, descending
#pragma unroll
    for (int tile = 0; tile < NS / 32; ++tile)
      tile_best<HALF, CAP, InT, FULL, NS>(g, h, z0, zstride, rows, hf, tile, tile > 0, best);
    rank_half<CAP, NS>(hf, best, hk[hf]);
  }
  grid_pick<CAP, FULL, NS>(g, h, hk[0], hk[1], gate, slot, w, score);
}

// the value of lane (lane ^ j) of the wave (j < 64 a power of two): DPP within rows of 16 lanes (quad_perm for 1
// and 2, row_shl/row_shr by 4, row_ror by 8), lane permutes across rows
__device__ __forceinline__ int xor_lanes32(int v, int j, int lane) {
  if (j == 1) return __builtin_amdgcn_update_dpp(v, v, 0xb1, 0xf, 0xf, false);    // quad_perm [1,0,3,2]
  if (j == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4e, 0xf, 0xf, false);    // quad_perm [2,3,0,1]
  if (j == 8) return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);   // row_ror:8
  if (j == 4) {   // lanes with bit 2 clear read lane + 4 (row_shl:4), the others lane - 4 (row_shr:4)
    const int u = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xf, 0xf, false);
    const int d = __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false);
    return (lane & 4) ? d : u;
  }
  return __shfl_xor(v, j);
}

// Descending bitonic sort of one selection key per lane over aligned groups of N lanes (N a power of two <= 64):
// lane i of a group ends with the group's i-th largest key.  The keys are non-negative doubles (their order is the
// unsigned order of their bits) and are compared as 64-bit integers.  Every lane of the wave takes part.
// K0 > 2: the steps before the merge of K0-lane blocks are skipped; every aligned block of K0 lanes must then hold a
// bitonic sequence (non-increasing, then non-decreasing, or the reverse).
template <int N, int K0 = 2>
__device__ __forceinline__ unsigned long long sort_lanes_desc(unsigned long long x, int lane) {
  const int idx = lane & (N - 1);
#pragma unroll
  for (int k = K0; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int ylo = xor_lanes32(static_cast<int>(x), j, lane);
      const int yhi = xor_lanes32(static_cast<int>(x >> 32), j, lane);
      const unsigned long long y = (static_cast<unsigned long long>(static_cast<uint32_t>(yhi)) << 32) |
                                   static_cast<uint32_t>(ylo);
      const bool keep_max = ((idx & j) == 0) == ((idx & k) == 0);
      x = ((x > y) == keep_max) ? x : y;
    }
  }
  return x;
}

// The grid pair (ra, rb) of a lane in the layout of sorted runs select_lanes uses for a full grid (ra = -1: none).
// CAP = 8 (20 pairs, lanes 0..31): lanes 0-7 row 0 (rb 0..7); 8-14 column 0 (ra 1..7); 16-18 row 1 (rb 1..3);
// 22-23 column 1 reversed (ra 3, 2).  CAP = 16 (50 pairs, lanes 0..63): 0-15 row 0; 16-30 column 0 (ra 1..15),
// 31 (3, 3); 32-38 row 1 (rb 1..7); 42-47 column 1 reversed (ra 7..2); 48-50 row 2 (rb 2..4); 62-63 column 2
// reversed (ra 4, 3).  Each run descends (rows and columns of the grid do), so every block of CAP lanes is one
// descending run, then an ascending one (or none), with key 0 between: a bitonic sequence.
template <int CAP>
__device__ __forceinline__ void grid_run_pair(int lane, int& ra, int& rb) {
  static_assert(CAP == 8 || CAP == 16, "run layouts for 8 and 16 picks");
  ra = -1;
  rb = 0;
  if constexpr (CAP == 8) {
    if (lane < 8) { ra = 0; rb = lane; }
    else if (lane < 15) { ra = lane - 7; rb = 0; }
    else if (lane >= 16 && lane < 19) { ra = 1; rb = lane - 15; }
    else if (lane == 22 || lane == 23) { ra = 25 - lane; rb = 1; }
  } else {
    if (lane < 16) { ra = 0; rb = lane; }
    else if (lane < 31) { ra = lane - 15; rb = 0; }
    else if (lane == 31) { ra = 3; rb = 3; }
    else if (lane < 39) { ra = 1; rb = lane - 31; }
    else if (lane >= 42 && lane < 48) { ra = 49 - lane; rb = 1; }
    else if (lane >= 48 && lane < 51) { ra = 2; rb = lane - 46; }
    else if (lane >= 62) { ra = 66 - lane; rb = 2; }
  }
}

// sort_lanes_desc of two independent keys per lane at once (each exchange step moves both), so that the two chains
// of dependent steps overlap
template <int N>
__device__ __forceinline__ void sort_lanes_desc2(unsigned long long& x0, unsigned long long& x1, int lane) {
  const int idx = lane & (N - 1);
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int a_lo = xor_lanes32(static_cast<int>(x0), j, lane);
      const int a_hi = xor_lanes32(static_cast<int>(x0 >> 32), j, lane);
      const int b_lo = xor_lanes32(static_cast<int>(x1), j, lane);
      const int b_hi = xor_lanes32(static_cast<int>(x1 >> 32), j, lane);
      const unsigned long long y0 = (static_cast<unsigned long long>(static_cast<uint32_t>(a_hi)) << 32) |
                                    static_cast<uint32_t>(a_lo);
      const unsigned long long y1 = (static_cast<unsigned long long>(static_cast<uint32_t>(b_hi)) << 32) |
                                    static_cast<uint32_t>(b_lo);
      const bool keep_max = ((idx & j) == 0) == ((idx & k) == 0);
      x0 = ((x0 > y0) == keep_max) ? x0 : y0;
      x1 = ((x1 > y1) == keep_max) ? x1 : y1;
    }
  }
}

// The picks of one address by a whole wave: address_wave's selection (the same keys, so the same picks, order,
// weights and scores) with the candidates spread over the lanes instead of sorted per lane.  sc: the NS raw sub-key
// scores of each half ([2][NS], as half_scores leaves them: score * inv = cosine), inv: the two halves' factors.
// NS = 32: lanes 32 hf + i key sub-key i of half hf and each half sorts across its 32 lanes; NS = 64: lane i keys
// sub-key i of each half, both sorted across the wave together.  Lane x < n_pairs(CAP) then keys grid pair x of the
// dominance-pruned grid (address_one) and the 64 lanes sort.  Lane p < CAP returns pick p.
template <int CAP, bool FULL, int NS = 32>
__device__ __forceinline__ void select_lanes(const AddrGeom& g, float log_scale, const float* sc, const float* inv,
                                             float gate, int& slot, float& w, float& score) {
  static_assert(NS == 32 || NS == 64, "32 or 64 sub-keys per half");
  const int lane = threadIdx.x & 63;
  using KL = KeyLayout<NS>;
  auto sort64 = [&](double v, auto n) {
    return __longlong_as_double(static_cast<long long>(
        sort_lanes_desc<decltype(n)::value>(static_cast<unsigned long long>(__double_as_longlong(v)), lane)));
  };
  double hk0, hk1;   // lane r < 16: the rank-r key of half 0 and of half 1, ranked
  if constexpr (NS == 32) {
    const int hf = lane >> 5, i = lane & 31;
    double c = hf == 0 ? half_key<KL::FS1>(sc[i], static_cast<double>(inv[0]), i)
                       : half_key<KL::FS2>(sc[32 + i], static_cast<double>(inv[1]), i);
    if (!FULL && i >= g.n_sub) c = key_invalid(c);   // sub-keys past n_sub are never picked
    c = sort64(c, std::integral_constant<int, 32>{});
    const double hk = i < 16 ? key_or(c, static_cast<uint32_t>(15 - i) << (hf == 0 ? KL::RS1 : KL::RS2)) : c;
    hk0 = hk;
    hk1 = __shfl(hk, (lane & 31) + 32);
  } else {
    double c0 = half_key<KL::FS1, NS>(sc[lane], static_cast<double>(inv[0]), lane);
    double c1 = half_key<KL::FS2, NS>(sc[NS + lane], static_cast<double>(inv[1]), lane);
    if (!FULL && lane >= g.n_sub) {
      c0 = key_invalid(c0);
      c1 = key_invalid(c1);
    }
    unsigned long long u0 = static_cast<unsigned long long>(__double_as_longlong(c0));
    unsigned long long u1 = static_cast<unsigned long long>(__double_as_longlong(c1));
    sort_lanes_desc2<64>(u0, u1, lane);   // both halves at once
    c0 = __longlong_as_double(static_cast<long long>(u0));
    c1 = __longlong_as_double(static_cast<long long>(u1));
    hk0 = lane < 16 ? key_or(c0, static_cast<uint32_t>(15 - lane) << KL::RS1) : c0;
    hk1 = lane < 16 ? key_or(c1, static_cast<uint32_t>(15 - lane) << KL::RS2) : c1;
  }
  // grid pair of this lane: pairs (ra, rb) with (ra + 1)(rb + 1) <= CAP
  constexpr int kGridLanes = n_pairs(CAP) <= 32 ? 32 : 64;
  int ra = -1, rb = 0;
  if constexpr (FULL && (CAP == 8 || CAP == 16)) {
    // laid out as sorted runs (the grid's rows and columns descend: both halves' keys are sorted), two per aligned
    // block of CAP lanes, the second reversed, so that every block is a bitonic sequence and the sort can start at
    // its merge of CAP-lane blocks: CAP = 8: row 0 | column 0 below it | row 1 right of column 0 and, reversed,
    // column 1 below row 1; CAP = 16 likewise with one more pair (row 2, column 2) and cell (3, 3) after column 0
    grid_run_pair<CAP>(lane, ra, rb);
  } else {   // row by row in lanes < n_pairs(CAP)
    int x = lane;
#pragma unroll
    for (int a = 0; a < CAP; ++a) {
      const int n_a = CAP / (a + 1);
      if (ra < 0) {
        if (x < n_a) {
          ra = a;
          rb = x;
        } else {
          x -= n_a;
        }
      }
    }
  }
  const double k0 = __shfl(hk0, max(ra, 0));
  const double k1 = __shfl(hk1, rb);
  double k = k0 + k1;
  if (ra < 0) k = 0.0;   // no candidate: below every key
  else if (!FULL && !(ra < g.c1 && rb < g.c1 && (ra + 1) * (rb + 1) <= g.kk)) k = key_invalid(k);
  if constexpr (FULL && (CAP == 8 || CAP == 16)) {
    k = __longlong_as_double(static_cast<long long>(sort_lanes_desc<kGridLanes, CAP>(
        static_cast<unsigned long long>(__double_as_longlong(k)), lane)));
  } else {
    k = sort64(k, std::integral_constant<int, kGridLanes>{});
  }
  const float cv = grid_score<NS>(k);
  const uint32_t f = static_cast<uint32_t>(__double_as_longlong(k));
  int si;
  if (FULL) {   // (NS - 1 - i1) * NS + (NS - 1 - i2) = NS^2 - 1 - slot
    si = NS * NS - 1 - static_cast<int>(f & static_cast<uint32_t>(NS * NS - 1));
  } else {
    const int i1 = NS - 1 - static_cast<int>((f >> KL::IB) & static_cast<uint32_t>(NS - 1));
    const int i2 = NS - 1 - static_cast<int>(f & static_cast<uint32_t>(NS - 1));
    si = min(i1 * g.n_sub + i2, g.n_sub * g.n_sub - 1);
  }
  const float scale = expf(log_scale);
  const float x0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), 0)) * scale;
  const bool live = lane < CAP && (FULL || lane < g.kk);
  const float e = live ? expf(cv * scale - x0) : 0.f;
  float sum = 0.f;
#pragma unroll
  for (int p = 0; p < CAP; ++p)   // in pick order, as address_wave sums
    sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p));
  const float wscale = gate / sum;
  slot = live ? si : 0;
  w = live ? e * wscale : 0.f;
  score = live ? cv : 0.f;
}

struct AddrArgs {
  AddrGeom g;
  const void* z;              // address rows
  int64_t z_stride;
  const void* gl;             // gate logit rows or nullptr
  int64_t g_stride;
  int B, T, pitch;
  int32_t* slot_out;          // [B][H][T][pitch]
  float* w_out;
  float* s_out;
  // a second address set (gridDim.z = 2, blockIdx.z = 1): its rows, picks, weights and scores (or nullptr); no gate
  const void* z2;
  int64_t z2_stride;
  int32_t* slot_out2;
  float* w_out2;
  float* s_out2;
};

// Head h's sub-keys of both halves, unit-normalised ([2][n_sub][HALF] floats), into LDS: one row per thread.
template <int HALF>
__device__ __forceinline__ void stage_keys(const AddrGeom& g, int h, float* kn, int tid, int nthreads) {
  for (int r = tid; r < 2 * g.n_sub; r += nthreads) {
    const int part = r >= g.n_sub;
    const float* src = g.keys[part] + (static_cast<int64_t>(h) * g.n_sub + (r - part * g.n_sub)) * HALF;
    float ss = 0.f;
    for (int d = 0; d < HALF; ++d) ss = fmaf(src[d], src[d], ss);
    const float n = fmaxf(sqrtf(ss), 1e-12f);
    for (int d = 0; d < HALF; ++d) kn[r * HALF + d] = src[d] / n;
  }
}


// inclusive prefix sum over the 64 lanes of a wave, by DPP: shifts by 1, 2, 4 and 8 lanes within each row of 16
// (lanes shifted in from outside the row read 0), then the last lane of row 0 added to row 1 and of row 2 to row 3
// (row_bcast:15), then lane 31 to rows 2 and 3 (row_bcast:31).  The whole wave must be active.
__device__ __forceinline__ int wave_incl_scan(int v, int) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2 and 3
  return v;
}


// Sum over the 8 consecutive lanes of a group (DPP: swap neighbours, swap pairs, mirror the halves of 8).
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

// 1 / x for normal positive x: hardware reciprocal and one Newton step (within an ulp or so)
__device__ __forceinline__ float fast_rcp(float x) {
  const float y = __builtin_amdgcn_rcpf(x);
  return fmaf(y, fmaf(-x, y, 1.f), y);
}

// Workgroup barrier that orders LDS accesses only: the scan shares nothing else between its threads, so global loads
// issued ahead (the next chunk's plan and values) and global stores (read-outs) need not complete at a barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------------------------------------------
// the chunk plan (written by plan_kernel, executed by scan_kernel; the layout is described in sdm_plan.h)
constexpr int kInline = 6;   // in-chunk read contributions kept in a position record
struct PlanGeom {
  int KP;   // pick pitch: 8 or 16
  // position record: u32 roff[KP], f32 rw[KP], u32 woff[KP], f32 wc[KP], then a 12-word tail
  __host__ __device__ constexpr int off_rw() const { return 4 * KP; }
  __host__ __device__ constexpr int off_woff() const { return 8 * KP; }
  __host__ __device__ constexpr int off_wc() const { return 12 * KP; }
  __host__ __device__ constexpr int off_tail() const { return 16 * KP; }
  __host__ __device__ constexpr int pos_bytes() const { return 16 * KP + 48; }
  __host__ __device__ constexpr int off_var() const { return kChunk * pos_bytes(); }
  // variable part: a 16-byte header, then 8-byte entries: the in-chunk read contributions past the inline ones
  // (at most 63 per position, 2016 per chunk), the records of slots written more than once (at most half the
  // writes) and their later writers (at most the writes)
  __host__ __device__ constexpr int max_entries() const { return kChunk * (kChunk - 1) / 2 + 3 * kChunk * KP / 2; }
  __host__ __device__ constexpr int stride() const { return (off_var() + 16 + 8 * max_entries() + 255) / 256 * 256; }
};

// The pick plan (picks of at most 8, at most 1,024 locations; written by plan_kernel<..., PICK = true>, executed by
// pick_scan_kernel):
//   read records R[8][64], 12 bytes each, record (i, p) for pick i of position p:
//     w0  read slot (bits 0..15; pads and positions past the chunk's end: M) | q (bits 16..21) | n_in (bits 24..31)
//     w1  read weight (0 for pads and when a reset earlier in the chunk hides the carried state)
//     w2  coefficient of the position's in-chunk read contribution number i (q its source position), 0 if i >= n_in
//   write records W[8][64], 12 bytes each:
//     w0  write slot if p owns it (the first writer of the slot the chunk keeps), else M (bits 0..10) | q (bits
//         11..16) of the slot's first later writer | n_l (bits 17..22) later writers | the entry index of the later
//         writers past the first (bits 23..31; a chunk holds at most 510 such entries, and they come first)
//     w1  lam^(L-1-p) * ww if owned, else 0
//     w2  the first later writer's lam^(L-1-q) * ww (0 if none)
//   variable part: a 16-byte header {bytes, flags (bit 31: the chunk holds a reset), n_ro, n_wo}; a table of 64
//   16-bit entry indices, position p's first contribution past the eighth; then n_wo entries of later writers past
//   the first of each owned slot (by record, ascending q) and n_ro entries of read contributions past the eighth of
//   each position (by position, ascending q): {c, q}.  The write entries come first: an owner walks its slot's in
//   sequence, so in a crowded chunk they should sit in the part the scan stages in LDS.  The records hold no entry
//   index of their own (12 bytes, not 16: the plans are written once and read once per call, so their size is
//   core traffic).
struct PickGeom {
  static constexpr int kRec = 12;   // bytes of a record
  __host__ __device__ static constexpr int off_w() { return kChunk * 8 * kRec; }
  __host__ __device__ static constexpr int off_var() { return 2 * kChunk * 8 * kRec; }
  // entries start after the header and the 16-bit table of the positions' first read entries
  __host__ __device__ static constexpr int off_ent() { return 16 + 2 * kChunk; }
  // at most sum_p max(p - 8, 0) = 1,540 contributions and 511 later writers past the inline ones
  __host__ __device__ static constexpr int max_entries() { return 1540 + 511; }
  __host__ __device__ static constexpr int stride() {
    return (off_var() + off_ent() + 8 * max_entries() + 255) / 256 * 256;
  }
};

// Bytes of a plan's variable part the scan stages in LDS (typical parts hold well under 1 KB; entries past the
// staged bytes are read from the plan in global memory, so a crowded chunk costs time, not LDS).
constexpr int kVarStage = 4096;

// threads of one scan workgroup: 64 positions x 8 lanes (column segments)
constexpr int kScanThreads = 512;

__host__ __device__ constexpr int pad4(int M) { return (M + 3) / 4 * 4; }

// LDS of one scan workgroup: the slab A[M + 1][CW] and the write counts cnt[M + 1] (row M, which pad picks read,
// stays zero), by chunk parity two buffers of the chunk's values s_v[64][CW] (in the value type, vb bytes each) and
// of its staged variable plan part, one buffer of the chunk's position records, the fade powers pw[68] and the
// variable-part sizes of all n_chunks plans.
__host__ __device__ constexpr size_t scan_lds_bytes(int M, int CW, int n_chunks, int KP, int vb) {
  return sizeof(float) * (static_cast<size_t>(M + 1) * CW + pad4(M + 1)) + 2 * static_cast<size_t>(vb) * kChunk * CW +
         2 * static_cast<size_t>(kVarStage) + static_cast<size_t>(kChunk) * PlanGeom{KP}.pos_bytes() +
         sizeof(float) * 68 + sizeof(int32_t) * pad4(n_chunks);
}

// static LDS of plan_kernel (fade powers, totals)
__host__ __device__ constexpr size_t plan_static_lds(int) { return 4 * (kChunk + 4) + 64; }
// plan_kernel's first-rank table: M 16-bit entries, padded to 16 bytes
__host__ __device__ constexpr size_t plan_rank_bytes(int M) { return (2 * static_cast<size_t>(M) + 15) / 16 * 16; }
// plan_kernel's dynamic LDS before the sub-keys: writer masks, first ranks, write weights by rank
__host__ __device__ constexpr size_t plan_dynamic_lds(int M, int KP) {
  return 8 * static_cast<size_t>(M) + plan_rank_bytes(M) + 4 * static_cast<size_t>(kChunk) * KP;
}

// ---------------------------------------------------------------------------------------------------------------
// host side: the shape plan of a call and launch helpers
struct Plan {
  int B, T, H, dh, d_a, half, n_sub, M, k, c1, kk, pitch, cap, n_chunks;
  int cw, cw32;     // scan: value columns per workgroup for bfloat16 and float32 values (0: does not fit)
  int groups;       // the most scan workgroups per (batch row, head) slab over both value types (workspace size)
  // forward workspace offsets
  size_t off_sizes, off_plans, off_sync, off_xch, off_gate, total;
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// widest column group per scan workgroup (32, 16 or 8 value columns) whose slab and buffers fit in LDS, for
// values of vb bytes (4 covers both value types)
inline int scan_columns(int M, int dh, int n_chunks, int KP, int vb) {
  for (int cw : {32, 16, 8})
    if (dh % cw == 0 && scan_lds_bytes(M, cw, n_chunks, KP, vb) <= kLdsBytes) return cw;
  return 0;
}

// core: the shape must suit the scan and the decode step too (head_dim); the addressing alone needs only the keys
inline int make_plan(const sdm_rt_dims* d, Plan* p, bool core = true) {
  if (!d) return set_err(SDM_RT_EINVAL, "dims is NULL");
  if (d->batch < 0 || d->seq_len < 0) return set_err(SDM_RT_EINVAL, "negative batch or seq_len");
  if (d->heads < 1) return set_err(SDM_RT_EINVAL, "heads must be >= 1");
  if (core && (d->head_dim < 8 || d->head_dim % 8 != 0))
    return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d must be a positive multiple of 8", d->head_dim);
  if (core && d->head_dim > 512) return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d exceeds 512", d->head_dim);
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
  p->n_chunks = (p->T + kChunk - 1) / kChunk;
  p->cw = p->cw32 = p->groups = 0;
  p->off_sizes = p->off_plans = p->off_sync = p->off_xch = p->off_gate = p->total = 0;
  if (!core) return SDM_RT_OK;
  // the column group of bfloat16 values (wider when it fits); float32 values may need a narrower one
  p->cw = scan_columns(p->M, p->dh, p->n_chunks, p->pitch, 2);
  p->cw32 = scan_columns(p->M, p->dh, p->n_chunks, p->pitch, 4);
  if (!p->cw)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations and T = %d do not fit a slab of 8 columns in LDS", p->M,
                   p->T);
  p->groups = p->dh / (p->cw32 ? p->cw32 : p->cw);   // the workspace is sized for the larger group count
  if (plan_static_lds(p->pitch) + plan_dynamic_lds(p->M, p->pitch) + 8 * static_cast<size_t>(p->n_sub) * p->half +
          256 > kLdsBytes)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations: writer masks and sub-keys do not fit in LDS", p->M);
  const size_t slabs = static_cast<size_t>(p->B) * p->H;
  const size_t n_plans = slabs * p->n_chunks;
  size_t o = 0;
  p->off_sizes = o;
  o = align_up(o + sizeof(int32_t) * n_plans, 256);
  p->off_plans = o;
  // the plans of either scan (the pick plan serves picks of at most 8)
  const int stride = p->pitch == 8 ? std::max(PlanGeom{8}.stride(), PickGeom::stride()) : PlanGeom{p->pitch}.stride();
  o = align_up(o + static_cast<size_t>(stride) * n_plans, 256);
  p->off_sync = o;   // per slab and group a progress counter, then one status word
  o = align_up(o + sizeof(uint32_t) * (slabs * p->groups + 1), 256);
  // per slab, chunk and group the 64 partial sums of squares of the out-norm (8 bytes each: the pick scan pairs every
  // sum with a flag that says it is written)
  p->off_xch = o;
  o = align_up(o + (d->out_norm && p->groups > 1 ? 8 * slabs * p->n_chunks * p->groups * kChunk : 0), 256);
  // with the write gate, a copy of the gate logits the forward read, [B*T][H] in the input type (4 bytes reserved)
  p->off_gate = o;
  o = align_up(o + (d->write_gate ? sizeof(float) * static_cast<size_t>(p->B) * p->T * p->H : 0), 256);
  p->total = o;
  return SDM_RT_OK;
}

// the scan's column group for values of in_dtype, or 0 with the error set
inline int scan_cw(const Plan& p, sdm_rt_dtype in_dtype) {
  const int cw = in_dtype == SDM_RT_BF16 ? p.cw : p.cw32;
  if (!cw)
    set_err(SDM_RT_EUNSUPPORTED, "M = %d locations and T = %d do not fit a slab of 8 float32 columns in LDS", p.M,
            p.T);
  return cw;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_err(SDM_RT_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return SDM_RT_OK;
}

// lets a kernel use all the LDS its static arrays leave free for dynamic LDS (once per kernel and process)
inline bool allow_lds(const void* fn) {
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess || fa.sharedSizeBytes > kLdsBytes) return false;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(kLdsBytes - fa.sharedSizeBytes)) == hipSuccess;
}
inline int lds_err(const char* what) {
  return set_err(SDM_RT_ELAUNCH, "%s: cannot enable %zu bytes of LDS", what, kLdsBytes);
}

// bytes of the prepared sub-key pieces of a shape (0: no bfloat16 matrix-core scoring)
inline int64_t key_pieces_bytes(const Plan& p) {
  if (!(p.half == 8 || p.half == 16 || p.half == 32) || p.n_sub > 64) return 0;
  const int nsp = key_piece_rows(p.n_sub);
  switch (p.half) {
    case 8: return KeyPieces<8>::bytes(p.H, nsp);
    case 16: return KeyPieces<16>::bytes(p.H, nsp);
    default: return KeyPieces<32>::bytes(p.H, nsp);
  }
}

inline AddrGeom addr_geom(const Plan& p, const sdm_rt_params* prm) {
  AddrGeom g;
  g.keys[0] = prm->keys1;
  g.keys[1] = prm->keys2;
  g.addr_b = prm->addr_b;
  g.log_scale = prm->log_scale;
  g.gate_bias = prm->gate_bias;
  const int64_t need = key_pieces_bytes(p);   // pieces too small for this shape are not read
  g.kpieces = need > 0 && prm->key_pieces && static_cast<int64_t>(prm->key_pieces_bytes) >= need
                  ? static_cast<const uint32_t*>(prm->key_pieces)
                  : nullptr;
  g.H = p.H;
  g.n_sub = p.n_sub;
  g.c1 = p.c1;
  g.kk = p.kk;
  return g;
}

// dispatch on the half width of an address (compile-time unrolled addressing)
template <template <int, typename> class F, typename InT, typename... Args>
int by_half(int half, Args&&... args) {
  switch (half) {
    case 1: return F<1, InT>::run(args...);
    case 2: return F<2, InT>::run(args...);
    case 3: return F<3, InT>::run(args...);
    case 4: return F<4, InT>::run(args...);
    case 6: return F<6, InT>::run(args...);
    case 8: return F<8, InT>::run(args...);
    case 12: return F<12, InT>::run(args...);
    case 16: return F<16, InT>::run(args...);
    case 24: return F<24, InT>::run(args...);
    case 32: return F<32, InT>::run(args...);
    default:
      return set_err(SDM_RT_EUNSUPPORTED, "addr_dim %d: half width must be one of 1,2,3,4,6,8,12,16,24,32", 2 * half);
  }
}

// the matrix-core addressing covers half widths 8, 16, 32 and up to 32 sub-keys per half
constexpr bool mf_half(int half) { return half == 8 || half == 16 || half == 32; }
inline bool use_mf(const Plan& p) { return mf_half(p.half) && p.n_sub <= 32; }
// the addressing entry point also takes 64 sub-keys per half on the matrix cores (two sub-key tiles)
inline bool use_mf64(const Plan& p) { return mf_half(p.half) && p.n_sub > 32 && p.n_sub <= 64; }
// no masked candidate: 32 sub-keys per half and 8 picks from the top 8 of each half
inline bool full_grid(const Plan& p) { return use_mf(p) && p.n_sub == 32 && p.c1 == 8 && p.kk == 8; }

inline int check_dtype(sdm_rt_dtype t, const char* what) {
  if (t != SDM_RT_F32 && t != SDM_RT_BF16) return set_err(SDM_RT_EINVAL, "%s: unknown dtype %d", what, (int)t);
  return SDM_RT_OK;
}

inline int check_params(const sdm_rt_params* prm, bool need_onorm, bool need_decay = true) {
  if (!prm) return set_err(SDM_RT_EINVAL, "params is NULL");
  if (!prm->keys1 || !prm->keys2) return set_err(SDM_RT_EINVAL, "keys1/keys2 must not be NULL");
  if (!prm->log_scale) return set_err(SDM_RT_EINVAL, "log_scale must not be NULL");
  if (need_decay && !prm->decay) return set_err(SDM_RT_EINVAL, "decay must not be NULL");
  if (need_onorm && !prm->onorm_w) return set_err(SDM_RT_EINVAL, "onorm_w must not be NULL when out_norm is set");
  return SDM_RT_OK;
}

// ---------------------------------------------------------------------------------------------------------------
// launchers defined in one translation unit each and used by the others

// address_kernel over B * T rows of one or two address sets (sdm_address_bf16.hip, sdm_address_f32.hip)
int launch_address_bf16(const Plan& p, const AddrArgs& a, hipStream_t st);
int launch_address_f32(const Plan& p, const AddrArgs& a, hipStream_t st);
inline int launch_address(const Plan& p, const AddrArgs& a, sdm_rt_dtype in_dtype, hipStream_t st) {
  return in_dtype == SDM_RT_BF16 ? launch_address_bf16(p, a, st) : launch_address_f32(p, a, st);
}

// The forward core (sdm_scan.hip): plan_kernel then scan_kernel.  read_out (float32 rows of H * dh, the read before
// the out-norm) and den_out ([B*T][H]) are optional outputs for the training forward.
struct CoreIO {
  const void* kz;
  int64_t kz_stride;
  const void* qz;
  int64_t qz_stride;
  const void* v;
  int64_t v_stride;
  const void* gate_logits;   // nullptr without the write gate
  int64_t g_stride;
  sdm_rt_dtype in_dtype;
  const uint8_t* reset;
  void* r_out;
  int64_t r_stride;
  sdm_rt_dtype out_dtype;
  const float* state_in_mem;
  const float* state_in_cnt;
  float* state_out_mem;
  float* state_out_cnt;
  float* read_out;
  float* den_out;
};
int run_core(const Plan& p, const sdm_rt_dims* dims, const sdm_rt_params* prm, const CoreIO& io, void* workspace,
             hipStream_t st);

// the current device's copy of sdm_rt_forward_noalloc's scratch array (sdm_noalloc.hip)
int scratch_ptr(void** out);

}  // namespace sdmrt
