// sdm_rt.hip -- HIP kernels for gfx950 and the C ABI declared in include/sdm_rt.h.
//
// One forward is four launches:
//   plan_kernel     per (chunk of 64 positions, head, batch row): product-key addressing of the chunk's write keys
//                   and read queries (pk_address :134-148; softmax weights and gate, prepare :203-207), then the
//                   chunk's plan: which earlier positions of the chunk each read sees (with their faded
//                   coefficients) and, for every location the chunk writes, the list of its writers
//   scan_kernel     per (batch row, head, group of CW value columns): the memory slab of M x CW float32 values plus
//                   the M write counts stays in LDS for the whole sequence; each chunk reads the carried state and
//                   the in-chunk writes its plan lists, then adds the chunk's faded writes (_chunk :215-241)
//   finish_kernel   per (token, head): r * rsqrt(mean(r^2) + eps) * onorm_w (finish :243-246)
// address_kernel runs the addressing alone for sdm_rt_address; a decode step (sdm_rt_decode_step) is one addressing
// launch for both address sets and decode_kernel, one token per stream; table_read_kernel is the weighted row read of
// TrainedSdm (sdm_rt_table_read).
//
// Decay bookkeeping in scan_kernel: the slab holds A with the true state S = mu * A (mu a per-slab scalar).  A chunk
// of L positions reads mu * lam^p * A[slot] at offset p, then mu <- mu * lam^L and each write at offset q adds
// lam^(L-1-q) / mu * w * v.  When mu falls below 2^-60 the slab is multiplied by mu once and mu reset to 1, so the
// slab is only rescaled about once every 60 / -log2(lam^64) chunks (never, at T = 2048, for lam >= 0.97) and
// lam = 0 (keep only the previous write) and lam = 1 (never fade) are exact.

#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <type_traits>

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
template <int FS>
__device__ __forceinline__ double half_key(float a, double inv, int i) {   // s = a * inv
  const unsigned long long b = __double_as_longlong(fma(static_cast<double>(a), inv, 6.0));
  const uint32_t lo = (static_cast<uint32_t>(b) & 0xfff80000u) | (static_cast<uint32_t>(31 - i) << FS);
  return __longlong_as_double((b & 0xffffffff00000000ull) | lo);
}
__device__ __forceinline__ double key_or(double k, uint32_t bits) {
  return __longlong_as_double(__double_as_longlong(k) | bits);
}
__device__ __forceinline__ double key_invalid(double k) {
  return __longlong_as_double((0x00100000ull << 32) | (__double_as_longlong(k) & 0xffffffffull));
}
// the mean score of a grid key, to within 2^-32
__device__ __forceinline__ float grid_score(double k) {
  const double v = __longlong_as_double(__double_as_longlong(k) & ~0x3ffffull);
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
                                                int rows, floatx16 (&acc)[2], float (&inv)[2]) {
  constexpr int S = HALF / 2;
  const int l = threadIdx.x & 63;
  const int kb = l >> 5, jl = l & 31;
  float ka[S], zb[2][S], ab[S];
  load_vals<S, float>(g.keys[hf] + (static_cast<int64_t>(h) * g.n_sub + min(jl, g.n_sub - 1)) * HALF + kb * S, ka);
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
    const float kinv = (FULL || jl < g.n_sub) ? inv_norm(__uint_as_float(kp[0]) + __uint_as_float(kp[1])) : 0.f;
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
// 32..63 feed zeros).
template <int HALF, bool FULL>
__device__ __forceinline__ void half_scores_bf16(const AddrGeom& g, int h, int hf, const bf16_t* z0, int64_t zstride,
                                                 int rows, floatx16 (&acc)[2], float (&inv)[2]) {
  static_assert(HALF % 8 == 0, "bfloat16 scoring feeds 8 dims per lane");
  constexpr int Q = (HALF + 15) / 16;
  const int l = threadIdx.x & 63;
  const int kb = l >> 5, jl = l & 31;
  const bool has = HALF >= 16 || kb == 0;
  const int d0 = hf * HALF + 8 * kb;   // first dim of the address this lane feeds
  float ka[Q][8], ab[Q][8];
  uint4 zr[2][Q];
  const float* krow = g.keys[hf] + (static_cast<int64_t>(h) * g.n_sub + min(jl, g.n_sub - 1)) * HALF + 8 * kb;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = min(32 * t + jl, rows - 1);
      zr[t][q] = has ? load_raw8(z0 + row * zstride + static_cast<int64_t>(h) * 2 * HALF + d0 + 16 * q)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
    if (has) {
      load_vals<8, float>(krow + 16 * q, ka[q]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) ka[q][e] = 0.f;
    }
    if (g.addr_b && has) {
      load_vals<8, float>(g.addr_b + h * 2 * HALF + d0 + 16 * q, ab[q]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) ab[q][e] = 0.f;
    }
  }
  {   // unit-normalised sub-key row
    float ks = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) ks = fmaf(ka[q][e], ka[q][e], ks);
    const auto kp = __builtin_amdgcn_permlane32_swap(__float_as_uint(ks), __float_as_uint(ks), false, false);
    const float kinv = (FULL || jl < g.n_sub) ? inv_norm(__uint_as_float(kp[0]) + __uint_as_float(kp[1])) : 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) ka[q][e] *= kinv;
  }
  floatx16 init = {};
  if (g.addr_b) {
    float cp = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) cp = fmaf(ka[q][e], ab[q][e], cp);
    const auto cw = __builtin_amdgcn_permlane32_swap(__float_as_uint(cp), __float_as_uint(cp), false, false);
    const float c = __uint_as_float(cw[0]) + __uint_as_float(cw[1]);
    init = __builtin_amdgcn_mfma_f32_32x32x2f32(kb == 0 ? c : 0.f, kb == 0 ? 1.f : 0.f, init, 0, 0, 0);
  }
  uint32_t kt[3][Q][4];   // the three bfloat16 terms, packed in pairs
#pragma unroll
  for (int q = 0; q < Q; ++q) {
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float x0 = ka[q][2 * e2], x1 = ka[q][2 * e2 + 1];
#pragma unroll
      for (int term = 0; term < 3; ++term) {
        const uint32_t p = pack_bf16(x0, x1);
        kt[term][q][e2] = p;
        x0 -= __uint_as_float(p << 16);   // exact
        x1 -= __uint_as_float(p & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const uint32_t wd[4] = {zr[t][q].x, zr[t][q].y, zr[t][q].z, zr[t][q].w};
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float v0 = __uint_as_float(wd[e2] << 16) + ab[q][2 * e2];
        const float v1 = __uint_as_float(wd[e2] & 0xffff0000u) + ab[q][2 * e2 + 1];
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
        const uint4 kq = make_uint4(kt[term][q][0], kt[term][q][1], kt[term][q][2], kt[term][q][3]);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kq),
                                                         __builtin_bit_cast(bf16x8, zr[t][q]), acc[t], 0, 0, 0);
      }
    }
  }
}

// Picks of address l (lane l) of the 64 rows z0[r * zstride + h * 2 * HALF ...], r < rows (rows past `rows` are
// clamped; their lanes' outputs are unspecified): the selection of address_one on offset keys, scores within 2^-31
// of float rounding.  FULL: n_sub = 32 and c1 = kk = CAP (no candidate is masked).  All 64 lanes of the wave must
// call it.
template <int HALF, int CAP, typename InT, bool FULL>
__device__ __forceinline__ void address_wave(const AddrGeom& g, int h, const InT* z0, int64_t zstride, int rows,
                                             float gate, int (&slot)[CAP], float (&w)[CAP], float (&score)[CAP]) {
  const int kb = (threadIdx.x & 63) >> 5;
  double hk[2][CAP];   // ranked half keys
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    floatx16 acc[2];
    float inv[2];
    if constexpr (sizeof(InT) == 2) half_scores_bf16<HALF, FULL>(g, h, hf, z0, zstride, rows, acc, inv);
    else half_scores_f32<HALF, InT, FULL>(g, h, hf, z0, zstride, rows, acc, inv);
    // after the swap below lane l holds every score of address row l
    const double dinv = static_cast<double>(kb ? inv[1] : inv[0]);
    double c[32];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0][r]), __float_as_uint(acc[1][r]), false,
                                                       false);
      const int i0 = 8 * (r / 4) + (r % 4);
      if (hf == 0) {
        c[r] = half_key<6>(__uint_as_float(sw[0]), dinv, i0);
        c[16 + r] = half_key<6>(__uint_as_float(sw[1]), dinv, i0 + 4);
      } else {
        c[r] = half_key<1>(__uint_as_float(sw[0]), dinv, i0);
        c[16 + r] = half_key<1>(__uint_as_float(sw[1]), dinv, i0 + 4);
      }
      if (!FULL) {   // sub-keys past n_sub are never picked
        if (i0 >= g.n_sub) c[r] = key_invalid(c[r]);
        if (i0 + 4 >= g.n_sub) c[16 + r] = key_invalid(c[16 + r]);
      }
    }
    top_k_desc<CAP, 32>(c);
#pragma unroll
    for (int r = 0; r < CAP; ++r) hk[hf][r] = key_or(c[r], static_cast<uint32_t>(15 - r) << (hf == 0 ? 15 : 11));
  }
  // combine over the dominance-pruned grid (see address_one)
  auto cell = [&](int ra, int rb) {
    const double k = hk[0][ra] + hk[1][rb];
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
    cv[p] = grid_score(pc[p]);
    const uint32_t f = static_cast<uint32_t>(__double_as_longlong(pc[p]));
    if (FULL) {
      si[p] = 1023 - static_cast<int>(f & 1023u);   // (31 - i1) * 32 + (31 - i2) = 1023 - slot
    } else {
      const int i1 = 31 - static_cast<int>((f >> 5) & 31u), i2 = 31 - static_cast<int>(f & 31u);
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

// sdm_rt_address: one thread per (token, head).  Grid: x = token tiles of 64, y = head.  MODE 1 and 2: the tile is
// addressed by the wave on the matrix cores (address_wave; 2 = no masked candidate), MODE 0: per thread with the
// sub-keys staged in LDS (address_one).
template <int HALF, int CAP, typename InT, int MODE>
__global__ void __launch_bounds__(64) address_kernel(AddrArgs a) {
  extern __shared__ float kn[];   // [2][n_sub][HALF] (per-thread path)
  const int h = blockIdx.y;
  const int64_t N = static_cast<int64_t>(a.B) * a.T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t n = n0 + threadIdx.x;
  if (blockIdx.z == 1) {   // the second address set
    a.z = a.z2;
    a.z_stride = a.z2_stride;
    a.gl = nullptr;
    a.slot_out = a.slot_out2;
    a.w_out = a.w_out2;
    a.s_out = a.s_out2;
  }
  const float gate =
      (a.gl && n < N) ? gate_of(static_cast<const InT*>(a.gl) + n * a.g_stride, h, a.g.gate_bias) : 1.f;
  int slot[CAP];
  float w[CAP], sc[CAP];
  if constexpr (MODE > 0) {
    address_wave<HALF, CAP, InT, MODE == 2>(a.g, h, static_cast<const InT*>(a.z) + n0 * a.z_stride, a.z_stride,
                                     static_cast<int>(min<int64_t>(64, N - n0)), gate, slot, w, sc);
    if (n >= N) return;
  } else {
    stage_keys<HALF>(a.g, h, kn, threadIdx.x, 64);
    __syncthreads();
    if (n >= N) return;
    const InT* zrow = static_cast<const InT*>(a.z) + n * a.z_stride + static_cast<int64_t>(h) * 2 * HALF;
    address_one<HALF, CAP, InT>(a.g, h, kn, zrow, gate, slot, w, sc);
  }
  const int b = static_cast<int>(n / a.T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * a.T);
  const int64_t base = ((static_cast<int64_t>(b) * a.g.H + h) * a.T + t) * a.pitch;
#pragma unroll
  for (int p = 0; p < CAP; ++p) {
    if (p < a.pitch) {
      const bool live = p < a.g.kk;
      a.slot_out[base + p] = live ? slot[p] : -1;
      if (a.w_out) a.w_out[base + p] = w[p];
      if (a.s_out) a.s_out[base + p] = sc[p];
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// the chunk plan
//
// One plan per (batch row, head, chunk) at a fixed stride in the workspace.  The scan reads its fixed-size part
// straight into registers and stages its variable part into LDS (KP = pick pitch, PR = position record bytes):
//   pos[64]          per position p: u16 slot[KP], f32 w[KP] (read picks and weights, pads 0), then the tail:
//                    u16 ri_begin | u16 ri_end (its in-chunk contributions past the first kInline, in the variable
//                    part), f32 csum (the sum of all its in-chunk read coefficients), u8 q[kInline] and u8 n_inline
//                    (bytes 8..15), f32 c[kInline] (the first kInline contributions), padding to PR bytes
//   wrec[64][KP]     write records of 8 bytes; distinct written slot u of the chunk is wrec[u % 64][u / 64] =
//                    {slot | q0 << 16 | xo << 22, c0 | more << 31}: q0 is the slot's first writer in the chunk and
//                    c0 = lam^(L-1-q0) * ww its coefficient; when later positions write the slot too (more = 1)
//                    their entries are ext[xo], ext[xo + 1], ... up to the one flagged last.  Slots with later
//                    writers come first.  Entries past the chunk's n_wu slots are null records {M, 0}: they read
//                    row M (always zero) and write nothing
//   variable part    u32 {n_ri, n_wu | reset << 31, n_ext, bytes} (reset: the chunk holds a reset, so the state it
//                    leaves holds only the writes after its last reset); ext[n_ext] = {c = lam^(L-1-q) * ww,
//                    q | last << 31};
//                    f32 ri_c[n_ri]; u8 ri_q[n_ri]
// An in-chunk read contribution (q, c) of position p: position q < p of the chunk wrote some of p's read slots;
// c = the sum over those slots of wr * ww * lam^(p-1-q).  Contributions run in ascending q.  sizes[] holds the
// bytes of each plan's variable part.
constexpr int kInline = 6;   // in-chunk contributions kept in the position record
struct PlanGeom {
  int KP;
  __host__ __device__ constexpr int pos_bytes() const { return (6 * KP + 16 + 4 * kInline + 15) / 16 * 16; }
  __host__ __device__ constexpr int off_tail() const { return 6 * KP; }
  __host__ __device__ constexpr int off_wrec() const { return kChunk * pos_bytes(); }
  __host__ __device__ constexpr int off_var() const { return off_wrec() + 8 * kChunk * KP; }
  __host__ __device__ constexpr int max_var() const {
    return (16 + 8 * kChunk * KP + 5 * (kChunk * (kChunk - 1) / 2) + 15) / 16 * 16;
  }
  __host__ __device__ constexpr int stride() const { return (off_var() + max_var() + 255) / 256 * 256; }
};

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
  int B, T, M, n_chunks;
};

// Bytes of a plan's variable part the scan stages in LDS.  Typical parts hold 1-2 KB; the worst case (every position
// reading every earlier one, every slot written by every position) is 14 KB at k <= 8.  Entries past the staged bytes
// are read from the plan in global memory, so a crowded chunk costs time, not LDS.
constexpr int kVarStage = 4096;
__host__ __device__ constexpr int var_stage(int KP) {
  return PlanGeom{KP}.max_var() < kVarStage ? PlanGeom{KP}.max_var() : kVarStage;
}

// static LDS of plan_kernel (picks, fade powers, totals)
__host__ __device__ constexpr size_t plan_static_lds(int KP) { return 2 * kChunk * KP * (2 + 4) + 4 * (kChunk + 4) + 16; }

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

// plan_kernel: block (chunk, head, batch row), 128 threads: wave 0 addresses the write keys of the chunk's positions,
// wave 1 the read queries (MODE 1, 2: on the matrix cores, MODE 0: per thread); then the writers of every slot are marked in
// 64-bit masks, each position's read contributions and each written slot's writer list are found, counted,
// prefix-summed within the wave and written out.
template <int HALF, int KP, typename InT, int MODE>
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

  __shared__ __attribute__((aligned(16))) uint16_t pk_slot[2][kChunk][KP];
  __shared__ __attribute__((aligned(16))) float pk_w[2][kChunk][KP];
  __shared__ float pw[kChunk + 4];
  __shared__ int tot[4];
  extern __shared__ unsigned long long wmask[];   // [M], then (per-thread path) the head's sub-keys [2][n_sub][HALF]
  float* kn = reinterpret_cast<float*>(wmask + M);

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

  // addressing
  {
    int slot[KP];
    float w[KP], sc[KP];
    const int64_t row0 = static_cast<int64_t>(b) * a.T + c0;
    const float gate = (set == 0 && a.gl && p < L)
                           ? gate_of(static_cast<const InT*>(a.gl) + (row0 + p) * a.g_stride, h, a.g.gate_bias)
                           : 1.f;
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
      pk_slot[set][p][j] = p < L ? static_cast<uint16_t>(slot[j]) : 0;
      pk_w[set][p][j] = p < L ? w[j] : 0.f;
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
    for (int j = 0; j < kk; ++j) atomicOr(&wmask[pk_slot[0][p][j]], 1ull << p);
  }
  __syncthreads();
  // weight with which position q wrote slot m (a position's picks are distinct locations)
  auto wweight = [&](int q, int m) {
    float r = 0.f;
#pragma unroll
    for (int g8 = 0; g8 < KP / 8; ++g8) {   // the row's picks and weights in 16-byte reads
      const uint4 sv = *reinterpret_cast<const uint4*>(&pk_slot[0][q][8 * g8]);
      const float4 wa = *reinterpret_cast<const float4*>(&pk_w[0][q][8 * g8]);
      const float4 wb = *reinterpret_cast<const float4*>(&pk_w[0][q][8 * g8 + 4]);
      const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
      const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sj = static_cast<int>((sw[j / 2] >> (16 * (j % 2))) & 0xffffu);
        if (8 * g8 + j < kk && sj == m) r = wv[j];
      }
    }
    return r;
  };
  int ms[KP];
  float ws[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    ms[j] = pk_slot[set][p][j];
    ws[j] = pk_w[set][p][j];
  }
  unsigned long long mk[KP];           // read side: the earlier writers of each read slot
  unsigned long long touched = 0ull;   // read side: every earlier position contributing to this one
  int n_a = 0, n_b = 0;                // read side: contributions; write side: distinct slots owned, later writers
  int n_m = 0;                         // write side: owned slots with later writers
  if (p < L) {
    if (set == 1) {
      const unsigned long long below = ((1ull << p) - 1ull) & (seg0 >= 0 ? ~((1ull << seg0) - 1ull) : ~0ull);
#pragma unroll
      for (int i = 0; i < KP; ++i) {
        mk[i] = i < kk ? wmask[ms[i]] & below : 0ull;
        touched |= mk[i];
      }
      n_a = max(__builtin_popcountll(touched) - kInline, 0);   // contributions past the inline ones
    } else {
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) {
          const unsigned long long mm = wmask[ms[j]] & keep;
          if (mm && __builtin_ctzll(mm) == p) {
            const int later = __builtin_popcountll(mm) - 1;
            ++n_a;
            n_b += later;
            n_m += later > 0;
          }
        }
      }
    }
  }
  const int inc_a = wave_incl_scan(n_a, p);
  const int inc_b = wave_incl_scan(n_b, p);
  const int inc_m = wave_incl_scan(n_m, p);
  if (p == 63) {
    if (set == 1) {
      tot[0] = inc_a;
    } else {
      tot[1] = inc_a;
      tot[2] = inc_b;
      tot[3] = inc_m;
    }
  }
  __syncthreads();
  const int n_ri = tot[0], n_wu = tot[1], n_ext = tot[2];
  const int64_t plan_id = (static_cast<int64_t>(b) * a.g.H + h) * a.n_chunks + c;
  unsigned char* plan = a.plans + plan_id * pg.stride();
  unsigned char* var = plan + pg.off_var();
  uint2* ext = reinterpret_cast<uint2*>(var + 16);
  float* ri_c = reinterpret_cast<float*>(var + 16 + 8 * n_ext);
  unsigned char* ri_q = var + 16 + 8 * n_ext + 4 * n_ri;
  if (tid == 0) {
    const int bytes = 16 + 8 * n_ext + 5 * n_ri;
    *reinterpret_cast<uint4*>(var) = make_uint4(n_ri, n_wu | (rmask ? 0x80000000u : 0u), n_ext, bytes);
    a.sizes[plan_id] = bytes;
  }
  if (set == 1) {
    // position record: slots, weights, then the tail
    uint32_t rec[pg.pos_bytes() / 4];
#pragma unroll
    for (int i = 0; i < pg.pos_bytes() / 4; ++i) rec[i] = 0u;
#pragma unroll
    for (int i = 0; i < KP; i += 2) rec[i / 2] = static_cast<uint32_t>(ms[i]) | (static_cast<uint32_t>(ms[i + 1]) << 16);
#pragma unroll
    for (int i = 0; i < KP; ++i) rec[KP / 2 + i] = seg0 >= 0 ? 0u : __float_as_uint(ws[i]);   // no state after a reset
    // in-chunk contributions in ascending q, and their coefficient sum: the first kInline into the record
    const int e0 = inc_a - n_a;
    int k = e0, j = 0;
    float csum = 0.f;
    uint32_t qb[2] = {0u, 0u};
    while (touched) {
      const int q = __builtin_ctzll(touched);
      touched &= touched - 1ull;
      float coef = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i)
        if ((mk[i] >> q) & 1ull) coef = fmaf(ws[i], wweight(q, ms[i]), coef);
      coef *= pw[p - 1 - q];
      if (j < kInline) {
        qb[j / 4] |= static_cast<uint32_t>(q) << (8 * (j % 4));
#pragma unroll
        for (int t = 0; t < kInline; ++t)
          if (t == j) rec[pg.off_tail() / 4 + 4 + t] = __float_as_uint(coef);
        ++j;
      } else {
        ri_q[k] = static_cast<unsigned char>(q);
        ri_c[k] = coef;
        ++k;
      }
      csum += coef;
    }
    rec[pg.off_tail() / 4] = static_cast<uint32_t>(e0) | (static_cast<uint32_t>(inc_a) << 16);
    rec[pg.off_tail() / 4 + 1] = __float_as_uint(csum);
    rec[pg.off_tail() / 4 + 2] = qb[0];
    rec[pg.off_tail() / 4 + 3] = qb[1] | (static_cast<uint32_t>(j) << 24);
    uint4* dst = reinterpret_cast<uint4*>(plan + p * pg.pos_bytes());
#pragma unroll
    for (int i = 0; i < pg.pos_bytes() / 16; ++i) dst[i] = make_uint4(rec[4 * i], rec[4 * i + 1], rec[4 * i + 2], rec[4 * i + 3]);
  } else {
    uint2* wrec = reinterpret_cast<uint2*>(plan + pg.off_wrec());
    // null records for group p's unused entries: row M, coefficient 0
#pragma unroll
    for (int k = 0; k < KP; ++k)
      if (p + kChunk * k >= n_wu) wrec[p * KP + k] = make_uint2(static_cast<uint32_t>(M), 0u);
    if (p >= L) return;
    // slots with later writers take the lowest indexes (records k = 0, 1, ...), so the scan's walks of the later
    // writers gather in the first record batches
    int u_m = inc_m - n_m, u_s = tot[3] + (inc_a - inc_m) - (n_a - n_m), e = inc_b - n_b;
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j >= kk) break;
      const int m = ms[j];
      unsigned long long mm = wmask[m] & keep;
      if (!mm || __builtin_ctzll(mm) != p) continue;   // p is the slot's first (kept) writer in the chunk
      mm &= mm - 1ull;
      const uint32_t cw = __float_as_uint(pw[L - 1 - p] * ws[j]) | (mm ? 0x80000000u : 0u);
      const int u = mm ? u_m++ : u_s++;
      wrec[(u & 63) * KP + (u >> 6)] =
          make_uint2(static_cast<uint32_t>(m) | (static_cast<uint32_t>(p) << 16) | (static_cast<uint32_t>(e) << 22), cw);
      while (mm) {
        const int q = __builtin_ctzll(mm);
        mm &= mm - 1ull;
        ext[e] = make_uint2(__float_as_uint(pw[L - 1 - q] * wweight(q, m)),
                            static_cast<uint32_t>(q) | (mm ? 0u : 0x80000000u));
        ++e;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// scan (executes the plans)
struct ScanArgs {
  const unsigned char* plans;  // [B][H][n_chunks][stride]
  const int32_t* sizes;        // [B][H][n_chunks]
  const void* v;               // value rows
  int64_t v_stride;
  const float* decay;          // [H]
  const float* state_in_mem;   // [B][H][M][dh] or nullptr
  const float* state_in_cnt;   // [B][H][M] or nullptr
  float* state_out_mem;
  float* state_out_cnt;
  void* r_out;                 // rows of H * dh; OutT
  int64_t r_stride;
  float* den_out;              // [B*T][H] read denominators (mean read), or nullptr
  int B, T, H, dh, M, n_chunks, read_mean;
  float read_eps;
};

constexpr int kScanThreads = 512;   // 64 positions x 8 lanes

__host__ __device__ constexpr int pad4(int M) { return (M + 3) / 4 * 4; }

// LDS of one scan workgroup: the slab A[M + 1][CW] and the write counts cnt[M + 1] (row M, which the plan's null
// write records read, stays zero), two buffers (chunk parity) of a chunk's staged variable plan part and its values
// s_v[64][CW] in float32, fade powers pw[68] and the variable-part sizes of all n_chunks plans.
__host__ __device__ constexpr size_t scan_lds_bytes(int M, int KP, int CW, int n_chunks) {
  return sizeof(float) * (static_cast<size_t>(M + 1) * CW + pad4(M + 1)) + 2 * var_stage(KP) +
         2 * sizeof(float) * kChunk * CW + sizeof(float) * 68 + sizeof(int32_t) * pad4(n_chunks);
}

// CPL consecutive values (CPL = 4, 2, 1) from LDS in one access; bfloat16 values are converted.
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

// registers holding the next chunk's plan records, variable-part pieces and values until they are used
template <int KP, int NV, typename VT, int CPL>
struct ChunkRegs {
  uint4 pos[PlanGeom{KP}.pos_bytes() / 16];   // the group's position record
  uint4 wrec[KP / 2];                         // the group's write records
  uint2 own_w[KP / 8];                        // write records k = l8 + 8 b (the lane's count updates)
  uint32_t own_slot[KP / 8];                  // read picks l8 + 8 b and their weights (the lane's count reads)
  float own_wt[KP / 8];
  uint4 var[NV];
  VT v[CPL];
  int pieces;
};

// The next chunk's loads, in three parts (PART 0: the group's position record; 1: its write records and the lane's
// count records; 2: the variable-part pieces and the values), issued in two phases of the current chunk so the vector
// memory path streams them while the current chunk works on LDS.  Record and value loads are
// unconditional (indexes clamped into the plan), so the compiler keeps them in flight; variable-part pieces past the
// plan's size are not loaded.
template <int PART, int KP, int NV, typename VT, int CPL>
__device__ __forceinline__ void fetch_chunk(ChunkRegs<KP, NV, VT, CPL>& r, const ScanArgs& a, int64_t slab, int b,
                                            int h, int col0, int c, int bytes, int tid, int p, int l8) {
  constexpr PlanGeom pg{KP};
  const unsigned char* base = a.plans + (slab * a.n_chunks + c) * pg.stride();
  const unsigned char* prec = base + p * pg.pos_bytes();
  if constexpr (PART == 0) {
    const uint4* ps = reinterpret_cast<const uint4*>(prec);
#pragma unroll
    for (int k = 0; k < pg.pos_bytes() / 16; ++k) r.pos[k] = ps[k];
  } else if constexpr (PART == 1) {
    const uint2* wrow = reinterpret_cast<const uint2*>(base + pg.off_wrec()) + p * KP;
    const uint4* ws = reinterpret_cast<const uint4*>(wrow);
#pragma unroll
    for (int k = 0; k < KP / 2; ++k) r.wrec[k] = ws[k];
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) {
      r.own_w[k] = wrow[l8 + 8 * k];
      r.own_slot[k] = reinterpret_cast<const uint16_t*>(prec)[l8 + 8 * k];
      r.own_wt[k] = reinterpret_cast<const float*>(prec + 2 * KP)[l8 + 8 * k];
    }
  } else {
    const uint4* vs = reinterpret_cast<const uint4*>(base + pg.off_var());
    r.pieces = min((bytes + 15) >> 4, var_stage(KP) / 16);   // the staged bytes only
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int piece = tid + k * kScanThreads;
      r.var[k] = vs[piece < r.pieces ? piece : 0];   // every lane loads (piece 0 stands in); staging skips the rest
    }
    const int row = min(c * kChunk + p, a.T - 1);
    const VT* vrow = static_cast<const VT*>(a.v) + (static_cast<int64_t>(b) * a.T + row) * a.v_stride +
                     static_cast<int64_t>(h) * a.dh + col0 + CPL * l8;
#pragma unroll
    for (int k = 0; k < CPL; ++k) r.v[k] = vrow[k];
  }
}

__device__ __forceinline__ uint32_t u4_word(const uint4& q, int i) {
  return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Scan of one (batch row, head) slab over CW of its value columns, 512 threads = 64 groups x 8 lanes of CW/8
// columns.  Per chunk:
//   S1 stage  the chunk's variable plan part and values (loaded into registers one chunk ahead) into LDS
//   S2 read   group = position: mu * lam^p * S_in rows of the read picks, plus the plan's in-chunk contributions
//             of earlier positions' values; the mean read divides by mu * lam^p * sum(w * cnt) + the plan's in-chunk
//             coefficient sum
//   S3 write  group g applies its KP write records (distinct slots; null records write nothing): the
//             writers' faded values, divided by mu after the fade, are added to the slot's row, and lane l8 adds
//             record l8's coefficients to the slot's count (one owner per row: no atomics)
// All sums run in fixed orders, so results are deterministic.
template <int CW, int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(kScanThreads) scan_kernel(ScanArgs a) {
  constexpr int CPL = CW / 8;
  constexpr PlanGeom pg{KP};
  constexpr int VS = var_stage(KP);                                            // staged variable-part bytes
  constexpr int NV = (VS / 16 + kScanThreads - 1) / kScanThreads;             // variable-part pieces per thread
  constexpr int NB = 8;                                                          // write records per batch
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int M = a.M;
  float* A = lds;                                       // [M + 1][CW]
  float* cnt = A + static_cast<size_t>(M + 1) * CW;     // [M + 1]
  unsigned char* var = reinterpret_cast<unsigned char*>(cnt + pad4(M + 1));   // [2][VS], by chunk parity
  float* s_v = reinterpret_cast<float*>(var + 2 * VS);                        // [2][64][CW], by chunk parity
  float* pw = s_v + 2 * kChunk * CW;
  int32_t* s_sizes = reinterpret_cast<int32_t*>(pw + 68);   // read from LDS: a scalar load in the loop would hold up
                                                            // every LDS wait behind a memory round trip

  const int cg = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int p = tid >> 3;    // position (read) or record group (write)
  const int l8 = tid & 7;    // column segment
  const int col0 = cg * CW;
  const int64_t slab = static_cast<int64_t>(b) * a.H + h;
  const float lam = a.decay[h];
  const int32_t* sizes = a.sizes + slab * a.n_chunks;

  for (int i = tid; i < (M + 1) * CW; i += kScanThreads) {
    const int m = i / CW;
    const int c = i - m * CW;
    A[i] = (a.state_in_mem && m < M) ? a.state_in_mem[(slab * M + m) * a.dh + col0 + c] : 0.f;
  }
  for (int m = tid; m <= M; m += kScanThreads) cnt[m] = (a.state_in_cnt && m < M) ? a.state_in_cnt[slab * M + m] : 0.f;
  for (int i = tid; i < a.n_chunks; i += kScanThreads) s_sizes[i] = sizes[i];
  if (tid <= kChunk) {
    float v = 1.f;   // lam^tid by repeated multiplication (exact for lam = 0 and lam = 1)
    for (int e = 0; e < tid; ++e) v *= lam;
    pw[tid] = v;
  }
  float mu = 1.f;

  // S1, stage: chunk c's variable plan part and values into the LDS buffers of its parity (a chunk is staged
  // during the previous chunk's write phase, so it needs no barrier of its own)
  auto stage = [&](int c, const ChunkRegs<KP, NV, VT, CPL>& r) {
    unsigned char* vb = var + (c & 1) * VS;
    float* sb = s_v + (c & 1) * kChunk * CW;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int piece = tid + k * kScanThreads;
      if (piece < r.pieces) reinterpret_cast<uint4*>(vb)[piece] = r.var[k];
    }
    float vv[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) vv[k] = to_f32(r.v[k]);
    lds_seg_store<CPL>(&sb[p * CW + CPL * l8], *reinterpret_cast<const Seg<CPL>*>(vv));
  };

  // the next chunk's registers alternate between two sets (the loop below is unrolled by two), so nothing is copied
  ChunkRegs<KP, NV, VT, CPL> ra, rb;
  fetch_chunk<0>(ra, a, slab, b, h, col0, 0, sizes[0], tid, p, l8);
  fetch_chunk<1>(ra, a, slab, b, h, col0, 0, sizes[0], tid, p, l8);
  fetch_chunk<2>(ra, a, slab, b, h, col0, 0, sizes[0], tid, p, l8);
  int next_bytes = a.n_chunks > 1 ? sizes[1] : 0;
  stage(0, ra);
  lds_barrier();
  const float lam_chunk = pw[kChunk];   // the fade of a full chunk, kept in a register

  auto chunk = [&](const int c, const ChunkRegs<KP, NV, VT, CPL>& nx, ChunkRegs<KP, NV, VT, CPL>& fut) {
    const int c0 = c * kChunk;
    const int L = min(kChunk, a.T - c0);
    const unsigned char* varc = var + (c & 1) * VS;   // this chunk's staged plan part and values
    const float* s_vc = s_v + (c & 1) * kChunk * CW;
    // this chunk's records
    int m[KP];
    float w[KP];
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const uint32_t word = u4_word(nx.pos[i / 8], (i % 8) / 2);
      m[i] = static_cast<int>(i % 2 ? word >> 16 : word & 0xffffu);
      w[i] = __uint_as_float(u4_word(nx.pos[(2 * KP + 4 * i) / 16], ((2 * KP + 4 * i) % 16) / 4));
    }
    auto tail = [&](int wd) { return u4_word(nx.pos[(pg.off_tail() + 4 * wd) / 16], ((pg.off_tail() + 4 * wd) % 16) / 4); };
    const uint32_t tail0 = tail(0);
    const float csum = __uint_as_float(tail(1));
    const int ri_b = tail0 & 0xffffu, ri_e = tail0 >> 16;
    const uint32_t qw0 = tail(2), qw1 = tail(3);
    const int n_in = qw1 >> 24;
    int iq[kInline];
    float ic[kInline];
#pragma unroll
    for (int t = 0; t < kInline; ++t) {
      iq[t] = static_cast<int>(((t < 4 ? qw0 : qw1) >> (8 * (t % 4))) & 0xffu);
      ic[t] = __uint_as_float(tail(4 + t));
    }
    uint2 wr[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k)
      wr[k] = make_uint2(u4_word(nx.wrec[k / 2], 2 * (k % 2)), u4_word(nx.wrec[k / 2], 2 * (k % 2) + 1));
    uint2 own_w[KP / 8];
    int own_slot[KP / 8];
    float own_wt[KP / 8];
#pragma unroll
    for (int k = 0; k < KP / 8; ++k) {
      own_w[k] = nx.own_w[k];
      own_slot[k] = static_cast<int>(nx.own_slot[k]);
      own_wt[k] = nx.own_wt[k];
    }
    const bool more = c + 1 < a.n_chunks;
    // the next chunk's loads, unconditional (the last chunk fetches itself again): with a fixed number of loads in
    // flight every later wait for this chunk's registers is exact and does not wait for them
    const int cn = more ? c + 1 : c;
    fetch_chunk<2>(fut, a, slab, b, h, col0, cn, next_bytes, tid, p, l8);
    fetch_chunk<0>(fut, a, slab, b, h, col0, cn, next_bytes, tid, p, l8);
    if (more) next_bytes = c + 2 < a.n_chunks ? s_sizes[c + 2] : 0;
    const uint32_t* hdr = reinterpret_cast<const uint32_t*>(varc);
    const int n_ri = hdr[0], n_ext = hdr[2];
    const bool chunk_reset = hdr[1] & 0x80000000u;
    // variable-part entries: from LDS within the staged bytes, else from the plan in global memory
    const unsigned char* gvar = a.plans + (slab * a.n_chunks + c) * pg.stride() + pg.off_var();
    const int o_ri_c = 16 + 8 * n_ext, o_ri_q = 16 + 8 * n_ext + 4 * n_ri;
    // With st = std::true_type the whole part is staged and the entries come from LDS only.  The two code paths
    // stay separate: a global load on a joined path makes every use wait for all vector-memory loads in flight,
    // the next chunk's prefetched records included.
    const bool all_staged = static_cast<int>(hdr[3]) <= VS;
    auto ext_at = [&](int e, auto st) {
      const int o = 16 + 8 * e;
      if constexpr (decltype(st)::value) return *reinterpret_cast<const uint2*>(varc + o);
      else return o + 8 <= VS ? *reinterpret_cast<const uint2*>(varc + o) : *reinterpret_cast<const uint2*>(gvar + o);
    };
    auto ri_c_at = [&](int k, auto st) {
      const int o = o_ri_c + 4 * k;
      if constexpr (decltype(st)::value) return *reinterpret_cast<const float*>(varc + o);
      else return o + 4 <= VS ? *reinterpret_cast<const float*>(varc + o) : *reinterpret_cast<const float*>(gvar + o);
    };
    auto ri_q_at = [&](int k, auto st) {
      const int o = o_ri_q + k;
      if constexpr (decltype(st)::value) return static_cast<int>(varc[o]);
      else return static_cast<int>(o < VS ? varc[o] : gvar[o]);
    };
    // S2: read
    if (p < L) {
      const float fin = mu * pw[p];
      float cpart = 0.f;   // the group's lanes share the count sum: lane l8 takes picks l8, l8 + 8
#pragma unroll
      for (int k = 0; k < KP / 8; ++k) cpart = fmaf(own_wt[k], cnt[own_slot[k]], cpart);
      // one batch of reads: the rows of the read picks (pad picks carry weight 0) and the values of the in-chunk
      // contributions kept in the record (unused entries read row 0 with coefficient 0)
      Seg<CPL> x[KP], vi[kInline];
#pragma unroll
      for (int i = 0; i < KP; ++i) x[i] = lds_seg<CPL>(&A[m[i] * CW + CPL * l8]);
#pragma unroll
      for (int t = 0; t < kInline; ++t) vi[t] = lds_seg<CPL>(&s_vc[(t < n_in ? iq[t] : 0) * CW + CPL * l8]);
      float acc[CPL];
#pragma unroll
      for (int k = 0; k < CPL; ++k) acc[k] = 0.f;
#pragma unroll
      for (int i = 0; i < KP; ++i) {
#pragma unroll
        for (int k = 0; k < CPL; ++k) acc[k] = fmaf(w[i], x[i].v[k], acc[k]);
      }
#pragma unroll
      for (int k = 0; k < CPL; ++k) acc[k] *= fin;
#pragma unroll
      for (int t = 0; t < kInline; ++t) {
        const float cf = t < n_in ? ic[t] : 0.f;
#pragma unroll
        for (int k = 0; k < CPL; ++k) acc[k] = fmaf(cf, vi[t].v[k], acc[k]);
      }
      auto ri_loop = [&](auto st) {
        for (int e = ri_b; e < ri_e; e += 4) {   // the rest, from the variable part, four at a time
          float cf[4];
          Seg<CPL> vq[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int ej = min(e + j, ri_e - 1);
            cf[j] = e + j < ri_e ? ri_c_at(ej, st) : 0.f;
            vq[j] = lds_seg<CPL>(&s_vc[ri_q_at(ej, st) * CW + CPL * l8]);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int k = 0; k < CPL; ++k) acc[k] = fmaf(cf[j], vq[j].v[k], acc[k]);
          }
        }
      };
      if (all_staged) {
        ri_loop(std::true_type{});
      } else {
        ri_loop(std::false_type{});
      }
      const float cn = sum8(cpart);
      if (a.read_mean) {
        const float den = fmaf(fin, cn, csum);
        if (a.den_out && cg == 0 && l8 == 0) a.den_out[(static_cast<int64_t>(b) * a.T + c0 + p) * a.H + h] = den;
        const float inv = fast_rcp(den + a.read_eps);
#pragma unroll
        for (int k = 0; k < CPL; ++k) acc[k] *= inv;
      }
      store_vals<CPL, OutT>(static_cast<OutT*>(a.r_out) + (static_cast<int64_t>(b) * a.T + c0 + p) * a.r_stride +
                               static_cast<int64_t>(h) * a.dh + col0 + CPL * l8, acc);
    }
    lds_barrier();
    fetch_chunk<1>(fut, a, slab, b, h, col0, cn, next_bytes, tid, p, l8);
    // fade the slab by lam^L (folded into mu; rescale the slab when mu gets small); a chunk with a reset empties it
    float fade = lam_chunk;
    if (L != kChunk) fade = pw[L];
    float mu_new = mu * fade;
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
    // S3: write; group p applies records p + 64 k, NB at a time (distinct slots; null records write nothing)
    auto write_phase = [&](auto st) {
      const float inv_mu = fast_rcp(mu_new);
#pragma unroll
      for (int k0 = 0; k0 < KP; k0 += NB) {
        Seg<CPL> x[NB], vq[NB];
        float dc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const uint32_t rx = wr[k0 + j].x;
          dc[j] = __uint_as_float(wr[k0 + j].y & 0x7fffffffu) * inv_mu;
          x[j] = lds_seg<CPL>(&A[(rx & 0xffffu) * CW + CPL * l8]);
          vq[j] = lds_seg<CPL>(&s_vc[((rx >> 16) & 63u) * CW + CPL * l8]);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
#pragma unroll
          for (int k = 0; k < CPL; ++k) x[j].v[k] = fmaf(dc[j], vq[j].v[k], x[j].v[k]);
          if (wr[k0 + j].y & 0x80000000u) {   // later writers of the slot in this chunk
            int e = wr[k0 + j].x >> 22;
            uint2 t;
            do {
              t = ext_at(e++, st);
              const float cf = __uint_as_float(t.x) * inv_mu;
              const Seg<CPL> vx = lds_seg<CPL>(&s_vc[(t.y & 63u) * CW + CPL * l8]);
#pragma unroll
              for (int k = 0; k < CPL; ++k) x[j].v[k] = fmaf(cf, vx.v[k], x[j].v[k]);
            } while (!(t.y & 0x80000000u));
          }
        }
        // lane l8's count update for record k0 + l8
        const uint2 ow = own_w[k0 / NB];
        const int mc = static_cast<int>(ow.x & 0xffffu);
        float dcc = __uint_as_float(ow.y & 0x7fffffffu) * inv_mu;
        if (ow.y & 0x80000000u) {
          int e = ow.x >> 22;
          uint2 t;
          do {
            t = ext_at(e++, st);
            dcc += __uint_as_float(t.x) * inv_mu;
          } while (!(t.y & 0x80000000u));
        }
        const float cold = cnt[mc];
#pragma unroll
        for (int j = 0; j < NB; ++j) {   // null records (row M) write nothing: no same-row write conflicts
          const int mj = static_cast<int>(wr[k0 + j].x & 0xffffu);
          if (mj != M) lds_seg_store<CPL>(&A[mj * CW + CPL * l8], x[j]);
        }
        if (mc != M) cnt[mc] = cold + dcc;
      }
    };
    if (all_staged) {
      write_phase(std::true_type{});
    } else {
      write_phase(std::false_type{});
    }
    if (more) stage(c + 1, fut);   // the other parity's buffers: free since the previous chunk's last barrier
    mu = mu_new;
    lds_barrier();
  };
  for (int c = 0; c < a.n_chunks; c += 2) {
    chunk(c, ra, rb);
    if (c + 1 >= a.n_chunks) break;
    chunk(c + 1, rb, ra);
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
// finish: 8 lanes per (token, head) row of dh float32 read-outs, 8 columns per lane and step (onorm_w nullptr: no
// norm, a copy in OutT)
template <typename OutT>
__global__ void __launch_bounds__(256) finish_kernel(const float* __restrict__ r, int64_t r_stride,
                                                     OutT* __restrict__ out, int64_t out_stride,
                                                     const float* __restrict__ onorm_w, int64_t rows, int H,
                                                     int dh, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 32 + (threadIdx.x >> 3);
  const int l8 = threadIdx.x & 7;
  const bool live = row < rows;   // every lane runs the cross-lane sum
  const int64_t n = live ? row / H : 0;
  const int h = live ? static_cast<int>(row - n * H) : 0;
  const float* src = r + n * r_stride + static_cast<int64_t>(h) * dh;
  constexpr int kMaxSteps = 8;    // dh <= 512
  float v[kMaxSteps][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxSteps; ++k) {
    const int c = 8 * l8 + 64 * k;
    if (live && c < dh) {
      const float4 x0 = *reinterpret_cast<const float4*>(src + c);
      const float4 x1 = *reinterpret_cast<const float4*>(src + c + 4);
      v[k][0] = x0.x; v[k][1] = x0.y; v[k][2] = x0.z; v[k][3] = x0.w;
      v[k][4] = x1.x; v[k][5] = x1.y; v[k][6] = x1.z; v[k][7] = x1.w;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
  ss = sum8(ss);
  if (!live) return;
  const float inv = onorm_w ? 1.f / sqrtf(ss / static_cast<float>(dh) + eps) : 1.f;
  OutT* dst = out + n * out_stride + static_cast<int64_t>(h) * dh;
#pragma unroll
  for (int k = 0; k < kMaxSteps; ++k) {
    const int c = 8 * l8 + 64 * k;
    if (c < dh) {
      float wv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f}, o[8];
      if (onorm_w) load_vals<8, float>(onorm_w + h * dh + c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[k][e] * inv * wv[e];
      store_vals<8, OutT>(dst + c, o);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// rms_norm: one wave per row; lanes take 8 consecutive values at a time
template <typename InT, typename OutT>
__global__ void __launch_bounds__(256) rms_norm_kernel(const InT* __restrict__ x, int64_t x_stride,
                                                       OutT* __restrict__ out, int64_t out_stride,
                                                       const float* __restrict__ w, int64_t rows, int d, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;   // whole waves
  const InT* src = x + row * x_stride;
  constexpr int kMax = 4;    // 8 * 64 * 4 = 2048 values per row in registers
  float v[kMax][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMax; ++k) {
    const int c = 8 * (lane + 64 * k);
    if (c < d) {
      load_vals<8, InT>(src + c, v[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  OutT* dst = out + row * out_stride;
#pragma unroll
  for (int k = 0; k < kMax; ++k) {
    const int c = 8 * (lane + 64 * k);
    if (c < d) {
      float wv[8];
      load_vals<8, float>(w + c, wv);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_f32(from_f32<InT>(v[k][e] * r)) * wv[e];   // .to(x.dtype) * w
      store_vals<8, OutT>(dst + c, o);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// decode step: one token per stream (the recurrence of forward_sequential, track4_onesdm_models.py:276-300)
//
// The state of stream b, head h is kept as (mem, cnt, scale): the true memory is scale * mem and the true counts
// scale * cnt.  A step (after an optional reset, which empties the memory) reads first, then fades the state by lam
// in O(1) (scale <- lam * scale) and adds its writes divided by the new scale; when the scale falls below 2^-60 (or
// to 0) the slab is multiplied by it once and the scale reset to 1.  So the cost of a step does not grow with the
// position.  One wave per (head, stream); lane l takes columns l, l + 64, ...
struct DecodeArgs {
  const int32_t* wslot;   // [B][H][pitch] write picks of this token (from the addressing)
  const float* wwt;       //   and their weights (gate included)
  const int32_t* rslot;   // read picks
  const float* rwt;
  const void* v;          // value rows (one per stream)
  int64_t v_stride;
  const float* decay;     // [H]
  const float* onorm_w;   // [H][dh]
  const uint8_t* reset;   // [B] or nullptr: 1 empties the stream's memory before it reads
  float* mem;             // [B][H][M][dh]
  float* cnt;             // [B][H][M]
  float* scale;           // [B][H]
  void* r_out;            // rows of H * dh (one per stream)
  int64_t r_stride;
  int out_bf16, H, dh, M, kk, pitch, read_mean, out_norm;
  float read_eps, out_norm_eps;
};

// the slab of one (stream, head) times f (0 empties it), float4 at a time; the caller fences
__device__ __forceinline__ void scale_slab(float* mem, float* cnt, int M, int dh, float f, int lane) {
  float4* m4 = reinterpret_cast<float4*>(mem);
  const int n4 = M * dh / 4;
  for (int i = lane; i < n4; i += 4 * 64) {
    float4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = i + 64 * u < n4 ? m4[i + 64 * u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i + 64 * u < n4) m4[i + 64 * u] = make_float4(x[u].x * f, x[u].y * f, x[u].z * f, x[u].w * f);
    }
  }
  for (int m = lane; m < M; m += 64) cnt[m] *= f;
}

template <typename VT, int KP>
__global__ void __launch_bounds__(64) decode_kernel(DecodeArgs a) {
  constexpr int kCols = 8;   // columns per lane: head_dim <= 512
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t sl = static_cast<int64_t>(b) * a.H + h;
  float* mem = a.mem + sl * a.M * a.dh;
  float* cnt = a.cnt + sl * a.M;
  const int kk = a.kk;
  // every load that does not depend on the state first, all issued together: the picks (pads: slot -1 read as
  // row 0 with weight 0; the weights of picks past kk are masked after the load), the value row, the scale, the
  // fade, the reset flag and the out-norm weights.  Loads stay unconditional (indexes clamped, null arrays read a
  // stand-in word of the scales): a load under a branch would be waited for on its own.
  int rsl[KP], wsl[KP];
  float rwv[KP], wwv[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    rsl[j] = max(a.rslot[sl * KP + j], 0);
    const float rw = a.rwt[sl * KP + j];
    rwv[j] = j < kk ? rw : 0.f;
    wsl[j] = max(a.wslot[sl * KP + j], 0);
    const float ww = a.wwt[sl * KP + j];
    wwv[j] = j < kk ? ww : 0.f;
  }
  const VT* vrow = static_cast<const VT*>(a.v) + static_cast<int64_t>(b) * a.v_stride + static_cast<int64_t>(h) * a.dh;
  float vv[kCols], onw[kCols];
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    const int cc = min(c, a.dh - 1);
    const float v0 = to_f32(vrow[cc]);
    vv[q] = c < a.dh ? v0 : 0.f;
    const float w0 = *(a.out_norm ? a.onorm_w + h * a.dh + cc : a.scale + sl);
    onw[q] = a.out_norm ? w0 : 1.f;
  }
  float mu = a.scale[sl];
  const float lam = a.decay[h];
  const uint8_t rst = *(a.reset ? a.reset + b : reinterpret_cast<const uint8_t*>(a.scale + sl));
  if (a.reset && rst) {   // a document starts here: the memory is emptied before the read
    scale_slab(mem, cnt, a.M, a.dh, 0.f, lane);
    mu = 1.f;
    __threadfence_block();
    __syncthreads();
  }
  // read: mu * sum_j wr_j * mem[sir_j], mu * sum_j wr_j * cnt[sir_j] (track4_onesdm_models.py:290-293); the rows
  // of all picks are loaded at once
  float acc[kCols];
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    acc[q] = 0.f;
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float row[KP];
#pragma unroll
      for (int j = 0; j < KP; ++j) row[j] = mem[static_cast<int64_t>(rsl[j]) * a.dh + c];   // weight 0 past kk
#pragma unroll
      for (int j = 0; j < KP; ++j) acc[q] = fmaf(rwv[j], row[j], acc[q]);
    }
  }
  float cr[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) cr[j] = cnt[rsl[j]];
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < KP; ++j) den = fmaf(rwv[j], cr[j], den);
  // finish (:243-246, without wo): mean read, then the per-head output norm
  const float dn = mu * den;
  const float rinv = a.read_mean ? 1.f / (dn + a.read_eps) : 1.f;
  float r[kCols];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    r[q] = c < a.dh ? (a.read_mean ? (mu * acc[q]) * rinv : mu * acc[q]) : 0.f;
    ss = fmaf(r[q], r[q], ss);
  }
  float on = 1.f;
  if (a.out_norm) {   // the wave sum: rows of 16 lanes by DPP, then the four row sums
    float s16 = sum8(ss);
    s16 += dpp_f<0x140>(s16);   // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s16), 48));
    ss = (r0 + r1) + (r2 + r3);
    on = rsqrtf(ss / static_cast<float>(a.dh) + a.out_norm_eps);
  }
#pragma unroll
  for (int q = 0; q < kCols; ++q) {
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float o = r[q];
      if (a.out_norm) o = o * on * onw[q];
      const int64_t at = static_cast<int64_t>(b) * a.r_stride + static_cast<int64_t>(h) * a.dh + c;
      if (a.out_bf16) static_cast<bf16_t*>(a.r_out)[at] = from_f32<bf16_t>(o);
      else static_cast<float*>(a.r_out)[at] = o;
    }
  }
  // fade (O(1) through the scale; rescale the slab when the scale gets small), then write (:294-298)
  float mu2 = mu * lam;
  if (!(mu2 >= kMuFloor)) {
    scale_slab(mem, cnt, a.M, a.dh, mu2, lane);
    mu2 = 1.f;
    __threadfence_block();
    __syncthreads();
  }
  const float inv = 1.f / mu2;
#pragma unroll
  for (int q = 0; q < kCols; ++q) {   // the picks of one token are distinct slots
    const int c = lane + 64 * q;
    if (c < a.dh) {
      float old[KP];
#pragma unroll
      for (int j = 0; j < KP; ++j) old[j] = mem[static_cast<int64_t>(wsl[j]) * a.dh + c];   // stored only below kk
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        if (j < kk) mem[static_cast<int64_t>(wsl[j]) * a.dh + c] = fmaf(wwv[j] * inv, vv[q], old[j]);
      }
    }
  }
  if (lane == 0) {
    float oc[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) oc[j] = cnt[wsl[j]];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j < kk) cnt[wsl[j]] = oc[j] + wwv[j] * inv;
    }
    a.scale[sl] = mu2;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// table read: the weighted sum of the picked rows of per-head value tables (TrainedSdm.forward's embedding_bag,
// track4_onesdm_models.py:448-455): out[n][h * dh + c] = sum_j w[n][h][j] * values[h][slot[n][h][j]][c] in float32,
// picks in order.  One wave per (token, head); lane l takes columns 4l, 4l + 256, ... (dh a multiple of 4).
template <int KP, typename VT, typename OutT>
__global__ void __launch_bounds__(256) table_read_kernel(const int32_t* __restrict__ slots,
                                                         const float* __restrict__ wts,
                                                         const VT* __restrict__ values, OutT* __restrict__ out,
                                                         int64_t out_stride, int B, int T, int H, int M, int dh,
                                                         int kk) {
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= static_cast<int64_t>(B) * T * H) return;   // whole waves
  const int64_t n = wave / H;
  const int h = static_cast<int>(wave - n * H);
  const int b = static_cast<int>(n / T);
  const int t = static_cast<int>(n - static_cast<int64_t>(b) * T);
  const int64_t pb = ((static_cast<int64_t>(b) * H + h) * T + t) * KP;
  int sl[KP];
  float w[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    sl[j] = min(max(slots[pb + j], 0), M - 1);   // pads (-1) and stray ids stay inside the table
    w[j] = j < kk ? wts[pb + j] : 0.f;
  }
  const VT* tab = values + static_cast<int64_t>(h) * M * dh;
  for (int c0 = 4 * lane; c0 < dh; c0 += 256) {
    float v[KP][4];
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      if (j < kk) {
        load_vals<4, VT>(tab + static_cast<int64_t>(sl[j]) * dh + c0, v[j]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[j][e] = 0.f;
      }
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KP; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(w[j], v[j][e], acc[e]);
    }
    store_vals<4, OutT>(out + n * out_stride + static_cast<int64_t>(h) * dh + c0, acc);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// host side
struct Plan {
  int B, T, H, dh, d_a, half, n_sub, M, k, c1, kk, pitch, cap, n_chunks;
  // workspace offsets
  size_t off_sizes, off_plans, off_rtmp, total;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// core: the shape must suit the scan and the decode step too (head_dim); the addressing alone needs only the keys
int make_plan(const sdm_rt_dims* d, Plan* p, bool core = true) {
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
  if (!core) return SDM_RT_OK;
  if (scan_lds_bytes(p->M, p->pitch, 8, p->n_chunks) > kLdsBytes)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations and T = %d do not fit a slab of 8 columns in LDS", p->M,
                   p->T);
  if (plan_static_lds(p->pitch) + 8 * static_cast<size_t>(p->M) + 8 * static_cast<size_t>(p->n_sub) * p->half + 256 >
      kLdsBytes)
    return set_err(SDM_RT_EUNSUPPORTED, "M = %d locations: writer masks and sub-keys do not fit in LDS", p->M);
  const size_t tok = static_cast<size_t>(p->B) * p->T;
  const size_t n_plans = static_cast<size_t>(p->B) * p->H * p->n_chunks;
  size_t o = 0;
  p->off_sizes = o;
  o = align_up(o + sizeof(int32_t) * n_plans, 256);
  p->off_plans = o;
  o = align_up(o + static_cast<size_t>(PlanGeom{p->pitch}.stride()) * n_plans, 256);
  p->off_rtmp = o;
  o = align_up(o + (d->out_norm ? sizeof(float) * tok * p->H * p->dh : 0), 256);
  p->total = o;
  return SDM_RT_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_err(SDM_RT_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return SDM_RT_OK;
}

// lets a kernel use all the LDS its static arrays leave free for dynamic LDS (once per kernel and process)
bool allow_lds(const void* fn) {
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess || fa.sharedSizeBytes > kLdsBytes) return false;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(kLdsBytes - fa.sharedSizeBytes)) == hipSuccess;
}
int lds_err(const char* what) { return set_err(SDM_RT_ELAUNCH, "%s: cannot enable %zu bytes of LDS", what, kLdsBytes); }

AddrGeom addr_geom(const Plan& p, const sdm_rt_params* prm) {
  AddrGeom g;
  g.keys[0] = prm->keys1;
  g.keys[1] = prm->keys2;
  g.addr_b = prm->addr_b;
  g.log_scale = prm->log_scale;
  g.gate_bias = prm->gate_bias;
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
bool use_mf(const Plan& p) { return mf_half(p.half) && p.n_sub <= 32; }
// no masked candidate: 32 sub-keys per half and 8 picks from the top 8 of each half
bool full_grid(const Plan& p) { return use_mf(p) && p.n_sub == 32 && p.c1 == 8 && p.kk == 8; }

template <int HALF, typename InT>
struct AddressLaunch {
  template <int CAP, int MODE>
  static void go(const Plan& p, const AddrArgs& a, hipStream_t st) {
    const int64_t N = static_cast<int64_t>(p.B) * p.T;
    dim3 grid(static_cast<unsigned>((N + 63) / 64), p.H, a.z2 ? 2 : 1);
    const size_t lds = MODE > 0 ? 0 : sizeof(float) * 2 * p.n_sub * HALF;
    hipLaunchKernelGGL((address_kernel<HALF, CAP, InT, MODE>), grid, dim3(64), lds, st, a);
  }
  static int run(const Plan& p, const AddrArgs& a, hipStream_t st) {
    if constexpr (mf_half(HALF)) {
      if (use_mf(p)) {
        if (full_grid(p)) go<8, 2>(p, a, st);
        else if (p.cap == 8) go<8, 1>(p, a, st);
        else go<16, 1>(p, a, st);
        return check_launch("address");
      }
    }
    if (p.cap == 8) go<8, 0>(p, a, st);
    else go<16, 0>(p, a, st);
    return check_launch("address");
  }
};

template <int HALF, typename InT>
struct PlanLaunch {
  template <int KP, int MODE>
  static int go(const Plan& p, const PlanArgs& a, hipStream_t st) {
    dim3 grid(p.n_chunks, p.H, p.B);
    const size_t lds = sizeof(unsigned long long) * p.M + (MODE > 0 ? 0 : sizeof(float) * 2 * p.n_sub * HALF);
    static const bool ok = allow_lds(reinterpret_cast<const void*>(&plan_kernel<HALF, KP, InT, MODE>));
    if (!ok) return lds_err("plan");
    hipLaunchKernelGGL((plan_kernel<HALF, KP, InT, MODE>), grid, dim3(128), lds, st, a);
    return check_launch("plan");
  }
  static int run(const Plan& p, const PlanArgs& a, hipStream_t st) {
    if constexpr (mf_half(HALF)) {
      if (use_mf(p)) return full_grid(p) ? go<8, 2>(p, a, st) : p.pitch == 8 ? go<8, 1>(p, a, st) : go<16, 1>(p, a, st);
    }
    return p.pitch == 8 ? go<8, 0>(p, a, st) : go<16, 0>(p, a, st);
  }
};

template <int CW, int KP, typename VT, typename OutT>
int launch_scan_t(const Plan& p, const ScanArgs& a, hipStream_t st) {
  const size_t lds = scan_lds_bytes(p.M, KP, CW, p.n_chunks);
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

// widest column group per scan workgroup (32, 16 or 8 value columns) whose slab, plan and values fit in LDS
template <typename VT>
int scan_columns(const Plan& p) {
  for (int cw : {32, 16, 8})
    if (p.dh % cw == 0 && scan_lds_bytes(p.M, p.pitch, cw, p.n_chunks) <= kLdsBytes) return cw;
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

int check_params(const sdm_rt_params* prm, bool need_onorm, bool need_decay = true) {
  if (!prm) return set_err(SDM_RT_EINVAL, "params is NULL");
  if (!prm->keys1 || !prm->keys2) return set_err(SDM_RT_EINVAL, "keys1/keys2 must not be NULL");
  if (!prm->log_scale) return set_err(SDM_RT_EINVAL, "log_scale must not be NULL");
  if (need_decay && !prm->decay) return set_err(SDM_RT_EINVAL, "decay must not be NULL");
  if (need_onorm && !prm->onorm_w) return set_err(SDM_RT_EINVAL, "onorm_w must not be NULL when out_norm is set");
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
  if (make_plan(dims, &p, false) != SDM_RT_OK) return 0;
  return p.pitch;
}

const char* sdm_rt_last_error(void) { return g_err; }

int sdm_rt_rms_norm(const void* x, int64_t x_row_stride, sdm_rt_dtype in_dtype, int64_t rows, int32_t d,
                    const float* w, float eps, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                    void* stream) {
  g_err[0] = 0;
  int rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (rows < 0 || d < 1) return set_err(SDM_RT_EINVAL, "rows must be >= 0 and d >= 1");
  if (d % 8 != 0 || d > 2048) return set_err(SDM_RT_EUNSUPPORTED, "d = %d must be a multiple of 8 up to 2048", d);
  if (rows == 0) return SDM_RT_OK;
  if (!x || !w || !out) return set_err(SDM_RT_EINVAL, "x, w and out must not be NULL");
  if (x_row_stride < d || out_row_stride < d) return set_err(SDM_RT_EINVAL, "row strides must be >= d");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
#define SDM_RT_NORM(IT, OT)                                                                                     \
  hipLaunchKernelGGL((rms_norm_kernel<IT, OT>), dim3(blocks), dim3(256), 0, st, static_cast<const IT*>(x),      \
                     x_row_stride, static_cast<OT*>(out), out_row_stride, w, rows, d, eps)
  if (in_dtype == SDM_RT_BF16) {
    if (out_dtype == SDM_RT_BF16) SDM_RT_NORM(bf16_t, bf16_t);
    else SDM_RT_NORM(bf16_t, float);
  } else {
    if (out_dtype == SDM_RT_BF16) SDM_RT_NORM(float, bf16_t);
    else SDM_RT_NORM(float, float);
  }
#undef SDM_RT_NORM
  return check_launch("rms_norm");
}

int sdm_rt_address(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* z, int64_t z_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, int32_t* slot_out,
                   float* score_out, float* weight_out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if ((rc = check_params(params, false, false))) return rc;
  if ((rc = check_dtype(in_dtype, "in_dtype"))) return rc;
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!z || !slot_out) return set_err(SDM_RT_EINVAL, "z and slot_out must not be NULL");
  if (z_row_stride < static_cast<int64_t>(p.H) * p.d_a)
    return set_err(SDM_RT_EINVAL, "z_row_stride %lld < heads * addr_dim", (long long)z_row_stride);
  if (gate_logits && gate_row_stride < p.H)
    return set_err(SDM_RT_EINVAL, "gate_row_stride %lld < heads", (long long)gate_row_stride);
  (void)workspace;   // the addressing alone needs no workspace
  (void)workspace_bytes;
  hipStream_t st = static_cast<hipStream_t>(stream);
  AddrArgs a{};
  a.g = addr_geom(p, params);
  a.z = z;
  a.z_stride = z_row_stride;
  a.gl = gate_logits;
  a.g_stride = gate_row_stride;
  a.B = p.B;
  a.T = p.T;
  a.pitch = p.pitch;
  a.slot_out = slot_out;
  a.w_out = weight_out;
  a.s_out = score_out;
  return in_dtype == SDM_RT_BF16 ? by_half<AddressLaunch, bf16_t>(p.half, p, a, st)
                                 : by_half<AddressLaunch, float>(p.half, p, a, st);
}

int sdm_rt_forward(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                   const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                   const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype, const uint8_t* reset,
                   void* r_out,
                   int64_t out_row_stride, sdm_rt_dtype out_dtype, const float* state_in_mem,
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
  int32_t* sizes = reinterpret_cast<int32_t*>(ws + p.off_sizes);
  unsigned char* plans = reinterpret_cast<unsigned char*>(ws + p.off_plans);
  float* rtmp = reinterpret_cast<float*>(ws + p.off_rtmp);

  PlanArgs pa{};
  pa.g = addr_geom(p, params);
  pa.kz = kz;
  pa.kz_stride = kz_row_stride;
  pa.qz = qz;
  pa.qz_stride = qz_row_stride;
  pa.gl = dims->write_gate ? gate_logits : nullptr;
  pa.g_stride = gate_row_stride;
  pa.decay = params->decay;
  pa.reset = reset;
  pa.plans = plans;
  pa.sizes = sizes;
  pa.B = p.B;
  pa.T = p.T;
  pa.M = p.M;
  pa.n_chunks = p.n_chunks;
  rc = in_dtype == SDM_RT_BF16 ? by_half<PlanLaunch, bf16_t>(p.half, p, pa, st)
                               : by_half<PlanLaunch, float>(p.half, p, pa, st);
  if (rc) return rc;

  ScanArgs s{};
  s.plans = plans;
  s.sizes = sizes;
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
  s.n_chunks = p.n_chunks;
  s.read_mean = dims->read_mean;
  s.read_eps = dims->read_eps;
  if (dims->out_norm) {
    s.r_out = rtmp;
    s.r_stride = static_cast<int64_t>(p.H) * p.dh;
    if ((rc = launch_scan(p, s, in_dtype, SDM_RT_F32, st))) return rc;
    const int64_t rows = static_cast<int64_t>(p.B) * p.T * p.H;
    const unsigned blocks = static_cast<unsigned>((rows + 31) / 32);
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

int sdm_rt_table_read(const sdm_rt_dims* dims, const int32_t* slots, const float* weights, const void* values,
                      sdm_rt_dtype values_dtype, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                      void* stream) {
  g_err[0] = 0;
  Plan p;
  int rc = make_plan(dims, &p, false);
  if (rc) return rc;
  if ((rc = check_dtype(values_dtype, "values_dtype"))) return rc;
  if ((rc = check_dtype(out_dtype, "out_dtype"))) return rc;
  if (p.dh < 4 || p.dh % 4 != 0) return set_err(SDM_RT_EUNSUPPORTED, "head_dim %d must be a positive multiple of 4", p.dh);
  if (p.B == 0 || p.T == 0) return SDM_RT_OK;
  if (!slots || !weights || !values || !out) return set_err(SDM_RT_EINVAL, "slots, weights, values and out must not be NULL");
  if (out_row_stride < static_cast<int64_t>(p.H) * p.dh)
    return set_err(SDM_RT_EINVAL, "out_row_stride %lld < heads * head_dim", (long long)out_row_stride);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t waves = static_cast<int64_t>(p.B) * p.T * p.H;
  const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
#define SDM_RT_TABLE(KP, VT, OT)                                                                                   \
  hipLaunchKernelGGL((table_read_kernel<KP, VT, OT>), dim3(blocks), dim3(256), 0, st, slots, weights,             \
                     static_cast<const VT*>(values), static_cast<OT*>(out), out_row_stride, p.B, p.T, p.H, p.M, p.dh, \
                     p.kk)
#define SDM_RT_TABLE_KP(VT, OT) \
  if (p.pitch == 8) SDM_RT_TABLE(8, VT, OT); else SDM_RT_TABLE(16, VT, OT)
  if (values_dtype == SDM_RT_BF16) {
    if (out_dtype == SDM_RT_BF16) { SDM_RT_TABLE_KP(bf16_t, bf16_t); } else { SDM_RT_TABLE_KP(bf16_t, float); }
  } else {
    if (out_dtype == SDM_RT_BF16) { SDM_RT_TABLE_KP(float, bf16_t); } else { SDM_RT_TABLE_KP(float, float); }
  }
#undef SDM_RT_TABLE_KP
#undef SDM_RT_TABLE
  return check_launch("table_read");
}

size_t sdm_rt_decode_workspace_bytes(const sdm_rt_dims* dims) {
  Plan p;
  if (make_plan(dims, &p) != SDM_RT_OK) return 0;
  return 2 * align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256) +
         2 * align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
}

int sdm_rt_decode_step(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* kz, int64_t kz_row_stride,
                       const void* qz, int64_t qz_row_stride, const void* v, int64_t v_row_stride,
                       const void* gate_logits, int64_t gate_row_stride, sdm_rt_dtype in_dtype,
                       const uint8_t* reset, float* state_mem, float* state_cnt, float* state_scale, void* r_out,
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
  char* ws = static_cast<char*>(workspace);
  const size_t si = align_up(sizeof(int32_t) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  const size_t sf = align_up(sizeof(float) * static_cast<size_t>(p.B) * p.H * p.pitch, 256);
  int32_t* wslot = reinterpret_cast<int32_t*>(ws);
  int32_t* rslot = reinterpret_cast<int32_t*>(ws + si);
  float* wwt = reinterpret_cast<float*>(ws + 2 * si);
  float* rwt = reinterpret_cast<float*>(ws + 2 * si + sf);
  // the picks of this token, [B][H][1][pitch]: write keys (gated) and read queries, in one launch
  AddrArgs aa{};
  aa.g = addr_geom(p, params);
  aa.B = p.B;
  aa.T = 1;
  aa.pitch = p.pitch;
  aa.z = kz;
  aa.z_stride = kz_row_stride;
  aa.gl = dims->write_gate ? gate_logits : nullptr;
  aa.g_stride = gate_row_stride;
  aa.slot_out = wslot;
  aa.w_out = wwt;
  aa.z2 = qz;
  aa.z2_stride = qz_row_stride;
  aa.slot_out2 = rslot;
  aa.w_out2 = rwt;
  rc = in_dtype == SDM_RT_BF16 ? by_half<AddressLaunch, bf16_t>(p.half, p, aa, st)
                               : by_half<AddressLaunch, float>(p.half, p, aa, st);
  if (rc) return rc;
  DecodeArgs da{};
  da.wslot = wslot;
  da.wwt = wwt;
  da.rslot = rslot;
  da.rwt = rwt;
  da.v = v;
  da.v_stride = v_row_stride;
  da.decay = params->decay;
  da.onorm_w = params->onorm_w;
  da.reset = reset;
  da.mem = state_mem;
  da.cnt = state_cnt;
  da.scale = state_scale;
  da.r_out = r_out;
  da.r_stride = out_row_stride;
  da.out_bf16 = out_dtype == SDM_RT_BF16;
  da.H = p.H;
  da.dh = p.dh;
  da.M = p.M;
  da.kk = p.kk;
  da.pitch = p.pitch;
  da.read_mean = dims->read_mean;
  da.out_norm = dims->out_norm;
  da.read_eps = dims->read_eps;
  da.out_norm_eps = dims->out_norm_eps;
  dim3 grid(p.H, p.B);
#define SDM_RT_DECODE(VT, KP) hipLaunchKernelGGL((decode_kernel<VT, KP>), grid, dim3(64), 0, st, da)
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

// the backward (forward with saved tensors, sdm_rt_backward)
#include "sdm_rt_grad.inc"
