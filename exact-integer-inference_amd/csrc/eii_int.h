// Exact integer helpers of the integer semantics, usable on host and device.
//
// Every function here returns the integer the reference defines; floating point appears
// only as a seed for an exact integer search whose result is verified by an integer
// inequality, so no result depends on float rounding.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define EII_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define EII_HD static inline
#endif

namespace eii {

constexpr int kV = 49152, kD = 576, kDFF = 1536, kNH = 9, kNKV = 3, kHD = 64, kNL = 30;
constexpr int kDMax = 12 * 128;          // python/intref.py:35
constexpr int kFRes = 15, kFScore = 7;   // python/intref.py:33-34
constexpr int64_t kEpsS = 6184753;       // python/intref.py:37
constexpr int kRIsqrt = 40;              // python/intref.py:38
constexpr int kQKVN = kD + 2 * kNKV * kHD;   // 960 = q | k | v output columns

// RS(x, n): n >= 1 -> (x + 2^(n-1)) >> n with an arithmetic shift (ties toward +inf);
// n <= 0 -> exact x * 2^-n (python/intref.py:42-50, c/intref.c:29-32).
EII_HD int64_t rs(int64_t x, int n) {
  if (n <= 0) return x * ((int64_t)1 << (-n));
  return (x + ((int64_t)1 << (n - 1))) >> n;
}

// SAT(x, bits): clip to [-2^(bits-1), 2^(bits-1) - 1]; bits >= 64 is no clip (c/intref.c:33-37).
EII_HD int64_t sat(int64_t x, int bits) {
  if (bits >= 64) return x;
  const int64_t hi = ((int64_t)1 << (bits - 1)) - 1, lo = -((int64_t)1 << (bits - 1));
  return x < lo ? lo : (x > hi ? hi : x);
}

EII_HD int64_t clamp_bits16(int64_t x) { return x < -32768 ? -32768 : (x > 32767 ? 32767 : x); }
EII_HD int64_t clamp_bits32(int64_t x) {
  return x < -2147483648LL ? -2147483648LL : (x > 2147483647LL ? 2147483647LL : x);
}

// Reciprocal root of the RMSNorm (python/intref.py:170-177, c/intref.c:96-104):
// with S = A*2^32 + B*2^17 + C = sum x^2 (A = sum hi^2, B = sum hi*lo, C = sum lo^2 over the
// 16-bit halves hi = x >> 16, lo = x & 0xFFFF) and Tt = S + EPS_S,
//   U = isqrt(floor(2^80 / Tt)).
// Since isqrt(floor(y)) = floor(sqrt(y)), U is the largest u >= 0 with u^2 * Tt <= 2^80.  A
// float64 estimate of 2^40 / sqrt(Tt) is within one unit of U (relative error below 2^-48 on a
// value below 2^29); the integer loops below then move u to the unique integer with
//   u^2 * Tt <= 2^80 < (u + 1)^2 * Tt,
// evaluated exactly with 64 x 64 -> 128-bit products.
typedef unsigned __int128 u128;

EII_HD u128 norm_total(int64_t A, int64_t B, int64_t C) {
  // A >= 0 and C >= 0 always; B is signed. The true S is >= 0.
  __int128 S = ((__int128)A << 32) + ((__int128)B << 17) + (__int128)C;
  return (u128)(S + kEpsS);
}

#if defined(__HIPCC__)
EII_HD uint64_t umulhi64(uint64_t a, uint64_t b) { return __umul64hi(a, b); }
#else
EII_HD uint64_t umulhi64(uint64_t a, uint64_t b) { return (uint64_t)(((u128)a * b) >> 64); }
#endif

// u^2 * Tt <= 2^80 for u < 2^31 and Tt = t_hi 2^64 + t_lo < 2^74, in 64-bit pieces:
// p Tt = p t_hi 2^64 + p t_lo with p = u^2 < 2^62.
EII_HD bool norm_fits(uint64_t u, u128 Tt) {
  const uint64_t p = u * u;
  const uint64_t t_hi = (uint64_t)(Tt >> 64), t_lo = (uint64_t)Tt;
  const uint64_t ph = p * t_hi;
  if (umulhi64(p, t_hi) != 0 || ph > ((uint64_t)1 << 16)) return false;   // p t_hi 2^64 > 2^80
  const uint64_t top = ph + umulhi64(p, t_lo);                              // floor(p Tt / 2^64)
  if (top != ((uint64_t)1 << 16)) return top < ((uint64_t)1 << 16);
  return p * t_lo == 0;
}

// The float64 estimate is within one of U (see above), so U is u - 1, u or u + 1 for
// u = floor(estimate); the loops also cover any larger miss.  Below 2^31 the estimate's absolute
// error is under 2^-17 (relative error below 2^-48), so when its fractional part lies more than
// 2^-16 from 0 and from 1, no integer separates it from 2^40 / sqrt(Tt) and its floor is U without
// the exact tests (which then only run for estimates next to an integer).
EII_HD int64_t norm_U(u128 Tt) {
  const double td = (double)(uint64_t)(Tt >> 64) * 18446744073709551616.0 + (double)(uint64_t)Tt;
  double ue = 1099511627776.0 / sqrt(td);           // 2^40 / sqrt(Tt)
  if (ue > 2147483647.0) ue = 2147483647.0;
  const double fl = floor(ue), fr = ue - fl;
  if (fr > 0x1p-16 && fr < 1.0 - 0x1p-16) return (int64_t)fl;
  uint64_t u = (uint64_t)ue;
  for (int it = 0; it < 64 && u > 0 && !norm_fits(u, Tt); ++it) --u;
  for (int it = 0; it < 64 && norm_fits(u + 1, Tt); ++it) ++u;
  return (int64_t)u;
}

// floor(num / den) for 0 <= num < 2^53, 1 <= den < 2^53 and a quotient below 2^20, given
// rden = 1.0 / (double)den.  The float64 quotient is within 2^-30 of the true one, so its
// truncation is off by at most one; the remainder test corrects it exactly.
EII_HD int64_t div_floor_q20(int64_t num, int64_t den, double rden) {
  int64_t q = (int64_t)((double)num * rden);
  const int64_t r = num - q * den;
  if (r < 0) q -= 1;
  else if (r >= den) q += 1;
  return q;
}

// Attention probability (python/intref.py:245-246, c/intref.c:180):
//   P = floor((e * 65536 + floor(Z / 2)) / Z), 0 <= e <= Z, Z >= 2^30; P <= 65536.
EII_HD int64_t attn_prob(int64_t e, int64_t Z, double rZ) {
  return div_floor_q20(e * 65536 + (Z >> 1), Z, rZ);
}

}  // namespace eii

namespace eii {

// ---------------------------------------------------------------- int8 limbs
// A signed activation a of W bytes (W = 2 or 4) is held as W int8 limb planes p_0..p_{W-1}:
//   p_{W-1} = a >> 8(W-1) (signed top byte), p_i = byte_i(a) - 128 for i < W-1, so
//   a = p_{W-1} * 256^(W-1) + sum_{i<W-1} (p_i + 128) * 256^i.
// For int8 weights w, sum_k a_k w_k = sum_i 256^i * P_i + limb_bias(W) * sum_k w_k with
// P_i = sum_k p_{i,k} w_k, each |P_i| <= 128 * 127 * K < 2^31 for K <= 2^17.
EII_HD int64_t limb_bias(int W) { return W == 2 ? 128 : 128LL * (1 + 256 + 65536); }

EII_HD int64_t limb_combine(const int32_t* P, int W, int64_t wsum) {
  int64_t acc = limb_bias(W) * wsum;
  for (int i = 0; i < W; ++i) acc += (int64_t)P[i] * ((int64_t)1 << (8 * i));
  return acc;
}

EII_HD void split_limbs(int32_t a, int W, int8_t* p) {
  for (int i = 0; i < W - 1; ++i) p[i] = (int8_t)(((a >> (8 * i)) & 0xFF) ^ 0x80);
  p[W - 1] = (int8_t)(a >> (8 * (W - 1)));
}

}  // namespace eii
