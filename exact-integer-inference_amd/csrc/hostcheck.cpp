// Host build of the integer helpers in eii_int.h, exported for CPU tests: the same source the
// kernels compile, checked on the CPU against exact Python integers.
#include <stdint.h>

#include "eii_int.h"

extern "C" {
int64_t eii_host_rs(int64_t x, int n) { return eii::rs(x, n); }
int64_t eii_host_sat(int64_t x, int bits) { return eii::sat(x, bits); }
int64_t eii_host_norm_U(int64_t A, int64_t B, int64_t C) { return eii::norm_U(eii::norm_total(A, B, C)); }
int64_t eii_host_attn_prob(int64_t e, int64_t Z) { return eii::attn_prob(e, Z, 1.0 / (double)Z); }
int64_t eii_host_div_floor_q20(int64_t num, int64_t den) { return eii::div_floor_q20(num, den, 1.0 / (double)den); }
// sum_k a_k w_k through the limb split of width W bytes (2 or 4), for a [K], w [K]
int64_t eii_host_limb_dot(const int32_t* a, const int8_t* w, int K, int W) {
  int32_t P[4] = {0, 0, 0, 0};
  int64_t wsum = 0;
  for (int k = 0; k < K; ++k) {
    int8_t p[4];
    eii::split_limbs(a[k], W, p);
    for (int i = 0; i < W; ++i) P[i] += (int32_t)p[i] * (int32_t)w[k];
    wsum += w[k];
  }
  return eii::limb_combine(P, W, wsum);
}
}
