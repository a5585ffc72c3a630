// Host build of the integer helpers in eii_int.h and of the kernels' index maps (index_maps.h),
// exported for CPU tests: the same source the kernels compile, checked on the CPU against exact
// Python integers and a CPU model of the kernels' data movement.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "eii_int.h"
#include "index_maps.h"

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

// ---------------------------------------------------------------------------------------------
// CPU model of the GEMM and attention index maps (index_maps.h, the functions the kernels use).
// v_mfma_i32_32x32x32_i8 is modelled from its documented operand and result layouts (idx::mfma_row);
// everything else runs the kernels' own index functions.
namespace {

using namespace eii;
using namespace eii::idx;

// D += A B over 32 x 32 x 32 int8 operands given as the 64 lanes' 16-byte fragments
void mfma_model(const int8_t (*A)[16], const int8_t (*B)[16], int32_t (*D)[16]) {
  for (int lane = 0; lane < 64; ++lane) {
    const int h = lane >> 5, c = lane & 31;
    for (int e = 0; e < 16; ++e) {
      const int i = mfma_row(e, h);
      int32_t s = 0;
      for (int k = 0; k < 32; ++k) s += (int32_t)A[32 * (k >> 4) + i][k & 15] * (int32_t)B[32 * (k >> 4) + c][k & 15];
      D[lane][e] += s;
    }
  }
}

uint64_t next_rand(uint64_t& st) {
  st = st * 6364136223846793005ULL + 1442695040888963407ULL;
  return st >> 33;
}

// stats: [0] tiles, [1] wrong limb sums, [2] accesses out of bounds (global, LDS), [3] LDS slots
// written twice or read unwritten, [4] output elements stored != once, [5] elements compared.
// plant (tests only): 1 = fragment reads ignore the LDS swizzle, 2 = the result row map is off by
// one row group, 3 = the skinny K split drops the last slice of wave 3.
template <int AW, int SHAPE>
void model_gemm(int M, int N, int K, int a_kb, uint64_t seed, int plant, int64_t* st) {
  using C = GemmCfg<AW, SHAPE>;
  const int ksl = K / 32, nb32_last = (N + 31) / 32 - 1;
  const size_t a_plane = (size_t)M * K, a_bytes = AW * a_plane;
  const size_t w_bytes = (size_t)(nb32_last + 1) * 32 * K;
  std::vector<int8_t> logical(a_bytes), planes(a_bytes), W((size_t)N * K), Wf(w_bytes, 0);
  uint64_t r = seed;
  for (auto& b : logical) b = (int8_t)next_rand(r);
  for (auto& b : W) b = (int8_t)next_rand(r);
  for (int l = 0; l < AW; ++l)
    for (int m = 0; m < M; ++m)
      for (int k = 0; k < K; ++k)
        planes[l * a_plane + (a_kb == 32 ? plane_offset32(m, k, M) : plane_offset(m, k, M))] =
            logical[(l * (size_t)M + m) * K + k];
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) Wf[w_fo_offset(n, k, ksl)] = W[(size_t)n * K + k];
  auto expect = [&](int l, int m, int n) {
    int32_t s = 0;
    for (int k = 0; k < K; ++k) s += (int32_t)logical[(l * (size_t)M + m) * K + k] * (int32_t)W[(size_t)n * K + k];
    return s;
  };
  std::vector<int> stored((size_t)M * N, 0);
  const int nMB = (M + C::BM - 1) / C::BM, nNB = (N + C::BN - 1) / C::BN;
  int8_t Af[64][16], Bf[64][16];
  auto rowmap = [&](int e, int h) { return plant == 2 ? mfma_row(e ^ 4, h) : mfma_row(e, h); };
  // the epilogue's element map over one wave's results (wave grid position wm, wn)
  auto epilogue = [&](int m0, int n0, int wm, int wn, std::vector<int32_t>& acc) {
    for (int lane = 0; lane < 64; ++lane)
      for (int tm = 0; tm < C::TM; ++tm)
        for (int tn = 0; tn < C::TN; ++tn)
          for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm * C::WM + 32 * tm + rowmap(e, lane >> 5), col = n0 + wn * C::WN + 32 * tn + (lane & 31);
            if (row >= M || col >= N) continue;
            ++stored[(size_t)row * N + col];
            for (int l = 0; l < AW; ++l) {
              ++st[5];
              if (acc[((((size_t)tm * C::TN + tn) * AW + l) * 64 + lane) * 16 + e] != expect(l, row, col)) ++st[1];
            }
          }
  };
  const size_t acc_n = (size_t)C::TM * C::TN * AW * 64 * 16;
  for (int mb = 0; mb < nMB; ++mb)
    for (int nb = 0; nb < nNB; ++nb) {
      ++st[0];
      const int m0 = mb * C::BM, n0 = nb * C::BN;
      if constexpr (C::kSkinny) {
        // K slices split over the 4 waves, fragments straight from global memory, the 4 partial
        // sums added
        std::vector<int32_t> acc(acc_n, 0);
        const int NS = K / 32;
        for (int w = 0; w < 4; ++w) {
          const int s0 = w * NS / 4, cnt = (w + 1) * NS / 4 - s0 - (plant == 3 && w == 3 ? 1 : 0);
          for (int i = 0; i < cnt; ++i) {
            const int sl = s0 + i;
            for (int l = 0; l < AW; ++l) {
              for (int lane = 0; lane < 64; ++lane) {
                const int m = std::min(m0 + (lane & 31), M - 1);
                const size_t off = (size_t)l * a_plane + a_src_off(0, m, sl >> 1, 2 * (sl & 1) + (lane >> 5), M, a_kb, 0);
                if (off + 16 > a_bytes) { ++st[2]; memset(Af[lane], 0, 16); continue; }
                memcpy(Af[lane], &planes[off], 16);
              }
              for (int tn = 0; tn < C::TN; ++tn) {
                for (int lane = 0; lane < 64; ++lane) {
                  const size_t off = w_frag(std::min(nb * C::TN + tn, nb32_last), ksl, sl, lane);
                  if (off + 16 > w_bytes) { ++st[2]; memset(Bf[lane], 0, 16); continue; }
                  memcpy(Bf[lane], &Wf[off], 16);
                }
                mfma_model(Af, Bf, (int32_t(*)[16]) & acc[(((size_t)tn * AW + l) * 64) * 16]);
              }
            }
          }
        }
        epilogue(m0, n0, 0, 0, acc);
        continue;
      }
      std::vector<std::vector<int32_t>> acc(4, std::vector<int32_t>(acc_n, 0));
      std::vector<int8_t> lds(C::kStage);
      std::vector<int> written(C::kStage / 16);
      for (int kb = 0; kb < K / 64; ++kb) {
        // direct-to-LDS loads: chunk i of thread tid lands at stage byte 16 (tid + 256 i)
        std::fill(written.begin(), written.end(), 0);
        for (int tid = 0; tid < C::kThreads; ++tid)
          for (int i = 0; i < C::kAChunks; ++i) {
            const AChunk ch = a_chunk(tid + C::kThreads * i, C::BM);
            const int m = std::min(m0 + ch.row, M - 1);
            const size_t src = a_src_off(ch.l, m, kb, lds_swz(ch.row, ch.cp), M, a_kb, a_plane);
            const int slot = tid + C::kThreads * i;
            if (src + 16 > a_bytes || 16 * (slot + 1) > C::kStage) { ++st[2]; continue; }
            if (written[slot]++) ++st[3];
            memcpy(&lds[16 * slot], &planes[src], 16);
          }
        for (int wave = 0; wave < 4; ++wave) {
          const int wm = wave / C::WGN, wn = wave % C::WGN;
          for (int ks = 0; ks < 2; ++ks)
            for (int tm = 0; tm < C::TM; ++tm)
              for (int l = 0; l < AW; ++l) {
                for (int lane = 0; lane < 64; ++lane) {
                  const int row = wm * C::WM + tm * 32 + (lane & 31), kc = 2 * ks + (lane >> 5);
                  const int off = plant == 1 ? l * C::kPlane + row * kLdsRow + kc * 16 : a_frag(l, row, kc, C::kPlane);
                  if (off < 0 || off + 16 > C::kStage) { ++st[2]; memset(Af[lane], 0, 16); continue; }
                  if (!written[off / 16]) ++st[3];
                  memcpy(Af[lane], &lds[off], 16);
                }
                for (int tn = 0; tn < C::TN; ++tn) {
                  const int nb32 = std::min((n0 + wn * C::WN + 32 * tn) >> 5, nb32_last);
                  for (int lane = 0; lane < 64; ++lane) {
                    const size_t off = w_frag(nb32, ksl, 2 * kb + ks, lane);
                    if (off + 16 > w_bytes) { ++st[2]; memset(Bf[lane], 0, 16); continue; }
                    memcpy(Bf[lane], &Wf[off], 16);
                  }
                  mfma_model(Af, Bf, (int32_t(*)[16]) & acc[wave][((((size_t)tm * C::TN + tn) * AW + l) * 64) * 16]);
                }
              }
        }
      }
      for (int wave = 0; wave < 4; ++wave) epilogue(m0, n0, wave / C::WGN, wave % C::WGN, acc[wave]);
    }
  for (int v : stored)
    if (v != 1) ++st[4];
}

}  // namespace

extern "C" {
// CPU model of one GEMM launch over all its tiles (index maps of gemm_kernel); returns the number of
// errors (stats[1] + .. + stats[4]; stats holds the 6 counters of model_gemm), -1 for a shape the kernels do not
// instantiate.
int64_t eii_host_gemm_model(int aw, int shape, int M, int N, int K, int a_kb, uint64_t seed, int plant, int64_t* stats) {
  for (int i = 0; i < 6; ++i) stats[i] = 0;
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || (a_kb != 32 && a_kb != 64)) return -1;
#define EII_MODEL(A, S) model_gemm<A, S>(M, N, K, a_kb, seed, plant, stats)
  if (aw == 2) {
    switch (shape) {
      case kShapeSquare: EII_MODEL(2, kShapeSquare); break;
      case kShapeNarrow: EII_MODEL(2, kShapeNarrow); break;
      case kShapeRow: EII_MODEL(2, kShapeRow); break;
      case kShapeSkinny: EII_MODEL(2, kShapeSkinny); break;
      case kShapeSkinny32: EII_MODEL(2, kShapeSkinny32); break;
      default: return -1;
    }
  } else if (aw == 4) {
    switch (shape) {
      case kShapeSquare: EII_MODEL(4, kShapeSquare); break;
      case kShapeSkinny: EII_MODEL(4, kShapeSkinny); break;
      case kShapeSkinny32: EII_MODEL(4, kShapeSkinny32); break;
      default: return -1;
    }
  } else {
    return -1;
  }
#undef EII_MODEL
  return stats[1] + stats[2] + stats[3] + stats[4];
}

// Attention's key order and operand layouts: (1) attn_key_perm is a permutation of the 32 keys of a
// tile; (2) QK: with A row i = K[attn_key_perm(i)] and B column c = Q[c] (64 dims as 2 K slices of
// 32), result register j of lane 32 h + c is the score of key 16 h + j and query c; (3) PV: with
// those scores as the B bytes (byte j of lane 32 h + c = P[c][16 h + j]) and A row d = V^T[d]
// (bytes 16 h .. of row c: keys 16 h ..), result register e of lane 32 h + c is ctx[c][mfma_row(e, h)]
// (d as rows).  Returns the number of mismatches (plant 1: the key order without its row-group swap).
int64_t eii_host_attn_model(uint64_t seed, int plant) {
  int64_t bad = 0;
  int seen[32] = {0};
  auto perm = [&](int i) { return plant == 1 ? ((i >> 3) * 8 + (i & 7)) : attn_key_perm(i); };
  for (int i = 0; i < 32; ++i) ++seen[perm(i)];
  for (int i = 0; i < 32; ++i) bad += seen[i] != 1;
  uint64_t r = seed;
  int8_t Kt[32][64], Q[32][64], P[32][32], Vt[32][32];   // keys x d, queries x d, queries x keys, d x keys
  for (auto& row : Kt) for (auto& v : row) v = (int8_t)next_rand(r);
  for (auto& row : Q) for (auto& v : row) v = (int8_t)next_rand(r);
  for (auto& row : P) for (auto& v : row) v = (int8_t)next_rand(r);
  for (auto& row : Vt) for (auto& v : row) v = (int8_t)next_rand(r);
  int8_t Af[64][16], Bf[64][16];
  int32_t D[64][16] = {};
  for (int s = 0; s < 2; ++s) {
    for (int lane = 0; lane < 64; ++lane) {
      const int h = lane >> 5, c = lane & 31;
      for (int b = 0; b < 16; ++b) {
        Af[lane][b] = Kt[perm(c)][32 * s + 16 * h + b];
        Bf[lane][b] = Q[c][32 * s + 16 * h + b];
      }
    }
    mfma_model(Af, Bf, D);
  }
  for (int lane = 0; lane < 64; ++lane)
    for (int j = 0; j < 16; ++j) {
      const int h = lane >> 5, c = lane & 31, key = 16 * h + j;
      int32_t s = 0;
      for (int d = 0; d < 64; ++d) s += (int32_t)Kt[key][d] * Q[c][d];
      bad += D[lane][j] != s;
    }
  int32_t E[64][16] = {};
  for (int lane = 0; lane < 64; ++lane) {
    const int h = lane >> 5, c = lane & 31;
    for (int b = 0; b < 16; ++b) {
      Af[lane][b] = Vt[c][16 * h + b];
      Bf[lane][b] = P[c][16 * h + b];   // the score register layout: byte j = key 16 h + j of query c
    }
  }
  mfma_model(Af, Bf, E);
  for (int lane = 0; lane < 64; ++lane)
    for (int e = 0; e < 16; ++e) {
      const int h = lane >> 5, c = lane & 31, d = mfma_row(e, h);
      int32_t s = 0;
      for (int key = 0; key < 32; ++key) s += (int32_t)Vt[d][key] * P[c][key];
      bad += E[lane][e] != s;
    }
  return bad;
}

// Score digits (attn_q_digits): every int16 query element is 256 (qh + qx) + ql with int8 digits
// and qx in {0, 1}, every key element 256 kh + kl + 128; on random and extreme 64-dimension rows the
// digit sums the MFMAs form give q . k exactly, and lo = 256 A8 + A0 + 128 sum q + 2^(sh - 1) (the
// kernel's int32 piece) stays inside int32.  Returns the number of mismatches (plant 1: qx dropped).
int64_t eii_host_attn_digits(uint64_t seed, int plant) {
  int64_t bad = 0;
  for (int q = -32768; q <= 32767; ++q) {
    QDigits d = attn_q_digits(q);
    if (plant == 1) d.qx = 0;
    bad += d.ql < -128 || d.ql > 127 || d.qh < -128 || d.qh > 127 || d.qx < 0 || d.qx > 1;
    bad += 256 * (d.qh + d.qx) + d.ql != q;
  }
  for (int k = -32768; k <= 32767; ++k) {
    const int kh = k >> 8, kl = (k & 255) - 128;
    bad += kh < -128 || kh > 127 || 256 * kh + kl + 128 != k;
  }
  uint64_t r = seed;
  int q[64], k[64];
  for (int t = 0; t < 4000; ++t) {
    for (int d = 0; d < 64; ++d) {
      const int mode = t % 8;   // random, and rows at the int16 extremes
      q[d] = mode == 1 ? 32767 : mode == 2 ? -32768 : mode == 3 ? 32640 + (int)(next_rand(r) % 128) : (int)(int16_t)next_rand(r);
      k[d] = mode == 1 || mode == 5 ? 32767 : mode == 2 || mode == 6 ? -32768 : (int)(int16_t)next_rand(r);
    }
    int64_t truth = 0, A16 = 0, A8 = 0, A0 = 0, sq = 0;
    for (int d = 0; d < 64; ++d) {
      truth += (int64_t)q[d] * k[d];
      QDigits g = attn_q_digits(q[d]);
      if (plant == 1) g.qx = 0;
      const int kh = k[d] >> 8, kl = (k[d] & 255) - 128;
      A16 += (int64_t)(g.qh + g.qx) * kh;
      A8 += (int64_t)(g.qh + g.qx) * kl + (int64_t)g.ql * kh;
      A0 += (int64_t)g.ql * kl;
      sq += q[d];
    }
    bad += 65536 * A16 + 256 * A8 + A0 + 128 * sq != truth;
    const int64_t lo = 256 * A8 + A0 + 128 * sq + ((int64_t)1 << 29);
    bad += lo < INT32_MIN || lo > INT32_MAX || A16 < INT32_MIN || A16 > INT32_MAX;
  }
  return bad;
}

// Fragment order of the weights: element (n, k) lands where the swizzle kernel's thread for
// (block n / 32, slice k / 32, lane 32 ((k % 32) / 16) + n % 32) writes byte k % 16, and the map is
// one-to-one over the padded matrix.  Returns the number of mismatches.
int64_t eii_host_wfrag_model(int N, int K) {
  const int ks = K / 32, nbl = (N + 31) / 32;
  std::vector<int> hit((size_t)nbl * 32 * K, 0);
  int64_t bad = 0;
  for (int n = 0; n < nbl * 32; ++n)
    for (int k = 0; k < K; ++k) {
      const size_t o = w_fo_offset(n, k, ks);
      const int lane = 32 * ((k & 31) >> 4) + (n & 31);
      if (o != w_frag(n >> 5, ks, k >> 5, lane) + (k & 15)) ++bad;
      if (o >= hit.size()) { ++bad; continue; }
      ++hit[o];
    }
  for (int v : hit) bad += v != 1;
  return bad;
}
}
