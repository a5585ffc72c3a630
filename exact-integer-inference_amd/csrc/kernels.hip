// gfx950 kernels of the exact integer forward (SmolLM2-135M shape).
//
// Integer projections run on v_mfma_i32_32x32x32_i8: activations wider than int8 travel as
// exact int8 limb planes (eii_int.h), written by their producers; every limb plane is
// multiplied with the same int8 weight tile, and the limb partial sums (each below 2^31) are
// recombined exactly in the epilogue, which also applies the reference's requantization and
// the fused RoPE, SiLU-gate and residual steps.  The elementwise kernels are one pass over HBM
// each; attention computes QK and PV as integer MFMA tiles with the reference's three-step
// exact softmax (row max, exp-table sum, rounded Q0.16 division).
#include <algorithm>
#include <type_traits>

#include "eii_int.h"
#include "kernels.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // 16-byte staging registers

namespace eii {

namespace {

using namespace idx;   // operand layouts, fragment addresses and tile shapes (index_maps.h)

constexpr int kBK = 64;          // K block: one MFMA K-step
// 16 bytes per lane from global memory straight into LDS: lane i writes lds + 16 i (lds is the
// wave's base address; every lane passes the same one).  Kept out of the kernel templates: the
// host compilation pass of a kernel that names the builtin directly drops the kernel's launch stub.
__device__ __forceinline__ void dma16(const void* src, void* lds) { __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0); }
// s_waitcnt immediate: vector memory count <= n, the other counters not waited for (gfx9 encoding)
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Limb planes of 4 int16 values packed in two dwords: (low bytes - 128, high bytes).
// (v_perm_b32 byte i = byte sel[i] of the 8 bytes d1:d0, d0 being bytes 0..3)
__device__ __forceinline__ uint32_t lo_bytes16(uint32_t d0, uint32_t d1) {
  return __builtin_amdgcn_perm(d1, d0, 0x06040200u) ^ 0x80808080u;
}
__device__ __forceinline__ uint32_t hi_bytes16(uint32_t d0, uint32_t d1) {
  return __builtin_amdgcn_perm(d1, d0, 0x07050301u);
}
// Limb byte l of a W-byte activation v (eii_int.h split_limbs): low bytes biased by -128, the top
// byte signed.
__device__ __forceinline__ uint32_t limb_byte(int32_t v, int l, int W) {
  const uint32_t b = ((uint32_t)v >> (8 * l)) & 0xFFu;
  return l == W - 1 ? b : (b ^ 0x80u);
}
// The 4 limb-l bytes of 4 consecutive values, packed little-endian.
__device__ __forceinline__ uint32_t limb_word(const int32_t* v, int l, int W) {
  return limb_byte(v[0], l, W) | (limb_byte(v[1], l, W) << 8) | (limb_byte(v[2], l, W) << 16) |
         (limb_byte(v[3], l, W) << 24);
}

// v + the value of the lane that DPP control CTRL selects, for an int64 moved as two dwords
template <int CTRL>
__device__ __forceinline__ int64_t dpp_add64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)((uint64_t)v >> 32), CTRL, 0xF, 0xF, false);
  return v + (int64_t)(((uint64_t)hi << 32) | lo);
}
// sum over each group of LPR lanes (16 or 64), in every lane of the group: within 16-lane rows by
// DPP (lane ^ 1, lane ^ 2, then the mirrored lane of the other quad of the 8 and of the other 8 of
// the row), across rows by lane shuffles
template <int LPR>
__device__ __forceinline__ int64_t group_sum64(int64_t v) {
  v = dpp_add64<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v = dpp_add64<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v = dpp_add64<0x141>(v);   // row_half_mirror
  v = dpp_add64<0x140>(v);   // row_mirror
  if constexpr (LPR > 16) v += __shfl_xor(v, 16);
  if constexpr (LPR > 32) v += __shfl_xor(v, 32);
  return v;
}

// ------------------------------------------------------------------------------ GEMM
// Persistent workgroups of 4 waves, two per CU, sweep BM x BN output tiles (128 x 128 for 2-limb
// activations, 64 x 128 for 4-limb, 64 x 192 for 2-limb residual GEMMs with N = 576) in a flat
// (tile, K block of 64) loop.  Activation limb planes go global -> LDS through 4 stages;
// each wave loads its weight fragments straight into registers (the weights are L2-resident)
// two steps ahead.  v_mfma_i32_32x32x32_i8 sustains about twice the int8 rate of the 16x16x64
// form on gfx950.
//
// Epilogue arithmetic for 2-limb inputs runs in float64 and is exact: with P1, P0 the limb
// partial sums (|P| < 2^25 for K <= 1536) and |m| <= 2^14,
//   acc * m / 2^sh + 2^-(sh+1) = P1 * (256 m / 2^sh) + P0 * (m / 2^sh) + (128 wsum m / 2^sh + 2^-(sh+1))
// is a sum of multiples of 2^-(sh+1) below 2^(49-sh), i.e. at most 50 significant bits, so both
// FMAs are exact, and round-to-nearest-even of that value is RS(acc * m, sh) (the 2^-(sh+1)
// offset turns the reference's round-half-up into a tie-free rounding).  4-limb inputs, whose
// acc * m reaches 2^62, use int64.
constexpr double kMagic = 6755399441055744.0;   // 1.5 * 2^52: y + kMagic rounds y to an integer
constexpr int kLoopPrio = 3;                     // wave priority of the GEMM main loop (epilogues run at 0)

__device__ __forceinline__ int32_t rne_i32(double y) {   // |y| < 2^31 after clamping
  return (int32_t)(uint32_t)(uint64_t)__double_as_longlong(y + kMagic);
}

// Per-column coefficients for 2-limb inputs, precomputed once per weight matrix (coef_kernel):
//   c0 = m 2^-sh,  cb = 128 wsum m 2^-sh + 2^-(sh+1).
// acc * m / 2^sh + 2^-(sh+1) for acc = 256 P1 + P0 + 128 wsum (exact, see above):
// c1 = 256 c0, formed once per column.
__device__ __forceinline__ double req2(int32_t P1, int32_t P0, double c1, double2 k) {
  return fma((double)P1, c1, fma((double)P0, k.x, k.y));
}
typedef int v16i __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// v_mfma_i32_32x32x32_i8 with the activations as the A operand and the weights as the B operand:
// D[m][n] = sum_k a[m,k] W[n,k].  Lane = 32 h + c, register j = 4 b + r holds row
// i = 8 b + 4 h + r, column c of the 32x32 tile: the 32 lanes of a half-wave hold 32
// consecutive columns of one row, so every epilogue store is a contiguous run.
// Tile shapes: GemmCfg (index_maps.h).

// Tiles in grouped order: G row blocks x all column blocks per group.  Each XCD (= blockIdx % 8,
// the hardware's round-robin dispatch) owns a contiguous range of that order, and the persistent
// workgroups of one XCD sweep it together, so concurrently running tiles of an XCD share
// activation rows and weight blocks in its L2.  G = 1 (row-major order) for K <= 576 when the
// whole weight matrix fits the L2 beside the operand stream (q/k/v, o, gate/up): the column tiles
// of a row block then run at the same time and read each activation K block once, where with
// G = 8 the 64 tiles an XCD runs at a time cover only part of a group's columns and the rest fetch
// the same rows again later (gate/up at 256 x 160 tokens: 162 -> 92 MB fetched per launch).  G = 8
// for the head, whose weights (28 MB) do not fit (8 row blocks share each weight block), and for
// the 1536-deep down projection, which row-major order made 3 % slower although it fetched less.
__device__ __forceinline__ void tile_coords(int v, int nMB, int nNB, int G, int& mb, int& nb) {
  const int grp = v / (G * nNB), first = grp * G;
  const int gs = min(nMB - first, G), in = v - grp * G * nNB;
  mb = first + in % gs;
  nb = in / gs;
}

__device__ __forceinline__ uint32_t pack16(int32_t a, int32_t b) { return (uint32_t)(a & 0xFFFF) | ((uint32_t)b << 16); }

template <int AW, int EPI, int NK, int SHAPE, bool NORM = false>
__global__ __launch_bounds__(256, SHAPE == kShapeSkinny || SHAPE == kShapeSkinny32 ? 1 : 2) void gemm_kernel(GemmArgs g) {
  using C = GemmCfg<AW, SHAPE>;
  static_assert(!NORM || (C::kSkinny && NK == 9 && AW == 2), "the RMSNorm prologue: skinny tiles, K = 576, 16-bit");
  static_assert(SHAPE != kShapeNarrow || EPI == EPI_RESID || EPI == EPI_I64 || EPI == EPI_REQ16 ||
                EPI == EPI_REQ32 || EPI == EPI_LOGITS,
                "the SiLU and QKV epilogues pair columns 32 apart within 64-column blocks");
  constexpr bool kSilu = EPI == EPI_SILU || EPI == EPI_SILU_I;
  static_assert((!kSilu && EPI != EPI_QKV) || C::WN == 64, "one 64-column pair block per wave");
  static_assert(NK >= 1, "at least one K block");
  // EPI_SILU: entries 32768 - kTabHalf .. 32768 + kTabHalf - 1 of a 16-bit SiLU table as int16
  // after the stages (the gate values cluster around 0: with 64 x 256 tiles the window fills the CU's
  // LDS beside two workgroups' stages, and about 0.3 % of the gates lie outside it)
  constexpr int kTabHalf = 4096;
  // EPI_SILU keeps the window as int32 (16- and 32-bit tables), EPI_SILU_I as int16
  using TabT = std::conditional_t<EPI == EPI_SILU, int32_t, int16_t>;
  constexpr int kTabBytes = kSilu ? 2 * kTabHalf * (int)sizeof(TabT) : 0;
  // skinny tiles: the RMSNorm prologue's limb bytes of up to kNormRows rows after the reduction area
  constexpr int kNormRows = 4;
  constexpr int kNormBytes = NORM ? AW * kNormRows * kD : 0;
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::kStages * C::kStage + kTabBytes + kNormBytes];
  const int nMB = (g.M + C::BM - 1) / C::BM, nNB = (g.N + C::BN - 1) / C::BN, nT = nMB * nNB;
  // this workgroup's tiles: v = v0, v0 + stride, ... < vend (kShapeSkinny: tile blockIdx.x alone)
  const int xcd = blockIdx.x & 7, per = (nT + 7) / 8, nwg_x = C::kSkinny ? 1 : gridDim.x >> 3;
  const int v0 = C::kSkinny ? (int)blockIdx.x : xcd * per + (blockIdx.x >> 3);
  const int vend = C::kSkinny ? nT : min(nT, (xcd + 1) * per);
  if (v0 >= vend) return;
  const int ntiles = (vend - v0 + nwg_x - 1) / nwg_x;
  constexpr int nk = NK;
  TabT* const tabw = (TabT*)(smem + C::kStages * C::kStage);
  int tab_half = 0;   // 0: no LDS window, every read goes to global memory
  if constexpr (kSilu) {
    if (!C::kSkinny) {   // (a skinny tile's few rows read the table in global memory)
      tab_half = kTabHalf;
      for (int i = threadIdx.x; i < 2 * kTabHalf; i += C::kThreads) tabw[i] = (TabT)g.aux_tab[32768 - kTabHalf + i];
    }
    __syncthreads();
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int fc = lane & 31, fh = lane >> 5;
  const uint8_t* Ab = (const uint8_t*)g.A;

  // Operand loads run ahead of the MFMAs on a fixed schedule, with steps in pairs (s, s + 1),
  // s even.  At the start of a pair, after the pair's one barrier, the activations of steps s + 2
  // and s + 3 go straight from global memory into LDS stages (s + 2) % 4 and (s + 3) % 4, which
  // were last read in steps s - 2 and s - 1 (lane i of a load lands at its base + 16 i, so each
  // lane fetches the chunk that belongs at its slot).  After its MFMAs, step s (s + 1) loads the
  // weight fragments of step s + 2 (s + 3) into the register set it just consumed.  A load of K
  // block 0 points the source pointers at its tile, later blocks advance them.  Past the last
  // tile the loads repeat the last tile (addresses stay valid, nothing reads them), so every
  // step issues the same loads and the memory-count waits are the same everywhere.  Rows past M
  // read row M - 1 and column blocks past N the last block; their results are never stored.
  // Both operands are laid out for contiguous 1 KB wave runs: K-blocked activation planes and
  // fragment-ordered weights.
  const size_t a_kstep = (size_t)g.M * 64;              // activation bytes between K blocks
  const int nb32_last = (g.N + 31) / 32 - 1;
  const uint8_t* a_src[C::kAChunks];
  const int8_t* w_src[C::TN];
  auto coords = [&](int j, int& mb, int& nb) __attribute__((always_inline)) {
    tile_coords(v0 + min(j, ntiles - 1) * nwg_x, nMB, nNB, g.tile_g, mb, nb);
  };
  auto point_a = [&](int mb) __attribute__((always_inline)) {
    const int m0 = mb * C::BM;
#pragma unroll
    for (int i = 0; i < C::kAChunks; ++i) {
      // LDS slot q (16 bytes) of the stage: limb plane l, row, physical chunk cp, which holds the
      // row's logical chunk lds_swz(row, cp)
      const AChunk ch = a_chunk(tid + C::kThreads * i, C::BM);
      const int m = min(m0 + ch.row, g.M - 1);
      a_src[i] = Ab + a_src_off(ch.l, m, 0, lds_swz(ch.row, ch.cp), g.M, g.a_kb, g.a_plane);
    }
  };
  auto point_w = [&](int nb) __attribute__((always_inline)) {
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn) {
      // this lane's B fragments: weight rows n0 + 64 wn + 32 tn + 0..31, the lane's 16 bytes of
      // each 32-column K slice
      const int nb32 = min((nb * C::BN + wn * C::WN + 32 * tn) >> 5, nb32_last);
      w_src[tn] = g.W + w_frag(nb32, (g.w_ld ? g.w_ld : g.K) / 32, 0, lane);
    }
  };
  // The pointers advance by one K block per load.  The increment goes through an empty asm so
  // that the compiler keeps one pointer set per operand instead of precomputing the addresses of
  // every step of the unrolled tile.
  auto opaque = [](size_t v) __attribute__((always_inline)) {
    __asm__ volatile("" : "+s"(v));
    return v;
  };
  auto load_a = [&](int st) __attribute__((always_inline)) {   // next K block -> stage st % 4
    uint8_t* stage = smem + (st & (C::kStages - 1)) * C::kStage;
#pragma unroll
    for (int i = 0; i < C::kAChunks; ++i)
      dma16(a_src[i], stage + (C::kThreads * i + 64 * wave) * 16);
    const size_t inc = opaque(a_kstep);
#pragma unroll
    for (int i = 0; i < C::kAChunks; ++i) a_src[i] += inc;
  };
  v4i wreg[2][C::TN][2];
  auto load_w = [&](auto SET) __attribute__((always_inline)) {   // next K block -> register set SET
    constexpr int set = decltype(SET)::value;
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) wreg[set][tn][ks] = *(const v4i*)(w_src[tn] + 1024 * ks);
    const size_t inc = opaque(2048);
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn) w_src[tn] += inc;
  };

  // the loads of step st (tile j, K block blk): block 0 re-points the pointers at tile j
  auto a_step = [&](int j, int blk, int st) __attribute__((always_inline)) {
    if (blk == 0) {
      int mb_, nb_;
      coords(j, mb_, nb_);
      point_a(mb_);
    }
    load_a(st);
  };
  auto w_step = [&](auto SET, int j, int blk) __attribute__((always_inline)) {
    if (blk == 0) {
      int mb_, nb_;
      coords(j, mb_, nb_);
      point_w(nb_);
    }
    load_w(SET);
  };

  v16i acc[C::TM][C::TN][AW];
#pragma unroll
  for (int a = 0; a < C::TM; ++a)
#pragma unroll
    for (int b = 0; b < C::TN; ++b)
#pragma unroll
      for (int l = 0; l < AW; ++l) acc[a][b][l] = v16i{};

  // Epilogue of tile (mb, nb).  Lane value (tm, tn, e) sits at tile row rw + 32 tm + roff(e)
  // (rw = wm WM + 4 fh) and tile column cw + 32 tn (cw = wn WN + fc): the 32 lanes of a half-wave
  // cover 32 consecutive columns of one row, so every load and store moves whole 128-byte lines.
  // Tiles inside M (all but the last row block) take a path without row tests, where every
  // address is a uniform row base (scalar registers, scalar arithmetic) plus the lane's fixed
  // 32-bit offset, so element addresses cost no vector instructions.  The last row block clamps
  // its loads to row M - 1 and tests the row at each store.
  auto epilogue_t = [&](auto FULL, int mb, int nb) __attribute__((always_inline)) {
    constexpr bool full = decltype(FULL)::value;
    const int m0 = mb * C::BM, n0 = nb * C::BN;
    const int rw = wm * C::WM + 4 * fh, cw = wn * C::WN + fc;
    auto roff = [](int e) { return mfma_row(e, 0); };   // + 4 fh, in rw
    auto live = [&](int tm, int e) { return full || m0 + rw + 32 * tm + roff(e) < g.M; };
    // a group of the wave's rows whose first row (tile row 32 tm + r0, lane half 0) lies past M: the
    // SiLU and q/k/v epilogues skip the whole group, a uniform branch (the last row block of a
    // launch; a skinny tile of a one-sequence decoding step keeps 1 of its 8 groups of 4 rows)
    auto dead = [&](int tm, int r0) { return !full && m0 + wm * C::WM + 32 * tm + r0 >= g.M; };
    const int rlast = g.M - 1 - m0;   // last valid tile row
    // the row stride passes through an empty asm so the per-element offsets are recomputed here
    // instead of being hoisted out of the tile loop (64 loop-invariant offsets would spill)
    int N = g.N;
    __asm__ volatile("" : "+s"(N));
    const int64_t bias = limb_bias(AW);
    auto acc64 = [&](int tm, int tn, int e, int32_t ws) -> int64_t {
      int64_t a = bias * (int64_t)ws;
#pragma unroll
      for (int l = 0; l < AW; ++l) a += (int64_t)acc[tm][tn][l][e] * ((int64_t)1 << (8 * l));
      return a;
    };
    // Element (tm, e, column offset col) of a row-major tile with rows of ld elements at `tile`:
    // the uniform part (tile, row 32 tm + roff(e), col) and the lane part (row rw, column cw) are
    // added separately.  rowL clamps the row for loads in the last row block.
    auto at = [&](auto* tile, int ld, uint32_t lane_b, int tm, int e, int col) {
      using T = std::remove_pointer_t<decltype(tile)>;
      return (T*)((char*)(tile + (size_t)(32 * tm + roff(e)) * ld + col) + lane_b);
    };
    auto atL = [&](auto* tile, int ld, uint32_t lane_b, int tm, int e, int col) {
      if constexpr (full) return at(tile, ld, lane_b, tm, e, col);
      else return tile + (size_t)min(rw + 32 * tm + roff(e), rlast) * ld + cw + col;
    };

    if constexpr (EPI == EPI_I64 || EPI == EPI_REQ16 || EPI == EPI_REQ32 || EPI == EPI_RESID || EPI == EPI_LOGITS) {
      using OT = std::conditional_t<EPI == EPI_I64, int64_t, std::conditional_t<EPI == EPI_REQ16, int16_t, int32_t>>;
      OT* tb = (OT*)g.out + (size_t)m0 * N + n0;
      const uint32_t lane_b = ((uint32_t)rw * (uint32_t)N + (uint32_t)cw) * (uint32_t)sizeof(OT);
      const double lo = EPI == EPI_REQ16 || EPI == EPI_REQ32 ? -ldexp(1.0, g.sat_bits - 1) : 0.0;
      const double hi = EPI == EPI_REQ16 || EPI == EPI_REQ32 ? ldexp(1.0, g.sat_bits - 1) - 1.0 : 0.0;
      // logits leave int32 iff RNE(y) does: y is never a tie, so iff y > 2^31 - 1/2 or y < -2^31 - 1/2
      double ymax = 0.0, ymin = 0.0;
      bool bad = false;
#pragma unroll
      for (int tn = 0; tn < C::TN; ++tn) {
        const int n = n0 + cw + 32 * tn;
        if (n >= g.N) continue;
        const int32_t ws = (AW == 4 || EPI == EPI_I64) && g.wsum ? g.wsum[n] : 0;
        int32_t mu = 0, sh = 1;
        double2 k = make_double2(0.0, 0.0);
        if constexpr (AW == 4 && EPI != EPI_I64) { mu = g.mult[n]; sh = g.shift[n]; }
        if constexpr (AW == 2 && EPI != EPI_I64) k = g.coef[n];
        const double c1 = 256.0 * k.x;
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm) {
          if constexpr (EPI == EPI_I64) {
            if (g.accumulate) {
#pragma unroll
              for (int e = 0; e < 16; ++e)
                if (live(tm, e)) {
                  OT* p = at(tb, N, lane_b, tm, e, 32 * tn);
                  *p = *p + acc64(tm, tn, e, ws);
                }
            } else {
#pragma unroll
              for (int e = 0; e < 16; ++e)
                if (live(tm, e)) __builtin_nontemporal_store(acc64(tm, tn, e, ws), at(tb, N, lane_b, tm, e, 32 * tn));
            }
            continue;
          }
          // residual epilogue: the loads of 8 rows issue together, then their updates
#pragma unroll
          for (int eh = 0; eh < 16; eh += 8) {
            int32_t xv[8];
            if constexpr (EPI == EPI_RESID) {
#pragma unroll
              for (int i = 0; i < 8; ++i) xv[i] = *atL(tb, N, lane_b, tm, eh + i, 32 * tn);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int e = eh + i;
              // RS(acc * m, sh): exact float64 2^-(sh+1)-offset form (2 limbs) or int64 (4 limbs)
              double y = 0.0;
              int64_t v = 0;
              if constexpr (AW == 2) y = req2(acc[tm][tn][1][e], acc[tm][tn][0][e], c1, k);
              else v = rs(acc64(tm, tn, e, ws) * mu, sh);
              int32_t q;
              if constexpr (EPI == EPI_REQ16 || EPI == EPI_REQ32) {
                q = AW == 2 ? rne_i32(fmin(fmax(y, lo), hi)) : (int32_t)sat(v, g.sat_bits);
              } else if constexpr (EPI == EPI_RESID) {
                q = AW == 2 ? rne_i32(fmin(fmax(rint(y) + (double)xv[i], -2147483648.0), 2147483647.0))
                            : (int32_t)clamp_bits32((int64_t)xv[i] + v);
              } else {   // EPI_LOGITS
                if constexpr (AW == 2) {
                  ymax = fmax(ymax, y);
                  ymin = fmin(ymin, y);
                  q = rne_i32(y);
                } else {
                  bad |= v != (int64_t)(int32_t)v;
                  q = (int32_t)v;
                }
              }
              if (live(tm, e)) {
                // the logits (8 GB at 256 x 160 tokens) stream past the caches instead of evicting
                // the operand tiles other workgroups are about to reuse
                if constexpr (EPI == EPI_LOGITS) __builtin_nontemporal_store((OT)q, at(tb, N, lane_b, tm, e, 32 * tn));
                else *at(tb, N, lane_b, tm, e, 32 * tn) = (OT)q;
              }
            }
          }
        }
      }
      if constexpr (EPI == EPI_LOGITS) {
        if (bad || ymax > 2147483647.5 || ymin < -2147483648.5) atomicOr(g.flag, 1);
      }
    } else if (n0 + wn * C::WN < g.N) {
      // columns c (tn = 0) and 32 + c (tn = 1) of the wave's 64-column block: (gate j, up j) for
      // EPI_SILU (weight rows stacked as [gate 32 | up 32] blocks), (d, d + 32) of one head for EPI_QKV
      const int nc = n0 + cw;
      const double2 k0 = g.coef[nc], k1 = g.coef[nc + 32];
      const double c10 = 256.0 * k0.x, c11 = 256.0 * k1.x;
      auto scaled = [&](int tm, int tn, int e) -> double {   // RS(acc * m, sh) of column nc + 32 tn, 2 limbs
        return req2(acc[tm][tn][1][e], acc[tm][tn][0][e], tn ? c11 : c10, tn ? k1 : k0);
      };
      auto value16 = [&](int tm, int tn, int e) -> int32_t {   // SAT16(RS(acc * m, sh))
        if constexpr (AW == 2) {
          return rne_i32(fmin(fmax(scaled(tm, tn, e), -32768.0), 32767.0));
        } else {
          const int n = nc + 32 * tn;
          return (int32_t)clamp_bits16(rs(acc64(tm, tn, e, g.wsum[n]) * g.mult[n], g.shift[n]));
        }
      };
      auto value16d = [&](int tm, int tn, int e) -> double {   // the same as a double
        if constexpr (AW == 2) return rint(fmin(fmax(scaled(tm, tn, e), -32768.0), 32767.0));
        else return (double)value16(tm, tn, e);
      };
      if constexpr (kSilu) {
        // gated limb planes (bits2 / 8 planes of M x N / 2 in 32-byte K blocks, plane_offset32): the
        // lane's gated column n0 / 2 + wn 32 + fc is column fc of 32-column block nb BN / 64 + wn
        const double lo = -ldexp(1.0, g.bits2 - 1), hi = ldexp(1.0, g.bits2 - 1) - 1.0;
        // RS(x, sh) = RNE(x 2^-sh + 2^-(sh+1)) for sh >= 1; for sh <= 0 the scaled value is an integer
        const double sc = ldexp(1.0, -g.sh2), half = g.sh2 >= 1 ? ldexp(0.5, -g.sh2) : 0.0;
        // 16-bit table entries times 16-bit up values: |silu up| < 2^30, so for shifts 1..30 the
        // product, its rounding offset and the shift stay in int32 (one 24-bit multiply)
        const int32_t rnd2 = EPI == EPI_SILU_I ? 1 << (g.sh2 - 1) : 0;
        const size_t pl = (size_t)g.M * (N / 2);
        // the 4 lanes of a quad hold 4 consecutive rows and the 8 quads of a half-wave the block's 32
        // columns, so each half-wave store covers one 128-byte line (4 rows x 32 bytes)
        uint8_t* tb = (uint8_t*)g.out + (size_t)(nb * (C::BN / 64) + wn) * g.M * 32 + (size_t)m0 * 32;
        const uint32_t lane_b4 = (uint32_t)(rw + (fc & 3)) * 32u + (uint32_t)(fc & ~3);
        // limb bytes (the low bytes carry the -128 bias, the top byte is signed) of rows r = 0..3 of
        // each 4-row group, then a 4 x 4 byte transpose across the lanes of a quad: lane j of the
        // quad ends with row j, columns 4 (fc / 4) .. + 3, one dword per plane
        const uint32_t xb = g.bits2 == 16 ? 0x80u : 0x808080u;
        const uint32_t sel1 = (lane & 1) ? 0x03070105u : 0x06020400u;
        const uint32_t sel2 = (lane & 2) ? 0x03020706u : 0x05040100u;
        auto tr4 = [&](uint32_t w) __attribute__((always_inline)) {
          uint32_t x = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xB1, 0xF, 0xF, false);
          w = __builtin_amdgcn_perm(x, w, sel1);
          x = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x4E, 0xF, 0xF, false);
          return __builtin_amdgcn_perm(x, w, sel2);
        };
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {   // rows 8 b + 4 h + 0..3 of the 32-row tile tm
            if (dead(tm, 8 * b)) continue;
            int32_t gv[4], sv[4], ui[4], vv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) { gv[r] = value16(tm, 0, 4 * b + r); ui[r] = value16(tm, 1, 4 * b + r); }
            // SiLU table reads: gates within the LDS window read it there; the others read global
            // memory, only in the groups of 64 gates where some lane needs it (32-bit offsets from
            // the table base; lanes served by LDS point at one shared line)
            bool inw[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int wi = gv[r] + tab_half;
              inw[r] = (uint32_t)wi < (uint32_t)(2 * tab_half);
              sv[r] = tabw[min(max(wi, 0), 2 * kTabHalf - 1)];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int32_t t = *(const int32_t*)((const char*)g.aux_tab + (uint32_t)(inw[r] ? 32768 : gv[r] + 32768) * 4u);
              if (!inw[r]) sv[r] = t;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if constexpr (EPI == EPI_SILU_I) {
                // SAT(RS(silu * up, sh2), bits2) in int32 (|silu up| < 2^30, sh2 in 1..30)
                const int32_t q = (__mul24(sv[r], ui[r]) + rnd2) >> g.sh2;
                vv[r] = g.bits2 == 16 ? min(max(q, -32768), 32767) : q;
              } else {
                // the product and the scaled sum are exact in float64
                vv[r] = rne_i32(fmin(fmax(fma((double)sv[r] * (double)ui[r], sc, half), lo), hi));
              }
            }
            const uint32_t v0 = (uint32_t)vv[0] ^ xb, v1 = (uint32_t)vv[1] ^ xb;
            const uint32_t v2 = (uint32_t)vv[2] ^ xb, v3 = (uint32_t)vv[3] ^ xb;
            const uint32_t t01 = __builtin_amdgcn_perm(v1, v0, 0x05010400u), t23 = __builtin_amdgcn_perm(v3, v2, 0x05010400u);
            const uint32_t p0 = tr4(__builtin_amdgcn_perm(t23, t01, 0x05040100u));
            const uint32_t p1 = tr4(__builtin_amdgcn_perm(t23, t01, 0x07060302u));
            uint32_t p2 = 0, p3 = 0;
            if (g.bits2 != 16) {
              const uint32_t u01 = __builtin_amdgcn_perm(v1, v0, 0x07030602u), u23 = __builtin_amdgcn_perm(v3, v2, 0x07030602u);
              p2 = tr4(__builtin_amdgcn_perm(u23, u01, 0x05040100u));
              p3 = tr4(__builtin_amdgcn_perm(u23, u01, 0x07060302u));
            }
            const int row = 32 * tm + 8 * b;   // + the lane's rw + (fc & 3)
            if (!full && m0 + rw + (fc & 3) + row >= g.M) continue;
            uint32_t* ob = (uint32_t*)(tb + (size_t)row * 32 + lane_b4);
            ob[0] = p0;
            *(uint32_t*)((uint8_t*)ob + pl) = p1;
            if (g.bits2 != 16) {
              *(uint32_t*)((uint8_t*)ob + 2 * pl) = p2;
              *(uint32_t*)((uint8_t*)ob + 3 * pl) = p3;
            }
          }
        }
      } else {   // EPI_QKV: heads 0..8 q and 9..11 k get RoPE, 12..14 v are stored as they are
        const int head = (n0 + wn * C::WN) >> 6;
        int ld = g.ldc ? g.ldc : g.N;   // output row stride, opaque like N
        __asm__ volatile("" : "+s"(ld));
        int16_t* tb = (int16_t*)g.out + (size_t)m0 * ld + n0;
        const uint32_t lane_b = ((uint32_t)rw * (uint32_t)ld + (uint32_t)cw) * 2u;
        if (head >= 12) {
          // v: int16 rows and, when requested, the V^T limb planes (4 consecutive rows per dword;
          // rows up to the tile end fit vt_stride, so no row test there)
          const size_t vcol = (size_t)((head - 12) * 64 + fc) * g.vt_stride, vpl = (size_t)192 * g.vt_stride;
#pragma unroll
          for (int tm = 0; tm < C::TM; ++tm) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              if (dead(tm, 8 * b)) continue;
              int32_t v1[4], v2[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int e = 4 * b + r;
                v1[r] = value16(tm, 0, e);
                v2[r] = value16(tm, 1, e);
                if (live(tm, e)) {
                  int16_t* op = at(tb, ld, lane_b, tm, e, 0);
                  op[0] = (int16_t)v1[r];
                  op[32] = (int16_t)v2[r];
                }
              }
              if (g.vt) {
                uint8_t* vp = g.vt + vcol + (m0 + rw + 32 * tm + 8 * b);
                const size_t d32 = (size_t)32 * g.vt_stride;
                *(uint32_t*)vp = limb_word(v1, 0, 2);
                *(uint32_t*)(vp + vpl) = limb_word(v1, 1, 2);
                *(uint32_t*)(vp + d32) = limb_word(v2, 0, 2);
                *(uint32_t*)(vp + d32 + vpl) = limb_word(v2, 1, 2);
              }
            }
          }
        } else {
          const int shr = head < 9 ? g.sh_q : g.sh_k;
          const double sc = ldexp(1.0, -shr), half = shr >= 1 ? ldexp(0.5, -shr) : 0.0;
#pragma unroll
          for (int tm = 0; tm < C::TM; ++tm) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              if (dead(tm, 8 * b)) continue;
              int32_t cs[4], sn[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int ps = g.pos[min(m0 + rw + 32 * tm + 8 * b + r, g.M - 1)];
                const uint32_t o = (uint32_t)ps * 128u + (uint32_t)fc * 4u;   // byte offset of [ps][fc]
                cs[r] = *(const int32_t*)((const char*)g.cosT + o);
                sn[r] = *(const int32_t*)((const char*)g.sinT + o);
              }
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int e = 4 * b + r;
                const double a1 = value16d(tm, 0, e), a2 = value16d(tm, 1, e);
                const double c = (double)cs[r], s2 = (double)sn[r];
                const int32_t o1 = rne_i32(fmin(fmax(fma(fma(a1, c, -a2 * s2), sc, half), -32768.0), 32767.0));
                const int32_t o2 = rne_i32(fmin(fmax(fma(fma(a2, c, a1 * s2), sc, half), -32768.0), 32767.0));
                if (!live(tm, e)) continue;
                int16_t* op = at(tb, ld, lane_b, tm, e, 0);
                op[0] = (int16_t)o1;
                op[32] = (int16_t)o2;
              }
            }
          }
        }
      }
    }
  };
  auto epilogue = [&](int mb, int nb) __attribute__((always_inline)) {
    // (the QKV epilogue keeps one copy: two of them exhaust the registers)
    if (EPI != EPI_QKV && (mb + 1) * C::BM <= g.M) epilogue_t(std::true_type{}, mb, nb);
    else epilogue_t(std::false_type{}, mb, nb);
  };

  // Step s computes from LDS stage s % 4 and weight register set s % 2.  Its loads are waited for
  // with explicit memory counts (loads complete in order): at a pair start, all but the weights
  // of step s + 1 (2 TN loads), followed by the barrier (which then carries no full memory fence,
  // so the later loads stay in flight); mid-pair, all but the activations of s + 1, s + 2 and the
  // weights of s + 1 issued since.  Every tile is unrolled (two tiles per iteration when NK is
  // odd), so the register set of each step is a compile-time constant and a tile is straight-line
  // code up to its epilogue.
  if constexpr (C::kSkinny) {
    // tile v0 in row-major order; wave w takes the 32-wide K slices [2 NK w / 4, 2 NK (w + 1) / 4)
    const int mb = v0 / nNB, nb = v0 % nNB;
    constexpr int NS = 2 * NK, NSW = (NS + 3) / 4;
    const int s0 = wave * NS / 4, cnt = (wave + 1) * NS / 4 - s0;
    const int m = min(mb * C::BM + fc, g.M - 1);
    const int kslices = (g.w_ld ? g.w_ld : g.K) / 32;
    // fragments as in the LDS path: row fc, bytes 16 fh .. 16 fh + 15 of slice s (chunk c of its
    // 64-byte K block in either plane layout); the weights of columns nb 64 + 32 tn + 0..31
    v4i af[NSW][AW], wf[NSW][C::TN];
#pragma unroll
    for (int i = 0; i < NSW; ++i)
      if (i < cnt) {
        const int sl = s0 + i;
        if constexpr (!NORM) {
          const size_t aoff = a_src_off(0, m, sl >> 1, 2 * (sl & 1) + fh, g.M, g.a_kb, 0);
#pragma unroll
          for (int l = 0; l < AW; ++l) af[i][l] = *(const v4i*)(Ab + (size_t)l * g.a_plane + aoff);
        }
#pragma unroll
        for (int tn = 0; tn < C::TN; ++tn) {
          const int nb32 = min(nb * C::TN + tn, nb32_last);
          wf[i][tn] = *(const v4i*)(g.W + w_frag(nb32, kslices, sl, lane));
        }
      }
    if constexpr (NORM) {
      // the values of rmsnorm_kernel's fast path with a wave per row (rmsnorm_kernel<., false,
      // 64>): wave w normalizes tile row w (lane c: columns 64 k + c) and leaves its limb bytes in
      // LDS, where the lanes of every wave read their fragments (rows past M: zero)
      const int R = min(g.M - mb * C::BM, kNormRows);
      uint8_t* stg = smem + C::kStages * C::kStage + kTabBytes;   // [2][kNormRows][576] limb bytes
      if (wave < R) {
        const int32_t* xr = g.nx + (size_t)(mb * C::BM + wave) * kD + lane;
        int32_t v[9], gv[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
          v[k] = xr[64 * k];
          gv[k] = 3 * g.ngain[64 * k + lane];
        }
        int64_t SA = 0, SB = 0, SC = 0;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
          const int32_t hi = v[k] >> 16, lo = v[k] & 0xFFFF;
          SA += (int64_t)hi * hi; SB += (int64_t)hi * lo; SC += (int64_t)lo * lo;
        }
        SA = group_sum64<64>(SA);
        SB = group_sum64<64>(SB);
        SC = group_sum64<64>(SC);
        const int32_t U = (int32_t)norm_U(norm_total(SA, SB, SC));   // < 2^29
        const int64_t rnd = (int64_t)1 << (g.nsh - 1);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
          const int32_t z = (int32_t)(((int64_t)v[k] * U + 32768) >> 16);
          const int32_t q = (int32_t)(((int64_t)z * gv[k] + rnd) >> g.nsh);
          const int32_t o = min(max(q, -32768), 32767);
#pragma unroll
          for (int l = 0; l < AW; ++l) stg[(l * kNormRows + wave) * kD + 64 * k + lane] = (uint8_t)limb_byte(o, l, AW);
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NSW; ++i)
        if (i < cnt) {
#pragma unroll
          for (int l = 0; l < AW; ++l)
            af[i][l] = fc < R ? *(const v4i*)(stg + (l * kNormRows + fc) * kD + 32 * (s0 + i) + 16 * fh) : v4i{};
        }
    }
    // wave 0 reads the epilogue's per-column coefficients and, lane c for tile row c, the residual
    // row or the position and its RoPE rows while the operands load, so the epilogue's own reads of
    // them hit the CU's cache instead of adding memory round trips after the reduction
    uint32_t touch = 0;
    if (wave == 0) {
      const int n = min(nb * C::BN + fc, g.N - 1), n2 = min(n + 32, g.N - 1);
      if constexpr (AW == 2 && EPI != EPI_I64) {
        touch = (uint32_t)__double_as_longlong(g.coef[n].x) ^ (uint32_t)__double_as_longlong(g.coef[n2].y);
      } else if constexpr (EPI != EPI_I64) {
        touch = (uint32_t)(g.mult[n] ^ g.shift[n] ^ g.wsum[n]);
      }
      const int mr = min(mb * C::BM + fc, g.M - 1);
      if constexpr (EPI == EPI_RESID) touch ^= (uint32_t)((const int32_t*)g.out)[(size_t)mr * g.N + nb * C::BN];
      if constexpr (EPI == EPI_QKV) {
        const int ps = g.pos[mr];
        touch ^= (uint32_t)(g.cosT[ps * 32] ^ g.sinT[ps * 32]);
      }
    }
#pragma unroll
    for (int i = 0; i < NSW; ++i)
      if (i < cnt) {
#pragma unroll
        for (int l = 0; l < AW; ++l)
#pragma unroll
          for (int tn = 0; tn < C::TN; ++tn) acc[0][tn][l] = mfma32(af[i][l], wf[i][tn], acc[0][tn][l]);
      }
    __asm__ volatile("" ::"v"(touch));   // keeps the reads
    // partial sums of waves 1..3 -> LDS as 16-byte groups [wave - 1][tn][l][e / 4][lane][e % 4];
    // wave 0 adds them (each partial and the total are limb sums over part of K, below 2^31) and runs
    // the epilogue
    v4i* red = (v4i*)smem;
    if (wave > 0) {
#pragma unroll
      for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
        for (int l = 0; l < AW; ++l)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            red[((((wave - 1) * C::TN + tn) * AW + l) * 4 + q) * 64 + lane] =
                v4i{acc[0][tn][l][4 * q], acc[0][tn][l][4 * q + 1], acc[0][tn][l][4 * q + 2], acc[0][tn][l][4 * q + 3]};
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
        for (int l = 0; l < AW; ++l)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const v4i p = red[(((w * C::TN + tn) * AW + l) * 4 + q) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[0][tn][l][4 * q + r] += p[r];
          }
    epilogue(mb, nb);
    return;
  }

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  __builtin_amdgcn_s_setprio(kLoopPrio);
  a_step(0, 0, 0);
  a_step(1 / nk, 1 % nk, 1);
  w_step(I0{}, 0, 0);
  w_step(I1{}, 1 / nk, 1 % nk);
  // step kb of tile jt: global step st = jt * nk + kb, cur = st % 2
  auto step = [&](auto CUR, int jt, int kb, int st) __attribute__((always_inline)) {
    constexpr int cur = decltype(CUR)::value;
    if constexpr (cur == 0) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * C::TN));
      __builtin_amdgcn_s_barrier();
      __asm__ volatile("" ::: "memory");
      a_step(jt + (kb + 2) / nk, (kb + 2) % nk, st + 2);
      a_step(jt + (kb + 3) / nk, (kb + 3) % nk, st + 3);
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * C::kAChunks + 2 * C::TN));
    }
    const uint8_t* base = smem + (st & (C::kStages - 1)) * C::kStage;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kc = 2 * ks + fh;   // this lane's 16-byte K chunk
      v4i af[C::TM][AW];   // all A fragments of this K step first, so their LDS latencies overlap
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
        for (int l = 0; l < AW; ++l) {
          const int row = wm * C::WM + tm * 32 + fc;
          af[tm][l] = *(const v4i*)(base + a_frag(l, row, kc, C::kPlane));
        }
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
        for (int l = 0; l < AW; ++l)
#pragma unroll
          for (int tn = 0; tn < C::TN; ++tn) acc[tm][tn][l] = mfma32(af[tm][l], wreg[cur][tn][ks], acc[tm][tn][l]);
    }
    // order: the first K slice's fragment reads, two MFMAs, the second slice's reads (their
    // latency hides behind the first slice's MFMAs), then the remaining MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, C::TM * AW, 0);   // LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);            // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, C::TM * AW, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * C::TM * AW * C::TN - 2, 0);
    // weights of st + 2, into the set this step just consumed
    w_step(CUR, jt + (kb + 2) / nk, (kb + 2) % nk);
    if (kb != nk - 1) return;

    // ---------------------------------------------------------------- epilogue
    // The epilogue runs at the lowest wave priority and the main loop at a raised one: the two
    // workgroups of a CU share its SIMDs, so one workgroup's epilogue (vector work, stores) issues
    // in the gaps of the other's MFMA loop instead of competing with it for issue slots.
    int mb, nb;
    coords(jt, mb, nb);
    __builtin_amdgcn_s_setprio(0);
    epilogue(mb, nb);
    __builtin_amdgcn_s_setprio(kLoopPrio);
#pragma unroll
    for (int a = 0; a < C::TM; ++a)
#pragma unroll
      for (int b = 0; b < C::TN; ++b)
#pragma unroll
        for (int l = 0; l < AW; ++l) acc[a][b][l] = v16i{};
  };
  auto tile = [&](auto PAR, int jt) __attribute__((always_inline)) {   // PAR = parity of the tile's first step
    constexpr int p0 = decltype(PAR)::value;
#pragma unroll
    for (int kb = 0; kb < nk; ++kb) {
      const int st = jt * nk + kb;
      if ((kb + p0) % 2 == 0) step(I0{}, jt, kb, st);
      else step(I1{}, jt, kb, st);
    }
  };
  if constexpr (nk % 2 == 0) {
    for (int jt = 0; jt < ntiles; ++jt) tile(I0{}, jt);
  } else {
    int jt = 0;
    for (; jt + 1 < ntiles; jt += 2) {
      tile(I0{}, jt);
      tile(I1{}, jt + 1);
    }
    if (jt < ntiles) tile(I0{}, jt);
  }
  // the loads issued past the last tile write this workgroup's LDS: drain them before it ends
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

template <int AW, int EPI, int SHAPE>
hipError_t launch_gemm_cfg(const GemmArgs& a_in, hipStream_t s) {
  using C = GemmCfg<AW, SHAPE>;
  GemmArgs a = a_in;
  a.tile_g = (size_t)a.N * a.K <= ((size_t)1 << 21) && a.K <= 576 ? 1 : 8;   // see tile_coords
  const int nT = ((a.M + C::BM - 1) / C::BM) * ((a.N + C::BN - 1) / C::BN);
  // two persistent workgroups per CU, a multiple of 8 so every XCD gets the same count; one
  // workgroup per tile for kShapeSkinny
  const int per_xcd = std::min((nT + 7) / 8, std::max(1, 2 * device_cus() / 8));
  const dim3 grid(C::kSkinny ? nT : 8 * per_xcd), block(C::kThreads);
  // K is a template parameter so each tile's K loop is straight-line code: the model's K
  // (576, 1536) for every epilogue, and 64, 128 for the operator entry points
  constexpr bool op = EPI == EPI_I64 || EPI == EPI_REQ16 || EPI == EPI_REQ32;
  switch (a.K / kBK) {
    case 9:
      if constexpr (AW == 2 && C::kSkinny && (EPI == EPI_QKV || EPI == EPI_SILU || EPI == EPI_SILU_I || EPI == EPI_LOGITS))
        if (a.nx) { hipLaunchKernelGGL((gemm_kernel<AW, EPI, 9, SHAPE, true>), grid, block, 0, s, a); break; }
      if (a.nx) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gemm_kernel<AW, EPI, 9, SHAPE>), grid, block, 0, s, a);
      break;
    case 24: hipLaunchKernelGGL((gemm_kernel<AW, EPI, 24, SHAPE>), grid, block, 0, s, a); break;
    case 1: if constexpr (op) { hipLaunchKernelGGL((gemm_kernel<AW, EPI, 1, SHAPE>), grid, block, 0, s, a); break; }
            return hipErrorInvalidValue;
    case 2: if constexpr (op) { hipLaunchKernelGGL((gemm_kernel<AW, EPI, 2, SHAPE>), grid, block, 0, s, a); break; }
            return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Tile shape per launch: 32 x 64 (32 x 32 without column pairs) skinny tiles for at most 256 rows, 64 x 192 for 2-limb residual
// GEMMs with N = 576, 64 x 256 for the wide 2-limb GEMMs (q/k/v, gate/up, the head: N >= 768, at
// most 1/16 of a tile column idle at N = 960), 128 x 128 (64 x 128 for 4 limbs) otherwise.
template <int AW, int EPI>
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
  // skinny tiles up to 256 rows (a 128-token prompt: 2.42 -> 1.62 ms per forward; 256 sequences'
  // decoding step: 3.08 -> 2.08 ms), except for the head beyond 32 rows, whose 28 MB of weights each
  // 32-row block would read again (the 64-row tiles read them half as often)
  if (a.M <= 256 && (EPI != EPI_LOGITS || a.M <= 32)) {
    if (a.nx && (a.K != 576 || a.M > 4 || !a.ngain || a.nsh < 10 || a.nsh > 40)) return hipErrorInvalidValue;
    if constexpr (EPI == EPI_SILU || EPI == EPI_SILU_I || EPI == EPI_QKV) return launch_gemm_cfg<AW, EPI, kShapeSkinny>(a, s);
    else return launch_gemm_cfg<AW, EPI, kShapeSkinny32>(a, s);
  }
  if (a.nx) return hipErrorInvalidValue;   // the RMSNorm prologue is a skinny-tile one
  if constexpr (AW == 2 && EPI == EPI_RESID)
    if (a.N % 192 == 0 && a.N % 128 != 0) return launch_gemm_cfg<AW, EPI, kShapeNarrow>(a, s);
  if constexpr (AW == 2 && EPI != EPI_RESID)
    if (a.N >= 768) return launch_gemm_cfg<AW, EPI, kShapeRow>(a, s);
  return launch_gemm_cfg<AW, EPI, kShapeSquare>(a, s);
}

// thread = 4 consecutive elements (k = 4 i .. 4 i + 3) of one row of the padded [M, Kp] operand
template <int SW, int W>
__global__ __launch_bounds__(256) void split_kernel(const void* a, int M, int K, int Kp, uint8_t* planes) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, n4 = (size_t)M * (Kp / 4);
  if (i >= n4) return;
  const size_t m = i / (Kp / 4), k = (i % (Kp / 4)) * 4;
  int32_t v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const size_t j = m * K + k + e;
    v[e] = k + e >= (size_t)K ? 0
           : SW == 1        ? (int32_t)((const int8_t*)a)[j]
           : SW == 2        ? (int32_t)((const int16_t*)a)[j]
                            : ((const int32_t*)a)[j];
  }
  const size_t n = (size_t)M * Kp;
#pragma unroll
  for (int l = 0; l < W; ++l) *(uint32_t*)(planes + l * n + plane_offset(m, k, M)) = limb_word(v, l, W);
}

// Weights [N, K] row-major -> fragment order over Kp columns (kernels.h swizzle_weights): thread =
// 16 bytes; columns past K and rows past N are zero
__global__ __launch_bounds__(256) void swizzle_kernel(const int8_t* W, int N, int K, int Kp, int8_t* Wf) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, ks = Kp / 32;
  if (i >= (size_t)((N + 31) / 32) * ks * 64) return;
  const int lane = (int)(i & 63);
  const size_t kc = (i >> 6) % ks, nb = (i >> 6) / ks;
  const size_t n = nb * 32 + (lane & 31), k = kc * 32 + 16 * (lane >> 5);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (n < (size_t)N) {
    const int8_t* src = W + n * K + k;
    if (K % 16 == 0 && k + 16 <= (size_t)K) {
      v = *(const uint4*)src;
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
      for (int b = 0; b < 16; ++b)
        if (k + b < (size_t)K) w[b >> 2] |= (uint32_t)(uint8_t)src[b] << (8 * (b & 3));
      v = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  *(uint4*)(Wf + w_frag((int)nb, (int)ks, (int)kc, lane)) = v;   // = Wf + 16 i
}

// out = SAT(RS(acc * mult[n], shift[n]), out_bits): thread = one element
template <typename OT>
__global__ __launch_bounds__(256) void requant_kernel(const int64_t* acc, int M, int N, const int32_t* mult,
                                                      const int32_t* shift, int out_bits, OT* out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * N) return;
  const int n = (int)(i % N);
  out[i] = (OT)sat(rs(acc[i] * (int64_t)mult[n], shift[n]), out_bits);
}

__global__ __launch_bounds__(256) void coef_kernel(const int32_t* mult, const int32_t* shift, const int32_t* wsum,
                                                   int N, double2* coef) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int sh = shift[n];
  const double c0 = ldexp((double)mult[n], -sh);
  coef[n] = make_double2(c0, fma((double)wsum[n] * 128.0, c0, ldexp(0.5, -sh)));
}

__global__ __launch_bounds__(256) void colsum_kernel(const int8_t* W, int N, int K, int32_t* wsum) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;
  int32_t s = 0;
  for (int k = lane; k < K; k += 64) s += W[(size_t)n * K + k];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) wsum[n] = s;
}

// ------------------------------------------------------------------------------ embed
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* ids, int M, const int8_t* emb_q,
                                                    const int32_t* emb_m, const int32_t* emb_sh,
                                                    int32_t* x, int* flag) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;     // 4 elements per thread
  if (t >= (size_t)M * (kD / 4)) return;
  const int row = (int)(t / (kD / 4)), c4 = (int)(t % (kD / 4));
  int64_t id = ids[row];
  if (id < 0 || id >= kV) { atomicOr(flag, 2); id = 0; }
  const uint32_t q4 = *(const uint32_t*)(emb_q + (size_t)id * kD + 4 * c4);
  const int64_t mu = emb_m[id];
  const int sh = emb_sh[id];
  int4 o;
  o.x = (int32_t)rs((int64_t)(int8_t)(q4 & 0xFF) * mu, sh);
  o.y = (int32_t)rs((int64_t)(int8_t)((q4 >> 8) & 0xFF) * mu, sh);
  o.z = (int32_t)rs((int64_t)(int8_t)((q4 >> 16) & 0xFF) * mu, sh);
  o.w = (int32_t)rs((int64_t)(int8_t)(q4 >> 24) * mu, sh);
  *(int4*)(x + (size_t)row * kD + 4 * c4) = o;
}

// ------------------------------------------------------------------------------ rmsnorm
// LPR lanes per row: 16 (4 rows per wave, for many rows) or 64 (a wave per row: a quarter of the
// serial work per lane, for the few rows of a decoding step).  Lane c of a row holds the VW = 64 /
// LPR columns 64 k + VW c .. + VW - 1, k = 0..8, so loads are 4 VW bytes, the limb bytes of a
// lane's VW columns leave together, and the row sums reduce inside the lane group, where every lane
// evaluates its own row's U.  Every product is a 32 x 32 -> 64 bit multiply-add: the squares through
// the 16-bit halves of x (python/intref.py:170-172), z = RS(x U, 16) with U < 2^29 and |z| <= 2^24
// (|x U| <= 2^40 since |x| <= sqrt(S)), then 3 z gain.  With int16 gains (the model's,
// python/intref.py:126-130) |3 z gain| < 2^41, so for output shifts in [10, 40] the shifted value
// fits int32 and saturates with one clamp; other shifts take the general int64 path.  WIDE: gains
// anywhere in int32 (the operator entry point), 3 gain and the product formed in int64
// (|3 z gain| < 2^58) and saturated before narrowing.  u_out / z_out (trace only, nullable): U per
// row and z per element (python/intref.py:183).
template <int OB, bool WIDE, int LPR>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const int32_t* x, int M, const int32_t* gain,
                                                      int sh_out, int bits_out, uint8_t* planes, void* plain,
                                                      int32_t* u_out, int32_t* z_out) {
  static_assert(LPR == 16 || LPR == 64, "16 or 64 lanes per row");
  constexpr int VW = 64 / LPR;
  const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR, c = threadIdx.x % LPR;
  const int rowc = min(row, M - 1);   // rows past M compute on row M - 1 and store nothing
  const int32_t* xr = x + (size_t)rowc * kD + VW * c;
  int32_t v[9][VW], g3[9][VW];
  auto load = [](const int32_t* p, int32_t (&d)[VW]) __attribute__((always_inline)) {
    if constexpr (VW == 4) {
      const int4 t = *(const int4*)p;
      d[0] = t.x; d[1] = t.y; d[2] = t.z; d[3] = t.w;
    } else {
      d[0] = *p;
    }
  };
  int64_t A = 0, B = 0, Cs = 0;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    load(xr + 64 * k, v[k]);
    load(gain + 64 * k + VW * c, g3[k]);
  }
#pragma unroll
  for (int k = 0; k < 9; ++k)
#pragma unroll
    for (int r = 0; r < VW; ++r) {
      const int32_t hi = v[k][r] >> 16, lo = v[k][r] & 0xFFFF;
      A += (int64_t)hi * hi; B += (int64_t)hi * lo; Cs += (int64_t)lo * lo;
      if constexpr (!WIDE) g3[k][r] *= 3;
    }
  A = group_sum64<LPR>(A);
  B = group_sum64<LPR>(B);
  Cs = group_sum64<LPR>(Cs);
  const int32_t U = (int32_t)norm_U(norm_total(A, B, Cs));   // < 2^29
  if (row >= M) return;
  if (u_out && c == 0) u_out[row] = U;
  const size_t pl = (size_t)M * kD, m64 = (size_t)M * 64;
  // the output shift is uniform: one copy of the loop per path
  auto body = [&](auto FAST) __attribute__((always_inline)) {
    const int64_t rnd = (int64_t)1 << (min(max(sh_out, 10), 40) - 1);
    auto zof = [&](int32_t xv) -> int32_t { return (int32_t)(((int64_t)xv * U + 32768) >> 16); };
    auto norm1 = [&](int32_t xv, int32_t gv) -> int32_t {
      const int32_t z = zof(xv);
      if constexpr (WIDE) {
        return (int32_t)sat(rs((int64_t)z * (3 * (int64_t)gv), sh_out), bits_out);
      } else if constexpr (decltype(FAST)::value) {
        const int32_t q = (int32_t)(((int64_t)z * gv + rnd) >> sh_out);
        return OB == 2 ? min(max(q, -32768), 32767) : q;
      } else {
        return (int32_t)sat(rs((int64_t)z * gv, sh_out), bits_out);
      }
    };
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      int32_t o[VW];
#pragma unroll
      for (int r = 0; r < VW; ++r) o[r] = norm1(v[k][r], g3[k][r]);
      const size_t e = (size_t)row * kD + 64 * k + VW * c;
      if (planes) {   // K-blocked planes: columns 64 k + VW c .. of the row at k M 64 + row 64 + VW c
        uint8_t* pb = planes + k * m64 + (size_t)row * 64 + VW * c;
#pragma unroll
        for (int l = 0; l < OB; ++l) {
          if constexpr (VW == 4) *(uint32_t*)(pb + l * pl) = limb_word(o, l, OB);
          else pb[l * pl] = (uint8_t)limb_byte(o[0], l, OB);
        }
      }
      if (plain) {
        if constexpr (VW == 4 && OB == 2) *(uint2*)((int16_t*)plain + e) = make_uint2(pack16(o[0], o[1]), pack16(o[2], o[3]));
        else if constexpr (VW == 4) *(int4*)((int32_t*)plain + e) = make_int4(o[0], o[1], o[2], o[3]);
        else if constexpr (OB == 2) ((int16_t*)plain)[e] = (int16_t)o[0];
        else ((int32_t*)plain)[e] = o[0];
      }
      if (z_out) {
        if constexpr (VW == 4) *(int4*)(z_out + e) = make_int4(zof(v[k][0]), zof(v[k][1]), zof(v[k][2]), zof(v[k][3]));
        else z_out[e] = zof(v[k][0]);
      }
    }
  };
  if (!WIDE && sh_out >= 10 && sh_out <= 40) body(std::true_type{});
  else body(std::false_type{});
}

// ------------------------------------------------------------------------------ rope
__global__ __launch_bounds__(256) void rope_kernel(int16_t* qkv, int M, const int32_t* pos,
                                                   const int32_t* cosT, const int32_t* sinT,
                                                   int sh_q, int bits_q, int sh_k, int bits_k) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;     // one (d, d+32) pair
  if (t >= (size_t)M * 384) return;
  const int row = (int)(t / 384), p = (int)(t % 384), h = p >> 5, d = p & 31;
  const int col = h * 64 + d;                                    // heads 0..8 q, 9..11 k
  const int sh = h < 9 ? sh_q : sh_k, bits = h < 9 ? bits_q : bits_k;
  int16_t* r = qkv + (size_t)row * kQKVN + col;
  const int64_t a1 = r[0], a2 = r[32];
  const int ps = pos[row];
  const int64_t c = cosT[ps * 32 + d], s = sinT[ps * 32 + d];
  r[0] = (int16_t)sat(rs(a1 * c - a2 * s, sh), bits);
  r[32] = (int16_t)sat(rs(a2 * c + a1 * s, sh), bits);
}

// ------------------------------------------------------------------------------ silu gate
template <int OB>
__global__ __launch_bounds__(256) void silu_kernel(const int16_t* gu, int M, const int32_t* silu,
                                                   int sh, int bits, uint8_t* planes, void* plain, int32_t* sg_out) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (size_t)M * kDFF) return;
  const size_t row = t / kDFF, j = t % kDFF;
  // gu rows hold [gate 32 | up 32] blocks: gate j at 64 (j / 32) + j % 32, up j 32 further
  const size_t gi = row * (2 * kDFF) + 64 * (j / 32) + j % 32;
  const int g = gu[gi];
  const int64_t u = gu[gi + 32];
  const int32_t o = (int32_t)sat(rs((int64_t)silu[g + 32768] * u, sh), bits);
  if (sg_out) sg_out[t] = silu[g + 32768];
  if (planes) {
#pragma unroll
    for (int l = 0; l < OB; ++l) planes[l * (size_t)M * kDFF + plane_offset32(row, j, M)] = (uint8_t)limb_byte(o, l, OB);
  }
  if (plain) {
    if constexpr (OB == 2) ((int16_t*)plain)[t] = (int16_t)o;
    else ((int32_t*)plain)[t] = o;
  }
}

// ------------------------------------------------------------------------------ attention
// A wave computes one query head 3 kvg + w (kv group kvg) for 32 queries of one sequence.  Up to 8
// key tiles a workgroup holds 4 such waves, consecutive in the order [query tile from the last]
// [sequence][head], so two workgroups fill a CU's 4 SIMDs with two waves each and share the exp
// table copy; the long rows run one wave per workgroup.  The waves share nothing but the exp
// table.  The longest query tiles are dispatched first.
//
// Scores run on v_mfma_i32_32x32x32_i8 as S^T[key][query] = K . Q^T over the head dimension (two
// K-steps of 32) with k = 256 KH + (KL' + 128), KL' = low byte - 128, KH = signed high byte, and q
// likewise or in the digits of attn_q_digits (index_maps.h).  A-operand row i carries key pi(i) = 16 ((i >> 2) & 1) + 4 (i >> 3) + (i & 3) of the
// key tile, the key that output row i denotes, so lane 32 h + c ends with query c and keys
// 16 h + j (output register j) of the tile: 16 consecutive keys of one query, which is the
// B-operand layout of ctx^T[d][query] = sum_key V^T[d][key] P^T[key][query] with operand byte j =
// key 16 h + j.  V^T limb planes (kernels.h) supply the matching A operand.  Key tiles are 32-row
// blocks aligned to row 0 of the batch; keys outside [sequence start, query] are masked.
//
// Exact sums (all partial MFMA sums fit int32):
//   sum_d q k = 65536 S_HH + 256 (S_HL + S_LH) + S_LL + 128 sum_d q
// with q in the digits of attn_q_digits (S_HH and S_HL with the high digits qh + qx), so the key
// rows need no sums; with q in k's form instead (the register-resident scores),
//   sum_d q k = 65536 S_HH + 256 (S_HL + S_LH) + S_LL + 128 (sum_d q + sum_d k) - 2^20
//   sum_key P v = 65536 C_1H + 256 (C_1L + C_0H) + C_0L + 128 sum_key P
// where P = 256 R1 + P0 with P0 = sext(P & 255) and R1 = (P + 128) >> 8 in [0, 256] (R1 goes
// into the MFMA as up to three int8 parts): a key with P = 0 adds nothing, so masked keys and
// the rows beyond a sequence need no correction terms.
//
// NKT > 0: the packed int16 scores of up to NKT key tiles stay in registers between the row-max,
// exp-sum and probability passes; NKT == 0: every pass recomputes the scores (long sequences).
constexpr int32_t kMasked = -32768;   // no score exceeds it, so the row max never picks it

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int32_t sum16x8(u32x4 d, int32_t s = 0) {   // s + the 8 int16 values in d
#pragma unroll
  for (int i = 0; i < 4; ++i) s += ((int32_t)(d[i] << 16) >> 16) + ((int32_t)d[i] >> 16);
  return s;
}

template <int OB, int NKT, int WPG, int KS = 1, bool KP = false>
__global__ __launch_bounds__(64 * WPG) __attribute__((amdgpu_waves_per_eu(2))) void attn_kernel(AttnArgs a) {
  static_assert(WPG == 1 || WPG == 4, "one wave per workgroup, or 4 waves");
  static_assert(KS == 1 || KS == WPG, "key tiles split over the waves of one task");
  static_assert(!KP || NKT == 0, "k limb planes serve the recomputing passes");
  __shared__ int32_t etab[kDMax + 2];                              // exp table, etab[1537] = 0
  __shared__ __attribute__((aligned(16))) int32_t sklw[WPG][32];   // per wave: 128 * sum_d k per key
  __shared__ __attribute__((aligned(16))) v4i qxw[NKT == 0 ? WPG : 1][2][64];   // per wave: qx digits
  // KS > 1: the waves' partial row maxima, exp sums, context sums and probability sums
  __shared__ int32_t xmax[KS][32];
  __shared__ uint64_t xz[KS][32];
  __shared__ int32_t xc[KS > 1 ? 6 * 16 : 1][64];
  __shared__ int32_t xsp[KS > 1 ? 64 : 1];

  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  int32_t* const skl = sklw[WPG == 1 ? 0 : tid >> 6];
  v4i (*const qxs)[64] = qxw[NKT == 0 && WPG > 1 ? tid >> 6 : 0];
  // this wave's (sequence, query head 3 kvg + w, query tile qt)
  int seq, kvg, w, qt;
  bool idle = false;
  if constexpr (WPG == 1 || KS > 1) {
    seq = blockIdx.x;
    kvg = blockIdx.y / 3;
    w = blockIdx.y % 3;
    qt = (a.q_first >> 5) + gridDim.z - 1 - blockIdx.z;
  } else {
    // task = 4 blockIdx.x + wave over [query tiles from the last][sequences][heads]
    const int nqt = (a.max_T + 31) / 32 - (a.q_first >> 5), per = a.B * kNH;
    const int task = 4 * (int)blockIdx.x + (tid >> 6), qr = task / per, rem = task - qr * per;
    idle = qr >= nqt;
    seq = idle ? 0 : rem / kNH;
    kvg = rem % kNH / 3;
    w = rem % 3;
    qt = (a.q_first >> 5) + nqt - 1 - qr;
  }
  const int s0 = a.seq_off[seq], T = a.kv_len ? a.kv_len : a.seq_off[seq + 1] - s0;
  idle = idle || 32 * qt >= T;
  if ((WPG == 1 || KS > 1) && idle) return;   // uniform over the workgroup
  // the exp table's loads go out first; their LDS stores and the barrier follow the query setup,
  // so the two memory round trips overlap.  Idle waves (4-wave workgroups) run the setup on a
  // valid query tile (their own may lie before the first) and leave after the barrier.
  constexpr int kTabPer = (kDMax + 2 + 64 * WPG - 1) / (64 * WPG);
  int32_t tabv[kTabPer];
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + 64 * WPG * j;
    tabv[j] = i <= kDMax ? a.exp_tab[i] : 0;
  }
  if (idle) qt = max(qt, a.q_first >> 5);

  const int hh = 3 * kvg + w;
  const int q0 = s0 + 32 * qt, qlast = min(q0 + 31, s0 + T - 1), qi = q0 + c;
  const int g0 = s0 >> 5, ntile = (qlast >> 5) - g0 + 1;
  const int pic = attn_key_perm(c);
  const int sh = a.shift_s;
  const int vts = vt_stride_for(a.M);

  // B operand: query qi (rows past the sequence read its last row), d = 32 s + 16 h + 0..15.  The
  // recomputing passes (kDig) take q as the digits of attn_q_digits (ql, qh; qx in LDS, read only in
  // waves where some q >= 32640), which spares them the per-key sums of k; with the scores held in
  // registers q takes k's form (low byte - 128, signed high byte) and the key sums go through LDS
  // (fewer registers and no branch in the one score pass; measured faster there)
  constexpr bool kDig = NKT == 0;
  v4i ql[2], qh[2];
  int32_t cq;
  bool qbig = false;
  if constexpr (!kDig) {
    const int16_t* qp = a.qkv + (size_t)min(qi, qlast) * kQKVN + hh * 64 + 16 * h;
    int32_t sum = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 d0 = *(const u32x4*)(qp + 32 * s), d1 = *(const u32x4*)(qp + 32 * s + 8);
      ql[s] = v4i{(int)lo_bytes16(d0[0], d0[1]), (int)lo_bytes16(d0[2], d0[3]), (int)lo_bytes16(d1[0], d1[1]),
                  (int)lo_bytes16(d1[2], d1[3])};
      qh[s] = v4i{(int)hi_bytes16(d0[0], d0[1]), (int)hi_bytes16(d0[2], d0[3]), (int)hi_bytes16(d1[0], d1[1]),
                  (int)hi_bytes16(d1[2], d1[3])};
      sum = sum16x8(d1, sum16x8(d0, sum));
    }
    sum += __shfl_xor(sum, 32);
    cq = 128 * sum - (1 << 20) + (1 << (sh - 1));   // with the rounding offset of RS(., sh)
  } else {
    const int16_t* qp = a.qkv + (size_t)min(qi, qlast) * kQKVN + hh * 64 + 16 * h;
    int32_t sum = 0;
    uint32_t anyx = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 d0 = *(const u32x4*)(qp + 32 * s), d1 = *(const u32x4*)(qp + 32 * s + 8);
      uint32_t wl[4] = {0, 0, 0, 0}, wh[4] = {0, 0, 0, 0}, wx[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t wd = e < 8 ? d0[e >> 1] : d1[(e - 8) >> 1];
        const QDigits g = attn_q_digits((e & 1) ? (int32_t)wd >> 16 : (int32_t)(wd << 16) >> 16);
        wl[e >> 2] |= ((uint32_t)g.ql & 0xFFu) << (8 * (e & 3));
        wh[e >> 2] |= ((uint32_t)g.qh & 0xFFu) << (8 * (e & 3));
        wx[e >> 2] |= (uint32_t)g.qx << (8 * (e & 3));
      }
      ql[s] = v4i{(int)wl[0], (int)wl[1], (int)wl[2], (int)wl[3]};
      qh[s] = v4i{(int)wh[0], (int)wh[1], (int)wh[2], (int)wh[3]};
      qxs[s][lane] = v4i{(int)wx[0], (int)wx[1], (int)wx[2], (int)wx[3]};
      anyx |= wx[0] | wx[1] | wx[2] | wx[3];
      sum = sum16x8(d1, sum16x8(d0, sum));
    }
    qbig = __any(anyx != 0);
    sum += __shfl_xor(sum, 32);
    cq = 128 * sum + (1 << (sh - 1));   // with the rounding offset of RS(., sh)
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + 64 * WPG * j;
    if (i < kDMax + 2) etab[i] = tabv[j];
  }
  __syncthreads();
  if (idle) return;   // (no workgroup barrier follows)

  // K rows of key tile g for this lane (row pi(c) of the tile, d = 32 s + 16 h + 0..15), loaded
  // one tile ahead of their use: int16 values, or with KP their limb bytes (d[s][0] low, d[s][1] high)
  struct KRows { u32x4 d[2][2]; };
  const int16_t* const kbase = a.qkv + kD + kvg * 64 + 16 * h;   // row offsets below 2^31 elements
  const uint8_t* const kpbase = KP ? a.kpl + kvg * 128 + 16 * h : nullptr;   // likewise bytes
  auto load_k = [&](int g, KRows& kr) __attribute__((always_inline)) {
    const uint32_t row = (uint32_t)min(32 * g + pic, a.M - 1);
    if constexpr (KP) {
      const uint8_t* kp = kpbase + row * (uint32_t)(3 * 128);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        kr.d[s][0] = *(const u32x4*)(kp + 32 * s);
        kr.d[s][1] = *(const u32x4*)(kp + 64 + 32 * s);
      }
    } else {
      const int16_t* kp = kbase + row * (uint32_t)kQKVN;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        kr.d[s][0] = *(const u32x4*)(kp + 32 * s);
        kr.d[s][1] = *(const u32x4*)(kp + 32 * s + 8);
      }
    }
  };
  // Scores SAT16(RS(q.k, sh)) of key tile g for this lane's query, keys 16 h + j.  The sum
  // acc + 2^(sh-1) = 65536 wv + lo16 with lo16 in [0, 65536) is evaluated in int32 pieces.
  // MODE Raw (shift >= 16 only): sc = the high parts wv, whose shifted and clamped values are the
  // scores; the row max of the scores is that of wv, shifted and clamped (both maps are monotone).
  // MODE Dist: sc = the exp table index d = min(rm - score, 1537) for the row max rm, masked keys
  // 1537 (entry 0).  For shift >= 16 with s' = wv >> (sh - 16) and score = SAT16(s'), d is
  // med3(rm - s', rm - 32767, min(1537, rm + 32768)): s' in range gives min(rm - s', 1537)
  // (rm - s' <= rm + 32768); s' > 32767 means rm = 32767 and d = 0 = rm - 32767; s' < -32768 gives
  // min(1537, rm + 32768).  One median instead of a clamp, a difference and a min.
  auto scores = [&](int g, const KRows& kr, int32_t (&sc)[16], auto MODE, int32_t rm = 0) __attribute__((always_inline)) {
    constexpr int mode = decltype(MODE)::value;
    constexpr bool raw = mode == 1;
    constexpr int32_t masked = raw ? INT32_MIN : mode == 2 ? kDMax + 1 : kMasked;
    v4i kl[2], kh[2];
    int32_t ks = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 d0 = kr.d[s][0], d1 = kr.d[s][1];
      if constexpr (KP) {
        kl[s] = __builtin_bit_cast(v4i, d0);
        kh[s] = __builtin_bit_cast(v4i, d1);
        continue;
      }
      kl[s] = v4i{(int)lo_bytes16(d0[0], d0[1]), (int)lo_bytes16(d0[2], d0[3]), (int)lo_bytes16(d1[0], d1[1]),
                  (int)lo_bytes16(d1[2], d1[3])};
      kh[s] = v4i{(int)hi_bytes16(d0[0], d0[1]), (int)hi_bytes16(d0[2], d0[3]), (int)hi_bytes16(d1[0], d1[1]),
                  (int)hi_bytes16(d1[2], d1[3])};
      if constexpr (!kDig) ks = sum16x8(d1, sum16x8(d0, ks));
    }
    if constexpr (!kDig) {
      ks += __shfl_xor(ks, 32);
      skl[pic] = 128 * ks;   // lanes c and c + 32 store the same value
      __builtin_amdgcn_wave_barrier();
    }
    v16i a16 = v16i{}, a8 = v16i{}, a0 = v16i{};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      a16 = mfma32(kh[s], qh[s], a16);
      a8 = mfma32(kh[s], ql[s], a8);
      a8 = mfma32(kl[s], qh[s], a8);
      a0 = mfma32(kl[s], ql[s], a0);
    }
    if (kDig && qbig) {   // the qx digits of queries >= 32640
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const v4i qx = qxs[s][lane];
        a16 = mfma32(kh[s], qx, a16);
        a8 = mfma32(kl[s], qx, a8);
      }
    }
    int32_t lo[16], wv[16];
    if constexpr (!kDig) {
      const v4i* kk = (const v4i*)&skl[16 * h];
      const v4i k4[4] = {kk[0], kk[1], kk[2], kk[3]};
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        lo[j] = a8[j] * 256 + a0[j] + k4[j >> 2][j & 3] + cq;
        wv[j] = a16[j] + (lo[j] >> 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        lo[j] = a8[j] * 256 + a0[j] + cq;
        wv[j] = a16[j] + (lo[j] >> 16);
      }
    }
    // the shift is uniform: one branch per tile
    if constexpr (raw) {
#pragma unroll
      for (int j = 0; j < 16; ++j) sc[j] = wv[j];
    } else if (mode == 2 && sh >= 16) {
      const int32_t dl = rm - 32767, dh = min(kDMax + 1, rm + 32768);
#pragma unroll
      for (int j = 0; j < 16; ++j) sc[j] = min(max(rm - (wv[j] >> (sh - 16)), dl), dh);
    } else if (sh >= 16) {
#pragma unroll
      for (int j = 0; j < 16; ++j) sc[j] = min(max(wv[j] >> (sh - 16), -32768), 32767);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        sc[j] = min(max(min(max(wv[j], -32769), 32768) * (1 << (16 - sh)) + ((lo[j] & 0xFFFF) >> sh), -32768), 32767);
      if constexpr (mode == 2) {
#pragma unroll
        for (int j = 0; j < 16; ++j) sc[j] = min(rm - sc[j], kDMax + 1);
      }
    }
    // keys past the query (the diagonal tile) and before the sequence start (its first tile when
    // the sequence does not start on a tile boundary): key 32 g + 16 h + j
    if (32 * g + 31 > q0) {
      const int last = qi - 32 * g - 16 * h;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (j > last) sc[j] = masked;
    }
    if (32 * g < s0) {
      const int first = s0 - 32 * g - 16 * h;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (j < first) sc[j] = masked;
    }
  };
  using Full = std::integral_constant<int, 0>;
  using Raw = std::integral_constant<int, 1>;
  using Dist = std::integral_constant<int, 2>;

  v16i C16[2], C8[2], C0[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) C16[i] = C8[i] = C0[i] = v16i{};
  int32_t SP = 0;
  double Zs = 0.0, rZs = 0.0, Zhs = 0.0;   // Z 2^-16, RN(2^16 / Z), floor(Z / 2) 2^-16
  // P = floor((e 65536 + floor(Z / 2)) / Z) (python/intref.py:245-246).  num / Z <= 65536.5 (e is
  // a term of Z), and num rZ + 2^-30 evaluated with one fma is within 2^-36 of num / Z + 2^-30, so
  // its floor is the true quotient or one more; the exact float64 remainder takes the one back.
  // Everything runs scaled by 2^-16 (num 2^-16 = e + floor(Z / 2) 2^-16 is one exact add), which
  // changes no rounding: the scaled quotient estimate and remainder are the unscaled ones exactly.
  auto prob = [&](int32_t e) __attribute__((always_inline)) -> int32_t {
    const double num = (double)e + Zhs;
    const double q = floor(fma(num, rZs, 0x1p-30));
    const double rem = fma(-q, Zs, num);
    return (int32_t)q - (rem < 0.0 ? 1 : 0);
  };
  // probabilities of key tile g (e values) into limb operands, then the P.V MFMAs.  R1 =
  // (P + 128) >> 8 in [0, 256] goes in as P1 = min(R1, 127) plus, in the waves where some R1
  // exceeds 127 (a key holding about half the weight or more), P1b = min(R1 - P1, 127) and
  // P1c = R1 - P1 - P1b, all with the weight of P1.
  // V^T limb fragments of key tile g (A operands of the two 32-row d tiles), loaded one tile ahead
  struct VFrag { v4i L[2], H[2]; };
  const size_t vpl = (size_t)192 * vts;
  const uint8_t* const vbase = a.vt + (size_t)(kvg * 64 + c) * vts + 16 * h;
  auto load_v = [&](int g, VFrag& vf) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const uint8_t* vp = vbase + (size_t)(32 * dt) * vts + (uint32_t)(32 * g);
      vf.L[dt] = *(const v4i*)vp;
      vf.H[dt] = *(const v4i*)(vp + vpl);
    }
  };
  auto pv = [&](const VFrag& vf, const int32_t (&ev)[16]) __attribute__((always_inline)) {
    // byte r of a word = element 4 i + r
    auto bytes4 = [](const int32_t (&v)[4]) __attribute__((always_inline)) {
      return __builtin_amdgcn_perm(__builtin_amdgcn_perm(v[3], v[2], 0x0c0c0400u),
                                   __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u), 0x05040100u);
    };
    uint32_t w0[4], w1[4];
    int32_t R1s[16];   // kept for the extra parts, which only waves with some R1 > 127 form
    int32_t rmax = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int32_t P[4], p1[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        P[r] = prob(ev[4 * i + r]);
        R1s[4 * i + r] = (P[r] + 128) >> 8;
        rmax = max(rmax, R1s[4 * i + r]);
        p1[r] = min(R1s[4 * i + r], 127);
      }
      SP += (P[0] + P[1]) + (P[2] + P[3]);
      w0[i] = bytes4(P);    // low bytes of P
      w1[i] = bytes4(p1);
    }
    const v4i P0 = v4i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
    const v4i P1 = v4i{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
    const v4i* VL = vf.L;
    const v4i* VH = vf.H;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      C16[dt] = mfma32(VH[dt], P1, C16[dt]);
      C8[dt] = mfma32(VH[dt], P0, C8[dt]);
      C8[dt] = mfma32(VL[dt], P1, C8[dt]);
      C0[dt] = mfma32(VL[dt], P0, C0[dt]);
    }
    if (__any(rmax > 127)) {
      uint32_t wb[4], wc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int32_t pb[4], pc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int32_t R1 = R1s[4 * i + r], p1 = min(R1, 127);
          pb[r] = min(R1 - p1, 127);
          pc[r] = R1 - p1 - pb[r];
        }
        wb[i] = bytes4(pb);
        wc[i] = bytes4(pc);
      }
      const v4i P1b = v4i{(int)wb[0], (int)wb[1], (int)wb[2], (int)wb[3]};
      const v4i P1c = v4i{(int)wc[0], (int)wc[1], (int)wc[2], (int)wc[3]};
      const bool three = __any(rmax > 254);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        C16[dt] = mfma32(VH[dt], P1b, C16[dt]);
        C8[dt] = mfma32(VL[dt], P1b, C8[dt]);
        if (three) {
          C16[dt] = mfma32(VH[dt], P1c, C16[dt]);
          C8[dt] = mfma32(VL[dt], P1c, C8[dt]);
        }
      }
    }
  };
  auto set_z = [&](int64_t Z, bool halves = true) __attribute__((always_inline)) {
    if (halves) Z += __shfl_xor(Z, 32);   // the two lane halves' keys (already added: false)
    const double Zd = (double)Z;   // Z < 2^43: exact
    Zs = Zd * 0x1p-16;
    rZs = (1.0 / Zd) * 65536.0;
    Zhs = (double)(Z >> 1) * 0x1p-16;
  };

  int32_t rowmax = kMasked;
  // with up to 5 key tiles the registers hold K and V one tile ahead of their use as well
  constexpr bool ahead = NKT > 0 && NKT <= 5 && KS == 1;
  KRows kr[ahead ? 2 : 1];
  VFrag vf[ahead ? 2 : 1];
  // KS > 1: wave ks of the task takes key tiles ks, ks + KS, ... (tile tg(i) of its slot i, nloc
  // slots); the waves meet in LDS for the row max, the exp sum and the context sums, and wave 0
  // writes the context
  const int ks = KS > 1 ? tid >> 6 : 0;
  const int nloc = KS == 1 ? ntile : ks < ntile ? (ntile - ks + KS - 1) / KS : 0;
  auto tg = [&](int i) __attribute__((always_inline)) { return KS == 1 ? i : ks + KS * i; };
  auto combine_max = [&](int32_t m) __attribute__((always_inline)) {   // m: both lane halves' max
    if constexpr (KS > 1) {
      if (h == 0) xmax[ks][c] = m;
      __syncthreads();
#pragma unroll
      for (int k = 0; k < KS; ++k) m = max(m, xmax[k][c]);
    }
    return m;
  };
  auto combine_z = [&](uint64_t Z) __attribute__((always_inline)) {   // the exp sum setup
    if constexpr (KS > 1) {
      Z += __shfl_xor(Z, 32);
      if (h == 0) xz[ks][c] = Z;
      __syncthreads();
      Z = 0;
#pragma unroll
      for (int k = 0; k < KS; ++k) Z += xz[k][c];
      set_z((int64_t)Z, false);
    } else {
      set_z((int64_t)Z, true);
    }
  };
  // context sums: wave 0's partial sums seed LDS, the other waves add theirs (exact int32 sums of
  // the single-wave totals) and leave, wave 0 reads the totals back; returns false in the waves
  // that leave
  auto combine_ctx = [&]() __attribute__((always_inline)) -> bool {
    if constexpr (KS > 1) {
      if (ks == 0) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            xc[(0 * 2 + dt) * 16 + j][lane] = C16[dt][j];
            xc[(1 * 2 + dt) * 16 + j][lane] = C8[dt][j];
            xc[(2 * 2 + dt) * 16 + j][lane] = C0[dt][j];
          }
        xsp[lane] = SP;
      }
      __syncthreads();
      if (ks != 0) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            atomicAdd(&xc[(0 * 2 + dt) * 16 + j][lane], C16[dt][j]);
            atomicAdd(&xc[(1 * 2 + dt) * 16 + j][lane], C8[dt][j]);
            atomicAdd(&xc[(2 * 2 + dt) * 16 + j][lane], C0[dt][j]);
          }
        atomicAdd(&xsp[lane], SP);
      }
      __syncthreads();
      if (ks != 0) return false;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          C16[dt][j] = xc[(0 * 2 + dt) * 16 + j][lane];
          C8[dt][j] = xc[(1 * 2 + dt) * 16 + j][lane];
          C0[dt][j] = xc[(2 * 2 + dt) * 16 + j][lane];
        }
      SP = xsp[lane];
    }
    return true;
  };

  // Long rows: every pass recomputes the scores, which the exp-sum and P.V passes take as exp table
  // indices (MODE Dist: masked keys at the zero entry, so no key tests).  The row-max and exp-sum passes
  // load the K rows of the wave's next tile while the current one computes (two slots per
  // iteration, so the buffer of each is a compile-time choice); the P.V pass, whose registers hold
  // the context sums, loads each tile's K and V at its start.
  auto recompute_passes = [&]() __attribute__((always_inline)) {
    KRows kb[2];
    auto max_pass = [&](auto RAW) __attribute__((always_inline)) {
      int32_t m = INT32_MIN;
      if (KS == 1 || nloc > 0) load_k(g0 + tg(0), kb[0]);
#pragma unroll 1
      for (int t0 = 0; t0 < nloc; t0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = t0 + u;
          if (t < nloc) {
            if (t + 1 < nloc) load_k(g0 + tg(t + 1), kb[u ^ 1]);
            int32_t sc[16];
            scores(g0 + tg(t), kb[u], sc, RAW);
#pragma unroll
            for (int j = 0; j < 16; ++j) m = max(m, sc[j]);
          }
        }
      }
      return m;
    };
    if (sh >= 16) rowmax = min(max(max_pass(Raw{}) >> (sh - 16), -32768), 32767);
    else rowmax = max_pass(Full{});
    rowmax = combine_max(max(rowmax, __shfl_xor(rowmax, 32)));
    {
      // the scores come as exp table indices (masked keys: the zero entry)
      auto ex = [&](int d) __attribute__((always_inline)) -> uint32_t { return (uint32_t)etab[d]; };
      uint64_t Z = 0;   // e <= 2^30: sums of three fit uint32
      if (KS == 1 || nloc > 0) load_k(g0 + tg(0), kb[0]);
#pragma unroll 1
      for (int t0 = 0; t0 < nloc; t0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = t0 + u;
          if (t < nloc) {
            if (t + 1 < nloc) load_k(g0 + tg(t + 1), kb[u ^ 1]);
            int32_t sc[16];
            scores(g0 + tg(t), kb[u], sc, Dist{}, rowmax);
#pragma unroll
            for (int j = 0; j < 15; j += 3) Z += ex(sc[j]) + ex(sc[j + 1]) + ex(sc[j + 2]);
            Z += ex(sc[15]);
          }
        }
      }
      combine_z(Z);
#pragma unroll 1
      for (int t = 0; t < nloc; ++t) {
        int32_t sc[16];
        load_k(g0 + tg(t), kr[0]);
        load_v(g0 + tg(t), vf[0]);
        scores(g0 + tg(t), kr[0], sc, Dist{}, rowmax);
#pragma unroll
        for (int j = 0; j < 16; ++j) sc[j] = (int32_t)ex(sc[j]);
        pv(vf[0], sc);
      }
    }
  };
  if constexpr (NKT > 0) {
    constexpr int NT = (NKT + KS - 1) / KS;   // key tiles per wave
    uint32_t pk[NT][8];   // packed int16 scores
    if constexpr (ahead) load_k(g0, kr[0]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (tg(t) < ntile) {
        if constexpr (ahead) {
          if (t + 1 < ntile) load_k(g0 + t + 1, kr[(t + 1) & 1]);
          else load_v(g0, vf[0]);   // the first V tile, while the last scores and the sums run
        } else {
          load_k(g0 + tg(t), kr[0]);
        }
        int32_t sc[16];
        scores(g0 + tg(t), kr[ahead ? t & 1 : 0], sc, Full{});
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pk[t][i] = ((uint32_t)sc[2 * i] & 0xFFFFu) | ((uint32_t)sc[2 * i + 1] << 16);
          rowmax = max(rowmax, max(sc[2 * i], sc[2 * i + 1]));
        }
      }
    }
    rowmax = combine_max(max(rowmax, __shfl_xor(rowmax, 32)));
    // The packed scores become packed byte offsets 4 min(rowmax - s, 1537) into the exp table
    // (rowmax - s lies in [0, 65535], so 16-bit lanes hold it and the shifted offset), 3 packed
    // operations per 2 keys, once for both lookup passes.  A masked key holds score kMasked, which
    // lies more than 1536 below the row max (table entry 1537 = 0) whenever the row max exceeds
    // kMasked + 1536.  In waves with a row whose every score is near -32768, the tiles holding keys
    // outside [sequence start, query] (the diagonal tile, and the first one when the sequence does
    // not start on a 32-row boundary) test the keys; the branch is uniform per tile.
    const bool clean = __all(rowmax > kMasked + kDMax);
    const u16x2 rm2 = (u16x2)(unsigned short)rowmax, cap2 = (u16x2)(unsigned short)(kDMax + 1);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (tg(t) < ntile) {
        if (!clean && (32 * (g0 + tg(t)) < s0 || 32 * (g0 + tg(t)) + 31 > q0)) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            uint32_t off[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              const int j = 2 * i + b, key = 32 * (g0 + tg(t)) + 16 * h + j;
              const int32_t sj = b ? (int32_t)pk[t][i] >> 16 : (int32_t)(pk[t][i] << 16) >> 16;
              off[b] = 4u * (uint32_t)(key < s0 || key > qi ? kDMax + 1 : min(rowmax - sj, kDMax + 1));
            }
            pk[t][i] = off[0] | (off[1] << 16);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            u16x2 d = rm2 - __builtin_bit_cast(u16x2, pk[t][i]);
            d = __builtin_elementwise_min(d, cap2) << (u16x2)(unsigned short)2;
            pk[t][i] = __builtin_bit_cast(uint32_t, d);
          }
        }
      }
    auto ex = [&](int t, int j) __attribute__((always_inline)) -> int32_t {
      const uint32_t p = pk[t][j >> 1], off = (j & 1) ? p >> 16 : p & 0xFFFFu;
      return *(const int32_t*)((const char*)etab + off);
    };
    // Z: e <= 2^30, so sums of three fit uint32
    uint64_t Z = 0;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (tg(t) < ntile) {
        uint32_t ev[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) ev[j] = ex(t, j);
#pragma unroll
        for (int j = 0; j < 15; j += 3) Z += ev[j] + ev[j + 1] + ev[j + 2];
        Z += ev[15];
      }
    combine_z(Z);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (tg(t) < ntile) {
        if constexpr (ahead) {
          if (t + 1 < ntile) load_v(g0 + t + 1, vf[(t + 1) & 1]);
        } else {
          load_v(g0 + tg(t), vf[0]);
        }
        int32_t ev[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) ev[j] = ex(t, j);
        pv(vf[ahead ? t & 1 : 0], ev);
      }
    if (!combine_ctx()) return;
  } else {
    recompute_passes();
    if (!combine_ctx()) return;
  }
  SP += __shfl_xor(SP, 32);

  if (qi > qlast || qi - s0 < a.q_first) return;
  // ctx of query qi, d = 32 dt + 8 b + 4 h + r (output register 4 b + r of tile dt)
  const int outM = a.kv_len ? a.out_M : a.M;
  const int qo = a.kv_len ? seq * (T - a.q_first) + qi - s0 - a.q_first : qi;   // output row
  const size_t orow = (size_t)qo * kD + hh * 64, pl = (size_t)outM * kD;
  // SAT(RS(acc, sh_ctx), bits_c) in float64, where every step is exact for the shifts the callers
  // admit (-30 .. 62): |C16| <= T 256 128 <= 2^29, so |acc| < 2^47; acc 2^-sh + 1/2 is exact
  // whenever its floor can differ from 0 or from a value past the saturation bounds
  const double sp128 = 128.0 * (double)SP, sc = ldexp(1.0, -a.sh_ctx);
  const double clo = -ldexp(1.0, a.bits_c - 1), chi = ldexp(1.0, a.bits_c - 1) - 1.0;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      int32_t cv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 4 * b + r;
        const double acc = fma((double)C16[dt][j], 65536.0, fma((double)C8[dt][j], 256.0, (double)C0[dt][j] + sp128));
        cv[r] = (int32_t)fmin(fmax(floor(fma(acc, sc, 0.5)), clo), chi);
      }
      const int d0 = 32 * dt + 8 * b + 4 * h;
      if (a.ctx_planes) {
#pragma unroll
        for (int l = 0; l < OB; ++l)
          *(uint32_t*)(a.ctx_planes + l * pl + plane_offset(qo, hh * 64 + d0, outM)) = limb_word(cv, l, OB);
      }
      if (a.ctx) {
        if constexpr (OB == 2) *(uint2*)((int16_t*)a.ctx + orow + d0) = make_uint2(pack16(cv[0], cv[1]), pack16(cv[2], cv[3]));
        else *(int4*)((int32_t*)a.ctx + orow + d0) = make_int4(cv[0], cv[1], cv[2], cv[3]);
      }
    }
}

// Decoding attention: one new query per sequence (the last of its kv_len cached rows) against
// all of them, python/intref.py:227-254 with T = kv_len and only the last query row.  Workgroup =
// one sequence and one kv group: NW waves per query head 3 kvg + hq (NW = 4 for few sequences,
// where the latency of one workgroup is the step's; 1 when the sequences fill the GPU).  The scores
// of all 3 heads come from MFMAs over 32-key tiles shared out among all the workgroup's waves (the
// 3 queries as B-operand columns) and go to LDS as SAT16 values with each wave's per-head max; then
// the keys go in 64-key chunks, chunk c to wave c % NW of each head: once the row max and the exp
// sum Z are known (through LDS and wave reductions), lane j forms key 64 c + j's probability
// P = floor((e 65536 + floor(Z / 2)) / Z) from a float64 quotient and an exact remainder
// correction; the lanes then, one per head dimension, sum P v over the chunk in int64 with each P
// taken from its lane by v_readlane, and the head's NW partial sums meet in LDS.  A wave's first
// value chunk is loaded before the reductions, so its latency hides behind them.  No key is
// masked: every cached key precedes the query.
// scores of 3 heads x kDecodeMaxKeys keys: 48 KB of LDS (kernels.h)
// LDS: exp table [1537] + 3 pad ints (the end stays 16-byte aligned), each wave's max of each head
// [3 NW][4] (an even count of ints, so the int64 arrays after them are 8-byte aligned), the exp
// sums [3 NW] and partial context sums [3 NW][64] as int64, the scores of 3 heads as int16, and per
// wave the 32 per-key sums of k of its current tile
__host__ __device__ inline int attn_decode_nmax(int NW) { return 12 * NW; }
__host__ __device__ inline size_t attn_decode_lds(int L, int NW) {
  return (size_t)(kDMax + 1 + 3) * 4 + (size_t)attn_decode_nmax(NW) * 4 + (size_t)3 * NW * (8 + 64 * 8) +
         (size_t)3 * ((L + 63) & ~63) * 2 + (size_t)3 * NW * 32 * 4;
}

template <int OB, int NW>
__global__ __launch_bounds__(64 * 3 * NW) void attn_decode_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) int32_t dsm[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hq = w / NW, kw = w % NW;
  const int seq = blockIdx.x, kvg = blockIdx.y, hh = 3 * kvg + hq;
  const int L = a.kv_len, Lp = (L + 63) & ~63;
  int32_t* etab = dsm;                                          // [1537] (+3 pad)
  int32_t* smax = dsm + kDMax + 1 + 3;                          // [3 NW][4]: each wave's max of each head
  int64_t* sz = (int64_t*)(smax + attn_decode_nmax(NW));        // [3 NW]
  int64_t* spart = sz + 3 * NW;                                 // [12][64]
  // the exp table's loads go out first and its LDS stores wait until after the scores (before the
  // first barrier), so the table's memory round trip overlaps the query and key loads
  constexpr int kTabPer = (kDMax + 1 + 64 * 3 * NW - 1) / (64 * 3 * NW);
  int32_t tabv[kTabPer];
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + 64 * 3 * NW * j;
    if (i <= kDMax) tabv[j] = a.exp_tab[i];
  }
  const int16_t* base = a.qkv + (size_t)a.seq_off[seq] * kQKVN;   // key 0 of the sequence
  int16_t* const sc_all = (int16_t*)(spart + 3 * NW * 64);      // [3][Lp]
  int32_t* const skl = (int32_t*)(sc_all + 3 * Lp) + 32 * w;     // per wave: 128 sum_d k per key

  // Scores of the 3 heads on v_mfma_i32_32x32x32_i8 with attn_kernel's operand forms and key order
  // (S^T = K . Q^T, k = 256 KH + KL' + 128 and q likewise, the per-key sums of k through LDS): the
  // B operand's columns 0..2 carry the heads' queries (the other columns repeat head 2 and are
  // dropped), and wave w of the 3 NW takes the 32-key tiles w, w + 3 NW, ...; lanes c < 3 of each
  // half end with head c's scores of keys 16 h + j, which go to LDS with the head's running max.
  const int c = lane & 31, h = lane >> 5, pic = attn_key_perm(c), sh = a.shift_s;
  v4i ql[2], qh[2];
  int32_t cq;
  {
    const int16_t* qp = base + (size_t)(L - 1) * kQKVN + (3 * kvg + min(c, 2)) * 64 + 16 * h;
    int32_t sum = 0;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const u32x4 d0 = *(const u32x4*)(qp + 32 * s2), d1 = *(const u32x4*)(qp + 32 * s2 + 8);
      ql[s2] = v4i{(int)lo_bytes16(d0[0], d0[1]), (int)lo_bytes16(d0[2], d0[3]), (int)lo_bytes16(d1[0], d1[1]),
                   (int)lo_bytes16(d1[2], d1[3])};
      qh[s2] = v4i{(int)hi_bytes16(d0[0], d0[1]), (int)hi_bytes16(d0[2], d0[3]), (int)hi_bytes16(d1[0], d1[1]),
                   (int)hi_bytes16(d1[2], d1[3])};
      sum = sum16x8(d1, sum16x8(d0, sum));
    }
    sum += __shfl_xor(sum, 32);
    cq = 128 * sum - (1 << 20) + (1 << (sh - 1));   // with the rounding offset of RS(., sh)
  }
  int32_t mxh = INT32_MIN;
  const int16_t* const kbase = base + kD + kvg * 64 + 16 * h;
  for (int tt = w; 32 * tt < L; tt += 3 * NW) {
    const int16_t* kp = kbase + (size_t)min(32 * tt + pic, L - 1) * kQKVN;   // keys past L re-read L - 1
    v4i kl[2], kh[2];
    int32_t ks = 0;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const u32x4 d0 = *(const u32x4*)(kp + 32 * s2), d1 = *(const u32x4*)(kp + 32 * s2 + 8);
      kl[s2] = v4i{(int)lo_bytes16(d0[0], d0[1]), (int)lo_bytes16(d0[2], d0[3]), (int)lo_bytes16(d1[0], d1[1]),
                   (int)lo_bytes16(d1[2], d1[3])};
      kh[s2] = v4i{(int)hi_bytes16(d0[0], d0[1]), (int)hi_bytes16(d0[2], d0[3]), (int)hi_bytes16(d1[0], d1[1]),
                   (int)hi_bytes16(d1[2], d1[3])};
      ks = sum16x8(d1, sum16x8(d0, ks));
    }
    ks += __shfl_xor(ks, 32);
    skl[pic] = 128 * ks;   // lanes c and c + 32 store the same value
    __builtin_amdgcn_wave_barrier();
    v16i a16 = v16i{}, a8 = v16i{}, a0 = v16i{};
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      a16 = mfma32(kh[s2], qh[s2], a16);
      a8 = mfma32(kh[s2], ql[s2], a8);
      a8 = mfma32(kl[s2], qh[s2], a8);
      a0 = mfma32(kl[s2], ql[s2], a0);
    }
    const v4i* kk = (const v4i*)&skl[16 * h];
    const v4i k4[4] = {kk[0], kk[1], kk[2], kk[3]};
    __builtin_amdgcn_wave_barrier();
    if (c < 3) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int32_t lo = a8[j] * 256 + a0[j] + k4[j >> 2][j & 3] + cq, wv = a16[j] + (lo >> 16);
        const int32_t sv = sh >= 16 ? min(max(wv >> (sh - 16), -32768), 32767)
                                    : min(max(min(max(wv, -32769), 32768) * (1 << (16 - sh)) + ((lo & 0xFFFF) >> sh), -32768), 32767);
        const int key = 32 * tt + 16 * h + j;
        if (key < L) {
          sc_all[c * Lp + key] = (int16_t)sv;
          mxh = max(mxh, sv);
        }
      }
    }
  }
  mxh = max(mxh, __shfl_xor(mxh, 32));
  if (lane < 3) smax[4 * w + lane] = mxh;
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + 64 * 3 * NW * j;
    if (i <= kDMax) etab[i] = tabv[j];
  }
  int16_t* const sc = sc_all + (size_t)hq * Lp;
  // the value rows of this wave's first chunk, loaded now (rows past L re-read row L - 1)
  const int16_t* vcol = base + kD + 192 + kvg * 64 + lane;
  int32_t vv[64];
  if (64 * kw < L) {
    const int n = min(64, L - 64 * kw);
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) vv[jj] = vcol[(size_t)(64 * kw + min(jj, n - 1)) * kQKVN];
  }
  __syncthreads();
  int32_t mx = INT32_MIN;
#pragma unroll
  for (int k = 0; k < 3 * NW; ++k) mx = max(mx, smax[4 * k + hq]);
  // Z = sum of the table entries of d = max - s <= 1536 (entries beyond are 0); Z >= 2^30
  int64_t Z = 0;
  for (int c = kw; 64 * c < L; c += NW) {
    const int j = 64 * c + lane;
    if (j < L) {
      const int d = mx - sc[j];
      Z += d <= kDMax ? etab[d] : 0;
    }
  }
  Z = group_sum64<64>(Z);
  if (lane == 0) sz[w] = Z;
  __syncthreads();
  Z = 0;
#pragma unroll
  for (int k = 0; k < NW; ++k) Z += sz[hq * NW + k];
  const int64_t zh = Z >> 1;
  const double zd = (double)Z;

  // P v over this wave's chunks: lane = head dimension
  int64_t cacc = 0;
  for (int c = kw; 64 * c < L; c += NW) {
    const int j = 64 * c + lane, n = min(64, L - 64 * c);
    if (c != kw) {
#pragma unroll
      for (int jj = 0; jj < 64; ++jj) vv[jj] = vcol[(size_t)(64 * c + min(jj, n - 1)) * kQKVN];
    }
    int32_t P = 0;
    if (j < L) {
      const int d = mx - sc[j];
      const int64_t num = (int64_t)(d <= kDMax ? etab[d] : 0) * 65536 + zh;   // < 2^47, exact in float64
      int64_t qt = (int64_t)floor((double)num / zd);
      const int64_t r = num - qt * Z;
      qt += r < 0 ? -1 : (r >= Z ? 1 : 0);
      P = (int32_t)qt;
    }
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) cacc += (int64_t)__builtin_amdgcn_readlane(P, jj) * vv[jj];
  }
  spart[w * 64 + lane] = cacc;
  __syncthreads();
  if (kw != 0) return;
#pragma unroll
  for (int k = 1; k < NW; ++k) cacc += spart[(w + k) * 64 + lane];

  // SAT(RS(acc, sh_ctx), bits_c) in float64: |acc| < 2^45, exact wherever the result is not
  // saturated (as in attn_kernel)
  const double clo = -ldexp(1.0, a.bits_c - 1), chi = ldexp(1.0, a.bits_c - 1) - 1.0;
  const int32_t cv = (int32_t)fmin(fmax(floor(fma((double)cacc, ldexp(1.0, -a.sh_ctx), 0.5)), clo), chi);
  const int outM = a.out_M, qo = seq;   // one output row per sequence
  const size_t pl = (size_t)outM * kD;
  if (a.ctx_planes) {
#pragma unroll
    for (int l = 0; l < OB; ++l) a.ctx_planes[l * pl + plane_offset(qo, hh * 64 + lane, outM)] = (uint8_t)limb_byte(cv, l, OB);
  }
  if (a.ctx) {
    if constexpr (OB == 2) ((int16_t*)a.ctx)[(size_t)qo * kD + hh * 64 + lane] = (int16_t)cv;
    else ((int32_t*)a.ctx)[(size_t)qo * kD + hh * 64 + lane] = cv;
  }
}

// V^T limb planes from qkv: thread = (d row, 4 consecutive token rows)
__global__ __launch_bounds__(256) void vt_kernel(const int16_t* qkv, int M, uint8_t* vt, int stride) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, ng = (size_t)stride / 4;
  if (i >= 192 * ng) return;
  const int d = (int)(i / ng), m0 = (int)(4 * (i % ng));
  int32_t v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = qkv[(size_t)min(m0 + r, M - 1) * kQKVN + kD + 192 + d];
  uint8_t* p = vt + (size_t)d * stride + m0;
  *(uint32_t*)p = limb_word(v, 0, 2);
  *(uint32_t*)(p + (size_t)192 * stride) = limb_word(v, 1, 2);
}

inline unsigned blocks_for(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t gemm(const GemmArgs& a, int a_bytes, int epi, hipStream_t s) {
  if (a.K % kBK != 0 || a.M <= 0 || a.N <= 0 || a.N % 4 != 0) return hipErrorInvalidValue;
  if (a.ldc && (epi != EPI_QKV || a.ldc < a.N || (int64_t)a.ldc * 64 >= ((int64_t)1 << 31))) return hipErrorInvalidValue;
  if (a_bytes == 2 && epi != EPI_I64 && !a.coef) return hipErrorInvalidValue;
#define EII_EPIS(AW)                                                     \
  switch (epi) {                                                         \
    case EPI_I64: return launch_gemm<AW, EPI_I64>(a, s);                 \
    case EPI_REQ16: return launch_gemm<AW, EPI_REQ16>(a, s);             \
    case EPI_REQ32: return launch_gemm<AW, EPI_REQ32>(a, s);             \
    case EPI_RESID: return launch_gemm<AW, EPI_RESID>(a, s);             \
    case EPI_LOGITS: return launch_gemm<AW, EPI_LOGITS>(a, s);           \
    case EPI_SILU:                                                       \
      if (a.tab_bits == 16 && a.sh2 >= 1 && a.sh2 <= 30) return launch_gemm<AW, EPI_SILU_I>(a, s); \
      return launch_gemm<AW, EPI_SILU>(a, s);                             \
    case EPI_QKV: return launch_gemm<AW, EPI_QKV>(a, s);                 \
  }
  if (a_bytes == 2) { EII_EPIS(2) }
  else if (a_bytes == 4) { EII_EPIS(4) }
#undef EII_EPIS
  return hipErrorInvalidValue;
}

hipError_t gemm_coef(const int32_t* mult, const int32_t* shift, const int32_t* wsum, int N, double2* coef,
                     hipStream_t s) {
  hipLaunchKernelGGL(coef_kernel, dim3((N + 255) / 256), dim3(256), 0, s, mult, shift, wsum, N, coef);
  return hipGetLastError();
}

hipError_t weight_colsum(const int8_t* W, int N, int K, int32_t* wsum, hipStream_t s) {
  hipLaunchKernelGGL(colsum_kernel, dim3((N + 3) / 4), dim3(256), 0, s, W, N, K, wsum);
  return hipGetLastError();
}

hipError_t embed(const int64_t* ids, int M, const int8_t* emb_q, const int32_t* emb_m,
                 const int32_t* emb_sh, int32_t* x, int* flag, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(blocks_for((size_t)M * (kD / 4))), dim3(256), 0, s, ids, M,
                     emb_q, emb_m, emb_sh, x, flag);
  return hipGetLastError();
}

hipError_t rmsnorm(const int32_t* x, int M, const int32_t* gain, int sh_out, int bits_out, uint8_t* planes,
                   void* plain, hipStream_t s, bool wide_gain, int32_t* u_out, int32_t* z_out) {
  if (bits_out != 16 && bits_out != 32) return hipErrorInvalidValue;
  // a wave per row while the rows leave most CUs idle anyway (shorter serial work per lane), else
  // 16 lanes per row
#define EII_NORM(OB, W, L) hipLaunchKernelGGL((rmsnorm_kernel<OB, W, L>), dim3((M + 256 / L - 1) / (256 / L)), dim3(256), \
                                              0, s, x, M, gain, sh_out, bits_out, planes, plain, u_out, z_out)
#define EII_NORM_L(OB, W) do { if (M <= 256) EII_NORM(OB, W, 64); else EII_NORM(OB, W, 16); } while (0)
  if (wide_gain) {
    if (bits_out == 16) EII_NORM_L(2, true);
    else EII_NORM_L(4, true);
  } else {
    if (bits_out == 16) EII_NORM_L(2, false);
    else EII_NORM_L(4, false);
  }
#undef EII_NORM_L
#undef EII_NORM
  return hipGetLastError();
}

hipError_t split_limbs(const void* a, int src_bytes, int M, int K, uint8_t* planes, hipStream_t s) {
  if (M <= 0 || K <= 0) return hipErrorInvalidValue;
  const int Kp = padded_k(K);
  dim3 grid(blocks_for((size_t)M * Kp / 4));
  if (src_bytes == 1) hipLaunchKernelGGL((split_kernel<1, 2>), grid, dim3(256), 0, s, a, M, K, Kp, planes);
  else if (src_bytes == 2) hipLaunchKernelGGL((split_kernel<2, 2>), grid, dim3(256), 0, s, a, M, K, Kp, planes);
  else if (src_bytes == 4) hipLaunchKernelGGL((split_kernel<4, 4>), grid, dim3(256), 0, s, a, M, K, Kp, planes);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t swizzle_weights(const int8_t* W, int N, int K, int8_t* Wf, hipStream_t s, int Kp) {
  if (Kp == 0) Kp = K;
  if (Kp % 32 != 0 || Kp < K || N <= 0 || K <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(swizzle_kernel, dim3(blocks_for((size_t)((N + 31) / 32) * (Kp / 32) * 64)), dim3(256), 0, s, W,
                     N, K, Kp, Wf);
  return hipGetLastError();
}

hipError_t gemm_i64_anyk(const uint8_t* planes, int a_bytes, const int8_t* Wf, const int32_t* wsum, int M, int N,
                         int Kp, int64_t* out, hipStream_t s, int a_kb) {
  if (Kp <= 0 || Kp % kBK != 0) return hipErrorInvalidValue;
  // passes over ranges of the K blocks, each a compiled K-block count (24, 9, 2 or 1), largest first
  int b0 = 0;
  const int nkb = Kp / kBK;
  while (b0 < nkb) {
    const int left = nkb - b0, nb = left >= 24 ? 24 : left >= 9 ? 9 : left >= 2 ? 2 : 1;
    GemmArgs g{planes + (size_t)b0 * M * 64, Wf + (size_t)b0 * 2 * 1024, M, N, nb * kBK, (size_t)M * Kp,
               b0 == 0 ? wsum : nullptr, nullptr, nullptr, out, 64, nullptr};
    g.w_ld = Kp;
    g.accumulate = b0 > 0;
    g.a_kb = a_kb;   // K block b0 (64 bytes) starts at byte b0 M 64 in both layouts
    const hipError_t e = gemm(g, a_bytes, EPI_I64, s);
    if (e != hipSuccess) return e;
    b0 += nb;
  }
  return hipSuccess;
}

hipError_t requant_i64(const int64_t* acc, int M, int N, const int32_t* mult, const int32_t* shift, int out_bits,
                       void* out, hipStream_t s) {
  const dim3 grid(blocks_for((size_t)M * N));
  if (out_bits == 16) hipLaunchKernelGGL(requant_kernel<int16_t>, grid, dim3(256), 0, s, acc, M, N, mult, shift, 16, (int16_t*)out);
  else if (out_bits == 32) hipLaunchKernelGGL(requant_kernel<int32_t>, grid, dim3(256), 0, s, acc, M, N, mult, shift, 32, (int32_t*)out);
  else if (out_bits == 64) hipLaunchKernelGGL(requant_kernel<int64_t>, grid, dim3(256), 0, s, acc, M, N, mult, shift, 64, (int64_t*)out);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t rope(int16_t* qkv, int M, const int32_t* pos, const int32_t* cosT, const int32_t* sinT, int sh_q,
                int bits_q, int sh_k, int bits_k, hipStream_t s) {
  hipLaunchKernelGGL(rope_kernel, dim3(blocks_for((size_t)M * 384)), dim3(256), 0, s, qkv, M, pos, cosT, sinT,
                     sh_q, bits_q, sh_k, bits_k);
  return hipGetLastError();
}

hipError_t silu_gate(const int16_t* gu, int M, const int32_t* silu, int sh, int bits, uint8_t* planes, void* plain,
                     hipStream_t s, int32_t* sg_out) {
  dim3 grid(blocks_for((size_t)M * kDFF));
  if (bits == 16) hipLaunchKernelGGL(silu_kernel<2>, grid, dim3(256), 0, s, gu, M, silu, sh, bits, planes, plain, sg_out);
  else hipLaunchKernelGGL(silu_kernel<4>, grid, dim3(256), 0, s, gu, M, silu, sh, bits, planes, plain, sg_out);
  return hipGetLastError();
}

// Scores and probabilities of every (sequence, head, query) row for traces (python/intref.py:238-253,
// its attn_score / attn_prob): one wave per row, lanes over the keys; the scores are written first and
// read back by the same lanes.  score_out int16 [B][9][T][T] (0 past the diagonal), prob_out int32
// [B][9][T][T]; sequence b holds rows b T .. b T + T - 1 of qkv.
__global__ __launch_bounds__(64) void attn_trace_kernel(const int16_t* qkv, int T, const int32_t* exp_tab, int shift_s,
                                                        int16_t* score_out, int32_t* prob_out) {
  const int qi = blockIdx.x, hh = blockIdx.y, b = blockIdx.z, lane = threadIdx.x, g = hh / 3;
  const int16_t* q = qkv + ((size_t)b * T + qi) * kQKVN + hh * 64;
  const size_t orow = (((size_t)b * kNH + hh) * T + qi) * T;
  int32_t mx = INT32_MIN;
  for (int j = lane; j < T; j += 64) {
    int32_t sv = 0;
    if (j <= qi) {
      const int16_t* k = qkv + ((size_t)b * T + j) * kQKVN + kD + g * 64;
      int64_t acc = 0;
      for (int d = 0; d < 64; ++d) acc += (int64_t)q[d] * k[d];
      sv = (int32_t)sat(rs(acc, shift_s), 16);
      mx = max(mx, sv);
    }
    score_out[orow + j] = (int16_t)sv;
  }
  for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
  int64_t Z = 0;
  for (int j = lane; j <= qi; j += 64) {
    const int d = mx - score_out[orow + j];
    Z += d <= kDMax ? exp_tab[d] : 0;
  }
  for (int o = 32; o > 0; o >>= 1) Z += __shfl_xor(Z, o);
  for (int j = lane; j < T; j += 64) {
    int32_t P = 0;
    if (j <= qi) {
      const int d = mx - score_out[orow + j];
      const int64_t e = d <= kDMax ? exp_tab[d] : 0;
      P = (int32_t)((e * 65536 + Z / 2) / Z);
    }
    prob_out[orow + j] = P;
  }
}

hipError_t attn_trace(const int16_t* qkv, int B, int T, const int32_t* exp_tab, int shift_s, int16_t* score_out,
                      int32_t* prob_out, hipStream_t s) {
  if (B <= 0 || T <= 0 || shift_s < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn_trace_kernel, dim3(T, kNH, B), dim3(64), 0, s, qkv, T, exp_tab, shift_s, score_out, prob_out);
  return hipGetLastError();
}

// k limb planes for the recomputing attention passes: thread = (row, kv group, 16 of its 64 k
// columns); out row r at kpl + 384 r, kv group g at + 128 g: 64 bytes low - 128, then 64 high
__global__ __launch_bounds__(256) void k_planes_kernel(const int16_t* qkv, int M, uint8_t* kpl) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * 12) return;
  const size_t r = i / 12;
  const int gc = (int)(i % 12), g = gc >> 2, c = gc & 3;
  const int16_t* src = qkv + r * kQKVN + kD + 64 * g + 16 * c;
  const u32x4 d0 = *(const u32x4*)src, d1 = *(const u32x4*)(src + 8);
  uint8_t* dst = kpl + r * 384 + 128 * g + 16 * c;
  *(u32x4*)dst = u32x4{lo_bytes16(d0[0], d0[1]), lo_bytes16(d0[2], d0[3]), lo_bytes16(d1[0], d1[1]),
                       lo_bytes16(d1[2], d1[3])};
  *(u32x4*)(dst + 64) = u32x4{hi_bytes16(d0[0], d0[1]), hi_bytes16(d0[2], d0[3]), hi_bytes16(d1[0], d1[1]),
                              hi_bytes16(d1[2], d1[3])};
}

hipError_t attention(const AttnArgs& a, hipStream_t s) {
  if (a.B <= 0 || a.max_T <= 0) return hipSuccess;
  if (!a.vt || a.shift_s < 1 || a.shift_s > 30 || a.max_kt < 1) return hipErrorInvalidValue;
  if (a.kv_len && (a.q_first < 0 || a.q_first >= a.kv_len || a.max_T != a.kv_len ||
                   a.out_M != a.B * (a.kv_len - a.q_first)))
    return hipErrorInvalidValue;
  if (a.kv_len && a.kv_len - a.q_first == 1 && a.kv_len <= kDecodeMaxKeys && a.out_M == a.B) {
    // decoding step: one query per sequence
    // 4 waves per head while the workgroups (3 per sequence) leave most CUs idle
    const dim3 grid(a.B, kNKV);
    if (3 * a.B < 256) {
      const size_t lds = attn_decode_lds(a.kv_len, 4);
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_decode_kernel<2, 4>), grid, dim3(768), lds, s, a);
      else hipLaunchKernelGGL((attn_decode_kernel<4, 4>), grid, dim3(768), lds, s, a);
    } else {
      const size_t lds = attn_decode_lds(a.kv_len, 1);
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_decode_kernel<2, 1>), grid, dim3(192), lds, s, a);
      else hipLaunchKernelGGL((attn_decode_kernel<4, 1>), grid, dim3(192), lds, s, a);
    }
    return hipGetLastError();
  }
  // query tiles from the one holding q_first (0 for a plain forward) to the end; workgroups of the
  // 3 heads of a kv group while up to 8 key tiles (256 keys) keep their scores in registers, of one
  // head for the longer rows, whose passes recompute the scores
  const int nqt = (a.max_T + 31) / 32 - (a.q_first >> 5);
  const dim3 grid((unsigned)(((size_t)nqt * a.B * kNH + 3) / 4)), block(256), grid1(a.B, kNH, nqt), block1(64);
  // with fewer than 2048 (sequence, head, query tile) tasks (a few sequences: fewer than two waves per
  // SIMD) each task's key tiles are split over the 4 waves of its workgroup, which shortens the
  // serial chain of the longest task
  const bool split = (size_t)nqt * a.B * kNH < 2048;
  if (a.max_kt <= 5) {
    if (split) {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 5, 4, 4>), grid1, block, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 5, 4, 4>), grid1, block, 0, s, a);
    } else {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 5, 4>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 5, 4>), grid, block, 0, s, a);
    }
  } else if (a.max_kt <= 8) {
    if (split) {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 8, 4, 4>), grid1, block, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 8, 4, 4>), grid1, block, 0, s, a);
    } else {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 8, 4>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 8, 4>), grid, block, 0, s, a);
    }
  } else {
    // the recomputing passes read the k limb planes when the caller gives a workspace for them
    const bool kp = a.kpl && !a.kv_len && attn_kpl_bytes(a.M) < ((size_t)1 << 31);
    if (kp) {
      const size_t n = (size_t)a.M * 12;
      hipLaunchKernelGGL(k_planes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.qkv, a.M, a.kpl);
    }
    if (split) {
      if (kp) {
        if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 0, 4, 4, true>), grid1, block, 0, s, a);
        else hipLaunchKernelGGL((attn_kernel<4, 0, 4, 4, true>), grid1, block, 0, s, a);
      } else {
        if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 0, 4, 4>), grid1, block, 0, s, a);
        else hipLaunchKernelGGL((attn_kernel<4, 0, 4, 4>), grid1, block, 0, s, a);
      }
    } else if (kp) {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 0, 1, 1, true>), grid1, block1, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 0, 1, 1, true>), grid1, block1, 0, s, a);
    } else {
      if (a.bits_c == 16) hipLaunchKernelGGL((attn_kernel<2, 0, 1>), grid1, block1, 0, s, a);
      else hipLaunchKernelGGL((attn_kernel<4, 0, 1>), grid1, block1, 0, s, a);
    }
  }
  return hipGetLastError();
}

// KV cache append: thread = (new row, 8 consecutive of its 960 columns), one 16-byte copy
__global__ __launch_bounds__(256) void kv_append_kernel(const int16_t* qkv, int B, int T_new, int cap, int p0,
                                                         int16_t* cache) {
  constexpr int kC8 = kQKVN / 8;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)B * T_new * kC8) return;
  const int r = (int)(i / kC8), c8 = (int)(i % kC8), b = r / T_new, t = r % T_new;
  const size_t crow = (size_t)b * cap + p0 + t;
  *(int4*)(cache + crow * kQKVN + 8 * c8) = *(const int4*)(qkv + (size_t)r * kQKVN + 8 * c8);
}

// V^T planes of cached positions [from, to) of every sequence.  Workgroup = (sequence, 64
// positions): the v columns of its rows come in as whole rows and pass through LDS (rows padded to
// 97 dwords, so the reads of one column at 64 consecutive positions hit 64 banks), then each plane
// row's bytes for those positions leave as one contiguous run.
__global__ __launch_bounds__(256) void kv_vt_kernel(const int16_t* cache, int cap, int from, int to, int nchunk,
                                                    uint8_t* vt, int stride) {
  __shared__ __attribute__((aligned(16))) int16_t tv[64][194];
  const int b = blockIdx.x / nchunk, t0 = from + 64 * (blockIdx.x % nchunk), n = min(64, to - t0);
  const size_t row0 = (size_t)b * cap + t0;
  for (int i = threadIdx.x; i < 64 * 24; i += 256) {   // 24 x 8 v values per row
    const int p = i / 24, q = i % 24;
    if (p < n) {
      const int4 v = *(const int4*)(cache + (row0 + p) * kQKVN + kD + 192 + 8 * q);
      int32_t* dst = (int32_t*)&tv[p][8 * q];
      dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 192 * 64; i += 256) {
    const int p = i & 63, d = i >> 6;
    if (p < n) {
      const uint32_t v = (uint16_t)tv[p][d];
      uint8_t* o = vt + (size_t)d * stride + row0 + p;
      o[0] = (uint8_t)(v ^ 0x80u);
      o[(size_t)192 * stride] = (uint8_t)(v >> 8);
    }
  }
}

hipError_t kv_append(const int16_t* qkv, int B, int T_new, int cap, int p0, int16_t* cache_qkv, hipStream_t s) {
  if (B <= 0 || T_new <= 0 || p0 < 0 || p0 + T_new > cap) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kv_append_kernel, dim3(blocks_for((size_t)B * T_new * (kQKVN / 8))), dim3(256), 0, s, qkv, B,
                     T_new, cap, p0, cache_qkv);
  return hipGetLastError();
}

hipError_t kv_build_vt(const int16_t* cache_qkv, int B, int cap, int from, int to, uint8_t* cache_vt, hipStream_t s) {
  if (B <= 0 || from < 0 || to > cap || from > to) return hipErrorInvalidValue;
  if (from == to) return hipSuccess;
  const int nchunk = (to - from + 63) / 64;
  hipLaunchKernelGGL(kv_vt_kernel, dim3((unsigned)((size_t)B * nchunk)), dim3(256), 0, s, cache_qkv, cap, from, to,
                     nchunk, cache_vt, vt_stride_for(B * cap));
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_pos_kernel(int32_t* pos, int n, int T_new, int p0) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) pos[i] = p0 + i % T_new;
}

hipError_t fill_positions(int32_t* pos, int B, int T_new, int p0, hipStream_t s) {
  const int n = B * T_new;
  hipLaunchKernelGGL(fill_pos_kernel, dim3((n + 255) / 256), dim3(256), 0, s, pos, n, T_new, p0);
  return hipGetLastError();
}

// one workgroup per row: each thread scans a strided slice keeping (value, lowest index), then
// a tree reduction in LDS that prefers the lower index on equal values
__global__ __launch_bounds__(256) void argmax_kernel(const int32_t* v, int n, int64_t* out) {
  __shared__ int32_t bv[256];
  __shared__ int32_t bi[256];
  const int32_t* row = v + (size_t)blockIdx.x * n;
  int32_t best = INT32_MIN;
  int32_t bidx = n;
  for (int j = threadIdx.x; j < n; j += 256) {
    const int32_t x = row[j];
    if (x > best || bidx == n) { best = x; bidx = j; }
  }
  bv[threadIdx.x] = best;
  bi[threadIdx.x] = bidx;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      const int32_t ov = bv[threadIdx.x + w], oi = bi[threadIdx.x + w];
      if (oi < n && (bi[threadIdx.x] == n || ov > bv[threadIdx.x] || (ov == bv[threadIdx.x] && oi < bi[threadIdx.x]))) {
        bv[threadIdx.x] = ov;
        bi[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = bi[0];
}

hipError_t argmax_rows(const int32_t* v, int rows, int n, int64_t* out, hipStream_t s) {
  if (rows <= 0 || n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, s, v, n, out);
  return hipGetLastError();
}

hipError_t build_vt(const int16_t* qkv, int M, uint8_t* vt, hipStream_t s) {
  const int stride = vt_stride_for(M);
  hipLaunchKernelGGL(vt_kernel, dim3(blocks_for((size_t)192 * (stride / 4))), dim3(256), 0, s, qkv, M, vt, stride);
  return hipGetLastError();
}

}  // namespace eii
