// Index maps of the GEMM and attention kernels: operand layouts in HBM and LDS, the fragment
// addresses of v_mfma_i32_32x32x32_i8, the tile shapes, and the attention key order.  The kernels
// compute every such address through these functions, and hostcheck.cpp runs the same functions in
// a CPU model of the kernels (direct-to-LDS loads into a simulated stage, fragment reads, the MFMA's
// operand and result layouts, the epilogue's element map), so an indexing mistake shows up on the
// CPU as a wrong limb sum, an access out of bounds or an element stored twice or never.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "eii_int.h"

namespace eii {

// ---------------------------------------------------------------- activation limb planes in HBM
// Plane l of the [M, K] activations: K-blocked, element (m, k) at byte plane_offset(m, k, M),
// i.e. [K / 64][M][64], so the 64-byte K slices of consecutive rows are contiguous.
EII_HD size_t plane_offset(size_t m, size_t k, size_t M) {
  return (k >> 6) * M * 64 + m * 64 + (k & 63);
}
// The gated MLP activations (the SiLU-gate product, input of the down projection) use 32-byte K
// blocks instead, [K / 32][M][32]: the gate/up epilogue then writes 4 consecutive rows x 32 gated
// columns of a wave as one whole 128-byte line (no partially written lines, whose write-back
// costs a fill from memory).  K block b of 64 bytes still starts at byte b M 64.
EII_HD size_t plane_offset32(size_t m, size_t k, size_t M) {
  return (k >> 5) * M * 32 + m * 32 + (k & 31);
}

namespace idx {

// ---------------------------------------------------------------- v_mfma_i32_32x32x32_i8
// D[i][j] += sum_k A[i][k] B[k][j], i, j, k < 32.  Lane 32 h + c holds bytes k = 16 h .. 16 h + 15
// of row c of A and of column c of B (16 bytes each), and result register e = 4 b + r holds
// D[mfma_row(e, h)][c].
EII_HD int mfma_row(int e, int h) { return 8 * (e >> 2) + 4 * h + (e & 3); }

// ---------------------------------------------------------------- GEMM tile shapes
//   kShapeSquare: 2 x 2 waves, 128 x 128 tiles for 2-limb activations, 64 x 128 for 4-limb;
//   kShapeNarrow: 2 x 2 waves, 64 x 192 tiles for N a multiple of 192 but not of 128 (N = 576: three
//     column blocks instead of four and a half, so the persistent workgroups get evenly sized tiles and
//     no half-empty ones), 2-limb activations only;
//   kShapeRow: 1 x 4 waves, 64 x 256 tiles for wide 2-limb GEMMs (q/k/v, gate/up, the head): the four
//     waves share one 64-row activation tile in LDS (half the LDS traffic of a 128-row tile per MFMA
//     column) and each loads its own weight columns;
//   kShapeSkinny: at most 32 rows (decoding steps): one 32 x 64 tile per workgroup, the K slices split
//     over the 4 waves, every operand fragment loaded straight into registers at the start (one memory
//     round trip instead of a pipelined K loop whose steps each wait for a weight load), the partial
//     sums added through LDS, and wave 0 running the epilogue; many small tiles spread the weight
//     reads over the CUs;
//   kShapeSkinny32: the same with 32 x 32 tiles, for the epilogues without column pairs (twice the
//     workgroups for the narrow residual GEMMs, N = 576).
constexpr int kShapeSquare = 0, kShapeNarrow = 1, kShapeRow = 2, kShapeSkinny = 3, kShapeSkinny32 = 4;
constexpr int kLdsRow = 64;   // bytes per row of an LDS activation stage: one 64-byte K block
template <int AW, int SHAPE>
struct GemmCfg {
  static constexpr bool kSkinny = SHAPE == kShapeSkinny || SHAPE == kShapeSkinny32;
  static_assert(SHAPE == kShapeSquare || kSkinny || AW == 2, "narrow and row tiles for 2-limb activations");
  static constexpr int kThreads = 256;                   // 4 waves; two workgroups share a CU
  static constexpr int WGM = SHAPE == kShapeRow || kSkinny ? 1 : 2, WGN = kSkinny ? 1 : 4 / WGM;   // wave grid
  static constexpr int BM = kSkinny ? 32 : SHAPE == kShapeSquare && AW == 2 ? 128 : 64;
  static constexpr int BN = SHAPE == kShapeSkinny32 ? 32 : kSkinny ? 64 : SHAPE == kShapeNarrow ? 192
                            : SHAPE == kShapeRow ? 256 : 128;
  static constexpr int WM = BM / WGM, WN = BN / WGN;     // wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;       // 32x32 tiles per wave
  static constexpr int kPlane = BM * kLdsRow;
  // activation limb planes (8 or 16 KB per stage), or for the skinny shapes the partial sums of
  // waves 1..3
  static constexpr int kStage = kSkinny ? 3 * TN * AW * 16 * 64 * 4 : AW * kPlane;
  static constexpr int kStages = kSkinny ? 1 : 4;          // loaded two and three steps ahead
  static constexpr int kAChunks = AW * BM * 4 / kThreads;   // 16-byte direct-to-LDS loads per thread
  static_assert(kAChunks * kThreads == AW * BM * 4, "chunk split");
};

// ---------------------------------------------------------------- activation stages in LDS
// Rows of a stage are 64 bytes (one K block); the 16-byte chunk c of row r sits at physical chunk
// c ^ ((r >> 2) & 3), so both the direct-to-LDS loads (lane order) and the 16-lane groups of the
// fragment reads (16 consecutive rows, one chunk) cover all 64 banks.  The map is an involution.
EII_HD int lds_swz(int row, int c) { return c ^ ((row >> 2) & 3); }
// Direct-to-LDS load q = tid + 256 i (thread tid's chunk i) of a stage of BM-row planes writes
// stage byte 16 q (lane j of a wave's load lands at the wave's base + 16 j): plane l, row, and
// physical chunk cp, which holds the row's logical chunk lds_swz(row, cp).
struct AChunk { int l, row, cp; };
EII_HD AChunk a_chunk(int q, int BM) { return AChunk{q / (4 * BM), (q >> 2) % BM, q & 3}; }
// Byte offset (from the planes' base) of logical 16-byte chunk c of 64-byte K block kb of row m in
// plane l, for K blocks of a_kb bytes: bytes 16 c of the 64-byte row (a_kb 64), or bytes 16 (c & 1)
// of the row in 32-byte block c >> 1 (a_kb 32).  Successive K blocks lie M 64 bytes apart.
EII_HD size_t a_src_off(int l, int m, int kb, int c, int M, int a_kb, size_t a_plane) {
  const int cb = a_kb >> 4;   // chunks per row of a block: 4 or 2
  return (size_t)l * a_plane + (size_t)kb * M * 64 + (size_t)(c / cb) * M * a_kb + (uint32_t)(m * a_kb + (c % cb) * 16);
}
// Stage byte offset of the A fragment bytes 16 kc .. 16 kc + 15 (kc = 2 ks + h: K slice ks of the
// block, lane half h) of stage row `row` in plane l.
EII_HD int a_frag(int l, int row, int kc, int plane_bytes) { return l * plane_bytes + row * kLdsRow + lds_swz(row, kc) * 16; }

// ---------------------------------------------------------------- weights in fragment order
// W [N, K] is stored as [ceil(N / 32)][K / 32][64 lanes][16 bytes]: lane 32 h + c of block nb32,
// K slice s holds columns 16 h .. 16 h + 15 of the slice in row 32 nb32 + c, the B operand of the
// MFMA for output columns 32 nb32 .. + 31 (rows past N are zero).
EII_HD size_t w_frag(int nb32, int kslices, int s, int lane) { return ((size_t)nb32 * kslices + s) * 1024 + (size_t)lane * 16; }
// where element (n, k) of W goes in that order
EII_HD size_t w_fo_offset(size_t n, size_t k, size_t kslices) {
  return w_frag((int)(n >> 5), (int)kslices, (int)(k >> 5), (int)(32 * ((k & 31) >> 4) + (n & 31))) + (k & 15);
}

// ---------------------------------------------------------------- attention
// A-operand row i of a 32-key tile carries key attn_key_perm(i), the key that result row i then
// denotes: with i = mfma_row(j, h), lane 32 h + c ends with keys 16 h + j (register j) of query c,
// which is the B-operand layout of the P.V product (bytes j = keys 16 h + j).
EII_HD int attn_key_perm(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }

// Int8 digits of the score MFMAs.  A query element is q = 256 (qh + qx) + ql with ql its low byte
// read as int8, qh = min((q + 128) >> 8, 127) and qx = ((q + 128) >> 8) - qh, which is 1 only for
// q >= 32640; a key element is k = 256 kh + kl + 128 with kh its signed high byte and kl its low
// byte - 128 (the V^T planes' form).  Then, summed over the 64 dimensions,
//   q . k = 65536 sum (qh + qx) kh + 256 sum ((qh + qx) kl + ql kh) + sum ql kl + 128 sum q,
// where the last term is one constant per query: no per-key sum is needed.
struct QDigits { int ql, qh, qx; };
EII_HD QDigits attn_q_digits(int q) {
  const int hd = (q + 128) >> 8, h = hd < 127 ? hd : 127;
  return QDigits{(int)(int8_t)(uint8_t)(q & 0xFF), h, hd - h};
}

}  // namespace idx
}  // namespace eii
