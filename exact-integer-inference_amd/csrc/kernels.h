// Launchers of the gfx950 kernels (kernels.hip).  All pointers are device pointers; every
// launcher enqueues on the given stream and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "index_maps.h"

namespace eii {

enum Epi : int {
  EPI_I64 = 0,     // out int64 [M, N] = exact accumulator
  EPI_REQ16 = 1,   // out int16 [M, N] = SAT(RS(acc * m[n], sh[n]), sat_bits)
  EPI_REQ32 = 2,   // out int32 [M, N] = SAT(RS(acc * m[n], sh[n]), sat_bits)
  EPI_RESID = 3,   // x int32 [M, N] = SAT32(x + RS(acc * m[n], sh[n]))
  EPI_LOGITS = 4,  // out int32 [M, N] = RS(acc * m[n], sh[n]); *flag |= 1 if it leaves int32
  // W = blocks of [32 gate rows | 32 up rows] (N = 2 * 1536): out = limb planes [bits2/8][M][N/2] of
  //   SAT(RS(aux_tab[SAT16(gate) + 32768] * SAT16(up), sh2), bits2)        (python/intref.py:268-275)
  EPI_SILU = 5,
  // W = q | k | v rows (N = 960, 16-bit outputs): RoPE on q heads (shift sh_q) and k heads (sh_k)
  // at positions pos[m] with cosT/sinT [rows, 32], out int16 [M, 960]        (python/intref.py:207-222)
  EPI_QKV = 6,
  // EPI_SILU with a 16-bit table and a gated shift in 1..30 (|silu up| < 2^30): the gated product
  // and its requantization in int32; gemm() selects it from EPI_SILU by itself
  EPI_SILU_I = 7,
};

// Activations enter the GEMM as int8 limb planes (eii_int.h split_limbs): a_bytes planes of
// M x K bytes, plane l at A + l * a_plane, lowest byte first, each plane K-blocked
// (index_maps.h: plane_offset, or plane_offset32 for the gated MLP activations).
// Weights enter the GEMM in MFMA fragment order (swizzle_weights): for each block of 32 output
// rows and each 32-column K slice, the 64 lanes' 16-byte operands in lane order,
// [ceil(N / 32)][K / 32][64][16] (lane 32 h + c: row 32 b + c, columns 16 h .. 16 h + 15 of
// the slice); rows past N are zero.
inline size_t swizzled_bytes(int N, int K) { return (size_t)((N + 31) / 32) * 32 * K; }
// W [N, K] row-major (any K) -> fragment order over Kp >= K columns (zero past K), Kp % 32 == 0
hipError_t swizzle_weights(const int8_t* W, int N, int K, int8_t* Wf, hipStream_t s, int Kp = 0);

struct GemmArgs {
  const void* A;          // limb planes of the [M, K] activations, 2 (16-bit) or 4 (32-bit) planes
  const int8_t* W;        // weights [N, K] (row = output channel) in fragment order
  int M, N, K;            // K % 64 == 0
  size_t a_plane;         // bytes between limb planes (M * K for a dense [L][M][K] layout)
  const int32_t* wsum;    // [N] sum_k W[n, k]
  const int32_t* mult;    // [N] m (|m| <= 2^14)
  const int32_t* shift;   // [N] requantization shift, 1..62
  void* out;
  int sat_bits;
  int* flag;
  // 2-limb inputs, every epilogue except EPI_I64: per-column float64 coefficients [N]
  // (m 2^-sh, 128 wsum m 2^-sh + 2^-(sh+1)) from gemm_coef
  const double2* coef = nullptr;
  // EPI_SILU: SiLU table [65536] (index gate + 32768) whose entries fit tab_bits bits
  const int32_t* aux_tab = nullptr;
  int sh2 = 0, bits2 = 16, tab_bits = 32;
  // EPI_QKV
  const int32_t* pos = nullptr;
  const int32_t* cosT = nullptr;
  const int32_t* sinT = nullptr;
  int sh_q = 0, sh_k = 0;
  // EPI_QKV: also write v as the key-contiguous V^T limb planes described below, or null
  uint8_t* vt = nullptr;
  int vt_stride = 0;
  // EPI_QKV: elements between output rows (0 = N), so a decoding step's rows can go straight to
  // their KV cache rows (row r at out + r ldc); 32 ldc 2 bytes must stay below 2^31
  int ldc = 0;
  // K of the whole fragment-ordered weight matrix when this launch covers a range of its K blocks
  // (W and A then point at the first block of the range); 0 = K
  int w_ld = 0;
  // EPI_I64 only: add the accumulators to the int64 values already in out (K-range passes after
  // the first); wsum may be null, meaning no limb bias term (the first pass adds it for all of K)
  bool accumulate = false;
  // K-block width of the activation planes in bytes: 64 (plane_offset) or 32 (plane_offset32)
  int a_kb = 64;
  // row blocks per group of the tile order (set by the launch)
  int tile_g = 8;
  // RMSNorm folded into the GEMM (K = 576, a_bytes 2, at most 4 rows: a wave per row in the
  // prologue): A is SAT(RS(3 RS(x U, 16) gain, nsh), 16) of x [M, 576] (the rmsnorm launcher's
  // values for gains in int16 and nsh in 10..40), formed from x instead of read as limb planes
  const int32_t* nx = nullptr;
  const int32_t* ngain = nullptr;
  int nsh = 0;
};

// V^T limb planes for attention: plane 0 = low bytes - 128, plane 1 = signed high bytes of v;
// each plane [192 rows = 64 kv group + d][vt_stride] bytes, column = token row.  vt_stride is M
// rounded up to a multiple of 128 (every row a GEMM tile can touch).
__host__ __device__ inline int vt_stride_for(int M) { return (M + 127) / 128 * 128; }
inline size_t vt_bytes(int M) { return (size_t)2 * 192 * vt_stride_for(M); }
// V^T planes from the v columns of qkv [M, 960] (for paths that do not fuse them into the projection)
hipError_t build_vt(const int16_t* qkv, int M, uint8_t* vt, hipStream_t s);

hipError_t gemm(const GemmArgs& a, int a_bytes, int epi, hipStream_t s);
// Exact int64 out [M, N] = A W^T for any K: A as limb planes of K rounded up to a multiple of 64
// (a_bytes 2 or 4), W in fragment order over the same padded K (zero columns past K), wsum [N];
// the K blocks run in passes of the GEMM's compiled K-block counts, accumulated in out.  a_kb: the
// planes' K-block width (GemmArgs::a_kb).
hipError_t gemm_i64_anyk(const uint8_t* planes, int a_bytes, const int8_t* Wf, const int32_t* wsum, int M, int N,
                         int Kp, int64_t* out, hipStream_t s, int a_kb = 64);
// out [M, N] (int16, int32 or int64 by out_bits; 64 = no saturation) = SAT(RS(acc * mult[n], shift[n]), out_bits)
// from exact int64 (in place when out == acc)
// accumulators (python/intref.py:189), in int64 as the reference
hipError_t requant_i64(const int64_t* acc, int M, int N, const int32_t* mult, const int32_t* shift, int out_bits,
                       void* out, hipStream_t s);
inline int padded_k(int K) { return (K + 63) / 64 * 64; }
hipError_t weight_colsum(const int8_t* W, int N, int K, int32_t* wsum, hipStream_t s);
hipError_t gemm_coef(const int32_t* mult, const int32_t* shift, const int32_t* wsum, int N, double2* coef,
                     hipStream_t s);

// x[m, c] = RS(emb_q[id, c] * emb_m[id], emb_sh[id]) (python/intref.py:163-166)
hipError_t embed(const int64_t* ids, int M, const int8_t* emb_q, const int32_t* emb_m,
                 const int32_t* emb_sh, int32_t* x, int* flag, hipStream_t s);

// out = SAT(RS(3 * RS(x * U, 16) * gain, sh_out), bits_out) as limb planes (bits/8 planes of
// M x 576, K-blocked) and/or plain int16/int32 [M, 576] (either pointer may be null).  Gains
// must be int16 unless wide_gain (any int32 gain, general int64 path); u_out int32 [M] and z_out
// int32 [M, 576] (nullable) receive the norm's U and z = RS(x U, 16).
hipError_t rmsnorm(const int32_t* x, int M, const int32_t* gain, int sh_out, int bits_out,
                   uint8_t* planes, void* plain, hipStream_t s, bool wide_gain = false,
                   int32_t* u_out = nullptr, int32_t* z_out = nullptr);

// plain [M, K] int8 (src_bytes 1), int16 (2) or int32 (4) -> K-blocked limb planes over K rounded
// up to a multiple of 64 (padded_k; the columns past K hold 0): 2 planes for 8/16-bit values, 4 for
// 32-bit ones
hipError_t split_limbs(const void* a, int src_bytes, int M, int K, uint8_t* planes, hipStream_t s);

// In-place rotate-half RoPE on the q (cols 0..575) and k (cols 576..767) parts of qkv [M, 960]
hipError_t rope(int16_t* qkv, int M, const int32_t* pos, const int32_t* cosT, const int32_t* sinT,
                int sh_q, int bits_q, int sh_k, int bits_k, hipStream_t s);

// gated[m, j] = SAT(RS(silu[gate + 32768] * up, sh), bits) with gu rows holding [gate 32 | up 32]
// blocks: gate j at column 64 (j / 32) + j % 32, up j 32 columns further
// sg_out int32 [M, 1536] (nullable, traces): the table values silu[gate + 32768]; planes (nullable)
// in the 32-byte K-block layout (plane_offset32), as the fused gate/up epilogue writes them
hipError_t silu_gate(const int16_t* gu, int M, const int32_t* silu, int sh, int bits,
                     uint8_t* planes, void* plain, hipStream_t s, int32_t* sg_out = nullptr);
// Trace of attention's scores and probabilities for B sequences of T rows each (see kernels.hip)
hipError_t attn_trace(const int16_t* qkv, int B, int T, const int32_t* exp_tab, int shift_s, int16_t* score_out,
                      int32_t* prob_out, hipStream_t s);

struct AttnArgs {
  const int16_t* qkv;      // [M, 960]: q rope | k rope (v is read from vt)
  const uint8_t* vt;       // V^T limb planes (vt_stride_for(M))
  const int32_t* seq_off;  // [B + 1] row offsets of the sequences
  const int32_t* exp_tab;  // [1537]
  void* ctx;               // plain [M, 576], int16 or int32, or null
  uint8_t* ctx_planes;     // K-blocked limb planes (bits_c/8 planes of M x 576), or null
  int M;
  int B, max_T;
  int max_kt;              // max over sequences of the 32-row key tiles it spans (attn_key_tiles)
  int shift_s;             // f_qr + f_kr + 3 - 7, >= 1
  int sh_ctx;              // 16 + f_v - f_c
  int bits_c;
  // Incremental decoding over a KV cache (kv_len = 0: a plain forward).  Sequence b holds kv_len
  // tokens at rows seq_off[b] ..; only query positions q_first .. kv_len - 1 are computed, and
  // the context of position t goes to row b (kv_len - q_first) + t - q_first of the ctx outputs,
  // which have out_M rows.
  int kv_len = 0, q_first = 0, out_M = 0;
  // Plain forwards whose rows span more than 8 key tiles: a workspace of attn_kpl_bytes(M) bytes
  // that the launcher fills with the k columns as limb planes (per row and kv group, 64 low bytes
  // - 128 then 64 signed high bytes), read by the passes that recompute the scores; null = the
  // kernel splits the k rows itself
  uint8_t* kpl = nullptr;
};
inline size_t attn_kpl_bytes(int M) { return (size_t)M * 3 * 128; }
// 32-row key tiles (aligned to multiples of 32 rows) spanned by a sequence at rows [s0, s0 + T)
inline int attn_key_tiles(int s0, int T) { return ((s0 + T - 1) >> 5) - (s0 >> 5) + 1; }
hipError_t attention(const AttnArgs& a, hipStream_t s);

// KV cache append: rows b T_new + i of qkv [B T_new, 960] go to row b cap + p0 + i of the cache
// rows (the V^T planes: kv_build_vt)
hipError_t kv_append(const int16_t* qkv, int B, int T_new, int cap, int p0, int16_t* cache_qkv, hipStream_t s);
// V^T planes (vt_stride_for(B cap)) of the cached positions [from, to) of every sequence, built
// from the cached v rows (single-token appends that the one-query decoding kernel serves leave
// them out until a step needs them)
hipError_t kv_build_vt(const int16_t* cache_qkv, int B, int cap, int from, int to, uint8_t* cache_vt, hipStream_t s);
// longest cache the one-query decoding attention serves (its scores of 3 heads sit in LDS); longer
// caches take the tiled kernel, which reads the V^T planes
constexpr int kDecodeMaxKeys = 8192;
// pos[b T_new + i] = p0 + i
hipError_t fill_positions(int32_t* pos, int B, int T_new, int p0, hipStream_t s);
// out[r] = the lowest index of the largest of the n values of row r
hipError_t argmax_rows(const int32_t* v, int rows, int n, int64_t* out, hipStream_t s);

}  // namespace eii
