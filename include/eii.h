/* libeii: exact integer forward of the SmolLM2-135M-shaped model on one MI355X (gfx950).
 *
 * C ABI for the hot path of the reference's integer engine.  All pointers named *_dev are
 * device pointers (e.g. a torch tensor's data_ptr()); `stream` is a hipStream_t or NULL for
 * the default stream.  Every call enqueues its work on the stream and returns without
 * waiting, except where stated.  The library owns the model's device arrays and its
 * activation workspace; the caller owns every input and output buffer.
 *
 * Status codes mirror the exit codes of the reference checkers (c/intref.c:63,67,215,
 * cuda/intref.cu:22,263-273): 0 ok, 2 file/format error, 3 device error, 4 a bound the
 * semantics require is violated (shift < 1, table too short, value out of range),
 * 5 invalid argument.  eii_last_error() describes the last failure of the calling thread.
 */
#ifndef EII_H
#define EII_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EII_OK 0
#define EII_E_IO 2
#define EII_E_DEVICE 3
#define EII_E_BOUND 4
#define EII_E_ARG 5

typedef struct eii_model eii_model;

/* Optional per-site dumps of one block (python/intref.py:183,198-285 `trace`).  Each non-NULL
 * pointer receives [rows, width] values in the site's declared width: int16 for 16-bit sites,
 * int32 for 32-bit sites (widths: q/norm/ctx 576, k/v 192, gate/up/gated 1536).  The norm
 * internals, attention matrices and unsaturated residual updates have fixed types:
 *   norm1_U, norm2_U int32 [rows]; norm1_z, norm2_z int32 [rows, 576] (|z| <= 2^24);
 *   attn_score int16 [B, 9, T, T] (0 past the diagonal), attn_prob int32 [B, 9, T, T] (Q0.16);
 *   o_res, down_res int64 [rows, 576] (RS(acc m, .) before the saturating add);
 *   silu_gate int32 [rows, 1536] (the SiLU table values). */
typedef struct {
  void* norm1_out; void* q_proj; void* k_proj; void* v_proj; void* q_rope; void* k_rope;
  void* attn_ctx; int32_t* resid_mid; void* norm2_out; void* gate_proj; void* up_proj;
  void* mlp_gated;
  int32_t* norm1_U; int32_t* norm1_z; int16_t* attn_score; int32_t* attn_prob; int64_t* o_res;
  int32_t* norm2_U; int32_t* norm2_z; int32_t* silu_gate; int64_t* down_res;
} eii_trace;

const char* eii_last_error(void);

/* Load a model.bin (python/export_vectors.py:24-45; read order of c/intref.c:70-91 and
 * cuda/intref.cu:184-206) onto `device`.  int64 fields are narrowed to the widths the
 * semantics allow and every narrowing is checked; per-row requantization shifts must be
 * >= 1 as python/intref.py:49 asserts. */
int eii_model_load(const char* model_bin_path, int device, eii_model** out);
void eii_model_free(eii_model* m);

/* Replace the RoPE tables by host arrays cos/sin int64 [rows, 32] (Q30), e.g. rows beyond
 * the 512 model.bin holds (python/intref.py:96-108 is defined for any T). */
int eii_model_set_rope(eii_model* m, const int64_t* cos_host, const int64_t* sin_host, int rows);
int eii_model_rope_rows(const eii_model* m);

/* (bits, f) of the 12 sites of layer l in fm order, into fm24[24]; f_y into *f_y. */
int eii_model_formats(const eii_model* m, int layer, int64_t* fm24, int64_t* f_y);

/* Batched forward (python/intref.py:288-301 for B independent sequences of T tokens).
 * ids_dev int64 [B*T].  Outputs, each optional (NULL = not written):
 *   embed_out_dev int32 [S*T, 576]; resid_out_dev int32 [30, S*T, 576] (after each block);
 *   logits_dev int32 [B*T, 49152] (f = 16; exact when |logit| < 2^31, which
 *   python/export_vectors.py:58 asserts; eii_check reports a logit outside int32).
 * dump_mask_host uint8 [B] (NULL = every sequence) selects the S sequences whose embedding and
 * residual states are written, packed in batch order; logits cover every sequence. */
int eii_forward(eii_model* m, const int64_t* ids_dev, int B, int T, int32_t* embed_out_dev,
                int32_t* resid_out_dev, int32_t* logits_dev, const uint8_t* dump_mask_host,
                void* stream);

/* Ragged batch: seq_lens_host[nseq] tokens per sequence, ids packed sequence after sequence;
 * dump_mask_host uint8 [nseq] as for eii_forward. */
int eii_forward_packed(eii_model* m, const int64_t* ids_dev, const int32_t* seq_lens_host, int nseq,
                       int32_t* embed_out_dev, int32_t* resid_out_dev, int32_t* logits_dev,
                       const uint8_t* dump_mask_host, void* stream);

/* Run eii_forward / eii_forward_packed as HIP graphs (on != 0) or as individual launches (0, the
 * default).  With graphs on, the first call for a batch shape and set of buffer pointers (ids,
 * outputs, dump mask) captures the forward's launches into a graph and replays it on `stream`;
 * later calls with the same shape and pointers replay that graph (no host work per kernel).  Growing the workspace or replacing the RoPE tables drops the graphs; profiling
 * (eii_profile_begin) runs the plain launches.  No counterpart in the reference. */
int eii_model_set_graphs(eii_model* m, int on);

/* Waits for `stream`, then reports data-dependent violations seen since the last check:
 * a token id outside [0, 49152) or a logit outside int32 (status 4). */
int eii_check(eii_model* m, void* stream);

/* One decoder block in place on x_dev int32 [B*T, 576] (python/intref.py:192-286),
 * optional per-site dumps. */
int eii_block(eii_model* m, int layer, int32_t* x_dev, int B, int T, const eii_trace* trace,
              void* stream);

/* Embedding lookup (python/intref.py:163-166): ids_dev int64 [M] -> x_dev int32 [M, 576]. */
int eii_embed(eii_model* m, const int64_t* ids_dev, int M, int32_t* x_dev, void* stream);

/* Final RMSNorm and tied head (python/intref.py:296-301): x_dev int32 [M, 576] ->
 * logits_dev int32 [M, 49152]. */
int eii_final(eii_model* m, const int32_t* x_dev, int M, int32_t* logits_dev, void* stream);

/* Kernel classes timed by eii_profile_begin/end. */
enum {
  EII_K_EMBED = 0, EII_K_NORM, EII_K_GEMM_QKV, EII_K_ROPE, EII_K_ATTN, EII_K_GEMM_O, EII_K_GEMM_GU,
  EII_K_SILU, EII_K_GEMM_DOWN, EII_K_GEMM_HEAD, EII_K_COUNT
};

/* Time every kernel launch of the model's forward/block/final calls with a pair of HIP events
 * recorded on the launch stream, for up to max_launches launches.  No counterpart in the
 * reference (which times whole runs, c/intref.c:225,256; cuda/intref.cu:283,302-304). */
int eii_profile_begin(eii_model* m, int max_launches);
/* Waits for `stream` and returns the summed milliseconds and launch counts per kernel class
 * into ms[EII_K_COUNT] and launches[EII_K_COUNT]; status 5 if launches were dropped. */
int eii_profile_end(eii_model* m, void* stream, double* ms, int* launches);

/* ---- incremental decoding with a KV cache ----
 * No counterpart in the reference, whose forward recomputes every position over the full prefix;
 * the cache is its stated next step (exact-integer-inference.tex:167, docs/CONFORMANCE.md:11).
 * Each position depends only on its prefix, so the logits of appended positions equal the rows
 * of a full forward (eii_forward) over the whole sequence. */
typedef struct eii_kv eii_kv;

/* A cache for B sequences of up to max_T positions each (q|k|v rows and V^T planes per layer). */
int eii_kv_create(eii_model* m, int B, int max_T, eii_kv** out);
void eii_kv_free(eii_kv* kv);
/* Positions held by every sequence; eii_kv_reset empties the cache. */
int eii_kv_length(const eii_kv* kv);
int eii_kv_reset(eii_kv* kv);
/* Appends T_new positions to every sequence: ids_dev int64 [B, T_new]; logits_dev int32
 * [B, T_new, 49152] (nullable) receives their logits.  A prompt is one append of its length,
 * each decoding step an append of 1.  After an error the cache contents are undefined: reset it. */
int eii_kv_append(eii_model* m, eii_kv* kv, const int64_t* ids_dev, int T_new, int32_t* logits_dev, void* stream);
/* Greedy choice: out_dev int64 [rows] = the lowest index of the largest of the n values of each row of
 * logits_dev int32 [rows, n] (numpy.argmax's tie rule). */
int eii_argmax(const int32_t* logits_dev, int rows, int n, int64_t* out_dev, void* stream);

/* ---- operator level (python/intref.py functions) ----
 * eii_gemm_i8, eii_gemm_i8_ws, eii_linear and eii_attention stage their operands (limb planes,
 * weights in fragment order, V^T planes and, for attention, k limb planes) in one device block
 * per GPU that the library keeps for
 * the life of the process and grows with hipMalloc when a call needs more; calls at sizes seen
 * before allocate nothing.  Calls on one GPU take the block in turn: each call's stream waits for
 * the previous call's work, whichever stream that was on. */

/* Row sums of int8 weights W_dev [N, K] into wsum_dev int32 [N]. */
int eii_weight_colsum(const int8_t* W_dev, int N, int K, int32_t* wsum_dev, void* stream);

/* Exact acc_dev int64 [M, N] = A W^T (python/intref.py:58-63 matmul_exact) with A_dev int8
 * (a_bits 8), int16 (16) or int32 (32) [M, K], W_dev int8 [N, K]; any K up to 131072 (zero-padded
 * to a multiple of 64 inside, which adds nothing), N a multiple of 4, M * K <= 2^31. */
int eii_gemm_i8(const void* A_dev, int a_bits, const int8_t* W_dev, int M, int N, int K,
                int64_t* acc_dev, void* stream);
/* The same with precomputed row sums (eii_weight_colsum). */
int eii_gemm_i8_ws(const void* A_dev, int a_bits, const int8_t* W_dev, const int32_t* wsum_dev,
                   int M, int N, int K, int64_t* acc_dev, void* stream);

/* eii_gemm_i8_ws without any allocation: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Operands are staged in a fixed 64 MiB device array per GPU that the library holds
 * until the process ends; needing more than that (limb planes of M x K rounded up to 64 columns,
 * 2 planes for 8/16-bit A and 4 for 32-bit, plus N rounded up to 32 rows x K weight bytes) is
 * status 4.  Calls on one GPU share that array: calls whose work overlaps on one GPU (different
 * streams, or host threads without ordering) race and must be serialized by the caller. */
int eii_gemm_i8_ws_noalloc(const void* A_dev, int a_bits, const int8_t* W_dev, const int32_t* wsum_dev,
                           int M, int N, int K, int64_t* acc_dev, void* stream);

/* Linear with requantization (python/intref.py:186-190):
 * out = SAT(RS(acc * mult[n], shift[n]), out_bits) evaluated in int64 on the exact accumulators,
 * for any int32 mult and shift[n] = n + f_in - f_out (the reference asserts shift >= 1 and
 * max |acc| * max mult < 2^63; a shift <= 0 is a left shift as RS defines it);
 * out_dev int16 (out_bits 16) or int32 (out_bits 32) [M, N].  A, W, M, N, K as eii_gemm_i8. */
int eii_linear(const void* A_dev, int a_bits, const int8_t* W_dev, const int32_t* wsum_dev,
               const int32_t* mult_dev, const int32_t* shift_dev, int M, int N, int K,
               int out_bits, void* out_dev, void* stream);

/* RMSNorm (python/intref.py:168-184): x_dev int32 [M, 576] -> out_dev [M, 576] of out_bits
 * (16 -> int16, 32 -> int32); gain_dev int32 [576] with exponent f_gain, any int32 gain (3 z gain
 * formed in int64 and saturated before narrowing, as c/intref.c:106-108); the three pointers
 * 16-byte aligned.  (A model.bin's gains must be int16, as quant_vec_int16 makes them,
 * python/intref.py:126-130; eii_model_load rejects wider ones with status 4.) */
int eii_rmsnorm(const int32_t* x_dev, int M, const int32_t* gain_dev, int f_gain, int f_out,
                int out_bits, void* out_dev, void* stream);

/* Attention of one block (python/intref.py:227-254) for nseq sequences packed by
 * seq_off_dev int32 [nseq + 1]: qkv_dev int16 [M, 960] holding q_rope | k_rope | v,
 * exp_tab_dev int32 [1537]; ctx_dev [M, 576] of bits_c (16 -> int16, 32 -> int32). */
int eii_attention(const int16_t* qkv_dev, const int32_t* seq_off_dev, int nseq, int max_T,
                  const int32_t* exp_tab_dev, int f_qr, int f_kr, int f_v, int f_c, int bits_c,
                  void* ctx_dev, void* stream);

/* RoPE of one block (python/intref.py:212-225), in place on the q and k columns of qkv_dev
 * int16 [M, 960] (q | k | v rows) for nseq sequences packed by seq_off_dev int32 [nseq + 1]
 * (contiguous from row 0): row r of sequence i is position r - seq_off[i]. cos_dev, sin_dev
 * int32 [rows, 32] hold rope_tables' Q30 values (python/intref.py:96-108). q heads:
 * SAT(RS(., 30 + f_q - f_qr), bits_qr), k heads likewise with f_k, f_kr, bits_kr (bits <= 16). */
int eii_rope(int16_t* qkv_dev, const int32_t* seq_off_dev, int nseq, const int32_t* cos_dev,
             const int32_t* sin_dev, int rows, int f_q, int f_qr, int bits_qr, int f_k, int f_kr,
             int bits_kr, void* stream);

/* SiLU gate of the MLP (python/intref.py:272-276): out_dev [M, 1536] of bits_m (16 -> int16,
 * 32 -> int32) = SAT(RS(silu_dev[g + 32768] * u, f_s + f_u - f_m), bits_m) for gate_dev and
 * up_dev int16 [M, 1536] and silu_dev int32 [65536] (silu_table at the gate's format,
 * python/intref.py:80-93); f_m is the gated format after the reference's min() for 32 bits. */
int eii_silu_gate(const int16_t* gate_dev, const int16_t* up_dev, int M, const int32_t* silu_dev,
                  int f_s, int f_u, int f_m, int bits_m, void* out_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* EII_H */
