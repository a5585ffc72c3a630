// Host side of libeii: model.bin loading, the batched forward and the C ABI (include/eii.h).
//
// model.bin is the reference's file ABI (python/export_vectors.py:24-45): sequential
// little-endian arrays, all scalars int64.  The loader narrows every field to the width the
// semantics allow (int8 weights, 14-bit multipliers, per-row shifts, Q30 tables) and rejects
// a file whose values do not fit, so the kernels never meet an out-of-range operand.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/eii.h"
#include "eii_int.h"
#include "kernels.h"

using namespace eii;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define HIPCHK(expr)                                                                        \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      return fail(EII_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));         \
  } while (0)

enum Site { NORM1 = 0, QP, KP, VP, QR, KR, CTX, NORM2, GATE, UP, SILU, GATED, NSITES };
const char* kSiteNames[NSITES] = {"norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope",
                                  "attn_ctx", "norm2_out", "gate_proj", "up_proj", "silu_gate", "mlp_gated"};
const int kMatN[7] = {576, 192, 192, 576, 1536, 1536, 576};
const int kMatK[7] = {576, 576, 576, 576, 576, 576, 1536};

struct Mat {            // device arrays of one projection (possibly several matrices stacked)
  int8_t* W = nullptr;  // [N, K] row-major (model arena)
  int32_t* mult = nullptr;
  int32_t* shift = nullptr;
  int32_t* wsum = nullptr;
  int N = 0, K = 0;
  double2* coef = nullptr;   // [N] float64 requantization coefficients for 2-limb inputs
  int8_t* Wf = nullptr;      // the same weights in the GEMM's fragment order (kernels.h)
};

struct Layer {
  int bits[NSITES], f[NSITES];
  int64_t fm[24];
  int f_m;               // gated exponent actually used (python/intref.py:274)
  int32_t *ln1, *ln2;
  int ln1_f, ln2_f;
  Mat qkv, o, gu, down;
  int32_t* silu;
};

// Device arena: one allocation for all model arrays.
struct Arena {
  std::vector<uint8_t> host;
  size_t off = 0;
  size_t take(size_t bytes) {
    off = (off + 255) & ~(size_t)255;
    size_t o = off;
    off += bytes;
    if (host.size() < off) host.resize(off);
    return o;
  }
};

}  // namespace

struct eii_model {
  int device = 0;
  uint8_t* dev = nullptr;           // arena base
  int8_t* wfrag = nullptr;          // fragment-ordered copies of every projection's weights
  // header arrays (device)
  int8_t* emb_q = nullptr;
  int32_t *emb_m = nullptr, *emb_sh = nullptr;   // embed shift n - 15
  Mat head;                                       // tied head: W = emb_q, shift = n + f_y - 16
  int32_t* fg = nullptr;
  int fg_f = 0, f_y = 0;
  int32_t* exp_tab = nullptr;
  int32_t *rope_c = nullptr, *rope_s = nullptr;   // [rope_rows, 32]
  int rope_rows = 0;
  bool rope_owned = false;
  Layer L[kNL];
  int64_t fy_raw = 0;
  // workspace
  size_t ws_rows = 0;
  int32_t* x = nullptr;            // [M, 576]
  void* h = nullptr;               // [M, 576] up to int32
  int16_t* qkv = nullptr;          // [M, 960]
  uint8_t* vt = nullptr;           // V^T limb planes (kernels.h vt_bytes)
  uint8_t* kpl = nullptr;          // k limb planes of long-row attention (kernels.h attn_kpl_bytes)
  void* ctx = nullptr;             // [M, 576] up to int32
  int16_t* gu = nullptr;           // [M, 3072]
  void* gated = nullptr;           // [M, 1536] up to int32
  int32_t* pos = nullptr;          // [M]
  int32_t* seq_off = nullptr;      // [nseq + 1]
  size_t seq_cap = 0;
  int max_kt = 0;                  // key tiles of the longest-spanning sequence of the batch
  std::vector<int32_t> last_lens;
  int* flags = nullptr;            // [1]: 1 logit overflow, 2 token id out of range
  // per-launch event timing between eii_profile_begin and eii_profile_end
  bool prof = false;
  std::vector<hipEvent_t> ev;      // start/stop pairs
  std::vector<int> ev_kind;
  size_t ev_used = 0;
  // HIP graphs of whole forwards (eii_model_set_graphs): captured on an internal stream the first
  // time a batch shape and set of output buffers is seen, replayed on the caller's stream after.
  // The graphs hold the workspace and table addresses, so growing the workspace or replacing the
  // RoPE tables drops them.
  struct FwdGraph {
    std::vector<int32_t> lens;
    const void *ids, *emb, *res, *lg;
    std::vector<uint8_t> mask;
    hipGraphExec_t exec;
  };
  bool graphs = false;
  hipStream_t cap_stream = nullptr;
  std::vector<FwdGraph> fwd_graphs;
};

// KV cache of incremental decoding: per layer the q|k|v rows (int16 [B cap][960], row b cap + t
// = position t of sequence b) and the V^T limb planes of those rows (vt_stride_for(B cap)).
struct eii_kv {
  int device = 0;
  int B = 0, cap = 0;              // sequences, positions per sequence (a multiple of 32)
  int len = 0;                     // positions held by every sequence
  int vt_len = 0;                  // positions whose V^T planes are written (single-token steps
                                   // served by the one-query decoding kernel leave them out)
  uint8_t* dev = nullptr;          // one allocation for all layers
  int16_t* qkv[kNL] = {};
  uint8_t* vt[kNL] = {};
  int32_t* seq_off = nullptr;      // [B + 1] = b cap
};

namespace {
// Records a start and stop event around the launches made in its scope, on their stream.
struct ProfScope {
  eii_model* m;
  hipStream_t s;
  size_t i = 0;
  bool on;
  ProfScope(eii_model* m_, int kind, hipStream_t s_) : m(m_), s(s_) {
    on = m->prof && m->ev_used + 2 <= m->ev.size();
    if (on) {
      i = m->ev_used;
      m->ev_used += 2;
      m->ev_kind[i / 2] = kind;
      (void)hipEventRecord(m->ev[i], s);
    }
  }
  ~ProfScope() {
    if (on) (void)hipEventRecord(m->ev[i + 1], s);
  }
};
}  // namespace

namespace {

// ------------------------------------------------------------------------------ loading
struct Reader {
  const uint8_t* p;
  size_t n, off = 0;
  bool ok = true;
  const uint8_t* bytes(size_t k) {
    if (off + k > n) { ok = false; return nullptr; }
    const uint8_t* r = p + off;
    off += k;
    return r;
  }
  int64_t i64() {
    const uint8_t* b = bytes(8);
    if (!b) return 0;
    int64_t v;
    memcpy(&v, b, 8);
    return v;
  }
  std::vector<int64_t> vec(size_t k) {
    std::vector<int64_t> v(k);
    const uint8_t* b = bytes(8 * k);
    if (b) memcpy(v.data(), b, 8 * k);
    return v;
  }
};

bool fits32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

int narrow32(const std::vector<int64_t>& v, int32_t* dst, int64_t lo, int64_t hi, const std::string& what) {
  for (size_t i = 0; i < v.size(); ++i) {
    if (v[i] < lo || v[i] > hi)
      return fail(EII_E_BOUND, what + "[" + std::to_string(i) + "] = " + std::to_string(v[i]) +
                                   " outside [" + std::to_string(lo) + ", " + std::to_string(hi) + "]");
    dst[i] = (int32_t)v[i];
  }
  return EII_OK;
}

int check_site(const Layer& L, int l, int s, bool allow32) {
  const int b = L.bits[s];
  if (!(b == 16 || (allow32 && b == 32)))
    return fail(EII_E_BOUND, "layer " + std::to_string(l) + " site " + kSiteNames[s] + ": " +
                                 std::to_string(b) + "-bit format is not supported here");
  if (L.f[s] < -64 || L.f[s] > 64)
    return fail(EII_E_BOUND, "layer " + std::to_string(l) + " site " + kSiteNames[s] + ": f out of range");
  return EII_OK;
}

int check_scalar_shift(int sh, const std::string& what) {
  if (sh < -30 || sh > 62) return fail(EII_E_BOUND, what + " shift " + std::to_string(sh) + " out of range");
  return EII_OK;
}

}  // namespace

extern "C" const char* eii_last_error(void) { return g_err.c_str(); }

extern "C" int eii_model_load(const char* path, int device, eii_model** out) {
  if (!path || !out) return fail(EII_E_ARG, "null argument");
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return fail(EII_E_IO, std::string(path) + ": cannot open");
  fseek(f, 0, SEEK_END);
  const long size = ftell(f);
  fseek(f, 0, SEEK_SET);
  const size_t expect = 154045048;
  if (size != (long)expect) {
    fclose(f);
    return fail(EII_E_IO, std::string(path) + ": " + std::to_string(size) + " bytes, a model.bin holds " +
                              std::to_string(expect));
  }
  std::vector<uint8_t> file(expect);
  const size_t got = fread(file.data(), 1, expect, f);
  fclose(f);
  if (got != expect) return fail(EII_E_IO, std::string(path) + ": short read");

  Reader rd{file.data(), file.size()};
  Arena ar;
  int rc;
  eii_model* M = new eii_model();
  M->device = device;

  // offsets into the arena, resolved to device pointers after the upload
  struct MatOff { size_t W, mult, shift, wsum; int N, K; size_t coef; };
  size_t o_embq = ar.take((size_t)kV * kD);
  memcpy(ar.host.data() + o_embq, rd.bytes((size_t)kV * kD), (size_t)kV * kD);
  const std::vector<int64_t> emb_m = rd.vec(kV), emb_n = rd.vec(kV), fgq = rd.vec(kD);
  const int64_t fg_f = rd.i64(), f_y = rd.i64();
  const std::vector<int64_t> expt = rd.vec(kDMax + 1), rc_ = rd.vec(512 * 32), rs_ = rd.vec(512 * 32);
  if (!rd.ok) { delete M; return fail(EII_E_IO, "short read in header"); }
  if (fg_f < -64 || fg_f > 64 || f_y < -64 || f_y > 64) { delete M; return fail(EII_E_BOUND, "final gain/f_y exponent out of range"); }
  M->fg_f = (int)fg_f;
  M->f_y = (int)f_y;

  size_t o_embm = ar.take(4 * kV), o_embsh = ar.take(4 * kV), o_headsh = ar.take(4 * kV), o_headws = ar.take(4 * kV);
  size_t o_headcoef = ar.take(16 * (size_t)kV);
  size_t o_fg = ar.take(4 * kD), o_exp = ar.take(4 * (kDMax + 1)), o_rc = ar.take(4 * 512 * 32), o_rs = ar.take(4 * 512 * 32);
  {
    std::vector<int64_t> esh(kV), hsh(kV);
    for (int i = 0; i < kV; ++i) { esh[i] = emb_n[i] - kFRes; hsh[i] = emb_n[i] + f_y - 16; }
    if ((rc = narrow32(emb_m, (int32_t*)(ar.host.data() + o_embm), -(1 << 14), 1 << 14, "emb_m")) ||
        (rc = narrow32(esh, (int32_t*)(ar.host.data() + o_embsh), 1, 62, "embedding shift emb_n - 15")) ||
        (rc = narrow32(hsh, (int32_t*)(ar.host.data() + o_headsh), 1, 62, "head shift emb_n + f_y - 16")) ||
        (rc = narrow32(fgq, (int32_t*)(ar.host.data() + o_fg), -32768, 32767, "final gain")) ||
        (rc = narrow32(expt, (int32_t*)(ar.host.data() + o_exp), 0, INT32_MAX, "exp table")) ||
        (rc = narrow32(rc_, (int32_t*)(ar.host.data() + o_rc), INT32_MIN, INT32_MAX, "rope cos")) ||
        (rc = narrow32(rs_, (int32_t*)(ar.host.data() + o_rs), INT32_MIN, INT32_MAX, "rope sin"))) {
      delete M;
      return rc;
    }
    if (expt[0] < 1) { delete M; return fail(EII_E_BOUND, "exp table entry 0 must be positive"); }
  }

  struct LayerOff { size_t ln1, ln2, silu; MatOff qkv, o, gu, down; };
  std::vector<LayerOff> lo(kNL);
  for (int l = 0; l < kNL; ++l) {
    Layer& L = M->L[l];
    for (int i = 0; i < 24; ++i) L.fm[i] = rd.i64();
    for (int s = 0; s < NSITES; ++s) {
      if (L.fm[2 * s] < 0 || L.fm[2 * s] > 64 || L.fm[2 * s + 1] < -64 || L.fm[2 * s + 1] > 64) {
        delete M;
        return fail(EII_E_BOUND, "layer " + std::to_string(l) + ": fm record out of range");
      }
      L.bits[s] = (int)L.fm[2 * s];
      L.f[s] = (int)L.fm[2 * s + 1];
    }
    const std::vector<int64_t> ln1 = rd.vec(kD);
    const int64_t ln1f = rd.i64();
    const std::vector<int64_t> ln2 = rd.vec(kD);
    const int64_t ln2f = rd.i64();
    if (!rd.ok) { delete M; return fail(EII_E_IO, "short read in layer " + std::to_string(l)); }
    if ((rc = check_site(L, l, NORM1, true)) || (rc = check_site(L, l, QP, false)) ||
        (rc = check_site(L, l, KP, false)) || (rc = check_site(L, l, VP, false)) ||
        (rc = check_site(L, l, QR, false)) || (rc = check_site(L, l, KR, false)) ||
        (rc = check_site(L, l, CTX, true)) || (rc = check_site(L, l, NORM2, true)) ||
        (rc = check_site(L, l, GATE, false)) || (rc = check_site(L, l, UP, false)) ||
        (rc = check_site(L, l, SILU, true)) || (rc = check_site(L, l, GATED, true))) {
      delete M;
      return rc;
    }
    if (ln1f < -64 || ln1f > 64 || ln2f < -64 || ln2f > 64) { delete M; return fail(EII_E_BOUND, "gain exponent out of range"); }
    L.ln1_f = (int)ln1f;
    L.ln2_f = (int)ln2f;
    L.f_m = L.bits[GATED] == 32 ? std::min(L.f[GATED], L.f[SILU] + L.f[UP]) : L.f[GATED];
    const int shift_s = L.f[QR] + L.f[KR] + 3 - kFScore;
    if (shift_s < 1) { delete M; return fail(EII_E_BOUND, "layer " + std::to_string(l) + ": score shift < 1"); }
    // the attention kernel evaluates scores in int32 pieces that need shift <= 30 (formats give <= 26)
    if (shift_s > 30) { delete M; return fail(EII_E_BOUND, "layer " + std::to_string(l) + ": score shift > 30"); }
    if ((rc = check_scalar_shift(21 + L.ln1_f - L.f[NORM1], "norm1")) ||
        (rc = check_scalar_shift(21 + L.ln2_f - L.f[NORM2], "norm2")) ||
        (rc = check_scalar_shift(30 + L.f[QP] - L.f[QR], "q rope")) ||
        (rc = check_scalar_shift(30 + L.f[KP] - L.f[KR], "k rope")) ||
        (rc = check_scalar_shift(shift_s, "score")) ||
        (rc = check_scalar_shift(16 + L.f[VP] - L.f[CTX], "context")) ||
        (rc = check_scalar_shift(L.f[SILU] + L.f[UP] - L.f_m, "gated"))) {
      delete M;
      return rc;
    }
    LayerOff& O = lo[l];
    O.ln1 = ar.take(4 * kD);
    O.ln2 = ar.take(4 * kD);
    // RMSNorm gains are int16 (python/intref.py:126-130 quant_vec_int16); the forward's norm kernel
    // relies on |3 gain| < 2^17
    if ((rc = narrow32(ln1, (int32_t*)(ar.host.data() + O.ln1), -32768, 32767, "ln1")) ||
        (rc = narrow32(ln2, (int32_t*)(ar.host.data() + O.ln2), -32768, 32767, "ln2"))) {
      delete M;
      return rc;
    }
    // projections, stacked: qkv = q | k | v, gu = gate | up
    O.qkv = {ar.take((size_t)960 * 576), ar.take(4 * 960), ar.take(4 * 960), ar.take(4 * 960), 960, 576, ar.take(16 * 960)};
    O.o = {ar.take((size_t)576 * 576), ar.take(4 * 576), ar.take(4 * 576), ar.take(4 * 576), 576, 576, ar.take(16 * 576)};
    O.gu = {ar.take((size_t)3072 * 576), ar.take(4 * 3072), ar.take(4 * 3072), ar.take(4 * 3072), 3072, 576,
            ar.take(16 * 3072)};
    O.down = {ar.take((size_t)576 * 1536), ar.take(4 * 576), ar.take(4 * 576), ar.take(4 * 576), 576, 1536,
              ar.take(16 * 576)};
    // matrix i -> (stack, row offset, f_in, f_out)
    const MatOff* dst[7] = {&O.qkv, &O.qkv, &O.qkv, &O.o, &O.gu, &O.gu, &O.down};
    const int row0[7] = {0, 576, 768, 0, 0, 32, 0};
    const int fin[7] = {L.f[NORM1], L.f[NORM1], L.f[NORM1], L.f[CTX], L.f[NORM2], L.f[NORM2], L.f_m};
    const int fout[7] = {L.f[QP], L.f[KP], L.f[VP], kFRes, L.f[GATE], L.f[UP], kFRes};
    static const char* names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    for (int i = 0; i < 7; ++i) {
      const int N = kMatN[i], K = kMatK[i];
      const uint8_t* wq = rd.bytes((size_t)N * K);
      const std::vector<int64_t> m = rd.vec(N), n = rd.vec(N);
      if (!rd.ok) { delete M; return fail(EII_E_IO, "short read in layer " + std::to_string(l)); }
      // stacked row of matrix row r: gate and up interleave in blocks of 32 rows
      // ([gate 32b..32b+31 | up 32b..32b+31]) so one wave's block holds (gate j, up j) pairs
      auto srow = [&](int r) { return (i == 4 || i == 5) ? 64 * (r / 32) + row0[i] + r % 32 : row0[i] + r; };
      std::vector<int64_t> sh(N);
      for (int r = 0; r < N; ++r) sh[r] = n[r] + fin[i] - fout[i];
      const std::string what = "layer " + std::to_string(l) + " " + names[i];
      std::vector<int32_t> m32(N), sh32(N);
      if ((rc = narrow32(m, m32.data(), -(1 << 14), 1 << 14, what + " m")) ||
          (rc = narrow32(sh, sh32.data(), 1, 62, what + " requant shift"))) {
        delete M;
        return rc;
      }
      for (int r = 0; r < N; ++r) {
        const int sr = srow(r);
        memcpy(ar.host.data() + dst[i]->W + (size_t)sr * K, wq + (size_t)r * K, K);
        ((int32_t*)(ar.host.data() + dst[i]->mult))[sr] = m32[r];
        ((int32_t*)(ar.host.data() + dst[i]->shift))[sr] = sh32[r];
      }
    }
    const std::vector<int64_t> silu = rd.vec(65536);
    if (!rd.ok) { delete M; return fail(EII_E_IO, "short read in layer " + std::to_string(l)); }
    O.silu = ar.take(4 * 65536);
    const int bs = L.bits[SILU];
    if ((rc = narrow32(silu, (int32_t*)(ar.host.data() + O.silu), -(1LL << (bs - 1)), (1LL << (bs - 1)) - 1,
                       "layer " + std::to_string(l) + " silu table"))) {
      delete M;
      return rc;
    }
  }
  if (rd.off != rd.n) { delete M; return fail(EII_E_IO, "model.bin has trailing bytes"); }

  // upload
  HIPCHK(hipSetDevice(device));
  if (hipMalloc(&M->dev, ar.host.size()) != hipSuccess) { delete M; return fail(EII_E_DEVICE, "hipMalloc of the model failed"); }
  if (hipMemcpy(M->dev, ar.host.data(), ar.host.size(), hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(M->dev); delete M; return fail(EII_E_DEVICE, "model upload failed");
  }
  uint8_t* d = M->dev;
  M->emb_q = (int8_t*)(d + o_embq);
  M->emb_m = (int32_t*)(d + o_embm);
  M->emb_sh = (int32_t*)(d + o_embsh);
  M->head = {M->emb_q, M->emb_m, (int32_t*)(d + o_headsh), (int32_t*)(d + o_headws), kV, kD,
             (double2*)(d + o_headcoef)};
  M->fg = (int32_t*)(d + o_fg);
  M->exp_tab = (int32_t*)(d + o_exp);
  M->rope_c = (int32_t*)(d + o_rc);
  M->rope_s = (int32_t*)(d + o_rs);
  M->rope_rows = 512;
  auto mat = [&](const MatOff& o) {
    return Mat{(int8_t*)(d + o.W), (int32_t*)(d + o.mult), (int32_t*)(d + o.shift), (int32_t*)(d + o.wsum), o.N, o.K,
               (double2*)(d + o.coef)};
  };
  for (int l = 0; l < kNL; ++l) {
    Layer& L = M->L[l];
    L.ln1 = (int32_t*)(d + lo[l].ln1);
    L.ln2 = (int32_t*)(d + lo[l].ln2);
    L.silu = (int32_t*)(d + lo[l].silu);
    L.qkv = mat(lo[l].qkv);
    L.o = mat(lo[l].o);
    L.gu = mat(lo[l].gu);
    L.down = mat(lo[l].down);
  }
  M->fy_raw = f_y;
  // weight row sums for the limb bias correction
  // weight row sums for the limb bias correction, then the float64 requantization coefficients
  hipError_t e = weight_colsum(M->head.W, kV, kD, M->head.wsum, nullptr);
  if (e == hipSuccess) e = gemm_coef(M->head.mult, M->head.shift, M->head.wsum, kV, M->head.coef, nullptr);
  for (int l = 0; l < kNL && e == hipSuccess; ++l) {
    Layer& L = M->L[l];
    Mat* ms[4] = {&L.qkv, &L.o, &L.gu, &L.down};
    for (Mat* m : ms) {
      if (e == hipSuccess) e = weight_colsum(m->W, m->N, m->K, m->wsum, nullptr);
      if (e == hipSuccess) e = gemm_coef(m->mult, m->shift, m->wsum, m->N, m->coef, nullptr);
    }
  }
  // fragment-ordered weights for the GEMMs (the arena keeps the row-major ones: the embedding
  // lookup reads emb_q by row)
  {
    std::vector<Mat*> all{&M->head};
    for (int l = 0; l < kNL; ++l) {
      Layer& L = M->L[l];
      all.insert(all.end(), {&L.qkv, &L.o, &L.gu, &L.down});
    }
    size_t total = 0;
    for (Mat* m : all) total += (swizzled_bytes(m->N, m->K) + 255) & ~(size_t)255;
    if (e == hipSuccess) e = hipMalloc(&M->wfrag, total);
    size_t off = 0;
    for (Mat* m : all) {
      if (e != hipSuccess) break;
      m->Wf = M->wfrag + off;
      off += (swizzled_bytes(m->N, m->K) + 255) & ~(size_t)255;
      e = swizzle_weights(m->W, m->N, m->K, m->Wf, nullptr);
    }
  }
  if (e == hipSuccess) e = hipMalloc(&M->flags, 16);
  if (e == hipSuccess) e = hipMemset(M->flags, 0, 16);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) { eii_model_free(M); return fail(EII_E_DEVICE, std::string("model setup: ") + hipGetErrorString(e)); }
  *out = M;
  return EII_OK;
}

static void free_ws(eii_model* m) {
  void* ps[] = {m->x, m->h, m->qkv, m->vt, m->kpl, m->ctx, m->gu, m->gated, m->pos};
  for (void* p : ps) if (p) (void)hipFree(p);
  m->x = nullptr; m->h = nullptr; m->qkv = nullptr; m->vt = nullptr; m->kpl = nullptr; m->ctx = nullptr; m->gu = nullptr;
  m->gated = nullptr; m->pos = nullptr;
  m->ws_rows = 0;
}

static void drop_graphs(eii_model* m) {
  for (auto& gr : m->fwd_graphs) (void)hipGraphExecDestroy(gr.exec);
  m->fwd_graphs.clear();
}

extern "C" void eii_model_free(eii_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  drop_graphs(m);
  if (m->cap_stream) (void)hipStreamDestroy(m->cap_stream);
  free_ws(m);
  if (m->seq_off) (void)hipFree(m->seq_off);
  if (m->rope_owned) { (void)hipFree(m->rope_c); (void)hipFree(m->rope_s); }
  if (m->flags) (void)hipFree(m->flags);
  for (hipEvent_t e : m->ev) (void)hipEventDestroy(e);
  if (m->dev) (void)hipFree(m->dev);
  if (m->wfrag) (void)hipFree(m->wfrag);
  delete m;
}

extern "C" int eii_model_set_rope(eii_model* m, const int64_t* c, const int64_t* s, int rows) {
  if (!m || !c || !s || rows <= 0) return fail(EII_E_ARG, "bad rope arguments");
  std::vector<int32_t> hc((size_t)rows * 32), hs((size_t)rows * 32);
  for (size_t i = 0; i < hc.size(); ++i) {
    if (!fits32(c[i]) || !fits32(s[i])) return fail(EII_E_BOUND, "rope table entry outside int32");
    hc[i] = (int32_t)c[i];
    hs[i] = (int32_t)s[i];
  }
  HIPCHK(hipSetDevice(m->device));
  int32_t *dc = nullptr, *ds = nullptr;
  HIPCHK(hipMalloc(&dc, hc.size() * 4));
  if (hipMalloc(&ds, hs.size() * 4) != hipSuccess) { (void)hipFree(dc); return fail(EII_E_DEVICE, "rope alloc"); }
  HIPCHK(hipDeviceSynchronize());
  if (hipMemcpy(dc, hc.data(), hc.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(ds, hs.data(), hs.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(dc); (void)hipFree(ds);
    return fail(EII_E_DEVICE, "rope upload");
  }
  if (m->rope_owned) { (void)hipFree(m->rope_c); (void)hipFree(m->rope_s); }
  drop_graphs(m);
  m->rope_c = dc;
  m->rope_s = ds;
  m->rope_rows = rows;
  m->rope_owned = true;
  return EII_OK;
}

extern "C" int eii_model_rope_rows(const eii_model* m) { return m ? m->rope_rows : 0; }

extern "C" int eii_model_formats(const eii_model* m, int layer, int64_t* fm24, int64_t* f_y) {
  if (!m || layer < 0 || layer >= kNL) return fail(EII_E_ARG, "bad layer");
  if (fm24) memcpy(fm24, m->L[layer].fm, sizeof(m->L[layer].fm));
  if (f_y) *f_y = m->fy_raw;
  return EII_OK;
}

// ------------------------------------------------------------------------------ forward
namespace {

int ensure_ws(eii_model* m, size_t rows) {
  if (rows <= m->ws_rows) return EII_OK;
  drop_graphs(m);
  free_ws(m);
  size_t r = rows;
  hipError_t e = hipSuccess;
  auto al = [&](void** p, size_t bytes) { if (e == hipSuccess) e = hipMalloc(p, bytes); };
  al((void**)&m->x, r * kD * 4);
  al(&m->h, r * kD * 4);
  al((void**)&m->qkv, r * kQKVN * 2);
  al((void**)&m->vt, vt_bytes((int)r));
  al((void**)&m->kpl, attn_kpl_bytes((int)r));
  al(&m->ctx, r * kD * 4);
  al((void**)&m->gu, r * 2 * kDFF * 2);
  al(&m->gated, r * kDFF * 4);
  al((void**)&m->pos, r * 4);
  if (e != hipSuccess) { free_ws(m); return fail(EII_E_DEVICE, "workspace allocation failed"); }
  m->ws_rows = r;
  m->last_lens.clear();
  return EII_OK;
}

// Uploads positions and sequence offsets for this batch shape (cached between calls).
int set_batch(eii_model* m, const std::vector<int32_t>& lens, hipStream_t s) {
  if (lens == m->last_lens) return EII_OK;
  size_t rows = 0;
  std::vector<int32_t> off(lens.size() + 1, 0), pos;
  int max_kt = 0;
  for (size_t i = 0; i < lens.size(); ++i) {
    off[i + 1] = off[i] + lens[i];
    max_kt = std::max(max_kt, attn_key_tiles(off[i], lens[i]));
    for (int t = 0; t < lens[i]; ++t) pos.push_back(t);
  }
  rows = pos.size();
  if (m->seq_cap < off.size()) {
    if (m->seq_off) (void)hipFree(m->seq_off);
    m->seq_off = nullptr;
    HIPCHK(hipMalloc(&m->seq_off, off.size() * 4));
    m->seq_cap = off.size();
  }
  HIPCHK(hipMemcpyAsync(m->seq_off, off.data(), off.size() * 4, hipMemcpyHostToDevice, s));
  if (rows) HIPCHK(hipMemcpyAsync(m->pos, pos.data(), rows * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipStreamSynchronize(s));    // the host vectors die at return
  m->last_lens = lens;
  m->max_kt = max_kt;
  return EII_OK;
}

GemmArgs gemm_args(const Mat& W, const void* planes, int M, void* out, int sat_bits) {
  GemmArgs g{planes, W.Wf, M, W.N, W.K, (size_t)M * W.K, W.wsum, W.mult, W.shift, out, sat_bits, nullptr};
  g.coef = W.coef;
  return g;
}

hipError_t copy_cols(void* dst, int dst_w, const void* src, int src_w, int col0, int ncols, int esz, int rows,
                     hipStream_t s) {
  return hipMemcpy2DAsync(dst, (size_t)dst_w * esz, (const uint8_t*)src + (size_t)col0 * esz, (size_t)src_w * esz,
                          (size_t)ncols * esz, rows, hipMemcpyDeviceToDevice, s);
}

// One decoder block (python/intref.py:192-286) on x [M, 576].  Norm outputs, the attention
// context and the gated product live in m->h, m->ctx and m->gated as int8 limb planes; with a
// trace the unfused q/k/v and gate/up projections run so their values can be dumped, and the
// producers also write plain copies into the trace buffers.
// One step of incremental decoding: T_new new positions of every sequence, from position p0;
// vt: the step's attention reads the V^T planes (the tiled kernel), so the append writes them too.
struct KvStep {
  eii_kv* kv;
  int T_new, p0;
  bool vt;
};

// At most 4 rows (decoding steps of up to 4 sequences) and no trace of the norm: the projection
// after an RMSNorm forms the normalized rows from x itself (GemmArgs::nx), in the rmsnorm
// launcher's fast path (gains in int16, which the loader enforces; output shift 10..40) for
// 16-bit norm outputs
bool fuse_norm(int M, int sh_out, int bits, const eii_trace* tr) {
  return !tr && M <= 4 && bits == 16 && sh_out >= 10 && sh_out <= 40;
}

int run_block(eii_model* m, int l, int32_t* x, int M, int nseq, int max_T, const eii_trace* tr, hipStream_t s,
              const KvStep* kv = nullptr) {
  const Layer& L = m->L[l];
  const int hb = L.bits[NORM1] / 8;
  uint8_t* h = (uint8_t*)m->h;
  const int sh_n1 = 21 + L.ln1_f - L.f[NORM1], sh_n2 = 21 + L.ln2_f - L.f[NORM2];
  if (!fuse_norm(M, sh_n1, L.bits[NORM1], tr)) {
    ProfScope ps(m, EII_K_NORM, s);
    HIPCHK(rmsnorm(x, M, L.ln1, sh_n1, L.bits[NORM1], h, tr ? tr->norm1_out : nullptr, s, false,
                   tr ? tr->norm1_U : nullptr, tr ? tr->norm1_z : nullptr));
  }
  const int sh_q = 30 + L.f[QP] - L.f[QR], sh_k = 30 + L.f[KP] - L.f[KR];
  {
    ProfScope ps(m, EII_K_GEMM_QKV, s);
    GemmArgs g = gemm_args(L.qkv, h, M, m->qkv, 16);
    if (fuse_norm(M, sh_n1, L.bits[NORM1], tr)) { g.nx = x; g.ngain = L.ln1; g.nsh = sh_n1; }
    if (!tr) {   // q, k, v projections with RoPE and the V^T planes in the epilogue
      g.pos = m->pos; g.cosT = m->rope_c; g.sinT = m->rope_s; g.sh_q = sh_q; g.sh_k = sh_k;
      if (!kv) { g.vt = m->vt; g.vt_stride = vt_stride_for(M); }
      // a single-token step whose attention reads no V^T planes writes its rows straight into
      // their cache rows (row b at position p0 of sequence b: stride cap rows)
      const bool direct = kv && !kv->vt && kv->T_new == 1 && (int64_t)kv->kv->cap * kQKVN * 64 < ((int64_t)1 << 31);
      if (direct) {
        g.out = kv->kv->qkv[l] + (size_t)kv->p0 * kQKVN;
        g.ldc = kv->kv->cap * kQKVN;
      }
      HIPCHK(gemm(g, hb, EPI_QKV, s));
      // decoding: the new rows join the cache, then (when this step's attention reads them) the
      // V^T planes of every position not yet covered, the new ones included, in one pass whose
      // stores run along the positions of each plane row
      if (kv && !direct) {
        eii_kv* c = kv->kv;
        HIPCHK(kv_append(m->qkv, nseq, kv->T_new, c->cap, kv->p0, c->qkv[l], s));
        if (kv->vt) HIPCHK(kv_build_vt(c->qkv[l], nseq, c->cap, c->vt_len, kv->p0 + kv->T_new, c->vt[l], s));
      }
    } else {
      HIPCHK(gemm(g, hb, EPI_REQ16, s));
    }
  }
  if (tr) {
    if (tr->q_proj) HIPCHK(copy_cols(tr->q_proj, kD, m->qkv, kQKVN, 0, kD, 2, M, s));
    if (tr->k_proj) HIPCHK(copy_cols(tr->k_proj, 192, m->qkv, kQKVN, kD, 192, 2, M, s));
    if (tr->v_proj) HIPCHK(copy_cols(tr->v_proj, 192, m->qkv, kQKVN, kD + 192, 192, 2, M, s));
    HIPCHK(rope(m->qkv, M, m->pos, m->rope_c, m->rope_s, sh_q, L.bits[QR], sh_k, L.bits[KR], s));
    if (tr->q_rope) HIPCHK(copy_cols(tr->q_rope, kD, m->qkv, kQKVN, 0, kD, 2, M, s));
    if (tr->k_rope) HIPCHK(copy_cols(tr->k_rope, 192, m->qkv, kQKVN, kD, 192, 2, M, s));
    HIPCHK(build_vt(m->qkv, M, m->vt, s));
    if (tr->attn_score || tr->attn_prob) {   // both written together: the probabilities re-read the scores
      if (!tr->attn_score || !tr->attn_prob) return fail(EII_E_ARG, "trace: attn_score and attn_prob go together");
      HIPCHK(attn_trace(m->qkv, nseq, max_T, m->exp_tab, L.f[QR] + L.f[KR] + 3 - kFScore, tr->attn_score,
                        tr->attn_prob, s));
    }
  }
  const int cb = L.bits[CTX] / 8;
  {
    ProfScope ps(m, EII_K_ATTN, s);
    AttnArgs a{m->qkv, m->vt, m->seq_off, m->exp_tab, tr ? tr->attn_ctx : nullptr, (uint8_t*)m->ctx, M, nseq, max_T,
               m->max_kt, L.f[QR] + L.f[KR] + 3 - kFScore, 16 + L.f[VP] - L.f[CTX], L.bits[CTX]};
    a.kpl = m->kpl;
    if (kv) {   // queries of the new positions against every cached key
      const int len = kv->p0 + kv->T_new;
      a.qkv = kv->kv->qkv[l];
      a.vt = kv->kv->vt[l];
      a.seq_off = kv->kv->seq_off;
      a.M = nseq * kv->kv->cap;
      a.max_T = a.kv_len = len;
      a.max_kt = (len + 31) / 32;
      a.q_first = kv->p0;
      a.out_M = M;
      a.kpl = nullptr;
    }
    HIPCHK(attention(a, s));
  }
  // traces: RS(acc m, n + f_c - 15) before the saturating add, from the exact int64 accumulators
  auto res_update = [&](const Mat& W, const void* planes, int planes_n, int64_t* out, int a_kb) -> int {
    HIPCHK(gemm_i64_anyk((const uint8_t*)planes, planes_n, W.Wf, W.wsum, M, W.N, W.K, out, s, a_kb));
    HIPCHK(requant_i64(out, M, W.N, W.mult, W.shift, 64, out, s));
    return EII_OK;
  };
  int rc;
  if (tr && tr->o_res && (rc = res_update(L.o, m->ctx, cb, tr->o_res, 64))) return rc;
  {
    ProfScope ps(m, EII_K_GEMM_O, s);
    HIPCHK(gemm(gemm_args(L.o, m->ctx, M, x, 32), cb, EPI_RESID, s));
  }
  if (tr && tr->resid_mid) HIPCHK(hipMemcpyAsync(tr->resid_mid, x, (size_t)M * kD * 4, hipMemcpyDeviceToDevice, s));
  const int h2b = L.bits[NORM2] / 8;
  if (!fuse_norm(M, sh_n2, L.bits[NORM2], tr)) {
    ProfScope ps(m, EII_K_NORM, s);
    HIPCHK(rmsnorm(x, M, L.ln2, sh_n2, L.bits[NORM2], h, tr ? tr->norm2_out : nullptr, s, false,
                   tr ? tr->norm2_U : nullptr, tr ? tr->norm2_z : nullptr));
  }
  const int gb = L.bits[GATED] / 8;
  const int sh_s = L.f[SILU] + L.f[UP] - L.f_m;
  {
    ProfScope ps(m, EII_K_GEMM_GU, s);
    if (!tr) {   // gate and up projections with the SiLU table and the gated product in the epilogue
      GemmArgs g = gemm_args(L.gu, h, M, m->gated, 16);
      g.aux_tab = L.silu; g.sh2 = sh_s; g.bits2 = L.bits[GATED]; g.tab_bits = L.bits[SILU];
      if (fuse_norm(M, sh_n2, L.bits[NORM2], tr)) { g.nx = x; g.ngain = L.ln2; g.nsh = sh_n2; }
      HIPCHK(gemm(g, h2b, EPI_SILU, s));
    } else {
      HIPCHK(gemm(gemm_args(L.gu, h, M, m->gu, 16), h2b, EPI_REQ16, s));
    }
  }
  if (tr) {
    // gu holds [gate 32 | up 32] blocks; de-interleave for the dumps
    if (tr->gate_proj)
      HIPCHK(hipMemcpy2DAsync(tr->gate_proj, 64, m->gu, 128, 64, (size_t)M * 48, hipMemcpyDeviceToDevice, s));
    if (tr->up_proj)
      HIPCHK(hipMemcpy2DAsync(tr->up_proj, 64, (const uint8_t*)m->gu + 64, 128, 64, (size_t)M * 48,
                              hipMemcpyDeviceToDevice, s));
    HIPCHK(silu_gate(m->gu, M, L.silu, sh_s, L.bits[GATED], (uint8_t*)m->gated, tr->mlp_gated, s, tr->silu_gate));
    if (tr->down_res && (rc = res_update(L.down, m->gated, gb, tr->down_res, 32))) return rc;
  }
  {
    ProfScope ps(m, EII_K_GEMM_DOWN, s);
    GemmArgs g = gemm_args(L.down, m->gated, M, x, 32);
    g.a_kb = 32;   // the gated planes' 32-byte K blocks
    HIPCHK(gemm(g, gb, EPI_RESID, s));
  }
  return EII_OK;
}

int run_final(eii_model* m, const int32_t* x, int M, int32_t* logits, hipStream_t s) {
  const int sh_n = 21 + m->fg_f - m->f_y;
  const bool fused = fuse_norm(M, sh_n, 16, nullptr);
  if (!fused) {
    ProfScope ps(m, EII_K_NORM, s);
    HIPCHK(rmsnorm(x, M, m->fg, sh_n, 16, (uint8_t*)m->h, nullptr, s));
  }
  GemmArgs g = gemm_args(m->head, m->h, M, logits, 32);
  g.flag = m->flags;
  if (fused) { g.nx = x; g.ngain = m->fg; g.nsh = sh_n; }
  ProfScope ps(m, EII_K_GEMM_HEAD, s);
  HIPCHK(gemm(g, 2, EPI_LOGITS, s));
  return EII_OK;
}

// Row runs of the sequences whose states are dumped: (first row in the batch, first row in the
// dump, rows); all sequences when mask is null.
struct DumpRun {
  size_t src, dst, rows;
};

std::vector<DumpRun> dump_runs(const std::vector<int32_t>& lens, const uint8_t* mask) {
  std::vector<DumpRun> runs;
  size_t src = 0, dst = 0;
  for (size_t i = 0; i < lens.size(); ++i) {
    if (!mask || mask[i]) {
      if (!runs.empty() && runs.back().src + runs.back().rows == src) runs.back().rows += lens[i];
      else runs.push_back({src, dst, (size_t)lens[i]});
      dst += lens[i];
    }
    src += lens[i];
  }
  return runs;
}

int forward_impl(eii_model* m, const int64_t* ids, const std::vector<int32_t>& lens, int32_t* emb_out,
                 int32_t* res_out, int32_t* logits, const uint8_t* dump_mask, hipStream_t s) {
  size_t M = 0;
  int max_T = 0;
  for (int32_t t : lens) {
    if (t <= 0) return fail(EII_E_ARG, "sequence length must be positive");
    M += t;
    max_T = std::max(max_T, (int)t);
  }
  if (M == 0) return EII_OK;
  // every kernel indexes rows in size_t; the bound keeps row counts and tile counts in int
  if (M > ((size_t)1 << 22)) return fail(EII_E_ARG, "more than 4194304 rows in one forward");
  if (max_T > m->rope_rows)
    return fail(EII_E_BOUND, "sequence of " + std::to_string(max_T) + " tokens exceeds the " +
                                 std::to_string(m->rope_rows) + " RoPE rows loaded (eii_model_set_rope)");
  if (max_T > 16384) return fail(EII_E_BOUND, "sequences longer than 16384 tokens are not supported");
  HIPCHK(hipSetDevice(m->device));
  int rc;
  if ((rc = ensure_ws(m, M)) || (rc = set_batch(m, lens, s))) return rc;
  if (m->graphs && !m->prof) {
    // replay the graph of this shape and these buffers, or capture it now (the positions and
    // sequence offsets it reads were uploaded by set_batch above, outside the graph)
    std::vector<uint8_t> mask;
    if (dump_mask) mask.assign(dump_mask, dump_mask + lens.size());
    for (auto& gr : m->fwd_graphs)
      if (gr.lens == lens && gr.ids == ids && gr.emb == emb_out && gr.res == res_out && gr.lg == logits &&
          gr.mask == mask) {
        HIPCHK(hipGraphLaunch(gr.exec, s));
        return EII_OK;
      }
    // capture records without running anything (the legacy default stream cannot be captured, so
    // an internal stream records); the replay below is ordered on the caller's stream
    if (!m->cap_stream) HIPCHK(hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking));
    HIPCHK(hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeThreadLocal));
    m->graphs = false;   // the launches below are recorded, not replayed
    rc = forward_impl(m, ids, lens, emb_out, res_out, logits, dump_mask, m->cap_stream);
    m->graphs = true;
    hipGraph_t graph = nullptr;
    const hipError_t ec = hipStreamEndCapture(m->cap_stream, &graph);
    if (rc) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (ec != hipSuccess) return fail(EII_E_DEVICE, std::string("graph capture: ") + hipGetErrorString(ec));
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) return fail(EII_E_DEVICE, std::string("graph instantiate: ") + hipGetErrorString(ei));
    if (m->fwd_graphs.size() >= 8) {   // a few shapes at a time
      (void)hipGraphExecDestroy(m->fwd_graphs.front().exec);
      m->fwd_graphs.erase(m->fwd_graphs.begin());
    }
    m->fwd_graphs.push_back({lens, ids, emb_out, res_out, logits, mask, exec});
    HIPCHK(hipGraphLaunch(exec, s));
    return EII_OK;
  }
  const int Mi = (int)M;
  const std::vector<DumpRun> runs = dump_runs(lens, dump_mask);
  size_t dump_rows = 0;
  for (const DumpRun& r : runs) dump_rows += r.rows;
  auto dump = [&](int32_t* out) -> hipError_t {   // the selected rows of x, packed
    for (const DumpRun& r : runs) {
      hipError_t e = hipMemcpyAsync(out + r.dst * kD, m->x + r.src * kD, r.rows * kD * 4, hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  };
  {
    ProfScope ps(m, EII_K_EMBED, s);
    HIPCHK(embed(ids, Mi, m->emb_q, m->emb_m, m->emb_sh, m->x, m->flags, s));
  }
  if (emb_out) HIPCHK(dump(emb_out));
  for (int l = 0; l < kNL; ++l) {
    if ((rc = run_block(m, l, m->x, Mi, (int)lens.size(), max_T, nullptr, s))) return rc;
    if (res_out) HIPCHK(dump(res_out + (size_t)l * dump_rows * kD));
  }
  if (logits) return run_final(m, m->x, Mi, logits, s);
  return EII_OK;
}

}  // namespace

extern "C" int eii_model_set_graphs(eii_model* m, int on) {
  if (!m) return fail(EII_E_ARG, "null model");
  if (!on) {
    HIPCHK(hipSetDevice(m->device));
    drop_graphs(m);
  }
  m->graphs = on != 0;
  return EII_OK;
}

extern "C" int eii_forward(eii_model* m, const int64_t* ids, int B, int T, int32_t* emb_out, int32_t* res_out,
                           int32_t* logits, const uint8_t* dump_mask, void* stream) {
  if (!m || !ids || B <= 0 || T <= 0) return fail(EII_E_ARG, "bad forward arguments");
  std::vector<int32_t> lens(B, T);
  return forward_impl(m, ids, lens, emb_out, res_out, logits, dump_mask, (hipStream_t)stream);
}

extern "C" int eii_forward_packed(eii_model* m, const int64_t* ids, const int32_t* seq_lens, int nseq,
                                  int32_t* emb_out, int32_t* res_out, int32_t* logits, const uint8_t* dump_mask,
                                  void* stream) {
  if (!m || !ids || !seq_lens || nseq <= 0) return fail(EII_E_ARG, "bad forward arguments");
  std::vector<int32_t> lens(seq_lens, seq_lens + nseq);
  return forward_impl(m, ids, lens, emb_out, res_out, logits, dump_mask, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------ decoding
extern "C" int eii_kv_create(eii_model* m, int B, int max_T, eii_kv** out) {
  if (!m || !out || B <= 0 || max_T <= 0) return fail(EII_E_ARG, "bad kv cache arguments");
  *out = nullptr;
  if (max_T > 16384) return fail(EII_E_BOUND, "sequences longer than 16384 tokens are not supported");
  const int cap = (max_T + 31) / 32 * 32;
  if ((size_t)B * cap > ((size_t)1 << 22)) return fail(EII_E_ARG, "more than 4194304 cached positions");
  HIPCHK(hipSetDevice(m->device));
  auto al256 = [](size_t n) { return (n + 255) & ~(size_t)255; };
  const size_t rows = (size_t)B * cap, qb = al256(rows * kQKVN * 2), vb = al256(vt_bytes((int)rows));
  eii_kv* kv = new eii_kv;
  kv->device = m->device;
  kv->B = B;
  kv->cap = cap;
  if (hipMalloc(&kv->dev, kNL * (qb + vb) + al256((size_t)(B + 1) * 4)) != hipSuccess) {
    delete kv;
    return fail(EII_E_DEVICE, "kv cache allocation failed");
  }
  for (int l = 0; l < kNL; ++l) {
    kv->qkv[l] = (int16_t*)(kv->dev + l * (qb + vb));
    kv->vt[l] = kv->dev + l * (qb + vb) + qb;
  }
  kv->seq_off = (int32_t*)(kv->dev + kNL * (qb + vb));
  std::vector<int32_t> off(B + 1);
  for (int b = 0; b <= B; ++b) off[b] = b * cap;
  if (hipMemcpy(kv->seq_off, off.data(), off.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(kv->dev);
    delete kv;
    return fail(EII_E_DEVICE, "kv cache upload failed");
  }
  *out = kv;
  return EII_OK;
}

extern "C" void eii_kv_free(eii_kv* kv) {
  if (!kv) return;
  (void)hipSetDevice(kv->device);
  (void)hipFree(kv->dev);
  delete kv;
}

extern "C" int eii_kv_length(const eii_kv* kv) { return kv ? kv->len : 0; }

extern "C" int eii_kv_reset(eii_kv* kv) {
  if (!kv) return fail(EII_E_ARG, "null kv cache");
  kv->len = 0;
  kv->vt_len = 0;
  return EII_OK;
}

extern "C" int eii_kv_append(eii_model* m, eii_kv* kv, const int64_t* ids, int T_new, int32_t* logits, void* stream) {
  if (!m || !kv || !ids || T_new <= 0) return fail(EII_E_ARG, "bad kv append arguments");
  if (kv->device != m->device) return fail(EII_E_ARG, "kv cache and model on different devices");
  const int p0 = kv->len, len = p0 + T_new;
  if (len > kv->cap)
    return fail(EII_E_BOUND, "the kv cache holds " + std::to_string(kv->cap) + " positions per sequence");
  if (len > m->rope_rows)
    return fail(EII_E_BOUND, "position " + std::to_string(len - 1) + " beyond the " + std::to_string(m->rope_rows) +
                                 " RoPE rows loaded (eii_model_set_rope)");
  const size_t M = (size_t)kv->B * T_new;
  if (M > ((size_t)1 << 22)) return fail(EII_E_ARG, "more than 4194304 rows in one append");
  HIPCHK(hipSetDevice(m->device));
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if ((rc = ensure_ws(m, M))) return rc;
  HIPCHK(fill_positions(m->pos, kv->B, T_new, p0, s));
  m->last_lens.clear();   // the positions no longer belong to the last plain batch
  {
    ProfScope ps(m, EII_K_EMBED, s);
    HIPCHK(embed(ids, (int)M, m->emb_q, m->emb_m, m->emb_sh, m->x, m->flags, s));
  }
  // the one-query decoding kernel (a single new position, at most kDecodeMaxKeys cached) reads
  // the cache rows only; every other step takes the tiled kernel, which reads the V^T planes
  const bool vt = !(T_new == 1 && len <= kDecodeMaxKeys);
  const KvStep step{kv, T_new, p0, vt};
  for (int l = 0; l < kNL; ++l)
    if ((rc = run_block(m, l, m->x, (int)M, kv->B, len, nullptr, s, &step))) return rc;
  kv->len = len;
  if (vt) kv->vt_len = len;
  if (logits) return run_final(m, m->x, (int)M, logits, s);
  return EII_OK;
}

extern "C" int eii_argmax(const int32_t* logits, int rows, int n, int64_t* out, void* stream) {
  if (!logits || !out || rows <= 0 || n <= 0) return fail(EII_E_ARG, "bad argmax arguments");
  HIPCHK(argmax_rows(logits, rows, n, out, (hipStream_t)stream));
  return EII_OK;
}

extern "C" int eii_profile_begin(eii_model* m, int max_launches) {
  if (!m || max_launches <= 0) return fail(EII_E_ARG, "bad profile arguments");
  HIPCHK(hipSetDevice(m->device));
  const size_t need = 2 * (size_t)max_launches;
  while (m->ev.size() < need) {
    hipEvent_t e;
    HIPCHK(hipEventCreate(&e));
    m->ev.push_back(e);
  }
  m->ev_kind.assign(m->ev.size() / 2, -1);
  m->ev_used = 0;
  m->prof = true;
  return EII_OK;
}

extern "C" int eii_profile_end(eii_model* m, void* stream, double* ms, int* launches) {
  if (!m || !ms || !launches) return fail(EII_E_ARG, "bad profile arguments");
  m->prof = false;
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  for (int k = 0; k < EII_K_COUNT; ++k) { ms[k] = 0.0; launches[k] = 0; }
  for (size_t i = 0; i < m->ev_used; i += 2) {
    float t = 0.f;
    HIPCHK(hipEventElapsedTime(&t, m->ev[i], m->ev[i + 1]));
    const int k = m->ev_kind[i / 2];
    if (k >= 0 && k < EII_K_COUNT) { ms[k] += t; launches[k] += 1; }
  }
  const int dropped = m->ev_used >= m->ev.size() ? 1 : 0;
  m->ev_used = 0;
  return dropped ? fail(EII_E_ARG, "profile buffer full: raise max_launches") : EII_OK;
}

extern "C" int eii_check(eii_model* m, void* stream) {
  if (!m) return fail(EII_E_ARG, "null model");
  HIPCHK(hipSetDevice(m->device));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  int f = 0;
  HIPCHK(hipMemcpy(&f, m->flags, 4, hipMemcpyDeviceToHost));
  HIPCHK(hipMemset(m->flags, 0, 4));
  if (f & 2) return fail(EII_E_BOUND, "token id outside [0, 49152)");
  if (f & 1) return fail(EII_E_BOUND, "a logit left the int32 range");
  return EII_OK;
}

extern "C" int eii_block(eii_model* m, int layer, int32_t* x, int B, int T, const eii_trace* tr, void* stream) {
  if (!m || !x || layer < 0 || layer >= kNL || B <= 0 || T <= 0) return fail(EII_E_ARG, "bad block arguments");
  if (T > m->rope_rows) return fail(EII_E_BOUND, "T exceeds the RoPE rows loaded");
  if (T > 16384) return fail(EII_E_BOUND, "sequences longer than 16384 tokens are not supported");
  HIPCHK(hipSetDevice(m->device));
  hipStream_t s = (hipStream_t)stream;
  std::vector<int32_t> lens(B, T);
  int rc;
  if ((rc = ensure_ws(m, (size_t)B * T)) || (rc = set_batch(m, lens, s))) return rc;
  return run_block(m, layer, x, B * T, B, T, tr, s);
}

extern "C" int eii_embed(eii_model* m, const int64_t* ids, int M, int32_t* x, void* stream) {
  if (!m || !ids || !x || M <= 0) return fail(EII_E_ARG, "bad embed arguments");
  HIPCHK(hipSetDevice(m->device));
  HIPCHK(embed(ids, M, m->emb_q, m->emb_m, m->emb_sh, x, m->flags, (hipStream_t)stream));
  return EII_OK;
}

extern "C" int eii_final(eii_model* m, const int32_t* x, int M, int32_t* logits, void* stream) {
  if (!m || !x || !logits || M <= 0) return fail(EII_E_ARG, "bad final arguments");
  HIPCHK(hipSetDevice(m->device));
  int rc;
  if ((rc = ensure_ws(m, M))) return rc;
  return run_final(m, x, M, logits, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------ operators
extern "C" int eii_weight_colsum(const int8_t* W, int N, int K, int32_t* wsum, void* stream) {
  if (!W || !wsum || N <= 0 || K <= 0) return fail(EII_E_ARG, "bad colsum arguments");
  HIPCHK(weight_colsum(W, N, K, wsum, (hipStream_t)stream));
  return EII_OK;
}

// K is zero-padded to a multiple of 64 for the GEMM (zero weight columns add nothing); every limb
// partial sum stays inside int32 while 128 * 127 * K < 2^31
constexpr int kMaxGemmK = 131072;
static int check_gemm_args(const void* A, int a_bits, const int8_t* W, int M, int N, int K) {
  if (!A || !W || M <= 0 || N <= 0 || K <= 0) return fail(EII_E_ARG, "bad gemm arguments");
  if (a_bits != 8 && a_bits != 16 && a_bits != 32) return fail(EII_E_ARG, "a_bits must be 8, 16 or 32");
  if (K > kMaxGemmK) return fail(EII_E_BOUND, "K above 131072 could overflow a limb partial sum");
  if ((size_t)M * padded_k(K) > ((size_t)1 << 31)) return fail(EII_E_ARG, "M * K above 2^31");
  return EII_OK;
}
// limb planes of an a_bits activation: 8- and 16-bit values travel as 2 planes, 32-bit as 4
static int limb_planes(int a_bits) { return a_bits == 32 ? 4 : 2; }

// Staging memory of the operator entry points (A split into K-blocked limb planes, W in fragment
// order, column sums, requantization coefficients, V^T planes): one block per device, kept for
// the life of the process and grown on demand, so calls at a size seen before allocate nothing.
// Calls on one device take the block in turn: a call holds the host lock while it enqueues its
// work, makes its stream wait for the event the previous call recorded (which may have been on
// another stream) and records its own when it is done.  Growing frees the old block with
// hipFree, which waits for the device to finish with it.
constexpr int kMaxDevices = 64;
struct StagingBlock {
  uint8_t* p = nullptr;
  size_t bytes = 0;
  hipEvent_t done = nullptr;
};
static std::mutex g_staging_mu;
static StagingBlock g_staging[kMaxDevices];

class Staging {
 public:
  Staging() : lk_(g_staging_mu) {}
  ~Staging() {
    if (blk_) (void)hipEventRecord(blk_->done, s_);
  }
  // The device's block, at least `bytes` long, for work enqueued on stream s.
  int take(size_t bytes, hipStream_t s) {
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(EII_E_DEVICE, "device ordinal out of range");
    StagingBlock& b = g_staging[dev];
    if (!b.done) HIPCHK(hipEventCreateWithFlags(&b.done, hipEventDisableTiming));
    else HIPCHK(hipStreamWaitEvent(s, b.done, 0));
    if (b.bytes < bytes) {
      if (b.p) HIPCHK(hipFree(b.p));
      b.p = nullptr;
      b.bytes = 0;
      HIPCHK(hipMalloc((void**)&b.p, bytes));
      b.bytes = bytes;
    }
    blk_ = &b;
    s_ = s;
    used_ = 0;
    return EII_OK;
  }
  // Consecutive 256-byte aligned pieces of the block, in the order of the sizes given to take().
  template <class T>
  T* carve(size_t bytes) {
    T* q = (T*)(blk_->p + used_);
    used_ += align(bytes);
    return q;
  }
  static size_t align(size_t bytes) { return (bytes + 255) & ~(size_t)255; }

 private:
  std::unique_lock<std::mutex> lk_;
  StagingBlock* blk_ = nullptr;
  hipStream_t s_ = nullptr;
  size_t used_ = 0;
};

static size_t operand_bytes(int a_bits, int M, int N, int K) {
  const int Kp = padded_k(K);
  return Staging::align((size_t)M * Kp * limb_planes(a_bits)) + Staging::align(swizzled_bytes(N, Kp));
}

// A [M, K] -> K-blocked limb planes, row-major W [N, K] -> fragment order, both over K padded to a
// multiple of 64, at the given device addresses (planes then wf)
static int stage_operands_at(const void* A, int a_bits, const int8_t* W, int M, int N, int K, uint8_t* planes,
                             int8_t* wf, hipStream_t s) {
  hipError_t e = split_limbs(A, a_bits / 8, M, K, planes, s);
  if (e == hipSuccess) e = swizzle_weights(W, N, K, wf, s, padded_k(K));
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("operand staging: ") + hipGetErrorString(e));
  return EII_OK;
}

static int stage_operands(const void* A, int a_bits, const int8_t* W, int M, int N, int K, Staging& st,
                          uint8_t*& planes, int8_t*& wf, hipStream_t s) {
  planes = st.carve<uint8_t>((size_t)M * padded_k(K) * limb_planes(a_bits));
  wf = st.carve<int8_t>(swizzled_bytes(N, padded_k(K)));
  return stage_operands_at(A, a_bits, W, M, N, K, planes, wf, s);
}

static int gemm_i8_staged(const void* A, int a_bits, const int8_t* W, const int32_t* wsum, int M, int N, int K,
                          int64_t* acc, Staging& st, hipStream_t s) {
  uint8_t* planes;
  int8_t* wf;
  int rc;
  if ((rc = stage_operands(A, a_bits, W, M, N, K, st, planes, wf, s))) return rc;
  const hipError_t e = gemm_i64_anyk(planes, limb_planes(a_bits), wf, wsum, M, N, padded_k(K), acc, s);
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("eii_gemm_i8: ") + hipGetErrorString(e));
  return EII_OK;
}

extern "C" int eii_gemm_i8_ws(const void* A, int a_bits, const int8_t* W, const int32_t* wsum, int M, int N, int K,
                              int64_t* acc, void* stream) {
  int rc;
  if ((rc = check_gemm_args(A, a_bits, W, M, N, K))) return rc;
  if (!wsum || !acc) return fail(EII_E_ARG, "null output");
  if (N % 4) return fail(EII_E_ARG, "N must be a multiple of 4");
  hipStream_t s = (hipStream_t)stream;
  Staging st;
  if ((rc = st.take(operand_bytes(a_bits, M, N, K), s))) return rc;
  return gemm_i8_staged(A, a_bits, W, wsum, M, N, K, acc, st, s);
}

extern "C" int eii_gemm_i8(const void* A, int a_bits, const int8_t* W, int M, int N, int K, int64_t* acc,
                           void* stream) {
  int rc;
  if ((rc = check_gemm_args(A, a_bits, W, M, N, K))) return rc;
  if (!acc) return fail(EII_E_ARG, "null output");
  if (N % 4) return fail(EII_E_ARG, "N must be a multiple of 4");
  hipStream_t s = (hipStream_t)stream;
  Staging st;
  if ((rc = st.take(operand_bytes(a_bits, M, N, K) + Staging::align((size_t)N * 4), s))) return rc;
  int32_t* ws = st.carve<int32_t>((size_t)N * 4);
  hipError_t e = weight_colsum(W, N, K, ws, s);
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("eii_gemm_i8: ") + hipGetErrorString(e));
  return gemm_i8_staged(A, a_bits, W, ws, M, N, K, acc, st, s);
}

// ---- allocation-free exact matmul
// Staging for eii_gemm_i8_ws_noalloc: a file-scope device array, one copy per GPU the library runs
// on, held until the process ends.  In host code `scratch` names a host-side stand-in, not device
// memory: its device address on the current GPU comes from hipGetSymbolAddress, once per device, and
// only that address is handed to kernels.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_dev[kMaxDevices];

static int scratch_on_current_device(uint8_t** out) {
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(EII_E_DEVICE, "device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(EII_E_DEVICE, std::string("scratch address: ") + hipGetErrorString(e));
    g_scratch_dev[dev] = (uint8_t*)p;
  }
  *out = g_scratch_dev[dev];
  return EII_OK;
}

extern "C" int eii_gemm_i8_ws_noalloc(const void* A, int a_bits, const int8_t* W, const int32_t* wsum, int M, int N,
                                      int K, int64_t* acc, void* stream) {
  int rc;
  if ((rc = check_gemm_args(A, a_bits, W, M, N, K))) return rc;
  if (!wsum || !acc) return fail(EII_E_ARG, "null output");
  if (N % 4) return fail(EII_E_ARG, "N must be a multiple of 4");
  const int Kp = padded_k(K);
  const size_t plane_bytes = Staging::align((size_t)M * Kp * limb_planes(a_bits));
  if (plane_bytes + swizzled_bytes(N, Kp) > kScratchBytes)
    return fail(EII_E_BOUND, "operands need " + std::to_string(plane_bytes + swizzled_bytes(N, Kp)) +
                                 " bytes of staging, above the 64 MiB scratch of the allocation-free entry point");
  uint8_t* base = nullptr;
  if ((rc = scratch_on_current_device(&base))) return rc;
  hipStream_t s = (hipStream_t)stream;
  // every byte the GEMM reads is written here first (planes over all of K padded, weights over every
  // 32-row block): nothing in the scratch needs clearing
  uint8_t* planes = base;
  int8_t* wf = (int8_t*)(base + plane_bytes);
  if ((rc = stage_operands_at(A, a_bits, W, M, N, K, planes, wf, s))) return rc;
  const hipError_t e = gemm_i64_anyk(planes, limb_planes(a_bits), wf, wsum, M, N, Kp, acc, s);
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("eii_gemm_i8_ws_noalloc: ") + hipGetErrorString(e));
  return EII_OK;
}

// The requantization runs on the exact int64 accumulators, in int64 as python/intref.py:189 does,
// so any int32 multiplier and shift behave as there (the reference asserts |acc| max m < 2^63).
extern "C" int eii_linear(const void* A, int a_bits, const int8_t* W, const int32_t* wsum, const int32_t* mult,
                          const int32_t* shift, int M, int N, int K, int out_bits, void* out, void* stream) {
  int rc;
  if ((rc = check_gemm_args(A, a_bits, W, M, N, K))) return rc;
  if (!wsum || !mult || !shift || !out) return fail(EII_E_ARG, "null argument");
  if (out_bits != 16 && out_bits != 32) return fail(EII_E_ARG, "out_bits must be 16 or 32");
  if (N % 4) return fail(EII_E_ARG, "N must be a multiple of 4");
  hipStream_t s = (hipStream_t)stream;
  Staging st;
  const size_t acc_bytes = (size_t)M * N * 8;
  if ((rc = st.take(operand_bytes(a_bits, M, N, K) + Staging::align(acc_bytes), s))) return rc;
  int64_t* acc = st.carve<int64_t>(acc_bytes);
  if ((rc = gemm_i8_staged(A, a_bits, W, wsum, M, N, K, acc, st, s))) return rc;
  const hipError_t e = requant_i64(acc, M, N, mult, shift, out_bits, out, s);
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("eii_linear: ") + hipGetErrorString(e));
  return EII_OK;
}

extern "C" int eii_rope(int16_t* qkv, const int32_t* seq_off, int nseq, const int32_t* cosT, const int32_t* sinT,
                        int rows, int f_q, int f_qr, int bits_qr, int f_k, int f_kr, int bits_kr, void* stream) {
  if (!qkv || !seq_off || !cosT || !sinT || nseq <= 0 || rows <= 0) return fail(EII_E_ARG, "bad rope arguments");
  if (bits_qr < 2 || bits_qr > 16 || bits_kr < 2 || bits_kr > 16)
    return fail(EII_E_ARG, "rope outputs are int16: bits must be 2..16");
  // |a1 c - a2 s| <= 2^46: a left shift of up to 16 stays inside int64
  const int sh_q = 30 + f_q - f_qr, sh_k = 30 + f_k - f_kr;
  if (sh_q < -16 || sh_q > 62 || sh_k < -16 || sh_k > 62) return fail(EII_E_BOUND, "rope shift out of range");
  hipStream_t s = (hipStream_t)stream;
  // positions restart at 0 in every sequence (python/intref.py:213): built on the host from the offsets
  std::vector<int32_t> off(nseq + 1);
  HIPCHK(hipMemcpyAsync(off.data(), seq_off, off.size() * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  std::vector<int32_t> pos;
  for (int i = 0; i < nseq; ++i) {
    const int T = off[i + 1] - off[i];
    if (off[i] < 0 || T <= 0) return fail(EII_E_ARG, "seq_off must increase by at least 1 per sequence");
    if (T > rows) return fail(EII_E_BOUND, "a sequence is longer than the RoPE rows given");
    if (off[i] != (int)pos.size()) return fail(EII_E_ARG, "seq_off must start at 0 and be contiguous");
    for (int t = 0; t < T; ++t) pos.push_back(t);
  }
  const int M = (int)pos.size();
  Staging st;
  int rc;
  if ((rc = st.take((size_t)M * 4, s))) return rc;
  int32_t* pos_dev = st.carve<int32_t>((size_t)M * 4);
  HIPCHK(hipMemcpyAsync(pos_dev, pos.data(), (size_t)M * 4, hipMemcpyHostToDevice, s));
  HIPCHK(rope(qkv, M, pos_dev, cosT, sinT, sh_q, bits_qr, sh_k, bits_kr, s));
  HIPCHK(hipStreamSynchronize(s));   // the host positions die at return
  return EII_OK;
}

extern "C" int eii_silu_gate(const int16_t* gate, const int16_t* up, int M, const int32_t* silu, int f_s, int f_u,
                             int f_m, int bits_m, void* out, void* stream) {
  if (!gate || !up || !silu || !out || M <= 0) return fail(EII_E_ARG, "bad silu gate arguments");
  if (bits_m != 16 && bits_m != 32) return fail(EII_E_ARG, "bits_m must be 16 or 32");
  // |silu u| < 2^46: a left shift of up to 16 stays inside int64
  const int sh = f_s + f_u - f_m;
  if (sh < -16 || sh > 62) return fail(EII_E_BOUND, "silu gate shift out of range");
  hipStream_t s = (hipStream_t)stream;
  Staging st;
  int rc;
  const size_t gu_bytes = (size_t)M * 2 * kDFF * 2;
  if ((rc = st.take(gu_bytes, s))) return rc;
  // the kernel reads rows of [gate 32 | up 32] blocks (the fused gate/up projection's layout)
  int16_t* gu = st.carve<int16_t>(gu_bytes);
  HIPCHK(hipMemcpy2DAsync(gu, 128, gate, 64, 64, (size_t)M * (kDFF / 32), hipMemcpyDeviceToDevice, s));
  HIPCHK(hipMemcpy2DAsync((uint8_t*)gu + 64, 128, up, 64, 64, (size_t)M * (kDFF / 32), hipMemcpyDeviceToDevice, s));
  HIPCHK(silu_gate(gu, M, silu, sh, bits_m, nullptr, out, s));
  return EII_OK;
}

extern "C" int eii_rmsnorm(const int32_t* x, int M, const int32_t* gain, int f_gain, int f_out, int out_bits,
                           void* out, void* stream) {
  if (!x || !gain || !out || M <= 0) return fail(EII_E_ARG, "bad rmsnorm arguments");
  // the kernel moves 4 columns per access
  if (((uintptr_t)x | (uintptr_t)gain | (uintptr_t)out) & 15) return fail(EII_E_ARG, "x, gain and out must be 16-byte aligned");
  if (out_bits != 16 && out_bits != 32) return fail(EII_E_ARG, "out_bits must be 16 or 32");
  int rc;
  if ((rc = check_scalar_shift(21 + f_gain - f_out, "norm"))) return rc;
  // gains anywhere in int32: the general int64 path
  HIPCHK(rmsnorm(x, M, gain, 21 + f_gain - f_out, out_bits, nullptr, out, (hipStream_t)stream, true));
  return EII_OK;
}

extern "C" int eii_attention(const int16_t* qkv, const int32_t* seq_off, int nseq, int max_T, const int32_t* exp_tab,
                             int f_qr, int f_kr, int f_v, int f_c, int bits_c, void* ctx, void* stream) {
  if (!qkv || !seq_off || !exp_tab || !ctx || nseq <= 0 || max_T <= 0) return fail(EII_E_ARG, "bad attention arguments");
  if (bits_c != 16 && bits_c != 32) return fail(EII_E_ARG, "bits_c must be 16 or 32");
  const int shift_s = f_qr + f_kr + 3 - kFScore;
  if (shift_s < 1) return fail(EII_E_BOUND, "score shift < 1");
  if (shift_s > 30) return fail(EII_E_BOUND, "score shift > 30");
  int rc = check_scalar_shift(16 + f_v - f_c, "context");
  if (rc) return rc;
  if (max_T > 16384) return fail(EII_E_BOUND, "sequences longer than 16384 tokens are not supported");
  hipStream_t s = (hipStream_t)stream;
  // the row offsets decide the launch shape: read them back
  std::vector<int32_t> off(nseq + 1);
  HIPCHK(hipMemcpyAsync(off.data(), seq_off, off.size() * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  int max_kt = 0;
  for (int i = 0; i < nseq; ++i) {
    const int T = off[i + 1] - off[i];
    if (off[i] < 0 || T <= 0 || T > max_T) return fail(EII_E_ARG, "seq_off must increase by 1..max_T per sequence");
    max_kt = std::max(max_kt, attn_key_tiles(off[i], T));
  }
  const int M = off[nseq];
  Staging st;
  if ((rc = st.take(Staging::align(vt_bytes(M)) + attn_kpl_bytes(M), s))) return rc;
  uint8_t* vt = st.carve<uint8_t>(vt_bytes(M));
  AttnArgs a{qkv, vt, seq_off, exp_tab, ctx, nullptr, M, nseq, max_T, max_kt, shift_s, 16 + f_v - f_c, bits_c};
  a.kpl = st.carve<uint8_t>(attn_kpl_bytes(M));
  hipError_t e = build_vt(qkv, M, vt, s);
  if (e == hipSuccess) e = attention(a, s);
  if (e != hipSuccess) return fail(EII_E_DEVICE, std::string("eii_attention: ") + hipGetErrorString(e));
  return EII_OK;
}
