// eii_check VECTORDIR [MODELDIR]: the conformance checker of the integer forward on an MI355X.
//
// Same command line, files, stdout grammar and exit codes as the reference checkers
// (c/intref.c:214-257, cuda/intref.cu:252-305): reads MODELDIR/model.bin (MODELDIR defaults to
// VECTORDIR) and VECTORDIR/ids.i64, exp_embed.i32, exp_resid_out.i32, exp_logits.i32, runs the
// forward through libeii and prints, per state,
//     "  MISMATCH <name> <bad> of <n>, first at <i> (got <g> expected <e>)"
//     "layer %2d: exact|DIFFERS"      (stopping at the first differing layer)
//     "logits: exact|DIFFERS"
// and finally "ALL STATES EXACT (<T> tokens, <s> s on device incl. comparisons)" or "FAIL (...)".
// Exit 0: every state exact, 1: a mismatch, 2: usage or file error, 3: device error.
//
// Sequences longer than the 512 RoPE rows of model.bin need MODELDIR/rope.i64: cos then sin,
// int64 [rows, 32] each (the closed form of python/intref.py:96-108), as eii.export_vectors
// writes it.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "eii.h"

namespace {

bool read_file(const std::string& path, std::vector<char>& out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  fseek(f, 0, SEEK_END);
  const long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  out.resize(n > 0 ? (size_t)n : 0);
  const bool ok = n >= 0 && fread(out.data(), 1, out.size(), f) == out.size();
  fclose(f);
  return ok;
}

template <class T>
bool read_array(const std::string& path, size_t count, std::vector<T>& out) {
  std::vector<char> raw;
  if (!read_file(path, raw) || raw.size() != count * sizeof(T)) {
    fprintf(stderr, "%s: missing or not %zu bytes\n", path.c_str(), count * sizeof(T));
    return false;
  }
  out.resize(count);
  memcpy(out.data(), raw.data(), raw.size());
  return true;
}

size_t compare(const char* name, const int32_t* got, const int32_t* exp, size_t n) {
  size_t bad = 0, first = 0;
  for (size_t i = 0; i < n; ++i)
    if (got[i] != exp[i]) {
      if (!bad) first = i;
      ++bad;
    }
  if (bad)
    printf("  MISMATCH %-10s %zu of %zu, first at %zu (got %d expected %d)\n", name, bad, n, first, got[first],
           exp[first]);
  return bad;
}

int device_fail(const char* what) {
  fprintf(stderr, "%s: %s\n", what, eii_last_error());
  return 3;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: eii_check VECTORDIR [MODELDIR]\n");
    return 2;
  }
  const std::string vdir = argv[1], mdir = argc > 2 ? argv[2] : argv[1];
  const size_t D = 576, V = 49152, NL = 30;

  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    fprintf(stderr, "no GPU device\n");
    return 2;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 3;
  printf("device: %s (%s, %.1f GiB)\n", prop.name, prop.gcnArchName, prop.totalGlobalMem / 1073741824.0);

  std::vector<char> idraw;
  if (!read_file(vdir + "/ids.i64", idraw) || idraw.empty() || idraw.size() % 8) {
    fprintf(stderr, "%s/ids.i64: missing or empty\n", vdir.c_str());
    return 2;
  }
  const size_t T = idraw.size() / 8, TD = T * D;
  std::vector<int32_t> exp_embed, exp_res, exp_log;
  if (!read_array(vdir + "/exp_embed.i32", TD, exp_embed) || !read_array(vdir + "/exp_resid_out.i32", NL * TD, exp_res) ||
      !read_array(vdir + "/exp_logits.i32", T * V, exp_log))
    return 2;

  eii_model* m = nullptr;
  int rc = eii_model_load((mdir + "/model.bin").c_str(), 0, &m);
  if (rc != EII_OK) {
    fprintf(stderr, "model.bin: %s\n", eii_last_error());
    return rc == EII_E_DEVICE ? 3 : 2;
  }
  if (T > (size_t)eii_model_rope_rows(m)) {
    std::vector<char> rope;
    if (!read_file(mdir + "/rope.i64", rope) || rope.size() % (2 * 32 * 8) || rope.size() / (2 * 32 * 8) < T) {
      fprintf(stderr, "T = %zu > %d RoPE rows and no %s/rope.i64 covering it\n", T, eii_model_rope_rows(m), mdir.c_str());
      eii_model_free(m);
      return 2;
    }
    const int rows = (int)(rope.size() / (2 * 32 * 8));
    const int64_t* c = (const int64_t*)rope.data();
    if ((rc = eii_model_set_rope(m, c, c + (size_t)rows * 32, rows)) != EII_OK) {
      fprintf(stderr, "rope.i64: %s\n", eii_last_error());
      eii_model_free(m);
      return rc == EII_E_DEVICE ? 3 : 2;
    }
  }

  const auto t0 = std::chrono::steady_clock::now();
  int64_t* ids = nullptr;
  int32_t *emb = nullptr, *res = nullptr, *lg = nullptr;
  if (hipMalloc(&ids, T * 8) != hipSuccess || hipMalloc(&emb, TD * 4) != hipSuccess ||
      hipMalloc(&res, NL * TD * 4) != hipSuccess || hipMalloc(&lg, T * V * 4) != hipSuccess ||
      hipMemcpy(ids, idraw.data(), T * 8, hipMemcpyHostToDevice) != hipSuccess)
    return device_fail("device buffers");
  if ((rc = eii_forward(m, ids, 1, (int)T, emb, res, lg, nullptr, nullptr)) != EII_OK) {
    fprintf(stderr, "forward: %s\n", eii_last_error());
    return rc == EII_E_DEVICE ? 3 : 2;
  }
  rc = eii_check(m, nullptr);
  if (rc == EII_E_DEVICE) return device_fail("forward");
  if (rc != EII_OK) printf("  %s\n", eii_last_error());   // a token id or a logit out of range

  std::vector<int32_t> h_emb(TD), h_res(NL * TD), h_lg(T * V);
  if (hipMemcpy(h_emb.data(), emb, TD * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(h_res.data(), res, NL * TD * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(h_lg.data(), lg, T * V * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return device_fail("copy back");

  size_t total_bad = rc == EII_OK ? 0 : 1;
  total_bad += compare("embed", h_emb.data(), exp_embed.data(), TD);
  for (size_t l = 0; l < NL && !total_bad; ++l) {
    const size_t bad = compare("resid_out", h_res.data() + l * TD, exp_res.data() + l * TD, TD);
    printf("layer %2zu: %s\n", l, bad ? "DIFFERS" : "exact");
    total_bad += bad;
  }
  if (!total_bad) {
    total_bad += compare("logits", h_lg.data(), exp_log.data(), T * V);
    printf("logits: %s\n", total_bad ? "DIFFERS" : "exact");
  }
  const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  printf("%s (%zu tokens, %.2f s on device incl. comparisons)\n", total_bad ? "FAIL" : "ALL STATES EXACT", T, s);
  (void)hipFree(ids); (void)hipFree(emb); (void)hipFree(res); (void)hipFree(lg);
  eii_model_free(m);
  return total_bad ? 1 : 0;
}
