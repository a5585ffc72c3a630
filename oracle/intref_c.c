/* ORACLE (test infrastructure only): integer-only C restatement of python/intref.py.
 *
 *   intref_c VECTORDIR [MODELDIR]
 *
 * Reads MODELDIR/model.bin (layout of python/export_vectors.py:24-45; MODELDIR defaults to
 * VECTORDIR), VECTORDIR/ids.i64 and, for sequences longer than the 512 RoPE rows of
 * model.bin, MODELDIR/rope.i64 (cos then sin, int64 [rows, 32]).  When VECTORDIR holds the
 * expected states (exp_embed.i32, exp_resid_out.i32, exp_logits.i32) it checks them and prints
 * the reference checkers' grammar (c/intref.c:207-257): "layer %2d: exact|DIFFERS",
 * "logits: exact|DIFFERS", "ALL STATES EXACT (...)" or "FAIL (...)", exit 0 / 1 / 2.  Without
 * them it computes and writes those three files.
 *
 * Every step follows python/intref.py in 64- and 128-bit integers (no floating point at all):
 * products accumulate in int64 (|a w| sums stay below 2^53 by the reference's own asserts), the
 * RMSNorm sum of squares in 128 bits with an integer square root, the softmax division as an
 * integer division.  Rows (tokens) are independent everywhere except in attention, which runs
 * per head and query; OpenMP spreads both over the host's cores.  Only tests/ and bench.py's CPU
 * baseline run it, to check the GPU engine's states; the engine never does.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;
typedef __int128 i128;
typedef unsigned __int128 u128;

#define V 49152
#define D 576
#define DFF 1536
#define NL 30
#define NH 9
#define NKV 3
#define HD 64
#define DMAX 1536
#define ROPE_FILE_ROWS 512
#define F_RES 15                 /* python/intref.py:33 */
#define EPS_S 6184753            /* python/intref.py:37 */

/* ---------------------------------------------------------------- semantics (intref.py:42-55) */
static inline i64 rs(i64 x, int n) { return n <= 0 ? x * ((i64)1 << -n) : (x + ((i64)1 << (n - 1))) >> n; }
static inline i64 sat(i64 x, int bits) {
    if (bits >= 64) return x;
    const i64 hi = ((i64)1 << (bits - 1)) - 1, lo = -hi - 1;
    return x < lo ? lo : (x > hi ? hi : x);
}

/* ---------------------------------------------------------------- model */
typedef struct { int8_t *q; i64 *m, *n; int N, K; } Mat;
typedef struct {
    i64 fm[24];
    i64 ln1[D], ln2[D], ln1f, ln2f;
    Mat w[7];          /* q k v o gate up down */
    i64 *silu;         /* [65536] */
} Layer;

static int8_t *emb_q;
static i64 *emb_m, *emb_n, fg[D], fg_f, f_y, exp_tab[DMAX + 1], *rope_cos, *rope_sin;
static int rope_rows;
static Layer L[NL];

static void *must_read(FILE *f, size_t bytes, const char *what) {
    void *p = malloc(bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) { fprintf(stderr, "short read: %s\n", what); exit(2); }
    return p;
}
static void read_into(FILE *f, void *dst, size_t bytes, const char *what) {
    if (fread(dst, 1, bytes, f) != bytes) { fprintf(stderr, "short read: %s\n", what); exit(2); }
}

static void load_model(const char *dir) {
    static const int NN[7] = {576, 192, 192, 576, 1536, 1536, 576}, KK[7] = {576, 576, 576, 576, 576, 576, 1536};
    char path[4096];
    snprintf(path, sizeof path, "%s/model.bin", dir);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "%s: cannot open\n", path); exit(2); }
    emb_q = must_read(f, (size_t)V * D, "emb_q");
    emb_m = must_read(f, (size_t)V * 8, "emb_m");
    emb_n = must_read(f, (size_t)V * 8, "emb_n");
    read_into(f, fg, sizeof fg, "final gain");
    read_into(f, &fg_f, 8, "final gain f");
    read_into(f, &f_y, 8, "f_y");
    read_into(f, exp_tab, sizeof exp_tab, "exp table");
    rope_rows = ROPE_FILE_ROWS;
    rope_cos = must_read(f, (size_t)ROPE_FILE_ROWS * 32 * 8, "rope cos");
    rope_sin = must_read(f, (size_t)ROPE_FILE_ROWS * 32 * 8, "rope sin");
    for (int l = 0; l < NL; l++) {
        Layer *Ly = &L[l];
        read_into(f, Ly->fm, sizeof Ly->fm, "fm");
        read_into(f, Ly->ln1, sizeof Ly->ln1, "ln1"); read_into(f, &Ly->ln1f, 8, "ln1 f");
        read_into(f, Ly->ln2, sizeof Ly->ln2, "ln2"); read_into(f, &Ly->ln2f, 8, "ln2 f");
        for (int j = 0; j < 7; j++) {
            Mat *w = &Ly->w[j];
            w->N = NN[j]; w->K = KK[j];
            w->q = must_read(f, (size_t)w->N * w->K, "weights");
            w->m = must_read(f, (size_t)w->N * 8, "row multipliers");
            w->n = must_read(f, (size_t)w->N * 8, "row shifts");
        }
        Ly->silu = must_read(f, 65536 * 8, "silu table");
    }
    char extra;
    if (fread(&extra, 1, 1, f) != 0) { fprintf(stderr, "%s: trailing bytes\n", path); exit(2); }
    fclose(f);
}

/* RoPE rows beyond model.bin from DIR/rope.i64 (cos then sin, [rows, 32]) */
static void load_rope(const char *dir, int need) {
    char path[4096];
    snprintf(path, sizeof path, "%s/rope.i64", dir);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "T = %d > %d RoPE rows and no %s\n", need, rope_rows, path); exit(2); }
    fseek(f, 0, SEEK_END);
    const long bytes = ftell(f);
    fseek(f, 0, SEEK_SET);
    const int rows = (int)(bytes / (2 * 32 * 8));
    if (rows < need || bytes != (long)rows * 2 * 32 * 8) { fprintf(stderr, "%s: too short\n", path); exit(2); }
    free(rope_cos); free(rope_sin);
    rope_cos = must_read(f, (size_t)rows * 32 * 8, "rope cos");
    rope_sin = must_read(f, (size_t)rows * 32 * 8, "rope sin");
    rope_rows = rows;
    fclose(f);
}

/* ---------------------------------------------------------------- steps */
/* floor(sqrt(v)) by Newton's method on integers, starting above the root */
static uint64_t isqrt_u128(u128 v) {
    if (v == 0) return 0;
    const uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
    const int bits = hi ? 128 - __builtin_clzll(hi) : 64 - __builtin_clzll(lo);
    u128 x = (u128)1 << ((bits + 1) / 2);          /* >= sqrt(v) */
    for (;;) {
        const u128 y = (x + v / x) >> 1;
        if (y >= x) break;
        x = y;
    }
    while (x * x > v) x--;
    while ((x + 1) * (x + 1) <= v) x++;
    return (uint64_t)x;
}

/* python/intref.py:168-184: out [T, D] = SAT(RS(3 RS(x U, 16) g, 21 + f_g - f_out), bits) */
static void rmsnorm(const i64 *x, int T, const i64 *g, int fg_, int f_out, int bits, i64 *out) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        const i64 *r = x + (size_t)t * D;
        i128 S = 0;
        for (int c = 0; c < D; c++) S += (i128)r[c] * r[c];
        const u128 den = (u128)(S + EPS_S);
        const i64 U = (i64)isqrt_u128(((u128)1 << 80) / den);
        for (int c = 0; c < D; c++) {
            const i64 z = rs(r[c] * U, 16);
            out[(size_t)t * D + c] = sat(rs(z * g[c] * 3, 21 + fg_ - f_out), bits);
        }
    }
}

/* python/intref.py:186-190 (and the o/down residual form with bits = 64) */
static void linear(const i64 *a, int T, const Mat *w, int f_in, int f_out, int bits, i64 *out) {
    const int N = w->N, K = w->K;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        const i64 *ar = a + (size_t)t * K;
        for (int n = 0; n < N; n++) {
            const int8_t *wr = w->q + (size_t)n * K;
            i64 acc = 0;
            for (int k = 0; k < K; k++) acc += ar[k] * wr[k];
            out[(size_t)t * N + n] = sat(rs(acc * w->m[n], (int)(w->n[n] + f_in - f_out)), bits);
        }
    }
}

/* python/intref.py:212-222: heads of 64, pairs (d, d + 32), positions 0..T-1 */
static void rope(i64 *a, int T, int nheads, int f_in, int f_o, int bits) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int h = 0; h < nheads; h++) {
            i64 *p = a + ((size_t)t * nheads + h) * HD;
            const i64 *C = rope_cos + (size_t)t * 32, *S = rope_sin + (size_t)t * 32;
            for (int d = 0; d < 32; d++) {
                const i64 a1 = p[d], a2 = p[d + 32];
                p[d] = sat(rs(a1 * C[d] - a2 * S[d], 30 + f_in - f_o), bits);
                p[d + 32] = sat(rs(a2 * C[d] + a1 * S[d], 30 + f_in - f_o), bits);
            }
        }
}

/* python/intref.py:227-254: causal GQA attention, one query row at a time */
static void attention(const i64 *qr, const i64 *kr, const i64 *v, int T, int shift_s, int f_v, int f_c, int bits_c,
                      i64 *ctx) {
#pragma omp parallel
    {
        i64 *s = malloc((size_t)T * 8), *e = malloc((size_t)T * 8);
#pragma omp for schedule(dynamic, 16) collapse(2)
        for (int hh = 0; hh < NH; hh++)
            for (int i = 0; i < T; i++) {
                const int g = hh / 3;
                const i64 *q = qr + ((size_t)i * NH + hh) * HD;
                i64 mx = INT64_MIN;
                for (int j = 0; j <= i; j++) {
                    const i64 *k = kr + ((size_t)j * NKV + g) * HD;
                    i64 acc = 0;
                    for (int d = 0; d < HD; d++) acc += q[d] * k[d];
                    s[j] = sat(rs(acc, shift_s), 16);
                    if (s[j] > mx) mx = s[j];
                }
                i64 Z = 0;
                for (int j = 0; j <= i; j++) {
                    const i64 dd = mx - s[j];
                    e[j] = dd <= DMAX ? exp_tab[dd] : 0;
                    Z += e[j];
                }
                i64 out[HD];
                memset(out, 0, sizeof out);
                for (int j = 0; j <= i; j++) {
                    const i64 P = (e[j] * 65536 + Z / 2) / Z;
                    if (!P) continue;
                    const i64 *vr = v + ((size_t)j * NKV + g) * HD;
                    for (int d = 0; d < HD; d++) out[d] += P * vr[d];
                }
                for (int d = 0; d < HD; d++) ctx[((size_t)i * NH + hh) * HD + d] = sat(rs(out[d], 16 + f_v - f_c), bits_c);
            }
        free(s); free(e);
    }
}

/* python/intref.py:192-286 on x [T, D] in place */
static void block(int l, i64 *x, int T) {
    const Layer *Ly = &L[l];
    const i64 *fm = Ly->fm;
    const int bits_h = (int)fm[0], f_h = (int)fm[1], f_q = (int)fm[3], f_k = (int)fm[5];
    const int bits_v = (int)fm[6], f_v = (int)fm[7], bits_qr = (int)fm[8], f_qr = (int)fm[9];
    const int bits_kr = (int)fm[10], f_kr = (int)fm[11], bits_c = (int)fm[12], f_c = (int)fm[13];
    const int bits_h2 = (int)fm[14], f_h2 = (int)fm[15], bits_g = (int)fm[16], f_g = (int)fm[17];
    const int bits_u = (int)fm[18], f_u = (int)fm[19], bits_s = (int)fm[20], f_s = (int)fm[21];
    const int bits_m = (int)fm[22], f_m0 = (int)fm[23];
    (void)bits_s;
    const size_t TD = (size_t)T * D, TK = (size_t)T * 192, TF = (size_t)T * DFF;
    i64 *h = malloc(TD * 8), *q = malloc(TD * 8), *k = malloc(TK * 8), *v = malloc(TK * 8), *ctx = malloc(TD * 8);
    i64 *tmp = malloc(TD * 8), *gg = malloc(TF * 8), *uu = malloc(TF * 8);

    rmsnorm(x, T, Ly->ln1, (int)Ly->ln1f, f_h, bits_h, h);
    linear(h, T, &Ly->w[0], f_h, f_q, (int)fm[2], q);
    linear(h, T, &Ly->w[1], f_h, f_k, (int)fm[4], k);
    linear(h, T, &Ly->w[2], f_h, f_v, bits_v, v);
    rope(q, T, NH, f_q, f_qr, bits_qr);
    rope(k, T, NKV, f_k, f_kr, bits_kr);
    attention(q, k, v, T, f_qr + f_kr + 3 - 7, f_v, f_c, bits_c, ctx);
    linear(ctx, T, &Ly->w[3], f_c, F_RES, 64, tmp);                      /* o_res, unsaturated */
    for (size_t i = 0; i < TD; i++) x[i] = sat(x[i] + tmp[i], 32);

    rmsnorm(x, T, Ly->ln2, (int)Ly->ln2f, f_h2, bits_h2, h);
    linear(h, T, &Ly->w[4], f_h2, f_g, bits_g, gg);
    linear(h, T, &Ly->w[5], f_h2, f_u, bits_u, uu);
    const int f_m = bits_m == 32 ? (f_m0 < f_s + f_u ? f_m0 : f_s + f_u) : f_m0;
    for (size_t i = 0; i < TF; i++) gg[i] = sat(rs(Ly->silu[gg[i] + 32768] * uu[i], f_s + f_u - f_m), bits_m);
    linear(gg, T, &Ly->w[6], f_m, F_RES, 64, tmp);                       /* down_res */
    for (size_t i = 0; i < TD; i++) x[i] = sat(x[i] + tmp[i], 32);
    free(h); free(q); free(k); free(v); free(ctx); free(tmp); free(gg); free(uu);
}

/* ---------------------------------------------------------------- driver */
static int32_t *read_i32(const char *dir, const char *name, size_t n, int *present) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) { *present = 0; return NULL; }
    int32_t *a = must_read(f, n * 4, name);
    fclose(f);
    return a;
}

static void write_i32(const char *dir, const char *name, const i64 *a, size_t n) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) { fprintf(stderr, "%s: cannot write\n", path); exit(2); }
    int32_t *b = malloc(n * 4);
    for (size_t i = 0; i < n; i++) b[i] = (int32_t)a[i];
    if (fwrite(b, 4, n, f) != n) { fprintf(stderr, "%s: short write\n", path); exit(2); }
    free(b);
    fclose(f);
}

static size_t compare(const char *name, const i64 *got, const int32_t *exp, size_t n) {
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < n; i++)
        if (got[i] != (i64)exp[i]) { if (!bad) first = i; bad++; }
    if (bad) printf("  MISMATCH %-12s %zu of %zu, first at %zu (got %lld expected %d)\n", name, bad, n, first,
                    (long long)got[first], exp[first]);
    return bad;
}

int main(int argc, char **argv) {
    if (argc < 2) { fprintf(stderr, "usage: intref_c VECTORDIR [MODELDIR]\n"); return 2; }
    const char *vdir = argv[1], *mdir = argc > 2 ? argv[2] : argv[1];
    load_model(mdir);
    char path[4096];
    snprintf(path, sizeof path, "%s/ids.i64", vdir);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "%s: cannot open\n", path); return 2; }
    fseek(f, 0, SEEK_END);
    const int T = (int)(ftell(f) / 8);
    fseek(f, 0, SEEK_SET);
    i64 *ids = must_read(f, (size_t)T * 8, "ids");
    fclose(f);
    if (T > rope_rows) load_rope(mdir, T);
    for (int t = 0; t < T; t++)
        if (ids[t] < 0 || ids[t] >= V) { fprintf(stderr, "token id %lld out of range\n", (long long)ids[t]); return 2; }

    const size_t TD = (size_t)T * D, TV = (size_t)T * V;
    int have = 1;
    int32_t *exp_embed = read_i32(vdir, "exp_embed.i32", TD, &have);
    int32_t *exp_res = read_i32(vdir, "exp_resid_out.i32", NL * TD, &have);
    int32_t *exp_log = read_i32(vdir, "exp_logits.i32", TV, &have);
    const int check = have && exp_embed && exp_res && exp_log;

    const double t0 = (double)clock();
#ifdef _OPENMP
    const double w0 = omp_get_wtime();
#endif
    i64 *x = malloc(TD * 8), *res = check ? NULL : malloc(NL * TD * 8);
    for (int t = 0; t < T; t++)                                                  /* intref.py:163-166 */
        for (int c = 0; c < D; c++)
            x[(size_t)t * D + c] = rs((i64)emb_q[(size_t)ids[t] * D + c] * emb_m[ids[t]], (int)(emb_n[ids[t]] - F_RES));
    size_t total_bad = 0;
    if (check) total_bad += compare("embed", x, exp_embed, TD);
    else write_i32(vdir, "exp_embed.i32", x, TD);
    for (int l = 0; l < NL && !total_bad; l++) {
        block(l, x, T);
        if (check) {
            const size_t bad = compare("resid_out", x, exp_res + (size_t)l * TD, TD);
            printf("layer %2d: %s\n", l, bad ? "DIFFERS" : "exact");
            fflush(stdout);
            total_bad += bad;
        } else {
            memcpy(res + (size_t)l * TD, x, TD * 8);
        }
    }
    if (!total_bad) {                                                            /* intref.py:296-301 */
        i64 *y = malloc(TD * 8), *lg = malloc(TV * 8);
        rmsnorm(x, T, fg, (int)fg_f, (int)f_y, 16, y);
#pragma omp parallel for schedule(static)
        for (int t = 0; t < T; t++)
            for (int n = 0; n < V; n++) {
                const int8_t *wr = emb_q + (size_t)n * D;
                i64 acc = 0;
                for (int c = 0; c < D; c++) acc += y[(size_t)t * D + c] * wr[c];
                lg[(size_t)t * V + n] = rs(acc * emb_m[n], (int)(emb_n[n] + f_y - 16));
            }
        if (check) {
            total_bad += compare("logits", lg, exp_log, TV);
            printf("logits: %s\n", total_bad ? "DIFFERS" : "exact");
        } else {
            write_i32(vdir, "exp_resid_out.i32", res, NL * TD);
            write_i32(vdir, "exp_logits.i32", lg, TV);
        }
        free(y); free(lg);
    }
    double wall = ((double)clock() - t0) / CLOCKS_PER_SEC;
#ifdef _OPENMP
    wall = omp_get_wtime() - w0;
#endif
    if (check) printf("%s (%d tokens, %.1f s)\n", total_bad ? "FAIL" : "ALL STATES EXACT", T, wall);
    else printf("WROTE STATES (%d tokens, %.1f s)\n", T, wall);
    return total_bad ? 1 : 0;
}
