/* Drives the C oracle under AddressSanitizer / UBSan: random logits and biases over every
 * routing geometry the oracle accepts (E up to 1024, top_k up to 64), tie-heavy inputs,
 * extreme logits, the permute with every EP offset, and the rejected geometries. Exits non-zero
 * on an invariant failure; the sanitizers abort on any memory or UB error. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int oracle_route_ds(const float*, const uint16_t*, int, int, int, int, int, float, int32_t*, float*);
int oracle_route_softmax(const float*, int, int, int, int32_t*, float*);
int oracle_permute(const int32_t*, const float*, int, int, int, int, int32_t*, int32_t*, int32_t*,
                   float*, int32_t*);
void oracle_sigmoid_batch(const float*, float*, int64_t);
void oracle_exp_batch(const float*, float*, int64_t);

static uint64_t rng = 88172645463325252ull;
static uint32_t next32(void) {
  rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
  return (uint32_t)(rng >> 16);
}
static float unif(void) { return (next32() & 0xffffff) / 16777216.0f; }

#define CHECK(c) do { if (!(c)) { fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); return 1; } } while (0)

static int run_case(int T, int E, int n_group, int topk_group, int top_k, int softmax, int ties,
                    int E_local, int offset) {
  float* x = malloc(sizeof(float) * (size_t)T * E);
  uint16_t* b = malloc(sizeof(uint16_t) * E);
  int32_t* idx = malloc(sizeof(int32_t) * (size_t)T * top_k);
  float* w = malloc(sizeof(float) * (size_t)T * top_k);
  for (size_t i = 0; i < (size_t)T * E; ++i) {
    float v = (unif() - 0.5f) * 8.0f;
    x[i] = ties ? roundf(v) : v;
    if ((next32() & 255) == 0) x[i] = (next32() & 1) ? 150.0f : -150.0f;
  }
  for (int e = 0; e < E; ++e) b[e] = ties ? 0 : (uint16_t)(0x3c00 + (next32() & 0x3ff)) ^ ((next32() & 1) << 15);
  int rc = softmax ? oracle_route_softmax(x, T, E, top_k, idx, w)
                   : oracle_route_ds(x, b, T, E, n_group, topk_group, top_k, 2.5f, idx, w);
  CHECK(rc == 0);
  for (size_t i = 0; i < (size_t)T * top_k; ++i) CHECK(idx[i] >= 0 && idx[i] < E && isfinite(w[i]));
  int32_t* counts = malloc(sizeof(int32_t) * E_local);
  int32_t* offs = malloc(sizeof(int32_t) * (E_local + 1));
  int32_t* st = malloc(sizeof(int32_t) * ((size_t)T * top_k + 1));
  float* sw = malloc(sizeof(float) * ((size_t)T * top_k + 1));
  int32_t* pair_of = malloc(sizeof(int32_t) * (size_t)T * top_k);
  int n = oracle_permute(idx, w, T, top_k, offset, E_local, counts, offs, st, sw, pair_of);
  CHECK(n >= 0 && n <= T * top_k && offs[E_local] == n);
  for (int e = 0; e < E_local; ++e)
    for (int p = offs[e] + 1; p < offs[e + 1]; ++p) CHECK(st[p - 1] < st[p]);
  free(x); free(b); free(idx); free(w); free(counts); free(offs); free(st); free(sw); free(pair_of);
  return 0;
}

int main(void) {
  int cases = 0;
  for (int it = 0; it < 400; ++it) {
    const int E = 64 << (next32() % 5);              /* 64 .. 1024 */
    const int softmax = next32() & 1;
    const int top_k = 1 + next32() % (E < 64 ? E : 64);
    int n_group = 1, topk_group = 1;
    if (!softmax) {
      do { n_group = 1 << (next32() % 6); } while (E % n_group);
      topk_group = 1 + next32() % n_group;
      if (top_k > topk_group * (E / n_group)) continue;
    }
    const int T = next32() % 70;
    const int E_local = 1 + next32() % E;
    const int offset = next32() % (E + 1);
    if (run_case(T, E, n_group, topk_group, top_k, softmax, next32() & 1, E_local, offset)) return 1;
    ++cases;
  }
  /* geometries the oracle must refuse without touching memory out of bounds */
  float x[4] = {0, 0, 0, 0};
  int32_t idx[4];
  float w[4];
  CHECK(oracle_route_ds(x, NULL, 1, 2048, 8, 4, 8, 1.0f, idx, w) == -1);   /* E too large */
  CHECK(oracle_route_ds(x, NULL, 1, 64, 3, 2, 8, 1.0f, idx, w) == -1);     /* groups */
  CHECK(oracle_route_ds(x, NULL, 1, 64, 8, 4, 65, 1.0f, idx, w) == -1);    /* top_k > 64 */
  CHECK(oracle_route_softmax(x, 1, 4, 5, idx, w) == -1);                   /* top_k > E */
  /* sigmoid / exp over a sweep of every binade, both signs, and the special values */
  enum { N = 1 << 16 };
  static float xs[N], ys[N];
  for (int i = 0; i < N; ++i) {
    uint32_t u = next32();
    float v;
    __builtin_memcpy(&v, &u, 4);
    xs[i] = isfinite(v) ? v : 0.0f;
  }
  xs[0] = INFINITY; xs[1] = -INFINITY; xs[2] = NAN;
  oracle_sigmoid_batch(xs, ys, N);
  for (int i = 3; i < N; ++i) CHECK(ys[i] >= 0.0f && ys[i] <= 1.0f);
  oracle_exp_batch(xs, ys, N);
  printf("oracle_check: %d routing/permute cases, %d sigmoid/exp values: ok\n", cases, N);
  return 0;
}
