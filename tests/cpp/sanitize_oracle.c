/* sanitize_oracle.c — drives every function of the CPU oracle (oracle/fqa_oracle.c) on
 * seeded random batches and on the edge cases the pack's status codes cover, for a build
 * under AddressSanitizer + UndefinedBehaviorSanitizer (tests/test_sanitize.py).  Host
 * code only.  Prints one line per case; any sanitizer report aborts with a non-zero exit.
 *
 * Besides running clean, it checks what holds for any input: the pack's row count equals
 * the sum of the new rows of an accepted batch, every block-table tail entry is -1, and
 * the decode plan's shares add up to 8 runs per decode page. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/fqa_oracle.h"

#define PAGE 16
#define NQ 32
#define NKV 8
#define D 128
#define STRIDE 6144

static uint64_t g_state = 0x9e3779b97f4a7c15ull;
static uint64_t next_u64(void) { /* splitmix64 */
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static int rnd(int lo, int hi) { return lo + (int)(next_u64() % (uint64_t)(hi - lo + 1)); }
static float rnd_unit(void) { return (float)((next_u64() >> 11) * (1.0 / 9007199254740992.0)); }
static uint16_t rnd_bf16(void) { return fqo_f32_to_bf16(4.0f * rnd_unit() - 2.0f); }

static void* xcalloc(size_t n, size_t sz) {
  void* p = calloc(n ? n : 1, sz);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(2);
  }
  return p;
}

static int failures = 0;
#define EXPECT(cond, ...)                    \
  do {                                       \
    if (!(cond)) {                           \
      fprintf(stderr, "FAIL: " __VA_ARGS__); \
      fprintf(stderr, "\n");                 \
      ++failures;                            \
    }                                        \
  } while (0)

/* One batch: R requests (decode or prefill, with a cached prefix), pages drawn without
 * repeats from a pool of `pool_pages`; then pack -> append -> decode + prefill. */
static void run_step(int R, int max_ctx, int pool_pages, int mode) {
  int max_blocks = (max_ctx + PAGE - 1) / PAGE;
  int32_t* computed = xcalloc(R, 4);
  int32_t* n_new = xcalloc(R, 4);
  int32_t* bt_off = xcalloc(R + 1, 4);
  int32_t* bt_pages = xcalloc((size_t)R * max_blocks + 1, 4);
  int32_t* perm = xcalloc(pool_pages, 4);
  for (int i = 0; i < pool_pages; ++i) perm[i] = i;
  for (int i = pool_pages - 1; i > 0; --i) {
    int j = rnd(0, i), t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  int used = 0, rows = 0;
  for (int r = 0; r < R; ++r) {
    int dec = rnd(0, 2) != 0;
    computed[r] = rnd(0, max_ctx / 2);
    n_new[r] = dec ? 1 : rnd(0, 80);
    if (computed[r] + n_new[r] > max_ctx) n_new[r] = max_ctx - computed[r];
    int nb = (computed[r] + n_new[r] + PAGE - 1) / PAGE;
    if (used + nb > pool_pages) nb = 0, n_new[r] = 0, computed[r] = 0;
    bt_off[r + 1] = bt_off[r] + nb;
    for (int g = 0; g < nb; ++g) bt_pages[bt_off[r] + g] = perm[used++];
    rows += n_new[r];
  }
  /* mode 6: decodes share their first pages (up to 4, and only cached ones) from a common
   * run at the end of the permutation, so shared-prefix groups form */
  if (mode == 6)
    for (int r = 0; r < R; ++r) {
      if (n_new[r] != 1) continue;
      const int k = computed[r] / PAGE < 4 ? computed[r] / PAGE : 4;
      for (int j = 0; j < k; ++j) bt_pages[bt_off[r] + j] = perm[pool_pages - 1 - j];
    }
  /* edge cases of the status codes */
  if (mode == 1 && R > 0) n_new[0] += PAGE * 4;  /* short table */
  if (mode == 2 && R > 0) computed[R - 1] = -3;   /* negative */
  if (mode == 3 && R > 0 && bt_off[R] > bt_off[R - 1]) bt_pages[bt_off[R - 1]] = pool_pages + 5;
  int max_rows = mode == 4 ? rows / 2 : rows + 8; /* mode 4: too many rows */
  int waves = 64, wave_cap = mode == 5 ? 1 : 64, tile = 64;
  int item_cap = max_rows / tile + R + 1;
  int32_t* cu = xcalloc(R + 1, 4);
  int32_t* qlen = xcalloc(R, 4);
  int32_t* pos = xcalloc(max_rows, 4);
  int32_t* req = xcalloc(max_rows, 4);
  int32_t* slot = xcalloc(max_rows, 4);
  int32_t* bt = xcalloc((size_t)R * max_blocks, 4);
  int32_t* drids = xcalloc(R, 4);
  int32_t* prids = xcalloc(R, 4);
  int32_t* dseqs = xcalloc((size_t)R * 4, 4);
  int32_t* dwaves = xcalloc((size_t)wave_cap * 8, 4);
  int32_t* items = xcalloc((size_t)item_cap * 4, 4);
  const int pre_cap = 8 * 16 * R;
  int32_t* dpfx = xcalloc((size_t)R * 8 + 8, 4);
  int32_t* ditems = xcalloc((size_t)pre_cap * 12 + 12, 4);
  int32_t meta[16];
  int st = fqo_pack(R, computed, n_new, bt_off, bt_pages, max_rows, max_blocks, pool_pages,
                    waves, 4, wave_cap, tile, item_cap, mode == 0, mode == 0 || mode == 6 ? 1 : 0,
                    pre_cap, cu,
                    qlen, pos, req, slot, bt, drids, prids, dseqs, dwaves, items, dpfx, ditems,
                    meta);
  printf("step R=%d mode=%d rows=%d status=%d\n", R, mode, rows, st);
  if (st == 0 || st == 4) { /* accepted (4: a page id outside the pool, flagged only) */
    EXPECT(meta[0] == rows, "rows %d != %d", meta[0], rows);
    for (int r = 0; r < R; ++r)
      for (int g = bt_off[r + 1] - bt_off[r]; g < max_blocks; ++g)
        EXPECT(bt[(size_t)r * max_blocks + g] == -1, "block-table tail not -1");
    long long runs = 0;
    for (int w = 0; w < meta[4]; ++w) runs += dwaves[8 * w + 3];
    long long dpages = 0;
    long long ppages = 0, pruns = 0;
    for (int i = 0; i < meta[1]; ++i) {
      dpages += computed[drids[i]] / PAGE + 1 - dpfx[8 * i];
      ppages += dpfx[8 * i];
    }
    EXPECT(runs == 8 * dpages, "decode shares cover %lld of %lld runs", runs, 8 * dpages);
    /* the prefix items cover each member's shared pages once per kv head */
    for (int i = 0; i < meta[10]; ++i)
      for (int j = 4; j < 12; ++j) pruns += ditems[12 * i + j] >= 0 ? ditems[12 * i + 3] - ditems[12 * i + 2] : 0;
    EXPECT(pruns == 8 * ppages, "prefix items cover %lld of %lld runs", pruns, 8 * ppages);

    int T = meta[0];
    uint16_t* qkv = xcalloc((size_t)(T ? T : 1) * STRIDE, 2);
    for (size_t i = 0; i < (size_t)T * STRIDE; ++i) qkv[i] = rnd_bf16();
    size_t pool_elems = (size_t)pool_pages * NKV * 2 * PAGE * D;
    uint16_t* pool = xcalloc(pool_elems, 2);
    for (size_t i = 0; i < pool_elems; ++i) pool[i] = rnd_bf16();
    float wq[D], wk[D];
    for (int d = 0; d < D; ++d) wq[d] = rnd_unit() + 0.5f, wk[d] = rnd_unit() + 0.5f;
    float* cs = xcalloc((size_t)max_ctx * D / 2, 4);
    float* sn = xcalloc((size_t)max_ctx * D / 2, 4);
    fqo_rope_tables(max_ctx, D, 1e6f, cs, sn);
    fqo_qknorm_rope_append(NQ, NKV, D, STRIDE, 1e-6f, qkv, wq, wk, cs, sn, max_ctx, pos, slot,
                           T, pool, pool_pages, mode & 1);
    uint16_t* out = xcalloc((size_t)(T ? T : 1) * NQ * D, 2);
    float* absv = xcalloc((size_t)(T ? T : 1) * NQ * D, 4);
    fqo_decode(NQ, NKV, D, STRIDE, 0.0883883f, qkv, pool, pool_pages, bt, max_blocks, cu, pos,
               drids, meta[1], out);
    fqo_prefill_absv(NQ, NKV, D, STRIDE, 0.0883883f, qkv, pool, pool_pages, bt, max_blocks, cu,
                     pos, prids, meta[2], out, absv);
    free(qkv), free(pool), free(cs), free(sn), free(out), free(absv);
  }
  free(computed), free(n_new), free(bt_off), free(bt_pages), free(perm), free(cu), free(qlen);
  free(pos), free(req), free(slot), free(bt), free(drids), free(prids), free(dseqs);
  free(dwaves), free(items), free(dpfx), free(ditems);
}

static void run_schedule(int n) {
  int32_t* ntok = xcalloc(n, 4);
  int32_t* comp = xcalloc(n, 4);
  int32_t* breq = xcalloc(n, 4);
  int32_t* bn = xcalloc(n, 4);
  for (int i = 0; i < n; ++i) {
    comp[i] = rnd(0, 3000);
    ntok[i] = comp[i] + rnd(-2, 3000); /* finished and over-finished requests too */
  }
  int R = fqo_schedule(n, ntok, comp, 8192, rnd(1, 2048), breq, bn);
  int sum = 0;
  for (int i = 0; i < R; ++i) sum += bn[i];
  printf("schedule n=%d -> %d requests, %d tokens\n", n, R, sum);
  EXPECT(sum <= 8192, "budget exceeded");
  free(ntok), free(comp), free(breq), free(bn);
}

static void run_sample(int B, int N) {
  float* lg = xcalloc((size_t)B * N, 4);
  float *it = xcalloc(B, 4), *tp = xcalloc(B, 4), *u = xcalloc(B, 4);
  int32_t* out = xcalloc(B, 4);
  double *thr = xcalloc(B, 8), *mass = xcalloc(B, 8);
  for (size_t i = 0; i < (size_t)B * N; ++i) lg[i] = 8.0f * rnd_unit() - 4.0f;
  for (int b = 0; b < B; ++b) {
    it[b] = b % 3 == 0 ? 0.f : 1.0f;
    tp[b] = b % 2 ? 0.9f : 1.0f;
    u[b] = rnd_unit();
  }
  fqo_sample(lg, B, N, N, it, tp, u, out, thr, mass);
  for (int b = 0; b < B; ++b) EXPECT(out[b] >= 0 && out[b] < N, "sampled token out of range");
  printf("sample %dx%d\n", B, N);
  free(lg), free(it), free(tp), free(u), free(out), free(thr), free(mass);
}

int main(void) {
  float c[4 * 64], s[4 * 64];
  fqo_rope_tables(4, D, 1e6f, c, s);
  EXPECT(c[0] == 1.0f && s[0] == 0.0f, "rope table row 0");
  EXPECT(fqo_pool_offset(NKV, D, 3, 2, 1, 5, 7) ==
             ((3LL * NKV + 2) * 2 + 1) * PAGE * D + 7 * PAGE + 5,
         "pool offset");
  run_step(0, 256, 64, 0);
  for (int mode = 0; mode <= 6; ++mode) run_step(6, 512, 400, mode);
  for (int k = 0; k < 3; ++k) run_step(rnd(8, 40), 1024, 2000, 6);
  for (int k = 0; k < 4; ++k) run_step(rnd(1, 24), 1024, 2000, 0);
  run_schedule(0);
  run_schedule(1);
  run_schedule(300);
  run_sample(5, 1000);
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
