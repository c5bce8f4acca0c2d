/*
 * fqa_oracle.c — CPU restatement of the reference engine's per-step attention path.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker / the reported CPU
 * baseline.  The product (flashqwen_amd, libfqa.so) never links or calls it.
 *
 * Every function follows a reference file:line (paths relative to the reference's
 * engine/src/).  Arithmetic is fp32 with bf16 inputs and bf16 outputs, the semantics
 * the reference kernels implement; differences are limited to summation order, the
 * exp implementation, and two-pass (exact-max) instead of online softmax, all of which
 * the attention tolerance (bf16 max-abs 2e-2, mean-abs 2e-3) absorbs.
 *
 * Pinning (see tests/test_oracle.py): the pack is checked against a second,
 * independent pure-Python restatement and hand-built cases with known answers; RoPE
 * and RMSNorm against torch fp64 library routines plus closed forms (pos 0 identity,
 * pair-norm preservation, relative-position invariance of q.k); attention against
 * torch's fp64 scaled_dot_product_attention and closed forms (single key -> V,
 * identical keys -> mean V, first causal row -> V[0], page-permutation invariance).
 */
#include "fqa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PAGE 16
/* pages compared for a shared decode prefix (FQA_DEC_PREFIX_CAP, include/fqa.h) */
#define FQA_DEC_PREFIX_CAP 8192
/* costs of the decode plan in cost units (FQA_DEC_PAGE_COST ..., include/fqa.h): a page
 * run, one in a sequence flagged shared, a stream's start, a shared-prefix member's */
#define FQA_DEC_PAGE_COST 8
#define FQA_DEC_SHARED_PAGE_COST 5
#define FQA_DEC_STREAM_COST 32
#define FQA_DEC_PREFIX_STREAM_COST 16
/* a decode stream's start cost: more for a shared-prefix member */
static int64_t stream_start_cost(int pfx) {
  return FQA_DEC_STREAM_COST + (pfx > 0 ? FQA_DEC_PREFIX_STREAM_COST : 0);
}
/* a page run's cost in a decode sequence (cheap: flagged FQA_DEC_SHARED and not the
 * first decode sequence with its first page) */
static int64_t page_cost(int cheap) {
  return cheap ? FQA_DEC_SHARED_PAGE_COST : FQA_DEC_PAGE_COST;
}

float fqo_bf16_to_f32(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

uint16_t fqo_f32_to_bf16(float f) {
  uint32_t bits;
  memcpy(&bits, &f, sizeof bits);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u); /* NaN */
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

int fqo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Pool layout of include/fqa.h: per (page, kv head) an 8 KiB run: K [16][D] then
 * V transposed [D][16].  The reference's layout is NHD [page][2][16][kv_dim]
 * (kv_store.h:13-16); only the addressing differs, not what is stored. */
int64_t fqo_pool_offset(int n_kv, int head_dim, int64_t page, int kvh, int plane, int tok,
                        int d) {
  int64_t base = ((page * n_kv + kvh) * 2 + plane) * (int64_t)PAGE * head_dim;
  return plane == 0 ? base + (int64_t)tok * head_dim + d : base + (int64_t)d * PAGE + tok;
}

/* RopeTables::Build (model_runtime.cu:111-126): float pow/cos/sin, angle = p * inv. */
void fqo_rope_tables(int max_pos, int head_dim, float theta, float* cos_tab, float* sin_tab) {
  int half = head_dim / 2;
  for (int p = 0; p < max_pos; ++p)
    for (int i = 0; i < half; ++i) {
      float inv = powf(theta, -2.0f * (float)i / (float)head_dim);
      float ang = (float)p * inv;
      cos_tab[(int64_t)p * half + i] = cosf(ang);
      sin_tab[(int64_t)p * half + i] = sinf(ang);
    }
}

/* Scheduler::BuildBatch (scheduler.cc:116-143) with every Grow succeeding: stable sort of
 * the running requests by Remaining() ascending, then n = min(remaining, budget) capped
 * at prefill_chunk when remaining > 1; stop when the budget is spent, skip finished
 * requests (remaining <= 0).  Returns the number of requests in the batch. */
int fqo_schedule(int n_running, const int32_t* num_tokens, const int32_t* computed,
                 int token_budget, int prefill_chunk, int32_t* batch_req, int32_t* batch_n) {
  int* order = (int*)malloc(sizeof(int) * (n_running > 0 ? n_running : 1));
  for (int i = 0; i < n_running; ++i) order[i] = i;
  /* insertion sort: stable */
  for (int i = 1; i < n_running; ++i) {
    int v = order[i], rv = num_tokens[v] - computed[v], j = i - 1;
    while (j >= 0 && num_tokens[order[j]] - computed[order[j]] > rv) {
      order[j + 1] = order[j];
      --j;
    }
    order[j + 1] = v;
  }
  int budget = token_budget, R = 0;
  for (int k = 0; k < n_running; ++k) {
    if (budget <= 0) break;
    int idx = order[k];
    int remaining = num_tokens[idx] - computed[idx];
    if (remaining <= 0) continue;
    int n = remaining < budget ? remaining : budget;
    if (remaining > 1 && n > prefill_chunk) n = prefill_chunk;
    batch_req[R] = idx;
    batch_n[R] = n;
    ++R;
    budget -= n;
  }
  free(order);
  return R;
}

static int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

/* Pack: UploadRows + PackBlockTables + SplitDecodePrefill (model_runtime.cu:47-91) and
 * EmitChunk's row generation (scheduler.h:66-72), plus the slot mapping implied by
 * StoreKvKernel (kv_store.cu:56-60) and this library's decode/prefill work plans. */
int fqo_pack(int R, const int32_t* computed, const int32_t* n_new, const int32_t* bt_off,
             const int32_t* bt_pages, int max_rows, int max_blocks, int64_t pool_pages,
             int dec_grid_waves, int dec_min_pages, int dec_wave_cap, int pre_tile_q,
             int pre_item_cap, int dec_share, int dec_prefix_pages, int dec_pre_cap,
             int32_t* cu_seqlens, int32_t* qlen, int32_t* positions,
             int32_t* row_req, int32_t* slot_mapping, int32_t* block_tables,
             int32_t* decode_rids, int32_t* prefill_rids, int32_t* dec_seqs,
             int32_t* dec_waves, int32_t* pre_items, int32_t* dec_prefix,
             int32_t* dec_pre_items, int32_t* meta) {
  for (int i = 0; i < 16; ++i) meta[i] = 0;
  meta[8] = R;
  /* structural checks: the smallest violated code wins */
  int code = 0;
  int64_t T64 = 0;
  for (int r = 0; r < R; ++r) {
    int c = 0;
    if (computed[r] < 0 || n_new[r] < 0) c = 5;
    else {
      int nb = bt_off[r + 1] - bt_off[r];
      int need = ceil_div((int64_t)computed[r] + n_new[r], PAGE);
      if (nb < need) c = 1;
      else if (nb > max_blocks) c = 2;
      T64 += n_new[r];
    }
    if (c && (code == 0 || c < code)) code = c;
  }
  if (T64 > max_rows && (code == 0 || 3 < code)) code = 3;
  if (code) {
    meta[7] = code;
    return code;
  }
  int T = (int)T64;

  /* SplitDecodePrefill: qlen, qstart (exclusive scan), classification by qlen == 1 */
  int acc = 0, nd = 0, np = 0, maxq = 1;
  for (int r = 0; r < R; ++r) {
    qlen[r] = n_new[r];
    cu_seqlens[r] = acc;
    acc += n_new[r];
    if (n_new[r] == 1) decode_rids[nd++] = r;
    else {
      prefill_rids[np++] = r;
      if (n_new[r] > maxq) maxq = n_new[r];
    }
  }
  cu_seqlens[R] = acc;
  for (int i = nd; i < R; ++i) decode_rids[i] = -1;
  for (int i = np; i < R; ++i) prefill_rids[i] = -1;

  /* rows (EmitChunk: pos = computed_ + k) and slot mapping */
  int bad_page = 0;
  for (int r = 0; r < R; ++r)
    for (int k = 0; k < n_new[r]; ++k) {
      int t = cu_seqlens[r] + k, p = computed[r] + k;
      positions[t] = p;
      row_req[t] = r;
      int page = bt_pages[bt_off[r] + p / PAGE];
      slot_mapping[t] = page * PAGE + p % PAGE;
    }
  /* PackBlockTables; the tail is defined as -1 (the reference leaves it stale) */
  for (int r = 0; r < R; ++r) {
    int nb = bt_off[r + 1] - bt_off[r];
    for (int g = 0; g < max_blocks; ++g) {
      int v = g < nb ? bt_pages[bt_off[r] + g] : -1;
      if (g < nb && (v < 0 || v >= pool_pages)) bad_page = 1;
      block_tables[(int64_t)r * max_blocks + g] = v;
    }
  }

  /* Shared prefixes (this library's decode plan; the reference reads every sequence's
   * pages itself): decode sequences with the same first page id (>= 0) form a group led
   * by the first of them.  Each member's common prefix with the leader (its LCP, at most
   * FQA_DEC_PREFIX_CAP pages; the leader's own is its page count) is capped at
   * computed / 16, so that every member keeps the page of its last key; the group's
   * prefix P is the minimum over the members.  With P >= dec_prefix_pages the members'
   * pages [0, P) are attended once for the whole group (prefix items) and each member's
   * decode streams cover pages [P, pages) only. */
  int32_t* pfx = (int32_t*)calloc(nd > 0 ? nd : 1, sizeof(int32_t));    /* P per member */
  int32_t* lead = (int32_t*)malloc(sizeof(int32_t) * (nd > 0 ? nd : 1)); /* leader or -1 */
  int n_groups = 0, n_pitems = 0;
  if (dec_prefix_pages > 0) {
    for (int di = 0; di < nd; ++di) {
      const int32_t f = bt_pages[bt_off[decode_rids[di]]];
      int first = -1, count = 0;
      for (int dj = 0; f >= 0 && dj < nd; ++dj)
        if (bt_pages[bt_off[decode_rids[dj]]] == f) {
          if (first < 0) first = dj;
          ++count;
        }
      lead[di] = count >= 2 ? first : -1;
    }
    for (int l = 0; l < nd; ++l) {
      if (lead[l] != l) continue; /* l leads a group */
      const int rl = decode_rids[l], pl = computed[rl] / PAGE + 1;
      int P = 0x7fffffff;
      for (int di = 0; di < nd; ++di) {
        if (lead[di] != l) continue;
        const int r = decode_rids[di], pages = computed[r] / PAGE + 1;
        int k = 0;
        if (di == l) k = pages;
        else
          while (k < pages && k < pl && bt_pages[bt_off[r] + k] == bt_pages[bt_off[rl] + k]) ++k;
        if (k > FQA_DEC_PREFIX_CAP) k = FQA_DEC_PREFIX_CAP;
        if (k > computed[r] / PAGE) k = computed[r] / PAGE;
        if (k < P) P = k;
      }
      if (P < dec_prefix_pages) continue;
      int M = 0;
      for (int di = 0; di < nd; ++di) M += lead[di] == l;
      const int Q = (M + 7) / 8, CP = P / 16 > 16 ? (P + 15) / 16 : 16, Cn = (P + CP - 1) / CP;
      ++n_groups;
      n_pitems += 8 * Cn * Q;
      for (int di = 0; di < nd; ++di)
        if (lead[di] == l) pfx[di] = P;
    }
    if (n_pitems > dec_pre_cap) { /* more prefix work than the plan holds: none */
      n_groups = n_pitems = 0;
      for (int di = 0; di < nd; ++di) pfx[di] = 0;
    }
  }
  /* A decode sequence whose first page is also another decode sequence's first page
   * (a shared prefix) is flagged shared (bit 30, FQA_DEC_SHARED in fqa.h, in both n_keys
   * fields) unless it is a group member (its streams then cover its own pages); a
   * negative id is never shared.  This build's load-hint and cost policy; the reference
   * has no plan to restate here. */
  /* dcheap: a shared sequence that is not the first (by decode index) with its first
   * page, whose pages the plan prices at FQA_DEC_SHARED_PAGE_COST (the first one's reads
   * bring them into the caches) */
  int32_t* dshared = (int32_t*)calloc(nd > 0 ? nd : 1, sizeof(int32_t));
  int32_t* dcheap = (int32_t*)calloc(nd > 0 ? nd : 1, sizeof(int32_t));
  for (int a = 0; a < nd; ++a) {
    const int32_t id = bt_pages[bt_off[decode_rids[a]]];
    int sh = 0, first = a;
    for (int b = 0; id >= 0 && b < nd; ++b)
      if (b != a && bt_pages[bt_off[decode_rids[b]]] == id) {
        sh = 1;
        if (b < first) first = b;
      }
    dshared[a] = sh && pfx[a] == 0;
    dcheap[a] = dshared[a] && first != a;
  }
  /* decode plan (stream-K): the (decode sequence, kv head) page streams [P, pages) end to
   * end in cost positions (the stream's start positions, then u per page, u =
   * page_cost), W = 8 * sum of the stream costs, cut into G equal shares
   * [w*W/G, (w+1)*W/G); a share takes the pages whose last position falls in it */
  int64_t total = 0, cost_total = 0;
  for (int di = 0; di < nd; ++di) {
    const int len = computed[decode_rids[di]] / PAGE + 1 - pfx[di];
    total += len;
    cost_total += (int64_t)len * page_cost(dcheap[di]) + stream_start_cost(pfx[di]);
  }
  int64_t W = 8 * cost_total;
  int minp = dec_min_pages > 0 ? dec_min_pages : 1;
  int G = 0;
  if (W > 0) {
    int64_t gmax = (W + (int64_t)FQA_DEC_PAGE_COST * minp - 1) / ((int64_t)FQA_DEC_PAGE_COST * minp);
    G = (int)(dec_grid_waves < gmax ? dec_grid_waves : gmax);
    /* dec_share (this library's plan for a decode that runs beside the prefill, fqa.h):
     * D = 783 * decode pages, P = prefill key-rows */
    uint64_t P = 0;
    if (dec_share)
      for (int pi = 0; pi < np; ++pi) {
        uint64_t n = (uint64_t)n_new[prefill_rids[pi]], c = (uint64_t)computed[prefill_rids[pi]];
        P += n * c + n * (n + 1) / 2;
      }
    /* a multiple of 32 waves in [32, N - 32] where the modelled decode time
     * D (36 G + 25 N) / (50 G) meets the prefill's P N / (N - G) (fqa.h) */
    if (dec_share && P > 0 && dec_grid_waves >= 64 && dec_grid_waves <= 4096) {
      uint64_t D = 783ull * (uint64_t)total, N = (uint64_t)dec_grid_waves;
      while (D >= (1ull << 30) || P >= (1ull << 30)) {
        D >>= 1;
        P >>= 1;
      }
      int gs = 32, top = (dec_grid_waves - 32) / 32 * 32;
      for (int g = 32; g <= top; g += 32) /* prefill(g) <= decode(g) */
        if (50 * P * N * (uint64_t)g <= D * (36 * (uint64_t)g + 25 * N) * (N - (uint64_t)g))
          gs = g;
      { /* one step further if the prefill there ends before the decode at gs */
        uint64_t g = (uint64_t)gs;
        if (gs + 32 <= top && 50 * P * N * g < D * (36 * g + 25 * N) * (N - g - 32)) gs += 32;
      }
      if (gs < G) G = gs;
    }
  }
  /* prefill plan: query tiles of pre_tile_q rows, ordered by key count descending
   * (longest first), ties by (prefill index, tile) ascending */
  int npi = 0;
  for (int pi = 0; pi < np; ++pi) npi += ceil_div(n_new[prefill_rids[pi]], pre_tile_q);

  if (G > dec_wave_cap || npi > pre_item_cap || W > 0x7fffffff) {
    for (int i = 0; i < 16; ++i) meta[i] = 0;
    meta[8] = R;
    meta[7] = 6;
    free(pfx);
    free(lead);
    free(dshared);
    free(dcheap);
    return 6;
  }
  {
    int64_t X = 0; /* cost prefix over decode indices */
    for (int di = 0; di < nd; ++di) {
      int r = decode_rids[di], pages = computed[r] / PAGE + 1 - pfx[di];
      dec_seqs[4 * di + 0] = r;
      dec_seqs[4 * di + 1] = cu_seqlens[r];
      dec_seqs[4 * di + 2] = computed[r] + 1;
      dec_seqs[4 * di + 3] = (int32_t)(8 * X);
      X += (int64_t)pages * page_cost(dcheap[di]) + stream_start_cost(pfx[di]);
    }
    /* Position x: the sequence, kv head and offset in the stream's cost span, and the
     * pages whose last position is below x (every stream's pages come after its start
     * positions). */
    int64_t* pstart = (int64_t*)malloc(sizeof(int64_t) * (nd + 1)); /* 8 * page prefix */
    pstart[0] = 0;
    for (int di = 0; di < nd; ++di)
      pstart[di + 1] = pstart[di] + 8 * (int64_t)(computed[decode_rids[di]] / PAGE + 1 - pfx[di]);
    for (int w = 0; w < G; ++w) {
      int64_t g0 = (int64_t)w * W / G, g1 = (int64_t)(w + 1) * W / G;
      int64_t below[2];
      int di = 0, kvh = 0, off = 0;
      for (int e = 1; e >= 0; --e) { /* g1, then g0 (whose stream is the share's start) */
        const int64_t x = e ? g1 : g0;
        int64_t start = 0;
        int d = 0;
        while (d < nd) {
          const int64_t cost = (int64_t)(computed[decode_rids[d]] / PAGE + 1 - pfx[d]) *
                                   page_cost(dcheap[d]) + stream_start_cost(pfx[d]);
          if (x < start + 8 * cost) break;
          start += 8 * cost;
          ++d;
        }
        if (d == nd) {
          below[e] = pstart[nd];
          continue;
        }
        const int64_t len = computed[decode_rids[d]] / PAGE + 1 - pfx[d];
        const int64_t u = page_cost(dcheap[d]);
        const int64_t sc = stream_start_cost(pfx[d]), cost = len * u + sc, rem = x - start;
        const int64_t o = rem % cost, skip = o > sc ? (o - sc) / u : 0;
        below[e] = pstart[d] + (rem / cost) * len + skip;
        di = d;
        kvh = (int)(rem / cost);
        off = (int)skip;
      }
      int r = decode_rids[di], page = pfx[di] + off;
      dec_waves[8 * w + 0] = di;
      dec_waves[8 * w + 1] = kvh;
      dec_waves[8 * w + 2] = page;
      dec_waves[8 * w + 3] = (int32_t)(below[1] - below[0]);
      dec_waves[8 * w + 4] = r;
      dec_waves[8 * w + 5] = cu_seqlens[r];
      dec_waves[8 * w + 6] = computed[r] + 1;
      dec_waves[8 * w + 7] = bt_pages[bt_off[r] + page];
    }
    free(pstart);
    for (int a = 0; a < nd; ++a)
      if (dshared[a]) dec_seqs[4 * a + 2] |= 1 << 30; /* (members: their own pages) */
    for (int w = 0; w < G; ++w) dec_waves[8 * w + 6] |= dec_seqs[4 * dec_waves[8 * w] + 2] & (1 << 30);
  }
  /* prefix items, groups by leader: for each kv head, chunk c of CP pages and octet q of
   * 8 members, {leader, kvh, page0, page1, member di x 8 (-1 past the group)}; member k
   * of a group: dec_prefix[di] = {P, first item, C | Q << 16, k} */
  for (int di = 0; dec_prefix && di < nd; ++di) /* NULL when dec_prefix_pages is 0 */
    for (int k = 0; k < 8; ++k) dec_prefix[8 * di + k] = 0;
  {
    int item = 0;
    for (int l = 0; l < nd && n_groups > 0; ++l) {
      if (lead[l] != l || pfx[l] == 0) continue;
      const int P = pfx[l];
      int M = 0;
      for (int di = 0; di < nd; ++di) M += lead[di] == l;
      const int Q = (M + 7) / 8, CP = P / 16 > 16 ? (P + 15) / 16 : 16, Cn = (P + CP - 1) / CP;
      int32_t* mem = (int32_t*)malloc(sizeof(int32_t) * 8 * Q);
      for (int k = 0; k < 8 * Q; ++k) mem[k] = -1;
      for (int di = 0, k = 0; di < nd; ++di)
        if (lead[di] == l) {
          dec_prefix[8 * di + 0] = P;
          dec_prefix[8 * di + 1] = item;
          dec_prefix[8 * di + 2] = Cn | (Q << 16);
          dec_prefix[8 * di + 3] = k;
          mem[k++] = di;
        }
      for (int kvh = 0; kvh < 8; ++kvh)
        for (int c = 0; c < Cn; ++c)
          for (int q = 0; q < Q; ++q, ++item) {
            int32_t* it = dec_pre_items + 12 * (int64_t)item;
            it[0] = l;
            it[1] = kvh;
            it[2] = c * CP;
            it[3] = (c + 1) * CP < P ? (c + 1) * CP : P;
            for (int j = 0; j < 8; ++j) it[4 + j] = mem[8 * q + j];
          }
      free(mem);
    }
  }
  free(pfx);
  free(lead);
  free(dshared);
  free(dcheap);
  {
    int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * 4 * (npi > 0 ? npi : 1));
    int k = 0;
    for (int pi = 0; pi < np; ++pi) {
      int r = prefill_rids[pi], q = n_new[r];
      for (int q0 = 0; q0 < q; q0 += pre_tile_q, ++k) {
        int q1 = q0 + pre_tile_q < q ? q0 + pre_tile_q : q;
        tmp[4 * k + 0] = r;
        tmp[4 * k + 1] = q0;
        tmp[4 * k + 2] = q1;
        tmp[4 * k + 3] = computed[r] + q1;
      }
    }
    /* stable sort by n_keys descending: rank = #(greater) + #(equal and earlier) */
    for (int i = 0; i < npi; ++i) {
      int rank = 0;
      for (int j = 0; j < npi; ++j)
        if (tmp[4 * j + 3] > tmp[4 * i + 3] || (tmp[4 * j + 3] == tmp[4 * i + 3] && j < i))
          ++rank;
      memcpy(&pre_items[4 * rank], &tmp[4 * i], 4 * sizeof(int32_t));
    }
    free(tmp);
  }

  meta[0] = T;
  meta[1] = nd;
  meta[2] = np;
  meta[3] = maxq;
  meta[4] = G;
  meta[5] = npi;
  meta[6] = G ? (int32_t)((W + G - 1) / G) : 0;
  meta[7] = bad_page ? 4 : 0;
  meta[9] = (int32_t)total;
  meta[10] = n_pitems;
  meta[11] = n_groups;
  meta[12] = (int32_t)W;
  return meta[7];
}

/* HeadNormRopeKernel (kernels.cu:97-131) + StoreKvKernel (kv_store.cu:48-64):
 * per q/k head: inv = 1/sqrt(mean(x^2) + eps); y = x*inv*w in fp32; rotate-half RoPE
 * on (y_i, y_{i+half}) with cos/sin[pos][i]; one bf16 rounding at the end.  q written
 * back in place; k and raw v appended to the pool at slot_mapping[t]. */
void fqo_qknorm_rope_append(int n_q, int n_kv, int D, int stride, float eps, uint16_t* qkv,
                            const float* wq, const float* wk, const float* cos_tab,
                            const float* sin_tab, int rope_max_pos,
                            const int32_t* positions, const int32_t* slot_mapping, int rows, uint16_t* pool,
                            int64_t pool_pages, int write_k_inplace) {
  int half = D / 2;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; ++t) {
    float x[512], y[512];
    int p = positions[t];
    if (p < 0 || p >= rope_max_pos) continue; /* no table row: the row is left untouched */
    int64_t slot = slot_mapping[t];
    int64_t page = slot / PAGE;
    int tok = (int)(slot % PAGE);
    /* slot >= 0: C division truncates, so slots -15..-1 would give page 0 */
    int page_ok = slot >= 0 && page < pool_pages;
    for (int g = 0; g < n_q + n_kv; ++g) {
      uint16_t* v = qkv + (int64_t)t * stride + (int64_t)g * D;
      const float* w = g < n_q ? wq : wk;
      float ss = 0.f;
      for (int i = 0; i < D; ++i) {
        x[i] = fqo_bf16_to_f32(v[i]);
        ss += x[i] * x[i];
      }
      float inv = 1.0f / sqrtf(ss / (float)D + eps);
      for (int i = 0; i < D; ++i) y[i] = x[i] * inv * w[i];
      uint16_t o[512];
      for (int i = 0; i < half; ++i) {
        float cs = cos_tab[(int64_t)p * half + i], sn = sin_tab[(int64_t)p * half + i];
        o[i] = fqo_f32_to_bf16(y[i] * cs - y[i + half] * sn);
        o[i + half] = fqo_f32_to_bf16(y[i + half] * cs + y[i] * sn);
      }
      if (g < n_q) {
        memcpy(v, o, sizeof(uint16_t) * D);
      } else {
        int kvh = g - n_q;
        if (write_k_inplace) memcpy(v, o, sizeof(uint16_t) * D);
        if (page_ok)
          for (int i = 0; i < D; ++i) pool[fqo_pool_offset(n_kv, D, page, kvh, 0, tok, i)] = o[i];
      }
    }
    if (page_ok)
      for (int kvh = 0; kvh < n_kv; ++kvh) {
        const uint16_t* vv = qkv + (int64_t)t * stride + (int64_t)(n_q + n_kv + kvh) * D;
        for (int i = 0; i < D; ++i) pool[fqo_pool_offset(n_kv, D, page, kvh, 1, tok, i)] = vv[i];
      }
  }
}

/* Gather keys [0, nkeys) of one request's kv head into float rows K[n][D], V[n][D].
 * A page id outside the pool (a batch the pack flags with status 4; the reference reads
 * out of bounds there) reads as zeros: its keys score 0 and add nothing to the output
 * numerator.  This is the path's convention for such pages, kept by both GPU kernels. */
static void gather_kv(int n_kv, int D, const uint16_t* pool, int64_t pool_pages,
                      const int32_t* bt_row, int nkeys, int kvh, float* K, float* V,
                      unsigned char* ok) {
  for (int kp = 0; kp < nkeys; ++kp) {
    int64_t page = bt_row[kp / PAGE];
    ok[kp] = 1;
    if (page < 0 || page >= pool_pages) {
      for (int d = 0; d < D; ++d) K[(int64_t)kp * D + d] = V[(int64_t)kp * D + d] = 0.f;
      continue;
    }
    int tok = kp % PAGE;
    const uint16_t* kb = pool + fqo_pool_offset(n_kv, D, page, kvh, 0, tok, 0);
    const uint16_t* vb = pool + fqo_pool_offset(n_kv, D, page, kvh, 1, 0, 0);
    for (int d = 0; d < D; ++d) {
      K[(int64_t)kp * D + d] = fqo_bf16_to_f32(kb[d]);
      V[(int64_t)kp * D + d] = fqo_bf16_to_f32(vb[d * PAGE + tok]);
    }
  }
}

static float dot_d(const float* a, const float* b, int D) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int d = 0; d < D; d += 8)
    for (int j = 0; j < 8; ++j) acc[j] += a[d + j] * b[d + j];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* softmax(scale * q.K^T over keys [0, nk)) V for one query row; P optionally rounded
 * to bf16 in the numerator (prefill, attn_cute.cu:128) but summed unrounded into l
 * (attn_cute.cu:122-127).  Output 0 when no key contributes (l == 0, attn_cute.cu:141). */
static void attend_row(const float* q, const float* K, const float* V, const unsigned char* ok,
                       int nk, int D, float scale, int round_p, float* s, uint16_t* out,
                       float* absv) {
  float m = -INFINITY;
  for (int k = 0; k < nk; ++k) {
    s[k] = ok[k] ? dot_d(q, K + (int64_t)k * D, D) * scale : -INFINITY;
    if (s[k] > m) m = s[k];
  }
  float acc[512];
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  float l = 0.f;
  if (m > -INFINITY)
    for (int k = 0; k < nk; ++k) {
      if (!ok[k]) continue;
      float p = expf(s[k] - m);
      l += p;
      float pv = round_p ? fqo_bf16_to_f32(fqo_f32_to_bf16(p)) : p;
      const float* vr = V + (int64_t)k * D;
      for (int d = 0; d < D; ++d) acc[d] += pv * vr[d];
    }
  float inv = l > 0.f ? 1.0f / l : 0.f;
  for (int d = 0; d < D; ++d) out[d] = fqo_f32_to_bf16(acc[d] * inv);
  if (absv) { /* sum_k p_k |V_kd| / sum_k p_k, for the rounding allowance of P */
    for (int d = 0; d < D; ++d) absv[d] = 0.f;
    if (m > -INFINITY)
      for (int k = 0; k < nk; ++k) {
        if (!ok[k]) continue;
        float p = expf(s[k] - m);
        const float* vr = V + (int64_t)k * D;
        for (int d = 0; d < D; ++d) absv[d] += p * fabsf(vr[d]);
      }
    for (int d = 0; d < D; ++d) absv[d] *= inv;
  }
}

/* CuteDecodeSplitKernel + CuteDecodeCombineKernel (attn_cute.cu:165-238) without the
 * split: for each qlen==1 request, the 4 query heads of each kv head attend keys
 * [0, pos]; fp32 P (the decode kernel does not round P). */
void fqo_decode(int n_q, int n_kv, int D, int stride, float scale, const uint16_t* qkv,
                const uint16_t* pool, int64_t pool_pages, const int32_t* block_tables,
                int max_blocks, const int32_t* cu_seqlens, const int32_t* positions,
                const int32_t* decode_rids, int n_decode, uint16_t* out) {
  int G = n_q / n_kv;
#pragma omp parallel for schedule(dynamic, 1)
  for (int w = 0; w < n_decode * n_kv; ++w) {
    int di = w / n_kv, kvh = w % n_kv;
    int r = decode_rids[di], row = cu_seqlens[r], nk = positions[row] + 1;
    float* K = (float*)malloc(sizeof(float) * (size_t)nk * D);
    float* V = (float*)malloc(sizeof(float) * (size_t)nk * D);
    float* s = (float*)malloc(sizeof(float) * (size_t)nk);
    unsigned char* ok = (unsigned char*)malloc((size_t)nk);
    gather_kv(n_kv, D, pool, pool_pages, block_tables + (int64_t)r * max_blocks, nk, kvh, K, V,
              ok);
    for (int g = 0; g < G; ++g) {
      int h = kvh * G + g;
      float q[512];
      for (int d = 0; d < D; ++d) q[d] = fqo_bf16_to_f32(qkv[(int64_t)row * stride + h * D + d]);
      attend_row(q, K, V, ok, nk, D, scale, 0, s, out + ((int64_t)row * n_q + h) * D, NULL);
    }
    free(K);
    free(V);
    free(s);
    free(ok);
  }
}

/* CutePrefillKernel (attn_cute.cu:30-147): for each qlen!=1 request and each of its
 * rows i, head h attends keys kpos <= pos[qstart+i] of kv head h/G, cached prefix
 * included; P rounded to bf16 before PV. */
void fqo_prefill(int n_q, int n_kv, int D, int stride, float scale, const uint16_t* qkv,
                 const uint16_t* pool, int64_t pool_pages, const int32_t* block_tables,
                 int max_blocks, const int32_t* cu_seqlens, const int32_t* positions,
                 const int32_t* prefill_rids, int n_prefill, uint16_t* out) {
  fqo_prefill_absv(n_q, n_kv, D, stride, scale, qkv, pool, pool_pages, block_tables,
                   max_blocks, cu_seqlens, positions, prefill_rids, n_prefill, out, NULL);
}

/* fqo_prefill, and (absv non-NULL) per output element sum_k p_k |V_kd| / sum_k p_k with
 * the row's fp32 weights: the scale of the error that rounding P to bf16 can put into an
 * output (each p_k moves by at most 2^-9 relative), for per-element test bounds. */
void fqo_prefill_absv(int n_q, int n_kv, int D, int stride, float scale, const uint16_t* qkv,
                      const uint16_t* pool, int64_t pool_pages, const int32_t* block_tables,
                      int max_blocks, const int32_t* cu_seqlens, const int32_t* positions,
                      const int32_t* prefill_rids, int n_prefill, uint16_t* out,
                      float* absv) {
  int G = n_q / n_kv;
#pragma omp parallel for schedule(dynamic, 1)
  for (int w = 0; w < n_prefill * n_kv; ++w) {
    int pi = w / n_kv, kvh = w % n_kv;
    int r = prefill_rids[pi], qs = cu_seqlens[r], ql = cu_seqlens[r + 1] - qs;
    if (ql <= 0) continue;
    int nk = 0;
    for (int i = 0; i < ql; ++i)
      if (positions[qs + i] + 1 > nk) nk = positions[qs + i] + 1;
    float* K = (float*)malloc(sizeof(float) * (size_t)nk * D);
    float* V = (float*)malloc(sizeof(float) * (size_t)nk * D);
    float* s = (float*)malloc(sizeof(float) * (size_t)nk);
    unsigned char* ok = (unsigned char*)malloc((size_t)nk);
    gather_kv(n_kv, D, pool, pool_pages, block_tables + (int64_t)r * max_blocks, nk, kvh, K, V,
              ok);
    for (int i = 0; i < ql; ++i) {
      int row = qs + i, kv_end = positions[row] + 1;
      for (int g = 0; g < G; ++g) {
        int h = kvh * G + g;
        float q[512];
        for (int d = 0; d < D; ++d) q[d] = fqo_bf16_to_f32(qkv[(int64_t)row * stride + h * D + d]);
        attend_row(q, K, V, ok, kv_end, D, scale, 1, s, out + ((int64_t)row * n_q + h) * D,
                 absv ? absv + ((int64_t)row * n_q + h) * D : NULL);
      }
    }
    free(K);
    free(V);
    free(s);
    free(ok);
  }
}

/* ArgmaxKernel + SampleKernel (kernels.cu:184-327) restated in fp64 for one row each:
 * inv_temp <= 0: index of the largest logit (smallest index among equals);
 * else w_i = exp((l_i - max) * inv_temp); with top_p < 1 the kept set is the fewest
 * largest weights whose mass reaches top_p * sum(w) (weights equal to the smallest kept
 * one included; the reference's 32-step bisection converges to this set); the token is
 * the first index, in vocabulary order, whose running kept mass reaches u * (kept mass),
 * skipping zero weights; the last token when the draw lies past the summed mass.
 * kept_thr[b] / kept_mass[b] (optional) receive the smallest kept weight and the kept
 * mass, so tests can judge a pick that fp32 rounding moved across a boundary. */
static int cmp_desc(const void* a, const void* b) {
  double x = *(const double*)a, y = *(const double*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}
void fqo_sample(const float* logits, int n_rows, int vocab, int64_t stride,
                const float* inv_temp, const float* top_p, const float* u, int32_t* out,
                double* kept_thr, double* kept_mass) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int b = 0; b < n_rows; ++b) {
    const float* lg = logits + (int64_t)b * stride;
    if (inv_temp[b] <= 0.f) {
      /* ArgmaxKernel (kernels.cu:184-214) step by step: 256 threads, thread t scans
       * columns t, t+256, ... keeping the first strict maximum above its start (-1e30,
       * column 0); then the tree reduction keeps the lower slot unless the upper one is
       * strictly larger. */
      float sval[256];
      int sidx[256];
      for (int t = 0; t < 256; ++t) {
        float best = -1e30f;
        int bi = 0;
        for (int i = t; i < vocab; i += 256)
          if (lg[i] > best) {
            best = lg[i];
            bi = i;
          }
        sval[t] = best;
        sidx[t] = bi;
      }
      for (int st = 128; st > 0; st >>= 1)
        for (int t = 0; t < st; ++t)
          if (sval[t + st] > sval[t]) {
            sval[t] = sval[t + st];
            sidx[t] = sidx[t + st];
          }
      out[b] = sidx[0];
      if (kept_thr) kept_thr[b] = 0.0;
      if (kept_mass) kept_mass[b] = 0.0;
      continue;
    }
    double m = -INFINITY;
    for (int i = 0; i < vocab; ++i) if (lg[i] > m) m = lg[i];
    double* w = (double*)malloc(sizeof(double) * (size_t)vocab);
    double z = 0.0;
    for (int i = 0; i < vocab; ++i) {
      w[i] = exp(((double)lg[i] - m) * (double)inv_temp[b]);
      z += w[i];
    }
    double thr = 0.0;
    if (top_p[b] < 1.f) {
      double* s = (double*)malloc(sizeof(double) * (size_t)vocab);
      memcpy(s, w, sizeof(double) * (size_t)vocab);
      qsort(s, (size_t)vocab, sizeof(double), cmp_desc);
      const double need = (double)top_p[b] * z;
      double acc = 0.0;
      thr = s[0];  /* top_p = 0 keeps the largest weight */
      for (int k = 0; k < vocab; ++k) {
        acc += s[k];
        thr = s[k];
        if (acc >= need) break;
      }
      free(s);
    }
    double mass = 0.0;
    for (int i = 0; i < vocab; ++i) if (w[i] >= thr) mass += w[i];
    const double target = (double)u[b] * mass;
    int pick = vocab - 1;
    double acc = 0.0;
    for (int i = 0; i < vocab; ++i) {
      if (w[i] < thr || w[i] <= 0.0) continue;
      acc += w[i];
      if (acc >= target) { pick = i; break; }
    }
    out[b] = pick;
    if (kept_thr) kept_thr[b] = thr;
    if (kept_mass) kept_mass[b] = mass;
    free(w);
  }
}
