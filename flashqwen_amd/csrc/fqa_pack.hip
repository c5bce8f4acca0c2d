// fqa_pack.hip — the GPU pack of one step's ragged batch, and the token-budget
// selection that produces it.
//
// Replaces the host half of the reference step: StepContext::PrepareInputs
// (engine/src/model_runtime.cu:295-302) with UploadRows (:47-52), PackBlockTables
// (:54-64) and SplitDecodePrefill (:66-91), the row generation of Request::EmitChunk
// (scheduler.h:66-72), and the slot arithmetic of StoreKvKernel (kv_store.cu:56-60).
// fqa_schedule restates Scheduler::BuildBatch's selection (scheduler.cc:116-143).
//
// Design: requests per step are few (<= FQA_MAX_REQS) while rows and block-table
// entries are many, so every workgroup of the pack recomputes the per-request scans
// in LDS (a few KB of L2 reads) and then writes its grid-stride share of the rows and
// the padded block tables.  One launch, no grid-wide synchronisation, no global atomics
// (the shared-prefix check hashes page ids with LDS atomics).
// Workgroup 0 alone writes the per-request arrays, `meta`, and checks page ids, so
// each output word has exactly one writer.
#include <climits>

#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kPackThreads = 1024;
constexpr int kPackWaves = kPackThreads / 64;
constexpr int kHashSlots = 2 * FQA_MAX_REQS;  // open addressing, never more than half full

// Workgroup barrier for LDS exchanges: waits for this wave's LDS (and scalar) accesses
// only.  __syncthreads would also wait for every outstanding global load; without that,
// loads issued before a scan stay in flight across it.  No kernel here reads global
// memory another thread of the same launch wrote.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

// Exclusive scan of one int per thread over a kPackThreads workgroup (DPP waves + one LDS
// exchange); the total goes to *total.  `sh` holds >= kPackWaves ints.
__device__ int block_excl_scan(int v, int* sh, int* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v);
  if (lane == kWave - 1) sh[w] = incl;
  lds_sync();
  const int sc = wave_incl_scan(lane < kPackWaves ? sh[lane] : 0);
  *total = __builtin_amdgcn_readlane(sc, kPackWaves - 1);
  const int below = __builtin_amdgcn_readlane(sc, w == 0 ? 0 : w - 1);
  lds_sync();
  return (w == 0 ? 0 : below) + incl - v;
}

// Max over the workgroup (every thread gets it).
__device__ int block_max(int v, int* sh) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  v = wave_extreme<true>(v, INT_MIN);
  if (lane == 0) sh[w] = v;
  lds_sync();
  v = wave_extreme<true>(lane < kPackWaves ? sh[lane] : INT_MIN, INT_MIN);
  lds_sync();
  return v;
}

// The per-request totals of pass 1 and the five exclusive scans of pass 2, each done
// for all values at once with DPP wave primitives (a shuffle-based version spent ~3 us
// per reduction in ds_bpermute latency chains).  Sums are of values the host bounds
// (rows <= max_rows <= 2^20, pages <= max_blocks <= 2^19 per request, <= 2 requests per
// thread); a thread partial that exceeds kPartCap is flagged instead of overflowing.
constexpr int kPartCap = 1 << 20;

struct Stats {
  int v[6];  // code (min), rows (sum), dpages (sum), dmax (max), qmax (max), overflow (max)
};

constexpr int kCounts = 6;
struct Counts {
  int v[kCounts];
};

// Exclusive scans of 5 values over the workgroup (*total gets the 5 sums) and, when
// `stats` (wave-uniform), the reduction of every thread's Stats into *st, in one LDS
// exchange: the wave-level DPP scans and reductions of all 11 values first, then one
// barrier, the second level, and a closing barrier.
__device__ Counts block_scan5_stats(const Counts& in, Counts* total, Stats* st, bool stats,
                                    Counts* shc, Stats* shs) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  Counts incl;
#pragma unroll
  for (int k = 0; k < kCounts; ++k) incl.v[k] = wave_incl_scan(in.v[k]);
  Stats r;
  if (stats) {
    r.v[0] = wave_extreme<false>(st->v[0], INT_MAX);
    r.v[1] = __builtin_amdgcn_readlane(wave_incl_scan(st->v[1]), 63);
    r.v[2] = __builtin_amdgcn_readlane(wave_incl_scan(st->v[2]), 63);
    r.v[3] = wave_extreme<true>(st->v[3], 0);
    r.v[4] = wave_extreme<true>(st->v[4], 1);
    r.v[5] = wave_extreme<true>(st->v[5], 0);
    if (lane == 0) shs[w] = r;
  }
  if (lane == kWave - 1) shc[w] = incl;
  lds_sync();
  const bool have = lane < kPackWaves;
  const Counts o = shc[have ? lane : 0];
  Counts out;
#pragma unroll
  for (int k = 0; k < kCounts; ++k) {
    const int sc = wave_incl_scan(have ? o.v[k] : 0);  // lane i: total of waves 0..i
    total->v[k] = __builtin_amdgcn_readlane(sc, kPackWaves - 1);
    const int below = __builtin_amdgcn_readlane(sc, w == 0 ? 0 : w - 1);
    out.v[k] = (w == 0 ? 0 : below) + incl.v[k] - in.v[k];
  }
  if (stats) {
    const Stats so = shs[have ? lane : 0];
    r.v[0] = wave_extreme<false>(have ? so.v[0] : INT_MAX, INT_MAX);
    r.v[1] = __builtin_amdgcn_readlane(wave_incl_scan(have ? so.v[1] : 0), 63);
    r.v[2] = __builtin_amdgcn_readlane(wave_incl_scan(have ? so.v[2] : 0), 63);
    r.v[3] = wave_extreme<true>(have ? so.v[3] : 0, 0);
    r.v[4] = wave_extreme<true>(have ? so.v[4] : 1, 1);
    r.v[5] = wave_extreme<true>(have ? so.v[5] : 0, 0);
    *st = r;
  }
  lds_sync();
  return out;
}

__device__ __forceinline__ int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// Largest i in [0, n] with a[i] <= x (a non-decreasing, a[0] <= x).
__device__ __forceinline__ int upper_index(const int* a, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The decode wavefronts of a step whose decode runs beside its prefill (fqa.h,
// dec_share); INT_MAX when the plan is left as it is.
__device__ int dec_share_waves(int N, long long dpages, unsigned long long keyrows) {
  constexpr int kStep = FQA_DEC_SHARE_STEP;
  if (keyrows == 0 || dpages <= 0 || N < 2 * kStep || N > 4096) return INT_MAX;
  unsigned long long D = (unsigned long long)FQA_DEC_SHARE_RATE * (unsigned long long)dpages;
  unsigned long long P = keyrows;
  while (D >= (1ull << 30) || P >= (1ull << 30)) {
    D >>= 1;
    P >>= 1;
  }
  const unsigned long long n = (unsigned long long)N;
  // decode(G) ~ D (36 G + 25 N) / (50 G), prefill(G) ~ P N / (N - G)
  // prefill no slower than decode at G (true at small G, false past the crossing)
  auto ok = [&](int G) {
    const unsigned long long g = (unsigned long long)G;
    return 50 * P * n * g <= D * (36 * g + 25 * n) * (n - g);
  };
  const int top = (N - kStep) / kStep * kStep;
  int lo = kStep, hi = top;
  if (!ok(lo)) return lo;
  while (lo < hi) {  // largest multiple of kStep in [kStep, top] with ok()
    const int mid = (lo + hi + kStep) / (2 * kStep) * kStep;
    if (ok(mid)) lo = mid; else hi = mid - kStep;
  }
  // one step further when the prefill there ends before the decode does at lo
  const unsigned long long g = (unsigned long long)lo;
  if (lo + kStep <= top && 50 * P * n * g < D * (36 * g + 25 * n) * (n - g - kStep))
    lo += kStep;
  return lo;
}

// A decode stream's start in the plan's cost units (fqa.h): FQA_DEC_STREAM_COST, plus
// FQA_DEC_PREFIX_STREAM_COST for a shared-prefix member (its stream always leaves a
// partial for the combine).
__host__ __device__ constexpr int stream_start_cost(int prefix_pages) {
  return FQA_DEC_STREAM_COST + (prefix_pages > 0 ? FQA_DEC_PREFIX_STREAM_COST : 0);
}

struct PackArgs {
  fqa_batch b;
  fqa_pack_cfg c;
  fqa_pack_out o;
};

// ---- shared-prefix groups (fqa_pack_cfg::dec_prefix_pages, fqa.h) ----------------------
// Two launches before the pack.  prefix_lcp_kernel, one workgroup per request: a decode
// request whose first page id (>= 0) starts another decode request too finds its group's
// leader (the smallest such request index) and the length of its common run of leading
// page ids with the leader's table (capped at FQA_DEC_PREFIX_CAP and at computed / 16),
// into dec_prefix[r][4] (-1 for every other request) and the leader into [r][5].
// prefix_plan_kernel, one workgroup: each group's prefix P (the smallest of its members'),
// the groups that reach dec_prefix_pages, their items, and per request its P
// (dec_prefix[r][6], which the pack reads with the other per-request values).
constexpr int kLcpThreads = 256;

__global__ void __launch_bounds__(kLcpThreads) prefix_lcp_kernel(PackArgs a) {
  __shared__ int s_lead, s_cnt, s_mis;
  const int r = blockIdx.x, tid = threadIdx.x;
  int R = a.b.n_reqs_dev ? *a.b.n_reqs_dev : a.b.n_reqs;
  R = min(max(R, 0), a.b.n_reqs);
  if (r >= R) return;
  if (tid == 0) {
    s_lead = INT_MAX;
    s_cnt = 0;
    s_mis = INT_MAX;
  }
  const int n = a.b.n_new[r], c = a.b.computed[r], o0 = a.b.bt_off[r], o1 = a.b.bt_off[r + 1];
  // the pack reports malformed requests; here they only stay out of every group
  const bool dec = n == 1 && c >= 0 && o0 >= 0 && o1 > o0;
  const int f = dec ? a.b.bt_pages[o0] : -1;
  __syncthreads();
  int q = -1, lead = -1;
  if (f >= 0) {  // uniform
    for (int j = tid; j < R; j += kLcpThreads) {
      const int nj = a.b.n_new[j], oj = a.b.bt_off[j], oj1 = a.b.bt_off[j + 1];
      const int cj = a.b.computed[j];
      const int fj = (nj == 1 && cj >= 0 && oj >= 0 && oj1 > oj) ? a.b.bt_pages[oj] : -1;
      if (fj == f) {
        atomicMin(&s_lead, j);
        atomicAdd(&s_cnt, 1);
      }
    }
    __syncthreads();
    if (s_cnt >= 2) {  // uniform
      const int L = s_lead;
      const int pages = min(c / kPage + 1, o1 - o0);
      int lcp;
      if (L == r) {
        lcp = pages;
      } else {
        const int ol = a.b.bt_off[L], ol1 = a.b.bt_off[L + 1];
        const int cmp = min(min(pages, min(a.b.computed[L] / kPage + 1, ol1 - ol)),
                            FQA_DEC_PREFIX_CAP);
        for (int base = 0; base < cmp; base += 4 * kLcpThreads) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int k = base + 4 * tid + e;
            if (k < cmp && a.b.bt_pages[o0 + k] != a.b.bt_pages[ol + k]) atomicMin(&s_mis, k);
          }
          __syncthreads();
          if (s_mis < cmp) break;  // uniform
        }
        lcp = min(s_mis, cmp);
      }
      q = min(min(lcp, FQA_DEC_PREFIX_CAP), c / kPage);
      lead = L;
    }
  }
  if (tid == 0) {
    a.o.dec_prefix[8LL * r + 4] = q;
    a.o.dec_prefix[8LL * r + 5] = lead;
  }
}

__global__ void __launch_bounds__(kPackThreads) prefix_plan_kernel(PackArgs a) {
  __shared__ int s_q[FQA_MAX_REQS], s_lead[FQA_MAX_REQS], s_di[FQA_MAX_REQS];
  __shared__ int s_gmin[FQA_MAX_REQS], s_gcnt[FQA_MAX_REQS], s_gbase[FQA_MAX_REQS];
  __shared__ int s_goff[FQA_MAX_REQS], s_mem[FQA_MAX_REQS], s_glist[FQA_MAX_REQS + 1];
  __shared__ int sh[kPackWaves];
  const int tid = threadIdx.x;
  int R = a.b.n_reqs_dev ? *a.b.n_reqs_dev : a.b.n_reqs;
  R = min(max(R, 0), a.b.n_reqs);
  const int minp = a.c.dec_prefix_pages;
  constexpr int kPasses = FQA_MAX_REQS / kPackThreads;
  // per request: its LCP result, leader, and decode index (exclusive scan of n == 1)
  int carry = 0;
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int r = pass * kPackThreads + tid;
    int isdec = 0;
    if (r < R) {
      const int q = a.o.dec_prefix[8LL * r + 4];
      s_q[r] = q;
      s_lead[r] = a.o.dec_prefix[8LL * r + 5];
      isdec = a.b.n_new[r] == 1;
      s_gmin[r] = INT_MAX;
      s_gcnt[r] = 0;
    }
    int tot;
    const int e = block_excl_scan(isdec, sh, &tot);
    if (r < R) s_di[r] = isdec ? carry + e : -1;
    carry += tot;
  }
  lds_sync();
  for (int r = tid; r < R; r += kPackThreads)
    if (s_q[r] >= 0) {
      atomicMin(&s_gmin[s_lead[r]], s_q[r]);
      atomicAdd(&s_gcnt[s_lead[r]], 1);
    }
  lds_sync();
  // per leader (request order): items and members of its group if it is used
  int carry_items = 0, carry_mem = 0, carry_groups = 0;
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int r = pass * kPackThreads + tid;
    int items = 0, mem = 0, grp = 0;
    if (r < R && s_q[r] >= 0 && s_lead[r] == r && s_gmin[r] >= minp) {
      const int P = s_gmin[r], M = s_gcnt[r];
      const int CP = P / 16 > 16 ? (P + 15) / 16 : 16;
      items = 8 * ((P + CP - 1) / CP) * ((M + 7) / 8);
      mem = M;
      grp = 1;
    }
    int ti, tm, tg;
    const int ei = block_excl_scan(items, sh, &ti);
    const int em = block_excl_scan(mem, sh, &tm);
    const int eg = block_excl_scan(grp, sh, &tg);
    if (r < R) {
      s_gbase[r] = carry_items + ei;
      s_goff[r] = carry_mem + em;
      if (grp) s_glist[carry_groups + eg] = r;
    }
    carry_items += ti;
    carry_mem += tm;
    carry_groups += tg;
  }
  const bool use = carry_groups > 0 && carry_items <= a.c.dec_pre_cap;
  const int n_items = use ? carry_items : 0, n_groups = use ? carry_groups : 0;
  lds_sync();
  // each member's rank in its group (members by request index = by decode index) and P
  for (int r = tid; r < R; r += kPackThreads) {
    const int L = s_lead[r];
    int P = 0;
    if (use && s_q[r] >= 0 && s_gmin[L] >= minp) {
      P = s_gmin[L];
      int k = 0;
      for (int j = L; j < r; ++j) k += s_q[j] >= 0 && s_lead[j] == L;
      s_mem[s_goff[L] + k] = s_di[r];
      const int M = s_gcnt[L], CP = P / 16 > 16 ? (P + 15) / 16 : 16;
      const int C = (P + CP - 1) / CP, Q = (M + 7) / 8;
      *reinterpret_cast<int4*>(a.o.dec_prefix + 8LL * s_di[r]) =
          make_int4(P, s_gbase[L], C | (Q << 16), k);
    } else if (s_di[r] >= 0) {
      *reinterpret_cast<int4*>(a.o.dec_prefix + 8LL * s_di[r]) = make_int4(0, 0, 0, 0);
    }
    a.o.dec_prefix[8LL * r + 6] = P;
  }
  if (tid == 0) {
    s_glist[n_groups] = INT_MAX;
    a.o.dec_prefix[7] = n_items | (n_groups << 20);
  }
  lds_sync();
  // the items: group (binary search over the groups' first items), then kv head, chunk,
  // octet
  for (int i = tid; i < n_items; i += kPackThreads) {
    int lo = 0, hi = n_groups - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_gbase[s_glist[mid]] <= i) lo = mid; else hi = mid - 1;
    }
    const int L = s_glist[lo], P = s_gmin[L], M = s_gcnt[L];
    const int CP = P / 16 > 16 ? (P + 15) / 16 : 16;
    const int C = (P + CP - 1) / CP, Q = (M + 7) / 8;
    const int local = i - s_gbase[L];
    const int qd = local % Q, ch = (local / Q) % C, kvh = local / (Q * C);
    int m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = 8 * qd + j < M ? s_mem[s_goff[L] + 8 * qd + j] : -1;
    int4* dst = reinterpret_cast<int4*>(a.o.dec_pre_items + 12LL * i);
    dst[0] = make_int4(s_di[L], kvh, ch * CP, min((ch + 1) * CP, P));
    dst[1] = make_int4(m[0], m[1], m[2], m[3]);
    dst[2] = make_int4(m[4], m[5], m[6], m[7]);
  }
}

__global__ void __launch_bounds__(kPackThreads) pack_kernel(PackArgs a) {
  __shared__ int s_comp[FQA_MAX_REQS];
  __shared__ int s_n[FQA_MAX_REQS];
  __shared__ int s_qstart[FQA_MAX_REQS + 1];
  __shared__ int s_btoff[FQA_MAX_REQS + 1];
  __shared__ int s_decidx[FQA_MAX_REQS + 1];
  __shared__ int s_preidx[FQA_MAX_REQS + 1];
  __shared__ int s_dstart[FQA_MAX_REQS + 1];  // by decode index: 8 * cost prefix
  __shared__ int s_dpages[FQA_MAX_REQS];      // by decode index: stream pages
  __shared__ int s_dpfx[FQA_MAX_REQS];        // by decode index: shared-prefix pages
  __shared__ int s_dpst[FQA_MAX_REQS + 1];    // by decode index: 8 * stream page prefix
  __shared__ int s_drid[FQA_MAX_REQS];        // by decode index: request
  __shared__ int s_dflag[FQA_MAX_REQS];       // by decode index: first page id, then the flag
  __shared__ int s_prer[FQA_MAX_REQS];        // by prefill index: request
  __shared__ int s_pit[FQA_MAX_REQS + 1];     // by prefill index: first item
  __shared__ int s_hkey[kHashSlots];          // first page ids of decode sequences
  __shared__ int s_hcnt[kHashSlots / 2];      // ... how many sequences start there (16 bits)
  __shared__ int s_hmin[kHashSlots];          // ... and the first of them (decode index)
  __shared__ Stats s_stats[kPackWaves];
  __shared__ Counts s_counts[kPackWaves];
  __shared__ int sh32[kPackWaves];
  __shared__ unsigned long long s_keyrows;  // prefill key-rows: sum n*c + n(n+1)/2

  const int tid = threadIdx.x;
  int R = a.b.n_reqs_dev ? *a.b.n_reqs_dev : a.b.n_reqs;
  if (R > a.b.n_reqs) R = a.b.n_reqs;  // the host bound sizes every array
  if (R < 0) R = 0;
  const int QT = a.c.pre_tile_q;
  const int maxb = a.c.max_blocks;
  // the shared-prefix hash starts empty (published by the scan's barriers)
  for (int i = tid; i < kHashSlots; i += kPackThreads) {
    s_hkey[i] = -1;
    if (i < kHashSlots / 2) s_hcnt[i] = 0;
    s_hmin[i] = INT_MAX;
  }
  if (tid == 0) s_keyrows = 0;

  // ---- per request: load, structural checks, totals, and the five exclusive scans
  // (rows, decode / prefill indices, decode pages, prefill items), one pass per 1024
  // requests; the totals are reduced with the last pass's scans -------------------------
  Stats st = {{INT_MAX, 0, 0, 0, 1, 0}};
  Counts carry = {{0, 0, 0, 0, 0, 0}};
  const int bt_end = a.b.bt_off[R];  // issued with the first loads, not after the scans
  for (int base = 0; base < R; base += kPackThreads) {
    const int r = base + tid;
    Counts v = {{0, 0, 0, 0, 0, 0}};
    // Loads at a clamped index, not under the lane condition: a conditional load is
    // waited for where its value merges with the default.
    const int rc = r < R ? r : R - 1;
    int c = a.b.computed[rc], n = a.b.n_new[rc], o0 = a.b.bt_off[rc];
    const int o1 = a.b.bt_off[rc + 1];
    // a decode sequence's first page id, for the shared-prefix check below (in flight
    // across the scan's barriers; other lanes re-read their own table offset)
    const int first = *(n == 1 && o0 >= 0 && o1 > o0 ? a.b.bt_pages + o0 : a.b.bt_off + rc);
    // pages of its shared prefix (prefix_plan_kernel), which its decode streams skip
    int pfx = a.c.dec_prefix_pages > 0 ? a.o.dec_prefix[8LL * rc + 6] : 0;
    if (r >= R) c = n = o0 = pfx = 0;
    if (r < R) {
      int cc = 0;
      if (c < 0 || n < 0) cc = FQA_PACK_NEGATIVE;
      else {
        const int nb = o1 - o0;
        if (nb < cdiv((long long)c + n, kPage)) cc = FQA_PACK_SHORT_TABLE;
        else if (nb > maxb) cc = FQA_PACK_WIDE_TABLE;
        st.v[1] = min(st.v[1] + min(n, kPartCap), kPartCap + 1);
        if (n == 1) {
          const int pg = c / kPage + 1 - pfx;
          st.v[2] = min(st.v[2] + min(pg, kPartCap), kPartCap + 1);
          st.v[3] = max(pg, st.v[3]);
        } else {
          st.v[4] = max(n, st.v[4]);
        }
      }
      if (cc) st.v[0] = min(st.v[0], cc);
      v.v[0] = n;
      v.v[1] = n == 1;
      v.v[2] = n != 1;
      // a decode stream's cost in the plan: its pages plus the per-stream overhead (more
      // for a shared-prefix member), and its pages; the shared sequences' cheaper pages
      // are taken off once the flags are known
      v.v[3] = n == 1 ? (c / kPage + 1 - pfx) * FQA_DEC_PAGE_COST + stream_start_cost(pfx) : 0;
      v.v[5] = n == 1 ? c / kPage + 1 - pfx : 0;
      v.v[4] = n != 1 ? (n + QT - 1) / QT : 0;
    }
    const bool last = base + kPackThreads >= R;
    if (last) st.v[5] = st.v[2] > kPartCap;
    Counts tot;
    const Counts e = block_scan5_stats(v, &tot, &st, last, s_counts, s_stats);
    if (r < R) {
      s_comp[r] = c;
      s_n[r] = n;
      s_btoff[r] = o0;
      const int qs = carry.v[0] + e.v[0], di = carry.v[1] + e.v[1];
      const int pi = carry.v[2] + e.v[2];
      s_qstart[r] = qs;
      s_decidx[r] = di;
      s_preidx[r] = pi;
      if (n == 1) {
        s_dstart[di] = 8 * (carry.v[3] + e.v[3]);
        s_dpst[di] = 8 * (carry.v[5] + e.v[5]);
        s_dpages[di] = c / kPage + 1 - pfx;
        s_dpfx[di] = pfx;
        s_drid[di] = r;
        s_dflag[di] = first;
      } else {
        s_prer[pi] = r;
        s_pit[pi] = carry.v[4] + e.v[4];
        if (a.c.dec_share && n > 0 && c >= 0)
          atomicAdd(&s_keyrows, (unsigned long long)n * (unsigned long long)c +
                                    (unsigned long long)n * (n + 1) / 2);
      }
    }
#pragma unroll
    for (int k = 0; k < kCounts; ++k) carry.v[k] += tot.v[k];
  }
  const int nd = carry.v[1], np = carry.v[2], npi = carry.v[4];
  // decode plan: W = 8 x (stream costs) cost units cut into G equal shares
  const int dpages = st.v[2];
  long long W = 8LL * carry.v[3];
  if (tid == 0) {
    s_btoff[R] = bt_end;
    s_qstart[R] = carry.v[0];
    s_decidx[R] = nd;
    s_preidx[R] = np;
    s_dstart[nd] = (int)W;
    s_dpst[nd] = 8 * dpages;
    s_pit[np] = npi;
  }
  lds_sync();
  int code = st.v[0];
  const int rows = st.v[1], qmax = st.v[4];
  if (rows > a.c.max_rows && code > FQA_PACK_ROWS) code = FQA_PACK_ROWS;
  if (code == INT_MAX && st.v[5]) code = FQA_PACK_ITEMS;  // decode pages beyond the plan's range
  if (code != INT_MAX) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? code : (tid == FQA_META_REQS ? R : 0);
    return;
  }
  // ---- decode sequences whose first page starts another decode sequence too (a shared
  // prefix): FQA_DEC_SHARED in their n_keys fields.  Page ids are hashed into LDS. -------
  auto slot_of = [](int id) { return (int)(((uint32_t)id * 2654435761u) >> 20) & (kHashSlots - 1); };
  if (nd > 1) {
    for (int d = tid; d < nd; d += kPackThreads) {
      const int id = s_dflag[d];
      if (id < 0) continue;  // not a page (flagged by the range check): never shared
      int h = slot_of(id);
      for (int probe = 0; probe < kHashSlots; ++probe, h = (h + 1) & (kHashSlots - 1)) {
        const int prev = atomicCAS(&s_hkey[h], -1, id);
        if (prev == -1 || prev == id) {
          atomicAdd(&s_hcnt[h >> 1], 1 << (16 * (h & 1)));  // counts <= 2048
          atomicMin(&s_hmin[h], d);
          break;
        }
      }
    }
    lds_sync();
  }
  // kCheap (beside FQA_DEC_SHARED in s_dflag, never stored): a shared sequence that is not
  // the first with its first page; its pages cost FQA_DEC_SHARED_PAGE_COST in the plan
  constexpr int kCheap = 1 << 29;
  for (int d = tid; d < nd; d += kPackThreads) {
    const int id = s_dflag[d];
    int shared = 0, first = d;
    if (id >= 0 && nd > 1) {
      int h = slot_of(id);
      for (int probe = 0; probe < kHashSlots; ++probe, h = (h + 1) & (kHashSlots - 1))
        if (s_hkey[h] == id) {
          shared = ((s_hcnt[h >> 1] >> (16 * (h & 1))) & 0xFFFF) > 1;
          first = s_hmin[h];
          break;
        }
    }
    // a group member's streams cover its own pages: no flag
    const bool fl = shared && s_dpfx[d] == 0;
    s_dflag[d] = fl ? (FQA_DEC_SHARED | (first != d ? kCheap : 0)) : 0;
  }
  // the cheap sequences' pages cost FQA_DEC_SHARED_PAGE_COST: take the difference off the
  // cost prefix (each thread rescans its own decode indices, which it flagged above)
  bool any_cheap = false;
  for (int d = tid; d < nd; d += kPackThreads) any_cheap |= (s_dflag[d] & kCheap) != 0;
  if (__syncthreads_or(any_cheap)) {
    int off = 0;
    for (int base = 0; base < nd; base += kPackThreads) {
      const int d = base + tid;
      const int v = d < nd && (s_dflag[d] & kCheap)
                        ? s_dpages[d] * (FQA_DEC_PAGE_COST - FQA_DEC_SHARED_PAGE_COST) : 0;
      int tot;
      const int e = block_excl_scan(v, sh32, &tot);
      if (d < nd) s_dstart[d] -= 8 * (off + e);
      off += tot;
    }
    W -= 8LL * off;
    if (tid == 0) s_dstart[nd] = (int)W;
    lds_sync();
  }


  const int T = rows;
  const int gtid = blockIdx.x * kPackThreads + tid;
  const int gsz = gridDim.x * kPackThreads;
  int G = 0;
  if (W > 0) {
    const int minp = a.c.dec_min_pages > 0 ? a.c.dec_min_pages : 1;
    // shares of at least FQA_DEC_PAGE_COST * minp units: each holds the last position of
    // a page of every stream it crosses
    const long long unit = (long long)FQA_DEC_PAGE_COST * minp;
    G = (int)min((long long)a.c.dec_grid_waves, (W + unit - 1) / unit);
    if (a.c.dec_share)  // CUs shared with a concurrent prefill (fqa.h)
      G = min(G, dec_share_waves(a.c.dec_grid_waves, dpages, s_keyrows));
  }
  if (G > a.c.dec_wave_cap || npi > a.c.pre_item_cap || W > INT_MAX) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? FQA_PACK_ITEMS : (tid == FQA_META_REQS ? R : 0);
    return;
  }

  // ---- the first iteration's page-id loads of rows, decode waves and block tables go
  // out together; the LDS-only work below (shared-prefix hash, item ranks) runs while
  // they are in flight, and their stores follow -------------------------------------------
  auto row_of = [&](int t, int& r, int& p) {
    r = upper_index(s_qstart, R, t);
    p = s_comp[r] + (t - s_qstart[r]);
  };
  // Cost position x lies in stream (d, h) at offset off: the stream's first
  // stream_start_cost positions are its overhead, then u per page (fqa.h).  Pages whose
  // last position is below x:
  auto locate = [&](int x, int& d, int& h, int& skip) {
    d = upper_index(s_dstart, nd, x);
    if (d >= nd) {  // x == W
      h = skip = 0;
      return dpages * 8;
    }
    const int sc = stream_start_cost(s_dpfx[d]);
    const int u = (s_dflag[d] & kCheap) ? FQA_DEC_SHARED_PAGE_COST : FQA_DEC_PAGE_COST;
    const int rem = x - s_dstart[d], cost = s_dpages[d] * u + sc;
    h = rem / cost;
    skip = max(0, rem % cost - sc) / u;  // pages of stream (d, h) before x
    return s_dpst[d] + h * s_dpages[d] + skip;
  };
  auto wave_of = [&](int w, int& di, int& kvh, int& page, int& n, int& r) {
    const int g0 = (int)((long long)w * W / G), g1 = (int)((long long)(w + 1) * W / G);
    int skip, d1, h1, s1;
    const int p0 = locate(g0, di, kvh, skip);
    n = locate(g1, d1, h1, s1) - p0;
    page = s_dpfx[di] + skip;
    r = s_drid[di];
  };
  auto bt_of = [&](int e, int& r, int& g) {
    r = e / maxb;
    g = e - r * maxb;
  };
  auto store_row = [&](int t, int r, int p, int page) {
    a.o.positions[t] = p;
    a.o.row_req[t] = r;
    a.o.slot_mapping[t] = page * kPage + p % kPage;
  };
  auto store_wave = [&](int w, int di, int kvh, int page, int n, int r, int id) {
    int4* dst = reinterpret_cast<int4*>(a.o.dec_waves + 8 * (long long)w);
    dst[0] = make_int4(di, kvh, page, n);
    dst[1] = make_int4(r, s_qstart[r], (s_comp[r] + 1) | (s_dflag[di] & FQA_DEC_SHARED), id);
  };
  const int bt_total = R * maxb;  // < 2^31: R <= 2048, max_blocks <= 2^19
  int r0 = 0, p0 = 0, page0 = 0, di1 = 0, kvh1 = 0, pg1 = 0, n1 = 0, r1 = 0, id1 = 0, bt0 = -1;
  if (gtid < T) {
    row_of(gtid, r0, p0);
    page0 = a.b.bt_pages[s_btoff[r0] + p0 / kPage];
  }
  if (gtid < G) {
    wave_of(gtid, di1, kvh1, pg1, n1, r1);
    id1 = a.b.bt_pages[s_btoff[r1] + pg1];
  }
  if (gtid < bt_total) {
    int r, g;
    bt_of(gtid, r, g);
    if (g < s_btoff[r + 1] - s_btoff[r]) bt0 = a.b.bt_pages[s_btoff[r] + g];
  }
  // workgroup 0: the first chunk of the page-id range check (16-byte loads, kPgVec per
  // thread; the scalar head and tail are the at most 3 ids on either side of 16-byte
  // alignment), checked at the end
  constexpr int kPgVec = 12;
  const int32_t* pg = a.b.bt_pages + s_btoff[0];
  const int npages = s_btoff[R] - s_btoff[0];
  const int pg_lead = min(npages, (int)(((16 - ((uintptr_t)pg & 15)) & 15) >> 2));
  const int pg_nvec = (npages - pg_lead) >> 2;
  const int pg_ntail = npages - pg_lead - 4 * pg_nvec;
  const int4* pgv_src = reinterpret_cast<const int4*>(pg + pg_lead);
  // Unconditional loads at clamped indices (a load under a lane condition would be
  // waited for where its value merges with the default); slots past the end are masked
  // where they are checked.
  int4 pgv[kPgVec];
  int pg_head_id = 0, pg_tail_id = 0;
  if (blockIdx.x == 0 && npages > 0) {
#pragma unroll
    for (int u = 0; u < kPgVec; ++u)
      pgv[u] = pgv_src[max(min(u * kPackThreads + tid, pg_nvec - 1), 0)];
    pg_head_id = pg[min(tid, npages - 1)];
    pg_tail_id = pg[max(min(pg_lead + 4 * pg_nvec + tid, npages - 1), 0)];
  }

  // ---- prefill items, sorted by key count descending (stable) --------------------
  // Tile t of prefill request r covers rows [t*QT, min((t+1)*QT, n)) and needs
  // c + min((t+1)*QT, n) keys, so per request the number of tiles with more keys than X
  // (and with exactly X) has a closed form; an item's rank is a sum over the prefill
  // requests.  A group of S lanes (S = np rounded up to a power of two, at most 64) per
  // item, its lanes splitting the prefill requests; QT is a power of two.
  {
    const int lane = tid & (kWave - 1), wv = tid >> 6;
    const int S = np >= 64 ? 64 : (np <= 1 ? 1 : 1 << (32 - __builtin_clz(np - 1)));
    const int per_wave = kWave / S, sub = lane / S, sl = lane % S;
    const int qsh = QT == 32 ? 5 : (QT == 64 ? 6 : 7);
    const int stride = gridDim.x * kPackWaves * per_wave;
    for (int i0 = (blockIdx.x * kPackWaves + wv) * per_wave; i0 < npi; i0 += stride) {
      const int i = i0 + sub;
      const bool live = i < npi;
      const int k = live ? upper_index(s_pit, np, i) : 0;  // the prefill owning item i
      const int r = s_prer[k];
      const int t = i - s_pit[k];
      const int n = s_n[r], c = s_comp[r];
      const int q0 = t * QT, q1 = min(q0 + QT, n);
      const int X = c + q1;
      int rank = 0;
      for (int kk = sl; kk < np && live; kk += S) {
        const int nt = s_pit[kk + 1] - s_pit[kk];
        if (nt == 0) continue;  // empty prefill
        const int rr = s_prer[kk];
        const int cc = s_comp[rr], nn = s_n[rr], y = X - cc;
        const int kq = y < 0 ? 0 : y >> qsh;
        rank += (cc + nn > X) + max(0, nt - 1 - kq);  // tiles with more keys than X
        // tiles with exactly X keys that come earlier in (request, tile) order
        const int te = (y > 0 && (y & (QT - 1)) == 0 && (y >> qsh) - 1 < nt - 1) ? (y >> qsh) - 1
                       : (cc + nn == X ? nt - 1 : -1);
        if (te >= 0 && (kk < k || (kk == k && te < t))) ++rank;
      }
      for (int m = 1; m < S; m <<= 1) rank += __shfl_xor(rank, m, kWave);
      if (live && sl == 0)
        *reinterpret_cast<int4*>(a.o.pre_items + 4 * (long long)rank) = make_int4(r, q0, q1, X);
    }
  }
  lds_sync();  // the decode flags are complete

  // ---- stores of the first iteration, then the rest of the grid-stride loops ---------
  if (gtid < T) store_row(gtid, r0, p0, page0);
  if (gtid < G) store_wave(gtid, di1, kvh1, pg1, n1, r1, id1);
  if (gtid < bt_total) a.o.block_tables[gtid] = bt0;
  for (int t = gtid + gsz; t < T; t += gsz) {
    int r, p;
    row_of(t, r, p);
    store_row(t, r, p, a.b.bt_pages[s_btoff[r] + p / kPage]);
  }
  for (int w = gtid + gsz; w < G; w += gsz) {
    int di, kvh, page, n, r;
    wave_of(w, di, kvh, page, n, r);
    store_wave(w, di, kvh, page, n, r, a.b.bt_pages[s_btoff[r] + page]);
  }
  for (int e = gtid + gsz; e < bt_total; e += gsz) {
    int r, g;
    bt_of(e, r, g);
    const int nb = s_btoff[r + 1] - s_btoff[r];
    a.o.block_tables[e] = g < nb ? a.b.bt_pages[s_btoff[r] + g] : -1;
  }
  for (int di = gtid; di < nd; di += gsz) {
    const int r = s_drid[di];
    *reinterpret_cast<int4*>(a.o.dec_seqs + 4 * (long long)di) =
        make_int4(r, s_qstart[r], (s_comp[r] + 1) | (s_dflag[di] & FQA_DEC_SHARED), s_dstart[di]);
  }

  if (blockIdx.x != 0) return;
  // the shared-prefix item and group counts (prefix_plan_kernel)
  const int pre_counts = a.c.dec_prefix_pages > 0 ? a.o.dec_prefix[7] : 0;
  // ---- workgroup 0: per-request arrays, meta, page-range check -------------------
  for (int r = tid; r <= R; r += kPackThreads) {
    a.o.cu_seqlens[r] = s_qstart[r];
    if (r < R) {
      int n = s_n[r];
      a.o.qlen[r] = n;
      // decode / prefill lists: slot i holds the i-th request of the class
      if (n == 1) a.o.decode_rids[s_decidx[r]] = r;
      else a.o.prefill_rids[s_preidx[r]] = r;
    }
  }
  for (int i = tid; i < R; i += kPackThreads) {
    if (i >= nd) a.o.decode_rids[i] = -1;
    if (i >= np) a.o.prefill_rids[i] = -1;
  }
  // page-id range check over the concatenated tables: the first chunk was loaded before
  // the hash and the item ranks
  int bad = 0;
  {
    const long long np64 = a.c.pool_pages;
    auto badv = [&](int v) { return v < 0 || (long long)v >= np64; };
    if (npages > 0) {
      bad |= (int)(tid < pg_lead && badv(pg_head_id)) | (int)(tid < pg_ntail && badv(pg_tail_id));
#pragma unroll
      for (int u = 0; u < kPgVec; ++u)
        if (u * kPackThreads + tid < pg_nvec)
          bad |= (int)badv(pgv[u].x) | (int)badv(pgv[u].y) | (int)badv(pgv[u].z) |
                 (int)badv(pgv[u].w);
    }
    for (int base = kPgVec * kPackThreads; base < pg_nvec; base += kPgVec * kPackThreads) {
      int4 v[kPgVec];
#pragma unroll
      for (int u = 0; u < kPgVec; ++u) {
        const int e = base + u * kPackThreads + tid;
        v[u] = e < pg_nvec ? pgv_src[e] : make_int4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kPgVec; ++u)
        bad |= (int)badv(v[u].x) | (int)badv(v[u].y) | (int)badv(v[u].z) | (int)badv(v[u].w);
    }
  }
  bad = block_max(bad, sh32);
  if (tid < FQA_META_LEN) {
    int v = 0;
    switch (tid) {
      case FQA_META_ROWS: v = T; break;
      case FQA_META_N_DECODE: v = nd; break;
      case FQA_META_N_PREFILL: v = np; break;
      case FQA_META_MAX_QLEN: v = qmax; break;
      case FQA_META_DEC_WAVES: v = G; break;
      case FQA_META_PRE_ITEMS: v = npi; break;
      case FQA_META_DEC_WAVE_PAGES: v = G ? (int)((W + G - 1) / G) : 0; break;
      case FQA_META_STATUS: v = bad ? FQA_PACK_PAGE_RANGE : FQA_PACK_OK; break;
      case FQA_META_REQS: v = R; break;
      case FQA_META_DEC_PAGES: v = (int)dpages; break;
      case FQA_META_DEC_PRE_ITEMS: v = pre_counts & 0xFFFFF; break;
      case FQA_META_DEC_GROUPS: v = pre_counts >> 20; break;
      case FQA_META_DEC_COST: v = (int)W; break;
      default: v = 0;
    }
    a.o.meta[tid] = v;
  }
}

// ---- token-budget selection (Scheduler::BuildBatch, scheduler.cc:116-143) ---------
constexpr int kSchedThreads = 1024;

// LDS of the selection.
struct SelectLds {
  long long key[FQA_MAX_REQS];  // (remaining << 32) | index: distinct, in the sort's order
  int rem[FQA_MAX_REQS];
  int rank[FQA_MAX_REQS];
  int order[FQA_MAX_REQS];
  int req[FQA_MAX_REQS];  // chosen requests, in batch order
  int n[FQA_MAX_REQS];    // ... and their rows
  int wsum[kSchedThreads / kWave];
  int wcnt[kSchedThreads / kWave];
};

// The selection of one step by a whole kSchedThreads workgroup, into sl.req / sl.n;
// returns the number of chosen requests (every thread).  Stable sort of the running
// requests by remaining ascending: rank(i) = #smaller + #equal-and-earlier, i.e. the
// number of smaller (remaining, index) keys, the R^2 comparisons spread over every thread
// of the workgroup (parts of the j range per i, summed with LDS atomics).  Then n_k = min(B, S_k) - min(B, S_{k-1}) with S the
// inclusive prefix of the per-request caps in sorted order: the greedy loop's budget
// bookkeeping in closed form.
__device__ int select_batch(const int32_t* __restrict__ num_tokens,
                            const int32_t* __restrict__ computed, int R, int budget, int chunk,
                            SelectLds& sl) {
  const int tid = threadIdx.x;
  for (int i = tid; i < R; i += kSchedThreads) {
    const int rem = num_tokens[i] - computed[i];
    sl.rem[i] = rem;
    sl.key[i] = (long long)((unsigned long long)(long long)rem << 32) | (unsigned)i;
    sl.rank[i] = 0;
  }
  lds_sync();
  {
    // rank(i) = #{j : key_j < key_i}: one 64-bit compare per pair, the keys of a wave's
    // j range read as LDS broadcasts
    const int parts = R > 0 && R < kSchedThreads ? kSchedThreads / R : 1;
    const int span = (R + parts - 1) / parts;
    for (int t = tid; t < R * parts; t += kSchedThreads) {
      const int i = t % R, p = t / R;
      const long long v = sl.key[i];
      const int j1 = min(R, (p + 1) * span);
      int cnt = 0;
#pragma unroll 8
      for (int j = p * span; j < j1; ++j) cnt += sl.key[j] < v;
      if (cnt) atomicAdd(&sl.rank[i], cnt);
    }
  }
  lds_sync();
  for (int i = tid; i < R; i += kSchedThreads) sl.order[sl.rank[i]] = i;
  lds_sync();
  // Only min(B, S) matters, so the prefix is taken with saturating adds at B + 1
  // (B <= 2^24 keeps every sum in int).
  const int lane = tid & (kWave - 1), w = tid >> 6;
  const int B = budget > 0 ? budget : 0, cap1 = B + 1;
  auto sat = [cap1](int x, int y) { const int s = x + y; return s < cap1 ? s : cap1; };
  int carry = 0;
  int ccount = 0;
  for (int base = 0; base < R; base += kSchedThreads) {
    const int k = base + tid;
    int cap = 0, idx = -1;
    if (k < R) {
      idx = sl.order[k];
      const int rem = sl.rem[idx];
      cap = rem <= 0 ? 0 : (rem > 1 && chunk < rem ? chunk : rem);
      cap = cap < cap1 ? cap : cap1;
    }
    int x = cap;
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowShr1, 0xf, 0xf, true));
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowShr2, 0xf, 0xf, true));
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowShr4, 0xf, 0xf, true));
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowShr8, 0xf, 0xf, true));
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowBcast15, 0xa, 0xf, false));
    x = sat(x, __builtin_amdgcn_update_dpp(0, x, kDppRowBcast31, 0xc, 0xf, false));
    if (lane == kWave - 1) sl.wsum[w] = x;
    lds_sync();
    int pre = carry;  // saturating prefix of the earlier waves
    for (int i = 0; i < w; ++i) pre = sat(pre, sl.wsum[i]);
    int tot = carry;
    for (int i = 0; i < kSchedThreads / kWave; ++i) tot = sat(tot, sl.wsum[i]);
    lds_sync();
    // exclusive prefix = the previous lane's saturated inclusive prefix (wave_shr:1)
    const int xe = __builtin_amdgcn_update_dpp(0, x, kDppWaveShr1, 0xf, 0xf, true);
    const int incl = sat(pre, x), excl = sat(pre, xe);
    const int hi = incl < B ? incl : B, lo = excl < B ? excl : B;
    const int n = hi - lo;
    const int take = n > 0;
    // compact the chosen requests in sorted order
    const int c = wave_incl_scan(take);
    if (lane == kWave - 1) sl.wcnt[w] = c;
    lds_sync();
    int cpre = 0, ctot = 0;
    for (int i = 0; i < kSchedThreads / kWave; ++i) {
      if (i < w) cpre += sl.wcnt[i];
      ctot += sl.wcnt[i];
    }
    if (take) {
      const int pos = ccount + cpre + c - 1;
      sl.req[pos] = idx;
      sl.n[pos] = n;
    }
    lds_sync();
    carry = tot;
    ccount += ctot;
  }
  return ccount;
}

__global__ void __launch_bounds__(kSchedThreads)
schedule_kernel(const int32_t* __restrict__ num_tokens, const int32_t* __restrict__ computed,
                int R, int budget, int chunk, int32_t* batch_req, int32_t* batch_n,
                int32_t* n_batch) {
  __shared__ SelectLds sl;
  const int cnt = select_batch(num_tokens, computed, R, budget, chunk, sl);
  for (int i = threadIdx.x; i < cnt; i += kSchedThreads) {
    batch_req[i] = sl.req[i];
    batch_n[i] = sl.n[i];
  }
  if (threadIdx.x == 0) *n_batch = cnt;
}

// Gather the chosen running requests into a compact fqa_batch.  Each workgroup
// recomputes the exclusive scan of table lengths, then copies its share of pages.
// kSelect: the workgroup first makes the selection itself (select_batch, the same in
// every workgroup) instead of reading fqa_schedule's, and workgroup 0 writes it out.
struct GatherArgs {
  const int32_t* num_tokens;  // kSelect: the running requests' token counts
  int budget, chunk;
  int32_t* batch_req;  // kSelect: written; else read
  int32_t* batch_n;
  int32_t* n_batch;
  int R_bound;
  const int32_t* run_computed;
  const int32_t* run_bt_off;
  const int32_t* run_bt_pages;
  int32_t* out_computed;
  int32_t* out_n_new;
  int32_t* out_bt_off;
  int32_t* out_bt_pages;
  int cap;
};

template <bool kSelect>
__global__ void __launch_bounds__(kPackThreads) gather_kernel(GatherArgs a) {
  static_assert(kPackThreads == kSchedThreads, "one workgroup size");
  __shared__ int s_off[FQA_MAX_REQS + 1];
  __shared__ int s_src[FQA_MAX_REQS];
  __shared__ int sh32[kPackWaves];
  __shared__ SelectLds sl;
  const int tid = threadIdx.x;
  int R;
  if constexpr (kSelect) {
    R = select_batch(a.num_tokens, a.run_computed, a.R_bound, a.budget, a.chunk, sl);
    if (blockIdx.x == 0) {
      for (int i = tid; i < R; i += kPackThreads) {
        a.batch_req[i] = sl.req[i];
        a.batch_n[i] = sl.n[i];
      }
      if (tid == 0) *a.n_batch = R;
    }
  } else {
    R = *a.n_batch;
    if (R > a.R_bound) R = a.R_bound;
  }
  auto req_of = [&](int i) { return kSelect ? sl.req[i] : a.batch_req[i]; };
  auto n_of = [&](int i) { return kSelect ? sl.n[i] : a.batch_n[i]; };
  int carry = 0;
  for (int base = 0; base < R; base += kPackThreads) {
    int i = base + tid, len = 0;
    if (i < R) {
      int q = req_of(i);
      s_src[i] = a.run_bt_off[q];
      len = a.run_bt_off[q + 1] - a.run_bt_off[q];
    }
    int tot;
    int e = block_excl_scan(len, sh32, &tot);
    if (i < R) s_off[i] = carry + e;
    carry += tot;
  }
  if (tid == 0) s_off[R] = carry;
  lds_sync();
  const int gtid = blockIdx.x * kPackThreads + tid, gsz = gridDim.x * kPackThreads;
  if (blockIdx.x == 0)
    for (int i = tid; i <= R; i += kPackThreads) {
      a.out_bt_off[i] = s_off[i] < a.cap ? s_off[i] : a.cap;
      if (i < R) {
        a.out_computed[i] = a.run_computed[req_of(i)];
        a.out_n_new[i] = n_of(i);
      }
    }
  const int total = carry < a.cap ? carry : a.cap;
  for (int e = gtid; e < total; e += gsz) {
    int i = upper_index(s_off, R, e);
    a.out_bt_pages[e] = a.run_bt_pages[s_src[i] + (e - s_off[i])];
  }
}

int gather_grid(int cap) {
  int grid = (cap + 4 * kPackThreads - 1) / (4 * kPackThreads);
  return grid < 1 ? 1 : (grid > 512 ? 512 : grid);
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" {

int fqa_schedule(const int32_t* num_tokens, const int32_t* computed, int32_t n_running,
                 int32_t token_budget, int32_t prefill_chunk, int32_t* batch_req,
                 int32_t* batch_n, int32_t* n_batch, void* stream) {
  if (n_running < 0 || n_running > FQA_MAX_REQS || prefill_chunk < 1 ||
      token_budget > (1 << 24) || !n_batch)
    return FQA_EINVAL;
  if (n_running > 0 && (!num_tokens || !computed || !batch_req || !batch_n)) return FQA_EINVAL;
  hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(kSchedThreads), 0, (hipStream_t)stream,
                     num_tokens, computed, n_running, token_budget, prefill_chunk, batch_req,
                     batch_n, n_batch);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int fqa_gather_batch(const int32_t* batch_req, const int32_t* batch_n, const int32_t* n_batch,
                     int32_t n_running, const int32_t* run_computed, const int32_t* run_bt_off,
                     const int32_t* run_bt_pages, int32_t* out_computed, int32_t* out_n_new,
                     int32_t* out_bt_off, int32_t* out_bt_pages, int32_t bt_pages_cap,
                     void* stream) {
  if (n_running < 0 || n_running > FQA_MAX_REQS || bt_pages_cap < 0) return FQA_EINVAL;
  if (!batch_req || !batch_n || !n_batch || !run_computed || !run_bt_off || !out_computed ||
      !out_n_new || !out_bt_off || (bt_pages_cap > 0 && (!run_bt_pages || !out_bt_pages)))
    return FQA_EINVAL;
  GatherArgs a{nullptr, 0, 0, const_cast<int32_t*>(batch_req), const_cast<int32_t*>(batch_n),
               const_cast<int32_t*>(n_batch), n_running, run_computed, run_bt_off, run_bt_pages,
               out_computed, out_n_new, out_bt_off, out_bt_pages, bt_pages_cap};
  hipLaunchKernelGGL(gather_kernel<false>, dim3(gather_grid(bt_pages_cap)), dim3(kPackThreads),
                     0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int fqa_schedule_gather(const int32_t* num_tokens, const int32_t* run_computed,
                        int32_t n_running, int32_t token_budget, int32_t prefill_chunk,
                        const int32_t* run_bt_off, const int32_t* run_bt_pages,
                        int32_t* batch_req, int32_t* batch_n, int32_t* n_batch,
                        int32_t* out_computed, int32_t* out_n_new, int32_t* out_bt_off,
                        int32_t* out_bt_pages, int32_t bt_pages_cap, void* stream) {
  if (n_running < 0 || n_running > FQA_MAX_REQS || prefill_chunk < 1 ||
      token_budget > (1 << 24) || bt_pages_cap < 0 || !n_batch || !run_bt_off ||
      !out_bt_off)
    return FQA_EINVAL;
  if (n_running > 0 && (!num_tokens || !run_computed || !batch_req || !batch_n ||
                        !out_computed || !out_n_new))
    return FQA_EINVAL;
  if (bt_pages_cap > 0 && (!run_bt_pages || !out_bt_pages)) return FQA_EINVAL;
  GatherArgs a{num_tokens, token_budget, prefill_chunk, batch_req, batch_n, n_batch, n_running,
               run_computed, run_bt_off, run_bt_pages, out_computed, out_n_new, out_bt_off,
               out_bt_pages, bt_pages_cap};
  hipLaunchKernelGGL(gather_kernel<true>, dim3(gather_grid(bt_pages_cap)), dim3(kPackThreads),
                     0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int fqa_pack(const fqa_batch* batch, const fqa_pack_cfg* cfg, const fqa_pack_out* out,
             void* stream) {
  if (!batch || !cfg || !out) return FQA_EINVAL;
  const int R = batch->n_reqs;
  if (R < 0 || R > FQA_MAX_REQS) return FQA_EINVAL;
  if (cfg->max_rows < 0 || cfg->max_rows > (1 << 20) || cfg->max_blocks < 1 ||
      cfg->max_blocks > (1 << 19) || cfg->pool_pages < 1 ||
      cfg->dec_wave_cap < 0 || cfg->pre_item_cap < 0 || cfg->dec_grid_waves < 1)
    return FQA_EINVAL;
  if (cfg->pre_tile_q != 32 && cfg->pre_tile_q != 64 && cfg->pre_tile_q != 128)
    return FQA_EINVAL;
  if (!batch->bt_off || !out->meta || !out->cu_seqlens || !out->dec_seqs) return FQA_EINVAL;
  if (R > 0 && (!batch->computed || !batch->n_new || !batch->bt_pages || !out->qlen ||
                !out->block_tables || !out->decode_rids || !out->prefill_rids))
    return FQA_EINVAL;
  if (cfg->max_rows > 0 && (!out->positions || !out->row_req || !out->slot_mapping))
    return FQA_EINVAL;
  if ((cfg->dec_wave_cap > 0 && !out->dec_waves) || (cfg->pre_item_cap > 0 && !out->pre_items))
    return FQA_EINVAL;
  long long work = (long long)R * cfg->max_blocks;
  if (cfg->max_rows > work) work = cfg->max_rows;
  long long grid = (work + kPackThreads - 1) / kPackThreads;
  grid = grid < 1 ? 1 : (grid > 256 ? 256 : grid);
  if (cfg->dec_prefix_pages < 0 || (cfg->dec_prefix_pages > 0 && cfg->dec_pre_cap < 0))
    return FQA_EINVAL;
  if (cfg->dec_prefix_pages > 0 && (!out->dec_prefix || (cfg->dec_pre_cap > 0 && !out->dec_pre_items)))
    return FQA_EINVAL;
  PackArgs a{*batch, *cfg, *out};
  if (cfg->dec_prefix_pages > 0 && R > 0) {
    hipLaunchKernelGGL(prefix_lcp_kernel, dim3((unsigned)R), dim3(kLcpThreads), 0,
                       (hipStream_t)stream, a);
    hipLaunchKernelGGL(prefix_plan_kernel, dim3(1), dim3(kPackThreads), 0, (hipStream_t)stream,
                       a);
  }
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)grid), dim3(kPackThreads), 0,
                     (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int32_t fqa_dec_wave_bound(int32_t n_reqs, int32_t dec_grid_waves) {
  (void)n_reqs;
  return dec_grid_waves > 0 ? dec_grid_waves : 0;
}

int32_t fqa_dec_default_waves(int32_t device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    return 0;
  return cus * 4;  // one decode wavefront per SIMD, 4 SIMDs per CU
}

int32_t fqa_pre_item_bound(int32_t n_reqs, int32_t max_rows, int32_t pre_tile_q) {
  if (n_reqs < 0 || max_rows < 0 || pre_tile_q < 1) return 0;
  return max_rows / pre_tile_q + n_reqs;
}

}  // extern "C"
