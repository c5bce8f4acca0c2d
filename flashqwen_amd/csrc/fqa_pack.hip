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
// the padded block tables.  One launch, no grid-wide synchronisation, no atomics.
// Workgroup 0 alone writes the per-request arrays, `meta`, and checks page ids, so
// each output word has exactly one writer.
#include <climits>

#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kPackThreads = 1024;
constexpr int kPackWaves = kPackThreads / 64;

// Exclusive scan of one value per thread over the workgroup; returns the thread's
// exclusive prefix and the total via *total.  `sh` holds >= kPackWaves values.
template <typename T>
__device__ T block_excl_scan(T v, T* sh, T* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    T y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) sh[w] = x;
  __syncthreads();
  T base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kPackThreads / kWave; ++i) {
    T s = sh[i];
    if (i < w) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

template <typename T, typename Op>
__device__ T block_reduce(T v, T* sh, Op op) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) v = op(v, __shfl_xor(v, d, kWave));
  if (lane == 0) sh[w] = v;
  __syncthreads();
  T r = sh[0];
#pragma unroll
  for (int i = 1; i < kPackThreads / kWave; ++i) r = op(r, sh[i]);
  __syncthreads();
  return r;
}

// The per-request totals of pass 1 (code: min, rows/dpages: saturating sum,
// dmax/qmax: max) reduced together, and the five exclusive scans of pass 2 done
// together.  Small kernels here are bound by instruction fetch (the instruction cache
// starts cold at every dispatch), so these loops are kept rolled: code size, not
// instruction count, sets their latency.
__device__ __forceinline__ int sat_add(int a, int b) {
  long long s = (long long)a + b;
  return s > INT_MAX ? INT_MAX : (int)s;
}

struct Stats {
  int v[5];  // code, rows, dpages, dmax, qmax
};

__device__ __forceinline__ void stats_combine(Stats& a, const Stats& b) {
  a.v[0] = min(a.v[0], b.v[0]);
  a.v[1] = sat_add(a.v[1], b.v[1]);
  a.v[2] = sat_add(a.v[2], b.v[2]);
  a.v[3] = max(a.v[3], b.v[3]);
  a.v[4] = max(a.v[4], b.v[4]);
}

__device__ Stats block_reduce_stats(Stats v, Stats* sh) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
#pragma unroll 1
  for (int d = 1; d < kWave; d <<= 1) {
    Stats o;
#pragma unroll
    for (int k = 0; k < 5; ++k) o.v[k] = __shfl_xor(v.v[k], d, kWave);
    stats_combine(v, o);
  }
  if (lane == 0) sh[w] = v;
  __syncthreads();
  Stats r = sh[0];
#pragma unroll 1
  for (int i = 1; i < kPackWaves; ++i) stats_combine(r, sh[i]);
  __syncthreads();
  return r;
}

struct Counts {
  int v[5];
};

__device__ Counts block_excl_scan5(const Counts& in, Counts* sh, Counts* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  Counts x = in;
#pragma unroll 1
  for (int d = 1; d < kWave; d <<= 1) {
    int y[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) y[k] = __shfl_up(x.v[k], d, kWave);
    if (lane >= d)
#pragma unroll
      for (int k = 0; k < 5; ++k) x.v[k] += y[k];
  }
  if (lane == kWave - 1) sh[w] = x;
  __syncthreads();
  Counts base = {{0, 0, 0, 0, 0}}, tot = {{0, 0, 0, 0, 0}};
#pragma unroll 1
  for (int i = 0; i < kPackWaves; ++i) {
    const Counts s = sh[i];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      if (i < w) base.v[k] += s.v[k];
      tot.v[k] += s.v[k];
    }
  }
  __syncthreads();
  *total = tot;
  Counts out;
#pragma unroll
  for (int k = 0; k < 5; ++k) out.v[k] = base.v[k] + x.v[k] - in.v[k];
  return out;
}

struct MinOp { __device__ int operator()(int a, int b) const { return a < b ? a : b; } };
struct MaxOp { __device__ int operator()(int a, int b) const { return a > b ? a : b; } };
struct SumOp64 {
  __device__ long long operator()(long long a, long long b) const { return a + b; }
};

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

struct PackArgs {
  fqa_batch b;
  fqa_pack_cfg c;
  fqa_pack_out o;
};

__global__ void __launch_bounds__(kPackThreads) pack_kernel(PackArgs a) {
  __shared__ int s_comp[FQA_MAX_REQS];
  __shared__ int s_n[FQA_MAX_REQS];
  __shared__ int s_qstart[FQA_MAX_REQS + 1];
  __shared__ int s_btoff[FQA_MAX_REQS + 1];
  __shared__ int s_decidx[FQA_MAX_REQS + 1];
  __shared__ int s_preidx[FQA_MAX_REQS + 1];
  __shared__ int s_decit[FQA_MAX_REQS + 1];  // exclusive prefix of decode pages
  __shared__ int s_dstart[FQA_MAX_REQS + 1];  // by decode index: 8 * page prefix
  __shared__ int s_dpages[FQA_MAX_REQS];      // by decode index: pages
  __shared__ int s_preit[FQA_MAX_REQS + 1];
  __shared__ Stats s_stats[kPackWaves];
  __shared__ Counts s_counts[kPackWaves];
  __shared__ int sh32[kPackWaves];

  const int tid = threadIdx.x;
  int R = a.b.n_reqs_dev ? *a.b.n_reqs_dev : a.b.n_reqs;
  if (R > a.b.n_reqs) R = a.b.n_reqs;  // the host bound sizes every array
  if (R < 0) R = 0;
  const int QT = a.c.pre_tile_q;
  const int maxb = a.c.max_blocks;

  // ---- pass 1: load, structural checks, totals ---------------------------------
  Stats st = {{INT_MAX, 0, 0, 0, 1}};
  for (int r = tid; r < R; r += kPackThreads) {
    const int c = a.b.computed[r], n = a.b.n_new[r];
    const int o0 = a.b.bt_off[r], o1 = a.b.bt_off[r + 1];
    s_comp[r] = c;
    s_n[r] = n;
    s_btoff[r] = o0;
    int cc = 0;
    if (c < 0 || n < 0) cc = FQA_PACK_NEGATIVE;
    else {
      const int nb = o1 - o0;
      if (nb < cdiv((long long)c + n, kPage)) cc = FQA_PACK_SHORT_TABLE;
      else if (nb > maxb) cc = FQA_PACK_WIDE_TABLE;
      st.v[1] = sat_add(st.v[1], n);
      if (n == 1) {
        const int pg = c / kPage + 1;
        st.v[2] = sat_add(st.v[2], pg);
        st.v[3] = max(pg, st.v[3]);
      } else {
        st.v[4] = max(n, st.v[4]);
      }
    }
    if (cc) st.v[0] = min(st.v[0], cc);
  }
  if (tid == 0) s_btoff[R] = a.b.bt_off[R];
  st = block_reduce_stats(st, s_stats);
  int code = st.v[0];
  const int rows = st.v[1], dpages = st.v[2], qmax = st.v[4];
  if (rows > a.c.max_rows && code > FQA_PACK_ROWS) code = FQA_PACK_ROWS;
  if (code != INT_MAX) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? code : (tid == FQA_META_REQS ? R : 0);
    return;
  }
  const int T = rows;

  // decode plan: W page runs (8 kv heads x pages) cut into G equal shares
  const long long W = 8LL * dpages;
  int G = 0;
  if (W > 0) {
    const int minp = a.c.dec_min_pages > 0 ? a.c.dec_min_pages : 1;
    G = (int)min((long long)a.c.dec_grid_waves, (W + minp - 1) / minp);
  }

  // ---- pass 2: exclusive scans over requests ------------------------------------
  {
    Counts carry = {{0, 0, 0, 0, 0}};
    for (int base = 0; base < R; base += kPackThreads) {
      const int r = base + tid;
      Counts v = {{0, 0, 0, 0, 0}};
      if (r < R) {
        const int n = s_n[r];
        v.v[0] = n;
        v.v[1] = n == 1;
        v.v[2] = n != 1;
        v.v[3] = n == 1 ? s_comp[r] / kPage + 1 : 0;  // pages of a decode stream
        v.v[4] = n != 1 ? (n + QT - 1) / QT : 0;
      }
      Counts tot;
      const Counts e = block_excl_scan5(v, s_counts, &tot);
      if (r < R) {
        s_qstart[r] = carry.v[0] + e.v[0];
        s_decidx[r] = carry.v[1] + e.v[1];
        s_preidx[r] = carry.v[2] + e.v[2];
        s_decit[r] = carry.v[3] + e.v[3];
        s_preit[r] = carry.v[4] + e.v[4];
      }
#pragma unroll
      for (int k = 0; k < 5; ++k) carry.v[k] += tot.v[k];
    }
    if (tid == 0) {
      s_qstart[R] = carry.v[0];
      s_decidx[R] = carry.v[1];
      s_preidx[R] = carry.v[2];
      s_decit[R] = carry.v[3];
      s_preit[R] = carry.v[4];
    }
    __syncthreads();
  }
  const int nd = s_decidx[R], np = s_preidx[R];
  const int npi = s_preit[R];
  if (G > a.c.dec_wave_cap || npi > a.c.pre_item_cap || dpages > INT_MAX / 8) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? FQA_PACK_ITEMS : (tid == FQA_META_REQS ? R : 0);
    return;
  }
  // decode streams by decode index: start of (di, kv head 0) and pages
  for (int r = tid; r < R; r += kPackThreads)
    if (s_n[r] == 1) {
      s_dstart[s_decidx[r]] = 8 * s_decit[r];
      s_dpages[s_decidx[r]] = s_comp[r] / kPage + 1;
    }
  if (tid == 0) s_dstart[nd] = (int)W;
  __syncthreads();
  const int gtid = blockIdx.x * kPackThreads + tid;
  const int gsz = gridDim.x * kPackThreads;

  // ---- rows: positions, request index, slot mapping ------------------------------
  for (int t = gtid; t < T; t += gsz) {
    int r = upper_index(s_qstart, R, t);
    int p = s_comp[r] + (t - s_qstart[r]);
    int page = a.b.bt_pages[s_btoff[r] + p / kPage];
    a.o.positions[t] = p;
    a.o.row_req[t] = r;
    a.o.slot_mapping[t] = page * kPage + p % kPage;
  }
  // ---- padded block tables -------------------------------------------------------
  {
    const long long total = (long long)R * maxb;
    for (long long e = gtid; e < total; e += gsz) {
      int r = (int)(e / maxb), g = (int)(e % maxb);
      int nb = s_btoff[r + 1] - s_btoff[r];
      a.o.block_tables[e] = g < nb ? a.b.bt_pages[s_btoff[r] + g] : -1;
    }
  }
  // ---- decode wave shares: where share w = [w*W/G, (w+1)*W/G) starts ----------------
  for (int w = gtid; w < G; w += gsz) {
    const long long g0 = (long long)w * W / G, g1 = (long long)(w + 1) * W / G;
    const int di = upper_index(s_dstart, nd, (int)g0);
    const int rem = (int)g0 - s_dstart[di], pg = s_dpages[di];
    *reinterpret_cast<int4*>(a.o.dec_waves + 4 * (long long)w) =
        make_int4(di, rem / pg, rem % pg, (int)(g1 - g0));
  }
  for (int r = gtid; r < R; r += gsz)
    if (s_n[r] == 1)
      *reinterpret_cast<int4*>(a.o.dec_seqs + 4 * (long long)s_decidx[r]) =
          make_int4(r, s_qstart[r], s_comp[r] + 1, 8 * s_decit[r]);
  // ---- prefill items, sorted by key count descending (stable) --------------------
  // Tile t of prefill request r covers rows [t*QT, min((t+1)*QT, n)) and needs
  // c + min((t+1)*QT, n) keys, so per request the number of tiles with more keys than X
  // (and with exactly X) has a closed form; an item's rank is a sum over requests.
  for (int i = blockIdx.x + tid * gridDim.x; i < npi; i += gsz) {
    const int r = upper_index(s_preit, R, i);  // the prefill request owning item i
    const int t = i - s_preit[r];
    const int n = s_n[r], c = s_comp[r];
    const int q0 = t * QT, q1 = min(q0 + QT, n);
    const int X = c + q1;
    int rank = 0;
    for (int rr = 0; rr < R; ++rr) {
      const int nt = s_preit[rr + 1] - s_preit[rr];
      if (nt == 0) continue;  // decode request or empty prefill
      const int cc = s_comp[rr], nn = s_n[rr], y = X - cc;
      const int k = y < 0 ? 0 : y / QT;
      rank += (cc + nn > X) + max(0, nt - 1 - k);  // tiles with more keys than X
      // tiles with exactly X keys that come earlier in (request, tile) order
      const int te = (y > 0 && y % QT == 0 && y / QT - 1 < nt - 1) ? y / QT - 1
                     : (cc + nn == X ? nt - 1 : -1);
      if (te >= 0 && (rr < r || (rr == r && te < t))) ++rank;
    }
    *reinterpret_cast<int4*>(a.o.pre_items + 4 * (long long)rank) = make_int4(r, q0, q1, X);
  }

  if (blockIdx.x != 0) return;
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
  // page-id range check over the concatenated tables: 16-byte loads, 4 in flight per
  // thread (the scalar head and tail are the at most 3 ids on either side of alignment)
  int bad = 0;
  {
    const int32_t* pg = a.b.bt_pages + s_btoff[0];
    const int npages = s_btoff[R] - s_btoff[0];
    const int lead = min(npages, (int)(((16 - ((uintptr_t)pg & 15)) & 15) >> 2));
    const int nvec = (npages - lead) >> 2;
    const int4* pv = reinterpret_cast<const int4*>(pg + lead);
    const long long np64 = a.c.pool_pages;
    auto badv = [&](int v) { return v < 0 || (long long)v >= np64; };
    for (int e = tid; e < lead; e += kPackThreads) bad |= badv(pg[e]);
    for (int e = lead + 4 * nvec + tid; e < npages; e += kPackThreads) bad |= badv(pg[e]);
    for (int base = 0; base < nvec; base += 4 * kPackThreads) {
      int4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = base + u * kPackThreads + tid;
        v[u] = e < nvec ? pv[e] : make_int4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) bad |= (int)badv(v[u].x) | (int)badv(v[u].y) | (int)badv(v[u].z) | (int)badv(v[u].w);
    }
  }
  bad = block_reduce(bad, sh32, MaxOp());
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
      default: v = 0;
    }
    a.o.meta[tid] = v;
  }
}

// ---- token-budget selection (Scheduler::BuildBatch, scheduler.cc:116-143) ---------
constexpr int kSchedThreads = 1024;

__global__ void __launch_bounds__(kSchedThreads)
schedule_kernel(const int32_t* __restrict__ num_tokens, const int32_t* __restrict__ computed,
                int R, int budget, int chunk, int32_t* batch_req, int32_t* batch_n,
                int32_t* n_batch) {
  __shared__ int s_rem[FQA_MAX_REQS];
  __shared__ int s_order[FQA_MAX_REQS];
  __shared__ long long s_wsum[kSchedThreads / kWave];
  __shared__ int s_wcnt[kSchedThreads / kWave];
  const int tid = threadIdx.x;
  for (int i = tid; i < R; i += kSchedThreads) s_rem[i] = num_tokens[i] - computed[i];
  __syncthreads();
  // stable sort by remaining ascending: rank = #smaller + #equal-and-earlier
  for (int i = tid; i < R; i += kSchedThreads) {
    int v = s_rem[i], rank = 0;
    for (int j = 0; j < R; ++j) {
      int u = s_rem[j];
      rank += (u < v) || (u == v && j < i);
    }
    s_order[rank] = i;
  }
  __syncthreads();
  // n_k = min(B, S_k) - min(B, S_{k-1}), S = inclusive prefix of per-request caps:
  // the greedy loop's budget bookkeeping in closed form.
  const int lane = tid & (kWave - 1), w = tid >> 6;
  long long carry = 0;
  int ccount = 0;
  for (int base = 0; base < R; base += kSchedThreads) {
    int k = base + tid;
    long long cap = 0;
    int idx = -1;
    if (k < R) {
      idx = s_order[k];
      int rem = s_rem[idx];
      cap = rem <= 0 ? 0 : (rem > 1 && chunk < rem ? chunk : rem);
    }
    long long x = cap;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      long long y = __shfl_up(x, d, kWave);
      if (lane >= d) x += y;
    }
    if (lane == kWave - 1) s_wsum[w] = x;
    __syncthreads();
    long long pre = 0, tot = 0;
    for (int i = 0; i < kSchedThreads / kWave; ++i) {
      if (i < w) pre += s_wsum[i];
      tot += s_wsum[i];
    }
    __syncthreads();
    long long incl = carry + pre + x, excl = incl - cap;
    long long B = budget;
    long long hi = incl < B ? incl : B, lo = excl < B ? excl : B;
    int n = (int)(hi - lo);
    if (B <= 0) n = 0;
    int take = n > 0;
    // compact the chosen requests in sorted order
    int c = take;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      int y = __shfl_up(c, d, kWave);
      if (lane >= d) c += y;
    }
    if (lane == kWave - 1) s_wcnt[w] = c;
    __syncthreads();
    int cpre = 0, ctot = 0;
    for (int i = 0; i < kSchedThreads / kWave; ++i) {
      if (i < w) cpre += s_wcnt[i];
      ctot += s_wcnt[i];
    }
    __syncthreads();
    if (take) {
      int pos = ccount + cpre + c - 1;
      batch_req[pos] = idx;
      batch_n[pos] = n;
    }
    carry += tot;
    ccount += ctot;
  }
  if (tid == 0) *n_batch = ccount;
}

// Gather the chosen running requests into a compact fqa_batch.  Each workgroup
// recomputes the exclusive scan of table lengths, then copies its share of pages.
__global__ void __launch_bounds__(kPackThreads)
gather_kernel(const int32_t* __restrict__ batch_req, const int32_t* __restrict__ batch_n,
              const int32_t* __restrict__ n_batch, int R_bound,
              const int32_t* __restrict__ run_computed, const int32_t* __restrict__ run_bt_off,
              const int32_t* __restrict__ run_bt_pages, int32_t* out_computed,
              int32_t* out_n_new, int32_t* out_bt_off, int32_t* out_bt_pages, int cap) {
  __shared__ int s_off[FQA_MAX_REQS + 1];
  __shared__ int s_src[FQA_MAX_REQS];
  __shared__ int sh32[kPackWaves];
  const int tid = threadIdx.x;
  int R = *n_batch;
  if (R > R_bound) R = R_bound;
  int carry = 0;
  for (int base = 0; base < R; base += kPackThreads) {
    int i = base + tid, len = 0;
    if (i < R) {
      int q = batch_req[i];
      s_src[i] = run_bt_off[q];
      len = run_bt_off[q + 1] - run_bt_off[q];
    }
    int tot;
    int e = block_excl_scan(len, sh32, &tot);
    if (i < R) s_off[i] = carry + e;
    carry += tot;
  }
  if (tid == 0) s_off[R] = carry;
  __syncthreads();
  const int gtid = blockIdx.x * kPackThreads + tid, gsz = gridDim.x * kPackThreads;
  if (blockIdx.x == 0)
    for (int i = tid; i <= R; i += kPackThreads) {
      out_bt_off[i] = s_off[i] < cap ? s_off[i] : cap;
      if (i < R) {
        out_computed[i] = run_computed[batch_req[i]];
        out_n_new[i] = batch_n[i];
      }
    }
  const int total = carry < cap ? carry : cap;
  for (int e = gtid; e < total; e += gsz) {
    int i = upper_index(s_off, R, e);
    out_bt_pages[e] = run_bt_pages[s_src[i] + (e - s_off[i])];
  }
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" {

int fqa_schedule(const int32_t* num_tokens, const int32_t* computed, int32_t n_running,
                 int32_t token_budget, int32_t prefill_chunk, int32_t* batch_req,
                 int32_t* batch_n, int32_t* n_batch, void* stream) {
  if (n_running < 0 || n_running > FQA_MAX_REQS || prefill_chunk < 1 || !n_batch)
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
  int grid = (bt_pages_cap + 4 * kPackThreads - 1) / (4 * kPackThreads);
  grid = grid < 1 ? 1 : (grid > 512 ? 512 : grid);
  hipLaunchKernelGGL(gather_kernel, dim3(grid), dim3(kPackThreads), 0, (hipStream_t)stream,
                     batch_req, batch_n, n_batch, n_running, run_computed, run_bt_off,
                     run_bt_pages, out_computed, out_n_new, out_bt_off, out_bt_pages,
                     bt_pages_cap);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int fqa_pack(const fqa_batch* batch, const fqa_pack_cfg* cfg, const fqa_pack_out* out,
             void* stream) {
  if (!batch || !cfg || !out) return FQA_EINVAL;
  const int R = batch->n_reqs;
  if (R < 0 || R > FQA_MAX_REQS) return FQA_EINVAL;
  if (cfg->max_rows < 0 || cfg->max_blocks < 1 || cfg->pool_pages < 1 ||
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
  long long grid = (work + 2 * kPackThreads - 1) / (2 * kPackThreads);
  grid = grid < 1 ? 1 : (grid > 256 ? 256 : grid);
  PackArgs a{*batch, *cfg, *out};
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
  return cus * 8;  // 2 decode wavefronts per SIMD (the kernel's register budget), 4 SIMDs
}

int32_t fqa_pre_item_bound(int32_t n_reqs, int32_t max_rows, int32_t pre_tile_q) {
  if (n_reqs < 0 || max_rows < 0 || pre_tile_q < 1) return 0;
  return max_rows / pre_tile_q + n_reqs;
}

}  // extern "C"
