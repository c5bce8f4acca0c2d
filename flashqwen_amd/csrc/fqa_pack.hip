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

constexpr int kPackThreads = 256;

// Exclusive scan of one value per thread over a 256-thread workgroup; returns the
// thread's exclusive prefix and the total via *total.  `sh` holds >= 4 ints.
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
  __shared__ int s_decit[FQA_MAX_REQS + 1];
  __shared__ int s_preit[FQA_MAX_REQS + 1];
  __shared__ long long sh64[4];
  __shared__ int sh32[4];

  const int tid = threadIdx.x;
  int R = a.b.n_reqs_dev ? *a.b.n_reqs_dev : a.b.n_reqs;
  if (R > a.b.n_reqs) R = a.b.n_reqs;  // the host bound sizes every array
  if (R < 0) R = 0;
  const int QT = a.c.pre_tile_q;
  const int maxb = a.c.max_blocks;

  // ---- pass 1: load, structural checks, totals ---------------------------------
  int code = INT_MAX;
  long long rows = 0, dpages = 0;
  int dmax = 0, qmax = 1;
  for (int r = tid; r < R; r += kPackThreads) {
    int c = a.b.computed[r], n = a.b.n_new[r];
    int o0 = a.b.bt_off[r], o1 = a.b.bt_off[r + 1];
    s_comp[r] = c;
    s_n[r] = n;
    s_btoff[r] = o0;
    int cc = 0;
    if (c < 0 || n < 0) cc = FQA_PACK_NEGATIVE;
    else {
      int nb = o1 - o0;
      if (nb < cdiv((long long)c + n, kPage)) cc = FQA_PACK_SHORT_TABLE;
      else if (nb > maxb) cc = FQA_PACK_WIDE_TABLE;
      rows += n;
      if (n == 1) {
        int pg = c / kPage + 1;
        dpages += pg;
        dmax = pg > dmax ? pg : dmax;
      } else if (n > qmax) {
        qmax = n;
      }
    }
    if (cc && cc < code) code = cc;
  }
  if (tid == 0) s_btoff[R] = a.b.bt_off[R];
  code = block_reduce(code, sh32, MinOp());
  rows = block_reduce(rows, sh64, SumOp64());
  dpages = block_reduce(dpages, sh64, SumOp64());
  dmax = block_reduce(dmax, sh32, MaxOp());
  qmax = block_reduce(qmax, sh32, MaxOp());
  if (rows > a.c.max_rows && code > FQA_PACK_ROWS) code = FQA_PACK_ROWS;
  if (code != INT_MAX) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? code : (tid == FQA_META_REQS ? R : 0);
    return;
  }
  const int T = (int)rows;

  // decode split size (pages per work item)
  int S;
  if (a.c.dec_target_items <= 0) S = dmax > 0 ? dmax : 1;
  else {
    int mins = a.c.dec_min_split > 0 ? a.c.dec_min_split : 1;
    long long s = (dpages + a.c.dec_target_items - 1) / a.c.dec_target_items;
    S = s > mins ? (int)s : mins;
  }

  // ---- pass 2: exclusive scans over requests ------------------------------------
  {
    int cq = 0, cd = 0, cp = 0, cdi = 0, cpi = 0;
    for (int base = 0; base < R; base += kPackThreads) {
      int r = base + tid;
      int n = 0, isd = 0, isp = 0, di = 0, pi = 0;
      if (r < R) {
        n = s_n[r];
        isd = n == 1;
        isp = !isd;
        di = isd ? cdiv(s_comp[r] / kPage + 1, S) : 0;
        pi = isp ? cdiv(n, QT) : 0;
      }
      int t0, t1, t2, t3, t4;
      int e0 = block_excl_scan(n, sh32, &t0);
      int e1 = block_excl_scan(isd, sh32, &t1);
      int e2 = block_excl_scan(isp, sh32, &t2);
      int e3 = block_excl_scan(di, sh32, &t3);
      int e4 = block_excl_scan(pi, sh32, &t4);
      if (r < R) {
        s_qstart[r] = cq + e0;
        s_decidx[r] = cd + e1;
        s_preidx[r] = cp + e2;
        s_decit[r] = cdi + e3;
        s_preit[r] = cpi + e4;
      }
      cq += t0; cd += t1; cp += t2; cdi += t3; cpi += t4;
    }
    if (tid == 0) {
      s_qstart[R] = cq;
      s_decidx[R] = cd;
      s_preidx[R] = cp;
      s_decit[R] = cdi;
      s_preit[R] = cpi;
    }
    __syncthreads();
  }
  const int nd = s_decidx[R], np = s_preidx[R];
  const int ndi = s_decit[R], npi = s_preit[R];
  if (ndi > a.c.dec_item_cap || npi > a.c.pre_item_cap) {
    if (blockIdx.x == 0 && tid < FQA_META_LEN)
      a.o.meta[tid] = tid == FQA_META_STATUS ? FQA_PACK_ITEMS : (tid == FQA_META_REQS ? R : 0);
    return;
  }

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
  // ---- decode items: one thread per decode sequence ------------------------------
  for (int r = gtid; r < R; r += gsz) {
    if (s_n[r] != 1) continue;
    int pages = s_comp[r] / kPage + 1;
    int it = s_decit[r];
    for (int s = 0; s * S < pages; ++s, ++it) {
      int pe = (s + 1) * S < pages ? (s + 1) * S : pages;
      int4 v = make_int4(r, s, s * S, pe);
      *reinterpret_cast<int4*>(a.o.dec_items + 4 * (long long)it) = v;
    }
  }
  // ---- prefill items, sorted by key count descending (stable) --------------------
  for (int i = gtid; i < npi; i += gsz) {
    // locate item i: request r with s_preit[r] <= i < s_preit[r+1] and prefill
    int r = upper_index(s_preit, R, i);
    int t = i - s_preit[r];
    int n = s_n[r], c = s_comp[r];
    int q0 = t * QT, q1 = q0 + QT < n ? q0 + QT : n;
    int nk = c + q1;
    int rank = 0;
    for (int rr = 0; rr < R; ++rr) {
      int nn = s_n[rr];
      if (nn == 1 || nn == 0) continue;
      int cc = s_comp[rr], nt = cdiv(nn, QT), j0 = s_preit[rr];
      for (int tt = 0; tt < nt; ++tt) {
        int qq1 = (tt + 1) * QT < nn ? (tt + 1) * QT : nn;
        int k = cc + qq1;
        rank += (k > nk) || (k == nk && j0 + tt < i);
      }
    }
    *reinterpret_cast<int4*>(a.o.pre_items + 4 * (long long)rank) = make_int4(r, q0, q1, nk);
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
      if (n == 1) a.o.dec_item_start[s_decidx[r]] = s_decit[r];
    }
  }
  for (int i = tid; i < R; i += kPackThreads) {
    if (i >= nd) a.o.decode_rids[i] = -1;
    if (i >= np) a.o.prefill_rids[i] = -1;
  }
  for (int i = tid; i <= R; i += kPackThreads) {
    if (i == nd) a.o.dec_item_start[i] = ndi;
    else if (i > nd) a.o.dec_item_start[i] = -1;
  }
  int bad = 0;
  const int npages = s_btoff[R] - s_btoff[0];
  for (int e = tid; e < npages; e += kPackThreads) {
    int v = a.b.bt_pages[s_btoff[0] + e];
    bad |= v < 0 || (long long)v >= a.c.pool_pages;
  }
  bad = block_reduce(bad, sh32, MaxOp());
  if (tid < FQA_META_LEN) {
    int v = 0;
    switch (tid) {
      case FQA_META_ROWS: v = T; break;
      case FQA_META_N_DECODE: v = nd; break;
      case FQA_META_N_PREFILL: v = np; break;
      case FQA_META_MAX_QLEN: v = qmax; break;
      case FQA_META_DEC_ITEMS: v = ndi; break;
      case FQA_META_PRE_ITEMS: v = npi; break;
      case FQA_META_SPLIT_PAGES: v = S; break;
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
  __shared__ int sh32[4];
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
      cfg->dec_item_cap < 0 || cfg->pre_item_cap < 0)
    return FQA_EINVAL;
  if (cfg->pre_tile_q != 32 && cfg->pre_tile_q != 64 && cfg->pre_tile_q != 128)
    return FQA_EINVAL;
  if (!batch->bt_off || !out->meta || !out->cu_seqlens || !out->dec_item_start) return FQA_EINVAL;
  if (R > 0 && (!batch->computed || !batch->n_new || !batch->bt_pages || !out->qlen ||
                !out->block_tables || !out->decode_rids || !out->prefill_rids))
    return FQA_EINVAL;
  if (cfg->max_rows > 0 && (!out->positions || !out->row_req || !out->slot_mapping))
    return FQA_EINVAL;
  if ((cfg->dec_item_cap > 0 && !out->dec_items) || (cfg->pre_item_cap > 0 && !out->pre_items))
    return FQA_EINVAL;
  long long work = (long long)R * cfg->max_blocks;
  if (cfg->max_rows > work) work = cfg->max_rows;
  long long grid = (work + 4 * kPackThreads - 1) / (4 * kPackThreads);
  grid = grid < 1 ? 1 : (grid > 256 ? 256 : grid);
  PackArgs a{*batch, *cfg, *out};
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)grid), dim3(kPackThreads), 0,
                     (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int32_t fqa_dec_item_bound(int32_t n_reqs, int32_t dec_target_items) {
  if (n_reqs < 0) return 0;
  return dec_target_items > 0 ? dec_target_items + n_reqs : n_reqs;
}

int32_t fqa_pre_item_bound(int32_t n_reqs, int32_t max_rows, int32_t pre_tile_q) {
  if (n_reqs < 0 || max_rows < 0 || pre_tile_q < 1) return 0;
  return max_rows / pre_tile_q + n_reqs;
}

}  // extern "C"
