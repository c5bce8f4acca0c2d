// fqa_rope_append.hip — fused per-head QK-RMSNorm + rotate-half RoPE + paged KV append.
//
// Replaces HeadNormRopeKernel (engine/src/kernels.cu:97-131, launched :133-139) and
// StoreKvKernel (engine/src/kv_store.cu:48-75), which the reference runs as two
// launches with one 128-thread block per (row, head) and one bf16 element per thread.
//
// W = 10/HPG wavefronts per row (HPG = heads per 16-lane group, a template parameter the
// host picks from the row count: few rows want many waves, many rows want each wave to
// amortise its load latency over more heads).  The 4 16-lane groups of wave s take heads
// g + 4*(s*HPG + i), i < HPG, with every load issued before any math and cos/sin and the
// norm weights loaded once: lane j holds dims [4j, 4j+4) and [64+4j, 64+4j+4), so both
// halves of every rotate-half pair sit in one lane and RoPE needs no data exchange; the
// sum of squares is a 16-lane butterfly.  q is written back in place, k into its page.
// V goes into the V^T [dim][16 tokens] rows of the page.  When 16 consecutive rows fill
// one page (every full page of a prefill), the page's 16 rows share its V^T: row tok
// reads 2 dims x 8 tokens per lane of kv head tok/2's half tok%2 (64 dims of 16 rows),
// transposes in registers (v_perm) and stores 16-byte pieces of V^T rows, so each row
// moves 1 KiB of V and the page goes out as contiguous 16-byte stores.  Rows of a partly
// filled page (decode rows, the ends of a chunk) write their column with 2-byte stores,
// split over the W waves; those must meet in one L2 before the line goes to HBM:
// workgroup b runs on XCD b % 8 and rows are dealt to XCDs in contiguous ranges, so a
// page's rows (except where a range ends) go through the same XCD's L2.
// Memory-bound: per row 12 KiB read, 8 KiB (q) + 4 KiB (k, v) written.
//
// fqa_qkv_proj_append runs the same kernel on the QKV projection's split-K partials
// (kPart): a row's values are the sum of the fp32 partials in split order, rounded to
// bf16 exactly as the projection's own reduction would round them, so the results match
// fqa_gemm + fqa_qknorm_rope_append bit for bit without the bf16 qkv round trip.
//
#include "fqa_common.h"
#include "fqa_append_math.h"
#include "fqa_gemm_internal.h"

namespace fqa {
namespace {

constexpr int kWavesPerBlock = 4;

struct AppendArgs {
  uint16_t* qkv;
  const float* wq;
  const float* wk;
  const float* cos_tab;
  const float* sin_tab;
  int rope_max_pos;
  const int32_t* positions;
  const int32_t* slots;
  const int32_t* meta;
  uint16_t* pool;
  long long pool_pages;
  int stride;
  float eps;
  int write_k;
  int blocks_per_xcd;
  // fused with the QKV projection: the row's qkv values are the sum of `splits` fp32
  // partials part[s][row][col] (row stride pstride, plane stride plane), rounded to bf16
  const float* part;
  int splits;
  int pstride;
  long long plane;
  int part_rows;
};

// The row's 4 (load4) or 2 (load2) qkv values from column col on, as packed bf16: from the
// qkv buffer, or (kPart) summed over the split partials in split order and rounded, the
// values the projection's own reduction writes.
template <bool kPart>
__device__ __forceinline__ uint2 load4(const AppendArgs& a, long long row, int col) {
  if constexpr (kPart) {
    const float* p = a.part + row * a.pstride + col;
    float4 s = *reinterpret_cast<const float4*>(p);
    for (int k = 1; k < a.splits; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(p + k * a.plane);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    return make_uint2(pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w));
  } else {
    return *reinterpret_cast<const uint2*>(a.qkv + row * a.stride + col);
  }
}
template <bool kPart>
__device__ __forceinline__ uint32_t load2(const AppendArgs& a, long long row, int col) {
  if constexpr (kPart) {
    const float* p = a.part + row * a.pstride + col;
    float2 s = *reinterpret_cast<const float2*>(p);
    for (int k = 1; k < a.splits; ++k) {
      const float2 v = *reinterpret_cast<const float2*>(p + k * a.plane);
      s.x += v.x;
      s.y += v.y;
    }
    return pack_bf16x2(s.x, s.y);
  } else {
    return *reinterpret_cast<const uint32_t*>(a.qkv + row * a.stride + col);
  }
}

// What the kernel does with a row (kMode): the fused norm + RoPE + append; the norm + RoPE
// alone (q and k in place, nothing appended: LaunchHeadNormRope); or the append alone of
// the row's k and v as they are in qkv (KvStore::StoreKV).
enum { kFused = 0, kNormOnly = 1, kStoreOnly = 2 };

template <int HPG, bool kPart, int kMode = kFused>
__global__ void __launch_bounds__(256) qknorm_rope_append_kernel(AppendArgs a) {
  constexpr int W = 10 / HPG;                  // waves per row
  constexpr int NKV = (kHkv + W - 1) / W;      // v heads per wave
  // rows past the projection's M have no partials
  const int T = kPart ? min(a.meta[FQA_META_ROWS], a.part_rows) : a.meta[FQA_META_ROWS];
  const int b = blockIdx.x;
  const int wid = ((b & 7) * a.blocks_per_xcd + (b >> 3)) * kWavesPerBlock + (threadIdx.x >> 6);
  const int row = wid / W, sw = wid % W;
  if (row >= T) return;
  const int pos = a.positions[row];
  const bool pos_ok = pos >= 0 && pos < a.rope_max_pos;
  if (!kPart && !pos_ok) return;  // no table row: leave the row untouched
  const int slot = kMode == kNormOnly ? -1 : a.slots[row];
  const long long page = slot / kPage;
  const bool page_ok = slot >= 0 && page < a.pool_pages;
  const int tok = slot % kPage;
  const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
  uint16_t* src = a.qkv + (long long)row * a.stride;

  // ---- q/k heads g + 4*(sw*HPG + i) ----------------------------------------------------
  uint2 lo[HPG], hi[HPG];
#pragma unroll
  for (int i = 0; i < HPG; ++i) {
    const int col = (g + 4 * (sw * HPG + i)) * kD;
    if (kMode == kStoreOnly && col < kHq * kD) continue;  // q heads: not stored
    lo[i] = load4<kPart>(a, row, col + 4 * j);
    hi[i] = load4<kPart>(a, row, col + 64 + 4 * j);
  }
  if (kPart && !pos_ok) {  // no table row: the projection's values, as unfused
#pragma unroll
    for (int i = 0; i < HPG; ++i) {
      const int head = g + 4 * (sw * HPG + i);
      if (head >= kHq && !a.write_k) continue;
      *reinterpret_cast<uint2*>(src + head * kD + 4 * j) = lo[i];
      *reinterpret_cast<uint2*>(src + head * kD + 64 + 4 * j) = hi[i];
    }
    return;
  }
  if constexpr (kMode == kStoreOnly) {
#pragma unroll
    for (int i = 0; i < HPG; ++i) {
      const int head = g + 4 * (sw * HPG + i);
      if (head < kHq || !page_ok) continue;
      uint16_t* kd = a.pool + run_offset(page, head - kHq) + tok * kD;
      *reinterpret_cast<uint2*>(kd + 4 * j) = lo[i];
      *reinterpret_cast<uint2*>(kd + 64 + 4 * j) = hi[i];
    }
  } else {
  const float4 c4 = *reinterpret_cast<const float4*>(a.cos_tab + (long long)pos * 64 + 4 * j);
  const float4 s4 = *reinterpret_cast<const float4*>(a.sin_tab + (long long)pos * 64 + 4 * j);
  const float4 q1 = *reinterpret_cast<const float4*>(a.wq + 4 * j);
  const float4 q2 = *reinterpret_cast<const float4*>(a.wq + 64 + 4 * j);
  const float4 k1 = *reinterpret_cast<const float4*>(a.wk + 4 * j);
  const float4 k2 = *reinterpret_cast<const float4*>(a.wk + 64 + 4 * j);
  const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int i = 0; i < HPG; ++i) {
    const int head = g + 4 * (sw * HPG + i);
    const bool is_k = head >= kHq;  // heads 32..39: only i >= 8
    const float wa[4] = {is_k ? k1.x : q1.x, is_k ? k1.y : q1.y, is_k ? k1.z : q1.z,
                         is_k ? k1.w : q1.w};
    const float wb[4] = {is_k ? k2.x : q2.x, is_k ? k2.y : q2.y, is_k ? k2.z : q2.z,
                         is_k ? k2.w : q2.w};
    uint2 olo, ohi;
    norm_rope_head(lo[i], hi[i], wa, wb, cs, sn, a.eps, olo, ohi);
    uint16_t* hs = src + head * kD;
    if (!is_k || a.write_k) {
      *reinterpret_cast<uint2*>(hs + 4 * j) = olo;
      *reinterpret_cast<uint2*>(hs + 64 + 4 * j) = ohi;
    }
    if (is_k && page_ok) {  // K [16 tokens][128] of the row's page
      uint16_t* kd = a.pool + run_offset(page, head - kHq) + tok * kD;
      *reinterpret_cast<uint2*>(kd + 4 * j) = olo;
      *reinterpret_cast<uint2*>(kd + 64 + 4 * j) = ohi;
    }
  }
  }  // kMode != kStoreOnly
  if constexpr (kMode == kNormOnly) return;

  // ---- v ------------------------------------------------------------------------------
  if (!page_ok) return;
  // Full page: rows lead..lead+15 hold this page's tokens 0..15 (their slots are
  // distinct and consecutive, so checking the first and the last suffices), and every
  // one of them has a table row (positions run consecutively within a request).
  const int lead = row - tok;
  bool full = lead >= 0 && lead + kPage <= T;
  if (full) {
    const int base_slot = slot - tok;
    full = a.slots[lead] == base_slot && a.slots[lead + kPage - 1] == base_slot + kPage - 1 &&
           a.positions[lead] >= 0 && a.positions[lead + kPage - 1] < a.rope_max_pos;
  }
  if (full) {
    // The page's 16 rows share its V^T: row tok moves kv head tok/2, dims 64*(tok%2) ..
    // +63, for all 16 tokens (one wave of the row: the first).  Lane l holds dims
    // d = 64*(tok%2) + 2*(l%32), d+1 of tokens 8*(l/32) .. +7, transposes them in
    // registers (v_perm) and stores two 16-byte pieces of V^T rows d and d+1.
    if (sw != 0) return;
    const int kvh = tok >> 1, d = 64 * (tok & 1) + 2 * (lane & 31), t0 = 8 * (lane >> 5);
    uint32_t x[8];
#pragma unroll
    for (int t = 0; t < 8; ++t)
      x[t] = load2<kPart>(a, (long long)lead + t0 + t, (kHq + kHkv + kvh) * kD + d);
    uint32_t y0[4], y1[4];  // dim d / d+1, tokens t0+2k, t0+2k+1
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      y0[k] = __builtin_amdgcn_perm(x[2 * k + 1], x[2 * k], 0x05040100u);
      y1[k] = __builtin_amdgcn_perm(x[2 * k + 1], x[2 * k], 0x07060302u);
    }
    uint16_t* vt = a.pool + run_offset(page, kvh) + kVOff + d * kPage + t0;
    *reinterpret_cast<uint4*>(vt) = make_uint4(y0[0], y0[1], y0[2], y0[3]);
    *reinterpret_cast<uint4*>(vt + kPage) = make_uint4(y1[0], y1[1], y1[2], y1[3]);
    return;
  }
  // Partly filled page: v heads sw*NKV .. : lane -> (kv head, DPL consecutive dims)
  constexpr int LPK = kWave / NKV;   // lanes per v head
  constexpr int DPL = kD / LPK;      // dims per lane (2, 4 or 16)
  const int kvh = sw * NKV + lane / LPK, d0 = (lane % LPK) * DPL;
  if (kvh >= kHkv) return;
  uint32_t wv[DPL / 2];
#pragma unroll
  for (int e = 0; e < DPL / 2; ++e) wv[e] = load2<kPart>(a, row, (kHq + kHkv + kvh) * kD + d0 + 2 * e);
  uint16_t* vt = a.pool + run_offset(page, kvh) + kVOff + d0 * kPage + tok;
#pragma unroll
  for (int e = 0; e < DPL / 2; ++e) {
    vt[(2 * e) * kPage] = (uint16_t)wv[e];
    vt[(2 * e + 1) * kPage] = (uint16_t)(wv[e] >> 16);
  }
}

bool dims_ok(const fqa_dims* d) {
  return d && d->n_q_heads == kHq && d->n_kv_heads == kHkv && d->head_dim == kD &&
         d->page_size == kPage && d->qkv_stride >= kQkvStride && d->qkv_stride % 4 == 0;
}

template <bool kPart, int kMode = kFused>
void launch_append(const AppendArgs& a, int hpg, dim3 grid, hipStream_t st) {
  const dim3 block(256);
  if (hpg == 1)
    hipLaunchKernelGGL((qknorm_rope_append_kernel<1, kPart, kMode>), grid, block, 0, st, a);
  else if (hpg == 2)
    hipLaunchKernelGGL((qknorm_rope_append_kernel<2, kPart, kMode>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((qknorm_rope_append_kernel<10, kPart, kMode>), grid, block, 0, st, a);
}

// Validates the append arguments and launches the append kernel (kPart: reading the
// projection's split partials `part`, splits > 1).
int append_launch(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                  const float* k_norm_w, const float* cos_tab, const float* sin_tab,
                  int32_t rope_max_pos, const int32_t* positions, const int32_t* slot_mapping,
                  const int32_t* meta, int32_t rows_bound, uint16_t* pool, int64_t pool_pages,
                  int32_t write_k_inplace, const float* part, int splits, int part_rows,
                  hipStream_t st, int mode = kFused) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (rows_bound < 0 || pool_pages < 1 || rope_max_pos < 1 || !meta) return FQA_EINVAL;
  if (rows_bound == 0) return FQA_OK;
  const bool norm = mode != kStoreOnly, store = mode != kNormOnly;
  if (!qkv || !positions || (norm && (!q_norm_w || !k_norm_w || !cos_tab || !sin_tab)) ||
      (store && (!slot_mapping || !pool)))
    return FQA_EINVAL;
  // Heads per lane group: 1 (10 waves per row) for decode-sized steps, 2 (5 waves per row)
  // above 512 rows (measured at 8192 rows: 2 took 31.9 us, 5 32.3, 10 35.2, 1 39.2).
  const int hpg = rows_bound <= 512 ? 1 : 2;
  const long long waves = (long long)rows_bound * (10 / hpg);
  const int blocks = (int)((waves + kWavesPerBlock - 1) / kWavesPerBlock);
  const int blocks_per_xcd = (blocks + 7) / 8;
  AppendArgs a{qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions, slot_mapping,
               meta, pool, pool_pages, dims->qkv_stride, dims->eps, write_k_inplace,
               blocks_per_xcd, part, splits, kQkvStride, (long long)part_rows * kQkvStride,
               part_rows};
  const dim3 grid(8 * blocks_per_xcd);
  if (part)
    launch_append<true>(a, hpg, grid, st);
  else if (mode == kNormOnly)
    launch_append<false, kNormOnly>(a, hpg, grid, st);
  else if (mode == kStoreOnly)
    launch_append<false, kStoreOnly>(a, hpg, grid, st);
  else
    launch_append<false>(a, hpg, grid, st);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" int fqa_qknorm_rope_append(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                                      const float* k_norm_w, const float* cos_tab,
                                      const float* sin_tab, int32_t rope_max_pos,
                                      const int32_t* positions,
                                      const int32_t* slot_mapping, const int32_t* meta,
                                      int32_t rows_bound, uint16_t* pool, int64_t pool_pages,
                                      int32_t write_k_inplace, void* stream) {
  return append_launch(dims, qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions,
                       slot_mapping, meta, rows_bound, pool, pool_pages, write_k_inplace, nullptr,
                       1, 0, (hipStream_t)stream);
}

extern "C" int fqa_qknorm_rope(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                               const float* k_norm_w, const float* cos_tab, const float* sin_tab,
                               int32_t rope_max_pos, const int32_t* positions,
                               const int32_t* meta, int32_t rows_bound, void* stream) {
  return append_launch(dims, qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions,
                       nullptr, meta, rows_bound, nullptr, 1, 1, nullptr, 1, 0,
                       (hipStream_t)stream, kNormOnly);
}

extern "C" int fqa_store_kv(const fqa_dims* dims, const uint16_t* qkv, const int32_t* positions,
                            const int32_t* slot_mapping, const int32_t* meta, int32_t rows_bound,
                            uint16_t* pool, int64_t pool_pages, void* stream) {
  // The kernel reads qkv only in this mode (q and k are not written back).
  return append_launch(dims, const_cast<uint16_t*>(qkv), nullptr, nullptr, nullptr, nullptr,
                       0x7fffffff, positions, slot_mapping, meta, rows_bound, pool, pool_pages,
                       0, nullptr, 1, 0, (hipStream_t)stream, kStoreOnly);
}

extern "C" int fqa_qkv_proj_append(const fqa_dims* dims, const uint16_t* x, int64_t ldx,
                                   const uint16_t* w_qkv, int64_t ldw, int32_t rows,
                                   int32_t hidden, uint16_t* qkv, const float* q_norm_w,
                                   const float* k_norm_w, const float* cos_tab,
                                   const float* sin_tab, int32_t rope_max_pos,
                                   const int32_t* positions, const int32_t* slot_mapping,
                                   const int32_t* meta, uint16_t* pool, int64_t pool_pages,
                                   int32_t write_k_inplace, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (rows < 0 || hidden <= 0 || pool_pages < 1 || rope_max_pos < 1 || !meta) return FQA_EINVAL;
  if (rows == 0) return FQA_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !positions || !slot_mapping ||
      !pool)
    return FQA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const GemmAppend app{q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions,
                       slot_mapping, meta, pool, pool_pages, dims->eps, write_k_inplace};
  bool appended = false;
  const int splits = gemm_launch_partials(x, ldx, w_qkv, ldw, qkv, dims->qkv_stride, rows,
                                          kQkvStride, hidden, workspace, workspace_bytes, st,
                                          &app, &appended);
  if (splits < 0) return splits;
  if (appended) return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
  return append_launch(dims, qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions,
                       slot_mapping, meta, rows, pool, pool_pages, write_k_inplace,
                       splits > 1 ? static_cast<const float*>(workspace) : nullptr, splits, rows,
                       st);
}
