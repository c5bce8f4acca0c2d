// fqa_prefill.hip — varlen causal FlashAttention-2 prefill over the paged pool (gfx950).
//
// Replaces CutePrefillKernel + LaunchAttnPrefillCute (engine/src/attn_cute.cu:30-163).
// Same semantics: for each qlen != 1 request and each of its rows, head h attends the
// keys of kv head h/4 with key pos <= query pos (the cached prefix included); scores
// q.k * scale in fp32; online softmax; P rounded to bf16 before PV (attn_cute.cu:128);
// fp32 accumulation; output bf16, 0 when l == 0.
//
// MI355X design:
//  * One 256-thread workgroup per (32 query rows, kv head); wave w owns query head w of
//    the kv head.  The 4 heads share every K/V tile, staged into LDS once (the
//    reference runs one block per query head and re-reads K/V 4x, attn_cute.cu:157).
//    At 212 VGPRs two workgroups share a CU, so one wave's MFMAs overlap another's
//    softmax on every SIMD.
//  * Transposed FA-2 on v_mfma_f32_32x32x16_bf16:
//        S^T[32 keys x 32 rows] = K[32 x 128] . Q^T[128 x 32]   (8 MFMAs per 32 keys)
//        O^T[128 x 32 rows]    += V^T[128 x 16 keys] . P^T      (4 MFMAs per 16 keys)
//    With rows as accumulator columns every lane owns one query row: the softmax row
//    max / sum is 16 in-lane values plus one exchange with lane^32, the rescale of O is
//    a per-lane scalar, and the S^T accumulator registers are already the P^T operand
//    (the key order inside the contraction is chosen to match, V^T is read to suit).
//  * Softmax VALU work per score, not MFMA, is the limit on CDNA (a wave64 VALU op
//    issues in 4 cycles, exp in more): scores are maxed raw, scaled inside the exp2
//    FMA, converted with v_cvt_pk_bf16_f32, summed two at a time with v_dot2 against
//    (1, 1), and O is rescaled lazily (only when the row max grows by more than 2^8).
//  * K/V tiles are 64 keys = 4 pages = four contiguous 8 KiB runs, double-buffered in
//    LDS (2 x 32 KiB) with XOR swizzles that make every fragment read bank-conflict
//    free and every fragment one 16-byte read; the next tile's global loads are in
//    flight during the current tile's MFMAs.
//  * Work items come from the pack sorted by key count, longest first.
#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kQT = 32;        // query rows per workgroup
constexpr int kKT = 64;        // keys per LDS tile (4 pages)
constexpr int kPagesPerTile = kKT / kPage;
constexpr int kRunBytes = kRunElems * 2;                 // 8 KiB
constexpr int kStageBytes = kPagesPerTile * kRunBytes;   // 32 KiB
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescale = 8.0f;  // lazy-rescale threshold (log2 units)

struct PreArgs {
  const uint16_t* qkv;
  const uint16_t* pool;
  long long pool_pages;
  const int32_t* bt;
  int max_blocks;
  const int32_t* cu;
  const int32_t* pos;
  const int32_t* items;
  const int32_t* meta;
  uint16_t* out;
  int stride;
  float scale_log2;
};

// LDS byte offset of K chunk (16 B = 8 dims) `c` of token `t` in page slot `ps`.
__device__ __forceinline__ int lds_k(int ps, int t, int c) {
  return ps * kRunBytes + t * 256 + ((c ^ t) << 4);
}
// LDS byte offset of V^T chunk `h` of dim row `d` in page slot `ps`.  A row's 16 tokens
// are stored as chunk 0 = tokens {0-3, 8-11}, chunk 1 = tokens {4-7, 12-15}: exactly the
// 8 keys one lane half contributes to a 16-key PV step.
// The chunk swizzle h ^ bit2(d) ^ bit3(d) keeps the 16-byte reads of 16 consecutive rows
// on distinct banks whether the LDS serves 8 lanes from 32 banks or 16 lanes from 64.
__device__ __forceinline__ int lds_v(int ps, int d, int h) {
  return ps * kRunBytes + kVOff * 2 + d * 32 + ((h ^ ((d >> 2) & 1) ^ ((d >> 3) & 1)) << 4);
}

// Keep the first `valid` (0..16) tokens of 8 bf16 tokens t0.. of one V^T row.
__device__ __forceinline__ uint2 keep_tokens(uint2 v, int t0, int valid) {
  uint32_t w[2] = {v.x, v.y};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ta = t0 + 2 * i;
    w[i] &= (ta < valid ? 0x0000ffffu : 0u) | (ta + 1 < valid ? 0xffff0000u : 0u);
  }
  return make_uint2(w[0], w[1]);
}

__global__ void __launch_bounds__(256, 2) prefill_kernel(PreArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kStageBytes];

  const int item = blockIdx.x >> 3, kvh = blockIdx.x & 7;
  if (item >= a.meta[FQA_META_PRE_ITEMS]) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int4 it = *reinterpret_cast<const int4*>(a.items + 4 * (long long)item);
  const int r = it.x, q0 = it.y, q1 = it.z, nkeys = it.w;
  const int qs = a.cu[r];
  const int32_t* btr = a.bt + (long long)r * a.max_blocks;
  const int nkb = (nkeys + kKT - 1) / kKT;

  const int col = lane & 31, hf = lane >> 5;
  const int i_row = q0 + col;  // row within the request
  const bool row_ok = i_row < q1;
  const int qpos = row_ok ? a.pos[qs + i_row] : -1;
  const int min_pos = a.pos[qs + q0];  // first row: smallest position of the tile
  const int h = kvh * kG + w;

  bf16x8 qf[8];
  {
    const uint16_t* q = a.qkv + (long long)(qs + (row_ok ? i_row : q0)) * a.stride + h * kD + hf * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qf[ks] = *reinterpret_cast<const bf16x8*>(q + ks * 16);
      if (!row_ok)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[ks][i] = (__bf16)0.0f;
    }
  }

  float16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m_run = -1e30f, l_run = 0.f;

  // ---- staging: per tile each thread moves 4 K chunks (16 B) and 2 V^T rows (32 B) ----
  // K chunk i of thread t: page slot i, token t/16, dims (t%16)*8..; V^T row j: page slot
  // 2j + t/128, dim t%128.
  uint4 sk[4];
  uint4 sv[2][2];
  // Fast path: every page of the tile is full and in range (all but a workgroup's last
  // tile, checked on scalar registers): plain loads, no masks.  Otherwise each page is
  // loaded only if it exists and is in range, and tokens past n_keys are zeroed (their
  // P is 0, and 0 x garbage must not become NaN in PV).
  auto stage_load = [&](int kb) {
    long long pg[kPagesPerTile];
    bool fast = (kb + 1) * kKT <= nkeys;
#pragma unroll
    for (int ps = 0; ps < kPagesPerTile; ++ps) {
      pg[ps] = fast ? btr[kb * kPagesPerTile + ps] : -1;
      fast = fast && pg[ps] >= 0 && pg[ps] < a.pool_pages;
    }
    if (fast) {
#pragma unroll
      for (int ps = 0; ps < kPagesPerTile; ++ps) {
        const uint16_t* run = a.pool + run_offset(pg[ps], kvh);
        sk[ps] = *reinterpret_cast<const uint4*>(run + tid * 8);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d = tid & 127;
        const uint16_t* src = a.pool + run_offset(pg[2 * j + (tid >> 7)], kvh) + kVOff + d * kPage;
        const uint4 lo = *reinterpret_cast<const uint4*>(src);
        const uint4 hi = *reinterpret_cast<const uint4*>(src + 8);
        // chunk 0 = tokens {0-3, 8-11}, chunk 1 = tokens {4-7, 12-15}
        sv[j][0] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        sv[j][1] = make_uint4(lo.z, lo.w, hi.z, hi.w);
      }
      return;
    }
#pragma unroll
    for (int ps = 0; ps < kPagesPerTile; ++ps) {
      const int pidx = kb * kPagesPerTile + ps;
      const int valid = nkeys - pidx * kPage;  // tokens of this page that exist (may be <= 0)
      const long long page = valid > 0 ? btr[pidx] : -1;
      const bool ok = page >= 0 && page < a.pool_pages;
      const uint16_t* run = a.pool + run_offset(ok ? page : 0, kvh);
      const int tk = tid >> 4;
      uint4 v = *reinterpret_cast<const uint4*>(run + tid * 8);
      const bool keep = ok && tk < valid;
      sk[ps] = keep ? v : make_uint4(0, 0, 0, 0);
      if ((ps >> 1) * 2 + (tid >> 7) == ps) {  // this thread's V^T row lives in page ps
        const int j = ps >> 1, d = tid & 127;
        const uint16_t* vr = run + kVOff + d * kPage;
        uint4 lo = *reinterpret_cast<const uint4*>(vr);
        uint4 hi = *reinterpret_cast<const uint4*>(vr + 8);
        if (!ok) lo = hi = make_uint4(0, 0, 0, 0);
        if (valid < kPage) {
          uint2 a0 = keep_tokens(make_uint2(lo.x, lo.y), 0, valid);
          uint2 a1 = keep_tokens(make_uint2(lo.z, lo.w), 4, valid);
          uint2 b0 = keep_tokens(make_uint2(hi.x, hi.y), 8, valid);
          uint2 b1 = keep_tokens(make_uint2(hi.z, hi.w), 12, valid);
          lo = make_uint4(a0.x, a0.y, a1.x, a1.y);
          hi = make_uint4(b0.x, b0.y, b1.x, b1.y);
        }
        sv[j][0] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        sv[j][1] = make_uint4(lo.z, lo.w, hi.z, hi.w);
      }
    }
  };
  auto stage_store = [&](int buf) {
    char* base = lds + buf * kStageBytes;
    const int tk = tid >> 4, cc = tid & 15;
#pragma unroll
    for (int ps = 0; ps < kPagesPerTile; ++ps)
      *reinterpret_cast<uint4*>(base + lds_k(ps, tk, cc)) = sk[ps];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ps = 2 * j + (tid >> 7), d = tid & 127;
      *reinterpret_cast<uint4*>(base + lds_v(ps, d, 0)) = sv[j][0];
      *reinterpret_cast<uint4*>(base + lds_v(ps, d, 1)) = sv[j][1];
    }
  };

  stage_load(0);
  stage_store(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) stage_load(kb + 1);
    const char* base = lds + buf * kStageBytes;
    // Both halves' S^T = K Q^T first, so half 0's softmax (VALU) runs while half 1's
    // MFMAs execute, and half 1's softmax while half 0's PV MFMAs execute.
    const bool live1 = kb * kKT + 32 < nkeys;  // second half has keys (wave-uniform)
    float16_t s2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j == 1 && !live1) break;
#pragma unroll
      for (int i = 0; i < 16; ++i) s2[j][i] = 0.f;
      const int ps = j * 2 + (col >> 4), t = col & 15;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(base + lds_k(ps, t, ks * 2 + hf));
        s2[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s2[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // two 32-key halves of the tile
      if (j == 1 && !live1) break;
      const int key0 = kb * kKT + j * 32;
      float16_t& s = s2[j];
      // online softmax over this lane's query row
      float mx = -INFINITY;
      if (key0 + 31 > min_pos) {  // the causal diagonal crosses these keys
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + (v >> 2) * 8 + hf * 4 + (v & 3);
          if (key > qpos) s[v] = -INFINITY;
          mx = fmaxf(mx, s[v]);
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
      }
      mx = max_xor32(mx);
      // Lazy rescale: the reference max only moves when the row max grows by more than
      // 2^kRescale, so P = exp2(s*scale - m) stays <= 2^kRescale and O, l are rescaled
      // on few tiles instead of every tile.
      const float m_new = fmaxf(m_run, mx * a.scale_log2);
      const bool grow = m_new > m_run + kRescale;
      if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform: skipped on most tiles
        const float corr = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        l_run *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] *= corr;
        m_run = grow ? m_new : m_run;
      }
      bf16x8 pt[2];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        // raw v_exp_f32: results below 2^-126 flush to 0, which a softmax weight can be
        const float p = __builtin_amdgcn_exp2f(fmaf(s[v], a.scale_log2, -m_run));
        pt[v >> 3][v & 7] = (__bf16)p;
      }
      // l sums the same bf16 P that multiplies V (one v_dot2 per pair instead of one add
      // per score), so the output weights are normalised exactly
      {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bf16x2_t pr = {pt[kc][2 * e], pt[kc][2 * e + 1]};
            l_run = __builtin_amdgcn_fdot2_f32_bf16(pr, one, l_run, false);
          }
      }
      // O^T += V^T P^T over the two pages (16 keys each) of this half
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int ps = j * 2 + kc;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const bf16x8 vf =
              *reinterpret_cast<const bf16x8*>(base + lds_v(ps, db * 32 + col, hf));
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pt[kc], o[db], 0, 0, 0);
        }
      }
    }
    if (kb + 1 < nkb) stage_store(buf ^ 1);
    __syncthreads();
  }

  if (!row_ok) return;
  const auto lr = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                   false, false);
  const float l = __uint_as_float(lr[0]) + __uint_as_float(lr[1]);
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* dst = a.out + (long long)(qs + i_row) * (kHq * kD) + h * kD + hf * 4;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint2 pk = make_uint2(pack_bf16x2(o[db][i * 4] * inv, o[db][i * 4 + 1] * inv),
                                  pack_bf16x2(o[db][i * 4 + 2] * inv, o[db][i * 4 + 3] * inv));
      *reinterpret_cast<uint2*>(dst + db * 32 + i * 8) = pk;
    }
}

bool dims_ok(const fqa_dims* d) {
  return d && d->n_q_heads == kHq && d->n_kv_heads == kHkv && d->head_dim == kD &&
         d->page_size == kPage && d->qkv_stride >= kQkvStride && d->qkv_stride % 8 == 0;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" int fqa_prefill(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                           int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* cu_seqlens, const int32_t* positions,
                           const int32_t* pre_items, const int32_t* meta, int32_t pre_tile_q,
                           int32_t pre_item_cap, uint16_t* out, void* stream) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (pre_tile_q != kQT) return FQA_EUNSUPPORTED;
  if (pre_item_cap < 0 || max_blocks < 1 || pool_pages < 1 || !meta) return FQA_EINVAL;
  if (pre_item_cap == 0) return FQA_OK;
  if (!qkv || !pool || !block_tables || !cu_seqlens || !positions || !pre_items || !out)
    return FQA_EINVAL;
  PreArgs a{qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions, pre_items,
            meta, out, dims->qkv_stride, dims->scale * kLog2e};
  hipLaunchKernelGGL(prefill_kernel, dim3(pre_item_cap * kHkv), dim3(256), 0,
                     (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
