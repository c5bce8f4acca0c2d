// fqa_prefill.hip — varlen causal FlashAttention-2 prefill over the paged pool (gfx950).
//
// Replaces CutePrefillKernel + LaunchAttnPrefillCute (engine/src/attn_cute.cu:30-163).
// Same semantics: for each qlen != 1 request and each of its rows, head h attends the
// keys of kv head h/4 with key pos <= query pos (the cached prefix included); scores
// q.k * scale in fp32; online softmax; P rounded to bf16 before PV (attn_cute.cu:128);
// fp32 accumulation; output bf16, 0 when l == 0.
//
// MI355X design:
//  * One 256-thread workgroup per (query tile of 64 rows, kv head): the 4 query heads
//    of the kv head share every K/V tile, which is staged into LDS once (the reference
//    runs one block per query head and re-reads K/V 4x, attn_cute.cu:157).
//    Wave w takes rows (w/2)*32 .. +32 and heads 2*(w%2), 2*(w%2)+1.
//  * Transposed FA-2 on v_mfma_f32_32x32x16_bf16:
//        S^T[32 keys x 32 rows] = K[32 x 128] . Q^T[128 x 32]   (8 MFMAs per head)
//        O^T[128 x 32 rows]    += V^T[128 x 32 keys] . P^T      (8 MFMAs per head)
//    With rows as accumulator columns every lane owns one query row: the softmax row
//    max / sum is 16 in-lane values plus one exchange with lane^32, the rescale of O is
//    a per-lane scalar, and the S^T accumulator registers are already the P^T operand
//    (the key order inside the contraction is chosen to match, V^T is read to suit).
//    Each K or V^T fragment read from LDS feeds both heads of the wave.
//  * K/V tiles are 32 keys = 2 pages = two contiguous 8 KiB runs, double-buffered in
//    LDS with XOR swizzles that make the fragment reads bank-conflict free; the next
//    tile's global loads are in flight during the current tile's MFMAs.
//  * Work items come from the pack sorted by key count, longest first.
#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kQT = 64;           // query rows per workgroup
constexpr int kKT = 32;           // keys per LDS tile (2 pages)
constexpr int kStageBytes = 2 * kRunElems * 2;  // 16 KiB
constexpr float kLog2e = 1.4426950408889634f;

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

// LDS byte offset of K chunk (16 B) `c` of token `t` in page slot `ps` of a stage.
__device__ __forceinline__ int lds_k(int ps, int t, int c) {
  return ps * (kRunElems * 2) + t * 256 + ((c ^ t) << 4);
}
// LDS byte offset of V^T unit (8 B = 4 tokens) `u` of dim row `d` in page slot `ps`.
__device__ __forceinline__ int lds_v(int ps, int d, int u) {
  return ps * (kRunElems * 2) + kVOff * 2 + d * 32 + ((u ^ ((d >> 3) & 3)) << 3);
}

__device__ __forceinline__ uint4 zero_tokens(uint4 v, int first_bad) {
  // v holds 8 consecutive tokens (bf16) of one V^T row; clear tokens >= first_bad
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (2 * i >= first_bad) w[i] &= 0xffff0000u;
    if (2 * i + 1 >= first_bad) w[i] &= 0x0000ffffu;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void __launch_bounds__(256) prefill_kernel(PreArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kStageBytes];

  const int item = blockIdx.x >> 3, kvh = blockIdx.x & 7;
  if (item >= a.meta[FQA_META_PRE_ITEMS]) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int4 it = *reinterpret_cast<const int4*>(a.items + 4 * (long long)item);
  const int r = it.x, q0 = it.y, q1 = it.z, nkeys = it.w;
  const int qs = a.cu[r];
  const int32_t* btr = a.bt + (long long)r * a.max_blocks;
  const int nkb = (nkeys + kKT - 1) / kKT;

  // ---- this wave's rows and heads ---------------------------------------------------
  const int col = lane & 31, hf = lane >> 5;
  const int i_row = q0 + (w >> 1) * 32 + col;  // row within the request
  const bool row_ok = i_row < q1;
  const int qpos = row_ok ? a.pos[qs + i_row] : -1;
  const int h0 = kvh * kG + (w & 1) * 2;
  const int wave_first = q0 + (w >> 1) * 32;
  const bool wave_live = wave_first < q1;
  // key blocks this wave needs: keys up to the last valid row's position
  const int wave_last = min(wave_first + 31, q1 - 1);
  const int wave_nkb = wave_live ? (a.pos[qs + wave_last] + kKT) / kKT : 0;
  const int wave_min_pos = wave_live ? a.pos[qs + wave_first] : 0;

  bf16x8 qf[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const uint16_t* q = a.qkv + (long long)(qs + i_row) * a.stride + (h0 + hh) * kD + hf * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (row_ok) qf[hh][ks] = *reinterpret_cast<const bf16x8*>(q + ks * 16);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[hh][ks][i] = (__bf16)0.0f;
    }
  }

  float16_t o[2][4];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[hh][db][i] = 0.f;
  float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.f, 0.f};

  // ---- staging: 1024 chunks of 16 B per tile, 4 per thread ----------------------------
  uint4 stg[4];
  auto stage_load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + i * 256, ps = c >> 9, e = c & 511;
      const int pidx = kb * 2 + ps;
      const int key_base = pidx * kPage;
      stg[i] = make_uint4(0, 0, 0, 0);
      if (key_base < nkeys) {
        const long long page = btr[pidx];
        if (page >= 0 && page < a.pool_pages) {
          const uint16_t* run = a.pool + run_offset(page, kvh);
          uint4 v = *reinterpret_cast<const uint4*>(run + e * 8);
          const int valid = nkeys - key_base;  // tokens of this page that exist
          if (valid < kPage) {
            if (e < 256) {
              if ((e >> 4) >= valid) v = make_uint4(0, 0, 0, 0);
            } else {
              v = zero_tokens(v, valid - ((e - 256) & 1) * 8);
            }
          }
          stg[i] = v;
        }
      }
    }
  };
  auto stage_store = [&](int buf) {
    char* base = lds + buf * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + i * 256, ps = c >> 9, e = c & 511;
      if (e < 256) {
        const int t = e >> 4, cc = e & 15;
        *reinterpret_cast<uint4*>(base + lds_k(ps, t, cc)) = stg[i];
      } else {
        const int e2 = e - 256, d = e2 >> 1, u = (e2 & 1) * 2;
        *reinterpret_cast<uint2*>(base + lds_v(ps, d, u)) = make_uint2(stg[i].x, stg[i].y);
        *reinterpret_cast<uint2*>(base + lds_v(ps, d, u + 1)) = make_uint2(stg[i].z, stg[i].w);
      }
    }
  };

  stage_load(0);
  stage_store(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) stage_load(kb + 1);
    if (kb < wave_nkb) {
      const char* base = lds + buf * kStageBytes;
      // S^T = K Q^T for both heads
      float16_t s[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) { s[0][i] = 0.f; s[1][i] = 0.f; }
      {
        const int key = col, ps = key >> 4, t = key & 15;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(base + lds_k(ps, t, ks * 2 + hf));
          s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[0][ks], s[0], 0, 0, 0);
          s[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[1][ks], s[1], 0, 0, 0);
        }
      }
      const bool need_mask = (kb + 1) * kKT - 1 > wave_min_pos;
      bf16x8 pt[2][2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float mx = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float x = s[hh][v] * a.scale_log2;
          if (need_mask) {
            const int key = kb * kKT + (v >> 2) * 8 + hf * 4 + (v & 3);
            if (key > qpos) x = -INFINITY;
          }
          s[hh][v] = x;
          mx = fmaxf(mx, x);
        }
        mx = wave_max_xor(mx, 32);
        const float m_new = fmaxf(m_run[hh], mx);
        const float corr = exp2f(m_run[hh] - m_new);
        float psum = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = exp2f(s[hh][v] - m_new);
          s[hh][v] = p;
          psum += p;
        }
        l_run[hh] = l_run[hh] * corr + psum;
        m_run[hh] = m_new;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[hh][db] *= corr;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            pt[hh][kc][j] = __builtin_bit_cast(__bf16, f32_to_bf16_bits(s[hh][kc * 8 + j]));
      }
      // O^T += V^T P^T
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int d = db * 32 + col;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const uint2 lo = *reinterpret_cast<const uint2*>(base + lds_v(kc, d, hf));
          const uint2 hi = *reinterpret_cast<const uint2*>(base + lds_v(kc, d, 2 + hf));
          const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
          const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
          o[0][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pt[0][kc], o[0][db], 0, 0, 0);
          o[1][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pt[1][kc], o[1][db], 0, 0, 0);
        }
      }
    }
    if (kb + 1 < nkb) stage_store(buf ^ 1);
    __syncthreads();
  }

  if (!row_ok) return;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    float l = l_run[hh] + __shfl_xor(l_run[hh], 32, kWave);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* dst = a.out + (long long)(qs + i_row) * (kHq * kD) + (h0 + hh) * kD + hf * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float16_t& v = o[hh][db];
        uint2 pk = make_uint2(pack_bf16x2(v[i * 4] * inv, v[i * 4 + 1] * inv),
                              pack_bf16x2(v[i * 4 + 2] * inv, v[i * 4 + 3] * inv));
        *reinterpret_cast<uint2*>(dst + db * 32 + i * 8) = pk;
      }
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
  hipLaunchKernelGGL(prefill_kernel, dim3(pre_item_cap * kHkv), dim3(256), 0, (hipStream_t)stream,
                     a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
