// fqa_decode.hip — GQA-shared split-K flash decoding over the paged pool (gfx950).
//
// Replaces CuteDecodeSplitKernel + CuteDecodeCombineKernel and their launcher
// (engine/src/attn_cute.cu:165-261).  Same semantics: for every qlen==1 request the
// 4 query heads of each kv head attend keys [0, pos]; scores q.k * scale in fp32;
// online softmax; partials merged by log-sum-exp; output bf16, 0 when l == 0.
//
// MI355X design:
//  * One wavefront per (work item, kv head).  A work item is a page range of one
//    sequence sized by the pack so that all sequences split into near-equal pieces
//    (the reference uses one split factor 128/n_decode for every sequence,
//    attn_cute.cu:249-251).  Each (page, kv head) is one contiguous 8 KiB run
//    (K [16][128] then V^T [128][16]) that the wave reads exactly once for all 4 heads.
//  * Both products run on MFMA in transposed form so that no operand is ever
//    shuffled between lanes:
//        S^T[16 keys x 16 cols] = K[16 x 128] . Q^T[128 x 16]  (4 x mfma 16x16x32 bf16)
//        O^T[128 x 16 cols]    += V^T[128 x 16 keys] . P^T    (8 x mfma 16x16x16 bf16)
//    Columns 0..3 are the 4 query heads (the rest carry zeros); the S^T accumulator
//    layout (lane = column, 4 consecutive keys per lane) is exactly the B-operand
//    layout P^T needs, and V^T's page layout gives each lane 4 consecutive keys of one
//    dim as one 8-byte load.  The kernel is HBM-bound; MFMA keeps the ALU out of the
//    way (about 5% of the CU's matrix rate at full HBM bandwidth).
//  * P is rounded to bf16 for the PV product (the reference's decode keeps P in fp32;
//    the difference is below the bf16 output rounding the tolerance allows).
//  * Pages rotate through four register buffers: while page p is processed the loads of
//    p+1..p+3 are in flight, 24 KiB per wave (HBM latency x bandwidth needs ~64 KiB in
//    flight per CU; at 2 waves per SIMD this gives ~190 KiB).
//  * Sequences whose plan has one split write bf16 directly; the others write fp32
//    partials (m, l, acc) and a combine wave per (sequence, kv head) merges them.
#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kDecWavesPerBlock = 4;
constexpr float kLog2e = 1.4426950408889634f;

struct DecArgs {
  const uint16_t* qkv;
  const uint16_t* pool;
  long long pool_pages;
  const int32_t* bt;
  int max_blocks;
  const int32_t* cu;
  const int32_t* pos;
  const int32_t* items;
  const int32_t* item_start;
  const int32_t* decode_rids;
  const int32_t* meta;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
  uint16_t* out;
  int stride;
  float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
};

struct PageFrag {
  bf16x8 k[4];
  short4_t v[8];
};

__device__ __forceinline__ void load_page(PageFrag& f, const uint16_t* run, int lane) {
  const int m = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    f.k[ks] = *reinterpret_cast<const bf16x8*>(run + m * kD + ks * 32 + g * 8);
#pragma unroll
  for (int b = 0; b < 8; ++b)
    f.v[b] = *reinterpret_cast<const short4_t*>(run + kVOff + (b * 16 + m) * kPage + g * 4);
}

struct DecState {
  float4_t acc[8];  // O^T: lane (col = head n, rows d = b*16 + 4g + j)
  float m;          // running max (exp2 domain), same in the 4 lanes of a column
  float l;          // running sum of this lane's 4 keys per page
};

// One page (16 keys) of online softmax for the 4 heads: S^T = K Q^T, P^T = exp2(S^T - m),
// O^T = O^T * corr + V^T P^T.
__device__ __forceinline__ void process_page(PageFrag& f, const bf16x8 (&qf)[4], int p, int L,
                                             int g, float scale_log2, DecState& st) {
  float4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.k[ks], qf[ks], s, 0, 0, 0);
  const int key0 = p * kPage + g * 4;
  float sv[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sv[j] = key0 + j < L ? s[j] * scale_log2 : -INFINITY;
    mx = fmaxf(mx, sv[j]);
  }
  if ((p + 1) * kPage > L) {  // last page: unwritten slots must not reach PV
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key0 + j >= L) f.v[b][j] = 0;
  }
  mx = wave_max_xor(mx, 16);
  mx = wave_max_xor(mx, 32);
  const float m_new = fmaxf(st.m, mx);
  const float corr = exp2f(st.m - m_new);
  float pj[4], psum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pj[j] = exp2f(sv[j] - m_new);
    psum += pj[j];
  }
  st.l = st.l * corr + psum;
  st.m = m_new;
  short4_t pt;
#pragma unroll
  for (int j = 0; j < 4; ++j) pt[j] = (short)f32_to_bf16_bits(pj[j]);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    st.acc[b] *= corr;
    st.acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(f.v[b], pt, st.acc[b], 0, 0, 0);
  }
}

__global__ void __launch_bounds__(kDecWavesPerBlock * kWave) decode_split_kernel(DecArgs a) {
  const int wave = blockIdx.x * kDecWavesPerBlock + (threadIdx.x >> 6);
  const int item = wave >> 3, kvh = wave & 7;
  if (item >= a.meta[FQA_META_DEC_ITEMS]) return;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;

  const int4 it = *reinterpret_cast<const int4*>(a.items + 4 * (long long)item);
  const int r = it.x, pb = it.z, pe = it.w;
  const int row = a.cu[r];
  const int L = a.pos[row] + 1;  // keys [0, L)
  const int32_t* btr = a.bt + (long long)r * a.max_blocks;

  // Q^T as the B operand: column n = head (kvh*4 + n) for n < 4, zeros elsewhere.
  bf16x8 qf[4];
  if (n < kG) {
    const uint16_t* q = a.qkv + (long long)row * a.stride + (kvh * kG + n) * kD + g * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(q + ks * 32);
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[ks][i] = (__bf16)0.0f;
  }

  DecState st;
#pragma unroll
  for (int b = 0; b < 8; ++b) st.acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -1e30f;
  st.l = 0.f;

  auto load = [&](PageFrag& f, bool& ok, int p) {
    const long long page = btr[p];
    ok = page >= 0 && page < a.pool_pages;
    load_page(f, a.pool + run_offset(ok ? page : 0, kvh), lane);
  };
  // Four page buffers in registers: page p is processed while p+1..p+3 are in flight
  // (24 KiB per wave).  The buffers rotate through a 4-way unrolled loop so every index
  // is static.
  PageFrag f0, f1, f2, f3;
  bool k0 = false, k1 = false, k2 = false, k3 = false;
  load(f0, k0, pb);
  if (pb + 1 < pe) load(f1, k1, pb + 1);
  if (pb + 2 < pe) load(f2, k2, pb + 2);
  for (int p = pb; p < pe; p += 4) {
    if (p + 3 < pe) load(f3, k3, p + 3);
    if (k0) process_page(f0, qf, p, L, g, a.scale_log2, st);
    if (p + 1 >= pe) break;
    if (p + 4 < pe) load(f0, k0, p + 4);
    if (k1) process_page(f1, qf, p + 1, L, g, a.scale_log2, st);
    if (p + 2 >= pe) break;
    if (p + 5 < pe) load(f1, k1, p + 5);
    if (k2) process_page(f2, qf, p + 2, L, g, a.scale_log2, st);
    if (p + 3 >= pe) break;
    if (p + 6 < pe) load(f2, k2, p + 6);
    if (k3) process_page(f3, qf, p + 3, L, g, a.scale_log2, st);
  }
  float l_run = st.l, m_run = st.m;
  float4_t* acc = st.acc;
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  if (n >= kG) return;

  const int pages = (L + kPage - 1) / kPage;
  if (pb == 0 && pe == pages) {  // the only split of this sequence: final output
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    uint16_t* o = a.out + (long long)row * (kHq * kD) + (kvh * kG + n) * kD + g * 4;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      uint2 v = make_uint2(pack_bf16x2(acc[b][0] * inv, acc[b][1] * inv),
                           pack_bf16x2(acc[b][2] * inv, acc[b][3] * inv));
      *reinterpret_cast<uint2*>(o + b * 16) = v;
    }
    return;
  }
  const long long slot = ((long long)item * kHkv + kvh) * kG + n;
  if (g == 0) {
    a.ws_m[slot] = m_run;
    a.ws_l[slot] = l_run;
  }
  float* wa = a.ws_acc + slot * kD + g * 4;
#pragma unroll
  for (int b = 0; b < 8; ++b) *reinterpret_cast<float4_t*>(wa + b * 16) = acc[b];
}

// Log-sum-exp merge of a sequence's split partials (attn_cute.cu:225-238): one wave per
// (decode sequence, query head), lane -> 2 dims; splits are folded with an online
// max so the loop carries no second pass and its loads can run ahead.
__global__ void __launch_bounds__(kDecWavesPerBlock * kWave) decode_combine_kernel(DecArgs a) {
  const int wave = blockIdx.x * kDecWavesPerBlock + (threadIdx.x >> 6);
  const int di = wave / kHq, h = wave % kHq;
  if (di >= a.meta[FQA_META_N_DECODE]) return;
  const int i0 = a.item_start[di], i1 = a.item_start[di + 1];
  if (i1 - i0 <= 1) return;
  const int lane = threadIdx.x & 63;
  const int kvh = h / kG, hh = h % kG;
  float gm = -1e30f, gl = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll 4
  for (int it = i0; it < i1; ++it) {
    const long long slot = ((long long)it * kHkv + kvh) * kG + hh;
    const float m = a.ws_m[slot], l = a.ws_l[slot];
    const float2 x = *reinterpret_cast<const float2*>(a.ws_acc + slot * kD + 2 * lane);
    const float mn = fmaxf(gm, m);
    const float co = exp2f(gm - mn), cn = exp2f(m - mn);
    gl = gl * co + l * cn;
    a0 = a0 * co + x.x * cn;
    a1 = a1 * co + x.y * cn;
    gm = mn;
  }
  const float inv = gl > 0.f ? 1.0f / gl : 0.f;
  const int row = a.cu[a.decode_rids[di]];
  *reinterpret_cast<uint32_t*>(a.out + (long long)row * (kHq * kD) + h * kD + 2 * lane) =
      pack_bf16x2(a0 * inv, a1 * inv);
}

bool dims_ok(const fqa_dims* d) {
  return d && d->n_q_heads == kHq && d->n_kv_heads == kHkv && d->head_dim == kD &&
         d->page_size == kPage && d->qkv_stride >= kQkvStride && d->qkv_stride % 8 == 0;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" {

int64_t fqa_decode_workspace_bytes(const fqa_dims* dims, int32_t dec_item_cap) {
  (void)dims;
  if (dec_item_cap < 0) return 0;
  return (int64_t)dec_item_cap * kHkv * kG * (2 + kD) * (int64_t)sizeof(float);
}

int fqa_decode(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
               int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
               const int32_t* cu_seqlens, const int32_t* positions, const int32_t* dec_items,
               const int32_t* dec_item_start, const int32_t* decode_rids, const int32_t* meta,
               int32_t dec_item_cap, int32_t n_reqs_bound, void* workspace, uint16_t* out,
               void* stream) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (dec_item_cap < 0 || n_reqs_bound < 0 || n_reqs_bound > FQA_MAX_REQS || max_blocks < 1 ||
      pool_pages < 1 || !meta)
    return FQA_EINVAL;
  if (dec_item_cap == 0 || n_reqs_bound == 0) return FQA_OK;
  if (!qkv || !pool || !block_tables || !cu_seqlens || !positions || !dec_items ||
      !dec_item_start || !decode_rids || !workspace || !out)
    return FQA_EINVAL;
  const long long slots = (long long)dec_item_cap * kHkv * kG;
  float* ws = static_cast<float*>(workspace);
  DecArgs a{qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions, dec_items,
            dec_item_start, decode_rids, meta, ws, ws + slots, ws + 2 * slots, out,
            dims->qkv_stride, dims->scale * kLog2e};
  const int waves1 = dec_item_cap * kHkv;
  hipLaunchKernelGGL(decode_split_kernel, dim3((waves1 + kDecWavesPerBlock - 1) / kDecWavesPerBlock),
                     dim3(kDecWavesPerBlock * kWave), 0, (hipStream_t)stream, a);
  const int waves2 = n_reqs_bound * kHq;
  hipLaunchKernelGGL(decode_combine_kernel,
                     dim3((waves2 + kDecWavesPerBlock - 1) / kDecWavesPerBlock),
                     dim3(kDecWavesPerBlock * kWave), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

}  // extern "C"
