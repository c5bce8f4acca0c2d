// fqa_decode.hip — GQA-shared split-K flash decoding over the paged pool (gfx950).
//
// Replaces CuteDecodeSplitKernel + CuteDecodeCombineKernel and their launcher
// (engine/src/attn_cute.cu:165-261).  Same semantics: for every qlen==1 request the
// 4 query heads of each kv head attend keys [0, pos]; scores q.k * scale in fp32;
// online softmax; partials merged by log-sum-exp; output bf16, 0 when l == 0.
//
// MI355X design:
//  * Stream-K split: the (sequence, kv head) page streams of all decode requests are
//    laid end to end and cut into equal shares, one per wavefront of a grid sized to
//    the machine (CUs x resident waves), so every wavefront streams the same number of
//    8 KiB runs and they all finish together (the reference fixes one split factor
//    128/n_decode for every sequence, attn_cute.cu:249-251, which leaves long tails when
//    lengths differ).  A stream inside one share is finished in place; a share boundary
//    that cuts a stream leaves fp32 partials, at most two per wavefront, which a
//    log-sum-exp combine merges.
//  * Each (page, kv head) is one contiguous 8 KiB run (K [16][128] then V^T [128][16])
//    read exactly once for all 4 query heads of the kv head.
//  * Both products run on MFMA in transposed form so that no operand is ever
//    shuffled between lanes:
//        S^T[16 keys x 16 cols] = K[16 x 128] . Q^T[128 x 16]  (4 x mfma 16x16x32 bf16)
//        O^T[128 x 16 cols]    += V^T[128 x 16 keys] . P^T    (2 x 8 x mfma 16x16x16 bf16)
//    Columns 0..3 are the 4 query heads (the rest carry zeros); the S^T accumulator
//    layout (lane = column, 4 consecutive keys per lane) is exactly the B-operand
//    layout P^T needs, and V^T's page layout gives each lane 4 consecutive keys of one
//    dim as one 8-byte load.  The kernel is HBM-bound; MFMA keeps the ALU out of the
//    way (about 5% of the CU's matrix rate at full HBM bandwidth).
//  * P keeps fp32 precision in the PV product, as in the reference: it is split into two
//    bf16 terms (hi + lo) and both go through the MFMA.
//  * One wavefront per SIMD (grid = CUs x 4, one workgroup per CU, which an LDS
//    reservation keeps to itself).  Each wave computes page p while page p+1 loads: one
//    to two 8 KiB pages in flight per wave, 4-8 MiB over the device.  On this part HBM
//    reads go faster with fewer requests in flight: a plain streaming read peaks at one
//    wave per SIMD, and this layout beat two waves per SIMD with one page each by 1% on
//    the 36-layer batch, 5% on the 64-sequence batch and 3% on the mixed step.
#include <mutex>

#include "fqa_common.h"

#include <type_traits>

namespace fqa {
namespace {

constexpr int kDecWavesPerBlock = 4;
// Page buffers per wave: page p is computed while page p+1 loads (180 VGPRs).
constexpr int kDecBufs = 2;
// Page buffers of a shared-prefix item's wavefront: its pages come from the caches (the
// group's other octets read them too), so more are kept in flight.
constexpr int kPrefixBufs = 4;
// A shared-prefix item holds up to 8 members: 2 sets of 16 MFMA columns (4 heads each).
constexpr int kPrefixSets = 2;
constexpr int kPrefixCols = 16 * kPrefixSets;
// LDS reserved by each split-kernel workgroup and never touched: with it one decode
// workgroup (one wave per SIMD) holds a CU alone.  Neither a second decode workgroup nor
// a prefill workgroup (48 KiB) fits beside it; a prefill wave sharing a SIMD with a decode
// wave slowed a mixed step by 30%.
constexpr int kDecExclusiveLds = 120 * 1024;
constexpr float kLog2e = 1.4426950408889634f;

struct DecArgs {
  const uint16_t* qkv;
  const uint16_t* pool;
  long long pool_pages;
  const int32_t* bt;
  int max_blocks;
  const int32_t* waves;  // [G][8] {di, kvh, page, n_runs, r, row, n_keys, first page id}
  const int32_t* seqs;   // [n_decode][4] {r, row, n_keys, 8*P}
  const int32_t* meta;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
  uint16_t* out;
  int stride;
  float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
  int wave_cap;      // rows of `waves`
  // shared-prefix plans (fqa_decode_prefix; NULL otherwise)
  const int32_t* prefix;  // [n_decode][8] {P, first item, C | Q << 16, k}
  const int32_t* pitems;  // [pre_cap][12] {leader, kvh, page0, page1, member x 8}
  float* pws_m;           // prefix partials: [pre_cap][32 columns]
  float* pws_l;
  float* pws_acc;         // [pre_cap][32][128]
  // a member's whole (uncut) stream: its partial, at the column its chunk-0 item gives it
  float* pms_m;
  float* pms_l;
  float* pms_acc;
  int pre_cap;
  int split_blocks;  // decode_split_kernel: workgroups past these run prefix items
};

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

struct PageFrag {
  bf16x8 k[4];
  short4_t v[8];
};

// One page run into registers, through a buffer resource over the 8 KiB run: each load is
// a 32-bit lane offset against one scalar base, not a 64-bit address add per load.  kNT:
// non-temporal loads, for pages no other sequence of the step reads (they stream through
// without displacing shared prefix pages from the caches, and read faster with nothing to
// reuse).  The hint is a template parameter: two copies of the loads that differ only in
// it would be merged.  !live: a zero-length resource, so the loads return zeros without
// touching memory (a refill past the end of a segment).
template <bool kNT>
__device__ __forceinline__ void load_page(PageFrag& f, const uint16_t* run, int lane, bool live) {
  const int m = lane & 15, g = lane >> 4;
  // word 3 0x00020000: the raw-buffer format gfx9 devices expect; num_records bounds the
  // run, so no load can leave it
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)run, (short)0, live ? kRunElems * 2 : 0, 0x00020000);
  constexpr int kAux = kNT ? 2 : 0;  // cache-policy operand: 2 is the nt bit
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (m * kD + ks * 32 + g * 8) * 2, 0, kAux);
    f.k[ks] = __builtin_bit_cast(bf16x8, v);
  }
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const i32x2 v = __builtin_amdgcn_raw_buffer_load_b64(
        rs, (kVOff + (b * 16 + m) * kPage + g * 4) * 2, 0, kAux);
    f.v[b] = __builtin_bit_cast(short4_t, v);
  }
}

struct DecState {
  float4_t acc[8];  // O^T: lane (col = head n, rows d = b*16 + 4g + j)
  float m;          // running max (exp2 domain), same in the 4 lanes of a column
  float l;          // running sum of this lane's 4 keys per page
};

// One page (16 keys) of online softmax for the 4 heads: S^T = K Q^T, P^T = exp2(S^T - m),
// O^T = O^T * corr + V^T P^T.  kFull: every key of the page is below L (no masking).
template <bool kFull>
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
    sv[j] = kFull || key0 + j < L ? s[j] * scale_log2 : -INFINITY;
    mx = fmaxf(mx, sv[j]);
  }
  if (!kFull && (p + 1) * kPage > L) {  // last page: unwritten slots must not reach PV
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key0 + j >= L) f.v[b][j] = 0;
  }
  mx = max_xor32(max_xor16(mx));
  const float m_new = fmaxf(st.m, mx);
  const float corr = __builtin_amdgcn_exp2f(st.m - m_new);
  float pj[4], psum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pj[j] = __builtin_amdgcn_exp2f(sv[j] - m_new);
    psum += pj[j];
  }
  st.l = st.l * corr + psum;
  st.m = m_new;
  // P stays fp32 as in the reference (attn_cute.cu:199): it enters the bf16 MFMA as two
  // bf16 terms, hi = bf16(p) and lo = bf16(p - hi) (p - hi is exact in fp32), so V^T P
  // carries ~16 significand bits of p.  The 8 extra MFMAs per page hide under the page
  // loads (configs 2, 4 and 5 within 0.5%).
  short4_t ph, pl;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t hi = f32_to_bf16_bits(pj[j]);
    ph[j] = (short)hi;
    pl[j] = (short)f32_to_bf16_bits(pj[j] - __uint_as_float(hi << 16));
  }
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    st.acc[b] *= corr;
    st.acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(f.v[b], ph, st.acc[b], 0, 0, 0);
    st.acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(f.v[b], pl, st.acc[b], 0, 0, 0);
  }
}

// Stream pages [pb, pe) of (sequence `seq`, kv head kvh) into `st`.
// kS query sets (16 columns each) over the same pages: one page load feeds kS
// process_page calls (shared-prefix items hold 8 members, 2 sets).  kFull: L = 16 * pe.
template <int kBufs, bool kNT, int kS, bool kFull = false>
__device__ __forceinline__ void stream_pages_n(const DecArgs& a, const int32_t* btr, int kvh,
                                               int pb, int pe, int L, const bf16x8 (&qf)[kS][4],
                                               int lane, DecState (&st)[kS], int first_page) {
  const int g = lane >> 4;
  // Page ids through the constant address space: scalar loads (lgkmcnt), so waiting for an
  // id does not also wait for the page loads issued before it.
  const __attribute__((address_space(4))) int32_t* btc =
      (const __attribute__((address_space(4))) int32_t*)btr;
  // one unsigned 32-bit scalar compare (negative ids wrap above any pool size); a 64-bit
  // compare runs on the VALU and needs a temporary register pair, which the allocator
  // may take from a page buffer still in flight (a full vmcnt drain)
  const uint32_t pool32 = (uint32_t)min(a.pool_pages, (long long)0x7fffffff);
  // (pe > pb: a segment holds at least one page, so min(p, pe - 1) indexes the segment)
  auto load = [&](PageFrag& f, bool& ok, int p) {
    const bool live = p < pe;
    const int page = (p == pb && first_page >= 0) ? first_page : btc[min(p, pe - 1)];
    ok = (uint32_t)page < pool32;
    load_page<kNT>(f, a.pool + run_offset(ok ? page : 0, kvh), lane, live);
  };
  // kBufs page buffers in registers: page p is processed while p+1..p+kBufs-1 are in
  // flight.  The buffers rotate through a kBufs-way unrolled loop so every index is
  // static.  Every refill is issued, past the segment's end as zero-length loads: the
  // compiler then counts the loads exactly and waits only for the page it computes next
  // (with conditional refills it waited for all of them, the refill just issued
  // included, and a wave never computed while its own loads were in flight).
  // A page outside the pool (the pack flags the batch) reads as zeros: its keys score 0
  // and add nothing to the numerator.  The online softmax merge is order-free, so such
  // keys are only counted here and merged into `st` once, after the loop.
  int n_zero = 0;
  PageFrag f[kBufs];
  bool ok[kBufs];
#pragma unroll
  for (int i = 0; i < kBufs; ++i) ok[i] = false;
#pragma unroll
  for (int i = 0; i + 1 < kBufs; ++i) load(f[i], ok[i], pb + i);
  for (int p = pb; p < pe; p += kBufs) {
#pragma unroll
    for (int i = 0; i < kBufs; ++i) {
      if (i > 0 && p + i >= pe) break;
      load(f[(i + kBufs - 1) % kBufs], ok[(i + kBufs - 1) % kBufs], p + i + kBufs - 1);
      if (ok[i]) {
#pragma unroll
        for (int q = 0; q < kS; ++q) process_page<kFull>(f[i], qf[q], p + i, L, g, a.scale_log2, st[q]);
      } else {
        n_zero += min(kPage, L - (p + i) * kPage);
      }
    }
  }
  if (n_zero > 0) {  // n_zero keys with score 0 and value 0 (uniform, rare)
#pragma unroll
    for (int q = 0; q < kS; ++q) {
      const float m_new = fmaxf(st[q].m, 0.f);
      const float corr = __builtin_amdgcn_exp2f(st[q].m - m_new);
      // st.l holds this lane's share of the row sum (summed over the 4 lanes of a column
      // at the end): lane group g = 0 takes the zero keys
      st[q].l = st[q].l * corr +
                ((lane >> 4) == 0 ? (float)n_zero * __builtin_amdgcn_exp2f(-m_new) : 0.f);
      st[q].m = m_new;
#pragma unroll
      for (int b = 0; b < 8; ++b) st[q].acc[b] *= corr;
    }
  }
}

template <int kBufs, bool kNT>
__device__ __forceinline__ void stream_pages(const DecArgs& a, const int32_t* btr, int kvh,
                                             int pb, int pe, int L, const bf16x8 (&qf)[4],
                                             int lane, DecState& st, int first_page) {
  stream_pages_n<kBufs, kNT, 1>(a, btr, kvh, pb, pe, L,
                                reinterpret_cast<const bf16x8(&)[1][4]>(qf), lane,
                                reinterpret_cast<DecState(&)[1]>(st), first_page);
}

// Column of member k (its k-th member, in decode order) of a shared-prefix group, head n,
// in the prefix partials of chunk c: item (first item + (kvh * C + c) * Q + k / 8),
// column (k % 8) * 4 + n.
__device__ __forceinline__ long long prefix_slot(const int4 info, int kvh, int c, int n) {
  const int C = info.z & 0xFFFF, Q = info.z >> 16, k = info.w;
  return ((long long)info.y + ((long long)kvh * C + c) * Q + (k >> 3)) * kPrefixCols +
         (k & 7) * kG + n;
}

// The pack's items fit dec_pre_cap; a workspace planned for fewer is never touched past its
// end (the group's rows are then left out).
__device__ __forceinline__ bool prefix_fits(const int4 info, int pre_cap) {
  const int C = info.z & 0xFFFF, Q = info.z >> 16;
  return (long long)info.y + 8LL * C * Q <= pre_cap;
}

// Shared-prefix item w, run by decode_split_kernel's workgroups past its shares (they take
// the CUs the shares leave as they finish): one wavefront streams pages [page0, page1) of
// the group leader's table (which its members' tables equal there) once for the 4 query
// heads of each of up to 8 members (2 sets of 16 MFMA columns: member j, head h at column
// 4j + h), with the decode's page loop and arithmetic, and leaves the 32 columns' fp32
// partials.
__device__ __forceinline__ void prefix_item(const DecArgs& a, int w) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int n_items = a.meta[FQA_META_DEC_PRE_ITEMS];
  if (w >= n_items || w >= a.pre_cap) return;
  const int4* it = reinterpret_cast<const int4*>(a.pitems + 12LL * w);
  const int4 i0 = it[0], i1 = it[1], i2 = it[2];
  const int lead = __builtin_amdgcn_readfirstlane(i0.x), kvh = __builtin_amdgcn_readfirstlane(i0.y);
  const int p0 = __builtin_amdgcn_readfirstlane(i0.z), p1 = __builtin_amdgcn_readfirstlane(i0.w);
  const int r = __builtin_amdgcn_readfirstlane(a.seqs[4LL * lead]);
  const int mem[8] = {i1.x, i1.y, i1.z, i1.w, i2.x, i2.y, i2.z, i2.w};
  bf16x8 qf[kPrefixSets][4];
  DecState st[kPrefixSets];
#pragma unroll
  for (int q = 0; q < kPrefixSets; ++q) {
    const int mj = mem[4 * q + (n >> 2)];
    if (mj >= 0) {
      const int row = a.seqs[4LL * mj + 1];
      const uint16_t* src = a.qkv + (long long)row * a.stride + (kvh * kG + (n & 3)) * kD + g * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[q][ks] = *reinterpret_cast<const bf16x8*>(src + ks * 32);
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[q][ks][i] = (__bf16)0.0f;
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) st[q].acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};
    st[q].m = -1e30f;
    st[q].l = 0.f;
  }
  // every key of [page0, page1) precedes each member's own (the prefix ends at or before
  // computed / 16 pages), so no key is masked: L = 16 * page1.  An item whose second set
  // is empty (4 members or fewer) streams the first set alone.
  const int32_t* btr = a.bt + (long long)r * a.max_blocks;
  if (__builtin_amdgcn_readfirstlane(i2.x) >= 0)
    stream_pages_n<kPrefixBufs, false, kPrefixSets, true>(a, btr, kvh, p0, p1, p1 * kPage, qf, lane,
                                                    st, -1);
  else
    stream_pages_n<kPrefixBufs, false, 1, true>(a, btr, kvh, p0, p1, p1 * kPage,
                                          reinterpret_cast<const bf16x8(&)[1][4]>(qf[0]), lane,
                                          reinterpret_cast<DecState(&)[1]>(st[0]), -1);
#pragma unroll
  for (int q = 0; q < kPrefixSets; ++q) {
    const float l_run = sum_rows4(st[q].l);
    const long long slot = (long long)w * kPrefixCols + 16 * q + n;
    if (g == 0) {
      a.pws_m[slot] = st[q].m;
      a.pws_l[slot] = l_run;
    }
    float* wa = a.pws_acc + slot * kD + g * 4;
#pragma unroll
    for (int b = 0; b < 8; ++b) *reinterpret_cast<float4_t*>(wa + b * 16) = st[q].acc[b];
  }
}

// One wavefront per share of the stream-K plan.  A share walks consecutive streams:
// the first may start mid-stream, the last may end mid-stream, the ones between are
// whole.  Whole streams are written as bf16 output; a cut stream leaves its partial in
// slot 2w (the share's first stream) or 2w+1 (its last).
template <int kBufs>
__global__ void __launch_bounds__(kDecWavesPerBlock * kWave) decode_split_kernel(DecArgs a) {
  __shared__ char lds_excl[kDecExclusiveLds];  // allocated, never accessed
  asm volatile("" ::"s"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds_excl));
  if (blockIdx.x >= a.split_blocks) {  // shared-prefix items, dispatched as CUs free up
    prefix_item(a, (blockIdx.x - a.split_blocks) * kDecWavesPerBlock +
                       __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    return;
  }
  // Everything a wave's loop indexes with is wave-uniform; readfirstlane says so, so that
  // block-table reads become scalar loads (see stream_pages).
  const int w = blockIdx.x * kDecWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  auto uni4 = [](int4 v) {
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  };
  // The wave's descriptor is read together with the wave count (one round trip, not two):
  // the row is in bounds for every wave of the grid, live or not.
  const int4* wd = reinterpret_cast<const int4*>(a.waves + 8 * (long long)min(w, a.wave_cap - 1));
  const int4 desc = uni4(wd[0]);
  int4 sq = uni4(wd[1]);  // {r, row, L, page id}
  const int n_waves = a.meta[FQA_META_DEC_WAVES];
  asm volatile("" ::"s"(desc.x), "s"(n_waves));  // both loads issued before the branch
  if (w >= n_waves) return;
  int di = desc.x, kvh = desc.y, page = desc.z, left = desc.w;
  // shared-prefix plans: a stream covers pages [P, pages) of its sequence; the row also
  // locates the group's prefix partials
  auto prefix_row = [&](int d) {
    const int4 v = *reinterpret_cast<const int4*>(a.prefix + 8LL * d);
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  };
  int4 pinfo = a.prefix ? prefix_row(di) : make_int4(0, 0, 0, 0);
  int P = pinfo.x;
  for (int seg = 0; left > 0; ++seg) {
    if (seg > 0) {
      sq = uni4(*reinterpret_cast<const int4*>(a.seqs + 4 * (long long)di));
      sq.w = -1;  // first page id of a later stream: read from the block table
      if (a.prefix) pinfo = prefix_row(di);
      P = pinfo.x;
      page = P;
    }
    // sequences that share their first page read through the caches (FQA_DEC_SHARED)
    const int r = sq.x, row = sq.y, L = sq.z & FQA_DEC_KEYS_MASK;
    const bool shared = (sq.z & FQA_DEC_SHARED) != 0;
    const int pages = (L + kPage - 1) / kPage;
    const int cnt = min(pages - page, left);

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
    if (shared)
      stream_pages<kBufs, false>(a, a.bt + (long long)r * a.max_blocks, kvh, page, page + cnt, L,
                                 qf, lane, st, sq.w);
    else
      stream_pages<kBufs, true>(a, a.bt + (long long)r * a.max_blocks, kvh, page, page + cnt, L,
                                qf, lane, st, sq.w);
    const float l_run = sum_rows4(st.l);

    if (n < kG) {
      if (page == P && cnt == pages - P && P > 0) {
        // a shared-prefix member's whole stream: the combine merges it with the prefix
        if (prefix_fits(pinfo, a.pre_cap)) {
          const long long slot = prefix_slot(pinfo, kvh, 0, n);
          if (g == 0) {
            a.pms_m[slot] = st.m;
            a.pms_l[slot] = l_run;
          }
          float* wa = a.pms_acc + slot * kD + g * 4;
#pragma unroll
          for (int b = 0; b < 8; ++b) *reinterpret_cast<float4_t*>(wa + b * 16) = st.acc[b];
        }
      } else if (page == P && cnt == pages - P) {  // whole stream: final output
        const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
        uint16_t* o = a.out + (long long)row * (kHq * kD) + (kvh * kG + n) * kD + g * 4;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          uint2 v = make_uint2(pack_bf16x2(st.acc[b][0] * inv, st.acc[b][1] * inv),
                               pack_bf16x2(st.acc[b][2] * inv, st.acc[b][3] * inv));
          *reinterpret_cast<uint2*>(o + b * 16) = v;
        }
      } else {
        const long long slot = (2LL * w + (seg > 0)) * kG + n;
        if (g == 0) {
          a.ws_m[slot] = st.m;
          a.ws_l[slot] = l_run;
        }
        float* wa = a.ws_acc + slot * kD + g * 4;
#pragma unroll
        for (int b = 0; b < 8; ++b) *reinterpret_cast<float4_t*>(wa + b * 16) = st.acc[b];
      }
    }
    left -= cnt;
    page = P;
    if (++kvh == kHkv) {
      kvh = 0;
      ++di;
    }
  }
}

// The HBM read floor of a decode plan: the same wavefront grid walks the same shares of
// the same (page, kv head) runs with the same per-lane loads as decode_split_kernel, but
// does no arithmetic beyond folding the loaded words into one value per lane.  The page
// loop is stream_pages' own (kDecBufs rotating buffers, every refill issued), and it
// reserves the same LDS, so its workgroups sit on the CUs as the decode's do.  The time
// of this kernel is what reading the decode's bytes in its access
// pattern costs on the device; decode_split_kernel's time over it is the price of the
// attention math and the bookkeeping.  `a.ws_m` receives one word per lane (the sink).
__global__ void __launch_bounds__(kDecWavesPerBlock * kWave) decode_read_floor_kernel(DecArgs a) {
  __shared__ char lds_excl[kDecExclusiveLds];  // placement as decode_split_kernel
  asm volatile("" ::"s"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds_excl));
  const int w = blockIdx.x * kDecWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int4 desc =
      *reinterpret_cast<const int4*>(a.waves + 8 * (long long)min(w, a.wave_cap - 1));
  const int n_waves = a.meta[FQA_META_DEC_WAVES];
  asm volatile("" ::"s"(desc.x), "s"(n_waves));  // one round trip, as decode_split_kernel
  if (w >= n_waves) return;
  int di = __builtin_amdgcn_readfirstlane(desc.x), kvh = __builtin_amdgcn_readfirstlane(desc.y);
  int page = __builtin_amdgcn_readfirstlane(desc.z), left = __builtin_amdgcn_readfirstlane(desc.w);
  const uint32_t pool32 = (uint32_t)min(a.pool_pages, (long long)0x7fffffff);
  uint32_t sink = 0;
  while (left > 0) {
    const int4 sq = *reinterpret_cast<const int4*>(a.seqs + 4 * (long long)di);
    const int P = a.prefix ? __builtin_amdgcn_readfirstlane(a.prefix[8LL * di]) : 0;
    const int r = __builtin_amdgcn_readfirstlane(sq.x);
    const int zf = __builtin_amdgcn_readfirstlane(sq.z);
    const int L = zf & FQA_DEC_KEYS_MASK;
    const bool shared = (zf & FQA_DEC_SHARED) != 0;  // the same load hints as the decode
    const int pages = (L + kPage - 1) / kPage;
    if (page < 0) page = P;
    const int cnt = min(pages - page, left);
    const __attribute__((address_space(4))) int32_t* btc =
        (const __attribute__((address_space(4))) int32_t*)(a.bt + (long long)r * a.max_blocks);
    auto walk = [&](auto nt_tag) {
      constexpr bool kNT = decltype(nt_tag)::value;
      const int pe = page + cnt;
      constexpr int kB = kDecBufs;
      PageFrag f[kB];
      auto ld = [&](PageFrag& x, int p) {
        const int id = btc[min(p, pe - 1)];
        load_page<kNT>(x, a.pool + run_offset((uint32_t)id < pool32 ? id : 0, kvh), lane, p < pe);
      };
      auto fold = [&](const PageFrag& x) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const uint4 k = __builtin_bit_cast(uint4, x.k[ks]);
          sink ^= k.x ^ k.y ^ k.z ^ k.w;
        }
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const uint2 v = __builtin_bit_cast(uint2, x.v[b]);
          sink ^= v.x ^ v.y;
        }
      };
#pragma unroll
      for (int i = 0; i + 1 < kB; ++i) ld(f[i], page + i);
      for (int p = page; p < pe; p += kB) {
#pragma unroll
        for (int i = 0; i < kB; ++i) {
          if (i > 0 && p + i >= pe) break;
          ld(f[(i + kB - 1) % kB], p + i + kB - 1);
          fold(f[i]);  // a zero-length load folds in zeros
        }
      }
    };
    if (shared)
      walk(std::false_type{});
    else
      walk(std::true_type{});
    left -= cnt;
    page = -1;  // the next stream's first page: P, known once its sequence is read
    if (++kvh == kHkv) {
      kvh = 0;
      ++di;
    }
  }
  reinterpret_cast<uint32_t*>(a.ws_m)[(long long)w * kWave + lane] = sink;
}

// Log-sum-exp merge of a cut stream's partials (attn_cute.cu:225-238): one wave per
// (decode sequence, kv head) stream, lane -> (head = lane/16, 8 dims).  A shared-prefix
// member's stream is always merged: its group's C prefix chunk partials, then its own.
// Stream s's pages take positions [F, S1), u per page, and a page belongs to the share
// holding its last position: the shares w_first..w_last (share w = [w*W/G, (w+1)*W/G))
// hold F + u - 1 and S1 - 1.  The stream is the last of w_first's streams (slot 2w+1), or
// its first (slot 2w) when w_first's share starts in s's own cost span [S0, F + u), and
// the first of every later share (slot 2w).
__global__ void __launch_bounds__(kDecWavesPerBlock * kWave) decode_combine_kernel(DecArgs a) {
  const int wave = blockIdx.x * kDecWavesPerBlock + (threadIdx.x >> 6);
  const int di = wave >> 3, kvh = wave & 7;
  // di < n_reqs_bound, the rows of `seqs`: the sequence is read with the counts (one round
  // trip, not two)
  const int4 sq = *reinterpret_cast<const int4*>(a.seqs + 4 * (long long)di);
  // the next sequence's cost start (the grid has 8 waves per row of `seqs`)
  const int nb = gridDim.x * kDecWavesPerBlock / kHkv;
  const int w_next = a.seqs[4 * (long long)min(di + 1, nb - 1) + 3];
  const int4 pinfo = a.prefix ? *reinterpret_cast<const int4*>(a.prefix + 8LL * di)
                              : make_int4(0, 0, 0, 0);
  const int pfx = pinfo.x;
  const int n_dec = a.meta[FQA_META_N_DECODE];
  asm volatile("" ::"v"(sq.x), "v"(pfx), "v"(w_next), "s"(n_dec));
  if (di >= n_dec) return;
  const long long G = a.meta[FQA_META_DEC_WAVES];
  // the plan's cost positions (fqa.h): each stream's start positions, then its pages
  const long long W = a.meta[FQA_META_DEC_COST];
  // a stream's pages: [P, pages) with a shared prefix
  const int pages = ((sq.z & FQA_DEC_KEYS_MASK) + kPage - 1) / kPage - pfx;
  const int sc = FQA_DEC_STREAM_COST + (pfx > 0 ? FQA_DEC_PREFIX_STREAM_COST : 0);
  // the stream's cost, 1/8 of the sequence's span, gives its page cost u
  const long long c = ((di + 1 < n_dec ? (long long)w_next : W) - sq.w) / kHkv;
  const int u = (int)((c - sc) / pages);
  const long long S0 = sq.w + (long long)kvh * c;
  const long long F = S0 + sc, S1 = F + (long long)pages * u;  // page positions [F, S1)
  // a page belongs to the share holding its last position: the first page's is F + u - 1,
  // the last page's S1 - 1
  const long long wf = ((F + u) * G - 1) / W, wl = (S1 * G - 1) / W;
  // a stream finished by one wavefront is final, unless a shared prefix precedes it
  if (wf == wl && pfx == 0) return;
  if (pfx > 0 && !prefix_fits(pinfo, a.pre_cap)) return;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 4, d0 = (lane & 15) * 8;
  float gm = -1e30f, gl = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto merge = [&](float m, float l, float4 x0, float4 x1) {
    const float mn = fmaxf(gm, m);
    const float co = exp2f(gm - mn), cn = exp2f(m - mn);
    gl = gl * co + l * cn;
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * co + xs[i] * cn;
    gm = mn;
  };
  // a shared prefix's C chunk partials (and, for a stream no wavefront cut, the stream's
  // own partial), 4 loads in flight at a time
  if (pfx > 0) {
    const int C = pinfo.z & 0xFFFF;
    const int nc = C + (wf == wl);
    for (int c0 = 0; c0 < nc; c0 += 4) {
      float m[4], l[4];
      float4 x0[4], x1[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c = min(c0 + k, nc - 1);
        const bool own = c == C;  // the uncut stream's partial
        const long long slot = prefix_slot(pinfo, kvh, own ? 0 : c, h);
        m[k] = (own ? a.pms_m : a.pws_m)[slot];
        l[k] = (own ? a.pms_l : a.pws_l)[slot];
        const float4* src =
            reinterpret_cast<const float4*>((own ? a.pms_acc : a.pws_acc) + slot * kD + d0);
        x0[k] = src[0];
        x1[k] = src[1];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (c0 + k < nc) merge(m[k], l[k], x0[k], x1[k]);
    }
  }
  // the cut stream's partials in batches of 4: all loads of a batch are issued before any
  // is used
  for (long long w0 = wf; w0 <= wl && wf < wl; w0 += 4) {
    float m[4], l[4];
    float4 x0[4], x1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const long long w = w0 + k;
      // the stream is wf's first unless wf's share starts in an earlier stream
      const long long sl = (w == wf && wf * W / G < S0) ? 2 * w + 1 : 2 * w;
      const long long slot = (w <= wl ? sl : 2 * wf) * kG + h;  // beyond wl: harmless reread
      m[k] = a.ws_m[slot];
      l[k] = a.ws_l[slot];
      const float4* src = reinterpret_cast<const float4*>(a.ws_acc + slot * kD + d0);
      x0[k] = src[0];
      x1[k] = src[1];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (w0 + k <= wl) merge(m[k], l[k], x0[k], x1[k]);
  }
  const float inv = gl > 0.f ? 1.0f / gl : 0.f;
  uint4 v = make_uint4(pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv),
                       pack_bf16x2(acc[4] * inv, acc[5] * inv), pack_bf16x2(acc[6] * inv, acc[7] * inv));
  *reinterpret_cast<uint4*>(a.out + (long long)sq.y * (kHq * kD) + (kvh * kG + h) * kD + d0) = v;
}

bool dims_ok(const fqa_dims* d) {
  return d && d->n_q_heads == kHq && d->n_kv_heads == kHkv && d->head_dim == kD &&
         d->page_size == kPage && d->qkv_stride >= kQkvStride && d->qkv_stride % 8 == 0;
}

// The checks and launches of fqa_decode with the partials in `ws` (fp32 m, l, acc for
// 2 * dec_wave_cap * 4 head slots).
int decode_launch(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                  int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                  const int32_t* dec_waves, const int32_t* dec_seqs, const int32_t* meta,
                  int32_t dec_wave_cap, int32_t n_reqs_bound, float* ws, uint16_t* out,
                  hipStream_t stream, const int32_t* dec_prefix = nullptr,
                  const int32_t* dec_pre_items = nullptr, int32_t dec_pre_cap = 0) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (dec_wave_cap < 0 || n_reqs_bound < 0 || n_reqs_bound > FQA_MAX_REQS || max_blocks < 1 ||
      pool_pages < 1 || !meta)
    return FQA_EINVAL;
  if (dec_wave_cap == 0 || n_reqs_bound == 0) return FQA_OK;
  if (!qkv || !pool || !block_tables || !dec_waves || !dec_seqs || !ws || !out)
    return FQA_EINVAL;
  const long long slots = 2LL * dec_wave_cap * kG;
  DecArgs a{qkv, pool, pool_pages, block_tables, max_blocks, dec_waves, dec_seqs, meta, ws,
            ws + slots, ws + 2 * slots, out, dims->qkv_stride, dims->scale * kLog2e, dec_wave_cap};
  if (dec_prefix) {
    // after the stream partials: the prefix chunk partials, m, l [pre_cap][32] and acc
    // [pre_cap][32][128], then as many for the members' uncut streams
    float* pws = ws + slots * (2 + kD);
    const long long ps = (long long)kPrefixCols * dec_pre_cap;
    a.prefix = dec_prefix;
    a.pitems = dec_pre_items;
    a.pws_m = pws;
    a.pws_l = pws + ps;
    a.pws_acc = pws + 2 * ps;
    float* pms = pws + ps * (2 + kD);
    a.pms_m = pms;
    a.pms_l = pms + ps;
    a.pms_acc = pms + 2 * ps;
    a.pre_cap = dec_pre_cap;
  }
  a.split_blocks = (dec_wave_cap + kDecWavesPerBlock - 1) / kDecWavesPerBlock;
  const int pre_blocks = a.prefix ? (dec_pre_cap + kDecWavesPerBlock - 1) / kDecWavesPerBlock : 0;
  hipLaunchKernelGGL(decode_split_kernel<kDecBufs>, dim3(a.split_blocks + pre_blocks),
                     dim3(kDecWavesPerBlock * kWave), 0, stream, a);
  const int waves2 = n_reqs_bound * kHkv;
  hipLaunchKernelGGL(decode_combine_kernel,
                     dim3((waves2 + kDecWavesPerBlock - 1) / kDecWavesPerBlock),
                     dim3(kDecWavesPerBlock * kWave), 0, stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}


// ---- fqa_decode_noalloc: the decode partials in a file-scope device array ----------
// Callers that cannot allocate (graph capture, serving loops that forbid hipMalloc) get
// the partials in `scratch`, sized for FQA_DECODE_NOALLOC_MAX_WAVES wavefronts
// (17,039,360 bytes), which every device the library runs on holds until the process
// ends.  Host code never passes `scratch` itself (in host code the name is a stand-in,
// not a device address): its device address is looked up once per device with
// hipGetSymbolAddress and kept in scratch_ptr[].  The split kernel writes every partial
// slot the combine reads in the same call, so nothing has to start at zero.
constexpr size_t kScratchBytes =
    2ull * FQA_DECODE_NOALLOC_MAX_WAVES * kG * (2 + kD) * sizeof(float);
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on its first use on the device.
int scratch_address(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FQA_ELAUNCH;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return FQA_ELAUNCH;
    scratch_ptr[dev] = p;
  }
  *out = static_cast<float*>(scratch_ptr[dev]);
  return FQA_OK;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" {

int64_t fqa_decode_workspace_bytes(const fqa_dims* dims, int32_t dec_wave_cap) {
  (void)dims;
  if (dec_wave_cap < 0) return 0;
  return 2LL * dec_wave_cap * kG * (2 + kD) * (int64_t)sizeof(float);
}

int fqa_decode(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
               int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
               const int32_t* dec_waves, const int32_t* dec_seqs, const int32_t* meta,
               int32_t dec_wave_cap, int32_t n_reqs_bound, void* workspace, uint16_t* out,
               void* stream) {
  return decode_launch(dims, qkv, pool, pool_pages, block_tables, max_blocks, dec_waves,
                       dec_seqs, meta, dec_wave_cap, n_reqs_bound,
                       static_cast<float*>(workspace), out, (hipStream_t)stream);
}

int fqa_decode_noalloc(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                       int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                       const int32_t* dec_waves, const int32_t* dec_seqs, const int32_t* meta,
                       int32_t dec_wave_cap, int32_t n_reqs_bound, uint16_t* out,
                       void* stream) {
  if (dec_wave_cap > FQA_DECODE_NOALLOC_MAX_WAVES) return FQA_EINVAL;
  float* ws = nullptr;
  if (dec_wave_cap > 0 && n_reqs_bound > 0) {
    const int rc = scratch_address(&ws);
    if (rc != FQA_OK) return rc;
  }
  return decode_launch(dims, qkv, pool, pool_pages, block_tables, max_blocks, dec_waves,
                       dec_seqs, meta, dec_wave_cap, n_reqs_bound, ws, out, (hipStream_t)stream);
}

int fqa_decode_read_floor_prefix(const uint16_t* pool, int64_t pool_pages,
                                 const int32_t* block_tables, int32_t max_blocks,
                                 const int32_t* dec_waves, const int32_t* dec_seqs,
                                 const int32_t* dec_prefix, const int32_t* meta,
                                 int32_t dec_wave_cap, void* sink, void* stream) {
  if (dec_wave_cap < 0 || max_blocks < 1 || pool_pages < 1 || !meta) return FQA_EINVAL;
  if (dec_wave_cap == 0) return FQA_OK;
  if (!pool || !block_tables || !dec_waves || !dec_seqs || !sink) return FQA_EINVAL;
  DecArgs a{nullptr, pool, pool_pages, block_tables, max_blocks, dec_waves, dec_seqs, meta,
            static_cast<float*>(sink), nullptr, nullptr, nullptr, kQkvStride, 0.f, dec_wave_cap};
  a.prefix = dec_prefix;
  hipLaunchKernelGGL(decode_read_floor_kernel,
                     dim3((dec_wave_cap + kDecWavesPerBlock - 1) / kDecWavesPerBlock),
                     dim3(kDecWavesPerBlock * kWave), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

int fqa_decode_read_floor(const uint16_t* pool, int64_t pool_pages, const int32_t* block_tables,
                          int32_t max_blocks, const int32_t* dec_waves, const int32_t* dec_seqs,
                          const int32_t* meta, int32_t dec_wave_cap, void* sink, void* stream) {
  return fqa_decode_read_floor_prefix(pool, pool_pages, block_tables, max_blocks, dec_waves,
                                      dec_seqs, nullptr, meta, dec_wave_cap, sink, stream);
}

int64_t fqa_decode_prefix_workspace_bytes(const fqa_dims* dims, int32_t dec_wave_cap,
                                          int32_t dec_pre_cap) {
  if (dec_wave_cap < 0 || dec_pre_cap < 0) return 0;
  return fqa_decode_workspace_bytes(dims, dec_wave_cap) +
         2 * (int64_t)kPrefixCols * dec_pre_cap * (2 + kD) * (int64_t)sizeof(float);
}

int fqa_decode_prefix(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                      int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                      const int32_t* dec_waves, const int32_t* dec_seqs,
                      const int32_t* dec_prefix, const int32_t* dec_pre_items,
                      const int32_t* meta, int32_t dec_wave_cap, int32_t dec_pre_cap,
                      int32_t n_reqs_bound, void* workspace, uint16_t* out, void* stream) {
  if (dec_pre_cap < 0 || !dec_prefix || (dec_pre_cap > 0 && !dec_pre_items)) return FQA_EINVAL;
  return decode_launch(dims, qkv, pool, pool_pages, block_tables, max_blocks, dec_waves,
                       dec_seqs, meta, dec_wave_cap, n_reqs_bound,
                       static_cast<float*>(workspace), out, (hipStream_t)stream, dec_prefix,
                       dec_pre_items, dec_pre_cap);
}

}  // extern "C"
