// fqa_prefill.hip — varlen causal FlashAttention-2 prefill over the paged pool (gfx950).
//
// Replaces CutePrefillKernel + LaunchAttnPrefillCute (engine/src/attn_cute.cu:30-163).
// Same semantics: for each qlen != 1 request and each of its rows, head h attends the
// keys of kv head h/4 with key pos <= query pos (the cached prefix included); scores
// q.k * scale in fp32; online softmax; P rounded to bf16 before PV (attn_cute.cu:128);
// fp32 accumulation; output bf16, 0 when l == 0.
//
// MI355X design:
//  * One 256-thread workgroup per (query tile, kv head); wave w owns query head w of the
//    kv head.  The 4 heads share every K/V tile, staged into LDS once (the reference runs
//    one block per query head and re-reads K/V 4x, attn_cute.cu:157).
//  * Two tile heights.  64 rows (the default): each wave runs two 32-row blocks, so every
//    K and V^T fragment it reads from LDS feeds two MFMAs and each staged half serves
//    twice the FLOPs; 256 registers, two workgroups per CU.  32 rows: 168 VGPRs, three
//    workgroups per CU, the next half's S^T MFMAs interleaved with this half's softmax.
//  * Transposed FA-2 on v_mfma_f32_32x32x16_bf16:
//        S^T[32 keys x 32 rows] = K[32 x 128] . Q^T[128 x 32]   (8 MFMAs per 32 keys)
//        O^T[128 x 32 rows]    += V^T[128 x 16 keys] . P^T      (4 MFMAs per 16 keys)
//    With rows as accumulator columns every lane owns one query row: the softmax row
//    max / sum is 16 in-lane values plus one exchange with lane^32, the rescale of O is
//    a per-lane scalar, and the S^T accumulator registers are already the P^T operand.
//    MFMA row r of S^T holds key perm(r) (bits 2 and 3 of r swapped), so the 8 keys a
//    lane half contributes to one page's PV step are 8 consecutive tokens: one 16-byte
//    chunk of the page's V^T row.
//  * Per score the softmax costs about as much VALU issue as the MFMAs take (a wave64
//    VALU op issues in ~4.5 cycles, exp in ~8-11), so it is kept minimal and hidden
//    behind MFMAs: scores are maxed raw, scaled inside the exp2 FMA, converted with
//    v_cvt_pk_bf16_f32, summed two at a time with v_dot2 against (1, 1), and O is
//    rescaled lazily (only when the row max grows by more than 2^8).  Measured, the
//    per-half staging (the 4 global->LDS instructions per wave, ~10% of the kernel) and
//    the softmax (~9%) are the largest costs after the MFMAs themselves.
//  * 32-row tiles: half t's exp/convert/sum is interleaved with the S^T MFMAs of half t+1
//    and the LDS reads of half t's V fragments, then half t's PV MFMAs issue back to back.
//    64-row tiles have no registers for a second S^T tile: per half the exps, the PV MFMAs
//    and half t+1's S^T MFMAs run in turn (fragments read one MFMA pair ahead), and the
//    other workgroup's wave on the SIMD fills the gaps.
//  * K/V staging is direct global->LDS (global_load_lds_dwordx4): a ring of three 16 KiB
//    buffers, one 32-key half (two 8 KiB page runs) each, filled two halves ahead.
//    Each wave moves one 4 KiB region (K or V^T of one page) per half; every lane picks
//    the global chunk that lands in its slot of the LDS layout (K chunk-major, V^T
//    XOR-swizzled), so fragment reads are conflict-free 16-byte reads and no VGPR
//    carries staged data.  The loads
//    are issued from inline assembly, so the compiler neither tracks them nor inserts
//    its own conservative waits: every wait on them is an explicit vmcnt count followed
//    by a barrier.  Vector-memory loads return in order, so other loads in the loop (the
//    64-row tile's register reloads, off the common path) can only make a count wait
//    longer, never too little.
//  * Work items come from the pack sorted by key count, longest first.

#include "fqa_common.h"

#include <type_traits>

namespace fqa {
namespace {

constexpr int kQT = 32;          // query rows per workgroup
constexpr int kHalfKeys = 32;    // keys per pipeline step (2 pages)
constexpr int kRunBytes = kRunElems * 2;       // 8 KiB: one (page, kv head) run
constexpr int kHalfBytes = 2 * kRunBytes;      // 16 KiB LDS buffer
constexpr int kRing = 3;                       // LDS buffers
constexpr int kAhead = kRing - 1;              // halves loaded ahead of the current one
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

// One 16-byte-per-lane global->LDS load: lane i's 16 bytes at base + off land at LDS
// byte lds + 16 i (`base` and `lds` wave-uniform).  The LDS address is an operand bound
// to M0, so the compiler owns M0; the LDS DMA needs one wait state after an M0 write.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "{m0}"(lds)
      : "memory");
}

// K layout in a page slot's LDS run, chunk-major: chunk (16 B = 8 dims) c of token t at
// byte c*256 + t*16.  The 16 tokens' reads of one chunk are 256 consecutive bytes (no bank
// conflict), and a lane's 8 K-fragment reads differ only by the constant ks*512.
__device__ __forceinline__ int lds_k(int ps, int t, int c) { return ps * kRunBytes + c * 256 + t * 16; }
// LDS byte offset of V^T chunk `h` (tokens 8h..8h+7) of dim row `d` in page slot `ps`.
// The swizzle h ^ bit3(d) keeps the 16-byte reads of 16 consecutive rows on distinct
// banks.
__device__ __forceinline__ int lds_v(int ps, int d, int h) {
  return ps * kRunBytes + kVOff * 2 + d * 32 + ((h ^ ((d >> 3) & 1)) << 4);
}

// Keep the first `valid` (0..16) tokens of 8 bf16 tokens t0.. of one V^T row.
__device__ __forceinline__ uint4 keep_tokens8(uint4 v, int t0, int valid) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ta = t0 + 2 * i;
    w[i] &= (ta < valid ? 0x0000ffffu : 0u) | (ta + 1 < valid ? 0xffff0000u : 0u);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// s_waitcnt with only vmcnt constrained (expcnt and lgkmcnt at their maxima).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// Workgroup barrier without the release fence __syncthreads adds (that fence would wait
// for every outstanding global->LDS load); the memory clobber keeps the compiler from
// moving LDS accesses across it.  Callers wait for what they need first.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// kRW row blocks of 32 rows per wave: wave w is query head w of the kv head for all 32 kRW
// rows of the item, and every K and V^T fragment it reads from LDS feeds kRW MFMAs.  One
// row block (168 VGPRs) runs 3 workgroups per CU; two (256) run 2 and halve the LDS
// fragment reads and staging instructions per FLOP.
template <int kRW>
__global__ void __launch_bounds__(256, kRW == 1 ? 3 : 2) prefill_kernel(PreArgs a) {
  constexpr int kLoads = 4;  // global->LDS loads per wave per half
  __shared__ __attribute__((aligned(1024))) char lds[kRing * kHalfBytes];
  auto ring = [&](int t) { return lds + (t % kRing) * kHalfBytes; };
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  const int item = blockIdx.x >> 3, kvh = blockIdx.x & 7;
  // the descriptor load does not wait for the count check (slots up to the grid bound
  // are readable)
  const int n_items = a.meta[FQA_META_PRE_ITEMS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = w;  // query head within the kv head
  const int4 it = *reinterpret_cast<const int4*>(a.items + 4 * (long long)item);
  asm volatile("" ::"s"(it.x), "s"(it.w), "s"(n_items));  // both loads before the check
  if (item >= n_items) return;
  const int r = __builtin_amdgcn_readfirstlane(it.x), q0 = __builtin_amdgcn_readfirstlane(it.y);
  const int q1 = __builtin_amdgcn_readfirstlane(it.z), nkeys = __builtin_amdgcn_readfirstlane(it.w);
  const int qs = a.cu[r];
  const int32_t* btr = a.bt + (long long)r * a.max_blocks;
  // The block tables are read-only for the kernel's lifetime: read them through the
  // constant address space so the loads are scalar.
  const __attribute__((address_space(4))) int32_t* btr_c =
      (const __attribute__((address_space(4))) int32_t*)btr;
  const int n_half = (nkeys + kHalfKeys - 1) / kHalfKeys;
  const int n_pages = (nkeys + kPage - 1) / kPage;

  const int col = lane & 31, hf = lane >> 5;
  // A request's new rows sit at positions computed .. computed+qlen-1 (the pack writes
  // positions[] that way, scheduler.h:66-72), and n_keys = computed + q1.
  const int computed = nkeys - q1;
  int i_row[kRW], qpos[kRW];
  bool row_ok[kRW];
#pragma unroll
  for (int rb = 0; rb < kRW; ++rb) {
    i_row[rb] = q0 + 32 * rb + col;  // row within the request
    row_ok[rb] = i_row[rb] < q1;
    qpos[rb] = row_ok[rb] ? computed + i_row[rb] : -1;
  }
  const int min_pos = computed + q0;  // smallest position of the wave
  const int h = kvh * kG + hw;

  bf16x8 qf[kRW][8];
#pragma unroll
  for (int rb = 0; rb < kRW; ++rb) {
    const uint16_t* q = a.qkv + (long long)(qs + (row_ok[rb] ? i_row[rb] : q0)) * a.stride + h * kD + hf * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qf[rb][ks] = *reinterpret_cast<const bf16x8*>(q + ks * 16);
      if (!row_ok[rb])
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[rb][ks][i] = (__bf16)0.0f;
    }
  }

  float16_t o[kRW][4];
  float m_run[kRW], l_run[kRW];
#pragma unroll
  for (int rb = 0; rb < kRW; ++rb) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rb][db][i] = 0.f;
    m_run[rb] = -1e30f;
    l_run[rb] = 0.f;
  }

  // ---- staging ----
  // Wave w moves page slot w/2 of each half: its K region (w even) or its V^T region
  // (w odd), 4 KiB as four 1 KiB global->LDS loads.  Load q, lane i writes LDS bytes
  // 16i.. of the region's q-th KiB, which hold
  //   K:   chunk 4q + i/16 of token i%16
  //   V^T: row 32q + i/2,  swizzle slot i%2   -> chunk (i%2) ^ bit3(row)
  // Page ids are scalar loads issued one half before their loads (one 64-byte
  // scalar-cache line holds the ids of 8 halves).  Ids kept in VGPRs instead would be
  // global loads, and the compiler would then wait for every outstanding global->LDS
  // load before touching those registers.
  const int st_ps = (w >> 1) & 1, st_v = w & 1;
  uint32_t st_off[kLoads];  // byte offset inside the 8 KiB run of this lane's chunk, per load
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int qd = j;
    if (st_v) {
      const int d = 32 * qd + (lane >> 1);
      st_off[j] = kVOff * 2 + d * 32 + (((lane & 1) ^ ((d >> 3) & 1)) << 4);
    } else {
      // global [16 tokens][128 dims]: token t's chunk c at t*256 + c*16
      st_off[j] = (lane & 15) * 256 + (4 * qd + (lane >> 4)) * 16;
    }
  }
  // Valid tokens (0..16) of the two page slots of the half in each ring buffer, 5 bits
  // per (buffer, slot); 0 also marks a page id outside the pool.
  unsigned long long pvbits = 0;
  auto pv = [&](int R, int ps) { return (int)((pvbits >> ((R * 2 + ps) * 5)) & 31); };

  const uint32_t pool_pages32 = (uint32_t)min(a.pool_pages, (int64_t)0x7fffffff);
  struct Ids { int id[2]; };
  auto load_ids = [&](int hx) {
    Ids x;
    x.id[0] = btr_c[2 * hx];
    x.id[1] = btr_c[min(2 * hx + 1, n_pages - 1)];
    return x;
  };
  // Where this wave's loads of half `hx` (page ids `ids`) come from and go to; records
  // the half's valid counts.
  struct Dma { const uint16_t* run; uint32_t dst; };
  auto stage_prep = [&](int hx, const Ids& ids) {
    const int R = hx % kRing;
    const int* id2 = ids.id;
    Dma dm;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int pidx = 2 * hx + ps;
      const int id = id2[ps];
      const int valid = min(max(nkeys - pidx * kPage, 0), kPage);
      // one unsigned compare: negative ids wrap above any pool size
      const bool ok = valid > 0 && (uint32_t)id < pool_pages32;
      const int sh = (R * 2 + ps) * 5;
      pvbits = (pvbits & ~(31ull << sh)) | ((unsigned long long)(ok ? valid : 0) << sh);
      // Every wave issues exactly kLoads loads per half (a bad page reads page 0, zeroed
      // later), so the vmcnt counts in half_step hold.
      if (ps == st_ps) {
        dm.run = a.pool + run_offset(ok ? id : 0, kvh);
        dm.dst = lds_base + R * kHalfBytes + st_ps * kRunBytes + st_v * (kVOff * 2);
      }
    }
    return dm;
  };
  auto stage_issue = [&](int hx, const Ids& ids) {
    const Dma dm = stage_prep(hx, ids);
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      dma16(dm.run, st_off[j], dm.dst + j * 1024);
  };
  // Zero what must not count in ring buffer R: V^T tokens past a page's valid count, and
  // all of K for a page that is missing or outside the pool.  Runs after the barrier
  // that publishes the buffer's loads; ends with a barrier of its own.
  auto stage_fix = [&](int hx) {
    const int R = hx % kRing;
    if (pv(R, 0) == kPage && pv(R, 1) == kPage) return;  // uniform
    char* base = ring(hx);
    if (tid < 256) {  // threads 0..255 cover both page slots
      const int ps = tid >> 7, d = tid & 127;
      const int valid = pv(R, ps);
      uint4* p0 = reinterpret_cast<uint4*>(base + lds_v(ps, d, 0));
      uint4* p1 = reinterpret_cast<uint4*>(base + lds_v(ps, d, 1));
      const uint4 v0 = *p0, v1 = *p1;  // both reads before any write
      *p0 = keep_tokens8(v0, 0, valid);
      *p1 = keep_tokens8(v1, 8, valid);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int c = tid * 2 + k, kps = c >> 8;  // 256 K chunks per page
        if (pv(R, kps) == 0) *reinterpret_cast<uint4*>(base + kps * kRunBytes + (c & 255) * 16) = make_uint4(0, 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    barrier();
  };

  // K fragment of S^T MFMA step ks: MFMA row `col` = key perm(col) of the half:
  // page slot col/16, token bit3(col)*4 | bit2(col)*8 | col%4.
  const int kf_tok = (col & 3) | (((col >> 2) & 1) << 3) | (((col >> 3) & 1) << 2);
  auto kfrag = [&](const char* base, int ks) {
    return *reinterpret_cast<const bf16x8*>(base + lds_k(col >> 4, kf_tok, ks * 2 + hf));
  };
  struct STile { float16_t s[kRW]; };
  auto s_tile = [&](const char* base) {
    STile st;
#pragma unroll
    for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) st.s[rb][i] = 0.f;
    // K fragments read one step ahead of their MFMAs (two in registers)
    bf16x8 kf[2];
    kf[0] = kfrag(base, 0);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks + 1 < 8) kf[(ks + 1) & 1] = kfrag(base, ks + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rb = 0; rb < kRW; ++rb)
        st.s[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks & 1], qf[rb][ks], st.s[rb], 0, 0, 0);
    }
    return st;
  };

  STile s_cur;
  Ids ids_next;  // page ids of the next half to issue
  // One pipeline step: half t lives in ring buffer t % kRing.  kNext: a half follows.
  auto half_step = [&](int t, auto next_tag) {
    constexpr bool kNext = decltype(next_tag)::value;
    // B(t): half t+1's loads have landed in every wave, and every wave has finished
    // reading buffer R3 (half t-1).
    if (t + kAhead - 1 < n_half) wait_vm<(kAhead - 2) * kLoads>(); else wait_vm<0>();
    barrier();
    if (t + kAhead < n_half) {
      stage_issue(t + kAhead, ids_next);
      if (t + kAhead + 1 < n_half) ids_next = load_ids(t + kAhead + 1);
    }
    if (kNext) stage_fix(t + 1);

    // online softmax of half t over this lane's query row: mask (diagonal halves only),
    // row max, lazy rescale.  Element v of S^T: MFMA row (v/4)*8 + hf*4 + v%4, i.e. key
    // (v/8)*16 + hf*8 + ((v/4)%2)*4 + v%4 of the half.
    const int key0 = t * kHalfKeys;
    if (key0 + kHalfKeys - 1 > min_pos) {  // the causal diagonal (or n_keys) crosses these keys
#pragma unroll
      for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + (v >> 3) * 16 + hf * 8 + ((v >> 2) & 1) * 4 + (v & 3);
          if (key > qpos[rb]) s_cur.s[rb][v] = -INFINITY;
        }
    }
    bool grow[kRW], any_grow = false;
    float m_new[kRW];
#pragma unroll
    for (int rb = 0; rb < kRW; ++rb) {
      const float16_t& sc = s_cur.s[rb];
      const float m0 = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
      const float m1 = fmaxf(fmaxf(sc[3], sc[4]), sc[5]);
      const float m2 = fmaxf(fmaxf(sc[6], sc[7]), sc[8]);
      const float m3 = fmaxf(fmaxf(sc[9], sc[10]), sc[11]);
      const float m4 = fmaxf(fmaxf(sc[12], sc[13]), sc[14]);
      float mx = fmaxf(fmaxf(fmaxf(m0, m1), m2), fmaxf(fmaxf(m3, m4), sc[15]));
      mx = max_xor32(mx);
      // Lazy rescale: the reference max only moves when the row max grows by more than
      // 2^kRescale, so P = exp2(s*scale - m) stays <= 2^kRescale and O, l are rescaled
      // on few halves instead of every one.
      m_new[rb] = fmaxf(m_run[rb], mx * a.scale_log2);
      grow[rb] = m_new[rb] > m_run[rb] + kRescale;
      any_grow |= grow[rb];
    }
    if (__builtin_amdgcn_ballot_w64(any_grow)) {  // wave-uniform: skipped on most halves
#pragma unroll
      for (int rb = 0; rb < kRW; ++rb) {
        const float corr = grow[rb] ? __builtin_amdgcn_exp2f(m_run[rb] - m_new[rb]) : 1.0f;
        l_run[rb] *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[rb][db] *= corr;
        m_run[rb] = grow[rb] ? m_new[rb] : m_run[rb];
      }
    }

    // P^T = exp2(S^T*scale - m) as bf16, and l += row sums of the same bf16 P
    const char* base = ring(t);
    bf16x8 pt[kRW][2];
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    auto row_sums = [&]() {
#pragma unroll
      for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bf16x2_t pr = {pt[rb][kc][2 * e], pt[rb][kc][2 * e + 1]};
            l_run[rb] = __builtin_amdgcn_fdot2_f32_bf16(pr, one, l_run[rb], false);
          }
    };
    auto exp_group = [&](int rb, int v0) {
#pragma unroll
      for (int v = v0; v < v0 + 4; ++v) {
        // raw v_exp_f32: results below 2^-126 flush to 0, which a softmax weight can be
        const float p = __builtin_amdgcn_exp2f(fmaf(s_cur.s[rb][v], a.scale_log2, -m_run[rb]));
        pt[rb][v >> 3][v & 7] = (__bf16)p;
      }
    };
    if constexpr (kRW == 1) {
      // phase 1: the exps of half t interleaved with the S^T MFMAs of half t+1 and the V^T
      // fragment reads of half t; phase 2: half t's PV MFMAs back to back
      bf16x8 vf[2][4];
      STile s_nxt;
      if constexpr (kNext) {
        // per ks of half t+1: its S^T MFMA, and on odd ks 4 exps of half t; V^T fragment
        // reads of half t spread over the first 4 steps
        const char* nb = ring(t + 1);
#pragma unroll
        for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s_nxt.s[rb][i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const bf16x8 kf = kfrag(nb, ks);
#pragma unroll
          for (int rb = 0; rb < kRW; ++rb)
            s_nxt.s[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[rb][ks], s_nxt.s[rb], 0, 0, 0);
          if (ks & 1) exp_group(0, 4 * (ks >> 1));
          if (ks < 4) {
            const int g = ks;
#pragma unroll
            for (int db = (g & 1) * 2; db < (g & 1) * 2 + 2; ++db)
              vf[g >> 1][db] = *reinterpret_cast<const bf16x8*>(base + lds_v(g >> 1, db * 32 + col, hf));
          }
        }
        row_sums();
      } else {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int db = 0; db < 4; ++db)
            vf[kc][db] = *reinterpret_cast<const bf16x8*>(base + lds_v(kc, db * 32 + col, hf));
#pragma unroll
        for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
          for (int v0 = 0; v0 < 16; v0 += 4) exp_group(rb, v0);
        row_sums();
      }
      // phase 2: O^T += V^T P^T over the two pages (16 keys each) of half t
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int rb = 0; rb < kRW; ++rb)
            o[rb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[kc][db], pt[rb][kc], o[rb][db], 0, 0, 0);
      if constexpr (kNext) s_cur = s_nxt;
    } else {
      // Two row blocks: no room for half t+1's S^T beside half t's (256 registers), so the
      // phases run in turn: the exps of half t, its PV MFMAs, then half t+1's S^T MFMAs;
      // the other wave on the SIMD overlaps them.
#pragma unroll
      for (int rb = 0; rb < kRW; ++rb)
#pragma unroll
        for (int v0 = 0; v0 < 16; v0 += 4) exp_group(rb, v0);
      row_sums();
      // V^T fragments read one step ahead of their MFMAs (two in registers)
      bf16x8 vfr[2];
      vfr[0] = *reinterpret_cast<const bf16x8*>(base + lds_v(0, col, hf));
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int kc = g >> 2, db = g & 3;
        if (g + 1 < 8)
          vfr[(g + 1) & 1] = *reinterpret_cast<const bf16x8*>(
              base + lds_v((g + 1) >> 2, ((g + 1) & 3) * 32 + col, hf));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rb = 0; rb < kRW; ++rb)
          o[rb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[g & 1], pt[rb][kc], o[rb][db], 0, 0, 0);
      }
      if constexpr (kNext) s_cur = s_tile(ring(t + 1));
    }
  };

  // prologue: halves 0..2 in flight, half 0 published and fixed, S^T of half 0
  ids_next = load_ids(0);
  stage_issue(0, ids_next);
  for (int hx = 1; hx < kAhead; ++hx)
    if (hx < n_half) stage_issue(hx, load_ids(hx));
  if (n_half > kAhead) ids_next = load_ids(kAhead);
  if (n_half >= kAhead) wait_vm<(kAhead - 1) * kLoads>(); else wait_vm<0>();
  barrier();
  stage_fix(0);
  s_cur = s_tile(ring(0));

  for (int t = 0; t + 1 < n_half; ++t) half_step(t, std::true_type{});
  half_step(n_half - 1, std::false_type{});

#pragma unroll
  for (int rb = 0; rb < kRW; ++rb) {
    if (!row_ok[rb]) continue;
    const auto lr = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run[rb]),
                                                     __float_as_uint(l_run[rb]), false, false);
    const float l = __uint_as_float(lr[0]) + __uint_as_float(lr[1]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* dst = a.out + (long long)(qs + i_row[rb]) * (kHq * kD) + h * kD + hf * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 pk = make_uint2(pack_bf16x2(o[rb][db][i * 4] * inv, o[rb][db][i * 4 + 1] * inv),
                                    pack_bf16x2(o[rb][db][i * 4 + 2] * inv, o[rb][db][i * 4 + 3] * inv));
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
  if (pre_tile_q != kQT && pre_tile_q != 2 * kQT) return FQA_EUNSUPPORTED;
  if (pre_item_cap < 0 || max_blocks < 1 || pool_pages < 1 || !meta) return FQA_EINVAL;
  if (pre_item_cap == 0) return FQA_OK;
  if (!qkv || !pool || !block_tables || !cu_seqlens || !positions || !pre_items || !out)
    return FQA_EINVAL;
  PreArgs a{qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions, pre_items,
            meta, out, dims->qkv_stride, dims->scale * kLog2e};
  if (pre_tile_q == kQT)
    hipLaunchKernelGGL(prefill_kernel<1>, dim3(pre_item_cap * kHkv), dim3(256), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(prefill_kernel<2>, dim3(pre_item_cap * kHkv), dim3(256), 0,
                       (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
