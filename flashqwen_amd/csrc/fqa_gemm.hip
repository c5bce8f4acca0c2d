// fqa_gemm.hip — the layer projections y = x · W^T on bf16 MFMA (gfx950).
//
// Replaces LaunchGemm (engine/src/kernels.cu:9-16: cublasGemmEx, bf16 in, fp32 compute,
// bf16 or fp32 out), which the step calls for QKV, o_proj, gate-up, down and lm_head
// (engine/src/model_runtime.cu:261, 280, 285, 288, 322).  x is [M, K] and W is [N, K],
// both K-contiguous (the reference's weight layout), y is [M, N].
//
// MI355X design:
//  * One workgroup per output tile, chosen by row count (gemm_plan): 32, 64 or 128 rows by
//    128 columns on 4 waves for decode-sized M, 256 x 128 on 8 waves up to 1024 rows,
//    256 x 256 on 8 waves above.  A wave owns a block of v_mfma_f32_32x32x16_bf16 tiles
//    (4 x 2 of them in the large tiles: 128 fp32 accumulators per lane).
//  * Both operand tiles of a k step (64 or 32 wide) move global -> LDS by DMA
//    (global_load_lds_dwordx4, 1 KiB per wave instruction) into a ring of 2 to 8 steps,
//    as deep as 160 KiB of LDS allows, every slot in flight.  The step's one barrier sits
//    before its last MFMAs, so the freed slot is refilled and the next step's first
//    fragments are read while those MFMAs run.  A DMA lane's 16 bytes land at LDS byte
//    16 * lane, so the bank swizzle (Tile::swz) is applied on the global side of the DMA.
//  * Shapes with few tiles (decode steps) split K over `splits` workgroups per tile so
//    that one round of workgroups fills the 256 CUs; each writes fp32 partials and a
//    second kernel sums them into y (or a fused consumer reads them: fqa_qkv_proj_append).
//  * Workgroups are dealt to the 8 XCDs round robin; tile_of() renumbers them so that the
//    workgroups on one XCD walk 8 m tiles per n tile and share W and x tiles in its L2.

#include "fqa_append_math.h"
#include "fqa_common.h"
#include "fqa_gemm_internal.h"

namespace fqa {
namespace {

constexpr int kGK = 64;  // K granularity of the shapes accepted (k steps are 32 or 64)

// Tile shapes.  kWM x kWN waves; a wave owns kTM x kTN blocks of 32 x 32 outputs; K
// advances kBK (32 or 64) per step, through a ring of kRing steps in LDS (kRing - 1 in
// flight ahead of the MFMAs).  An LDS row of a step holds kBK bf16 (kPitch bytes) in
// 16-byte chunks, chunk c of row r at c ^ swz(r): (r >> 1) & 7 for 8 chunks, (r >> 2) & 3
// for 4.  A ds_read_b128 is served 16 lanes at a time from the 64 banks (256 bytes); the
// 16 lanes of a fragment read take one chunk of 16 consecutive rows, and with this swizzle
// those land on 16 distinct 16-byte bank groups.
template <int kWM_, int kWN_, int kTM_, int kTN_, int kRing_, int kBK_ = 64>
struct Tile {
  static constexpr int kWM = kWM_, kWN = kWN_, kTM = kTM_, kTN = kTN_, kRing = kRing_;
  static constexpr int kBK = kBK_, kPitch = kBK * 2, kChunks = kBK / 8, kKK = kBK / 16;
  static constexpr int kRowsPerDma = 1024 / kPitch;
  static constexpr int kBM = kWM * kTM * 32, kBN = kWN * kTN * 32;
  static constexpr int kABytes = kBM * kPitch, kBBytes = kBN * kPitch;
  static constexpr int kStage = kABytes + kBBytes;
  static constexpr int kWaves = kWM * kWN, kThreads = 64 * kWaves;
  // DMA instructions per wave per step
  static constexpr int kDmaA = kBM / kRowsPerDma / kWaves, kDmaB = kBN / kRowsPerDma / kWaves;
  static_assert(kBK == 32 || kBK == 64, "k step");
  static_assert(kWaves == 4 || kWaves == 8, "4 or 8 waves");
  static_assert(kDmaA * kRowsPerDma * kWaves == kBM && kDmaB * kRowsPerDma * kWaves == kBN,
                "DMA split");
  static_assert(kRing * kStage <= 160 * 1024, "LDS");
  static_assert((kRing - 1) * (kDmaA + kDmaB) < 64, "vmcnt");
  __device__ static int swz(int r) { return kChunks == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); }
};
using TileL = Tile<2, 4, 4, 2, 2, 64>;  // 256 x 256 on 8 waves: prefill-sized M
using TileL8 = Tile<4, 2, 2, 2, 3>;     // 256 x 128 on 8 waves: 129..1024 rows
using TileM = Tile<2, 2, 2, 2, 5>;      // 128 x 128
using TileS = Tile<1, 4, 2, 1, 6>;      // 64 x 128
using TileT = Tile<1, 4, 1, 1, 8>;      // 32 x 128: a few decode rows

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w;
  void* y;
  float* part;  // [splits][M][N] fp32 when splits > 1
  long long ldx, ldw, ldy;
  int M, N, K;
  int splits;
  int m_tiles, n_tiles;
  float* amax_v;  // argmax mode: per (row, n tile) the tile's largest value and its column
  int* amax_i;
  GemmAppend app;  // append mode: y is the qkv buffer (row stride ldy)
};

__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "{m0}"(lds)
      : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// Wait until at most n * kPer of this wave's loads are outstanding, n in [0, kMax].
template <int kPer, int kMax>
__device__ __forceinline__ void wait_steps(int n) {
  if constexpr (kMax <= 0) {
    wait_vm<0>();
  } else {
    if (n >= kMax)
      wait_vm<kMax * kPer>();
    else
      wait_steps<kPer, kMax - 1>(n);
  }
}
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup -> (m tile, n tile, split).  Workgroups are dealt to the 8 XCDs round robin,
// so the linear id is first turned into an index that runs contiguously within an XCD;
// that index walks the tiles in groups of 8 m tiles per n tile (consecutive workgroups on
// an XCD share a W tile, and 4 consecutive n tiles share the group's x tiles in L2).
__device__ __forceinline__ void tile_of(const GemmArgs& a, int& tm, int& tn, int& sp) {
  const int G = a.m_tiles * a.n_tiles * a.splits;
  const int L = blockIdx.x;
  int t = L;
  if ((G & 7) == 0) t = (L & 7) * (G >> 3) + (L >> 3);
  const int per = a.m_tiles * a.n_tiles;
  sp = t / per;
  t -= sp * per;
  constexpr int kGroup = 8;
  const int span = kGroup * a.n_tiles;
  const int g = t / span, m0 = g * kGroup;
  const int gs = min(a.m_tiles - m0, kGroup);
  const int r = t - g * span;
  tm = m0 + r % gs;
  tn = r / gs;
}

// Append mode: the bf16 output tile is staged in LDS with this row pitch (16 bytes of
// padding rotate consecutive rows across the banks).
template <class T>
constexpr int kTilePitch = T::kBN * 2 + 16;
// ... followed by the tile rows' positions and slots (int32 each)
template <class T>
constexpr int kAppendLds = T::kBM * kTilePitch<T> + T::kBM * 8;
template <class T, bool kAppend>
constexpr int kGemmLds = kAppend && kAppendLds<T> > T::kRing * T::kStage
                             ? kAppendLds<T>
                             : T::kRing * T::kStage;

template <class T>
__device__ void append_epilogue(const GemmArgs& a, char* lds, const float16_t (&acc)[T::kTM][T::kTN],
                                int row0, int col0, int wm, int wn, int w, int lane);

template <class T, bool kF32Out, bool kPartial, bool kArgmax = false, bool kAppend = false>
__global__ void __launch_bounds__(T::kThreads, 1) gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kGemmLds<T, kAppend>];
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w % T::kWM, wn = w / T::kWM;
  int tm, tn, sp;
  tile_of(a, tm, tn, sp);
  const int row0 = tm * T::kBM, col0 = tn * T::kBN;
  // split sp takes k steps sp, sp + splits, sp + 2 splits, ...: the splits of a tile run
  // side by side and read adjacent pieces of the same W rows
  const int nst = a.K / T::kBK;
  const int n_my = (nst - sp + a.splits - 1) / a.splits;
  const int kstride = a.splits * T::kBK;
  const uint16_t* xk = a.x + (long long)sp * T::kBK;
  const uint16_t* wk = a.w + (long long)sp * T::kBK;

  // DMA sources: wave w's instruction i covers rows kRowsPerDma (w kDmaA + i) + lane /
  // kChunks of the x tile (likewise of the W tile); lane fills LDS chunk lane % kChunks
  // of its row, so it reads global chunk (lane % kChunks) ^ swz(row)
  const int drow = lane / T::kChunks, dlc = lane % T::kChunks;
  uint32_t off_a[T::kDmaA], off_b[T::kDmaB];
#pragma unroll
  for (int i = 0; i < T::kDmaA; ++i) {
    const int tr = T::kRowsPerDma * (w * T::kDmaA + i) + drow;  // row within the tile
    const int r = min(row0 + tr, a.M - 1);
    off_a[i] = (uint32_t)((long long)r * a.ldx * 2) + (dlc ^ T::swz(tr)) * 16;
  }
#pragma unroll
  for (int i = 0; i < T::kDmaB; ++i) {
    const int tr = T::kRowsPerDma * (w * T::kDmaB + i) + drow;
    off_b[i] = (uint32_t)((long long)(col0 + tr) * a.ldw * 2) + (dlc ^ T::swz(tr)) * 16;
  }
  // load q (0 .. kDmaA + kDmaB - 1) of this wave's share of the workgroup's j-th k step
  auto issue_one = [&](int j, int q) {
    const uint32_t dst = lds_base + (j % T::kRing) * T::kStage;
    if (q < T::kDmaA)
      dma16(xk + (long long)j * kstride, off_a[q], dst + (w * T::kDmaA + q) * 1024);
    else
      dma16(wk + (long long)j * kstride, off_b[q - T::kDmaA],
            dst + T::kABytes + (w * T::kDmaB + q - T::kDmaA) * 1024);
  };
  auto issue = [&](int j) {
#pragma unroll
    for (int q = 0; q < T::kDmaA + T::kDmaB; ++q) issue_one(j, q);
  };

  // fragment reads: lane reads row (lane & 31) of a 32-row block, k chunk 2 kk + lane/32,
  // stored at chunk (2 kk + lane/32) ^ swz(lane & 31)
  const int a_off = (wm * T::kTM * 32 + (lane & 31)) * T::kPitch;
  const int b_off = T::kABytes + (wn * T::kTN * 32 + (lane & 31)) * T::kPitch;
  int phk[T::kKK];
#pragma unroll
  for (int kk = 0; kk < T::kKK; ++kk) phk[kk] = ((2 * kk + (lane >> 5)) ^ T::swz(lane & 31)) * 16;

  float16_t acc[T::kTM][T::kTN];
#pragma unroll
  for (int rb = 0; rb < T::kTM; ++rb)
#pragma unroll
    for (int cb = 0; cb < T::kTN; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.f;

  // Pipeline: every ring slot holds a step in flight.  The one barrier per step sits
  // before the step's last MFMAs: by then every wave has read all of the step's
  // fragments, so its slot is refilled (step s + kRing) and the next step's first
  // fragments are read while those MFMAs run.
  bf16x8 af[2][T::kTM], bfg[2][T::kTN];
  auto read_frags = [&](int buf, int s, int kk) {
    const char* sb = lds + (s % T::kRing) * T::kStage;
#pragma unroll
    for (int rb = 0; rb < T::kTM; ++rb)
      af[buf][rb] = *reinterpret_cast<const bf16x8*>(sb + a_off + rb * 32 * T::kPitch + phk[kk]);
#pragma unroll
    for (int cb = 0; cb < T::kTN; ++cb)
      bfg[buf][cb] = *reinterpret_cast<const bf16x8*>(sb + b_off + cb * 32 * T::kPitch + phk[kk]);
  };
  constexpr int kPer = T::kDmaA + T::kDmaB;
#pragma unroll
  for (int j = 0; j < T::kRing; ++j)
    if (j < n_my) issue(j);
  wait_steps<kPer, T::kRing - 1>(min(T::kRing - 1, n_my - 1));
  barrier();  // step 0 landed for every wave
  read_frags(0, 0, 0);
  for (int s = 0; s < n_my; ++s) {
#pragma unroll
    for (int kk = 0; kk < T::kKK; ++kk) {
      if (kk + 1 < T::kKK) {
        read_frags((kk + 1) & 1, s, kk + 1);
      } else if (s + 1 < n_my) {
        // step s + 1 landed (steps up to s + kRing - 1 may still be in flight)
        wait_steps<kPer, T::kRing - 2>(min(T::kRing - 2, n_my - 2 - s));
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of step s done
        barrier();
        read_frags(0, s + 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this sub-step's MFMAs
      // On the last sub-step the freed slot's refill (step s + kRing) is issued one load
      // after each MFMA, so the wave's load issue overlaps its own MFMAs.
      const bool refill = kk + 1 == T::kKK && s + T::kRing < n_my;
      constexpr int kMfma = T::kTM * T::kTN;
#pragma unroll
      for (int q = 0; q < (kMfma > kPer ? kMfma : kPer); ++q) {
        if (q < kMfma) {
          const int rb = q / T::kTN, cb = q % T::kTN;
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfg[kk & 1][cb], af[kk & 1][rb],
                                                                acc[rb][cb], 0, 0, 0);
        }
        if (q < kPer && refill) issue_one(s + T::kRing, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if constexpr (kAppend) {
    append_epilogue<T>(a, lds, acc, row0, col0, wm, wn, w, lane);
    return;
  }
  if constexpr (kArgmax) {
    // per row of the tile: the largest value and its column (ties in the reference's greedy order, greedy_key), over
    // this lane's values, then lane ^ 32 (the other column half of the same row), then
    // the tile's kWN column waves through LDS (free once every wave's reads are done)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    barrier();
    float* sv = reinterpret_cast<float*>(lds);
    int* si = reinterpret_cast<int*>(lds + T::kBM * T::kWN * 4);
#pragma unroll
    for (int rb = 0; rb < T::kTM; ++rb) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      uint32_t bk = 0xffffffffu;
#pragma unroll
      for (int cb = 0; cb < T::kTN; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc[rb][cb][4 * q + e];
            const int n = col0 + (wn * T::kTN + cb) * 32 + 8 * q + 4 * (lane >> 5) + e;
            const uint32_t k = greedy_key(n);
            if (v > bv || (v == bv && k < bk)) {
              bv = v;
              bi = n;
              bk = k;
            }
          }
      const float ov = __shfl_xor(bv, 32, kWave);
      const int oi = __shfl_xor(bi, 32, kWave);
      if (ov > bv || (ov == bv && greedy_key(oi) < greedy_key(bi))) {
        bv = ov;
        bi = oi;
      }
      const int r = (wm * T::kTM + rb) * 32 + (lane & 31);  // row within the tile
      if (lane < 32) {
        sv[r * T::kWN + wn] = bv;
        si[r * T::kWN + wn] = bi;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    barrier();
    for (int r = threadIdx.x; r < T::kBM; r += T::kThreads) {
      const int m = row0 + r;
      if (m >= a.M) continue;
      float bv = sv[r * T::kWN];
      int bi = si[r * T::kWN];
      for (int k = 1; k < T::kWN; ++k)
        if (sv[r * T::kWN + k] > bv ||
            (sv[r * T::kWN + k] == bv && greedy_key(si[r * T::kWN + k]) < greedy_key(bi))) {
          bv = sv[r * T::kWN + k];
          bi = si[r * T::kWN + k];
        }
      // row-major by row, so the reduction reads each row's maxima contiguously (these
      // scattered 4-byte stores are a few hundred per tile of a long kernel)
      a.amax_v[(long long)m * a.n_tiles + tn] = bv;
      a.amax_i[(long long)m * a.n_tiles + tn] = bi;
    }
    return;
  }

  // The MFMAs compute the transposed block (W fragments as the 32-row operand), so
  // accumulator (rb, cb) registers 4q..4q+3 of lane hold row 32 rb + lane % 32 and the 4
  // consecutive columns 32 cb + 8 q + 4 (lane / 32) + 0..3 of the wave's block: one
  // 16-byte (fp32) or 8-byte (bf16) store each, a quarter of the store instructions of
  // a row-per-register layout
#pragma unroll
  for (int rb = 0; rb < T::kTM; ++rb) {
    const int m = row0 + (wm * T::kTM + rb) * 32 + (lane & 31);
    if (m >= a.M) continue;
#pragma unroll
    for (int cb = 0; cb < T::kTN; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = col0 + (wn * T::kTN + cb) * 32 + 8 * q + 4 * (lane >> 5);
        const float4 v = make_float4(acc[rb][cb][4 * q], acc[rb][cb][4 * q + 1],
                                     acc[rb][cb][4 * q + 2], acc[rb][cb][4 * q + 3]);
        if (kPartial)
          *reinterpret_cast<float4*>(a.part + ((long long)sp * a.M + m) * a.N + n) = v;
        else if (kF32Out)
          *reinterpret_cast<float4*>(static_cast<float*>(a.y) + m * a.ldy + n) = v;
        else
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + m * a.ldy + n) =
              make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
      }
  }
}

// The QKV projection's epilogue fused with the per-head norm + RoPE + paged append
// (fqa_qknorm_rope_append on the tile's rows, same results bit for bit): the tile's
// values are rounded to bf16 (what fqa_gemm would write) and staged in LDS, then
//  * q / k tiles: one 16-lane group per (row, head) runs norm_rope_head on the row's
//    head (the append kernel's lane layout and arithmetic), q goes to qkv, k to its page
//    (and to qkv with write_k); rows without a RoPE table row keep the projection's values;
//  * v tiles: a page whose 16 rows are all in the tile is written by its first row as
//    whole V^T rows (a register transpose of the 16 staged rows); other rows store their
//    token's column.
// v is not written to qkv.  Rows at or past meta[FQA_META_ROWS] are not written.
template <class T>
__device__ void append_epilogue(const GemmArgs& a, char* lds, const float16_t (&acc)[T::kTM][T::kTN],
                                int row0, int col0, int wm, int wn, int w, int lane) {
  constexpr int kTP = kTilePitch<T>;
  constexpr int kNH = T::kBN / kD;  // heads in the tile
  const GemmAppend& p = a.app;
  int* s_pos = reinterpret_cast<int*>(lds + T::kBM * kTP);
  int* s_slot = s_pos + T::kBM;
  const int T_rows = min(p.meta[FQA_META_ROWS], a.M);
  // the rows' positions and slots, loaded while the tile goes to LDS (-1: no such row)
  int my_pos = -1, my_slot = -1;
  if (threadIdx.x < T::kBM && row0 + (int)threadIdx.x < T_rows) {
    my_pos = p.positions[row0 + threadIdx.x];
    my_slot = p.slots[row0 + threadIdx.x];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's reads of the ring are done
  barrier();                           // ... and every wave's: the LDS is free
#pragma unroll
  for (int rb = 0; rb < T::kTM; ++rb)
#pragma unroll
    for (int cb = 0; cb < T::kTN; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = (wm * T::kTM + rb) * 32 + (lane & 31);
        const int c = (wn * T::kTN + cb) * 32 + 8 * q + 4 * (lane >> 5);
        *reinterpret_cast<uint2*>(lds + r * kTP + c * 2) =
            make_uint2(pack_bf16x2(acc[rb][cb][4 * q], acc[rb][cb][4 * q + 1]),
                       pack_bf16x2(acc[rb][cb][4 * q + 2], acc[rb][cb][4 * q + 3]));
      }
  if (threadIdx.x < T::kBM) {
    s_pos[threadIdx.x] = my_pos;
    s_slot[threadIdx.x] = my_slot;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  barrier();

  const int head0 = col0 / kD;
  uint16_t* qkv = static_cast<uint16_t*>(a.y);
  if (head0 < kHq + kHkv) {  // q or k heads (a tile never mixes kinds: 4096, 5120 | kBN)
    const int g = lane >> 4, j = lane & 15;
    const bool is_k = head0 >= kHq;
    const float* wv = is_k ? p.wk : p.wq;
    const float4 w1 = *reinterpret_cast<const float4*>(wv + 4 * j);
    const float4 w2 = *reinterpret_cast<const float4*>(wv + 64 + 4 * j);
    const float wa[4] = {w1.x, w1.y, w1.z, w1.w}, wb[4] = {w2.x, w2.y, w2.z, w2.w};
    // (row, head) pairs in batches of kB per lane group: every load of a batch (staged
    // values, positions, then the cos/sin rows) is issued before any is used
    constexpr int kB = 8;
    constexpr int kPerGroup = T::kBM * kNH / (T::kWaves * 4);
    static_assert(kPerGroup % kB == 0, "batches");
    for (int b0 = 0; b0 < kPerGroup; b0 += kB) {
      int rt[kB], pos[kB];
      uint2 lo[kB], hv[kB];
      float4 c4[kB], s4[kB];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int hr = (b0 + b) * T::kWaves * 4 + w * 4 + g;  // (row, head) of this group
        rt[b] = hr / kNH;
        const int hi = hr % kNH;
        pos[b] = s_pos[rt[b]];
        const char* src = lds + rt[b] * kTP + (hi * kD + 4 * j) * 2;
        lo[b] = *reinterpret_cast<const uint2*>(src);
        hv[b] = *reinterpret_cast<const uint2*>(src + 128);
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int pc = pos[b] >= 0 && pos[b] < p.rope_max_pos ? pos[b] : 0;
        c4[b] = *reinterpret_cast<const float4*>(p.cos_tab + (long long)pc * 64 + 4 * j);
        s4[b] = *reinterpret_cast<const float4*>(p.sin_tab + (long long)pc * 64 + 4 * j);
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int hr = (b0 + b) * T::kWaves * 4 + w * 4 + g;
        const int row = row0 + rt[b], head = head0 + hr % kNH;
        const bool pos_ok = pos[b] >= 0 && pos[b] < p.rope_max_pos;  // false: no such row too
        const float cs[4] = {c4[b].x, c4[b].y, c4[b].z, c4[b].w};
        const float sn[4] = {s4[b].x, s4[b].y, s4[b].z, s4[b].w};
        uint2 olo, ohi;
        norm_rope_head(lo[b], hv[b], wa, wb, cs, sn, p.eps, olo, ohi);  // all lanes
        if (row >= T_rows) continue;
        if (!pos_ok) {  // no table row: the projection's values, as unfused
          olo = lo[b];
          ohi = hv[b];
        }
        if (!is_k || p.write_k) {
          uint16_t* d = qkv + (long long)row * a.ldy + head * kD + 4 * j;
          *reinterpret_cast<uint2*>(d) = olo;
          *reinterpret_cast<uint2*>(d + 64) = ohi;
        }
        if (is_k && pos_ok) {
          const int slot = s_slot[rt[b]];
          const long long page = slot / kPage;
          if (slot >= 0 && page < p.pool_pages) {
            uint16_t* kd = p.pool + run_offset(page, head - kHq) + (slot % kPage) * kD + 4 * j;
            *reinterpret_cast<uint2*>(kd) = olo;
            *reinterpret_cast<uint2*>(kd + 64) = ohi;
          }
        }
      }
    }
    return;
  }
  // v heads: one wave per row; lane l holds dims 2l, 2l+1 of each head
  for (int rt = w; rt < T::kBM; rt += T::kWaves) {
    const int row = row0 + rt;
    if (row >= T_rows) break;
    const int pos = s_pos[rt];
    if (pos < 0 || pos >= p.rope_max_pos) continue;  // the append skips such rows
    const int slot = s_slot[rt];
    const long long page = slot / kPage;
    if (slot < 0 || page >= p.pool_pages) continue;
    const int tok = slot % kPage, lt = rt - tok;  // the page's first row, in the tile
    // A page whose rows all lie in the tile (and that the append kernel would write whole:
    // same test) is written by its first row; any other row writes its own column.  Both
    // give the same bytes.
    bool whole = lt >= 0 && lt + kPage <= T::kBM && row0 + lt + kPage <= T_rows;
    if (whole)
      whole = s_slot[lt] == slot - tok && s_slot[lt + kPage - 1] == slot - tok + kPage - 1 &&
              s_pos[lt] >= 0 && s_pos[lt + kPage - 1] < p.rope_max_pos;
    if (whole && tok != 0) continue;
#pragma unroll
    for (int hi = 0; hi < kNH; ++hi) {
      const int kvh = head0 + hi - kHq - kHkv;
      uint16_t* vt = p.pool + run_offset(page, kvh) + kVOff + 2 * lane * kPage;
      if (whole) {
        uint32_t x[kPage];
#pragma unroll
        for (int t = 0; t < kPage; ++t)
          x[t] = *reinterpret_cast<const uint32_t*>(lds + (rt + t) * kTP + (hi * kD + 2 * lane) * 2);
        uint32_t y0[8], y1[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          y0[k] = __builtin_amdgcn_perm(x[2 * k + 1], x[2 * k], 0x05040100u);
          y1[k] = __builtin_amdgcn_perm(x[2 * k + 1], x[2 * k], 0x07060302u);
        }
        uint4* v4 = reinterpret_cast<uint4*>(vt);
        v4[0] = make_uint4(y0[0], y0[1], y0[2], y0[3]);
        v4[1] = make_uint4(y0[4], y0[5], y0[6], y0[7]);
        v4[2] = make_uint4(y1[0], y1[1], y1[2], y1[3]);
        v4[3] = make_uint4(y1[4], y1[5], y1[6], y1[7]);
      } else {
        const uint32_t x = *reinterpret_cast<const uint32_t*>(lds + rt * kTP + (hi * kD + 2 * lane) * 2);
        vt[tok] = (uint16_t)x;
        vt[kPage + tok] = (uint16_t)(x >> 16);
      }
    }
  }
}

// Row m's token: the largest of its per-tile maxima, ties in the reference's greedy order
// (greedy_key).  One wave per row.
__global__ void __launch_bounds__(256) gemm_argmax_reduce_kernel(GemmArgs a, int32_t* out) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (m >= a.M) return;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const float* rv = a.amax_v + (long long)m * a.n_tiles;
  const int* ri = a.amax_i + (long long)m * a.n_tiles;
  // 8 tiles per lane per round, all loads issued before any compare (clamped indices;
  // the repeats of the last tile change nothing)
  for (int t0 = 0; t0 < a.n_tiles; t0 += 8 * kWave) {
    float v[8];
    int i[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = min(t0 + k * kWave + lane, a.n_tiles - 1);
      v[k] = rv[t];
      i[k] = ri[t];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (v[k] > bv || (v[k] == bv && greedy_key(i[k]) < greedy_key(bi))) {
        bv = v[k];
        bi = i[k];
      }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (ov > bv || (ov == bv && greedy_key(oi) < greedy_key(bi))) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) out[m] = bv > kGreedyFloor ? bi : 0;  // nothing above -1e30: 0, as fqa_sample
}

// y = sum over the splits of the fp32 partials, 4 columns per thread.
template <bool kF32Out>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(GemmArgs a) {
  const long long q = (long long)blockIdx.x * 256 + threadIdx.x;  // float4 index
  const int n4 = a.N / 4;
  if (q >= (long long)a.M * n4) return;
  const int m = (int)(q / n4), n = (int)(q % n4) * 4;
  const long long plane = (long long)a.M * a.N;
  float4 s = *reinterpret_cast<const float4*>(a.part + (long long)m * a.N + n);
  for (int k = 1; k < a.splits; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(a.part + k * plane + (long long)m * a.N + n);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  if (kF32Out) {
    *reinterpret_cast<float4*>(static_cast<float*>(a.y) + m * a.ldy + n) = s;
  } else {
    const uint2 p = make_uint2(pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + m * a.ldy + n) = p;
  }
}

// The launch plan of one call: up to 128 rows the tile with the fewest rows that covers
// M (tile 1, 2, 3 = 128, 64, 32 rows by 128 columns); up to 1024 rows 256 x 128 (tile 4);
// above, 256 x 256 (tile 0) when N allows.  When the tiles alone leave CUs idle, K is
// split so that tiles x splits fill the 256 CUs once (the kernels run one workgroup per
// CU).
struct GemmPlan {
  int tile, bm, bn, splits, m_tiles, n_tiles;
};
GemmPlan gemm_plan(int M, int N, int K) {
  GemmPlan p;
  p.tile = M > 1024 && N % 256 == 0 ? 0 : M > 128 ? 4 : M > 64 ? 1 : M > 32 ? 2 : 3;
  // 129..256 rows over few columns (o_proj, down: 32 tiles of 256 x 128, split 8 ways):
  // two 128-row tiles halve the split count and the partial traffic (measured 23.0 ->
  // 21.2 us on o_proj at 256 rows; with 48 or more tiles the 256-row tile wins)
  if (M > 128 && M <= 256 && N / 128 < 40) p.tile = 1;
  p.bm = p.tile == 0 || p.tile == 4 ? 256 : p.tile == 1 ? 128 : p.tile == 2 ? 64 : 32;
  p.bn = p.tile == 0 ? 256 : 128;
  p.m_tiles = (M + p.bm - 1) / p.bm;
  p.n_tiles = N / p.bn;
  const int tiles = p.m_tiles * p.n_tiles;
  const int nst = K / kGK;
  int s = tiles >= 160 ? 1 : 256 / tiles;
  if (s > 16) s = 16;
  if (s > nst) s = nst;
  p.splits = s < 1 ? 1 : s;
  return p;
}

bool gemm_shape_ok(int M, int N, int K) {
  return M >= 0 && N > 0 && K > 0 && N % 128 == 0 && K % kGK == 0;
}

template <class T>
void launch_argmax(const GemmArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((gemm_kernel<T, false, false, true>),
                     dim3((unsigned)(a.m_tiles * a.n_tiles)), dim3(T::kThreads), 0, st, a);
}
template <class T>
void launch_gemm(const GemmArgs& a, bool f32, hipStream_t st) {
  const dim3 grid((unsigned)(a.m_tiles * a.n_tiles * a.splits));
  const dim3 block(T::kThreads);
  if (a.splits > 1)
    hipLaunchKernelGGL((gemm_kernel<T, false, true>), grid, block, 0, st, a);
  else if (f32)
    hipLaunchKernelGGL((gemm_kernel<T, true, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<T, false, false>), grid, block, 0, st, a);
}
}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" int64_t fqa_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K) {
  if (!gemm_shape_ok(M, N, K) || M == 0) return 0;
  const GemmPlan p = gemm_plan(M, N, K);
  return p.splits > 1 ? (int64_t)p.splits * M * N * 4 : 0;
}

namespace fqa {

// Validates a call and fills the kernel arguments and plan; FQA_OK or an FQA_E code.
static int gemm_prepare(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                        int64_t ldy, int32_t M, int32_t N, int32_t K, void* workspace,
                        int64_t workspace_bytes, GemmArgs& a, GemmPlan& p) {
  if (M < 0 || N <= 0 || K <= 0) return FQA_EINVAL;
  if (!gemm_shape_ok(M, N, K)) return FQA_EUNSUPPORTED;
  if (M == 0) return FQA_OK;
  if (!x || !w || !y) return FQA_EINVAL;
  if (ldx < K || ldw < K || ldy < N || ldx % 8 || ldw % 8 || ldy % 4) return FQA_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)y & 15)) return FQA_EINVAL;
  // DMA lane offsets are 32-bit: every row start of x and W must lie within 4 GiB
  if ((int64_t)(M - 1) * ldx * 2 >= (int64_t)1 << 32 || (int64_t)(N - 1) * ldw * 2 >= (int64_t)1 << 32)
    return FQA_EUNSUPPORTED;
  p = gemm_plan(M, N, K);
  if ((int64_t)p.m_tiles * p.n_tiles * p.splits > 0x7fffffff) return FQA_EINVAL;
  a = GemmArgs{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), y, nullptr,
               ldx, ldw, ldy, M, N, K, p.splits, p.m_tiles, p.n_tiles};
  if (p.splits > 1) {
    if (!workspace || workspace_bytes < (int64_t)p.splits * M * N * 4 || ((uintptr_t)workspace & 15))
      return FQA_EINVAL;
    a.part = static_cast<float*>(workspace);
  }
  return FQA_OK;
}

static void gemm_launch_main(const GemmArgs& a, const GemmPlan& p, bool f32, hipStream_t st) {
  switch (p.tile) {
    case 0: launch_gemm<TileL>(a, f32, st); break;
    case 4: launch_gemm<TileL8>(a, f32, st); break;
    case 1: launch_gemm<TileM>(a, f32, st); break;
    case 2: launch_gemm<TileS>(a, f32, st); break;
    default: launch_gemm<TileT>(a, f32, st); break;
  }
}

int gemm_launch_partials(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                         int64_t ldy, int32_t M, int32_t N, int32_t K, void* workspace,
                         int64_t workspace_bytes, hipStream_t st, const GemmAppend* app,
                         bool* appended) {
  GemmArgs a;
  GemmPlan p;
  if (appended) *appended = false;
  const int rc = gemm_prepare(x, ldx, w, ldw, y, ldy, M, N, K, workspace, workspace_bytes, a, p);
  if (rc != FQA_OK || M == 0) return rc;
  if (app && p.splits == 1 && N == kQkvStride && (p.tile == 0 || p.tile == 4)) {
    a.app = *app;
    const dim3 grid((unsigned)(a.m_tiles * a.n_tiles));
    if (p.tile == 0)
      hipLaunchKernelGGL((gemm_kernel<TileL, false, false, false, true>), grid,
                         dim3(TileL::kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemm_kernel<TileL8, false, false, false, true>), grid,
                         dim3(TileL8::kThreads), 0, st, a);
    if (appended) *appended = true;
    return 1;
  }
  gemm_launch_main(a, p, false, st);
  return p.splits;
}

}  // namespace fqa

extern "C" int fqa_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                        int64_t ldy, int32_t M, int32_t N, int32_t K, int32_t y_f32,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  GemmArgs a;
  GemmPlan p;
  const int rc = gemm_prepare(x, ldx, w, ldw, y, ldy, M, N, K, workspace, workspace_bytes, a, p);
  if (rc != FQA_OK || M == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  gemm_launch_main(a, p, y_f32 != 0, st);
  if (p.splits > 1) {
    const long long n4 = (long long)M * (N / 4);
    const unsigned blocks = (unsigned)((n4 + 255) / 256);
    if (y_f32)
      hipLaunchKernelGGL((gemm_reduce_kernel<true>), dim3(blocks), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((gemm_reduce_kernel<false>), dim3(blocks), dim3(256), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}

// The argmax plan: the projection's tiles without a K split (every tile sees whole rows
// of its columns).
static bool argmax_plan(int32_t M, int32_t N, int32_t K, GemmPlan& p) {
  if (!gemm_shape_ok(M, N, K) || M == 0) return false;
  p = gemm_plan(M, N, K);
  p.splits = 1;
  return true;
}

extern "C" int64_t fqa_gemm_argmax_workspace_bytes(int32_t M, int32_t N, int32_t K) {
  GemmPlan p;
  if (!argmax_plan(M, N, K, p)) return 0;
  return (int64_t)p.n_tiles * M * 8;
}

extern "C" int fqa_gemm_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw,
                               int32_t M, int32_t N, int32_t K, int32_t* out, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return FQA_EINVAL;
  if (!gemm_shape_ok(M, N, K)) return FQA_EUNSUPPORTED;
  if (M == 0) return FQA_OK;
  if (!x || !w || !out || !workspace) return FQA_EINVAL;
  if (ldx < K || ldw < K || ldx % 8 || ldw % 8) return FQA_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)workspace & 15)) return FQA_EINVAL;
  if ((int64_t)(M - 1) * ldx * 2 >= (int64_t)1 << 32 || (int64_t)(N - 1) * ldw * 2 >= (int64_t)1 << 32)
    return FQA_EUNSUPPORTED;
  GemmPlan p;
  argmax_plan(M, N, K, p);
  if (workspace_bytes < (int64_t)p.n_tiles * M * 8) return FQA_EINVAL;
  if ((int64_t)p.m_tiles * p.n_tiles > 0x7fffffff) return FQA_EINVAL;
  GemmArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), nullptr, nullptr,
             ldx, ldw, 0, M, N, K, 1, p.m_tiles, p.n_tiles,
             static_cast<float*>(workspace),
             reinterpret_cast<int*>(static_cast<char*>(workspace) + (int64_t)p.n_tiles * M * 4)};
  hipStream_t st = (hipStream_t)stream;
  switch (p.tile) {
    case 0: launch_argmax<TileL>(a, st); break;
    case 4: launch_argmax<TileL8>(a, st); break;
    case 1: launch_argmax<TileM>(a, st); break;
    case 2: launch_argmax<TileS>(a, st); break;
    default: launch_argmax<TileT>(a, st); break;
  }
  hipLaunchKernelGGL(gemm_argmax_reduce_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, a,
                     out);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
