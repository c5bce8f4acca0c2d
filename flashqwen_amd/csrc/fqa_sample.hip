// fqa_sample.hip — token sampling over fp32 logits (gfx950).
//
// Replaces ArgmaxKernel + SampleKernel + LaunchSampleBatch (engine/src/kernels.cu:184-327):
// per row, greedy argmax when inv_temp <= 0, else temperature + top-p nucleus sampling
// with the caller's uniform draw u: weights w = exp((l - max) * inv_temp), the kept set
// is the fewest largest weights whose mass reaches top_p * sum(w), and the token is the
// first index at which the running kept mass reaches u * (kept mass).
//
// MI355X design: one 1024-thread workgroup per row.  Wave w owns a contiguous segment of
// the row and its lanes read consecutive elements (coalesced 256-byte wave loads), so
// index order is (segment, step, lane) and the inverse-CDF pick keeps vocabulary order.
// The reference finds the top-p threshold by 32 bisection passes over the row, each
// recomputing every weight; here it is a 3-level radix select on the weights' float bits
// (bits 30..20, 19..9, 8..0; positive floats order like their bit patterns), with exact
// integer mass histograms in LDS: the exact smallest kept weight after 3 levels, and with
// it each wave's kept mass.  A top-p row is read 3 times in full (max + sum, level 1, level 2): level 2 also
// copies the weights of the boundary bin into LDS, and level 3 runs on that copy.  Only
// when the boundary bin holds more than 16384 weights is the row read a 4th time for level
// 3.  A temperature-only row is read once (its kept mass per wave is the rescaled pass-1
// sum), against 35 reads in the reference; the pick then reads 1/16 of one wave's segment
// twice.

#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kSThreads = 1024;
constexpr int kSWaves = kSThreads / kWave;
constexpr int kBins = 2048;  // histogram bins per radix level (levels use 11, 11, 9 bits)
constexpr int kChunk = 2;    // 256-element steps whose loads a wave issues back to back
// Histogram masses are exact integers: a weight with exponent field E adds its 24-bit
// significand, and a bin's mass is that sum times 2^(max(E, 1) - 150) (every bin holds one
// exponent).  ds_add_u64 runs at several times the rate of ds_add_f32 on gfx950, whose
// float adds were most of a top-p row's time; the sums also no longer depend on the order
// the atomics land in, so the kept set is the same on every run.
__device__ __forceinline__ unsigned long long significand(uint32_t bits) {
  return (bits & 0x7fffffu) | (bits >= 0x800000u ? 0x800000u : 0u);
}
__device__ __forceinline__ float bin_mass(unsigned long long sum, int exp_field) {
  return ldexpf((float)sum, max(exp_field, 1) - 150);
}

struct SampArgs {
  const float* logits;
  int vocab;
  long long stride;
  const float* inv_temp;
  const float* top_p;
  const float* u;
  int* out;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ float wave_scan(float v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float x = __shfl_up(v, o, kWave);
    if (lane >= o) v += x;
  }
  return v;
}

// Descending scan of a mass histogram: the bin at which the mass of bins above it plus
// `above` first reaches `need` (need <= above + the histogram's total).  Returns the bin
// and, in *above_out, the mass above it.  Every thread takes 2 bins, highest first.
__device__ int find_crossing(const float* hist, int nbins, float above, float need,
                             float* sh, int* sres, float* sres_f, float* above_out) {
  const int t = threadIdx.x;
  const int b0 = nbins - 1 - 2 * t, b1 = b0 - 1;
  const float m0 = b0 >= 0 ? hist[b0] : 0.f, m1 = b1 >= 0 ? hist[b1] : 0.f;
  const float local = m0 + m1;
  // exclusive block scan of `local` in thread order (= descending bins)
  const int lane = t & (kWave - 1), w = t >> 6;
  const float incl = wave_scan(local);
  __syncthreads();
  if (lane == kWave - 1) sh[w] = incl;
  if (t == 0) {
    *sres = 0;  // lowest bin unless a crossing is found
    *sres_f = above;
  }
  __syncthreads();
  float before = above;
  for (int i = 0; i < w; ++i) before += sh[i];
  before += incl - local;
  if (before < need && before + local >= need) {
    if (b0 >= 0 && before + m0 >= need) {
      *sres = b0;
      *sres_f = before;
    } else {
      *sres = b1;
      *sres_f = before + m0;
    }
  }
  __syncthreads();
  *above_out = *sres_f;
  return *sres;
}

// Wave w of the row covers [seg0, seg1), a whole number of 256-element steps except at
// the row's end; in a step lane l holds elements s0 + 4l .. s0 + 4l + 3, so vocabulary
// order is (wave, step, lane, element).  With kVec4 (16-byte aligned rows) a lane loads its
// 4 logits as one float4: a wave load moves 1 KiB.
template <bool kVec4>
__device__ __forceinline__ void load4(const float* lg, int i, int end, float (&x)[4]) {
  if (kVec4 && i + 3 < end) {
    const float4 v = *reinterpret_cast<const float4*>(lg + i);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = i + e < end ? lg[i + e] : -INFINITY;
  }
}

template <bool kVec4>
__global__ void __launch_bounds__(kSThreads) sample_kernel(SampArgs a) {
  __shared__ float hist[kBins];
  __shared__ float sh[kSWaves];
  __shared__ float sh2[kSWaves];
  __shared__ int sres;
  __shared__ float sres_f;
  __shared__ int s_pick;

  const int row = blockIdx.x;
  const int N = a.vocab;
  const float* lg = a.logits + (long long)row * a.stride;
  const int t = threadIdx.x, lane = t & (kWave - 1), w = t >> 6;
  constexpr int kStep = 4 * kWave;
  const int seg = ((N + kSWaves * kStep - 1) / (kSWaves * kStep)) * kStep;
  const int seg0 = min(w * seg, N), seg1 = min(seg0 + seg, N);
  const float it = a.inv_temp[row];
  // calls f(index, logit) for this lane's elements, in vocabulary order per lane.  The
  // segment is walked in chunks of kChunk steps whose loads are all issued before any
  // element is used, so a wave keeps kChunk KiB in flight instead of waiting out one
  // load's latency per step.
  auto for_each = [&](auto&& f) {
    for (int c0 = seg0; c0 < seg1; c0 += kChunk * kStep) {
      float x[kChunk][4];
      if (kVec4 && c0 + kChunk * kStep <= seg1) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
          const float4 v = *reinterpret_cast<const float4*>(lg + c0 + u * kStep + 4 * lane);
          x[u][0] = v.x; x[u][1] = v.y; x[u][2] = v.z; x[u][3] = v.w;
        }
      } else {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) load4<kVec4>(lg, c0 + u * kStep + 4 * lane, seg1, x[u]);
      }
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int i = c0 + u * kStep + 4 * lane;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (i + e < seg1) f(i + e, x[u][e]);
      }
    }
  };

  if (it <= 0.f) {  // greedy: largest logit, the reference's tie order (greedy_key)
    float best = -INFINITY;
    int bi = N;
    uint32_t bk = 0xffffffffu;
    for_each([&](int i, float v) {
      const uint32_t k = greedy_key(i);
      if (v > best || (v == best && k < bk)) {
        best = v;
        bi = i;
        bk = k;
      }
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(best, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      const uint32_t ok = __shfl_xor(bk, o, kWave);
      if (ov > best || (ov == best && ok < bk)) {
        best = ov;
        bi = oi;
        bk = ok;
      }
    }
    __shared__ int wbi[kSWaves];
    __shared__ uint32_t wbk[kSWaves];
    if (lane == 0) {
      sh[w] = best;
      wbi[w] = bi;
      wbk[w] = bk;
    }
    __syncthreads();
    if (t == 0) {
      float b = sh[0];
      int i0 = wbi[0];
      uint32_t k0 = wbk[0];
      for (int k = 1; k < kSWaves; ++k)
        if (sh[k] > b || (sh[k] == b && wbk[k] < k0)) {
          b = sh[k];
          i0 = wbi[k];
          k0 = wbk[k];
        }
      a.out[row] = b > kGreedyFloor ? i0 : 0;  // nothing above -1e30 (all -inf/NaN): 0
    }
    return;
  }

  // pass 1: row max and total weight together (online: the running sum is rescaled when
  // the running max grows), merged across lanes and waves the same way
  float lm = -INFINITY, ls = 0.f;
  for_each([&](int, float v) {
    if (v == -INFINITY) return;  // a masked token weighs 0 (and -inf - -inf is NaN)
    if (v > lm) {
      ls = ls * __expf((lm - v) * it) + 1.f;
      lm = v;
    } else {
      ls += __expf((v - lm) * it);
    }
  });
  auto merge = [&](float& m0, float& s0v, float m1, float s1) {
    const float mn = fmaxf(m0, m1);
    if (mn == -INFINITY) return;
    s0v = (m0 == -INFINITY ? 0.f : s0v * __expf((m0 - mn) * it)) +
          (m1 == -INFINITY ? 0.f : s1 * __expf((m1 - mn) * it));
    m0 = mn;
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) merge(lm, ls, __shfl_xor(lm, o, kWave), __shfl_xor(ls, o, kWave));
  if (lane == 0) {
    sh[w] = lm;
    sh2[w] = ls;
  }
  __syncthreads();
  float m = sh[0], Z = sh2[0];
  for (int k = 1; k < kSWaves; ++k) merge(m, Z, sh[k], sh2[k]);
  auto weight = [&](float v) { return __expf((v - m) * it); };

  // skm[w]: the kept mass of wave w's segment
  __shared__ float skm[kSWaves];
  __shared__ unsigned long long hcnt[kBins];         // levels 1 and 2
  __shared__ unsigned long long hcnt3[kSWaves][512];  // level 3, one per wave
  __shared__ unsigned long long s_kmc[kSWaves];
  __shared__ int s_ncand;
  uint32_t thr = 0;  // kept: weights whose bits are >= thr (all, without top-p)
  const float tp = a.top_p[row];
  if (tp < 1.f) {
    // pass 2: level-1 histogram (weight bits 30..20).  Weights below
    // x_min = (1 - top_p) * Z / (2N) are left out: all of them together weigh less than
    // (1 - top_p) * Z / 2, so the top-p boundary lies above them.
    const float need = fmaxf(tp * Z, 1e-37f);  // top_p = 0 still keeps the largest weight
    const float x_min = 0.5f * (1.f - tp) * Z / (float)N;
    for (int b = t; b < kBins; b += kSThreads) hcnt[b] = 0ull;
    __syncthreads();
    for_each([&](int, float v) {
      const uint32_t bits = __float_as_uint(weight(v));
      if (__uint_as_float(bits) >= x_min) atomicAdd(&hcnt[(bits >> 20) & 2047], significand(bits));
    });
    __syncthreads();
    for (int b = t; b < kBins; b += kSThreads) hist[b] = bin_mass(hcnt[b], b >> 3);
    __syncthreads();
    float above;
    const int b1 = find_crossing(hist, kBins, 0.f, need, sh, &sres, &sres_f, &above);
    const int e1 = b1 >> 3;  // the exponent field of every weight in bin b1
    // pass 3: level 2, bits 19..9 of the weights in bin b1.  The same pass sums, per
    // lane, the weights above bin b1 (all kept) and copies the weights in bin b1 into LDS
    // (low 20 bits and the wave, in the level-3 histograms' memory); when they all fit,
    // level 3 and the kept masses come from that copy and the row is not read again.
    uint32_t* cand = reinterpret_cast<uint32_t*>(&hcnt3[0][0]);
    constexpr int kCandCap = kSWaves * 512 * 2;
    for (int b = t; b < kBins; b += kSThreads) hcnt[b] = 0ull;
    if (t == 0) s_ncand = 0;
    __syncthreads();
    float km1 = 0.f;
    for_each([&](int, float v) {
      const float wv = weight(v);
      const uint32_t bits = __float_as_uint(wv);
      const int bb = (int)(bits >> 20);
      if (bb > b1) {
        km1 += wv;
      } else if (bb == b1) {
        atomicAdd(&hcnt[(bits >> 9) & 2047], significand(bits));
        const int slot = atomicAdd(&s_ncand, 1);
        if (slot < kCandCap) cand[slot] = ((uint32_t)w << 20) | (bits & 0xfffffu);
      }
    });
    __syncthreads();
    for (int b = t; b < kBins; b += kSThreads) hist[b] = bin_mass(hcnt[b], e1);
    __syncthreads();
    const int b2 = find_crossing(hist, kBins, above, need, sh, &sres, &sres_f, &above);
    const uint32_t hi = ((uint32_t)b1 << 11) | (uint32_t)b2;
    const int nc = s_ncand;
    if (nc <= kCandCap) {
      // level 3 over the copied weights of (b1, b2), then each wave's kept mass: the
      // weights above bin b1 plus its copied weights at or above the threshold
      for (int b = t; b < 512; b += kSThreads) hcnt[b] = 0ull;
      if (t < kSWaves) s_kmc[t] = 0ull;
      __syncthreads();
      for (int i = t; i < nc; i += kSThreads) {
        const uint32_t bits = ((uint32_t)b1 << 20) | (cand[i] & 0xfffffu);
        if ((bits >> 9) == hi) atomicAdd(&hcnt[bits & 511], significand(bits));
      }
      __syncthreads();
      if (t < 512) hist[t] = bin_mass(hcnt[t], e1);
      __syncthreads();
      const int b3 = find_crossing(hist, 512, above, need, sh, &sres, &sres_f, &above);
      thr = (hi << 9) | (uint32_t)b3;
      for (int i = t; i < nc; i += kSThreads) {
        const uint32_t bits = ((uint32_t)b1 << 20) | (cand[i] & 0xfffffu);
        if (bits >= thr) atomicAdd(&s_kmc[cand[i] >> 20], significand(bits));
      }
      __syncthreads();
      const float km = wave_sum(km1);
      if (lane == 0) skm[w] = km + bin_mass(s_kmc[w], e1);
    } else {
      // pass 4: level 3 (bits 8..0 of the weights in (b1, b2)) as one histogram per
      // wave, and per wave the mass of the weights above (b1, b2), which are all kept:
      // the kept mass per wave then follows from the histograms without another pass
      unsigned long long* h3 = &hcnt3[0][0];
      for (int b = t; b < kSWaves * 512; b += kSThreads) h3[b] = 0ull;
      __syncthreads();
      float km_hi = 0.f;
      for_each([&](int, float v) {
        const float wv = weight(v);
        const uint32_t bits = __float_as_uint(wv);
        if ((bits >> 9) > hi) km_hi += wv;
        else if ((bits >> 9) == hi) atomicAdd(&hcnt3[w][bits & 511], significand(bits));
      });
      __syncthreads();
      if (t < 512) {
        unsigned long long c = 0;
        for (int k = 0; k < kSWaves; ++k) c += hcnt3[k][t];
        hist[t] = bin_mass(c, e1);
      }
      __syncthreads();
      const int b3 = find_crossing(hist, 512, above, need, sh, &sres, &sres_f, &above);
      thr = (hi << 9) | (uint32_t)b3;
      unsigned long long c = 0;
      for (int b = b3 + lane; b < 512; b += kWave) c += hcnt3[w][b];
      float km = km_hi + bin_mass(c, e1);
      km = wave_sum(km);
      if (lane == 0) skm[w] = km;
    }
  } else {
    // every weight is kept: wave w's mass is its pass-1 sum rescaled to the row max
    if (t < kSWaves) skm[t] = sh[t] == -INFINITY ? 0.f : sh2[t] * __expf((sh[t] - m) * it);
  }
  __syncthreads();

  // the pick: the wave whose kept mass [before, before + km) holds the draw u * total;
  // its segment is split into kSWaves sub-segments whose kept masses all waves sum at
  // once, and the wave owning the sub-segment that holds the draw walks it step by step
  // to the first kept token whose running mass reaches the draw
  auto kept = [&](float v) {
    const float wv = weight(v);
    return __float_as_uint(wv) >= thr ? wv : 0.f;
  };
  float total = 0.f;
  for (int k = 0; k < kSWaves; ++k) total += skm[k];
  const float target = a.u[row] * total;
  int ws = -1;
  float before = 0.f;
  {
    float acc = 0.f;
    for (int k = 0; k < kSWaves; ++k) {
      if (ws < 0 && acc <= target && target < acc + skm[k]) {
        ws = k;
        before = acc;
      }
      acc += skm[k];
    }
  }
  if (ws < 0) {  // a draw past the summed mass (rounding): the last token
    if (t == 0) a.out[row] = N - 1;
    return;
  }
  const int S0 = min(ws * seg, N), S1 = min(S0 + seg, N);
  const int sub = ((S1 - S0 + kSWaves * kStep - 1) / (kSWaves * kStep)) * kStep;
  const int u0 = min(S0 + w * sub, S1), u1 = min(u0 + sub, S1);
  float m2 = 0.f;
  for (int s0 = u0; s0 < u1; s0 += kStep) {
    const int i = s0 + 4 * lane;
    float x[4];
    load4<kVec4>(lg, i, u1, x);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i + e < u1) m2 += kept(x[e]);
  }
  m2 = wave_sum(m2);
  if (lane == 0) sh2[w] = m2;
  if (t == 0) s_pick = N - 1;
  __syncthreads();
  // the walker: the last sub-segment with kept mass that starts at or below the draw
  // (the first one with kept mass if rounding puts the draw below them all)
  int wk = -1, first = -1;
  float b2v = before, wb = before;
  for (int k = 0; k < kSWaves; ++k) {
    if (sh2[k] > 0.f) {
      if (first < 0) first = k;
      if (b2v <= target) {
        wk = k;
        wb = b2v;
      }
    }
    b2v += sh2[k];
  }
  if (wk < 0) {
    wk = first;
    wb = before;
  }
  if (w == wk) {
    float acc = wb;
    int last = -1;  // the last kept token walked so far
    for (int s0 = u0; s0 < u1; s0 += kStep) {
      const int i = s0 + 4 * lane;
      float x[4], kw[4];
      load4<kVec4>(lg, i, u1, x);
      float lsum = 0.f;
      int llast = -1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kw[e] = i + e < u1 ? kept(x[e]) : 0.f;
        lsum += kw[e];
        if (kw[e] > 0.f) llast = i + e;
      }
      const float incl = wave_scan(lsum);
      const float step = __shfl(incl, kWave - 1, kWave);
      // the first lane whose running mass reaches the draw, then its first such element
      const unsigned long long hit = __ballot(lsum > 0.f && acc + incl >= target);
      if (hit) {
        const int l = (int)__builtin_ctzll(hit);
        if (lane == l) {
          float run = acc + incl - lsum;
          // the first element whose running sum reaches the draw; if rounding leaves the
          // lane's own running sum short, its last kept element
          int pick = -1;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            run += kw[e];
            if (pick < 0 && kw[e] > 0.f && run >= target) pick = i + e;
          }
          s_pick = pick >= 0 ? pick : llast;
        }
        last = -2;
        break;
      }
      const unsigned long long has = __ballot(llast >= 0);
      if (has) last = __shfl(llast, 63 - __builtin_clzll(has), kWave);
      acc += step;
    }
    if (last >= 0 && lane == 0) s_pick = last;  // the draw lies past this sub-segment's sum
  }
  __syncthreads();
  if (t == 0) a.out[row] = s_pick;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" int fqa_sample(const float* logits, int32_t n_rows, int32_t vocab,
                          int64_t row_stride, const float* inv_temp, const float* top_p,
                          const float* u, int32_t* out, void* stream) {
  if (n_rows < 0 || vocab < 1 || vocab > (1 << 24) || row_stride < vocab) return FQA_EINVAL;
  if (n_rows == 0) return FQA_OK;
  if (!logits || !inv_temp || !top_p || !u || !out) return FQA_EINVAL;
  SampArgs a{logits, vocab, row_stride, inv_temp, top_p, u, out};
  const bool vec4 = ((uintptr_t)logits & 15) == 0 && (row_stride & 3) == 0;
  if (vec4)
    hipLaunchKernelGGL(sample_kernel<true>, dim3((unsigned)n_rows), dim3(kSThreads), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3((unsigned)n_rows), dim3(kSThreads), 0,
                       (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
