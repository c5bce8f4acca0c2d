// fqa_compat.hpp — the reference engine's own attention-path signatures, implemented over
// the C ABI of fqa.h.  Header-only; link with libfqa.so and amdhip64.
//
// A maintainer swaps the engine's declarations for these and leaves the call sites of
// ModelRuntime::RunLayersBody (engine/src/model_runtime.cu:263-278) and
// StepContext::PrepareInputs (:295-302) as they are:
//
//   fq::StepContext(max_rows, slots, max_ctx), PrepareInputs(in, rng, s)   model_runtime.h:119-136
//   fq::RopeTables::Build(spec, max_ctx), Cos(), Sin()                     model_runtime.h:21-29
//   fq::LaunchHeadNormRope(buf, wq, wk, cos, sin, pos, M, n_q, n_kv,
//                          head_dim, stride, eps, s)                        kernels.cuh:28-31
//   fq::KvStore(spec, max_ctx, gpu_mem_fraction), StoreKV(layer, qkv, bt,
//               bt_stride, bt_row, pos, M, s), KV(l), NumBlocks()           kv_store.h:24-39
//   fq::LaunchAttnDecodeCute(q, q_stride, cache_kv, out, n_heads, n_kv,
//                            head_dim, pos, qstart, decode_rids, n_decode,
//                            bt, max_blocks, block_size, scale, pm, pl, pa, s)   attn_cute.h:14-20
//   fq::LaunchAttnPrefillCute(q, q_stride, cache_kv, out, n_heads, n_kv,
//                             head_dim, pos, qstart, qlen, rids, R, max_qlen,
//                             bt, max_blocks, block_size, scale, s)              attn_cute.h:7-12
//
// How the pieces meet.  The reference launchers take the host-packed arrays of the step
// (pos, req, qstart, qlen, decode/prefill rids, bt).  Here StepContext::PrepareInputs
// produces the same arrays on the GPU with fqa_pack, together with the work plans the
// kernels need (slot mapping, the stream-K decode plan, the prefill items), and registers
// itself as the context of its stream.  Each Launch* call finds the plan through its
// stream and checks that the arrays it was given are that context's.  KvStore registers
// each layer's pool with its page count, which the launchers look up from `cache_kv`
// (the reference signatures do not carry it).
//
// Differences a caller sees:
//  * the pool layout is this library's (fqa.h: K [16][128] + V^T [128][16] per page and kv
//    head), so the pool must be written through StoreKV / the fqa_* appends;
//  * the decode's split partials live in the context's workspace: pm / pl / pa are
//    accepted for the signature and not used;
//  * a rejected call throws std::runtime_error (the reference asserts or exits);
//  * LaunchHeadNormRope leaves rows whose position has no row in the cos/sin tables
//    untouched (a RopeTables' row count is looked up through Cos(); a table built
//    elsewhere is taken to hold the StepContext's max_ctx rows);
//  * the rows of a request must be contiguous in ForwardInput with consecutive positions,
//    which is what Request::EmitChunk produces (scheduler.h:66-72) and what the reference's
//    attention kernels assume (row qstart[r] + i at position pos[qstart[r]] + i).
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "fqa.h"
#include "fqa_step.hpp"

namespace fq {

using bf16 = __hip_bfloat16;

// sampler.h:7-10
struct SampleParams {
  float temp;
  float top_p;
};

// One forward's flattened rows and per-request block tables (model_runtime.h:35-63).
struct ForwardInput {
  std::vector<int> tokens, positions, req_index, logits_rows;
  std::vector<std::vector<int>> block_tables;
  std::vector<SampleParams> sample_params;

  void Clear() {
    tokens.clear();
    positions.clear();
    req_index.clear();
    logits_rows.clear();
    block_tables.clear();
    sample_params.clear();
  }
  int NumRows() const { return static_cast<int>(tokens.size()); }
  int AddRequest(std::vector<int> block_table) {
    block_tables.push_back(std::move(block_table));
    return static_cast<int>(block_tables.size()) - 1;
  }
  void AddRow(int token, int position, int req) {
    tokens.push_back(token);
    positions.push_back(position);
    req_index.push_back(req);
  }
  void SampleLastRow(SampleParams sp) {
    logits_rows.push_back(static_cast<int>(tokens.size()) - 1);
    sample_params.push_back(sp);
  }
};

namespace detail {

inline void Fail(const std::string& what) { throw std::runtime_error("fqa_compat: " + what); }

// Registries: the step context of each stream, and the page count of each pool layer.
template <class Ctx>
struct Registry {
  std::mutex mu;
  std::map<hipStream_t, const Ctx*> by_stream;
  std::map<const void*, int64_t> pool_pages;
  std::map<const void*, int> rope_rows;  // RopeTables: rows of the table at Cos()
};

}  // namespace detail

class StepContext;

namespace detail {
inline Registry<StepContext>& Reg() {
  static Registry<StepContext> r;
  return r;
}
inline const StepContext& ContextOf(hipStream_t s) {
  auto& r = Reg();
  std::lock_guard<std::mutex> lock(r.mu);
  auto it = r.by_stream.find(s);
  if (it == r.by_stream.end()) Fail("no StepContext prepared on this stream");
  return *it->second;
}
inline int64_t PoolPagesOf(const void* layer) {
  auto& r = Reg();
  std::lock_guard<std::mutex> lock(r.mu);
  auto it = r.pool_pages.find(layer);
  if (it == r.pool_pages.end()) Fail("cache_kv is not a layer of a KvStore");
  return it->second;
}
// Rows of the cos table at `cos_tab` if a RopeTables built it; otherwise `fallback` (a
// table built elsewhere is taken to hold max_ctx rows, as the reference assumes).
inline int RopeRowsOf(const float* cos_tab, int fallback) {
  auto& r = Reg();
  std::lock_guard<std::mutex> lock(r.mu);
  auto it = r.rope_rows.find(cos_tab);
  return it == r.rope_rows.end() ? fallback : it->second;
}
inline fqa_dims Dims(int n_heads, int n_kv, int head_dim, int block_size, int stride, float eps,
                     float scale) {
  if (n_heads != 32 || n_kv != 8 || head_dim != 128 || block_size != FQA_PAGE_TOKENS)
    Fail("only the Qwen3-8B attention shape (32/8/128, 16-token blocks) is supported");
  return fqa_dims{n_heads, n_kv, head_dim, block_size, stride, eps, scale};
}
}  // namespace detail

// The per-forward batch context (model_runtime.h:119-136): the reference's members, with
// the device halves written by fqa_pack instead of host loops + H2D copies.
class StepContext {
 public:
  fqa::DeviceBuffer<int> ids, pos, req;
  fqa::DeviceBuffer<int> lrows;
  fqa::DeviceBuffer<int> qstart, qlen;  // qstart holds R + 1 entries (cu_seqlens)
  fqa::DeviceBuffer<int> decode_rids, prefill_rids;
  fqa::DeviceBuffer<int> bt;
  fqa::DeviceBuffer<float> invT, topp, u;

  int max_blocks = 0;
  int bt_stride = 0;
  int n_rows = 0, n_sample = 0;
  int n_decode = 0, n_prefill = 0, prefill_max_qlen = 1;

  StepContext(int max_rows, int slots, int max_ctx, int device = 0)
      : max_rows_(max_rows), slots_(slots), max_ctx_(max_ctx) {
    if (max_rows < 1 || slots < 1 || slots > FQA_MAX_REQS || max_ctx < 1)
      detail::Fail("StepContext sizes");
    max_blocks = (max_ctx + FQA_PAGE_TOKENS - 1) / FQA_PAGE_TOKENS;
    int waves = fqa_dec_default_waves(device);
    if (waves <= 0) waves = 1024;
    dec_cap_ = fqa_dec_wave_bound(slots, waves);
    pre_cap_ = fqa_pre_item_bound(slots, max_rows, FQA_PRE_TILE_Q);
    // the pool's page count is unknown here: pages are range-checked by each kernel
    // against the KvStore layer it reads
    cfg_ = {max_rows, max_blocks, 0x7fffffff, waves, 8, dec_cap_, FQA_PRE_TILE_Q, pre_cap_};
    ids = fqa::DeviceBuffer<int>(max_rows);
    pos = fqa::DeviceBuffer<int>(max_rows);
    req = fqa::DeviceBuffer<int>(max_rows);
    lrows = fqa::DeviceBuffer<int>(slots);
    qstart = fqa::DeviceBuffer<int>(slots + 1);
    qlen = fqa::DeviceBuffer<int>(slots);
    decode_rids = fqa::DeviceBuffer<int>(slots);
    prefill_rids = fqa::DeviceBuffer<int>(slots);
    bt = fqa::DeviceBuffer<int>((size_t)slots * max_blocks);
    invT = fqa::DeviceBuffer<float>(slots);
    topp = fqa::DeviceBuffer<float>(slots);
    u = fqa::DeviceBuffer<float>(slots);
    computed_ = fqa::DeviceBuffer<int32_t>(slots);
    n_new_ = fqa::DeviceBuffer<int32_t>(slots);
    bt_off_ = fqa::DeviceBuffer<int32_t>(slots + 1);
    bt_pages_ = fqa::DeviceBuffer<int32_t>((size_t)slots * max_blocks);
    slot_ = fqa::DeviceBuffer<int32_t>(max_rows);
    dseqs_ = fqa::DeviceBuffer<int32_t>((size_t)slots * 4);
    dwaves_ = fqa::DeviceBuffer<int32_t>((size_t)dec_cap_ * 8);
    items_ = fqa::DeviceBuffer<int32_t>((size_t)pre_cap_ * 4);
    meta_ = fqa::DeviceBuffer<int32_t>(FQA_META_LEN);
    fqa_dims d{32, 8, 128, FQA_PAGE_TOKENS, 6144, 1e-6f, 0.f};
    ws_ = fqa::DeviceBuffer<unsigned char>((size_t)fqa_decode_workspace_bytes(&d, dec_cap_));
  }
  StepContext(const StepContext&) = delete;
  StepContext& operator=(const StepContext&) = delete;
  ~StepContext() {
    auto& r = detail::Reg();
    std::lock_guard<std::mutex> lock(r.mu);
    for (auto it = r.by_stream.begin(); it != r.by_stream.end();)
      it = it->second == this ? r.by_stream.erase(it) : std::next(it);
  }

  // model_runtime.cu:295-302: rows, block tables, the decode/prefill split and the
  // sampling rows.  The split's host counts are computed here as the reference does
  // (SplitDecodePrefill, :66-91), because the launchers take them as host ints; the device
  // arrays come from fqa_pack.
  void PrepareInputs(const ForwardInput& in, std::mt19937& rng, hipStream_t stream) {
    n_rows = in.NumRows();
    const int R = static_cast<int>(in.block_tables.size());
    if (n_rows > max_rows_ || R > slots_) detail::Fail("batch larger than the context");
    if ((int)in.positions.size() != n_rows || (int)in.req_index.size() != n_rows)
      detail::Fail("ForwardInput rows are ragged");
    h_comp_.assign(R, 0);
    h_n_.assign(R, 0);
    for (int t = 0; t < n_rows; ++t) {
      const int r = in.req_index[t];
      if (r < 0 || r >= R) detail::Fail("row of an unknown request");
      if (t > 0 && r < in.req_index[t - 1]) detail::Fail("rows must be grouped by request");
      if (h_n_[r] == 0) h_comp_[r] = in.positions[t];
      else if (in.positions[t] != h_comp_[r] + h_n_[r]) detail::Fail("positions not consecutive");
      ++h_n_[r];
    }
    n_decode = n_prefill = 0;
    prefill_max_qlen = 1;
    for (int r = 0; r < R; ++r) {
      if (h_n_[r] == 1) ++n_decode;
      else {
        ++n_prefill;
        prefill_max_qlen = std::max(prefill_max_qlen, h_n_[r]);
      }
    }
    bt_stride = max_blocks;
    h_off_.assign(R + 1, 0);
    h_pages_.clear();
    for (int r = 0; r < R; ++r) {
      if ((int)in.block_tables[r].size() > max_blocks) detail::Fail("block table beyond max_ctx");
      h_pages_.insert(h_pages_.end(), in.block_tables[r].begin(), in.block_tables[r].end());
      h_off_[r + 1] = (int)h_pages_.size();
    }
    if (R) {
      computed_.Upload(h_comp_.data(), R, stream);
      n_new_.Upload(h_n_.data(), R, stream);
    }
    bt_off_.Upload(h_off_.data(), R + 1, stream);
    if (!h_pages_.empty()) bt_pages_.Upload(h_pages_.data(), h_pages_.size(), stream);
    if (n_rows) ids.Upload(in.tokens.data(), n_rows, stream);
    fqa_batch b{computed_.D(), n_new_.D(), bt_off_.D(), bt_pages_.D(), nullptr, R};
    fqa_pack_out o{qstart.D(), qlen.D(), pos.D(), req.D(), slot_.D(), bt.D(), decode_rids.D(),
                   prefill_rids.D(), dseqs_.D(), dwaves_.D(), items_.D(), meta_.D()};
    fqa::Check(fqa_pack(&b, &cfg_, &o, stream), "fqa_pack");
    FillSampling(in, rng, stream);
    n_reqs_ = R;
    auto& reg = detail::Reg();
    std::lock_guard<std::mutex> lock(reg.mu);
    reg.by_stream[stream] = this;
  }

  // The plan fqa_pack wrote, for the launchers.
  const int32_t* SlotMapping() const { return slot_.D(); }
  const int32_t* DecWaves() const { return dwaves_.D(); }
  const int32_t* DecSeqs() const { return dseqs_.D(); }
  const int32_t* PreItems() const { return items_.D(); }
  const int32_t* Meta() const { return meta_.D(); }
  void* Workspace() const { return ws_.D(); }
  int DecWaveCap() const { return dec_cap_; }
  int PreItemCap() const { return pre_cap_; }
  int MaxCtx() const { return max_ctx_; }
  int Requests() const { return n_reqs_; }

 private:
  // FillSampling (model_runtime.cu:93-108): the same draws from the same generator.
  void FillSampling(const ForwardInput& in, std::mt19937& rng, hipStream_t stream) {
    n_sample = static_cast<int>(in.logits_rows.size());
    if (n_sample > slots_) detail::Fail("more sampling rows than slots");
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    h_invT_.resize(n_sample);
    h_topp_.resize(n_sample);
    h_u_.resize(n_sample);
    for (int i = 0; i < n_sample; ++i) {
      const SampleParams& sp = in.sample_params[i];
      h_invT_[i] = sp.temp > 0.0f ? 1.0f / sp.temp : 0.0f;
      h_topp_[i] = sp.top_p;
      h_u_[i] = dist(rng);
    }
    if (n_sample) {
      lrows.Upload(in.logits_rows.data(), n_sample, stream);
      invT.Upload(h_invT_.data(), n_sample, stream);
      topp.Upload(h_topp_.data(), n_sample, stream);
      u.Upload(h_u_.data(), n_sample, stream);
    }
  }

  int max_rows_, slots_, max_ctx_;
  int dec_cap_ = 0, pre_cap_ = 0, n_reqs_ = 0;
  fqa_pack_cfg cfg_{};
  // host copies the async uploads read (kept until the next PrepareInputs)
  std::vector<int32_t> h_comp_, h_n_, h_off_, h_pages_;
  std::vector<float> h_invT_, h_topp_, h_u_;
  fqa::DeviceBuffer<int32_t> computed_, n_new_, bt_off_, bt_pages_, slot_, dseqs_, dwaves_,
      items_, meta_;
  fqa::DeviceBuffer<unsigned char> ws_;
};

// RopeTables::Build (model_runtime.cu:111-126): float tables [max_ctx][head_dim/2].
class RopeTables {
 public:
  template <class Spec>
  void Build(const Spec& spec, int max_ctx) {
    {
      auto& r = detail::Reg();
      std::lock_guard<std::mutex> lock(r.mu);
      r.rope_rows.erase(cos_.D());  // a rebuild replaces the table
    }
    const int half = spec.head_dim / 2;
    std::vector<float> c((size_t)max_ctx * half), s((size_t)max_ctx * half);
    fqa::Check(fqa_rope_tables(max_ctx, spec.head_dim, spec.rope_theta, c.data(), s.data()),
               "fqa_rope_tables");
    cos_ = fqa::DeviceBuffer<float>(c.size());
    sin_ = fqa::DeviceBuffer<float>(s.size());
    cos_.Upload(c.data(), c.size(), nullptr);
    sin_.Upload(s.data(), s.size(), nullptr);
    fqa::HipCheck(hipDeviceSynchronize(), "rope upload");
    auto& r = detail::Reg();
    std::lock_guard<std::mutex> lock(r.mu);
    r.rope_rows[cos_.D()] = max_ctx;
  }
  RopeTables() = default;
  RopeTables(const RopeTables&) = delete;
  RopeTables& operator=(const RopeTables&) = delete;
  ~RopeTables() {
    auto& r = detail::Reg();
    std::lock_guard<std::mutex> lock(r.mu);
    r.rope_rows.erase(cos_.D());
  }
  const float* Cos() const { return cos_.D(); }
  const float* Sin() const { return sin_.D(); }

 private:
  fqa::DeviceBuffer<float> cos_, sin_;
};

// The paged KV pool (kv_store.h:24-39): one array per layer, sized from the device's free
// memory under gpu_mem_fraction exactly as the reference sizes it (fqa_pool_pages_device).
class KvStore {
 public:
  template <class Spec>
  KvStore(const Spec& spec, int max_ctx, float gpu_mem_fraction) : layers_(spec.num_layers) {
    CheckSpec(spec);
    const fqa_dims d = detail::Dims(spec.num_heads, spec.num_kv_heads, spec.head_dim,
                                    FQA_PAGE_TOKENS, 6144, spec.rms_eps, 0.f);
    int64_t pages = 0;
    const int rc = fqa_pool_pages_device(&d, gpu_mem_fraction, spec.num_layers, max_ctx, &pages);
    if (rc == FQA_ENOSPACE)
      detail::Fail("not enough VRAM for even one full-length sequence at max_ctx=" +
                   std::to_string(max_ctx) + " (" + std::to_string(pages) + " blocks)");
    fqa::Check(rc, "fqa_pool_pages_device");
    Allocate(pages);
  }
  // A pool of an explicit page count (no free-memory query).
  template <class Spec>
  KvStore(const Spec& spec, int64_t num_blocks) : layers_(spec.num_layers) {
    CheckSpec(spec);
    Allocate(num_blocks);
  }
  KvStore(const KvStore&) = delete;
  KvStore& operator=(const KvStore&) = delete;
  ~KvStore() {
    auto& r = detail::Reg();
    std::lock_guard<std::mutex> lock(r.mu);
    for (auto& b : kv_) r.pool_pages.erase(b.D());
  }

  // kv_store.cu:66-75: k (normalised in qkv by LaunchHeadNormRope) and v of every row
  // into the row's slot of layer `layer`.
  void StoreKV(int layer, const bf16* qkv, const int* bt_, int bt_stride, const int* bt_row,
               const int* pos, int M, hipStream_t stream) const {
    if (layer < 0 || layer >= layers_) detail::Fail("StoreKV: layer out of range");
    if (M <= 0) return;
    const StepContext& ctx = detail::ContextOf(stream);
    if (bt_ != ctx.bt.D() || bt_stride != ctx.bt_stride || bt_row != ctx.req.D() ||
        pos != ctx.pos.D() || M != ctx.n_rows)
      detail::Fail("StoreKV: arrays are not the stream's StepContext's");
    const fqa_dims d{32, 8, 128, FQA_PAGE_TOKENS, 6144, 1e-6f, 0.f};
    fqa::Check(fqa_store_kv(&d, reinterpret_cast<const uint16_t*>(qkv), pos, ctx.SlotMapping(),
                            ctx.Meta(), M, kv_[layer].D(), num_blocks_, stream),
               "fqa_store_kv");
  }

  bf16* KV(int layer) const { return reinterpret_cast<bf16*>(kv_[layer].D()); }
  int BlockSize() const { return FQA_PAGE_TOKENS; }
  int NumBlocks() const { return static_cast<int>(num_blocks_); }

 private:
  template <class Spec>
  static void CheckSpec(const Spec& spec) {
    detail::Dims(spec.num_heads, spec.num_kv_heads, spec.head_dim, FQA_PAGE_TOKENS, 6144, 0.f, 0.f);
    if (spec.num_layers < 1) detail::Fail("num_layers");
  }
  void Allocate(int64_t pages) {
    if (pages < 1) detail::Fail("KvStore: no pages");
    num_blocks_ = pages;
    const fqa_dims d{32, 8, 128, FQA_PAGE_TOKENS, 6144, 0.f, 0.f};
    const size_t elems = (size_t)fqa_pool_bytes(&d, pages) / 2;
    for (int l = 0; l < layers_; ++l) kv_.emplace_back(elems);  // may throw: nothing registered yet
    auto& r = detail::Reg();
    std::lock_guard<std::mutex> lock(r.mu);
    for (auto& b : kv_) r.pool_pages[b.D()] = pages;
  }
  int layers_;
  int64_t num_blocks_ = 0;
  std::vector<fqa::DeviceBuffer<uint16_t>> kv_;
};

// kernels.cuh:28-31: per-head RMSNorm + rotate-half RoPE of the q and k heads of M rows,
// in place.
inline void LaunchHeadNormRope(bf16* buf, const float* wq, const float* wk, const float* cos_tab,
                               const float* sin_tab, const int* pos, int M, int n_q, int n_kv,
                               int head_dim, int stride, float eps, hipStream_t s) {
  if (M <= 0) return;
  const StepContext& ctx = detail::ContextOf(s);
  if (pos != ctx.pos.D() || M != ctx.n_rows)
    detail::Fail("LaunchHeadNormRope: pos / M are not the stream's StepContext's");
  const fqa_dims d = detail::Dims(n_q, n_kv, head_dim, FQA_PAGE_TOKENS, stride, eps, 0.f);
  // rows past the table's end are left untouched by the kernel, never read past it
  fqa::Check(fqa_qknorm_rope(&d, reinterpret_cast<uint16_t*>(buf), wq, wk, cos_tab, sin_tab,
                             detail::RopeRowsOf(cos_tab, ctx.MaxCtx()), pos, ctx.Meta(), M, s),
             "fqa_qknorm_rope");
}

// attn_cute.h:14-20: decode attention of the qlen == 1 requests (split + combine).
inline void LaunchAttnDecodeCute(const bf16* q, int q_stride, const bf16* cache_kv, bf16* out,
                                 int n_heads, int n_kv, int head_dim, const int* pos,
                                 const int* qstart, const int* decode_rids, int n_decode,
                                 const int* bt, int max_blocks, int block_size, float scale,
                                 float* pm, float* pl, float* pa, hipStream_t s) {
  (void)pm;
  (void)pl;
  (void)pa;
  if (n_decode <= 0) return;  // attn_cute.cu:247
  const StepContext& ctx = detail::ContextOf(s);
  if (pos != ctx.pos.D() || qstart != ctx.qstart.D() || decode_rids != ctx.decode_rids.D() ||
      bt != ctx.bt.D() || max_blocks != ctx.bt_stride || n_decode != ctx.n_decode)
    detail::Fail("LaunchAttnDecodeCute: arrays are not the stream's StepContext's");
  const fqa_dims d = detail::Dims(n_heads, n_kv, head_dim, block_size, q_stride, 1e-6f, scale);
  fqa::Check(fqa_decode(&d, reinterpret_cast<const uint16_t*>(q),
                        reinterpret_cast<const uint16_t*>(cache_kv), detail::PoolPagesOf(cache_kv),
                        bt, max_blocks, ctx.DecWaves(), ctx.DecSeqs(), ctx.Meta(), ctx.DecWaveCap(),
                        n_decode, ctx.Workspace(), reinterpret_cast<uint16_t*>(out), s),
             "fqa_decode");
}

// attn_cute.h:7-12: causal varlen prefill attention of the qlen != 1 requests.
inline void LaunchAttnPrefillCute(const bf16* q, int q_stride, const bf16* cache_kv, bf16* out,
                                  int n_heads, int n_kv, int head_dim, const int* pos,
                                  const int* qstart, const int* qlen, const int* rids, int R,
                                  int max_qlen, const int* bt, int max_blocks, int block_size,
                                  float scale, hipStream_t s) {
  if (R <= 0) return;  // attn_cute.cu:155
  const StepContext& ctx = detail::ContextOf(s);
  if (pos != ctx.pos.D() || qstart != ctx.qstart.D() || qlen != ctx.qlen.D() ||
      rids != ctx.prefill_rids.D() || R != ctx.n_prefill || max_qlen != ctx.prefill_max_qlen ||
      bt != ctx.bt.D() || max_blocks != ctx.bt_stride)
    detail::Fail("LaunchAttnPrefillCute: arrays are not the stream's StepContext's");
  const fqa_dims d = detail::Dims(n_heads, n_kv, head_dim, block_size, q_stride, 1e-6f, scale);
  fqa::Check(fqa_prefill(&d, reinterpret_cast<const uint16_t*>(q),
                         reinterpret_cast<const uint16_t*>(cache_kv), detail::PoolPagesOf(cache_kv),
                         bt, max_blocks, qstart, pos, ctx.PreItems(), ctx.Meta(), FQA_PRE_TILE_Q,
                         ctx.PreItemCap(), reinterpret_cast<uint16_t*>(out), s),
             "fqa_prefill");
}

}  // namespace fq
