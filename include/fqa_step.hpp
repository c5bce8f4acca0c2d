// fqa_step.hpp — C++ host-side mirror of the reference engine's per-step attention
// interface, over the C ABI of fqa.h.  Header-only; link with libfqa.so and amdhip64.
//
// Reference interface it mirrors (engine/src/):
//   StepContext::StepContext(max_rows, slots, max_ctx)      model_runtime.h:119-136
//   StepContext::PrepareInputs(ForwardInput, rng, stream)   model_runtime.cu:295-302
//   LaunchHeadNormRope(...) + KvStore::StoreKV(...)          kernels.cuh:28-31, kv_store.h:29-31
//   LaunchAttnDecodeCute(...)                                attn_cute.h:14-20
//   LaunchAttnPrefillCute(...)                               attn_cute.h:7-12
//   GraphCache (decode-step capture)                         model_runtime.h:160-201
//
// Differences a caller sees: PrepareInputs takes the batch as plain host vectors (the
// reference's ForwardInput rows are derived on the device from computed/n per request),
// and errors throw std::runtime_error with the FQA_E* code instead of exit(1).
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "fqa.h"

namespace fqa {

inline void Check(int rc, const char* what) {
  if (rc != FQA_OK) throw std::runtime_error(std::string(what) + " failed: " + std::to_string(rc));
}
inline void HipCheck(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Owning device buffer (the reference's DeviceBuffer, cuda_helpers.h:38-78).
template <class T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t n) : n_(n) {
    if (n) HipCheck(hipMalloc(&p_, n * sizeof(T)), "hipMalloc");
  }
  DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) { Free(); p_ = o.p_; n_ = o.n_; o.p_ = nullptr; o.n_ = 0; }
    return *this;
  }
  ~DeviceBuffer() { Free(); }
  T* D() const { return p_; }
  size_t Size() const { return n_; }
  void Upload(const T* h, size_t n, hipStream_t s) {
    HipCheck(hipMemcpyAsync(p_, h, n * sizeof(T), hipMemcpyHostToDevice, s), "upload");
  }

 private:
  void Free() { if (p_) (void)hipFree(p_); p_ = nullptr; }
  T* p_ = nullptr;
  size_t n_ = 0;
};

// One step's batch as the scheduler hands it over (Request::EmitChunk, scheduler.h:66-72):
// request r adds n_new[r] rows at positions computed[r]..; block_tables[r] are its pages.
struct BatchInput {
  std::vector<int32_t> computed, n_new;
  std::vector<std::vector<int32_t>> block_tables;
};

class StepContext {
 public:
  // dec_share: RunLayer / RunLayerBounded will be given a side stream, so the pack plans a
  // mixed batch's decode for the CUs the concurrent prefill leaves (fqa.h, dec_share).
  // dec_prefix_pages > 0: decode sequences sharing at least that many leading pages attend
  // them once per group (fqa_decode_prefix), with up to dec_pre_cap prefix items a step.
  StepContext(int max_rows, int slots, int max_ctx, int64_t pool_pages, int device = 0,
              int dec_grid_waves = 0, int dec_min_pages = 8, bool dec_share = false,
              int dec_prefix_pages = 0, int dec_pre_cap = 4096)
      : max_rows_(max_rows), slots_(slots), max_ctx_(max_ctx), pool_pages_(pool_pages) {
    if (slots > FQA_MAX_REQS) throw std::runtime_error("slots > FQA_MAX_REQS");
    max_blocks_ = (max_ctx + FQA_PAGE_TOKENS - 1) / FQA_PAGE_TOKENS;
    dims_ = {32, 8, 128, FQA_PAGE_TOKENS, 6144, 1e-6f, 1.0f / std::sqrt(128.0f)};
    if (dec_grid_waves <= 0) dec_grid_waves = fqa_dec_default_waves(device);
    if (dec_grid_waves <= 0) dec_grid_waves = 1024;
    dec_cap_ = fqa_dec_wave_bound(slots, dec_grid_waves);
    pre_cap_ = fqa_pre_item_bound(slots, max_rows, FQA_PRE_TILE_Q);
    prefix_ = dec_prefix_pages > 0;
    dpre_cap_ = prefix_ ? dec_pre_cap : 0;
    cfg_ = {max_rows, max_blocks_, pool_pages, dec_grid_waves, dec_min_pages, dec_cap_, FQA_PRE_TILE_Q,
            pre_cap_, dec_share ? 1 : 0, prefix_ ? dec_prefix_pages : 0, dpre_cap_};
    computed_ = DeviceBuffer<int32_t>(slots);
    n_new_ = DeviceBuffer<int32_t>(slots);
    bt_off_ = DeviceBuffer<int32_t>(slots + 1);
    bt_pages_ = DeviceBuffer<int32_t>((size_t)slots * max_blocks_);
    cu_ = DeviceBuffer<int32_t>(slots + 1);
    qlen_ = DeviceBuffer<int32_t>(slots);
    pos_ = DeviceBuffer<int32_t>(max_rows);
    req_ = DeviceBuffer<int32_t>(max_rows);
    slot_ = DeviceBuffer<int32_t>(max_rows);
    bt_ = DeviceBuffer<int32_t>((size_t)slots * max_blocks_);
    drids_ = DeviceBuffer<int32_t>(slots);
    prids_ = DeviceBuffer<int32_t>(slots);
    dseqs_ = DeviceBuffer<int32_t>((size_t)slots * 4);
    dwaves_ = DeviceBuffer<int32_t>((size_t)dec_cap_ * 8);
    items_ = DeviceBuffer<int32_t>((size_t)pre_cap_ * 4);
    meta_ = DeviceBuffer<int32_t>(FQA_META_LEN);
    nreq_ = DeviceBuffer<int32_t>(1);
    if (prefix_) {
      dprefix_ = DeviceBuffer<int32_t>((size_t)std::max(slots, 1) * 8);
      dpre_items_ = DeviceBuffer<int32_t>((size_t)std::max(dpre_cap_, 1) * 12);
    }
    ws_ = DeviceBuffer<unsigned char>(
        (size_t)(prefix_ ? fqa_decode_prefix_workspace_bytes(&dims_, dec_cap_, dpre_cap_)
                         : fqa_decode_workspace_bytes(&dims_, dec_cap_)));
    std::vector<float> c((size_t)max_ctx * 64), s((size_t)max_ctx * 64);
    Check(fqa_rope_tables(max_ctx, 128, 1.0e6f, c.data(), s.data()), "fqa_rope_tables");
    cos_ = DeviceBuffer<float>(c.size());
    sin_ = DeviceBuffer<float>(s.size());
    cos_.Upload(c.data(), c.size(), nullptr);
    sin_.Upload(s.data(), s.size(), nullptr);
    HipCheck(hipDeviceSynchronize(), "rope upload");
    HipCheck(hipEventCreateWithFlags(&fork_, hipEventDisableTiming), "event");
    HipCheck(hipEventCreateWithFlags(&join_, hipEventDisableTiming), "event");
  }

  // StepContext::PrepareInputs: upload the per-request batch and pack it on the GPU.
  void PrepareInputs(const BatchInput& in, hipStream_t stream) {
    UploadBatch(in, stream);
    fqa_batch b{computed_.D(), n_new_.D(), bt_off_.D(), bt_pages_.D(), nullptr, n_reqs_};
    fqa_pack_out o = PackOut();
    Check(fqa_pack(&b, &cfg_, &o, stream), "fqa_pack");
  }

  // The host half of PrepareInputs: copy the batch (and its request count) to the device.
  // With Pack / RunLayerBounded, the device half can be captured once (StepGraph) and
  // replayed for every batch.
  void UploadBatch(const BatchInput& in, hipStream_t stream) {
    const int R = (int)in.computed.size();
    if (R > slots_) throw std::runtime_error("batch larger than slots");
    h_off_.assign(R + 1, 0);
    h_pages_.clear();
    rows_ = 0;
    for (int r = 0; r < R; ++r) {
      h_pages_.insert(h_pages_.end(), in.block_tables[r].begin(), in.block_tables[r].end());
      h_off_[r + 1] = (int32_t)h_pages_.size();
      rows_ += in.n_new[r];
    }
    if (h_pages_.size() > bt_pages_.Size()) throw std::runtime_error("block tables too long");
    if (R) {
      computed_.Upload(in.computed.data(), R, stream);
      n_new_.Upload(in.n_new.data(), R, stream);
    }
    bt_off_.Upload(h_off_.data(), R + 1, stream);
    if (!h_pages_.empty()) bt_pages_.Upload(h_pages_.data(), h_pages_.size(), stream);
    h_nreq_ = R;
    nreq_.Upload(&h_nreq_, 1, stream);
    n_reqs_ = R;
    has_decode_ = has_prefill_ = false;
    for (int r = 0; r < R; ++r) (in.n_new[r] == 1 ? has_decode_ : has_prefill_) = true;
  }

  // The device half: fqa_pack over the uploaded batch with the request count read on the
  // device and grids sized from the context's bounds (slots, max_rows).
  void Pack(hipStream_t stream) const {
    fqa_batch b{computed_.D(), n_new_.D(), bt_off_.D(), bt_pages_.D(), nreq_.D(), slots_};
    fqa_pack_out o = PackOut();
    Check(fqa_pack(&b, &cfg_, &o, stream), "fqa_pack");
  }
  // RunLayer for any batch within the bounds: rows and requests bounded by max_rows and
  // slots, both attention kernels launched (each does nothing without its kind of rows).
  // With `side`, the decode runs on it beside the prefill, queued first (see RunLayer).
  void RunLayerBounded(uint16_t* qkv, const float* q_norm, const float* k_norm,
                       uint16_t* pool_layer, uint16_t* out, hipStream_t stream,
                       hipStream_t side = nullptr) const {
    Check(fqa_qknorm_rope_append(&dims_, qkv, q_norm, k_norm, cos_.D(), sin_.D(), max_ctx_,
                                 pos_.D(), slot_.D(), meta_.D(), max_rows_, pool_layer,
                                 pool_pages_, 0, stream),
          "fqa_qknorm_rope_append");
    if (side) Fork(stream, side);
    Decode(qkv, pool_layer, out, slots_, side ? side : stream);
    Check(fqa_prefill(&dims_, qkv, pool_layer, pool_pages_, bt_.D(), max_blocks_, cu_.D(),
                      pos_.D(), items_.D(), meta_.D(), FQA_PRE_TILE_Q, pre_cap_, out, stream),
          "fqa_prefill");
    if (side) Join(stream, side);
  }

  // LaunchHeadNormRope + KvStore::StoreKV for one layer (fused).
  void HeadNormRopeStoreKV(uint16_t* qkv, const float* q_norm, const float* k_norm,
                           uint16_t* pool_layer, hipStream_t stream) const {
    Check(fqa_qknorm_rope_append(&dims_, qkv, q_norm, k_norm, cos_.D(), sin_.D(), max_ctx_,
                                 pos_.D(), slot_.D(), meta_.D(), rows_, pool_layer, pool_pages_,
                                 0, stream),
          "fqa_qknorm_rope_append");
  }
  // LaunchGemm(QKV) + LaunchHeadNormRope + StoreKV for one layer, fused
  // (fqa_qkv_proj_append): x [rows, hidden] bf16 (row stride ldx), w_qkv [6144, hidden].
  // `workspace` holds fqa_gemm_workspace_bytes(max_rows, 6144, hidden) bytes.
  void QkvProjAppend(const uint16_t* x, int64_t ldx, const uint16_t* w_qkv, int hidden,
                     uint16_t* qkv, const float* q_norm, const float* k_norm,
                     uint16_t* pool_layer, void* workspace, int64_t workspace_bytes,
                     hipStream_t stream) const {
    Check(fqa_qkv_proj_append(&dims_, x, ldx, w_qkv, hidden, rows_, hidden, qkv, q_norm, k_norm,
                              cos_.D(), sin_.D(), max_ctx_, pos_.D(), slot_.D(), meta_.D(),
                              pool_layer, pool_pages_, 0, workspace, workspace_bytes, stream),
          "fqa_qkv_proj_append");
  }
  // LaunchAttnDecodeCute.
  void AttnDecode(const uint16_t* qkv, const uint16_t* pool_layer, uint16_t* out,
                  hipStream_t stream) const {
    if (!has_decode_) return;
    Decode(qkv, pool_layer, out, n_reqs_, stream);
  }
  // LaunchAttnPrefillCute.
  void AttnPrefill(const uint16_t* qkv, const uint16_t* pool_layer, uint16_t* out,
                   hipStream_t stream) const {
    if (!has_prefill_) return;
    Check(fqa_prefill(&dims_, qkv, pool_layer, pool_pages_, bt_.D(), max_blocks_, cu_.D(),
                      pos_.D(), items_.D(), meta_.D(), FQA_PRE_TILE_Q, pre_cap_, out, stream),
          "fqa_prefill");
  }
  // The attention block of one layer (model_runtime.cu:263-278).  With `side` and a
  // mixed batch, the decode is queued on `side` first and the prefill on `stream` after
  // it: the two write disjoint output rows and only read the pool.  Each decode workgroup
  // holds a CU alone (its LDS reservation), so the decode takes its CUs first and the
  // prefill fills the others; with dec_share the decode plan leaves the prefill a share of
  // the CUs in proportion to its work (config 4: 0.695 -> 0.653 ms per step).
  // `stream` waits for `side` before returning.
  void RunLayer(uint16_t* qkv, const float* q_norm, const float* k_norm, uint16_t* pool_layer,
                uint16_t* out, hipStream_t stream, hipStream_t side = nullptr) const {
    HeadNormRopeStoreKV(qkv, q_norm, k_norm, pool_layer, stream);
    if (side && has_decode_ && has_prefill_) {
      Fork(stream, side);
      AttnDecode(qkv, pool_layer, out, side);
      AttnPrefill(qkv, pool_layer, out, stream);
      Join(stream, side);
      return;
    }
    AttnDecode(qkv, pool_layer, out, stream);
    AttnPrefill(qkv, pool_layer, out, stream);
  }

  const int32_t* Meta() const { return meta_.D(); }
  int Rows() const { return rows_; }

  StepContext(const StepContext&) = delete;
  StepContext& operator=(const StepContext&) = delete;
  ~StepContext() {
    if (fork_) (void)hipEventDestroy(fork_);
    if (join_) (void)hipEventDestroy(join_);
  }

 private:
  // fqa_decode, or fqa_decode_prefix when the context plans shared-prefix groups
  void Decode(const uint16_t* qkv, const uint16_t* pool_layer, uint16_t* out, int n_reqs_bound,
              hipStream_t stream) const {
    if (prefix_)
      Check(fqa_decode_prefix(&dims_, qkv, pool_layer, pool_pages_, bt_.D(), max_blocks_,
                              dwaves_.D(), dseqs_.D(), dprefix_.D(), dpre_items_.D(), meta_.D(),
                              dec_cap_, dpre_cap_, n_reqs_bound, ws_.D(), out, stream),
            "fqa_decode_prefix");
    else
      Check(fqa_decode(&dims_, qkv, pool_layer, pool_pages_, bt_.D(), max_blocks_, dwaves_.D(),
                       dseqs_.D(), meta_.D(), dec_cap_, n_reqs_bound, ws_.D(), out, stream),
            "fqa_decode");
  }
  // side starts after everything queued on stream so far; stream continues after side.
  // Events record and wait only (capture-safe).
  void Fork(hipStream_t stream, hipStream_t side) const {
    HipCheck(hipEventRecord(fork_, stream), "fork record");
    HipCheck(hipStreamWaitEvent(side, fork_, 0), "fork wait");
  }
  void Join(hipStream_t stream, hipStream_t side) const {
    HipCheck(hipEventRecord(join_, side), "join record");
    HipCheck(hipStreamWaitEvent(stream, join_, 0), "join wait");
  }

  fqa_pack_out PackOut() const {
    return fqa_pack_out{cu_.D(), qlen_.D(), pos_.D(), req_.D(), slot_.D(), bt_.D(),
                        drids_.D(), prids_.D(), dseqs_.D(), dwaves_.D(), items_.D(), meta_.D(),
                        prefix_ ? dprefix_.D() : nullptr, prefix_ ? dpre_items_.D() : nullptr};
  }

  int max_rows_, slots_, max_ctx_, max_blocks_ = 0;
  int64_t pool_pages_;
  int dec_cap_ = 0, pre_cap_ = 0, n_reqs_ = 0, rows_ = 0;
  bool prefix_ = false;  // shared-prefix decode groups (dec_prefix_pages > 0)
  int dpre_cap_ = 0;
  bool has_decode_ = false, has_prefill_ = false;
  fqa_dims dims_{};
  fqa_pack_cfg cfg_{};
  std::vector<int32_t> h_off_, h_pages_;
  int32_t h_nreq_ = 0;  // host copy the request-count upload reads (kept until the copy ran)
  DeviceBuffer<int32_t> computed_, n_new_, bt_off_, bt_pages_;
  DeviceBuffer<int32_t> cu_, qlen_, pos_, req_, slot_, bt_, drids_, prids_, dseqs_, dwaves_, items_,
      meta_, nreq_, dprefix_, dpre_items_;
  DeviceBuffer<unsigned char> ws_;
  DeviceBuffer<float> cos_, sin_;
  hipEvent_t fork_ = nullptr, join_ = nullptr;
};

// Buffers of one layer's attention block.
struct LayerBuffers {
  uint16_t* qkv;
  const float* q_norm;
  const float* k_norm;
  uint16_t* pool;
  uint16_t* out;
};

// One step captured as a HIP graph (the reference's GraphCache, model_runtime.h:160-201):
// the pack and every layer's attention block.  Counts are read on the device from `meta`,
// so where the reference keeps one graph per (rows, decodes) shape, one graph here serves
// every batch within the context's bounds: per step, UploadBatch outside the graph, then
// Launch.  The captured launches allocate nothing and record no memset.
class StepGraph {
 public:
  // With `side`, each layer's decode is a branch parallel to its prefill (RunLayer).
  StepGraph(const StepContext& ctx, const std::vector<LayerBuffers>& layers,
            hipStream_t stream, hipStream_t side = nullptr) {
    HipCheck(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "begin capture");
    try {
      ctx.Pack(stream);
      for (const LayerBuffers& l : layers)
        ctx.RunLayerBounded(l.qkv, l.q_norm, l.k_norm, l.pool, l.out, stream, side);
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    HipCheck(hipStreamEndCapture(stream, &graph_), "end capture");
    HipCheck(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0), "instantiate");
  }
  StepGraph(const StepGraph&) = delete;
  StepGraph& operator=(const StepGraph&) = delete;
  ~StepGraph() {
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
  }
  void Launch(hipStream_t stream) const { HipCheck(hipGraphLaunch(exec_, stream), "launch"); }

 private:
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t exec_ = nullptr;
};

}  // namespace fqa
