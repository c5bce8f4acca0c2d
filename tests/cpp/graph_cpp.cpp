// graph_cpp.cpp — one scheduler-driven workload run twice over 3 layers: eagerly
// (StepContext::PrepareInputs + RunLayer) and as a captured step graph replayed for every
// batch (StepContext::UploadBatch + StepGraph::Launch, include/fqa_step.hpp).  Every step's
// attention output and the final pools must be bit-identical.  The graph runs each
// layer's decode on a parallel branch (StepGraph's side stream).  For
// tests/test_gpu_graph.py.
//
// With the environment variable FQA_DEC_SHARE=1 both runs build the context with dec_share
// (the pack plans a mixed batch's decode for the CUs the concurrent prefill leaves) and the
// eager run also puts decode on the side stream.  FQA_DEC_PREFIX=N builds both with
// dec_prefix_pages N (decodes sharing at least N leading pages attend them once per group).
//
// argv: script norm_weights [out];  script as tests/cpp/serve_cpp.cpp.  Prints
// "steps S layers L compared N mismatched M" and exits 0 iff M == 0.  With `out`, the
// graph run's steps are written for the oracle check (little-endian, per step):
//   int32 t, R, T; computed[R], n_new[R], bt_off[R+1], bt_pages[bt_off[R]];
//   per layer: uint16 qkv[T*6144] (the step's input), uint16 attn[T*4096]; int32 meta[16]
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <vector>

#include "../../include/fqa_sched.hpp"
#include "../../include/fqa_step.hpp"

static uint64_t mix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
static uint16_t bf16_of(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFF + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}

struct Spec {
  int id, arrival, cancel, max_new, max_ctx;
  std::vector<int32_t> stop, prompt;
};

int main(int argc, char** argv) {
  if (argc != 3 && argc != 4) return 2;
  FILE* dump = argc == 4 ? std::fopen(argv[3], "wb") : nullptr;
  if (argc == 4 && !dump) return 2;
  std::ifstream in(argv[1]);
  int n_blocks, n_slots, budget, chunk, use_cache, n_steps, n_seqs;
  in >> n_blocks >> n_slots >> budget >> chunk >> use_cache >> n_steps >> n_seqs;
  std::vector<Spec> specs(n_seqs);
  for (auto& s : specs) {
    int ns, np;
    in >> s.id >> s.arrival >> s.cancel >> s.max_new >> s.max_ctx >> ns;
    s.stop.resize(ns);
    for (auto& x : s.stop) in >> x;
    in >> np;
    s.prompt.resize(np);
    for (auto& x : s.prompt) in >> x;
  }
  int max_ctx = 0;
  in >> max_ctx;
  if (!in) return 2;
  std::vector<float> w(256);
  {
    FILE* f = std::fopen(argv[2], "rb");
    if (!f || std::fread(w.data(), 4, 256, f) != 256) return 2;
    std::fclose(f);
  }
  constexpr int kLayers = 3;
  const char* share_env = std::getenv("FQA_DEC_SHARE");
  const bool dec_share = share_env && share_env[0] == '1';
  const char* prefix_env = std::getenv("FQA_DEC_PREFIX");
  const int dec_prefix = prefix_env ? std::atoi(prefix_env) : 0;
  long long compared = 0, mismatched = 0;
  int steps_run = 0;
  try {
    hipStream_t s, side;
    fqa::HipCheck(hipStreamCreate(&s), "stream");
    fqa::HipCheck(hipStreamCreate(&side), "stream");
    fqa::DeviceBuffer<float> d_w(256);
    d_w.Upload(w.data(), 256, s);
    const size_t pool_elems = (size_t)n_blocks * 8 * 4096;
    // eager outputs per step and layer, compared against the graph run
    std::vector<std::vector<uint16_t>> eager_out;
    std::vector<uint16_t> eager_pools;

    for (int mode = 0; mode < 2; ++mode) {
      fqa::StepContext ctx(budget, n_slots, max_ctx, n_blocks, 0, 0, 8, dec_share, dec_prefix);
      std::vector<fqa::DeviceBuffer<uint16_t>> pool, qkv, out;
      std::vector<fqa::LayerBuffers> lb;
      for (int l = 0; l < kLayers; ++l) {
        pool.emplace_back(pool_elems);
        qkv.emplace_back((size_t)budget * 6144);
        out.emplace_back((size_t)budget * 4096);
        fqa::HipCheck(hipMemsetAsync(pool[l].D(), 0, pool_elems * 2, s), "memset");
      }
      for (int l = 0; l < kLayers; ++l)
        lb.push_back({qkv[l].D(), d_w.D(), d_w.D() + 128, pool[l].D(), out[l].D()});
      std::unique_ptr<fqa::StepGraph> graph;
      // the graph puts each layer's decode on a parallel branch (a second stream)
      if (mode == 1) graph = std::make_unique<fqa::StepGraph>(ctx, lb, s, side);

      fqa::BlockAllocator alloc(n_blocks);
      fqa::HostScheduler sched(alloc, fqa::SchedConfig{n_slots, budget, chunk, use_cache != 0});
      std::map<int, fqa::Sequence*> live;
      int k = 0;
      for (int t = 0; t < n_steps; ++t) {
        for (auto& sp : specs) {
          if (sp.arrival == t) {
            auto q = std::make_unique<fqa::Sequence>();
            q->id = sp.id;
            q->tokens = sp.prompt;
            q->prompt_len = (int)sp.prompt.size();
            q->max_new = sp.max_new;
            q->max_ctx = sp.max_ctx;
            q->stop_ids = sp.stop;
            live[sp.id] = q.get();
            sched.Submit(std::move(q));
          }
          if (sp.cancel == t && live.count(sp.id)) live[sp.id]->cancelled = true;
        }
        sched.Refill();
        fqa::SchedBatch b;
        if (!sched.BuildBatch(b)) continue;
        const int T = b.rows;
        std::vector<std::vector<uint16_t>> inputs(kLayers);
        for (int l = 0; l < kLayers; ++l) {  // the step's inputs, outside any graph
          std::vector<uint16_t>& h = inputs[l];
          h.resize((size_t)T * 6144);
          for (int row = 0; row < T; ++row)
            for (int c = 0; c < 6144; ++c) {
              const uint64_t x = mix(((uint64_t)t << 44) ^ ((uint64_t)l << 40) ^
                                     ((uint64_t)row << 16) ^ (uint64_t)c);
              h[(size_t)row * 6144 + c] = bf16_of((float)(x >> 40) * (4.0f / 16777216.0f) - 2.0f);
            }
          qkv[l].Upload(h.data(), h.size(), s);
          fqa::HipCheck(hipStreamSynchronize(s), "sync");
        }
        fqa::BatchInput bi{b.computed, b.n_new, b.block_tables};
        if (mode == 0) {
          ctx.PrepareInputs(bi, s);
          for (auto& l : lb) ctx.RunLayer(l.qkv, l.q_norm, l.k_norm, l.pool, l.out, s,
                                     dec_share ? side : nullptr);
        } else {
          ctx.UploadBatch(bi, s);
          graph->Launch(s);
        }
        if (mode == 1 && dump) {
          const int R = (int)b.computed.size();
          std::vector<int32_t> off(R + 1, 0), pages;
          for (int r = 0; r < R; ++r) {
            pages.insert(pages.end(), b.block_tables[r].begin(), b.block_tables[r].end());
            off[r + 1] = (int32_t)pages.size();
          }
          const int32_t hdr[3] = {t, R, T};
          std::fwrite(hdr, 4, 3, dump);
          std::fwrite(b.computed.data(), 4, R, dump);
          std::fwrite(b.n_new.data(), 4, R, dump);
          std::fwrite(off.data(), 4, R + 1, dump);
          std::fwrite(pages.data(), 4, pages.size(), dump);
        }
        for (int l = 0; l < kLayers; ++l) {
          std::vector<uint16_t> h((size_t)T * 4096);
          fqa::HipCheck(hipMemcpyAsync(h.data(), out[l].D(), h.size() * 2, hipMemcpyDeviceToHost,
                                       s), "d2h");
          fqa::HipCheck(hipStreamSynchronize(s), "sync");
          if (mode == 1 && dump) {
            std::fwrite(inputs[l].data(), 2, inputs[l].size(), dump);
            std::fwrite(h.data(), 2, h.size(), dump);
          }
          if (mode == 0) {
            eager_out.push_back(std::move(h));
          } else {
            const auto& e = eager_out[k];
            ++compared;
            if (e.size() != h.size() || std::memcmp(e.data(), h.data(), h.size() * 2) != 0)
              ++mismatched;
          }
          ++k;
        }
        if (mode == 1 && dump) {
          int32_t meta[16];
          fqa::HipCheck(hipMemcpy(meta, ctx.Meta(), 64, hipMemcpyDeviceToHost), "meta");
          std::fwrite(meta, 4, 16, dump);
        }
        std::vector<int32_t> sampled;
        for (int si : b.sample_seqs)
          sampled.push_back(
              (int32_t)(((long long)b.seqs[si]->id * 7919 + (long long)t * 104729) % 50000));
        sched.Apply(b, sampled);
        for (auto& r : sched.TakeRetired()) live.erase(r->id);
        if (mode == 0) ++steps_run;
      }
      // final pools
      std::vector<uint16_t> hp(pool_elems * kLayers);
      for (int l = 0; l < kLayers; ++l)
        fqa::HipCheck(hipMemcpyAsync(hp.data() + l * pool_elems, pool[l].D(), pool_elems * 2,
                                     hipMemcpyDeviceToHost, s), "d2h");
      fqa::HipCheck(hipStreamSynchronize(s), "sync");
      if (mode == 0) {
        eager_pools = std::move(hp);
      } else {
        ++compared;
        if (std::memcmp(eager_pools.data(), hp.data(), hp.size() * 2) != 0) ++mismatched;
      }
    }
    (void)hipStreamDestroy(side);
    (void)hipStreamDestroy(s);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "graph_cpp: %s\n", e.what());
    return 1;
  }
  if (dump) std::fclose(dump);
  std::printf("steps %d layers %d compared %lld mismatched %lld\n", steps_run, kLayers, compared,
              mismatched);
  return mismatched == 0 ? 0 : 3;
}
