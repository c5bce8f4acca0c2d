// serve_cpp.cpp — a serving loop in C++: the host scheduler (include/fqa_sched.hpp) builds
// each step's batch from live request state and the attention path runs it on the GPU
// through the C++ step mirror (include/fqa_step.hpp), over one KV pool that persists
// across steps (appends, preemption, prefix-cache block reuse).  For
// tests/test_gpu_serve.py, which replays every step through the CPU oracle.
//
// argv: script norm_weights out
//   script: as tests/cpp/sched_cpp.cpp (n_blocks = pool pages), plus a trailing max_ctx.
//   norm_weights: float32 q_norm[128], k_norm[128].
//   out, per step with a batch: int32 step, R, T; computed[R]; n_new[R]; bt_off[R+1];
//   bt_pages[bt_off[R]]; uint16 qkv[T][6144] (the step's input); uint16 attn[T][4096];
//   int32 meta[16].  qkv rows are drawn from a fixed hash of (step, row).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <vector>

#include "../../include/fqa_sched.hpp"
#include "../../include/fqa_step.hpp"

static uint64_t mix(uint64_t x) {  // splitmix64 finaliser
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
static uint16_t bf16_of(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFF + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  std::ifstream in(argv[1]);
  int n_blocks, n_slots, budget, chunk, use_cache, n_steps, n_seqs;
  in >> n_blocks >> n_slots >> budget >> chunk >> use_cache >> n_steps >> n_seqs;
  struct Spec {
    int id, arrival, cancel, max_new, max_ctx;
    std::vector<int32_t> stop, prompt;
  };
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
  std::vector<float> wq(128), wk(128);
  {
    FILE* f = std::fopen(argv[2], "rb");
    if (!f || std::fread(wq.data(), 4, 128, f) != 128 || std::fread(wk.data(), 4, 128, f) != 128)
      return 2;
    std::fclose(f);
  }
  FILE* out = std::fopen(argv[3], "wb");
  if (!out) return 2;

  try {
    hipStream_t s;
    fqa::HipCheck(hipStreamCreate(&s), "stream");
    fqa::StepContext ctx(budget, n_slots, max_ctx, n_blocks);
    const size_t pool_elems = (size_t)n_blocks * 8 * 4096;
    fqa::DeviceBuffer<uint16_t> d_pool(pool_elems), d_qkv((size_t)budget * 6144),
        d_out((size_t)budget * 4096);
    fqa::DeviceBuffer<float> d_wq(128), d_wk(128);
    fqa::HipCheck(hipMemsetAsync(d_pool.D(), 0, pool_elems * 2, s), "memset");
    d_wq.Upload(wq.data(), 128, s);
    d_wk.Upload(wk.data(), 128, s);

    fqa::BlockAllocator alloc(n_blocks);
    fqa::HostScheduler sched(alloc, fqa::SchedConfig{n_slots, budget, chunk, use_cache != 0});
    std::map<int, fqa::Sequence*> live;
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
      if (sched.BuildBatch(b)) {
        const int R = (int)b.seqs.size(), T = b.rows;
        // the step's qkv input
        std::vector<uint16_t> qkv((size_t)T * 6144);
        for (int row = 0; row < T; ++row)
          for (int c = 0; c < 6144; ++c) {
            const uint64_t h = mix(((uint64_t)t << 40) ^ ((uint64_t)row << 16) ^ (uint64_t)c);
            qkv[(size_t)row * 6144 + c] = bf16_of((float)(h >> 40) * (4.0f / 16777216.0f) - 2.0f);
          }
        d_qkv.Upload(qkv.data(), qkv.size(), s);
        fqa::BatchInput bi{b.computed, b.n_new, b.block_tables};
        ctx.PrepareInputs(bi, s);
        ctx.RunLayer(d_qkv.D(), d_wq.D(), d_wk.D(), d_pool.D(), d_out.D(), s);
        std::vector<uint16_t> attn((size_t)T * 4096);
        std::vector<int32_t> meta(16);
        fqa::HipCheck(hipMemcpyAsync(attn.data(), d_out.D(), attn.size() * 2,
                                     hipMemcpyDeviceToHost, s), "d2h");
        fqa::HipCheck(hipMemcpyAsync(meta.data(), ctx.Meta(), 64, hipMemcpyDeviceToHost, s),
                      "d2h");
        fqa::HipCheck(hipStreamSynchronize(s), "sync");
        std::vector<int32_t> off(R + 1, 0), pages;
        for (int r = 0; r < R; ++r) {
          pages.insert(pages.end(), b.block_tables[r].begin(), b.block_tables[r].end());
          off[r + 1] = (int32_t)pages.size();
        }
        const int32_t hdr[3] = {t, R, T};
        std::fwrite(hdr, 4, 3, out);
        std::fwrite(b.computed.data(), 4, R, out);
        std::fwrite(b.n_new.data(), 4, R, out);
        std::fwrite(off.data(), 4, R + 1, out);
        std::fwrite(pages.data(), 4, pages.size(), out);
        std::fwrite(qkv.data(), 2, qkv.size(), out);
        std::fwrite(attn.data(), 2, attn.size(), out);
        std::fwrite(meta.data(), 4, 16, out);
        std::vector<int32_t> sampled;
        for (int si : b.sample_seqs)
          sampled.push_back(
              (int32_t)(((long long)b.seqs[si]->id * 7919 + (long long)t * 104729) % 50000));
        sched.Apply(b, sampled);
      }
      for (auto& r : sched.TakeRetired()) live.erase(r->id);
    }
    std::fclose(out);
    (void)hipStreamDestroy(s);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "serve_cpp: %s\n", e.what());
    return 1;
  }
  return 0;
}
