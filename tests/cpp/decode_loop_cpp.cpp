// decode_loop_cpp.cpp — the serving loop with tokens produced on the device: the host
// scheduler (include/fqa_sched.hpp) builds each step's batch; every row's input is the
// embedding of its token; per layer the QKV projection fused with norm/RoPE/append
// (StepContext::QkvProjAppend), the attention (decode + prefill) and the o_proj
// projection (fqa_gemm) run on the GPU; the last row of every sequence that completes
// its prompt or decode step goes through lm_head (fqa_gemm, fp32 logits) and fqa_sample,
// the greedy rows' tokens come from the fused lm_head + greedy pick (fqa_gemm_argmax over
// all the rows, the sampled rows' picks then taken from fqa_sample), and the tokens go
// back to the scheduler (Apply).  Random weights, no MLP or
// residual: the loop exercises the boundary entry points end to end.  For
// tests/test_gpu_decode_loop.py.
//
// argv: script vocab hidden layers out_dir
//   script as tests/cpp/serve_cpp.cpp.  Writes out_dir/steps.bin: per step with samples,
//   int32 t, n; per sample int32 seq id, float inv_temp, top_p, u, int32 token; then bf16
//   hidden[n][hidden] (the rows lm_head read).  out_dir/w_lm.bin: bf16 [vocab][hidden].
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
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
static float unit(uint64_t h) { return (float)(h >> 40) * (1.0f / 16777216.0f); }  // [0, 1)
// n values uniform in [-a, a), keyed by (tag, index)
static std::vector<uint16_t> weights(uint64_t tag, size_t n, float a) {
  std::vector<uint16_t> w(n);
  for (size_t i = 0; i < n; ++i) w[i] = bf16_of((2.0f * unit(mix((tag << 40) ^ i)) - 1.0f) * a);
  return w;
}

int main(int argc, char** argv) {
  if (argc != 6) return 2;
  const int vocab = std::atoi(argv[2]), hidden = std::atoi(argv[3]), layers = std::atoi(argv[4]);
  const std::string out_dir = argv[5];
  std::ifstream in(argv[1]);
  int n_blocks, n_slots, budget, chunk, use_cache, n_steps, n_seqs;
  in >> n_blocks >> n_slots >> budget >> chunk >> use_cache >> n_steps >> n_seqs;
  struct Spec {
    int id, arrival, cancel, max_new, max_ctx;
    std::vector<int32_t> stop, prompt;
  };
  std::vector<Spec> specs(n_seqs);
  for (auto& sp : specs) {
    int ns, np;
    in >> sp.id >> sp.arrival >> sp.cancel >> sp.max_new >> sp.max_ctx >> ns;
    sp.stop.resize(ns);
    for (auto& x : sp.stop) in >> x;
    in >> np;
    sp.prompt.resize(np);
    for (auto& x : sp.prompt) in >> x;
  }
  int max_ctx = 0;
  in >> max_ctx;
  if (!in || vocab < 128 || vocab % 128 || hidden < 128 || hidden % 128 || layers < 1) return 2;
  FILE* out = std::fopen((out_dir + "/steps.bin").c_str(), "wb");
  if (!out) return 2;

  try {
    hipStream_t s;
    fqa::HipCheck(hipStreamCreate(&s), "stream");
    fqa::StepContext ctx(budget, n_slots, max_ctx, n_blocks);
    const size_t pool_elems = (size_t)n_blocks * 8 * 4096;

    // weights: embedding, per layer W_qkv and W_o, lm_head
    const std::vector<uint16_t> emb = weights(1, (size_t)vocab * hidden, 1.7f);
    const std::vector<uint16_t> w_lm = weights(2, (size_t)vocab * hidden, 1.7f / std::sqrt((float)hidden));
    {
      FILE* f = std::fopen((out_dir + "/w_lm.bin").c_str(), "wb");
      if (!f) return 2;
      std::fwrite(w_lm.data(), 2, w_lm.size(), f);
      std::fclose(f);
    }
    std::vector<fqa::DeviceBuffer<uint16_t>> pool, w_qkv, w_o;
    for (int l = 0; l < layers; ++l) {
      pool.emplace_back(pool_elems);
      fqa::HipCheck(hipMemsetAsync(pool[l].D(), 0, pool_elems * 2, s), "memset");
      const auto wq = weights(10 + 2 * l, (size_t)6144 * hidden, 1.7f / std::sqrt((float)hidden));
      const auto wo = weights(11 + 2 * l, (size_t)hidden * 4096, 1.7f / std::sqrt(4096.0f));
      w_qkv.emplace_back(wq.size());
      w_qkv[l].Upload(wq.data(), wq.size(), s);
      w_o.emplace_back(wo.size());
      w_o[l].Upload(wo.data(), wo.size(), s);
      fqa::HipCheck(hipStreamSynchronize(s), "sync");  // wq, wo go out of scope
    }
    fqa::DeviceBuffer<uint16_t> d_lm(w_lm.size()), x((size_t)budget * hidden),
        qkv((size_t)budget * 6144), attn((size_t)budget * 4096), xs((size_t)n_slots * hidden);
    d_lm.Upload(w_lm.data(), w_lm.size(), s);
    std::vector<float> ones(256, 1.0f);
    fqa::DeviceBuffer<float> norm_w(256), logits((size_t)n_slots * vocab), d_it(n_slots),
        d_tp(n_slots), d_u(n_slots);
    norm_w.Upload(ones.data(), 256, s);
    fqa::DeviceBuffer<int32_t> d_tok(n_slots), d_greedy(n_slots);
    const int64_t am_bytes = fqa_gemm_argmax_workspace_bytes(n_slots, vocab, hidden);
    fqa::DeviceBuffer<unsigned char> am_ws((size_t)std::max<int64_t>(am_bytes, 16));
    int64_t ws_bytes = 0;  // the largest split-K workspace any step's shapes need
    for (int m = 1; m <= budget; ++m)
      ws_bytes = std::max({ws_bytes, fqa_gemm_workspace_bytes(m, 6144, hidden),
                           fqa_gemm_workspace_bytes(m, hidden, 4096),
                           m <= n_slots ? fqa_gemm_workspace_bytes(m, vocab, hidden) : 0});
    fqa::DeviceBuffer<unsigned char> ws((size_t)std::max<int64_t>(ws_bytes, 16));
    fqa::HipCheck(hipStreamSynchronize(s), "sync");

    fqa::BlockAllocator alloc(n_blocks);
    fqa::HostScheduler sched(alloc, fqa::SchedConfig{n_slots, budget, chunk, use_cache != 0});
    std::map<int, fqa::Sequence*> live;
    std::vector<uint16_t> hx;
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
        // inputs: the embedding of each row's token
        hx.assign((size_t)T * hidden, 0);
        std::vector<int> row0(R);
        for (int r = 0, row = 0; r < R; ++r) {
          row0[r] = row;
          for (int k = 0; k < b.n_new[r]; ++k, ++row) {
            const int tok = b.seqs[r]->tokens[b.computed[r] + k];
            std::memcpy(&hx[(size_t)row * hidden], &emb[(size_t)(tok % vocab) * hidden], hidden * 2);
          }
        }
        x.Upload(hx.data(), hx.size(), s);
        ctx.PrepareInputs(fqa::BatchInput{b.computed, b.n_new, b.block_tables}, s);
        for (int l = 0; l < layers; ++l) {
          ctx.QkvProjAppend(x.D(), hidden, w_qkv[l].D(), hidden, qkv.D(), norm_w.D(),
                            norm_w.D() + 128, pool[l].D(), ws.D(), ws_bytes, s);
          ctx.AttnDecode(qkv.D(), pool[l].D(), attn.D(), s);
          ctx.AttnPrefill(qkv.D(), pool[l].D(), attn.D(), s);
          fqa::Check(fqa_gemm(attn.D(), 4096, w_o[l].D(), 4096, x.D(), hidden, T, hidden, 4096, 0,
                              ws.D(), ws_bytes, s),
                     "o_proj");
        }
        // lm_head + sampling on the rows whose sequences produce a token this step
        const int n = (int)b.sample_seqs.size();
        std::vector<int32_t> sampled(n);
        if (n > 0) {
          std::vector<float> it(n), tp(n), u(n);
          for (int i = 0; i < n; ++i) {
            const int r = b.sample_seqs[i];
            const int id = b.seqs[r]->id;
            const uint16_t* src = x.D() + (size_t)(row0[r] + b.n_new[r] - 1) * hidden;
            fqa::HipCheck(hipMemcpyAsync(xs.D() + (size_t)i * hidden, src, hidden * 2,
                                         hipMemcpyDeviceToDevice, s), "gather");
            it[i] = id % 2 ? 0.0f : 1.0f;  // odd ids greedy, even ids temperature 1
            tp[i] = id % 4 == 0 ? 0.9f : 1.0f;
            u[i] = unit(mix(((uint64_t)id << 32) ^ (uint64_t)t));
          }
          d_it.Upload(it.data(), n, s);
          d_tp.Upload(tp.data(), n, s);
          d_u.Upload(u.data(), n, s);
          fqa::Check(fqa_gemm(xs.D(), hidden, d_lm.D(), hidden, logits.D(), vocab, n, vocab, hidden,
                              1, ws.D(), ws_bytes, s),
                     "lm_head");
          fqa::Check(fqa_sample(logits.D(), n, vocab, vocab, d_it.D(), d_tp.D(), d_u.D(), d_tok.D(), s),
                     "fqa_sample");
          // every row through the fused lm_head + greedy pick; the greedy rows keep it
          fqa::Check(fqa_gemm_argmax(xs.D(), hidden, d_lm.D(), hidden, n, vocab, hidden,
                                     d_greedy.D(), am_ws.D(), am_bytes, s),
                     "fqa_gemm_argmax");
          std::vector<uint16_t> hs((size_t)n * hidden);
          std::vector<int32_t> greedy(n);
          fqa::HipCheck(hipMemcpyAsync(sampled.data(), d_tok.D(), n * 4, hipMemcpyDeviceToHost, s), "d2h");
          fqa::HipCheck(hipMemcpyAsync(greedy.data(), d_greedy.D(), n * 4, hipMemcpyDeviceToHost, s), "d2h");
          fqa::HipCheck(hipMemcpyAsync(hs.data(), xs.D(), hs.size() * 2, hipMemcpyDeviceToHost, s), "d2h");
          fqa::HipCheck(hipStreamSynchronize(s), "sync");
          for (int i = 0; i < n; ++i)
            if (it[i] <= 0.0f) sampled[i] = greedy[i];
          const int32_t hdr[2] = {t, n};
          std::fwrite(hdr, 4, 2, out);
          for (int i = 0; i < n; ++i) {
            const int32_t id = b.seqs[b.sample_seqs[i]]->id;
            std::fwrite(&id, 4, 1, out);
            std::fwrite(&it[i], 4, 1, out);
            std::fwrite(&tp[i], 4, 1, out);
            std::fwrite(&u[i], 4, 1, out);
            std::fwrite(&sampled[i], 4, 1, out);
          }
          std::fwrite(hs.data(), 2, hs.size(), out);
        } else {
          fqa::HipCheck(hipStreamSynchronize(s), "sync");
        }
        sched.Apply(b, sampled);
      }
      for (auto& r : sched.TakeRetired()) live.erase(r->id);
    }
    std::fclose(out);
    (void)hipStreamDestroy(s);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "decode_loop_cpp: %s\n", e.what());
    return 1;
  }
  return 0;
}
