// sched_cpp.cpp — drives include/fqa_sched.hpp through a scripted workload for
// tests/test_sched.py and prints one trace line per event, compared there against an
// independent Python model of the same scheduler.
//
// Input (whitespace-separated integers on stdin):
//   n_blocks n_slots token_budget prefill_chunk use_prefix_cache n_steps n_seqs
//   per sequence: id arrival_step cancel_step max_new max_ctx n_stop stop... n_prompt tok...
// cancel_step < 0: never.  The token sampled for sequence `id` at step t is
// (id * 7919 + t * 104729) % 50000 (both sides compute it).
// Output lines:
//   B t  <rows> <n_seqs> then per seq: id computed n_new n_blocks blocks...
//   S t  <n_sample> ids...
//   F t  free=<n> running=<ids...> waiting=<ids...>
//   R t  id finished error n_tokens     (retired this step)
#include <cstdio>
#include <iostream>
#include <map>
#include <vector>

#include "../../include/fqa_sched.hpp"

int main() {
  int n_blocks, n_slots, budget, chunk, use_cache, n_steps, n_seqs;
  if (!(std::cin >> n_blocks >> n_slots >> budget >> chunk >> use_cache >> n_steps >> n_seqs))
    return 2;
  struct Spec {
    int id, arrival, cancel, max_new, max_ctx;
    std::vector<int32_t> stop, prompt;
  };
  std::vector<Spec> specs(n_seqs);
  for (auto& s : specs) {
    int ns, np;
    std::cin >> s.id >> s.arrival >> s.cancel >> s.max_new >> s.max_ctx >> ns;
    s.stop.resize(ns);
    for (auto& x : s.stop) std::cin >> x;
    std::cin >> np;
    s.prompt.resize(np);
    for (auto& x : s.prompt) std::cin >> x;
  }
  fqa::BlockAllocator alloc(n_blocks);
  fqa::SchedConfig cfg{n_slots, budget, chunk, use_cache != 0};
  fqa::HostScheduler sched(alloc, cfg);
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
      std::printf("B %d %d %d", t, b.rows, (int)b.seqs.size());
      for (size_t i = 0; i < b.seqs.size(); ++i) {
        std::printf(" %d %d %d %d", b.seqs[i]->id, b.computed[i], b.n_new[i],
                    (int)b.block_tables[i].size());
        for (int x : b.block_tables[i]) std::printf(" %d", x);
      }
      std::printf("\n");
      std::vector<int32_t> sampled;
      std::printf("S %d %d", t, (int)b.sample_seqs.size());
      for (int si : b.sample_seqs) {
        const int id = b.seqs[si]->id;
        sampled.push_back((int32_t)(((long long)id * 7919 + (long long)t * 104729) % 50000));
        std::printf(" %d", id);
      }
      std::printf("\n");
      sched.Apply(b, sampled);
    }
    for (auto& r : sched.TakeRetired()) {
      std::printf("R %d %d %d %d %d\n", t, r->id, (int)r->finished, (int)r->error,
                  r->NumTokens());
      live.erase(r->id);
    }
    std::printf("F %d free=%d running=", t, alloc.NumFree());
    for (auto& r : sched.Running()) std::printf("%d,", r->id);
    std::printf(" waiting=");
    for (auto& r : sched.Waiting()) std::printf("%d,", r->id);
    std::printf("\n");
  }
  return 0;
}
