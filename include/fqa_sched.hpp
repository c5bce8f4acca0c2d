// fqa_sched.hpp — host-side producer of the attention path's batches: the engine's paged
// KV block allocator and its continuous-batching scheduler, restated in C++ so that live
// request state (not synthetic tables) feeds fqa_pack.  Header-only, no HIP dependency.
//
// Reference it mirrors (engine/src/):
//   BlockAllocator (refcounted LRU free list + prefix cache)   block_allocator.h:21-103
//   HashBlock (block content hash chain)                       scheduler.cc:16-24
//   Scheduler::AcquirePrefix / CacheBlocks                     scheduler.cc:26-57
//   Scheduler::Grow (preempt the youngest running request)     scheduler.cc:74-98
//   Scheduler::Refill / BuildBatch / Step's bookkeeping        scheduler.cc:100-154
//   Request::EmitChunk / Advance / AcceptSampled               scheduler.h:57-98
//
// One step:  sched.Refill();  sched.BuildBatch(&batch);  <fqa_pack + layers on batch>;
//            sched.Apply(batch, sampled_tokens);
// `batch.computed / n_new / block_tables` are exactly fqa::BatchInput's fields
// (include/fqa_step.hpp), so `fqa::StepContext::PrepareInputs` takes them as they are.
//
// Differences from the reference (deliberate):
//  * After a preemption the batch is rebuilt from scratch.  The reference keeps
//    building, so a request preempted after it was already emitted into the batch would
//    run with freed blocks (scheduler.cc:131-140 with :85-96).
//  * Requests carry no output sink: cancellation is a flag, and over-capacity retirement
//    is reported through Sequence::error instead of a sink callback.
#pragma once

#include <algorithm>
#include <cstdint>
#include <deque>
#include <memory>
#include <numeric>
#include <unordered_map>
#include <vector>

namespace fqa {

constexpr int kSchedBlockTokens = 16;  // tokens per KV page (FQA_PAGE_TOKENS)

// Refcounted block ids [0, num_blocks) with an LRU list of the free ones.  A free block
// keeps its content hash, so CacheLookup can take it back (a prefix-cache hit) until
// AllocOne hands it out again and drops the hash.  The LRU list is intrusive (prev/next
// arrays over block ids): every operation is O(1) and allocation-free.
class BlockAllocator {
 public:
  explicit BlockAllocator(int num_blocks)
      : n_(num_blocks), ref_(num_blocks, 0), hash_(num_blocks, 0), prev_(num_blocks + 1),
        next_(num_blocks + 1), in_free_(num_blocks, 1) {
    // node n_ is the list head; blocks start free in id order
    int last = n_;
    for (int b = 0; b < n_; ++b) {
      next_[last] = b;
      prev_[b] = last;
      last = b;
    }
    next_[last] = n_;
    prev_[n_] = last;
    n_free_ = n_;
  }

  int NumBlocks() const { return n_; }
  int NumFree() const { return n_free_; }
  int RefCount(int b) const { return ref_[b]; }
  static int BlocksFor(int n_tok) { return (n_tok + kSchedBlockTokens - 1) / kSchedBlockTokens; }

  // Pop the least recently freed block; its cached hash (if any) is forgotten.
  bool AllocOne(int& out) {
    if (n_free_ == 0) return false;
    const int b = next_[n_];
    Unlink(b);
    if (hash_[b]) {
      auto it = cached_.find(hash_[b]);
      if (it != cached_.end() && it->second == b) cached_.erase(it);
      hash_[b] = 0;
    }
    ref_[b] = 1;
    out = b;
    return true;
  }
  void FreeOne(int b) {
    if (--ref_[b] == 0) PushBack(b);
  }
  // Grow a block table to cover num_tokens; false as soon as the pool is dry (the
  // blocks taken so far stay in the table).
  bool Grow(std::vector<int32_t>& table, int num_tokens) {
    const int need = BlocksFor(num_tokens);
    while ((int)table.size() < need) {
      int b;
      if (!AllocOne(b)) return false;
      table.push_back(b);
    }
    return true;
  }
  void Free(std::vector<int32_t>& table) {
    for (int b : table) FreeOne(b);
    table.clear();
  }
  // A block holding the content `hash`, referenced once more (taken off the free list if
  // it was free), or -1.
  int CacheLookup(uint64_t hash) {
    auto it = cached_.find(hash);
    if (it == cached_.end()) return -1;
    const int b = it->second;
    if (ref_[b] == 0) Unlink(b);
    ++ref_[b];
    return b;
  }
  // Record that block b holds `hash` (first writer wins, a block keeps its first hash).
  void CacheInsert(int b, uint64_t hash) {
    if (hash_[b] || cached_.count(hash)) return;
    hash_[b] = hash;
    cached_[hash] = b;
  }
  // Free blocks, least recently freed first (for tests).
  std::vector<int> FreeOrder() const {
    std::vector<int> v;
    for (int b = next_[n_]; b != n_; b = next_[b]) v.push_back(b);
    return v;
  }

 private:
  void Unlink(int b) {
    next_[prev_[b]] = next_[b];
    prev_[next_[b]] = prev_[b];
    in_free_[b] = 0;
    --n_free_;
  }
  void PushBack(int b) {
    const int last = prev_[n_];
    next_[last] = b;
    prev_[b] = last;
    next_[b] = n_;
    prev_[n_] = b;
    in_free_[b] = 1;
    ++n_free_;
  }

  int n_, n_free_ = 0;
  std::vector<int> ref_;
  std::vector<uint64_t> hash_;
  std::vector<int> prev_, next_;
  std::vector<unsigned char> in_free_;
  std::unordered_map<uint64_t, int> cached_;
};

// Content hash of tokens [start, start+n) chained onto the parent block's hash; never 0
// (0 marks "no hash").  The constants and steps are the reference's (scheduler.cc:16-24):
// hashes must agree for cached prefixes to be found.
inline uint64_t HashBlock(uint64_t parent, const std::vector<int32_t>& tokens, int start,
                          int n) {
  uint64_t h = parent ^ 0x9E3779B97F4A7C15ull;
  for (int i = 0; i < n; ++i) {
    h ^= (uint64_t)(uint32_t)tokens[start + i];
    h *= 0x100000001B3ull;
    h = (h << 27) | (h >> 37);
  }
  return h ? h : 1;
}

// One request's generation state (the reference's Request minus its output sink).
struct Sequence {
  int id = 0;                       // caller's handle
  std::vector<int32_t> tokens;      // prompt, then generated tokens
  int prompt_len = 0;
  int max_new = 0;                  // generate at most this many tokens
  int max_ctx = 0;                  // ... and stop when the context reaches this
  std::vector<int32_t> stop_ids;
  bool cancelled = false;           // set by the caller; dropped at the next Refill

  std::vector<int32_t> blocks;      // KV block table
  int computed = 0;                 // tokens whose K/V are in the cache
  int num_new = 0;                  // rows in the current step
  int cached_blocks = 0;            // leading blocks already recorded in the prefix cache
  uint64_t last_hash = 0;           // hash of block cached_blocks - 1
  bool finished = false;
  bool error = false;               // retired: a single sequence exceeds the pool

  int NumTokens() const { return (int)tokens.size(); }
  int Remaining() const { return NumTokens() - computed; }
  int Generated() const { return NumTokens() - prompt_len; }
};

struct SchedConfig {
  int n_slots = 64;          // running sequences at most
  int token_budget = 1024;   // rows per step
  int prefill_chunk = 512;   // rows per step for one sequence with more than one to go
  bool use_prefix_cache = true;
};

// One step's batch in batch order: what fqa::BatchInput takes (computed, n_new,
// block_tables), plus the rows' tokens and which requests sample a token.
struct SchedBatch {
  std::vector<Sequence*> seqs;
  std::vector<int32_t> computed, n_new;
  std::vector<std::vector<int32_t>> block_tables;
  std::vector<int32_t> tokens;        // all rows, batch order
  std::vector<int32_t> sample_rows;   // row index of each sampling request's last row
  std::vector<int32_t> sample_seqs;   // batch index of each sampling request
  int rows = 0;
  void Clear() {
    seqs.clear();
    computed.clear();
    n_new.clear();
    block_tables.clear();
    tokens.clear();
    sample_rows.clear();
    sample_seqs.clear();
    rows = 0;
  }
  bool Empty() const { return seqs.empty(); }
};

class HostScheduler {
 public:
  HostScheduler(BlockAllocator& alloc, const SchedConfig& cfg) : alloc_(alloc), cfg_(cfg) {}

  void Submit(std::unique_ptr<Sequence> s) { waiting_.push_back(std::move(s)); }
  bool Busy() const { return !waiting_.empty() || !running_.empty(); }
  const std::vector<std::unique_ptr<Sequence>>& Running() const { return running_; }
  const std::deque<std::unique_ptr<Sequence>>& Waiting() const { return waiting_; }
  // Sequences retired since the last call (finished, cancelled or over capacity).
  std::vector<std::unique_ptr<Sequence>> TakeRetired() { return std::move(retired_); }

  // Drop cancelled sequences; admit waiting ones into free slots, adopting any cached
  // prefix of a sequence that holds no blocks (scheduler.cc:100-117).
  void Refill() {
    DropCancelled(waiting_);
    DropCancelled(running_);
    while ((int)running_.size() < cfg_.n_slots && !waiting_.empty()) {
      if (waiting_.front()->blocks.empty()) AcquirePrefix(waiting_.front().get());
      running_.push_back(std::move(waiting_.front()));
      waiting_.pop_front();
    }
  }

  // The unified token budget (scheduler.cc:119-143): running sequences in stable order of
  // rows still to compute, each taking min(remaining, budget) rows, capped at
  // prefill_chunk when more than one row remains; blocks grown on the way, preempting
  // the youngest other running sequence whenever the pool is dry.
  bool BuildBatch(SchedBatch& batch) {
    for (bool restart = true; restart;) {
      restart = false;
      batch.Clear();
      std::vector<int> order(running_.size());
      std::iota(order.begin(), order.end(), 0);
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        return running_[a]->Remaining() < running_[b]->Remaining();
      });
      std::vector<Sequence*> ordered;
      for (int i : order) ordered.push_back(running_[i].get());
      int budget = cfg_.token_budget;
      for (Sequence* s : ordered) {
        if (budget <= 0) break;
        const int rem = s->Remaining();
        if (rem <= 0) continue;
        int n = std::min(rem, budget);
        if (rem > 1) n = std::min(n, cfg_.prefill_chunk);
        const GrowResult g = Grow(s, s->computed + n);
        if (g != GrowResult::kOk) {  // s retired, or another sequence preempted: rebuild
          restart = true;
          break;
        }
        Emit(batch, s, n);
        budget -= n;
      }
    }
    return !batch.Empty();
  }

  // After the forward: advance every batch sequence by its rows, hand each sampling
  // sequence its token (sampled[i] for batch.sample_seqs[i]), record full blocks in the
  // prefix cache, and retire finished sequences (scheduler.cc:146-154, scheduler.h:76-98).
  void Apply(const SchedBatch& batch, const std::vector<int32_t>& sampled) {
    for (Sequence* s : batch.seqs) s->computed += s->num_new;
    for (size_t i = 0; i < batch.sample_seqs.size(); ++i) {
      Sequence* s = batch.seqs[batch.sample_seqs[i]];
      if (s->Remaining() != 0) continue;
      s->tokens.push_back(sampled[i]);
      const bool stop = std::find(s->stop_ids.begin(), s->stop_ids.end(), sampled[i]) !=
                        s->stop_ids.end();
      if (s->Generated() >= s->max_new || stop || s->NumTokens() >= s->max_ctx)
        s->finished = true;
    }
    if (cfg_.use_prefix_cache)
      for (Sequence* s : batch.seqs) CacheBlocks(s);
    for (Sequence* s : batch.seqs)
      if (s->finished) Retire(s);
  }

 private:
  enum class GrowResult { kOk, kPreempted, kRetired };

  void Emit(SchedBatch& b, Sequence* s, int n) {
    const int bi = (int)b.seqs.size();
    b.seqs.push_back(s);
    b.computed.push_back(s->computed);
    b.n_new.push_back(n);
    b.block_tables.push_back(s->blocks);
    for (int k = 0; k < n; ++k) b.tokens.push_back(s->tokens[s->computed + k]);
    b.rows += n;
    if (s->computed + n == s->NumTokens()) {
      b.sample_rows.push_back(b.rows - 1);
      b.sample_seqs.push_back(bi);
    }
    s->num_new = n;
  }

  // scheduler.cc:74-98: grow s's table to cover `upto` tokens; while the pool is dry,
  // preempt the youngest running sequence other than s (blocks freed, recomputed from
  // scratch on resume, back at the front of the waiting queue).  With no other sequence
  // left, s itself is retired with an error.
  GrowResult Grow(Sequence* s, int upto) {
    bool preempted = false;
    while (!alloc_.Grow(s->blocks, upto)) {
      int k = (int)running_.size() - 1;
      while (k >= 0 && running_[k].get() == s) --k;
      if (k < 0) {
        s->error = true;
        Retire(s);
        return GrowResult::kRetired;
      }
      Sequence* v = running_[k].get();
      alloc_.Free(v->blocks);
      v->computed = 0;
      v->cached_blocks = 0;
      v->last_hash = 0;
      waiting_.push_front(std::move(running_[k]));
      running_.erase(running_.begin() + k);
      preempted = true;
    }
    return preempted ? GrowResult::kPreempted : GrowResult::kOk;
  }

  // scheduler.cc:26-43: take the longest cached run of leading full blocks (never the
  // block holding the last prompt token, which must be computed to sample from).
  void AcquirePrefix(Sequence* s) {
    if (!cfg_.use_prefix_cache) return;
    const int limit = (s->NumTokens() - 1) / kSchedBlockTokens;
    uint64_t parent = 0;
    int nb = 0;
    for (; nb < limit; ++nb) {
      const uint64_t h = HashBlock(parent, s->tokens, nb * kSchedBlockTokens, kSchedBlockTokens);
      const int b = alloc_.CacheLookup(h);
      if (b < 0) break;
      s->blocks.push_back(b);
      parent = h;
    }
    if (nb > 0) {
      s->computed = nb * kSchedBlockTokens;
      s->cached_blocks = nb;
      s->last_hash = parent;
    }
  }

  // scheduler.cc:45-57: record the full blocks computed so far.
  void CacheBlocks(Sequence* s) {
    const int full = s->computed / kSchedBlockTokens;
    uint64_t parent = s->last_hash;
    for (int i = s->cached_blocks; i < full; ++i) {
      parent = HashBlock(parent, s->tokens, i * kSchedBlockTokens, kSchedBlockTokens);
      alloc_.CacheInsert(s->blocks[i], parent);
    }
    s->cached_blocks = full;
    s->last_hash = parent;
  }

  void Retire(Sequence* s) {
    alloc_.Free(s->blocks);
    for (auto it = running_.begin(); it != running_.end(); ++it)
      if (it->get() == s) {
        retired_.push_back(std::move(*it));
        running_.erase(it);
        return;
      }
  }

  template <class Q>
  void DropCancelled(Q& q) {
    for (auto it = q.begin(); it != q.end();) {
      if ((*it)->cancelled) {
        alloc_.Free((*it)->blocks);
        retired_.push_back(std::move(*it));
        it = q.erase(it);
      } else {
        ++it;
      }
    }
  }

  BlockAllocator& alloc_;
  const SchedConfig cfg_;
  std::deque<std::unique_ptr<Sequence>> waiting_;
  std::vector<std::unique_ptr<Sequence>> running_;
  std::vector<std::unique_ptr<Sequence>> retired_;
};

}  // namespace fqa
