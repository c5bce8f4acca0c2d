"""Independent Python model of the engine's block allocator and scheduler (engine/src/
block_allocator.h:21-103, scheduler.cc:16-154, scheduler.h:57-98), with the one
documented difference of include/fqa_sched.hpp: a preemption rebuilds the batch from
scratch.  Plain lists and dicts, written from the reference's behaviour rather than from
the C++ header: the LRU free list is a Python list (append = most recently freed, pop(0)
= least), the prefix cache a dict.  Used by tests/test_sched.py to check the C++ trace."""
from __future__ import annotations

BLOCK = 16
MASK64 = (1 << 64) - 1


def hash_block(parent: int, tokens: list[int], start: int, n: int) -> int:
    """scheduler.cc:16-24: FNV-style multiply with a 27-bit rotate, seeded by the parent."""
    h = parent ^ 0x9E3779B97F4A7C15
    for i in range(n):
        h ^= tokens[start + i] & 0xFFFFFFFF
        h = (h * 0x100000001B3) & MASK64
        h = ((h << 27) | (h >> 37)) & MASK64
    return h if h else 1


class Allocator:
    def __init__(self, n: int):
        self.n = n
        self.ref = [0] * n
        self.hash = [0] * n
        self.cached: dict[int, int] = {}
        self.free = list(range(n))

    def alloc_one(self):
        if not self.free:
            return None
        b = self.free.pop(0)
        if self.hash[b]:
            if self.cached.get(self.hash[b]) == b:
                del self.cached[self.hash[b]]
            self.hash[b] = 0
        self.ref[b] = 1
        return b

    def free_one(self, b: int):
        self.ref[b] -= 1
        if self.ref[b] == 0:
            self.free.append(b)

    def grow(self, table: list[int], num_tokens: int) -> bool:
        need = -(-num_tokens // BLOCK)
        while len(table) < need:
            b = self.alloc_one()
            if b is None:
                return False
            table.append(b)
        return True

    def release(self, table: list[int]):
        for b in table:
            self.free_one(b)
        table.clear()

    def lookup(self, h: int) -> int:
        b = self.cached.get(h)
        if b is None:
            return -1
        if self.ref[b] == 0:
            self.free.remove(b)
        self.ref[b] += 1
        return b

    def insert(self, b: int, h: int):
        if self.hash[b] or h in self.cached:
            return
        self.hash[b] = h
        self.cached[h] = b


class Seq:
    def __init__(self, sid, prompt, max_new, max_ctx, stop):
        self.id, self.tokens, self.prompt_len = sid, list(prompt), len(prompt)
        self.max_new, self.max_ctx, self.stop = max_new, max_ctx, list(stop)
        self.blocks: list[int] = []
        self.computed = self.num_new = self.cached_blocks = 0
        self.last_hash = 0
        self.finished = self.error = self.cancelled = False

    def remaining(self):
        return len(self.tokens) - self.computed


class Scheduler:
    def __init__(self, alloc: Allocator, n_slots, budget, chunk, use_cache, selection_check=None):
        self.a, self.n_slots, self.budget, self.chunk, self.use_cache = (
            alloc, n_slots, budget, chunk, use_cache)
        self.waiting: list[Seq] = []
        self.running: list[Seq] = []
        self.retired: list[Seq] = []
        self.selection_check = selection_check  # called with (running, picked) when no preemption

    def _acquire_prefix(self, s: Seq):
        if not self.use_cache:
            return
        limit = (len(s.tokens) - 1) // BLOCK
        parent, nb = 0, 0
        while nb < limit:
            h = hash_block(parent, s.tokens, nb * BLOCK, BLOCK)
            b = self.a.lookup(h)
            if b < 0:
                break
            s.blocks.append(b)
            parent = h
            nb += 1
        if nb:
            s.computed, s.cached_blocks, s.last_hash = nb * BLOCK, nb, parent

    def _retire(self, s: Seq):
        self.a.release(s.blocks)
        self.running.remove(s)
        self.retired.append(s)

    def refill(self):
        for q in (self.waiting, self.running):
            for s in [x for x in q if x.cancelled]:
                self.a.release(s.blocks)
                q.remove(s)
                self.retired.append(s)
        while len(self.running) < self.n_slots and self.waiting:
            s = self.waiting.pop(0)
            if not s.blocks:
                self._acquire_prefix(s)
            self.running.append(s)

    def build(self):
        while True:
            order = sorted(range(len(self.running)), key=lambda i: self.running[i].remaining())
            seqs = [self.running[i] for i in order]
            snapshot = [(s.id, len(s.tokens), s.computed) for s in self.running]
            batch, budget, rebuild = [], self.budget, False
            for s in seqs:
                if budget <= 0:
                    break
                rem = s.remaining()
                if rem <= 0:
                    continue
                n = min(rem, budget)
                if rem > 1:
                    n = min(n, self.chunk)
                ok, preempted = self._grow(s, s.computed + n)
                if not ok or preempted:
                    rebuild = True
                    break
                batch.append((s, s.computed, n, list(s.blocks)))
                s.num_new = n
                budget -= n
            if not rebuild:
                if self.selection_check:
                    self.selection_check(snapshot, [(s.id, n) for s, _, n, _ in batch])
                return batch

    def _grow(self, s: Seq, upto: int):
        preempted = False
        while not self.a.grow(s.blocks, upto):
            victims = [x for x in self.running if x is not s]
            if not victims:
                s.error = True
                self._retire(s)
                return False, preempted
            v = victims[-1]
            self.a.release(v.blocks)
            v.computed = v.cached_blocks = v.last_hash = 0
            self.running.remove(v)
            self.waiting.insert(0, v)
            preempted = True
        return True, preempted

    def apply(self, batch, sampled: dict[int, int]):
        for s, _, _, _ in batch:
            s.computed += s.num_new
        for s, _, _, _ in batch:
            if s.remaining() == 0 and s.id in sampled:
                t = sampled[s.id]
                s.tokens.append(t)
                if (len(s.tokens) - s.prompt_len >= s.max_new or t in s.stop
                        or len(s.tokens) >= s.max_ctx):
                    s.finished = True
        if self.use_cache:
            for s, _, _, _ in batch:
                full = s.computed // BLOCK
                parent = s.last_hash
                for i in range(s.cached_blocks, full):
                    parent = hash_block(parent, s.tokens, i * BLOCK, BLOCK)
                    self.a.insert(s.blocks[i], parent)
                s.cached_blocks, s.last_hash = full, parent
        for s, _, _, _ in batch:
            if s.finished:
                self._retire(s)


def sampled_token(sid: int, t: int) -> int:
    return (sid * 7919 + t * 104729) % 50000


def run_trace(n_blocks, n_slots, budget, chunk, use_cache, n_steps, specs, selection_check=None):
    """The trace sched_cpp prints for the same script (see tests/cpp/sched_cpp.cpp)."""
    a = Allocator(n_blocks)
    sch = Scheduler(a, n_slots, budget, chunk, use_cache, selection_check)
    live: dict[int, Seq] = {}
    out = []
    for t in range(n_steps):
        for sp in specs:
            if sp["arrival"] == t:
                s = Seq(sp["id"], sp["prompt"], sp["max_new"], sp["max_ctx"], sp["stop"])
                live[s.id] = s
                sch.waiting.append(s)
            if sp["cancel"] == t and sp["id"] in live:
                live[sp["id"]].cancelled = True
        sch.refill()
        batch = sch.build()
        if batch:
            rows = sum(n for _, _, n, _ in batch)
            line = f"B {t} {rows} {len(batch)}"
            for s, c, n, bl in batch:
                line += f" {s.id} {c} {n} {len(bl)}" + "".join(f" {x}" for x in bl)
            out.append(line)
            smp = [s for s, c, n, _ in batch if c + n == len(s.tokens)]
            out.append(f"S {t} {len(smp)}" + "".join(f" {s.id}" for s in smp))
            sch.apply(batch, {s.id: sampled_token(s.id, t) for s in smp})
        for s in sch.retired:
            out.append(f"R {t} {s.id} {int(s.finished)} {int(s.error)} {len(s.tokens)}")
            live.pop(s.id, None)
        sch.retired = []
        out.append(f"F {t} free={len(a.free)} running=" + "".join(f"{s.id}," for s in sch.running)
                   + " waiting=" + "".join(f"{s.id}," for s in sch.waiting))
    return out
