"""Independent pure-Python restatements used to pin the C oracle (tests only).

Written per row / per request from the reference's definitions, deliberately in a
different shape from oracle/fqa_oracle.c (dicts and per-row loops instead of scans), so a
shared mistake is unlikely:

  build_batch   Scheduler::BuildBatch (engine/src/scheduler.cc:116-143): the greedy loop
                over running requests stably sorted by Remaining().
  pack          EmitChunk rows (scheduler.h:66-72), PackBlockTables + SplitDecodePrefill
                (model_runtime.cu:54-91), slot = bt[p/16]*16 + p%16 (kv_store.cu:56-60),
                plus this library's decode/prefill plans as documented in include/fqa.h.
  argmax_kernel ArgmaxKernel (engine/src/kernels.cu:184-214) simulated thread by thread:
                its strided scans and its shared-memory tree, which fix the greedy tie
                order.
"""
from __future__ import annotations

PAGE = 16


def build_batch(num_tokens, computed, budget, chunk):
    order = sorted(range(len(num_tokens)), key=lambda i: (num_tokens[i] - computed[i], i))
    out = []
    for i in order:
        if budget <= 0:
            break
        rem = num_tokens[i] - computed[i]
        if rem <= 0:
            continue
        n = min(rem, budget)
        if rem > 1:
            n = min(n, chunk)
        out.append((i, n))
        budget -= n
    return out


def _cdiv(a, b):
    return -(-a // b)


def pack(computed, n_new, tables, *, max_rows, max_blocks, pool_pages, dec_grid_waves,
         dec_min_pages, dec_wave_cap, pre_tile_q, pre_item_cap, dec_share=0,
         dec_prefix_pages=0, dec_pre_cap=0, prefix_cap=8192):
    R = len(computed)
    meta = [0] * 16
    meta[8] = R
    codes = []
    rows_total = 0
    for c, n, t in zip(computed, n_new, tables):
        if c < 0 or n < 0:
            codes.append(5)
            continue
        if len(t) < _cdiv(c + n, PAGE):
            codes.append(1)
        elif len(t) > max_blocks:
            codes.append(2)
        rows_total += n
    if rows_total > max_rows:
        codes.append(3)
    if codes:
        meta[7] = min(codes)
        return {"meta": meta}

    res = {"positions": [], "row_req": [], "slot_mapping": [], "cu_seqlens": [],
           "qlen": list(n_new)}
    for r in range(R):
        res["cu_seqlens"].append(len(res["positions"]))
        for k in range(n_new[r]):
            p = computed[r] + k
            res["positions"].append(p)
            res["row_req"].append(r)
            res["slot_mapping"].append(tables[r][p // PAGE] * PAGE + p % PAGE)
    res["cu_seqlens"].append(len(res["positions"]))
    dec = [r for r in range(R) if n_new[r] == 1]
    pre = [r for r in range(R) if n_new[r] != 1]
    res["decode_rids"] = dec + [-1] * (R - len(dec))
    res["prefill_rids"] = pre + [-1] * (R - len(pre))
    bt = []
    bad = False
    for t in tables:
        row = list(t) + [-1] * (max_blocks - len(t))
        bad |= any(not (0 <= v < pool_pages) for v in t)
        bt.extend(row)
    res["block_tables"] = bt

    # shared prefixes: decode sequences grouped by their first page id (>= 0), led by the
    # first; a group's prefix is the shortest of its members' common runs of leading pages
    # with the leader (capped at prefix_cap, and at computed // 16 so that every member
    # keeps its last key's page), used when it reaches dec_prefix_pages
    groups = {}
    for di, r in enumerate(dec):
        if tables[r][0] >= 0:
            groups.setdefault(tables[r][0], []).append(di)
    prefix = [0] * len(dec)
    group_list = []  # (members, P), by leader
    if dec_prefix_pages > 0:
        for members in sorted(groups.values(), key=lambda m: m[0]):
            if len(members) < 2:
                continue
            lt = tables[dec[members[0]]]
            P = None
            for di in members:
                t = tables[dec[di]]
                pages = computed[dec[di]] // PAGE + 1
                common = 0
                for a, b in zip(t[:pages], lt[:computed[dec[members[0]]] // PAGE + 1]):
                    if a != b:
                        break
                    common += 1
                common = min(common, prefix_cap, computed[dec[di]] // PAGE)
                P = common if P is None else min(P, common)
            if P >= dec_prefix_pages:
                group_list.append((members, P))
        n_items = 0
        for members, P in group_list:
            cp = max(16, -(-P // 16))
            n_items += 8 * -(-P // cp) * -(-len(members) // 8)
        if n_items > dec_pre_cap:
            group_list = []
        for members, P in group_list:
            for di in members:
                prefix[di] = P
    # decode sequences whose first page starts another decode sequence too (group members
    # aside): FQA_DEC_SHARED (bit 30) in both n_keys fields, and a cheaper page cost
    from collections import Counter
    firsts = Counter(tables[r][0] for r in dec if tables[r][0] >= 0)
    shared = [tables[r][0] >= 0 and firsts[tables[r][0]] > 1 and not prefix[di]
              for di, r in enumerate(dec)]
    # ... priced cheaper unless the first (by decode index) to start at its page
    seen = set()
    cheap = []
    for di, r in enumerate(dec):
        cheap.append(shared[di] and tables[r][0] in seen)
        seen.add(tables[r][0])
    # decode stream-K plan: concatenate streams (di, kvh) over pages [prefix, pages), each
    # preceded by STREAM_COST start positions, a page taking PAGE_COST positions (5 in a
    # cheap one) and marked at its last one (None: a position that marks no page);
    # cut into G equal shares of positions, a share taking the pages marked in it
    PAGE_COST, SHARED_PAGE_COST = 8, 5
    STREAM_COST, PREFIX_STREAM_COST = 32, 16  # a member's stream always leaves a partial
    runs = []  # None or (di, kvh, page), for every cost position, in order
    seqs = []
    P = X = 0
    for di, r in enumerate(dec):
        pages = computed[r] // PAGE + 1
        u = SHARED_PAGE_COST if cheap[di] else PAGE_COST
        seqs.append([r, res["cu_seqlens"][r], computed[r] + 1, 8 * X])
        start = STREAM_COST + (PREFIX_STREAM_COST if prefix[di] else 0)
        for kvh in range(8):
            runs.extend([None] * start)
            for pg in range(prefix[di], pages):
                runs.extend([None] * (u - 1) + [(di, kvh, pg)])
        P += pages - prefix[di]
        X += (pages - prefix[di]) * u + start
    W = len(runs)
    G = min(dec_grid_waves, _cdiv(W, PAGE_COST * max(1, dec_min_pages))) if W else 0
    # dec_share: a decode beside the prefill gets a multiple of 32 wavefronts in
    # [32, N - 32]: the largest g whose modelled prefill time P N / (N - g) is no more than
    # the decode's D (36 g + 25 N) / (50 g), or g + 32 when the prefill there ends before
    # the decode at g; D = 783 x decode pages, P = prefill key-rows, halved together until
    # both fit 30 bits
    keyrows = sum(n_new[r] * computed[r] + n_new[r] * (n_new[r] + 1) // 2 for r in pre)
    N = dec_grid_waves
    if dec_share and W and keyrows and 64 <= N <= 4096:
        D, K = 783 * P, keyrows
        while D >= 1 << 30 or K >= 1 << 30:
            D, K = D >> 1, K >> 1
        top = (N - 32) // 32 * 32
        ok = [g for g in range(32, top + 1, 32)
              if 50 * K * N * g <= D * (36 * g + 25 * N) * (N - g)]
        g = max(ok) if ok else 32
        if g + 32 <= top and 50 * K * N * g < D * (36 * g + 25 * N) * (N - g - 32):
            g += 32
        G = min(G, g)
    waves = []
    for w in range(G):
        g0, g1 = w * W // G, (w + 1) * W // G
        # a share starts at the first page marked at or after its start
        di, kvh, pg = next(x for x in runs[g0:] if x is not None)
        r = dec[di]
        n = sum(x is not None for x in runs[g0:g1])
        waves.append([di, kvh, pg, n, r, res["cu_seqlens"][r], computed[r] + 1, tables[r][pg]])
    # prefill items: tiles sorted by key count descending, stable
    tiles = []
    for r in pre:
        q = n_new[r]
        for q0 in range(0, q, pre_tile_q):
            q1 = min(q0 + pre_tile_q, q)
            tiles.append([r, q0, q1, computed[r] + q1])
    items = sorted(tiles, key=lambda x: -x[3])  # Python's sort is stable
    if G > dec_wave_cap or len(items) > pre_item_cap:
        meta = [0] * 16
        meta[8], meta[7] = R, 6
        return {"meta": meta}
    for di, s in enumerate(seqs):
        s[2] |= (1 << 30) if shared[di] else 0
    for wv in waves:
        wv[6] |= (1 << 30) if shared[wv[0]] else 0
    res["dec_seqs"] = seqs
    res["dec_waves"] = waves
    res["pre_items"] = items
    # prefix items: per group (by leader), kv head, chunk of cp pages, octet of 8 members
    pitems, dpfx = [], [[0, 0, 0, 0] for _ in dec]
    for members, Pg in group_list:
        cp = max(16, -(-Pg // 16))
        nc, nq = -(-Pg // cp), -(-len(members) // 8)
        base = len(pitems)
        for k, di in enumerate(members):
            dpfx[di] = [Pg, base, nc | (nq << 16), k]
        padded = members + [-1] * (8 * nq - len(members))
        for kvh in range(8):
            for c in range(nc):
                for q in range(nq):
                    pitems.append([members[0], kvh, c * cp, min((c + 1) * cp, Pg)]
                                  + padded[8 * q:8 * q + 8])
    res["dec_prefix"] = dpfx
    res["dec_pre_items"] = pitems
    meta[10], meta[11], meta[12] = len(pitems), len(group_list), W
    meta[0] = rows_total
    meta[1], meta[2] = len(dec), len(pre)
    meta[3] = max([1] + [n_new[r] for r in pre])
    meta[4], meta[5] = G, len(items)
    meta[6] = _cdiv(W, G) if G else 0
    meta[7] = 4 if bad else 0
    meta[9] = P
    res["meta"] = meta
    return res


def argmax_kernel(row):
    """One row of ArgmaxKernel with its 256 threads: thread t keeps the first column of
    t, t+256, ... whose logit is strictly above its running best (start -1e30, column 0);
    then for s = 128, 64, .., 1 slot t < s takes slot t+s's pair when that value is
    strictly larger."""
    import numpy as np

    lg = np.asarray(row, np.float32)
    sval, sidx = [], []
    for t in range(256):
        best, bi = np.float32(-1e30), 0
        for i in range(t, len(lg), 256):
            if lg[i] > best:
                best, bi = lg[i], i
        sval.append(best)
        sidx.append(bi)
    s = 128
    while s > 0:
        for t in range(s):
            if sval[t + s] > sval[t]:
                sval[t], sidx[t] = sval[t + s], sidx[t + s]
        s >>= 1
    return sidx[0]
