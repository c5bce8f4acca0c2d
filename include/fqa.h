/*
 * fqa.h — C ABI of the MI355X (gfx950) per-step attention path.
 *
 * The path replaces, one for one, the attention block of the reference engine's
 * forward step (engine/src/model_runtime.cu:261-278 per layer, and the host pack
 * StepContext::PrepareInputs at model_runtime.cu:295-302 once per step):
 *
 *   fqa_schedule            <- Scheduler::BuildBatch token-budget selection   (scheduler.cc:116-143)
 *   fqa_schedule_gather     <- the same selection + the chosen requests' batch, one launch
 *   fqa_pack                <- StepContext::PrepareInputs: UploadRows, PackBlockTables,
 *                              SplitDecodePrefill                             (model_runtime.cu:47-91, 295-302)
 *   fqa_rope_tables         <- RopeTables::Build                              (model_runtime.cu:111-126)
 *   fqa_qknorm_rope_append  <- LaunchHeadNormRope + KvStore::StoreKV          (kernels.cu:97-139, kv_store.cu:48-75)
 *   fqa_qknorm_rope         <- LaunchHeadNormRope alone                       (kernels.cu:97-139)
 *   fqa_store_kv            <- KvStore::StoreKV alone                         (kv_store.cu:48-75)
 *   fqa_decode              <- LaunchAttnDecodeCute (split + combine)         (attn_cute.cu:165-261)
 *   fqa_prefill             <- LaunchAttnPrefillCute                          (attn_cute.cu:30-163)
 *   fqa_pool_bytes, fqa_pool_pages(_device)
 *                           <- KvStore pool sizing                            (kv_store.cu:10-46)
 *   fqa_sample              <- LaunchSampleBatch (greedy / temperature + top-p) (kernels.cu:184-327)
 *   fqa_gemm                <- LaunchGemm (QKV, o_proj, gate-up, down, lm_head) (kernels.cu:9-16)
 *   fqa_qkv_proj_append     <- LaunchGemm(QKV) + LaunchHeadNormRope + StoreKV (model_runtime.cu:261-268)
 *   fqa_gemm_argmax         <- LaunchGemm(lm_head) + ArgmaxKernel, greedy rows (model_runtime.cu:322-325)
 *
 * Conventions (all entry points):
 *   - Plain device pointers and sizes; every launch goes on the caller's hipStream_t
 *     (passed as void*, NULL = default stream). Nothing allocates; nothing synchronises.
 *   - Return 0 on success, a negative FQA_E* code for a rejected call (no kernel is
 *     launched then), never exit().  The reference aborts on these (assert / CUDA_CHECK,
 *     attn_cute.cu:156,248, cuda_helpers.h:15-23).
 *   - Counts that only the device knows after fqa_pack (rows, decode/prefill lists, work
 *     items) are read by the later kernels from the pack's `meta` array, so a whole step
 *     is stream-ordered with no host round trip; the host passes only upper bounds for
 *     grid sizing.  A launch is therefore capture-safe (no hipMemset, no host sync).
 *
 * Supported shape: Qwen3-8B attention (32 q heads, 8 kv heads, head_dim 128, 16-token
 * pages, GQA group 4), the only shape the reference kernels accept (attn_cute.cu:248).
 *
 * KV pool layout (one array per layer, bf16):
 *   page p, kv head h occupies one contiguous 8 KiB run at element offset
 *       ((p * n_kv_heads + h) * 2) * 16 * 128
 *   holding K as [16 tokens][128 dims] followed by V transposed as [128 dims][16 tokens].
 *   Slot s = page * 16 + token-in-page, as in the reference (kv_store.cu:56-60).
 *   All pool offsets are 64-bit: one layer of a 200 GB pool exceeds 2^31 elements.
 */
#ifndef FQA_H_
#define FQA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FQA_OK 0
#define FQA_EINVAL (-1)       /* null pointer, negative size, size over a stated maximum */
#define FQA_EUNSUPPORTED (-2) /* shape other than 32/8/128/16 */
#define FQA_ELAUNCH (-3)      /* hipGetLastError() after a launch */
#define FQA_ENOSPACE (-4)     /* fqa_pool_pages: the pool cannot hold one max_ctx sequence */

/* Query rows per prefill work item that the step helpers (fqa_step.hpp, fqa_compat.hpp,
 * flashqwen_amd.step) plan with. */
#define FQA_PRE_TILE_Q 64

#define FQA_PAGE_TOKENS 16
/* Flag in the n_keys field of dec_seqs and dec_waves (fqa_pack_out): the decode
 * sequence's first page is also the first page of another decode sequence in the batch
 * (a shared prefix).  The decode reads such a sequence's pages through the caches and
 * every other sequence's with non-temporal loads, which do not displace the shared pages.
 * n_keys = field & FQA_DEC_KEYS_MASK. */
#define FQA_DEC_SHARED (1 << 30)
#define FQA_DEC_KEYS_MASK (FQA_DEC_SHARED - 1)
#define FQA_MAX_REQS 2048 /* max requests in one step (reference: `slots`, args.h:13) */
/* Costs in the decode plan's stream-K cut, in cost units.  A page run costs
 * FQA_DEC_PAGE_COST, or FQA_DEC_SHARED_PAGE_COST in a "cheap" sequence: one flagged
 * FQA_DEC_SHARED that is not the first decode sequence (by decode index) with its first
 * page (the first one's reads bring the shared pages into the caches; the others' pages
 * then stream ~1.5x faster, measured on config 5). */
#define FQA_DEC_PAGE_COST 8
#define FQA_DEC_SHARED_PAGE_COST 5
/* Cost of starting a decode stream: each (sequence, kv head) stream counts its pages plus
 * this, so a wavefront whose share holds many short streams gets fewer pages (a stream
 * start costs a few dependent loads; 4 page runs). */
#define FQA_DEC_STREAM_COST 32
/* ... and this more for a shared-prefix member's stream (dec_prefix_pages): such a stream
 * always leaves a partial for the combine (config 5: 0, 16 and 32 measured 669, 668 and
 * 670.6 us). */
#define FQA_DEC_PREFIX_STREAM_COST 16
/* Pages of a decode sequence compared with its group leader's for a shared prefix
 * (fqa_pack_cfg::dec_prefix_pages). */
#define FQA_DEC_PREFIX_CAP 8192

/* Indices into the int32 `meta` array written by fqa_pack. */
enum {
  FQA_META_ROWS = 0,         /* T: query rows in the step                      */
  FQA_META_N_DECODE = 1,     /* requests with qlen == 1                        */
  FQA_META_N_PREFILL = 2,    /* requests with qlen != 1                        */
  FQA_META_MAX_QLEN = 3,     /* max(1, max prefill qlen) (model_runtime.cu:82) */
  FQA_META_DEC_WAVES = 4,    /* decode wavefronts with work this step         */
  FQA_META_PRE_ITEMS = 5,    /* prefill work items (request, query tile)      */
  FQA_META_DEC_WAVE_PAGES = 6, /* cost units of a decode share (ceil(W / G))       */
  FQA_META_STATUS = 7,       /* 0 or an FQA_PACK_* code                       */
  FQA_META_REQS = 8,         /* R                                             */
  FQA_META_DEC_PAGES = 9,    /* sum over decode sequences of their stream pages */
  FQA_META_DEC_PRE_ITEMS = 10, /* shared-prefix items (dec_prefix_pages)        */
  FQA_META_DEC_GROUPS = 11,  /* shared-prefix groups                            */
  FQA_META_DEC_COST = 12,    /* W: the decode plan's cost positions              */
  FQA_META_LEN = 16
};

/* Pack status codes (meta[FQA_META_STATUS]). On 1..3 and 5 every count is zeroed, so
 * the later kernels of the step do no work. On 4 counts stand; the attention and append
 * kernels skip any page id outside [0, pool_pages). */
enum {
  FQA_PACK_OK = 0,
  FQA_PACK_SHORT_TABLE = 1, /* block table shorter than ceil((computed+n)/16)   */
  FQA_PACK_WIDE_TABLE = 2,  /* block table longer than max_blocks               */
  FQA_PACK_ROWS = 3,        /* sum of n over requests > max_rows                */
  FQA_PACK_PAGE_RANGE = 4,  /* a page id outside [0, pool_pages)                */
  FQA_PACK_NEGATIVE = 5,    /* negative computed or n                           */
  FQA_PACK_ITEMS = 6        /* prefill items or decode waves exceed capacity    */
};

typedef struct fqa_dims {
  int32_t n_q_heads;  /* 32                                    */
  int32_t n_kv_heads; /* 8                                     */
  int32_t head_dim;   /* 128                                   */
  int32_t page_size;  /* 16                                    */
  int32_t qkv_stride; /* row stride of qkv in elements (6144)  */
  float eps;          /* RMSNorm epsilon (1e-6)                */
  float scale;        /* softmax scale 1/sqrt(head_dim)        */
} fqa_dims;

/* The ragged batch of one step, in batch order (what Scheduler::BuildBatch hands to
 * Forward through ForwardInput, scheduler.h:66-72): request r contributes rows
 * (pos = computed[r] + k, k < n_new[r]) and owns pages bt_pages[bt_off[r] .. bt_off[r+1]).
 * All arrays are device arrays.  If `n_reqs_dev` is non-NULL the request count is read
 * from it on the device (fqa_schedule's output) and `n_reqs` is only an upper bound. */
typedef struct fqa_batch {
  const int32_t* computed; /* [R] tokens already in the KV cache          */
  const int32_t* n_new;    /* [R] rows this step                          */
  const int32_t* bt_off;   /* [R+1] offsets into bt_pages                 */
  const int32_t* bt_pages; /* concatenated block tables (page ids)        */
  const int32_t* n_reqs_dev;
  int32_t n_reqs;
} fqa_batch;

/* Everything the pack writes (device arrays, caller-allocated at capacity).
 *
 * Decode plan (stream-K): the decode requests' (sequence, kv head) page streams are laid
 * end to end in cost units, stream (di, kvh) of pages[di] pages costing
 * c = pages[di] * u + s, u = FQA_DEC_PAGE_COST (FQA_DEC_SHARED_PAGE_COST in a cheap
 * sequence, above), s = FQA_DEC_STREAM_COST (+ FQA_DEC_PREFIX_STREAM_COST for a
 * shared-prefix member): it spans [X[di]*8 + kvh*c, + c), where pages = ceil(n_keys/16)
 * and X is the exclusive prefix of the costs over decode indices; the first s positions
 * of a stream stand for its start, then page k takes positions [s + k*u, s + (k+1)*u).
 * The W = 8*sum(c) positions (meta[FQA_META_DEC_COST]) are cut into G =
 * min(dec_grid_waves, ceil(W / (FQA_DEC_PAGE_COST * dec_min_pages))) equal contiguous
 * shares, share w = [floor(w*W/G), floor((w+1)*W/G)), one per decode wavefront (each at
 * least FQA_DEC_PAGE_COST positions), which streams the pages whose last position falls
 * in it; dec_waves[w] = {di, kvh, page, n_runs, r, row, n_keys, page id} is the stream
 * and page it starts at, how many pages it streams, the first stream's request, row and
 * key count, and its first page (so a wavefront's first loads need no further lookups).
 * dec_seqs[di] = {r, row = qstart[r], n_keys = computed[r]+1,
 * 8*X[di]}.  The n_keys fields of both carry FQA_DEC_SHARED.  Prefill plan: one item
 * per pre_tile_q query rows of each prefill request, pre_items[i] = {r, q0, q1,
 * n_keys = computed + q1}, ordered by n_keys descending (stable). */
typedef struct fqa_pack_out {
  int32_t* cu_seqlens;     /* [R+1]  qstart = cu_seqlens[r]                   */
  int32_t* qlen;           /* [R]                                             */
  int32_t* positions;      /* [max_rows]                                      */
  int32_t* row_req;        /* [max_rows] request index of each row            */
  int32_t* slot_mapping;   /* [max_rows] page*16 + pos%16                     */
  int32_t* block_tables;   /* [R * max_blocks], tail padded with -1           */
  int32_t* decode_rids;    /* [R] qlen==1 requests, increasing; pad -1        */
  int32_t* prefill_rids;   /* [R] the others, increasing; pad -1              */
  int32_t* dec_seqs;       /* [R][4] per decode index: {r, row, n_keys, 8*P}  */
  int32_t* dec_waves;      /* [dec_wave_cap][8] see the decode plan above     */
  int32_t* pre_items;      /* [pre_cap][4] {r, q0, q1, n_keys}                */
  int32_t* meta;           /* [FQA_META_LEN]                                  */
  /* with dec_prefix_pages (otherwise NULL): */
  int32_t* dec_prefix;     /* [R][8] per decode index {P, first item, C | Q << 16, k};
                              columns 4..7 are the pack's working space         */
  int32_t* dec_pre_items;  /* [dec_pre_cap][12] {leader di, kvh, page0, page1,
                              member di x 8 (-1 past the group)}                */
} fqa_pack_out;

typedef struct fqa_pack_cfg {
  int32_t max_rows;          /* capacity of the per-row arrays (<= 2^20)   */
  int32_t max_blocks;        /* block table stride (<= 2^19)               */
  int64_t pool_pages;        /* pages in the per-layer pool                */
  int32_t dec_grid_waves;    /* decode wavefronts to spread the work over (>= 1) */
  int32_t dec_min_pages;     /* give no wavefront fewer page runs than this   */
  int32_t dec_wave_cap;      /* capacity of dec_waves (>= dec_grid_waves)  */
  int32_t pre_tile_q;        /* query rows per prefill item: 32, 64 or 128 */
  int32_t pre_item_cap;      /* capacity of pre_items                      */
  int32_t dec_share;         /* nonzero: the decode runs beside the prefill (see below) */
  int32_t dec_prefix_pages;  /* >0: attend shared decode prefixes of at least this many
                                pages once per group (see below); 0: off            */
  int32_t dec_pre_cap;       /* capacity of dec_pre_items                    */
} fqa_pack_cfg;

/* dec_prefix_pages (shared-prefix decode): decode sequences whose first page id (>= 0)
 * is the same form a group, led by the first of them in decode order.  Each member's
 * common prefix with the leader (the longest run of equal leading page ids, at most
 * FQA_DEC_PREFIX_CAP pages; the leader's is its own page count) is capped at
 * computed / 16 pages (every member keeps the page of its last key); the group's prefix
 * P is the smallest over its members.  When P >= dec_prefix_pages, keys [0, 16 P) of
 * every member are attended once for the whole group: the group's M members in octets of
 * 8 (Q = ceil(M/8)), its P pages in C chunks of CP = max(16, ceil(P/16)) pages, one
 * prefix item per (kv head, chunk, octet), in that order, groups by leader:
 * dec_pre_items[i] = {leader, kvh, c*CP, min((c+1)*CP, P), the octet's member decode
 * indices}.  Member k of the group (by decode index) gets dec_prefix[di] = {P, the
 * group's first item, C | Q << 16, k} and its decode streams cover pages [P, pages) only
 * (the plan above with pages - P in place of pages, and dec_waves' page counted from the
 * sequence's first page, so from P on; the shared flag is not set on it).
 * If the groups need more than dec_pre_cap items, none is used.  Decode with
 * fqa_decode_prefix: fqa_decode does not read these arrays. */

/* dec_share: the caller runs the step's decode concurrently with its prefill (the decode
 * queued first on a second stream; fqa_step.hpp's RunLayer with a side stream, the
 * Python AttnStep with dec_share=True).  A decode workgroup holds a CU alone (its LDS
 * reservation), so when the batch has both decode and prefill rows the decode plan is
 * cut to fewer wavefronts and the prefill gets the other CUs.  With N = dec_grid_waves
 * (<= 4096; N = 4 x CUs is the device), the decode's time on G of the N wavefronts beside
 * the prefill is modelled as D (0.72 + 0.5 N/G) (it streams HBM: half the CUs still read
 * at ~2/3 of the rate, and the prefill beside it costs it ~22%) and the prefill's as
 * P N / (N - G) (it is MFMA-bound), with
 *   D = FQA_DEC_SHARE_RATE * decode pages,  P = prefill key-rows = sum n*c + n(n+1)/2
 * (FQA_DEC_SHARE_RATE: prefill key-rows per decode page at the two kernels' measured
 * rates on MI355X, ~78k key-rows and ~100 pages per microsecond; 0.72 and 0.5 fit the
 * decode alone and beside config 4's prefill at 512-1024 wavefronts).  G is a multiple of
 * 32 (one 4-wavefront workgroup per XCD, 8 XCDs, so every XCD keeps the same CUs for the
 * prefill) in [32, N - 32]: the largest Glo with prefill <= decode, i.e.
 * 50 P N Glo <= D (36 Glo + 25 N)(N - Glo), or Glo + 32 if the prefill there is shorter
 * than the decode at Glo (50 P N Glo < D (36 Glo + 25 N)(N - Glo - 32)); never more
 * than the plan without dec_share.  D and P are first shifted right together until both
 * fit 30 bits.  Zero: the plan as without it. */
#define FQA_DEC_SHARE_RATE 783
#define FQA_DEC_SHARE_STEP 32

/* --- host-side helpers (no device work) ------------------------------------------ */

/* cos/sin tables [max_pos][head_dim/2], float, angle = p * theta^(-2i/head_dim),
 * computed in float exactly as RopeTables::Build (model_runtime.cu:111-126). Host memory. */
int fqa_rope_tables(int32_t max_pos, int32_t head_dim, float theta, float* cos_tab,
                    float* sin_tab);

/* Bytes of one layer's pool for `pages` pages (replaces KvStore's per-block sizing,
 * kv_store.cu:24-26). */
int64_t fqa_pool_bytes(const fqa_dims* dims, int64_t pages);

/* Pages of a pool sized the way KvStore's constructor sizes it (kv_store.cu:10-33): the
 * bytes left of total_bytes * fraction (the product taken in float, as the reference's
 * `totalb * gpu_mem_fraction`) after used_bytes, in whole blocks of
 * layers x 2 x page_size x n_kv_heads x head_dim bf16 (one block = one page of every
 * layer).  *pages receives the count (capped at 2^31 - 1) in every case; the return is
 * FQA_ENOSPACE when it is below ceil(max_ctx / page_size) (the reference throws), FQA_OK
 * otherwise.  At Qwen3-8B's 36 layers one page costs 2.25 MiB, so a 288 GB device at
 * fraction 0.9 with 20 GB used holds ~101k pages (1.6M tokens).  Any positive finite
 * fraction is accepted, above 1 too, as the reference's constructor accepts it; FQA_EINVAL
 * for a fraction <= 0 or not finite. */
int fqa_pool_pages(const fqa_dims* dims, uint64_t total_bytes, uint64_t used_bytes,
                   float fraction, int32_t layers, int32_t max_ctx, int64_t* pages);

/* fqa_pool_pages with total and used bytes from the current device's hipMemGetInfo
 * (used = total - free), as the reference's constructor reads cudaMemGetInfo. */
int fqa_pool_pages_device(const fqa_dims* dims, float fraction, int32_t layers,
                          int32_t max_ctx, int64_t* pages);

/* Upper bounds for plan capacities and launch grids, from host-known sizes. */
int32_t fqa_dec_wave_bound(int32_t n_reqs, int32_t dec_grid_waves);

/* A decode grid that fills the device: CUs x 4, one decode wavefront per SIMD. */
int32_t fqa_dec_default_waves(int32_t device);
int32_t fqa_pre_item_bound(int32_t n_reqs, int32_t max_rows, int32_t pre_tile_q);

/* Bytes of the decode workspace fqa_decode needs for `dec_wave_cap` wavefronts. */
int64_t fqa_decode_workspace_bytes(const fqa_dims* dims, int32_t dec_wave_cap);

/* --- device entry points (stream-ordered launches) -------------------------------- */

/* Token-budget selection of Scheduler::BuildBatch (scheduler.cc:116-143) on the GPU:
 * stable-sorts the running requests by remaining = num_tokens - computed, then takes
 * n = min(remaining, budget left, prefill_chunk if remaining > 1) in that order.
 * Writes batch_req[R] (index into the running arrays), batch_n[R], and *n_batch (R).
 * Block tables must already cover each chosen request's computed + n tokens (the
 * allocator's Grow stays on the host). One workgroup; n_running <= FQA_MAX_REQS,
 * token_budget <= 2^24. */
int fqa_schedule(const int32_t* num_tokens, const int32_t* computed, int32_t n_running,
                 int32_t token_budget, int32_t prefill_chunk, int32_t* batch_req,
                 int32_t* batch_n, int32_t* n_batch, void* stream);

/* Gather the running requests chosen by fqa_schedule into a fqa_batch:
 * out_computed/out_n_new/out_bt_off[0..R] and out_bt_pages (concatenated tables).
 * run_bt_off/run_bt_pages are the running requests' tables. bt_pages_cap bounds
 * out_bt_pages; rows past it are dropped and flagged by status 1 in the pack. */
int fqa_gather_batch(const int32_t* batch_req, const int32_t* batch_n,
                     const int32_t* n_batch, int32_t n_running, const int32_t* run_computed,
                     const int32_t* run_bt_off, const int32_t* run_bt_pages,
                     int32_t* out_computed, int32_t* out_n_new, int32_t* out_bt_off,
                     int32_t* out_bt_pages, int32_t bt_pages_cap, void* stream);

/* fqa_schedule and fqa_gather_batch in one launch: every workgroup of the gather makes
 * the selection itself (the same in each), workgroup 0 writes it to batch_req / batch_n
 * / n_batch, and the chosen requests are gathered as fqa_gather_batch gathers them.
 * The same arguments and results as the two calls in turn. */
int fqa_schedule_gather(const int32_t* num_tokens, const int32_t* run_computed,
                        int32_t n_running, int32_t token_budget, int32_t prefill_chunk,
                        const int32_t* run_bt_off, const int32_t* run_bt_pages,
                        int32_t* batch_req, int32_t* batch_n, int32_t* n_batch,
                        int32_t* out_computed, int32_t* out_n_new, int32_t* out_bt_off,
                        int32_t* out_bt_pages, int32_t bt_pages_cap, void* stream);

/* The GPU pack (replaces StepContext::PrepareInputs' host loops + H2D copies,
 * model_runtime.cu:47-91): rows, slot mapping, padded block tables, decode/prefill
 * split by qlen, and the decode/prefill work plans. One launch. */
int fqa_pack(const fqa_batch* batch, const fqa_pack_cfg* cfg, const fqa_pack_out* out,
             void* stream);

/* Fused per-head QK-RMSNorm + rotate-half RoPE on the q and k heads of each row and the
 * paged append of k and v (replaces HeadNormRopeKernel + StoreKvKernel).  q is normalised
 * in place in `qkv` (the attention kernels read it from there, as in the reference);
 * k and v go to the pool at slot_mapping[t].  With `write_k_inplace` the normalised k is
 * also written back into qkv, leaving qkv bit-identical to the reference's.
 * Rows: meta[FQA_META_ROWS] (device) <= rows_bound (host, grid size).  The tables hold
 * rope_max_pos positions; a row whose position is outside [0, rope_max_pos) is left
 * untouched and appends nothing (the reference would read past its table). */
int fqa_qknorm_rope_append(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                           const float* k_norm_w, const float* cos_tab, const float* sin_tab,
                           int32_t rope_max_pos, const int32_t* positions, const int32_t* slot_mapping,
                           const int32_t* meta, int32_t rows_bound, uint16_t* pool,
                           int64_t pool_pages, int32_t write_k_inplace, void* stream);

/* The two halves of fqa_qknorm_rope_append as separate launches, for callers that keep the
 * reference's two calls (LaunchHeadNormRope, kernels.cu:133-139, decl. kernels.cuh:28-31;
 * KvStore::StoreKV, kv_store.cu:66-75, decl. kv_store.h:29-31).
 * fqa_qknorm_rope: the norm + RoPE of the q and k heads of each row, written back in place
 * into qkv (q and k, as the reference leaves them); nothing is appended.  Rows whose
 * position is outside [0, rope_max_pos) are left untouched.
 * fqa_store_kv: the paged append of each row's k and v exactly as they are in qkv (k
 * normalised by fqa_qknorm_rope before, as the reference's order has it) at
 * slot_mapping[t]; qkv is only read.  Rows with a negative position or a slot outside
 * the pool append nothing.  Running the two in this order leaves qkv and the pool exactly
 * as fqa_qknorm_rope_append with write_k_inplace = 1 does. */
int fqa_qknorm_rope(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                    const float* k_norm_w, const float* cos_tab, const float* sin_tab,
                    int32_t rope_max_pos, const int32_t* positions, const int32_t* meta,
                    int32_t rows_bound, void* stream);
int fqa_store_kv(const fqa_dims* dims, const uint16_t* qkv, const int32_t* positions,
                 const int32_t* slot_mapping, const int32_t* meta, int32_t rows_bound,
                 uint16_t* pool, int64_t pool_pages, void* stream);

/* GQA-shared split-K flash decoding over the pack's stream-K decode plan: wavefront w
 * streams its share of page runs; each (page, kv head) run is read once for all 4 query
 * heads of the kv head.  A stream that lies inside one share is finished by that
 * wavefront; a stream cut by share boundaries leaves fp32 partials (m, l, acc) that a
 * log-sum-exp combine merges.  Output rows out[row] ([n_q_heads][head_dim] bf16, row
 * stride n_q_heads*head_dim).  `workspace` must hold
 * fqa_decode_workspace_bytes(dims, dec_wave_cap) bytes; n_reqs_bound bounds the
 * decode requests (combine grid), and dec_seqs must hold at least n_reqs_bound rows (the
 * combine reads the row of every index below it before checking the decode count).  The split kernel runs 4 wavefronts per workgroup and
 * reserves 120 KiB of LDS per workgroup, so each workgroup holds its CU alone while it
 * runs: work queued on other streams meanwhile gets the CUs the decode does not hold.
 * fqa_dec_default_waves sizes the plan to one workgroup per CU. */
int fqa_decode(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
               int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
               const int32_t* dec_waves, const int32_t* dec_seqs, const int32_t* meta,
               int32_t dec_wave_cap, int32_t n_reqs_bound, void* workspace, uint16_t* out,
               void* stream);

/* fqa_decode over a plan made with dec_prefix_pages (fqa_pack_cfg): the split kernel
 * attends each member's (kv head) stream from page P on and leaves its partial; workgroups
 * launched past its shares (they run as the shares' CUs free up) take one prefix item per
 * wavefront: pages [page0, page1) of the group leader's table for the 4 query heads of each
 * of the item's (up to 8) members, at the decode's precision, into fp32 partials.  The
 * combine merges a member's stream with its group's C chunk partials (log-sum-exp).  dec_prefix / dec_pre_items
 * are the pack's arrays, dec_pre_cap their capacity (0: no prefix items).  `workspace`
 * must hold fqa_decode_prefix_workspace_bytes(dims, dec_wave_cap, dec_pre_cap) bytes.
 * The same output as fqa_decode up to fp32 rounding (the prefix keys are summed in
 * chunks, then merged). */
int64_t fqa_decode_prefix_workspace_bytes(const fqa_dims* dims, int32_t dec_wave_cap,
                                          int32_t dec_pre_cap);
int fqa_decode_prefix(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                      int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                      const int32_t* dec_waves, const int32_t* dec_seqs,
                      const int32_t* dec_prefix, const int32_t* dec_pre_items,
                      const int32_t* meta, int32_t dec_wave_cap, int32_t dec_pre_cap,
                      int32_t n_reqs_bound, void* workspace, uint16_t* out, void* stream);

/* fqa_decode without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops and harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The partials live in a fixed device array of the library
 * (17,039,360 bytes per device, held until the process ends); dec_wave_cap above
 * FQA_DECODE_NOALLOC_MAX_WAVES is FQA_EINVAL.  The array's device address is looked up
 * on the first call on each device (hipGetSymbolAddress); no call allocates or frees.
 * Every call on one device shares that device's array: calls that overlap in time on one
 * device (different streams, or different host threads) race and must be serialised by
 * the caller.  Results are bit-identical to fqa_decode's.  dec_seqs must hold at least
 * n_reqs_bound rows, as for fqa_decode. */
#define FQA_DECODE_NOALLOC_MAX_WAVES 4096
int fqa_decode_noalloc(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                       int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                       const int32_t* dec_waves, const int32_t* dec_seqs, const int32_t* meta,
                       int32_t dec_wave_cap, int32_t n_reqs_bound, uint16_t* out,
                       void* stream);

/* Varlen causal FlashAttention-2 prefill on bf16 MFMA over the pack's prefill plan:
 * one workgroup per (query tile, kv head) computes all 4 query heads of the kv head
 * from one LDS-staged copy of each K/V tile.  Mask: key pos <= query pos (cached
 * prefix included).  Output rows out[cu_seqlens[r] + i].  Row i of request r is at
 * position computed[r] + i, as fqa_pack writes positions[] (scheduler.h:66-72); the kernel
 * derives it from the work item rather than loading positions[].  pre_tile_q must be the
 * pack's: 64 (each wave runs two 32-row blocks of one query head, so every K/V fragment
 * it reads feeds two MFMAs; FQA_PRE_TILE_Q, the fastest) or 32; other values return
 * FQA_EUNSUPPORTED. */
int fqa_prefill(const fqa_dims* dims, const uint16_t* qkv, const uint16_t* pool,
                int64_t pool_pages, const int32_t* block_tables, int32_t max_blocks,
                const int32_t* cu_seqlens, const int32_t* positions,
                const int32_t* pre_items, const int32_t* meta, int32_t pre_tile_q,
                int32_t pre_item_cap, uint16_t* out, void* stream);

/* Token sampling over fp32 logits, one row per sampling request (LaunchSampleBatch,
 * kernels.cu:184-327; SampleParams, sampler.h): row b of `logits` (row stride
 * `row_stride` floats, `vocab` entries) yields out[b]:
 *   inv_temp[b] <= 0: greedy, the index of the largest logit; equal logits resolve as the
 *     reference's ArgmaxKernel resolves them (kernels.cu:184-214: 256 strided scans and a
 *     tree reduction), i.e. the column with the smallest (bit-reversed column % 256,
 *     column / 256); a row with nothing above -1e30 (its starting value) gives 0;
 *   inv_temp[b] > 0: weights w_i = exp((l_i - max) * inv_temp[b]); with top_p[b] < 1 only
 *     the largest weights are kept, the fewest whose mass reaches top_p[b] * sum(w) (all
 *     weights equal to the smallest kept one included); the token is the first index i
 *     (in vocabulary order) at which the running sum of kept weights reaches
 *     u[b] * (kept mass), u[b] in [0, 1) the caller's uniform draw; a token of zero
 *     weight is never picked (the reference can pick one for u = 0 exactly), and a
 *     draw past the summed mass picks the last token, as in the reference.
 * One 1024-thread workgroup per row.  Weights are summed in fp32 (as the reference does),
 * so a draw that lands within the rounding of a cumulative-mass boundary can pick either
 * neighbour.  vocab in [1, 2^24], n_rows >= 0. */
int fqa_sample(const float* logits, int32_t n_rows, int32_t vocab, int64_t row_stride,
               const float* inv_temp, const float* top_p, const float* u, int32_t* out,
               void* stream);

/* The layer projections y = x . W^T (LaunchGemm, kernels.cu:9-16, called at
 * model_runtime.cu:261, 280, 285, 288, 322): x [M, K] bf16 (row stride ldx), W [N, K] bf16
 * (row stride ldw; the reference's weight layout), y [M, N] (row stride ldy) in bf16
 * (y_f32 = 0, rounded to nearest even) or fp32 (y_f32 = 1, as for the reference's
 * lm_head); fp32 accumulation.  Requires N % 128 == 0 and K % 64 == 0 (FQA_EUNSUPPORTED
 * otherwise: every Qwen3-8B projection qualifies), ldx and ldw multiples of 8 and ldy of 4
 * elements, x, W and y 16-byte aligned, and every row start of x and W within 4 GiB of
 * its base.  Shapes with few 256 x 128 output tiles split K over several workgroups and
 * need `workspace` (16-byte aligned) of fqa_gemm_workspace_bytes(M, N, K) bytes (0: none;
 * its contents need no initialisation).  M = 0 is a no-op. */
int64_t fqa_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K);
int fqa_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
             int32_t M, int32_t N, int32_t K, int32_t y_f32, void* workspace,
             int64_t workspace_bytes, void* stream);

/* lm_head fused with the greedy pick (LaunchGemm(lm_head) + ArgmaxKernel,
 * model_runtime.cu:322-325, kernels.cu:184-327): out[m] = the column of the largest value of
 * row m of x . W^T (fp32 accumulation over the whole of K per tile, never split), ties and
 * rows without a value above -1e30 resolved as fqa_sample's greedy rows resolve them.  Where
 * fqa_gemm's plan for the same shape does not split K (every lm_head shape: 1187 column
 * tiles at vocab 151936), the values are the fp32 logits fqa_gemm writes with y_f32 = 1,
 * so the pick equals fqa_sample's greedy pick on those logits; where fqa_gemm splits K its
 * logits are summed in another order and can differ in the last bit.  Every row of x is
 * picked greedily: in a batch that mixes greedy and sampled rows, either gather the greedy
 * rows of x into a compact x first, or pick every row and then run fqa_gemm (fp32) +
 * fqa_sample on the sampled rows only and let their picks overwrite.
 * The logits are never written: each output tile leaves its row maxima in `workspace`
 * (fqa_gemm_argmax_workspace_bytes(M, N, K) bytes, 16-byte aligned) and a second kernel
 * reduces them.  Shape rules as fqa_gemm. */
int64_t fqa_gemm_argmax_workspace_bytes(int32_t M, int32_t N, int32_t K);
int fqa_gemm_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t M,
                    int32_t N, int32_t K, int32_t* out, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* The QKV projection fused with fqa_qknorm_rope_append (model_runtime.cu:261-268:
 * LaunchGemm into buf_.qkv, LaunchHeadNormRope, StoreKV): qkv = x . w_qkv^T for `rows`
 * rows (x [rows, hidden] bf16, row stride ldx; w_qkv [6144, hidden], row stride ldw), then
 * per row the norm + RoPE + append of fqa_qknorm_rope_append with the same arguments and
 * results (rows_bound = rows; meta[FQA_META_ROWS] must not exceed rows).  The bf16 qkv of
 * the unfused path is never written and read back:
 *   - when the projection splits K (decode-sized row counts), the append kernel reads the
 *     fp32 split partials directly, summed in the order fqa_gemm's reduction uses;
 *   - otherwise (513..1024 rows, and from 1281 rows on: the tiles alone fill the device)
 *     the projection's epilogue rounds its tile to bf16 in LDS and applies the norm, RoPE
 *     and append there.
 * Either way the results are bit-identical to fqa_gemm followed by fqa_qknorm_rope_append,
 * and only q (and k with write_k_inplace) of qkv is written, for rows below
 * meta[FQA_META_ROWS]; v goes to the pool only.  workspace: fqa_gemm_workspace_bytes(rows,
 * 6144, hidden) bytes. */
int fqa_qkv_proj_append(const fqa_dims* dims, const uint16_t* x, int64_t ldx,
                        const uint16_t* w_qkv, int64_t ldw, int32_t rows, int32_t hidden,
                        uint16_t* qkv, const float* q_norm_w, const float* k_norm_w,
                        const float* cos_tab, const float* sin_tab, int32_t rope_max_pos,
                        const int32_t* positions, const int32_t* slot_mapping,
                        const int32_t* meta, uint16_t* pool, int64_t pool_pages,
                        int32_t write_k_inplace, void* workspace, int64_t workspace_bytes,
                        void* stream);

/* The HBM read floor of a decode plan (a measurement aid, no counterpart in the
 * reference): the same grid walks the same shares of the same (page, kv head) runs of
 * fqa_pack's decode plan with fqa_decode's per-lane loads, but computes nothing; each
 * lane folds its loaded words into one 32-bit value written to `sink`
 * (dec_wave_cap x 64 x 4 bytes).  Its time bounds what fqa_decode can reach on that
 * plan. */
int fqa_decode_read_floor(const uint16_t* pool, int64_t pool_pages, const int32_t* block_tables,
                          int32_t max_blocks, const int32_t* dec_waves, const int32_t* dec_seqs,
                          const int32_t* meta, int32_t dec_wave_cap, void* sink, void* stream);
/* The same over a plan made with dec_prefix_pages: the streams' pages only (the prefix
 * items' reads are not included). */
int fqa_decode_read_floor_prefix(const uint16_t* pool, int64_t pool_pages,
                                 const int32_t* block_tables, int32_t max_blocks,
                                 const int32_t* dec_waves, const int32_t* dec_seqs,
                                 const int32_t* dec_prefix, const int32_t* meta,
                                 int32_t dec_wave_cap, void* sink, void* stream);

/* Library version string. */
const char* fqa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FQA_H_ */
