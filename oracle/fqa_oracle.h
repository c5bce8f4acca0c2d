/*
 * fqa_oracle.h — CPU restatement (C99 + OpenMP, fp32 accumulate) of the reference
 * engine's per-step attention path.  TEST INFRASTRUCTURE ONLY: the checker for the
 * HIP library and the CPU baseline of bench.py.  Nothing in the product links it.
 *
 * Same data formats as include/fqa.h (batch arrays, pack outputs, pool layout), host
 * memory throughout.  bf16 values are uint16_t bit patterns.
 */
#ifndef FQA_ORACLE_H_
#define FQA_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> float, round-to-nearest-even (the rounding of __float2bfloat16). */
float fqo_bf16_to_f32(uint16_t b);
uint16_t fqo_f32_to_bf16(float f);

void fqo_rope_tables(int max_pos, int head_dim, float theta, float* cos_tab, float* sin_tab);

int fqo_schedule(int n_running, const int32_t* num_tokens, const int32_t* computed,
                 int token_budget, int prefill_chunk, int32_t* batch_req, int32_t* batch_n);

/* Returns the pack status; fills every output exactly as fqa_pack specifies. */
int fqo_pack(int n_reqs, const int32_t* computed, const int32_t* n_new, const int32_t* bt_off,
             const int32_t* bt_pages, int max_rows, int max_blocks, int64_t pool_pages,
             int dec_grid_waves, int dec_min_pages, int dec_wave_cap, int pre_tile_q,
             int pre_item_cap, int dec_share, int dec_prefix_pages, int dec_pre_cap,
             int32_t* cu_seqlens, int32_t* qlen, int32_t* positions,
             int32_t* row_req, int32_t* slot_mapping, int32_t* block_tables,
             int32_t* decode_rids, int32_t* prefill_rids, int32_t* dec_seqs,
             int32_t* dec_waves, int32_t* pre_items, int32_t* dec_prefix,
             int32_t* dec_pre_items, int32_t* meta);

void fqo_qknorm_rope_append(int n_q, int n_kv, int head_dim, int qkv_stride, float eps,
                            uint16_t* qkv, const float* wq, const float* wk,
                            const float* cos_tab, const float* sin_tab, int rope_max_pos,
                            const int32_t* positions, const int32_t* slot_mapping, int rows,
                            uint16_t* pool, int64_t pool_pages, int write_k_inplace);

void fqo_decode(int n_q, int n_kv, int head_dim, int qkv_stride, float scale,
                const uint16_t* qkv, const uint16_t* pool, int64_t pool_pages,
                const int32_t* block_tables, int max_blocks, const int32_t* cu_seqlens,
                const int32_t* positions, const int32_t* decode_rids, int n_decode,
                uint16_t* out);

void fqo_prefill(int n_q, int n_kv, int head_dim, int qkv_stride, float scale,
                 const uint16_t* qkv, const uint16_t* pool, int64_t pool_pages,
                 const int32_t* block_tables, int max_blocks, const int32_t* cu_seqlens,
                 const int32_t* positions, const int32_t* prefill_rids, int n_prefill,
                 uint16_t* out);
void fqo_prefill_absv(int n_q, int n_kv, int head_dim, int qkv_stride, float scale,
                      const uint16_t* qkv, const uint16_t* pool, int64_t pool_pages,
                      const int32_t* block_tables, int max_blocks, const int32_t* cu_seqlens,
                      const int32_t* positions, const int32_t* prefill_rids, int n_prefill,
                      uint16_t* out, float* absv);

/* Float view of one pooled key or value: returns pool element offset of
 * (page, kv head, plane 0=K/1=V, token-in-page, dim). */
int64_t fqo_pool_offset(int n_kv, int head_dim, int64_t page, int kvh, int plane, int tok,
                        int d);

int fqo_num_threads(void);

/* LaunchSampleBatch (kernels.cu:184-327) in fp64; kept_thr / kept_mass may be NULL. */
void fqo_sample(const float* logits, int n_rows, int vocab, int64_t stride,
                const float* inv_temp, const float* top_p, const float* u, int32_t* out,
                double* kept_thr, double* kept_mass);

#ifdef __cplusplus
}
#endif

#endif
