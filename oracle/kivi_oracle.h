/*
 * kivi_oracle.h -- CPU restatement of Jacq's int4-KIVI paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * path (jacq_amd/csrc).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never links it and
 * never falls back to it.
 *
 * Every function cites the reference file:line it restates (paths are
 * relative to the reference repository root):
 *   writer   integrations/vllm_kivi/source_patch.py:1517-1775
 *   planner  integrations/vllm_kivi/source_patch.py:488-553
 *   decode   crates/jac-codegen-cuda/tests/snapshots/kernels/
 *            decode_attention_kivi_paged_library_flash.cu:35-158
 *   merge    crates/jac-codegen-cuda/src/variants.rs:3548-3565
 *
 * Geometry is runtime (the reference bakes NH=40/NKV=8/HD=128/BS=32/R=128 in
 * as constexpr).  Page size is separated from the quantisation group: the
 * reference requires page == group == 32; here page may be any divisor of
 * the group (16 or 32).  With page == group every formula reduces to the
 * reference's.  A group that spans several pages writes its K scale/zero to
 * every page of the group; decode reads them from the group's first page.
 */
#ifndef JACQ_KIVI_ORACLE_H
#define JACQ_KIVI_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kivi_geo {
  int32_t nh;         /* query heads */
  int32_t nkv;        /* kv heads */
  int32_t hd;         /* head dim */
  int32_t page;       /* tokens per physical page */
  int32_t group;      /* KIVI quantisation group (32) */
  int32_t residual;   /* fp16 residual window R; scratch rows = R + group */
  int32_t max_pages;  /* block-table row width */
} kivi_geo;

typedef struct kivi_subchunk {
  int32_t start_seq_len;
  int32_t num_new;
  int32_t scratch_start;
  int32_t age_out_page;            /* -1 == None */
  int32_t post_shift_residual_len; /* -1 == None */
} kivi_subchunk;

/* IEEE-754 binary16 conversions (round to nearest, ties to even). */
uint16_t kivi_f32_to_f16(float x);
float kivi_f16_to_f32(uint16_t h);

/* source_patch.py:1655-1659 (split_old_tokens), generalised to runtime R/group. */
int32_t kivi_split_old_tokens(int32_t seq_len, int32_t residual, int32_t group);

/* Pack one 32-token group from a token-major fp16 row source into pages.
 * rows[t] points at HD fp16 values of token t of the group, per kv head h.
 * source_patch.py:1532-1581 (K) and :1583-1620 (V). */
void kivi_ref_pack_group(const kivi_geo* g, int32_t h, const uint16_t* const* k_rows,
                         const uint16_t* const* v_rows, const int32_t* block_table,
                         int32_t logical_group, uint8_t* k_code, uint16_t* k_scale,
                         uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                         uint16_t* v_zero);

/* kivi_cache_write_launch, source_patch.py:1661-1697: append one token
 * (new_k/new_v [NKV,HD]) to a sequence whose length AFTER the append is
 * seq_len; age out one group when the split moves; shift the scratch. */
void kivi_ref_cache_write(const kivi_geo* g, uint8_t* k_code, uint16_t* k_scale,
                          uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                          uint16_t* v_zero, uint16_t* k_scr, uint16_t* v_scr,
                          const uint16_t* new_k, const uint16_t* new_v,
                          const int32_t* block_table, int32_t seq_len);

/* kivi_cache_write_batched_launch, source_patch.py:1737-1775: append num_new
 * tokens (token-major [num_new,NKV,HD]) starting at start_seq_len, then at
 * most one age-out.  Returns 0, or -1 when the call would need more than one
 * age-out or overflow the scratch (the reference leaves that to the planner). */
int32_t kivi_ref_cache_write_batched(const kivi_geo* g, uint8_t* k_code, uint16_t* k_scale,
                                     uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                                     uint16_t* v_zero, uint16_t* k_scr, uint16_t* v_scr,
                                     const uint16_t* new_k, const uint16_t* new_v,
                                     const int32_t* block_table, int32_t start_seq_len,
                                     int32_t num_new);

/* plan_batched_write, source_patch.py:504-553.  Writes up to cap sub-chunks
 * and returns the number produced, or a negative error code:
 * -1 start<0, -2 num_new<1, -3 residual/group not positive, -4 cap too small. */
int32_t kivi_ref_plan_batched_write(int32_t start_seq_len, int32_t num_new,
                                    int32_t residual, int32_t group,
                                    kivi_subchunk* out, int32_t cap);

/* Paged KIVI decode for one sequence, fp32 online softmax in the reference's
 * token order (snapshot :51-158).  q [NH,HD] fp16, out [NH,HD] fp32. */
void kivi_ref_decode_online(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                            const uint8_t* k_code, const uint16_t* k_scale,
                            const uint16_t* k_zero, const uint8_t* v_code,
                            const uint16_t* v_scale, const uint16_t* v_zero,
                            const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                            float* out);

/* Independent float64 two-pass softmax attention over the same dequantised
 * tokens (the structure of specs/kernels/paged_attn/reference.cu:35-106). */
void kivi_ref_decode_twopass(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                             const uint8_t* k_code, const uint16_t* k_scale,
                             const uint16_t* k_zero, const uint8_t* v_code,
                             const uint16_t* v_scale, const uint16_t* v_zero,
                             const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                             double* out);

/* Sparse-retained decode (variants.rs:2620-2740): old tokens from the first
 * num_retained_pages entries of the compact retained_table (clamped to the
 * dense old pages and the table width), residual rows at the dense SEQ_LEN
 * boundary. */
void kivi_ref_decode_sparse_retained(const kivi_geo* g, const uint16_t* q,
                                     const int32_t* retained_table, const uint8_t* k_code,
                                     const uint16_t* k_scale, const uint16_t* k_zero,
                                     const uint8_t* v_code, const uint16_t* v_scale,
                                     const uint16_t* v_zero, const uint16_t* k_scr,
                                     const uint16_t* v_scr, int32_t seq_len,
                                     int32_t num_retained_pages, float* out);
/* The same window through the float64 two-pass attention. */
void kivi_ref_decode_sparse_retained_twopass(const kivi_geo* g, const uint16_t* q,
                                             const int32_t* retained_table,
                                             const uint8_t* k_code, const uint16_t* k_scale,
                                             const uint16_t* k_zero, const uint8_t* v_code,
                                             const uint16_t* v_scale, const uint16_t* v_zero,
                                             const uint16_t* k_scr, const uint16_t* v_scr,
                                             int32_t seq_len, int32_t num_retained_pages,
                                             double* out);

/* Batch driver for the CPU baseline: q [B,NH,HD], seq_lens [B], block_tables
 * [B,max_pages], scratch [B,NKV,R+group,HD], out [B,NH,HD].  Runs
 * kivi_ref_decode_online per (sequence, kv head) with the G query heads of a
 * group sharing one dequantisation, parallelised over nthreads (OpenMP). */
void kivi_ref_decode_batch(const kivi_geo* g, const uint16_t* q, const int32_t* seq_lens,
                           const int32_t* block_tables, const uint8_t* k_code,
                           const uint16_t* k_scale, const uint16_t* k_zero,
                           const uint8_t* v_code, const uint16_t* v_scale,
                           const uint16_t* v_zero, const uint16_t* k_scr,
                           const uint16_t* v_scr, int32_t batch, float* out,
                           int32_t nthreads);

/* Split-K LSE merge (variants.rs:3548-3565) of nsplit partials
 * m[nsplit], l[nsplit], acc[nsplit][hd] into out[hd]. */
void kivi_ref_lse_merge(int32_t nsplit, int32_t hd, const float* m, const float* l,
                        const float* acc, float* out);

/* Split-K decode: the token range of one sequence is cut into chunks of
 * chunk tokens; each chunk runs the online softmax and the partials are
 * merged with kivi_ref_lse_merge.  Used to pin split-K == single pass. */
void kivi_ref_decode_splitk(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                            const uint8_t* k_code, const uint16_t* k_scale,
                            const uint16_t* k_zero, const uint8_t* v_code,
                            const uint16_t* v_scale, const uint16_t* v_zero,
                            const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                            int32_t chunk, float* out);

/* check_block_table_width (source_patch.py:692-707) at runtime geometry:
 * returns the number of table entries a sequence of seq_len needs, or -1 if
 * seq_len is outside [1, max_seq_len]. */
int32_t kivi_ref_required_pages(int32_t seq_len, int32_t residual, int32_t group,
                                int32_t page, int32_t max_seq_len);

#ifdef __cplusplus
}
#endif

#endif
