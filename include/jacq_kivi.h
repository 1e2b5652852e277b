/*
 * jacq_kivi.h -- C ABI of the MI355X (gfx950) int4-KIVI paged KV-cache library
 * (libjacq_kivi.so).
 *
 * Two groups of entry points:
 *
 *  1. The reference's callable launch contract, ABI v1, unchanged: same
 *     symbol names, argument order, block-table format, packed-int4 code
 *     layout and fp16 scale/zero layout.  Geometry is fixed per symbol, as in
 *     the reference (NH=40, NKV=8, HD=128, page=group=32, residual=128,
 *     124-entry block table; the *_tp2_local symbols use NH=20, NKV=4).
 *     Citations are to the reference repository.
 *
 *  2. Additive runtime-geometry entry points (jacq_kivi_*): batches of
 *     sequences, page size 16 or 32 with a 32-token quantisation group, head
 *     dim 64 or 128, any GQA ratio up to 16, any residual window that is a
 *     multiple of the group, and block tables wider than 124 entries.  Per
 *     sequence they compute exactly what the v1 symbols compute.
 *
 * Conventions (both groups):
 *  - every pointer is caller-owned device memory.  The v1 symbols and the
 *    writers never allocate: the v1 decodes take their split-K workspace from
 *    static device arrays of the library (8 regions of 16 MiB per GPU, one
 *    per stream that runs v1 decodes, held until the process ends; a ninth
 *    stream's v1 decode is an error).  The library allocates a pinned status
 *    word per device (jacq_kivi_init) and, for jacq_kivi_decode /
 *    jacq_kivi_decode_sparse_retained calls that pass no workspace, one
 *    split-K workspace per (device, stream), at most 16 streams per device:
 *    allocated on the stream's first such decode for at least 256 sequences
 *    and replaced by a larger one when a larger batch needs it; the smaller
 *    one is kept (a captured graph may still use it) until
 *    jacq_kivi_release_workspaces;
 *  - every call is asynchronous on `stream`; a cache write followed by a
 *    decode on the same stream is ordered;
 *  - fp16 tensors are IEEE binary16 bit patterns (jacq_half_t), bit
 *    compatible with __half / torch.float16.
 *
 * Tensor layouts (P = page size, G = 32 = quantisation group, RS = R + G):
 *   K_CODE_PAGES, V_CODE_PAGES  uint8  [num_pages, NKV, P, HD/2]
 *                               channel d of token t: byte d/2, low nibble
 *                               for even d, high nibble for odd d
 *   K_SCALE_PAGES, K_ZERO_PAGES fp16   [num_pages, NKV, HD]     (per group,
 *                               written to every page of the group)
 *   V_SCALE_PAGES, V_ZERO_PAGES fp16   [num_pages, NKV, P, HD/G]
 *   K/V_RESIDUAL_SCRATCH        fp16   [NKV, RS, HD] per sequence
 *   BLOCK_TABLE                 int32  logical page -> physical page
 */
#ifndef JACQ_KIVI_H
#define JACQ_KIVI_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t jacq_half_t;

/* Version of the reference launch contract the v1 symbols implement
 * (integrations/vllm_kivi/abi.py:36, JACQ_KIVI_ABI_VERSION = 1). */
#define JACQ_KIVI_ABI_VERSION 1
/* Version of the additive jacq_kivi_* runtime-geometry surface. */
#define JACQ_KIVI_EXT_VERSION 1

/* ------------------------------------------------------------------------ */
/* 1. Reference contract, ABI v1                                             */
/* ------------------------------------------------------------------------ */

/* Paged KIVI decode of one query token for one sequence; O [NH,HD] fp32.
 * Replaces jac_launch, crates/jac-codegen-cuda/tests/snapshots/kernels/
 * decode_attention_kivi_paged_library_flash.cu:164-172 (declared at
 * integrations/vllm_kivi/source_patch.py:570-576). */
void jac_launch(const jacq_half_t* Q, const int32_t* BLOCK_TABLE,
                const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                const jacq_half_t* K_RESIDUAL_SCRATCH, const jacq_half_t* V_RESIDUAL_SCRATCH,
                int SEQ_LEN, float* O, hipStream_t stream);

/* TP=2 local-rank geometry NH=20/NKV=4; source_patch.py:578-584. */
void jac_launch_tp2_local(const jacq_half_t* Q, const int32_t* BLOCK_TABLE,
                          const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                          const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                          const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                          const jacq_half_t* K_RESIDUAL_SCRATCH,
                          const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN, float* O,
                          hipStream_t stream);

/* Sparse-retained decode: the old tokens come from the first
 * NUM_RETAINED_PAGES entries of the compact RETAINED_BLOCK_TABLE (clamped to
 * the dense old pages of SEQ_LEN), the residual window from the scratch at the
 * dense SEQ_LEN boundary.  Replaces jac_launch_sparse_retained,
 * crates/jac-codegen-cuda/src/variants.rs:2620-2740 (declared at
 * integrations/vllm_kivi/source_patch.py:589-595). */
void jac_launch_sparse_retained(const jacq_half_t* Q, const int32_t* RETAINED_BLOCK_TABLE,
                                const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                                const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                                const jacq_half_t* V_SCALE_PAGES,
                                const jacq_half_t* V_ZERO_PAGES,
                                const jacq_half_t* K_RESIDUAL_SCRATCH,
                                const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN,
                                int NUM_RETAINED_PAGES, float* O, hipStream_t stream);

/* source_patch.py:597-603. */
void jac_launch_sparse_retained_tp2_local(
    const jacq_half_t* Q, const int32_t* RETAINED_BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
    const jacq_half_t* K_SCALE_PAGES, const jacq_half_t* K_ZERO_PAGES,
    const uint8_t* V_CODE_PAGES, const jacq_half_t* V_SCALE_PAGES,
    const jacq_half_t* V_ZERO_PAGES, const jacq_half_t* K_RESIDUAL_SCRATCH,
    const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN, int NUM_RETAINED_PAGES, float* O,
    hipStream_t stream);

/* NUM_QUERIES (<= 160) queries of ONE sequence, query i attending to the
 * first SEQ_LENS[i] tokens; Q/O [NUM_QUERIES,NH,HD].  Replaces
 * jac_launch_batched, crates/jac-codegen-cuda/src/variants.rs:2776-2930
 * (declared at source_patch.py:608-614). */
void jac_launch_batched(const jacq_half_t* Q, const int32_t* SEQ_LENS,
                        const int32_t* BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
                        const jacq_half_t* K_SCALE_PAGES, const jacq_half_t* K_ZERO_PAGES,
                        const uint8_t* V_CODE_PAGES, const jacq_half_t* V_SCALE_PAGES,
                        const jacq_half_t* V_ZERO_PAGES, const jacq_half_t* K_RESIDUAL_SCRATCH,
                        const jacq_half_t* V_RESIDUAL_SCRATCH, int NUM_QUERIES, float* O,
                        hipStream_t stream);

/* source_patch.py:616-622. */
void jac_launch_batched_tp2_local(const jacq_half_t* Q, const int32_t* SEQ_LENS,
                                  const int32_t* BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
                                  const jacq_half_t* K_SCALE_PAGES,
                                  const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                                  const jacq_half_t* V_SCALE_PAGES,
                                  const jacq_half_t* V_ZERO_PAGES,
                                  const jacq_half_t* K_RESIDUAL_SCRATCH,
                                  const jacq_half_t* V_RESIDUAL_SCRATCH, int NUM_QUERIES,
                                  float* O, hipStream_t stream);

/* Single-token cache write (NEW_K/NEW_V [NKV,HD]); SEQ_LEN is the length
 * after the append.  Replaces jac_launch_cache_write, variants.rs:3226-3253
 * (declared at source_patch.py:643-648). */
void jac_launch_cache_write(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                            jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                            jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                            jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                            const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                            const int32_t* BLOCK_TABLE, int SEQ_LEN, hipStream_t stream);

/* NUM_NEW (<= 160) token-major tokens [NUM_NEW,NKV,HD] appended at
 * START_SEQ_LEN.  Replaces jac_launch_cache_write_batched,
 * variants.rs:3186-3268 (declared at source_patch.py:653-658). */
void jac_launch_cache_write_batched(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                                    jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                                    jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                                    jacq_half_t* K_RESIDUAL_SCRATCH,
                                    jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                                    const jacq_half_t* NEW_V, const int32_t* BLOCK_TABLE,
                                    int START_SEQ_LEN, int NUM_NEW, hipStream_t stream);

/* The hand-written writer's host entry, source_patch.py:624-629 / :1661-1697.
 * SLOT_MAPPING is accepted and ignored, as in the reference (:1667-1675).
 * NKV_RUNTIME selects 8 (global) or 4 (TP=2 local).  The reference declares
 * this with C++ linkage and __half pointers; that overload is exported too
 * (end of this header), so a hipified reference binding links unchanged. */
void kivi_cache_write_launch(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                             jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                             jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                             jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                             const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                             const int64_t* SLOT_MAPPING, const int32_t* BLOCK_TABLE,
                             int seq_len, int NKV_RUNTIME, hipStream_t stream);

/* source_patch.py:631-637 / :1737-1775. */
void kivi_cache_write_batched_launch(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                                     jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                                     jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                                     jacq_half_t* K_RESIDUAL_SCRATCH,
                                     jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                                     const jacq_half_t* NEW_V, const int64_t* SLOT_MAPPING,
                                     const int32_t* BLOCK_TABLE, int START_SEQ_LEN, int NUM_NEW,
                                     int NKV_RUNTIME, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 2. Runtime-geometry surface                                               */
/* ------------------------------------------------------------------------ */

/* Status codes of the jacq_kivi_* functions. */
#define JACQ_KIVI_OK 0
#define JACQ_KIVI_EINVAL 1   /* argument outside the supported contract */
#define JACQ_KIVI_EHIP 2     /* a HIP runtime call failed */
#define JACQ_KIVI_ENOMEM 3   /* workspace allocation failed / too small */
#define JACQ_KIVI_ETIMEOUT 4 /* a split-K merge wait of an earlier decode ran out */

typedef struct jacq_kivi_geometry {
  int32_t num_heads;         /* NH */
  int32_t num_kv_heads;      /* NKV; NH % NKV == 0, NH / NKV <= 16 */
  int32_t head_dim;          /* HD: 64 or 128 */
  int32_t page_size;         /* P: 16 or 32 tokens per physical page */
  int32_t group_size;        /* quantisation group: 32 */
  int32_t residual;          /* R: fp16 window, positive multiple of 32 */
  int32_t max_pages_per_seq; /* block-table row width */
  int32_t num_pages;         /* physical pages in the pool */
} jacq_kivi_geometry;

/* ABI v1 contract version (1) and runtime-geometry surface version. */
int jacq_kivi_abi_version(void);
int jacq_kivi_ext_version(void);

/* Message of the last error reported by a jacq_kivi_* call on this thread. */
const char* jacq_kivi_last_error(void);

/* Per-device set-up of the current device (no counterpart in the reference,
 * whose symbols keep no state): device properties and a pinned status word
 * the decode kernels set when a split-K merge times out.  Every entry point
 * does it on its first call on a device; calling it first keeps that
 * one-time host allocation out of later calls (and out of graph captures). */
int jacq_kivi_init(void);

/* Merge time-out status of the current device (no counterpart in the
 * reference).  A decode's split-K merge waits at most 1 s for the partials of
 * its own launch; if that runs out (its stream wavefronts never ran, e.g.
 * starved on a shared device) it writes NaN for the merged outputs and sets
 * the device's status word.  While the word is set, every jacq_kivi_* decode
 * returns JACQ_KIVI_ETIMEOUT without launching and every v1 decode symbol
 * prints the error and exits(1), as its other launch errors do.  This call
 * synchronises `stream`, and when the word is set it waits for the device,
 * zeroes every workspace the library owns on the device and `workspace`
 * (when not NULL; flags a timed-out merge left behind would otherwise be read
 * by a graph replay carrying the same epoch), clears the word and returns
 * JACQ_KIVI_ETIMEOUT; otherwise JACQ_KIVI_OK.  Call it with no decode running
 * on the device.  A timed-out merge also poisons the workspace it ran on
 * (its first 8 bytes): until that workspace is zeroed here, every merged
 * segment of a decode on it -- a graph replay included, which never passes
 * through the host checks -- is NaN and sets the status word again, never a
 * finite value built from a stale partial. */
int jacq_kivi_decode_status(void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Frees every split-K workspace the library allocated on the current device
 * for jacq_kivi_* decodes without a workspace (no counterpart in the
 * reference).  It synchronises the device first.  Graphs captured with such a
 * decode hold the freed addresses and must not be replayed afterwards.  The
 * static arrays (v1 decodes, jacq_kivi_decode_noalloc) are not affected. */
int jacq_kivi_release_workspaces(void);

/* Test hook (no counterpart in the reference): with microseconds > 0 every
 * later matrix-core decode's merge waits for a tag that no wavefront stores
 * and gives up after that long, so tests can force the time-out path from the
 * host (every kernel still exits normally).  0 restores normal operation. */
void jacq_kivi_test_force_merge_timeout(uint32_t microseconds);

/* Test hook (no counterpart in the reference): device allocations
 * (hipMalloc) the library has made in this process -- the split-K
 * workspaces of jacq_kivi_* decodes called without one.  The v1 symbols, the
 * writers and jacq_kivi_decode_noalloc never add to it. */
int64_t jacq_kivi_test_device_allocations(void);

/* Geometry check (integrations/vllm_kivi/layout.py:51-74 and the supported
 * geometry checks of source_patch.py:744-756, generalised). */
int jacq_kivi_check_geometry(const jacq_kivi_geometry* geo);

/* Longest sequence the geometry addresses: old-token capacity of the table
 * (whole groups) + R.  4096 for the v1 geometry (abi.py:48-53). */
int64_t jacq_kivi_max_seq_len(const jacq_kivi_geometry* geo);

/* check_block_table_width, source_patch.py:692-707, at runtime geometry:
 * JACQ_KIVI_OK when a table of `width` entries covers a sequence of
 * `seq_len` tokens, JACQ_KIVI_EINVAL otherwise (message names the bound). */
int jacq_kivi_check_block_table_width(const jacq_kivi_geometry* geo, int64_t width,
                                      int64_t seq_len);

/* Bytes of split-K workspace jacq_kivi_decode needs for `batch` sequences. */
size_t jacq_kivi_decode_workspace_size(const jacq_kivi_geometry* geo, int32_t batch);

/* Decode one query token per sequence for `batch` sequences.
 *   Q             [batch, NH, HD] fp16
 *   SEQ_LENS      [batch] int32 (device), tokens each query attends to
 *   BLOCK_TABLES  [batch, max_pages_per_seq] int32
 *   K/V_SCR       [batch, NKV, R+32, HD] fp16
 *   O             [batch, NH, HD] fp32
 * workspace may be NULL (the library then uses its own for `stream`) or at
 * least jacq_kivi_decode_workspace_size bytes.  Its contents on entry do not
 * matter: the split-K partials a call stores are tagged with that call's
 * 64-bit launch epoch (random start, top bit set) and each flag is cleared
 * when read.  Two calls that can run at the same time must not share a
 * workspace.  Returns JACQ_KIVI_ETIMEOUT, launching nothing, while the
 * device's merge status is set (jacq_kivi_decode_status).  Sequence lengths are clamped to [0, jacq_kivi_max_seq_len] on the
 * device, as the reference kernel clamps (snapshot :74-83). */
int jacq_kivi_decode(const jacq_kivi_geometry* geo, const jacq_half_t* Q,
                     const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLES,
                     const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                     const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                     const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                     const jacq_half_t* K_RESIDUAL_SCRATCH,
                     const jacq_half_t* V_RESIDUAL_SCRATCH, int32_t batch, float* O,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* One decode step of the cache in one launch: append one token per sequence
 * (quantising the 32-token group that ages out of the residual window where
 * one does, and shifting the scratch), then decode one query per sequence
 * over the new state.  It replaces the reference's per-token pair
 * kivi_cache_write(SEQ_LEN) followed by kivi_decode(SEQ_LEN) on one stream
 * (integrations/vllm_kivi/source_patch.py:3259-3288; the writer :1661-1697,
 * the decode as jacq_kivi_decode) and leaves pages, scales, zeros and the
 * scratch bit for bit as jacq_kivi_cache_append(START_LENS = SEQ_LENS - 1,
 * num_new = 1) would, and O as jacq_kivi_decode(SEQ_LENS) on that state
 * computes it (the same kernel, to its run split).
 *   NEW_K, NEW_V  [batch, NKV, HD] fp16, the token at position SEQ_LENS - 1
 *   SEQ_LENS      [batch] int32 (device), lengths after the write, >= 1
 *   pages and scratch are written in place (jacq_kivi_cache_append's arrays)
 * workspace: NULL or at least jacq_kivi_write_decode_workspace_size bytes,
 * contents on entry irrelevant (as jacq_kivi_decode's). */
size_t jacq_kivi_write_decode_workspace_size(const jacq_kivi_geometry* geo, int32_t batch);
int jacq_kivi_write_decode(const jacq_kivi_geometry* geo, const jacq_half_t* Q,
                           const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                           const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLES,
                           uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                           jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                           jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                           jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                           int32_t batch, float* O, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* jacq_kivi_decode with no allocation at all.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as jacq_kivi_decode without the
 * workspace: the split-K partials go to a static 32 MiB device array of the
 * library (one copy per GPU, held until the process ends), enough for 256
 * sequences at the long-context geometry (64/8 heads, HD 128).  A batch that
 * needs more is refused with JACQ_KIVI_ENOMEM and nothing launched.
 * jacq_kivi_init() must have run on the device first (its set-up is the only
 * allocation; otherwise JACQ_KIVI_EINVAL).  Every call on a GPU shares that
 * GPU's array: calls that can overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller. */
int jacq_kivi_decode_noalloc(const jacq_kivi_geometry* geo, const jacq_half_t* Q,
                             const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLES,
                             const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                             const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                             const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                             const jacq_half_t* K_RESIDUAL_SCRATCH,
                             const jacq_half_t* V_RESIDUAL_SCRATCH, int32_t batch, float* O,
                             hipStream_t stream);

/* Sparse-retained decode of one sequence at a runtime geometry (the
 * jac_launch_sparse_retained window, variants.rs:2667-2680).
 *   Q                     [NH, HD] fp16
 *   RETAINED_BLOCK_TABLE  compact physical-page ids of the retained old pages
 *   K/V_SCR               [NKV, R+32, HD] fp16
 *   O                     [NH, HD] fp32
 * NUM_RETAINED_PAGES must be in [0, max_pages_per_seq] and <= num_pages, and
 * SEQ_LEN in [1, jacq_kivi_max_seq_len] (the checks of source_patch.py:942-945
 * at this geometry); the device clamps NUM_RETAINED_PAGES to the dense old
 * pages of SEQ_LEN.  At page 16 the retained pages are taken in whole 32-token
 * groups.  workspace as for jacq_kivi_decode (batch 1). */
int jacq_kivi_decode_sparse_retained(
    const jacq_kivi_geometry* geo, const jacq_half_t* Q, int32_t SEQ_LEN,
    const int32_t* RETAINED_BLOCK_TABLE, int32_t NUM_RETAINED_PAGES,
    const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
    const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
    const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
    const jacq_half_t* K_RESIDUAL_SCRATCH, const jacq_half_t* V_RESIDUAL_SCRATCH, float* O,
    void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Append num_new tokens to each of `batch` sequences in one launch.
 *   NEW_K/NEW_V   [batch, num_new, NKV, HD] fp16, token-major per sequence
 *   START_LENS    [batch] int32 (device), length of each sequence before
 *                 the append
 * Any num_new >= 1: every group that ages out is quantised (bit-identical to
 * feeding the tokens one at a time through jac_launch_cache_write) and the
 * residual scratch ends holding the newest tokens.  When
 * residual_len + num_new <= R + 32 (at most one age-out) the scratch goes
 * through exactly the reference's append-then-shift states; otherwise only
 * its first residual_len rows are defined. */
int jacq_kivi_cache_append(const jacq_kivi_geometry* geo, uint8_t* K_CODE_PAGES,
                           jacq_half_t* K_SCALE_PAGES, jacq_half_t* K_ZERO_PAGES,
                           uint8_t* V_CODE_PAGES, jacq_half_t* V_SCALE_PAGES,
                           jacq_half_t* V_ZERO_PAGES, jacq_half_t* K_RESIDUAL_SCRATCH,
                           jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                           const jacq_half_t* NEW_V, const int32_t* BLOCK_TABLES,
                           const int32_t* START_LENS, int32_t num_new, int32_t batch,
                           hipStream_t stream);

/* One entry of the batched-write plan, source_patch.py:495-501.
 * age_out_page / post_shift_residual_len are -1 for None. */
typedef struct jacq_kivi_subchunk {
  int32_t start_seq_len;
  int32_t num_new;
  int32_t scratch_start;
  int32_t age_out_page;
  int32_t post_shift_residual_len;
} jacq_kivi_subchunk;

/* plan_batched_write, source_patch.py:504-553 (host only).  Returns the
 * number of sub-chunks written to `out` (at most `cap`), or -1 with
 * jacq_kivi_last_error() set (the reference raises ValueError). */
int32_t jacq_kivi_plan_batched_write(int32_t start_seq_len, int32_t num_new, int32_t residual,
                                     int32_t group, jacq_kivi_subchunk* out, int32_t cap);

/* Measurement hook (no counterpart in the reference; for benchmarks and
 * profilers).  jacq_kivi_profile_start enables recording for the next
 * max_calls decode calls and max_calls cache-write calls: each records HIP
 * events on its own stream around its kernels.  jacq_kivi_profile_stop
 * disables recording, waits for the events and writes, per call (at most cap
 * entries), the milliseconds of the decode kernel and of what follows it on
 * the stream until the decode's end event; it returns the number of decode
 * calls written or -1.  The matrix-core decode is one kernel (its split-K
 * merge runs in the same launch).  With split != 0 the kernel is launched
 * with start / stop events stamped at its own start and end (that launch form
 * delays the next kernel by a few microseconds); with split == 0 plain
 * records bracket the decode: kernel_ms then holds the whole decode and
 * merge_ms zero.  jacq_kivi_profile_write_ms then writes the per-call
 * milliseconds of the cache-write kernel recorded in the same window. */
/* Profiling, additive, no counterpart in the reference: per-workgroup stamps
 * of the following matrix-core decodes into `buffer` (device memory,
 * capacity x 4 uint64): buffer[4b..4b+3] = {start, end} in s_memrealtime
 * ticks (100 MHz), HW_ID | XCC_ID << 32, and for a stream workgroup its work
 * units (bits 0-31) and the ticks until its first quantised group was in LDS
 * (bits 32-63); 0 for the merge workgroups, which follow the stream ones.
 * NULL turns it off. */
int jacq_kivi_profile_wave_stamps(uint64_t* buffer, int32_t capacity);
int jacq_kivi_profile_start(int32_t max_calls, int32_t split);
int32_t jacq_kivi_profile_stop(float* kernel_ms, float* merge_ms, int32_t cap);
int32_t jacq_kivi_profile_write_ms(float* ms, int32_t cap);

#ifdef __cplusplus
}
#endif

#ifdef __cplusplus
/* The two writer entry points with the reference's own C++ declaration
 * (source_patch.py:624-637, `__half` and `cudaStream_t` as hipify maps
 * them): same mangled names as the reference binding expects.  They forward
 * to the C-linkage functions above. */
#include <hip/hip_fp16.h>

void kivi_cache_write_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
                             __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES,
                             __half* V_SCALE_PAGES, __half* V_ZERO_PAGES,
                             __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
                             const __half* NEW_K, const __half* NEW_V,
                             const int64_t* SLOT_MAPPING, const int* BLOCK_TABLE, int seq_len,
                             int NKV_RUNTIME, hipStream_t stream);

void kivi_cache_write_batched_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
                                     __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES,
                                     __half* V_SCALE_PAGES, __half* V_ZERO_PAGES,
                                     __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
                                     const __half* NEW_K, const __half* NEW_V,
                                     const int64_t* SLOT_MAPPING, const int* BLOCK_TABLE,
                                     int START_SEQ_LEN, int NUM_NEW, int NKV_RUNTIME,
                                     hipStream_t stream);
#endif

#endif /* JACQ_KIVI_H */
