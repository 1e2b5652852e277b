// kivi_kernels.h -- argument blocks and launchers of the gfx950 KIVI kernels.
#pragma once

#include "kivi_common.h"

namespace jacq {

struct AppendArgs {
  uint8_t* k_code;
  uint16_t* k_scale;
  uint16_t* k_zero;
  uint8_t* v_code;
  uint16_t* v_scale;
  uint16_t* v_zero;
  uint16_t* k_scr;
  uint16_t* v_scr;
  int64_t scr_stride;  // elements between sequences' scratch (0: shared)
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t new_stride;  // elements between sequences' new tokens
  const int32_t* block_tables;
  int64_t bt_stride;          // entries between sequences' block-table rows
  const int32_t* start_lens;  // device lengths before the append, or null
  int start_len;              // used when start_lens is null
  int num_new;
};

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_stride;  // elements between queries (NH*HD)
  const int32_t* seq_lens;  // device lengths, or null
  int seq_len;              // used when seq_lens is null
  const int32_t* block_tables;
  int64_t bt_stride;  // 0: every query shares one table (jac_launch_batched)
  const uint8_t* k_code;
  const uint16_t* k_scale;
  const uint16_t* k_zero;
  const uint8_t* v_code;
  const uint16_t* v_scale;
  const uint16_t* v_zero;
  const uint16_t* k_scr;
  const uint16_t* v_scr;
  int64_t scr_stride;  // 0: every query shares one scratch
  float* out;
  int64_t out_stride;
  float* ws_ml;   // [batch, NKV, max_splits, G, 2]  (m, l)
  float* ws_acc;  // [batch, NKV, max_splits, G, HD]
  uint64_t* ws_flag;  // matrix-core kernel: per partial slot, the epoch of the launch that stored it
  int max_splits;  // VALU kernel: split slots per (sequence, kv head)
  int batch;       // sequences (queries) in the call
  int waves;       // matrix-core kernel: wavefronts sharing the tile stream
  uint64_t* stamps = nullptr;  // matrix-core kernel, profiling: 4 words per workgroup, or null
  int stamp_cap = 0;           // workgroups the stamp buffer holds
  int merge_wgs = 0;       // matrix-core kernel: merge workgroups after the stream wavefronts
  uint64_t epoch = 0;      // matrix-core kernel: this launch's tag (set by the launcher)
  uint64_t merge_timeout = 0;  // matrix-core kernel: s_memrealtime ticks a merge waits at most
  uint64_t merge_skew = 0;     // matrix-core kernel: 0; 1 only in the forced-timeout test
  int retained_pages = -1;  // >= 0: sparse-retained window (compact block table)
  uint32_t* status = nullptr;  // matrix-core kernel: set to 1 when a merge wait runs out
  uint64_t* ws_poison = nullptr;  // matrix-core kernel: the workspace's poison word
  int per_query = 0;  // matrix-core kernel: cut each query's streams by its own length alone
  // Fused write + decode (jacq_kivi_write_decode): the writer's arrays (one
  // new token per sequence; its length before the write is seq_lens - 1), the
  // count of stream wavefronts at the front of the grid that do the writer's
  // work before their runs, and per (sequence, kv head,
  // K | V) the epoch of the launch whose writer finished that age-out.
  AppendArgs wr{};
  uint64_t* ws_wflag = nullptr;
  int writer_waves = 0;
};

// Decode window of one sequence.  Dense: the split rule (decode_window).
// Sparse-retained (variants.rs:2667-2680): the old tokens are the first
// retained_pages entries of a compact table, clamped to [0, dense old pages]
// and to the table width (whole 32-token groups when a page holds 16); the
// residual rows keep the dense boundary, so evicted pages are skipped and are
// never read as residual tokens.
__host__ __device__ inline void window_of(const KiviGeo& g, int retained_pages, int seq_len,
                                          int* old_valid, int* residual_valid) {
  decode_window(g, seq_len, old_valid, residual_valid);
  if (retained_pages >= 0) {
    int pages = retained_pages;
    const int dense_pages = *old_valid / g.page;
    if (pages > dense_pages) pages = dense_pages;
    if (pages > g.max_pages) pages = g.max_pages;
    *old_valid = pages * g.page / kGroup * kGroup;
  }
}

hipError_t launch_append(const KiviGeo& g, const AppendArgs& a, int batch, hipStream_t stream);
// `between`, when not null, is recorded on the stream after the main kernel
// and before the split-K merge (profiling).
hipError_t launch_decode(const KiviGeo& g, const DecodeArgs& a, int batch, hipStream_t stream,
                         hipEvent_t between = nullptr);
// Profiling events of the matrix-core decode (each may be null): with
// main_end, the kernel's own start and end stamped by the command processor;
// without it, a plain record before the kernel; `end` is recorded after it.
struct LaunchEvents {
  hipEvent_t start = nullptr, main_end = nullptr, end = nullptr;
};
// Per-workgroup profiling stamps of the next matrix-core decodes (null: off).
void set_wave_stamps(uint64_t* buf, int cap);
hipError_t launch_decode_mfma(const KiviGeo& g, const DecodeArgs& a, int batch,
                              hipStream_t stream, const LaunchEvents& ev = LaunchEvents());
// Test-only: with us > 0 every later matrix-core decode's merge waits for an
// epoch no wavefront stores and gives up after `us` microseconds; 0 restores
// normal operation.
void set_test_merge_timeout_us(uint32_t us);
// wavefronts the matrix-core decode launches on a device with `cus` CUs:
// as many as are resident at once
int decode_stream_waves(const KiviGeo& g, int cus);

}  // namespace jacq
