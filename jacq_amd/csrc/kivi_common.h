// kivi_common.h -- shared definitions of the gfx950 KIVI kernels.
//
// Geometry is runtime (the reference bakes it in as constexpr per translation
// unit, decode_attention_kivi_paged_library_flash.cu:14-24); the kernels
// take one KiviGeo by value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jacq {

constexpr int kGroup = 32;  // KIVI quantisation group (tokens for K, channels for V)

struct KiviGeo {
  int nh;         // query heads
  int nkv;        // kv heads
  int hd;         // head dim (64 | 128)
  int page;       // tokens per physical page (16 | 32)
  int residual;   // fp16 residual window R (multiple of 32)
  int max_pages;  // block-table row width
  int num_pages;  // physical page capacity (INT32_MAX when unknown)
  int gqa;        // nh / nkv
  int rs;         // scratch rows = R + 32
  int lq;         // old-token capacity: (max_pages*page) rounded down to whole groups
};

// source_patch.py:1655-1659
__host__ __device__ inline int split_old_tokens(int seq_len, int residual) {
  const int quantizable = seq_len - residual;
  if (quantizable < 0) return 0;
  return (quantizable / kGroup) * kGroup;
}

// Decode window (snapshot :74-83 at runtime geometry): tokens [0, old_valid)
// come from pages, [old_valid, old_valid + residual_valid) from scratch.
__host__ __device__ inline void decode_window(const KiviGeo& g, int seq_len, int* old_valid,
                                              int* residual_valid) {
  int bounded = seq_len;
  if (bounded < 0) bounded = 0;
  if (bounded > g.lq + g.residual) bounded = g.lq + g.residual;
  int quantizable = bounded - g.residual;
  if (quantizable < 0) quantizable = 0;
  int ov = (quantizable / kGroup) * kGroup;
  if (ov > g.lq) ov = g.lq;
  int rv = bounded - ov;
  if (rv < 0) rv = 0;
  if (rv > g.rs) rv = g.rs;
  *old_valid = ov;
  *residual_valid = rv;
}

// Split-K plan of one sequence of n tokens: about kSplitTarget tokens per
// split, at most kMaxSplits splits unless that would make a split longer
// than kMaxSplitTokens, chunks of whole 32-token groups.  It depends on n
// alone, so a sequence decodes to the same bits whatever else is in the batch
// (single and batched calls agree exactly).
constexpr int kSplitTarget = 512;
constexpr int kMaxSplits = 16;
constexpr int kMaxSplitTokens = 4096;

__host__ __device__ inline int split_count(long long n) {
  long long s = (n + kSplitTarget - 1) / kSplitTarget;
  if (s > kMaxSplits) s = kMaxSplits;
  const long long s_min = (n + kMaxSplitTokens - 1) / kMaxSplitTokens;
  if (s < s_min) s = s_min;
  if (s < 1) s = 1;
  return (int)s;
}

__host__ __device__ inline void split_plan(int n, int* nsplit, int* chunk) {
  const int s = split_count(n);
  int c = (n + s - 1) / s;
  c = ((c + kGroup - 1) / kGroup) * kGroup;
  if (c < kGroup) c = kGroup;
  *chunk = c;
  *nsplit = n > 0 ? (n + c - 1) / c : 1;
}

// ---- quantiser arithmetic shared by the writer and the fused step ----
// static_cast<int>(rintf(x)) clamped to [0, 15] (source_patch.py:1517-1522),
// with the conversion CUDA and gfx950 hardware perform: out-of-range values
// saturate, NaN becomes 0.  Clamped in the float domain, because an
// out-of-range float -> int conversion is undefined in C++ and the compiler
// may assume it does not happen.
__device__ inline int clamp_code(float x) {
  const float r = __builtin_rintf(x);
  if (r >= 15.0f) return 15;
  if (r >= 0.0f) return (int)r;
  return 0;  // negative or NaN
}

// fminf / fmaxf of the reference's age-out kernels (source_patch.py:1555-1558,
// :1598-1599): a NaN operand is dropped, NaN results only when both are NaN.
// For a +0 / -0 pair, min gives -0 and max +0 (C Annex F's recommendation;
// LLVM's minnum leaves it open, so it is written out).  Both are then
// commutative and associative: the partial reductions below may merge in any
// order and still give one sequential loop's bits.
__device__ inline float min_num(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  if (a == b) return __uint_as_float(__float_as_uint(a) | __float_as_uint(b));
  return b < a ? b : a;
}
__device__ inline float max_num(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  if (a == b) return __uint_as_float(__float_as_uint(a) & __float_as_uint(b));
  return b > a ? b : a;
}

__device__ inline float h2f(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

__device__ inline uint16_t f2h(float f) {  // round to nearest even (v_cvt_f16_f32)
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}

}  // namespace jacq
