/*
 * kivi_oracle.c -- CPU restatement of Jacq's int4-KIVI paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY (see kivi_oracle.h).  Plain C99 + optional OpenMP.
 *
 * Layouts (reference formulas kept bit-for-bit, source_patch.py:1565-1578,
 * :1604, :1630; snapshot :100-101, :117, :134), with P = page size:
 *   K_CODE/V_CODE byte  ((page*NKV + h)*P + slot)*(HD/2) + d/2
 *                       channel d even -> low nibble, odd -> high nibble
 *   K_SCALE/K_ZERO      (page*NKV + h)*HD + d
 *   V_SCALE/V_ZERO      ((page*NKV + h)*P + slot)*(HD/group) + d/group
 *   scratch             (h*(R+group) + r)*HD + d   (per sequence)
 */
#include "kivi_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- binary16 <-> binary32, written from the IEEE-754 bit definitions ---- */

uint16_t kivi_f32_to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) { /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  }
  const int32_t e = (int32_t)exp - 127 + 15; /* rebiased exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e <= 0) {
    /* subnormal half (or zero): value = man_full * 2^(exp-150); target unit 2^-24 */
    if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
    const uint32_t full = man | 0x800000u;     /* 24-bit significand */
    const uint32_t shift = (uint32_t)(14 - e); /* 14..24 */
    uint32_t q = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q); /* q may carry into the first normal: still correct */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* carry may reach inf: correct */
  return (uint16_t)(sign | q);
}

float kivi_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: normalise */
      int32_t e = -1;
      do {
        man <<= 1;
        e++;
      } while (!(man & 0x400u));
      man &= 0x3ffu;
      u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---- split rule: source_patch.py:1655-1659 ---- */

int32_t kivi_split_old_tokens(int32_t seq_len, int32_t residual, int32_t group) {
  const int32_t quantizable = seq_len - residual;
  if (quantizable < 0) return 0;
  return (quantizable / group) * group;
}

static inline int32_t scratch_rows(const kivi_geo* g) { return g->residual + g->group; }

/* clamp_code, source_patch.py:1517-1522: static_cast<int>(rintf(x)) clamped
 * to [0, 15].  rintf rounds ties to even.  The float -> int conversion is
 * CUDA's cvt.rzi.s32.f32 (and gfx950's v_cvt_i32_f32): out-of-range values
 * saturate and NaN becomes 0.  C leaves that conversion undefined, so it is
 * spelled out here in the float domain: NaN -> 0, +inf -> 15, -inf -> 0. */
static inline int32_t clamp_code(float x) {
  const float r = rintf(x);
  if (r >= 15.0f) return 15;
  if (r >= 0.0f) return (int32_t)r;
  return 0; /* negative or NaN */
}

/* fminf / fmaxf, source_patch.py:1555-1558 (K) and :1598-1599 (V).  A NaN
 * operand is dropped (the other one is returned; NaN only when both are).
 * The sign of a zero result is not fixed by fminf's contract; C's Annex F
 * (F.10.9.2) recommends min(-0, +0) = -0 and max(-0, +0) = +0, which makes
 * both operations commutative and associative, so a reduction in any order
 * gives the same bits.  Equal nonzero operands have equal bits, so the OR /
 * AND below only matters for a +0 / -0 pair. */
static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static inline float min_num(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  if (a == b) return bits_f32(f32_bits(a) | f32_bits(b));
  return b < a ? b : a;
}
static inline float max_num(float a, float b) {
  if (b != b) return a;
  if (a != a) return b;
  if (a == b) return bits_f32(f32_bits(a) & f32_bits(b));
  return b > a ? b : a;
}

/* ---- group pack: K source_patch.py:1532-1581, V :1583-1620 ---- */

void kivi_ref_pack_group(const kivi_geo* g, int32_t h, const uint16_t* const* k_rows,
                         const uint16_t* const* v_rows, const int32_t* block_table,
                         int32_t logical_group, uint8_t* k_code, uint16_t* k_scale,
                         uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                         uint16_t* v_zero) {
  const int32_t HD = g->hd, GS = g->group, P = g->page, NKV = g->nkv;
  const int32_t hdp = HD / 2, hdg = HD / GS;
  const int32_t pages_per_group = GS / P;
  const int32_t first_logical_page = logical_group * pages_per_group;

  /* K: per channel over the group's GS tokens. */
  for (int32_t d = 0; d < HD; ++d) {
    float mn = kivi_f16_to_f32(k_rows[0][d]);
    float mx = mn;
    for (int32_t t = 1; t < GS; ++t) {
      const float x = kivi_f16_to_f32(k_rows[t][d]);
      mn = min_num(mn, x);
      mx = max_num(mx, x);
    }
    float scale = (mx - mn) / 15.0f;
    if (!(scale > 0.0f)) scale = 1.0f;
    const uint16_t sh = kivi_f32_to_f16(scale), zh = kivi_f32_to_f16(mn);
    for (int32_t pg = 0; pg < pages_per_group; ++pg) {
      const int64_t phys = block_table[first_logical_page + pg];
      k_scale[(phys * NKV + h) * HD + d] = sh;
      k_zero[(phys * NKV + h) * HD + d] = zh;
    }
    for (int32_t t = 0; t < GS; ++t) {
      const int32_t code = clamp_code((kivi_f16_to_f32(k_rows[t][d]) - mn) / scale);
      const int64_t phys = block_table[first_logical_page + t / P];
      uint8_t* byte = &k_code[((phys * NKV + h) * P + (t % P)) * hdp + d / 2];
      if (d & 1)
        *byte = (uint8_t)((*byte & 0x0fu) | (uint8_t)(code << 4));
      else
        *byte = (uint8_t)((*byte & 0xf0u) | (uint8_t)code);
    }
  }

  /* V: per token, per GS-channel group. */
  for (int32_t t = 0; t < GS; ++t) {
    const int64_t phys = block_table[first_logical_page + t / P];
    const int32_t slot = t % P;
    for (int32_t cg = 0; cg < hdg; ++cg) {
      const int32_t d0 = cg * GS;
      float mn = kivi_f16_to_f32(v_rows[t][d0]);
      float mx = mn;
      for (int32_t c = 1; c < GS; ++c) {
        const float x = kivi_f16_to_f32(v_rows[t][d0 + c]);
        mn = min_num(mn, x);
        mx = max_num(mx, x);
      }
      float scale = (mx - mn) / 15.0f;
      if (!(scale > 0.0f)) scale = 1.0f;
      const int64_t pidx = ((phys * NKV + h) * P + slot) * hdg + cg;
      v_scale[pidx] = kivi_f32_to_f16(scale);
      v_zero[pidx] = kivi_f32_to_f16(mn);
      for (int32_t c = 0; c < GS; c += 2) {
        const int32_t c0 = clamp_code((kivi_f16_to_f32(v_rows[t][d0 + c]) - mn) / scale);
        const int32_t c1 = clamp_code((kivi_f16_to_f32(v_rows[t][d0 + c + 1]) - mn) / scale);
        v_code[((phys * NKV + h) * P + slot) * hdp + (d0 + c) / 2] =
            (uint8_t)((c0 & 0x0f) | ((c1 & 0x0f) << 4));
      }
    }
  }
}

/* Pack the group held in scratch rows [0, group) of every kv head. */
static void pack_from_scratch(const kivi_geo* g, const uint16_t* k_scr, const uint16_t* v_scr,
                              const int32_t* block_table, int32_t logical_group,
                              uint8_t* k_code, uint16_t* k_scale, uint16_t* k_zero,
                              uint8_t* v_code, uint16_t* v_scale, uint16_t* v_zero) {
  const int32_t RS = scratch_rows(g), HD = g->hd, GS = g->group;
  const uint16_t** kr = (const uint16_t**)malloc(sizeof(void*) * (size_t)GS);
  const uint16_t** vr = (const uint16_t**)malloc(sizeof(void*) * (size_t)GS);
  for (int32_t h = 0; h < g->nkv; ++h) {
    for (int32_t t = 0; t < GS; ++t) {
      kr[t] = k_scr + ((int64_t)h * RS + t) * HD;
      vr[t] = v_scr + ((int64_t)h * RS + t) * HD;
    }
    kivi_ref_pack_group(g, h, kr, vr, block_table, logical_group, k_code, k_scale, k_zero,
                        v_code, v_scale, v_zero);
  }
  free(kr);
  free(vr);
}

/* shift_scratch_after_age_out_kernel, source_patch.py:1635-1648:
 * scratch[h, r] <- scratch[h, r + group] for r < residual_len, forward order. */
static void shift_scratch(const kivi_geo* g, uint16_t* scr, int32_t residual_len) {
  const int32_t RS = scratch_rows(g), HD = g->hd;
  for (int32_t h = 0; h < g->nkv; ++h)
    for (int32_t r = 0; r < residual_len; ++r)
      memmove(scr + ((int64_t)h * RS + r) * HD, scr + ((int64_t)h * RS + r + g->group) * HD,
              sizeof(uint16_t) * (size_t)HD);
}

/* ---- kivi_cache_write_launch, source_patch.py:1661-1697 ---- */

void kivi_ref_cache_write(const kivi_geo* g, uint8_t* k_code, uint16_t* k_scale,
                          uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                          uint16_t* v_zero, uint16_t* k_scr, uint16_t* v_scr,
                          const uint16_t* new_k, const uint16_t* new_v,
                          const int32_t* block_table, int32_t seq_len) {
  const int32_t R = g->residual, GS = g->group, RS = scratch_rows(g), HD = g->hd;
  const int32_t prev_seq_len = seq_len - 1;
  const int32_t prev_old = kivi_split_old_tokens(prev_seq_len, R, GS);
  const int32_t next_old = kivi_split_old_tokens(seq_len, R, GS);
  const int32_t prev_res = prev_seq_len - prev_old;
  const int32_t next_res = seq_len - next_old;
  /* append_scratch_token_kernel, :1622-1633 */
  for (int32_t h = 0; h < g->nkv; ++h) {
    memcpy(k_scr + ((int64_t)h * RS + prev_res) * HD, new_k + (int64_t)h * HD, 2 * (size_t)HD);
    memcpy(v_scr + ((int64_t)h * RS + prev_res) * HD, new_v + (int64_t)h * HD, 2 * (size_t)HD);
  }
  if (next_old > prev_old) {
    pack_from_scratch(g, k_scr, v_scr, block_table, prev_old / GS, k_code, k_scale, k_zero,
                      v_code, v_scale, v_zero);
    shift_scratch(g, k_scr, next_res);
    shift_scratch(g, v_scr, next_res);
  }
}

/* ---- kivi_cache_write_batched_launch, source_patch.py:1705-1775 ---- */

int32_t kivi_ref_cache_write_batched(const kivi_geo* g, uint8_t* k_code, uint16_t* k_scale,
                                     uint16_t* k_zero, uint8_t* v_code, uint16_t* v_scale,
                                     uint16_t* v_zero, uint16_t* k_scr, uint16_t* v_scr,
                                     const uint16_t* new_k, const uint16_t* new_v,
                                     const int32_t* block_table, int32_t start_seq_len,
                                     int32_t num_new) {
  const int32_t R = g->residual, GS = g->group, RS = scratch_rows(g), HD = g->hd;
  const int32_t prev_old = kivi_split_old_tokens(start_seq_len, R, GS);
  const int32_t prev_res = start_seq_len - prev_old;
  const int32_t end = start_seq_len + num_new;
  const int32_t next_old = kivi_split_old_tokens(end, R, GS);
  const int32_t next_res = end - next_old;
  if (num_new < 1 || prev_res + num_new > RS || next_old - prev_old > GS) return -1;
  /* append_scratch_tokens_batched_kernel, :1705-1719 (token-major input) */
  for (int32_t tok = 0; tok < num_new; ++tok)
    for (int32_t h = 0; h < g->nkv; ++h) {
      memcpy(k_scr + ((int64_t)h * RS + prev_res + tok) * HD,
             new_k + ((int64_t)tok * g->nkv + h) * HD, 2 * (size_t)HD);
      memcpy(v_scr + ((int64_t)h * RS + prev_res + tok) * HD,
             new_v + ((int64_t)tok * g->nkv + h) * HD, 2 * (size_t)HD);
    }
  if (next_old > prev_old) {
    pack_from_scratch(g, k_scr, v_scr, block_table, prev_old / GS, k_code, k_scale, k_zero,
                      v_code, v_scale, v_zero);
    shift_scratch(g, k_scr, next_res);
    shift_scratch(g, v_scr, next_res);
  }
  return 0;
}

/* ---- plan_batched_write, source_patch.py:504-553 ---- */

int32_t kivi_ref_plan_batched_write(int32_t start_seq_len, int32_t num_new,
                                    int32_t residual, int32_t group,
                                    kivi_subchunk* out, int32_t cap) {
  if (start_seq_len < 0) return -1;
  if (num_new < 1) return -2;
  if (residual <= 0 || group <= 0) return -3;
  const int32_t capacity = residual + group;
  int32_t n = 0, seq_len = start_seq_len, remaining = num_new;
  while (remaining > 0) {
    const int32_t prev_old = kivi_split_old_tokens(seq_len, residual, group);
    const int32_t prev_res = seq_len - prev_old;
    const int32_t room = capacity - prev_res;
    const int32_t take = remaining < room ? remaining : room;
    if (take <= 0) return -5; /* planning invariant violated */
    const int32_t new_len = seq_len + take;
    const int32_t next_old = kivi_split_old_tokens(new_len, residual, group);
    if (n >= cap) return -4;
    out[n].start_seq_len = seq_len;
    out[n].num_new = take;
    out[n].scratch_start = prev_res;
    if (next_old > prev_old) {
      out[n].age_out_page = prev_old / group;
      out[n].post_shift_residual_len = new_len - next_old;
    } else {
      out[n].age_out_page = -1;
      out[n].post_shift_residual_len = -1;
    }
    ++n;
    seq_len = new_len;
    remaining -= take;
  }
  return n;
}

/* ---- decode ---- */

/* Window bounds of snapshot :74-83 at runtime geometry.  LQ = old-token
 * capacity of the block table rounded down to whole groups. */
static void decode_window(const kivi_geo* g, int32_t seq_len, int32_t* old_valid,
                          int32_t* residual_valid) {
  const int32_t R = g->residual, GS = g->group;
  const int32_t lq = ((g->max_pages * g->page) / GS) * GS;
  int32_t bounded = seq_len;
  if (bounded < 0) bounded = 0;
  if (bounded > lq + R) bounded = lq + R;
  int32_t quantizable = bounded - R;
  if (quantizable < 0) quantizable = 0;
  int32_t ov = (quantizable / GS) * GS;
  if (ov > lq) ov = lq;
  int32_t rv = bounded - ov;
  if (rv < 0) rv = 0;
  if (rv > R + GS) rv = R + GS;
  *old_valid = ov;
  *residual_valid = rv;
}

/* Dequantise token s of kv head h into k[HD], v[HD] (fp32, as kivi4_unpack4,
 * snapshot :35-40: float(code) * float(scale) + float(zero)). */
static void load_token(const kivi_geo* g, int32_t h, const int32_t* block_table,
                       const uint8_t* k_code, const uint16_t* k_scale, const uint16_t* k_zero,
                       const uint8_t* v_code, const uint16_t* v_scale, const uint16_t* v_zero,
                       const uint16_t* k_scr, const uint16_t* v_scr, int32_t old_valid,
                       int32_t s, float* k, float* v) {
  const int32_t HD = g->hd, P = g->page, GS = g->group, NKV = g->nkv, RS = scratch_rows(g);
  const int32_t hdp = HD / 2, hdg = HD / GS;
  if (s < old_valid) {
    const int64_t phys = block_table[s / P];
    const int64_t kparam_page = block_table[(s / GS) * (GS / P)]; /* group's first page */
    const int32_t slot = s % P;
    const uint8_t* kc = k_code + ((phys * NKV + h) * P + slot) * hdp;
    const uint8_t* vc = v_code + ((phys * NKV + h) * P + slot) * hdp;
    const uint16_t* ks = k_scale + (kparam_page * NKV + h) * HD;
    const uint16_t* kz = k_zero + (kparam_page * NKV + h) * HD;
    const int64_t vpi = ((phys * NKV + h) * P + slot) * hdg;
    for (int32_t d = 0; d < HD; ++d) {
      const int32_t kq = (kc[d / 2] >> ((d & 1) * 4)) & 0xf;
      const int32_t vq = (vc[d / 2] >> ((d & 1) * 4)) & 0xf;
      k[d] = (float)kq * kivi_f16_to_f32(ks[d]) + kivi_f16_to_f32(kz[d]);
      v[d] = (float)vq * kivi_f16_to_f32(v_scale[vpi + d / GS]) +
             kivi_f16_to_f32(v_zero[vpi + d / GS]);
    }
  } else {
    const int32_t r = s - old_valid;
    for (int32_t d = 0; d < HD; ++d) {
      k[d] = kivi_f16_to_f32(k_scr[((int64_t)h * RS + r) * HD + d]);
      v[d] = kivi_f16_to_f32(v_scr[((int64_t)h * RS + r) * HD + d]);
    }
  }
}

/* Online softmax over tokens [t0, t1) for the G query heads of kv head h.
 * m, l [G]; acc [G][HD].  snapshot :85-156. */
static void online_range(const kivi_geo* g, int32_t h, const float* qf, const int32_t* bt,
                         const uint8_t* k_code, const uint16_t* k_scale, const uint16_t* k_zero,
                         const uint8_t* v_code, const uint16_t* v_scale, const uint16_t* v_zero,
                         const uint16_t* k_scr, const uint16_t* v_scr, int32_t old_valid,
                         int32_t t0, int32_t t1, float* m, float* l, float* acc, float* k,
                         float* v) {
  const int32_t HD = g->hd, G = g->nh / g->nkv;
  const float scale_attn = 1.0f / sqrtf((float)HD);
  for (int32_t s = t0; s < t1; ++s) {
    load_token(g, h, bt, k_code, k_scale, k_zero, v_code, v_scale, v_zero, k_scr, v_scr,
               old_valid, s, k, v);
    for (int32_t gi = 0; gi < G; ++gi) {
      const float* qh = qf + (int64_t)(h * G + gi) * HD;
      float dot = 0.0f;
      for (int32_t d = 0; d < HD; ++d) dot += qh[d] * k[d];
      const float score = dot * scale_attn;
      const float m_new = fmaxf(m[gi], score);
      const float corr = expf(m[gi] - m_new);
      const float p = expf(score - m_new);
      l[gi] = l[gi] * corr + p;
      float* a = acc + (int64_t)gi * HD;
      for (int32_t d = 0; d < HD; ++d) a[d] = a[d] * corr + p * v[d];
      m[gi] = m_new;
    }
  }
}

static void decode_kv_head(const kivi_geo* g, int32_t h, const uint16_t* q, const int32_t* bt,
                           const uint8_t* k_code, const uint16_t* k_scale,
                           const uint16_t* k_zero, const uint8_t* v_code,
                           const uint16_t* v_scale, const uint16_t* v_zero,
                           const uint16_t* k_scr, const uint16_t* v_scr, int32_t ov,
                           int32_t rv, float* out) {
  const int32_t HD = g->hd, G = g->nh / g->nkv;
  float* qf = (float*)malloc(sizeof(float) * (size_t)g->nh * HD);
  float* m = (float*)malloc(sizeof(float) * (size_t)G);
  float* l = (float*)malloc(sizeof(float) * (size_t)G);
  float* acc = (float*)calloc((size_t)G * HD, sizeof(float));
  float* k = (float*)malloc(sizeof(float) * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * (size_t)HD);
  for (int32_t i = h * G * HD; i < (h + 1) * G * HD; ++i) qf[i] = kivi_f16_to_f32(q[i]);
  for (int32_t gi = 0; gi < G; ++gi) {
    m[gi] = -1.0e30f;
    l[gi] = 0.0f;
  }
  online_range(g, h, qf, bt, k_code, k_scale, k_zero, v_code, v_scale, v_zero, k_scr, v_scr, ov,
               0, ov + rv, m, l, acc, k, v);
  for (int32_t gi = 0; gi < G; ++gi) {
    const float inv_l = 1.0f / fmaxf(l[gi], 1.0e-30f);
    for (int32_t d = 0; d < HD; ++d) out[(int64_t)(h * G + gi) * HD + d] = acc[gi * HD + d] * inv_l;
  }
  free(qf);
  free(m);
  free(l);
  free(acc);
  free(k);
  free(v);
}

void kivi_ref_decode_online(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                            const uint8_t* k_code, const uint16_t* k_scale,
                            const uint16_t* k_zero, const uint8_t* v_code,
                            const uint16_t* v_scale, const uint16_t* v_zero,
                            const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                            float* out) {
  int32_t ov, rv;
  decode_window(g, seq_len, &ov, &rv);
  for (int32_t h = 0; h < g->nkv; ++h)
    decode_kv_head(g, h, q, block_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero,
                   k_scr, v_scr, ov, rv, out);
}

static void twopass_window(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                           const uint8_t* k_code, const uint16_t* k_scale,
                           const uint16_t* k_zero, const uint8_t* v_code,
                           const uint16_t* v_scale, const uint16_t* v_zero,
                           const uint16_t* k_scr, const uint16_t* v_scr, int32_t ov, int32_t rv,
                           double* out) {
  const int32_t HD = g->hd, G = g->nh / g->nkv;
  const int32_t n = ov + rv;
  float* k = (float*)malloc(sizeof(float) * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * (size_t)HD);
  double* kd = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1) * HD);
  double* vd = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1) * HD);
  double* sc = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  const double scale_attn = 1.0 / sqrt((double)HD);
  for (int32_t h = 0; h < g->nkv; ++h) {
    /* gather + dequantise (exact products in double) */
    for (int32_t s = 0; s < n; ++s) {
      if (s < ov) {
        const int64_t phys = block_table[s / g->page];
        const int64_t kp = block_table[(s / g->group) * (g->group / g->page)];
        const int32_t slot = s % g->page;
        const int32_t hdp = HD / 2, hdg = HD / g->group;
        const uint8_t* kc = k_code + ((phys * g->nkv + h) * g->page + slot) * hdp;
        const uint8_t* vc = v_code + ((phys * g->nkv + h) * g->page + slot) * hdp;
        const int64_t vpi = ((phys * g->nkv + h) * g->page + slot) * hdg;
        for (int32_t d = 0; d < HD; ++d) {
          const int32_t kq = (kc[d / 2] >> ((d & 1) * 4)) & 0xf;
          const int32_t vq = (vc[d / 2] >> ((d & 1) * 4)) & 0xf;
          kd[(int64_t)s * HD + d] =
              (double)kq * (double)kivi_f16_to_f32(k_scale[(kp * g->nkv + h) * HD + d]) +
              (double)kivi_f16_to_f32(k_zero[(kp * g->nkv + h) * HD + d]);
          vd[(int64_t)s * HD + d] =
              (double)vq * (double)kivi_f16_to_f32(v_scale[vpi + d / g->group]) +
              (double)kivi_f16_to_f32(v_zero[vpi + d / g->group]);
        }
      } else {
        load_token(g, h, block_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero, k_scr,
                   v_scr, ov, s, k, v);
        for (int32_t d = 0; d < HD; ++d) {
          kd[(int64_t)s * HD + d] = k[d];
          vd[(int64_t)s * HD + d] = v[d];
        }
      }
    }
    for (int32_t gi = 0; gi < G; ++gi) {
      const uint16_t* qh = q + (int64_t)(h * G + gi) * HD;
      double mx = -INFINITY;
      for (int32_t s = 0; s < n; ++s) { /* pass 1: scores and max */
        double dot = 0.0;
        for (int32_t d = 0; d < HD; ++d) dot += (double)kivi_f16_to_f32(qh[d]) * kd[(int64_t)s * HD + d];
        sc[s] = dot * scale_attn;
        if (sc[s] > mx) mx = sc[s];
      }
      double den = 0.0;
      for (int32_t s = 0; s < n; ++s) {
        sc[s] = exp(sc[s] - mx);
        den += sc[s];
      }
      double* o = out + (int64_t)(h * G + gi) * HD;
      for (int32_t d = 0; d < HD; ++d) { /* pass 2: normalised weights times V */
        double a = 0.0;
        for (int32_t s = 0; s < n; ++s) a += sc[s] * vd[(int64_t)s * HD + d];
        o[d] = n > 0 ? a / den : 0.0;
      }
    }
  }
  free(k);
  free(v);
  free(kd);
  free(vd);
  free(sc);
}

void kivi_ref_decode_twopass(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                             const uint8_t* k_code, const uint16_t* k_scale,
                             const uint16_t* k_zero, const uint8_t* v_code,
                             const uint16_t* v_scale, const uint16_t* v_zero,
                             const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                             double* out) {
  int32_t ov, rv;
  decode_window(g, seq_len, &ov, &rv);
  twopass_window(g, q, block_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero, k_scr,
                 v_scr, ov, rv, out);
}

/* ---- sparse-retained decode, variants.rs:2620-2740 ---- */

/* Window of variants.rs:2667-2680: the old tokens are the first
 * num_retained_pages entries of the compact table, clamped to [0, dense old
 * pages] and to the table width (whole groups at page 16); the residual rows
 * keep the dense SEQ_LEN boundary, so evicted pages are skipped and never read
 * as residual tokens. */
static void sparse_window(const kivi_geo* g, int32_t seq_len, int32_t num_retained_pages,
                          int32_t* old_valid, int32_t* residual_valid) {
  int32_t dense_ov;
  decode_window(g, seq_len, &dense_ov, residual_valid);
  int32_t pages = num_retained_pages < 0 ? 0 : num_retained_pages;
  const int32_t dense_pages = dense_ov / g->page;
  if (pages > dense_pages) pages = dense_pages;
  if (pages > g->max_pages) pages = g->max_pages;
  *old_valid = (pages * g->page / g->group) * g->group;
}

void kivi_ref_decode_sparse_retained(const kivi_geo* g, const uint16_t* q,
                                     const int32_t* retained_table, const uint8_t* k_code,
                                     const uint16_t* k_scale, const uint16_t* k_zero,
                                     const uint8_t* v_code, const uint16_t* v_scale,
                                     const uint16_t* v_zero, const uint16_t* k_scr,
                                     const uint16_t* v_scr, int32_t seq_len,
                                     int32_t num_retained_pages, float* out) {
  int32_t ov, rv;
  sparse_window(g, seq_len, num_retained_pages, &ov, &rv);
  for (int32_t h = 0; h < g->nkv; ++h)
    decode_kv_head(g, h, q, retained_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero,
                   k_scr, v_scr, ov, rv, out);
}

void kivi_ref_decode_sparse_retained_twopass(const kivi_geo* g, const uint16_t* q,
                                             const int32_t* retained_table,
                                             const uint8_t* k_code, const uint16_t* k_scale,
                                             const uint16_t* k_zero, const uint8_t* v_code,
                                             const uint16_t* v_scale, const uint16_t* v_zero,
                                             const uint16_t* k_scr, const uint16_t* v_scr,
                                             int32_t seq_len, int32_t num_retained_pages,
                                             double* out) {
  int32_t ov, rv;
  sparse_window(g, seq_len, num_retained_pages, &ov, &rv);
  twopass_window(g, q, retained_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero, k_scr,
                 v_scr, ov, rv, out);
}

void kivi_ref_decode_batch(const kivi_geo* g, const uint16_t* q, const int32_t* seq_lens,
                           const int32_t* block_tables, const uint8_t* k_code,
                           const uint16_t* k_scale, const uint16_t* k_zero,
                           const uint8_t* v_code, const uint16_t* v_scale,
                           const uint16_t* v_zero, const uint16_t* k_scr,
                           const uint16_t* v_scr, int32_t batch, float* out,
                           int32_t nthreads) {
  const int64_t scr_seq = (int64_t)g->nkv * scratch_rows(g) * g->hd;
  const int64_t qo_seq = (int64_t)g->nh * g->hd;
  const int32_t work = batch * g->nkv;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#else
  (void)nthreads;
#endif
  for (int32_t w = 0; w < work; ++w) {
    const int32_t b = w / g->nkv, h = w % g->nkv;
    int32_t ov, rv;
    decode_window(g, seq_lens[b], &ov, &rv);
    decode_kv_head(g, h, q + b * qo_seq, block_tables + (int64_t)b * g->max_pages, k_code,
                   k_scale, k_zero, v_code, v_scale, v_zero, k_scr + b * scr_seq,
                   v_scr + b * scr_seq, ov, rv, out + b * qo_seq);
  }
}

/* ---- split-K LSE merge, variants.rs:3548-3565 ---- */

void kivi_ref_lse_merge(int32_t nsplit, int32_t hd, const float* m, const float* l,
                        const float* acc, float* out) {
  float gm = -1.0e30f;
  for (int32_t w = 0; w < nsplit; ++w) gm = fmaxf(gm, m[w]);
  float gl = 0.0f;
  for (int32_t d = 0; d < hd; ++d) out[d] = 0.0f;
  for (int32_t w = 0; w < nsplit; ++w) {
    const float corr = expf(m[w] - gm);
    gl += l[w] * corr;
    for (int32_t d = 0; d < hd; ++d) out[d] += acc[(int64_t)w * hd + d] * corr;
  }
  const float inv_l = 1.0f / fmaxf(gl, 1.0e-30f);
  for (int32_t d = 0; d < hd; ++d) out[d] *= inv_l;
}

void kivi_ref_decode_splitk(const kivi_geo* g, const uint16_t* q, const int32_t* block_table,
                            const uint8_t* k_code, const uint16_t* k_scale,
                            const uint16_t* k_zero, const uint8_t* v_code,
                            const uint16_t* v_scale, const uint16_t* v_zero,
                            const uint16_t* k_scr, const uint16_t* v_scr, int32_t seq_len,
                            int32_t chunk, float* out) {
  const int32_t HD = g->hd, G = g->nh / g->nkv;
  int32_t ov, rv;
  decode_window(g, seq_len, &ov, &rv);
  const int32_t n = ov + rv;
  const int32_t ns = n > 0 ? (n + chunk - 1) / chunk : 1;
  float* qf = (float*)malloc(sizeof(float) * (size_t)g->nh * HD);
  float* m = (float*)malloc(sizeof(float) * (size_t)ns * G);
  float* l = (float*)malloc(sizeof(float) * (size_t)ns * G);
  float* acc = (float*)calloc((size_t)ns * G * HD, sizeof(float));
  float* k = (float*)malloc(sizeof(float) * (size_t)HD);
  float* v = (float*)malloc(sizeof(float) * (size_t)HD);
  float* pm = (float*)malloc(sizeof(float) * (size_t)ns);
  float* pl = (float*)malloc(sizeof(float) * (size_t)ns);
  float* pa = (float*)malloc(sizeof(float) * (size_t)ns * HD);
  for (int32_t i = 0; i < g->nh * HD; ++i) qf[i] = kivi_f16_to_f32(q[i]);
  for (int32_t h = 0; h < g->nkv; ++h) {
    for (int32_t c = 0; c < ns; ++c) {
      for (int32_t gi = 0; gi < G; ++gi) {
        m[c * G + gi] = -1.0e30f;
        l[c * G + gi] = 0.0f;
      }
      memset(acc + (int64_t)c * G * HD, 0, sizeof(float) * (size_t)G * HD);
      const int32_t t0 = c * chunk, t1 = (c + 1) * chunk < n ? (c + 1) * chunk : n;
      online_range(g, h, qf, block_table, k_code, k_scale, k_zero, v_code, v_scale, v_zero,
                   k_scr, v_scr, ov, t0, t1, m + c * G, l + c * G, acc + (int64_t)c * G * HD, k,
                   v);
    }
    for (int32_t gi = 0; gi < G; ++gi) {
      for (int32_t c = 0; c < ns; ++c) {
        pm[c] = m[c * G + gi];
        pl[c] = l[c * G + gi];
        memcpy(pa + (int64_t)c * HD, acc + ((int64_t)c * G + gi) * HD, sizeof(float) * (size_t)HD);
      }
      kivi_ref_lse_merge(ns, HD, pm, pl, pa, out + (int64_t)(h * G + gi) * HD);
    }
  }
  free(qf);
  free(m);
  free(l);
  free(acc);
  free(k);
  free(v);
  free(pm);
  free(pl);
  free(pa);
}

/* ---- check_block_table_width, source_patch.py:692-707 ---- */

int32_t kivi_ref_required_pages(int32_t seq_len, int32_t residual, int32_t group,
                                int32_t page, int32_t max_seq_len) {
  if (seq_len < 1 || seq_len > max_seq_len) return -1;
  /* pages that hold whole aged groups; with page == group == 32 this is the
   * reference's (seq_len - RESIDUAL) / BLOCK_SIZE */
  return kivi_split_old_tokens(seq_len, residual, group) / page;
}
