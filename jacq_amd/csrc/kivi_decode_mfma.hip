// kivi_decode_mfma.hip -- paged int4-KIVI decode attention on CDNA4 matrix cores.
//
// Work decomposition ("stream" split-K).  Every (sequence, kv head) is a
// stream of 32-token tiles (its quantised groups, then its fp16 residual
// tokens); the streams of the whole batch are concatenated and cut into one
// equal contiguous run per wavefront.  A wavefront therefore does the same
// amount of work as every other one whatever the context-length mix, stays
// resident for its whole run (no per-split prologue), and prefetches the next
// tile's block-table entries (scalar loads) and bytes while it computes the
// current one.  A run that covers a whole (sequence, kv head) writes O
// directly; otherwise it leaves an online-softmax partial (m, l, acc) that
// kivi_combine_stream_kernel merges with the log-sum-exp rule of the
// reference's split-K decode (crates/jac-codegen-cuda/src/variants.rs:3548-3565).
//
// All G query heads of a kv head share each tile: they form the 16-wide N
// (QK) / M (PV) side of v_mfma_f32_16x16x32_f16 tiles, so every KV byte is
// read from HBM once per step (the reference reads it G times, one warp per
// query head, decode_attention_kivi_paged_library_flash.cu:51-60).
//
// Per 32-token group (lane l: c = l % 16, j = l / 16):
//   QK^T   S^T[t, g] = sum_d K[t, d] Q[g, d]   (M = tokens, N = heads, K = d)
//          K = code * s_d + z_d is never dequantised: the A operand holds the
//          codes as exact fp16 (1024 + c, or 1024 + 16c, made by OR-ing a nibble
//          into the mantissa of 0x6400), the B operand holds q_gd * s_d as an
//          fp16 hi + lo pair (rebuilt per group: K scales are per group), and
//          sum_d q_gd z_d - 1024 sum_d B_gd -- a per-head constant -- comes
//          from three more MFMAs against broadcast operands.
//   softmax  in registers: lane (c, j) holds S for head c and tokens
//          8j..8j+7 -- exactly the A-operand layout PV needs for P, so P never
//          leaves registers.  Rescaling is lazy (only when a head's running max
//          grows by more than 2^8).
//   PV     O[g, ch] = sum_t P[g, t] V[t, ch]  (M = heads, N = channels, K = t)
//          lane c owns channels CPL*c .. CPL*c+CPL-1 (one V scale group), so
//          V = code * s_t + z_t is dequantised with one packed-fp16 FMA per
//          two values, and sum_t P z_t accumulates in one extra MFMA per group.
#include <type_traits>

#include "kivi_kernels.h"

namespace jacq {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kRescaleThreshold = 8.0f;  // log2 units

__device__ inline floatx4 mfma(half8_t a, half8_t b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline half8_t as_h8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }
__device__ inline u32x4 as_u4(half8_t v) { return __builtin_bit_cast(u32x4, v); }
__device__ inline half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ inline uint32_t as_u(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Bit constants of the nibble -> fp16 conversion, held in registers so that
// mask-and-merge is one v_and_or_b32 (VOP3 takes no literal operands here).
struct Nibble {
  uint32_t lo;      // 0x000F000F (SGPR)
  uint32_t hi;      // 0x00F000F0 (SGPR)
  uint32_t magic;   // 0x64006400, the fp16 pair (1024, 1024) (VGPR)
  uint32_t sel[4];  // v_perm selectors: byte k of two dwords -> bytes 0 and 2
  __device__ Nibble() {
    asm("s_mov_b32 %0, 0xf000f" : "=s"(lo));
    asm("s_mov_b32 %0, 0xf000f0" : "=s"(hi));
    asm("v_mov_b32 %0, 0x64006400" : "=v"(magic));
#pragma unroll
    for (int k = 0; k < 4; ++k)
      sel[k] = (uint32_t)k | 0x0C00u | ((uint32_t)(4 + k) << 16) | 0x0C000000u;
  }
};

// 8 int4 codes of one dword (channel k at bits 4k..4k+3) -> A operand of one
// k-step in the order [c0, c4, c1, c5, c2, c6, c3, c7]; odd channels carry a
// factor 16 (their nibble sits in bits 4..7 of the mantissa).
__device__ inline u32x4 unpack_codes(uint32_t x, const Nibble& nb) {
  const uint32_t x8 = x >> 8;
  u32x4 r;
  r[0] = (x & nb.lo) | nb.magic;
  r[1] = (x & nb.hi) | nb.magic;
  r[2] = (x8 & nb.lo) | nb.magic;
  r[3] = (x8 & nb.hi) | nb.magic;
  return r;
}

// Natural fp16 pairs (v0,v1),(v2,v3),(v4,v5),(v6,v7) -> the unpack order above.
__device__ inline u32x4 perm_pairs(u32x4 d) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
  return r;
}

// True when both fp16 values of a pair have magnitude below 64.
__device__ inline bool small_pair(uint32_t v) {
  return (v & 0x7FFFu) < 0x5400u && ((v >> 16) & 0x7FFFu) < 0x5400u;
}

template <int HD, int P>
struct Cfg {
  static constexpr int KS = HD / 32;       // k-steps of the QK^T product
  static constexpr int CPL = HD / 16;      // V channels per lane = PV N-tiles
  static constexpr int HDP = HD / 2;       // packed bytes per token row
  static constexpr int HDG = HD / kGroup;  // V scale groups per token
  static constexpr int KCB = HD / 8;       // K code bytes per lane per token
  static constexpr int PPG = kGroup / P;   // pages per 32-token group
  typedef typename std::conditional<HD == 128, u32x4, u32x2>::type kvec;
  typedef typename std::conditional<HD == 128, u32x2, uint32_t>::type pvec;
};

// Per-lane offsets inside a 32-token group, fixed for the whole kernel.
struct LaneMap {
  int kpg[2], koff[2];  // K tile tt: page within the group, byte offset in the page
  int vpg, voff;        // V rows 8j..8j+7: page within the group, byte offset
  int spg, soff;        // V scale/zero of token lane%32: page within the group, element offset
  int ksoff;            // K scale/zero: element offset in the page's row
};

template <int HD, int P>
__device__ inline LaneMap lane_map(int lane) {
  using C = Cfg<HD, P>;
  const int c = lane & 15, j = lane >> 4, t = lane & 31;
  LaneMap m;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tau = 8 * (c >> 2) + 4 * tt + (c & 3);  // token of MFMA row c in tile tt
    m.kpg[tt] = tau / P;
    m.koff[tt] = (tau % P) * C::HDP + j * C::KCB;
  }
  m.vpg = (8 * j) / P;
  m.voff = ((8 * j) % P) * C::HDP + c * (C::CPL / 2);
  m.spg = t / P;
  m.soff = (t % P) * C::HDG;
  m.ksoff = (HD / 32) * t;
  return m;
}

// One quantised 32-token group in flight.  The K and V codes go straight
// from global memory to this wave's LDS buffer (global_load_lds), each lane
// loading exactly the bytes it later feeds to the MFMAs, so the reads back
// are contiguous per lane; the scale / zero words travel in registers.
template <int HD, int P>
struct Stage {
  typename Cfg<HD, P>::pvec ksz;  // K scale (lanes < 32) / zero (lanes >= 32)
  typename Cfg<HD, P>::pvec vsz;  // V scale / zero of token lane%32, every channel group
};

// LDS image of one group's codes: [tile][lane] K bytes, [row][lane] V bytes.
// global_load_lds places lane i's data at byte 16*i for 16-byte loads and at
// byte 4*i for loads of 4 bytes or fewer.
template <int HD>
struct CodeBuf {
  uint8_t k[2][64 * (HD / 8)];
  uint8_t v[8][64 * 4];
};

struct StageBases {  // per-lane pointers with the kv head folded in
  const uint8_t* kcode;
  const uint8_t* vcode;
  const uint16_t* ksz;  // k_scale or k_zero by lane half
  const uint16_t* vsz;  // v_scale or v_zero by lane half
  uint32_t code_page;   // bytes per physical page of K or V codes (all kv heads)
  uint32_t vsz_page;    // elements per physical page of V scales
  uint32_t ksz_page;    // elements per physical page of K scales
};

typedef const __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

template <int HD, int P>
__device__ inline void load_stage(Stage<HD, P>& st, CodeBuf<HD>* buf, const StageBases& sb,
                                  const LaneMap& lm, uint32_t p0, uint32_t p1) {
  using C = Cfg<HD, P>;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint32_t phys = lm.kpg[tt] ? p1 : p0;
    const uint8_t* src = sb.kcode + (uint64_t)phys * sb.code_page + lm.koff[tt];
    if constexpr (HD == 128) {
      __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)buf->k[tt], 16, 0, 0);
    } else {
      __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)buf->k[tt], 4, 0, 0);
      __builtin_amdgcn_global_load_lds((gptr_t)(src + 4), (lptr_t)(buf->k[tt] + 256), 4, 0, 0);
    }
  }
  {
    const uint32_t phys = lm.vpg ? p1 : p0;
    const uint8_t* base = sb.vcode + (uint64_t)phys * sb.code_page + lm.voff;
#pragma unroll
    for (int r = 0; r < 8; ++r)
      __builtin_amdgcn_global_load_lds((gptr_t)(base + r * C::HDP), (lptr_t)buf->v[r],
                                       C::CPL / 2, 0, 0);
  }
  st.ksz = *(const typename C::pvec*)(sb.ksz + (uint64_t)p0 * sb.ksz_page + lm.ksoff);
  const uint32_t sphys = lm.spg ? p1 : p0;
  st.vsz = *(const typename C::pvec*)(sb.vsz + (uint64_t)sphys * sb.vsz_page + lm.soff);
}

template <int HD>
struct WaveState {
  floatx4 o[HD / 16];  // O tiles: lane holds O[4j+i][CPL*c + nt]
  floatx4 ob;          // sum_t P z_t: applies to every channel of lane c
  float m;             // running max (log2 domain) of head c
  float l;             // this lane's share of the running denominator
};

template <int HD>
__device__ inline void rescale(WaveState<HD>& st, float corr, int j) {
  // corr of head c lives in lanes c, c+16, ...; O rows are heads 4j+i.
  float ci[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ci[i] = __shfl(corr, 4 * j + i, 64);
#pragma unroll
  for (int nt = 0; nt < HD / 16; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) st.o[nt][i] *= ci[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) st.ob[i] *= ci[i];
  st.l *= corr;
}

// Online-softmax update for raw scores s[tt][i] of tokens 8j + 4tt + i and
// head c; the log2-domain score is fma(s, kscale, kbias).  Returns P as the
// PV A operand.
template <int HD>
__device__ inline half8_t softmax_tile(WaveState<HD>& st, floatx4 s0, floatx4 s1, float kscale,
                                       float kbias, int j) {
  const float raw = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                          fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
  float mx = __builtin_fmaf(raw, kscale, kbias);
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (__builtin_amdgcn_ballot_w64(mx > st.m + kRescaleThreshold)) {
    const float m_new = fmaxf(st.m, mx);
    const float corr = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
    rescale<HD>(st, corr, j);
  }
  const float off = kbias - st.m;
  float p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], kscale, off));
    p[4 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], kscale, off));
  }
  half8_t pa;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    sum += p[i];
    pa[i] = (_Float16)p[i];
  }
  st.l += sum;
  return pa;
}

// Dequantise the lane's V channels CPL*c + 2k (low nibbles) and + 2k + 1
// (high nibbles) for its 8 tokens and accumulate PV.  kBig: some |scale| >= 64,
// where -1024 * scale overflows fp16; then the offset is removed with an
// exact subtraction first.
template <int HD, bool kBig>
__device__ inline void pv_group(WaveState<HD>& st, half8_t pa, const uint32_t* vc, u32x4 vs4,
                                const Nibble& nb) {
  constexpr int CPL = HD / 16;
  const half8_t sv = as_h8(vs4);
  const half8_t inv16 = {(_Float16)0.0625f, (_Float16)0.0625f, (_Float16)0.0625f,
                         (_Float16)0.0625f, (_Float16)0.0625f, (_Float16)0.0625f,
                         (_Float16)0.0625f, (_Float16)0.0625f};
  const half8_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                         (_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                         (_Float16)-1024.f, (_Float16)-1024.f};
  const u32x4 s_lo = vs4;
  const u32x4 s_hi = as_u4(sv * inv16);
  u32x4 n_lo = {0u, 0u, 0u, 0u}, n_hi = {0u, 0u, 0u, 0u};
  if constexpr (!kBig) {
    n_lo = as_u4(sv * m1024);           // -1024 s, exact
    n_hi = as_u4(as_h8(s_hi) * m1024);  // -64 s, exact
  }
  const half2_t m1024_2 = {(_Float16)-1024.f, (_Float16)-1024.f};
#pragma unroll
  for (int k = 0; k < CPL / 2; ++k) {
    u32x4 lo, hi;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t y = __builtin_amdgcn_perm(vc[2 * q + 1], vc[2 * q], nb.sel[k]);
      const uint32_t xl = (y & nb.lo) | nb.magic;  // (1024 + c, 1024 + c')
      const uint32_t xh = (y & nb.hi) | nb.magic;  // (1024 + 16c, 1024 + 16c')
      if constexpr (!kBig) {
        lo[q] = as_u(__builtin_elementwise_fma(as_h2(xl), as_h2(s_lo[q]), as_h2(n_lo[q])));
        hi[q] = as_u(__builtin_elementwise_fma(as_h2(xh), as_h2(s_hi[q]), as_h2(n_hi[q])));
      } else {
        lo[q] = as_u((as_h2(xl) + m1024_2) * as_h2(s_lo[q]));
        hi[q] = as_u((as_h2(xh) + m1024_2) * as_h2(s_hi[q]));
      }
    }
    st.o[2 * k] = mfma(pa, as_h8(lo), st.o[2 * k]);
    st.o[2 * k + 1] = mfma(pa, as_h8(hi), st.o[2 * k + 1]);
  }
}

// Everything one (sequence, kv head) needs while its tiles are processed.
template <int HD>
struct SegCtx {
  half8_t qn[HD / 32];  // B operand of Q, natural channel order (bias, residual tiles)
  half8_t qp[HD / 32];  // B operand of Q in the unpack order, odd channels / 16
};

// One quantised 32-token group: QK^T, online softmax, PV.
template <int HD, int P>
__device__ inline void group_compute(WaveState<HD>& st, const SegCtx<HD>& q, const Stage<HD, P>& cur,
                                     const CodeBuf<HD>* buf, uint16_t (*ksz_s)[HD],
                                     uint16_t (*vsz_s)[HD / kGroup][kGroup], const LaneMap& lm,
                                     const Nibble& nb, float sscale, int lane) {
  using C = Cfg<HD, P>;
  constexpr int KS = C::KS, CPL = C::CPL, HDG = C::HDG;
  const int c = lane & 15, j = lane >> 4, which = lane >> 5, t32 = lane & 31;
  const half8_t neg1024 = {(_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                           (_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                           (_Float16)-1024.f, (_Float16)-1024.f};
  // scales / zeros through LDS into the operand layouts
  *(typename C::pvec*)&ksz_s[which][lm.ksoff] = cur.ksz;
  if constexpr (HDG == 4) {
    vsz_s[which][0][t32] = (uint16_t)cur.vsz[0];
    vsz_s[which][1][t32] = (uint16_t)(cur.vsz[0] >> 16);
    vsz_s[which][2][t32] = (uint16_t)cur.vsz[1];
    vsz_s[which][3][t32] = (uint16_t)(cur.vsz[1] >> 16);
  } else {
    vsz_s[which][0][t32] = (uint16_t)cur.vsz;
    vsz_s[which][1][t32] = (uint16_t)(cur.vsz >> 16);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
  __builtin_amdgcn_wave_barrier();
  typename C::kvec kc[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    if constexpr (HD == 128) {
      kc[tt] = *(const u32x4*)&buf->k[tt][16 * lane];
    } else {
      kc[tt][0] = *(const uint32_t*)&buf->k[tt][4 * lane];
      kc[tt][1] = *(const uint32_t*)&buf->k[tt][256 + 4 * lane];
    }
  }
  uint32_t vc[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if constexpr (CPL == 8)
      vc[r] = *(const uint32_t*)&buf->v[r][4 * lane];
    else
      vc[r] = *(const uint16_t*)&buf->v[r][4 * lane];
  }

  // ---- S^T = K Q^T; B = q*s as fp16 hi + lo (lo = fma(q, s, -hi)) ----
  floatx4 bias = {0.f, 0.f, 0.f, 0.f}, s0 = bias, s1 = bias;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 sv = *(const u32x4*)&ksz_s[0][j * (HD / 4) + 8 * ks];
    const u32x4 zv = *(const u32x4*)&ksz_s[1][j * (HD / 4) + 8 * ks];
    const half8_t sp = as_h8(perm_pairs(sv));
    const half8_t qs = q.qp[ks] * sp;
    const half8_t ql = __builtin_elementwise_fma(q.qp[ks], sp, -qs);
    bias = mfma(as_h8(zv), q.qn[ks], bias);  // sum_d z_d q_gd
    bias = mfma(neg1024, qs, bias);           // -1024 sum_d B_gd
    bias = mfma(neg1024, ql, bias);
    const half8_t x0 = as_h8(unpack_codes(kc[0][ks], nb));
    const half8_t x1 = as_h8(unpack_codes(kc[1][ks], nb));
    s0 = mfma(x0, qs, s0);
    s1 = mfma(x1, qs, s1);
    s0 = mfma(x0, ql, s0);
    s1 = mfma(x1, ql, s1);
  }
  // every row of the bias tile holds the same per-head constant
  const half8_t pa = softmax_tile<HD>(st, s0, s1, sscale, bias[0] * sscale, j);

  // ---- V dequant (packed fp16) and PV ----
  const int vg = (CPL * c) / kGroup;
  const u32x4 vs4 = *(const u32x4*)&vsz_s[0][vg][8 * j];
  const u32x4 vz4 = *(const u32x4*)&vsz_s[1][vg][8 * j];
  st.ob = mfma(pa, as_h8(vz4), st.ob);
  const bool small =
      small_pair(vs4[0]) && small_pair(vs4[1]) && small_pair(vs4[2]) && small_pair(vs4[3]);
  if (__builtin_amdgcn_ballot_w64(!small) == 0)
    pv_group<HD, false>(st, pa, vc, vs4, nb);
  else
    pv_group<HD, true>(st, pa, vc, vs4, nb);
  __builtin_amdgcn_wave_barrier();  // LDS reads above precede the next group's writes
}

// Tiles of one sequence: 32-token tiles of its decode window, at least one so
// that an empty sequence still produces its (zero) output.
__device__ inline int seq_tiles(const KiviGeo& g, const DecodeArgs& a, int b, int* ov, int* n) {
  int o, r;
  decode_window(g, a.seq_lens ? a.seq_lens[b] : a.seq_len, &o, &r);
  *ov = o;
  *n = o + r;
  return max(1, (o + r + kGroup - 1) / kGroup);
}

__device__ inline int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}

// Total tiles of the concatenated streams (all sequences x kv heads).
__device__ inline int64_t stream_tiles(const KiviGeo& g, const DecodeArgs& a, int lane) {
  int64_t tot = 0;
  for (int base = 0; base < a.batch; base += 64) {
    int T = 0, ov, n;
    if (base + lane < a.batch) T = seq_tiles(g, a, base + lane, &ov, &n);
    tot += wave_sum_i(T);
  }
  return tot * g.nkv;
}

// Wavefronts that share the stream: at most gridDim.x, and at least
// kMinTilesPerWave tiles each so that tiny batches do not scatter.
constexpr int kMinTilesPerWave = 8;
__device__ inline int64_t stream_waves(int64_t tiles, int grid) {
  int64_t w = (tiles + kMinTilesPerWave - 1) / kMinTilesPerWave;
  if (w < 1) w = 1;
  return w < grid ? w : grid;
}

// Start of a sequence's stream (in tiles, times NKV) and its tile count.
struct SeqSpan {
  int b;
  int64_t start;  // global tile index of (b, kv head 0)
  int tiles;      // tiles per kv head
};

// The sequence whose streams contain global tile x.
__device__ inline SeqSpan locate(const KiviGeo& g, const DecodeArgs& a, int64_t x, int lane) {
  int64_t run = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int bb = base + lane;
    int T = 0, ov, n;
    if (bb < a.batch) T = seq_tiles(g, a, bb, &ov, &n);
    const int incl = wave_incl_scan(T, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(bb < a.batch && run + (int64_t)g.nkv * incl > x);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      const int Tf = __shfl(T, f, 64), If = __shfl(incl, f, 64);
      return {base + f, run + (int64_t)g.nkv * (If - Tf), Tf};
    }
    run += (int64_t)g.nkv * __shfl(incl, 63, 64);
  }
  return {a.batch, run, 1};
}

template <int HD, int P>
__global__ __launch_bounds__(64) void kivi_decode_stream_kernel(KiviGeo g, DecodeArgs a) {
  using C = Cfg<HD, P>;
  constexpr int KS = C::KS, CPL = C::CPL;
  __shared__ __attribute__((aligned(16))) uint16_t ksz_s[2][HD];
  __shared__ __attribute__((aligned(16))) uint16_t vsz_s[2][C::HDG][kGroup];
  __shared__ __attribute__((aligned(16))) CodeBuf<HD> bufA;
  __shared__ __attribute__((aligned(16))) CodeBuf<HD> bufB;

  const int lane = threadIdx.x, c = lane & 15, j = lane >> 4;
  const int G = g.gqa, NKV = g.nkv;
  const int64_t TT = stream_tiles(g, a, lane);
  const int64_t W = stream_waves(TT, gridDim.x);
  const int w = blockIdx.x;
  if (w >= W) return;
  const int64_t x0 = (int64_t)w * TT / W, x1 = (int64_t)(w + 1) * TT / W;
  if (x0 >= x1) return;

  const Nibble nb;
  const LaneMap lm = lane_map<HD, P>(lane);
  const float sscale = 1.4426950408889634f / __builtin_sqrtf((float)HD);  // log2(e)/sqrt(HD)
  const int which = lane >> 5;

  SeqSpan sp = locate(g, a, x0, lane);
  int kvh = (int)((x0 - sp.start) / sp.tiles);
  int t = (int)((x0 - sp.start) % sp.tiles);
  int64_t x = x0;
  while (x < x1) {
    const int b = sp.b, h = kvh;
    int ov, n;
    const int T = seq_tiles(g, a, b, &ov, &n);
    const int t_beg = t;
    const int t_fin = (int)min((int64_t)T, t + (x1 - x));

    // ---- segment setup: Q operands and softmax state ----
    SegCtx<HD> q;
    const uint16_t* qh = a.q + (int64_t)b * a.q_stride + (int64_t)h * G * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (c < G) v = *(const u32x4*)(qh + c * HD + j * (HD / 4) + 8 * ks);
      q.qn[ks] = as_h8(v);
      const half8_t div = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f,
                           (_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f};
      q.qp[ks] = as_h8(perm_pairs(v)) * div;
    }
    WaveState<HD> st;
#pragma unroll
    for (int nt = 0; nt < CPL; ++nt) st.o[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    st.ob = floatx4{0.f, 0.f, 0.f, 0.f};
    st.m = -1.0e30f;
    st.l = 0.0f;

    // ---- quantised groups, two stages in flight ----
    const int tq_end = min(t_fin, ov / kGroup);
    if (t_beg < tq_end) {
      const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
      StageBases sb;
      sb.code_page = (uint32_t)(NKV * P * C::HDP);
      sb.vsz_page = (uint32_t)(NKV * P * C::HDG);
      sb.ksz_page = (uint32_t)(NKV * HD);
      sb.kcode = a.k_code + (int64_t)h * P * C::HDP;
      sb.vcode = a.v_code + (int64_t)h * P * C::HDP;
      sb.ksz = (which ? a.k_zero : a.k_scale) + (int64_t)h * HD;
      sb.vsz = (which ? a.v_zero : a.v_scale) + (int64_t)h * P * C::HDG;
      auto page = [&](int tile, int k) -> uint32_t {
        return (uint32_t)bt[tile * C::PPG + (C::PPG == 2 ? k : 0)];
      };
      Stage<HD, P> A, B;
      load_stage<HD, P>(A, &bufA, sb, lm, page(t_beg, 0), page(t_beg, 1));
      uint32_t n0 = 0, n1 = 0;  // pages of the next group to load
      if (t_beg + 1 < tq_end) {
        n0 = page(t_beg + 1, 0);
        n1 = page(t_beg + 1, 1);
      }
      for (int i = t_beg; i < tq_end; i += 2) {
        if (i + 1 < tq_end) {
          load_stage<HD, P>(B, &bufB, sb, lm, n0, n1);
          if (i + 2 < tq_end) {
            n0 = page(i + 2, 0);
            n1 = page(i + 2, 1);
          }
        }
        group_compute<HD, P>(st, q, A, &bufA, ksz_s, vsz_s, lm, nb, sscale, lane);
        if (i + 1 >= tq_end) break;
        if (i + 2 < tq_end) {
          load_stage<HD, P>(A, &bufA, sb, lm, n0, n1);
          if (i + 3 < tq_end) {
            n0 = page(i + 3, 0);
            n1 = page(i + 3, 1);
          }
        }
        group_compute<HD, P>(st, q, B, &bufB, ksz_s, vsz_s, lm, nb, sscale, lane);
      }
    }

    // ---- fp16 residual tiles ----
    const uint16_t* kscr = a.k_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
    const uint16_t* vscr = a.v_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
    for (int i = max(t_beg, ov / kGroup); i < t_fin; ++i) {
      const int t0 = i * kGroup;
      const int tn = min(kGroup, n - t0);  // 0 only for an empty sequence
      const int r0 = t0 - ov;              // scratch row of token t0
      floatx4 s[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tl = 8 * (c >> 2) + 4 * tt + (c & 3);
        s[tt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          u32x4 kv = {0u, 0u, 0u, 0u};
          if (tl < tn)
            kv = *(const u32x4*)(kscr + (int64_t)(r0 + tl) * HD + j * (HD / 4) + 8 * ks);
          s[tt] = mfma(as_h8(kv), q.qn[ks], s[tt]);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          if (8 * j + 4 * tt + ii >= tn) s[tt][ii] = -INFINITY;
      }
      const half8_t pa = softmax_tile<HD>(st, s[0], s[1], sscale, 0.0f, j);
      // V rows 8j..8j+7, channels CPL*c.. : fp16 values straight from scratch
      uint32_t vr[8][CPL / 2];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int tl = 8 * j + r;
#pragma unroll
        for (int wd = 0; wd < CPL / 2; ++wd) vr[r][wd] = 0u;
        if (tl < tn) {
          const uint32_t* src = (const uint32_t*)(vscr + (int64_t)(r0 + tl) * HD + CPL * c);
#pragma unroll
          for (int wd = 0; wd < CPL / 2; ++wd) vr[r][wd] = src[wd];
        }
      }
#pragma unroll
      for (int nt = 0; nt < CPL; ++nt) {
        u32x4 vb;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const uint32_t va = vr[2 * qq][nt >> 1], vb2 = vr[2 * qq + 1][nt >> 1];
          vb[qq] = (nt & 1) ? __builtin_amdgcn_perm(vb2, va, 0x07060302u)
                            : __builtin_amdgcn_perm(vb2, va, 0x05040100u);
        }
        st.o[nt] = mfma(pa, as_h8(vb), st.o[nt]);
      }
    }

    // ---- segment output: O directly, or a partial for the combine kernel ----
    float lsum = st.l;
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    const bool whole = (t_beg == 0 && t_fin == T);
    const int64_t piece = (int64_t)b * NKV + h + w;
    float rowscale[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = __shfl(lsum, 4 * j + i, 64);
      rowscale[i] = whole ? 1.0f / fmaxf(li, 1.0e-30f) : 1.0f;
    }
    float* dst = whole ? a.out + (int64_t)b * a.out_stride + (int64_t)h * G * HD
                       : a.ws_acc + piece * G * HD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * j + i;
      if (row < G) {
        float v[CPL];
#pragma unroll
        for (int nt = 0; nt < CPL; ++nt) v[nt] = (st.o[nt][i] + st.ob[i]) * rowscale[i];
        float* p = dst + (int64_t)row * HD + CPL * c;
#pragma unroll
        for (int q4 = 0; q4 < CPL / 4; ++q4)
          *(floatx4*)(p + 4 * q4) = floatx4{v[4 * q4], v[4 * q4 + 1], v[4 * q4 + 2], v[4 * q4 + 3]};
      }
    }
    if (!whole && j == 0 && c < G) {
      a.ws_ml[(piece * G + c) * 2] = st.m;
      a.ws_ml[(piece * G + c) * 2 + 1] = lsum;
    }

    x += t_fin - t_beg;
    t = 0;
    if (++kvh == NKV) {
      kvh = 0;
      sp.b += 1;
    }
  }
}

// Log-sum-exp merge of the partials of one (sequence, kv head) left by the
// wavefronts whose runs cut it (variants.rs:3548-3565).  One workgroup per
// (kv head, sequence); a separate launch, so every partial is visible across
// the GPU's L2 slices without device-scope fences in the decode kernel.
__global__ __launch_bounds__(256) void kivi_combine_stream_kernel(KiviGeo g, DecodeArgs a) {
  __shared__ int64_t span_s[3];  // tiles before sequence b (x NKV), total tiles, T_b
  __shared__ float inv_s[16], mx_s[16];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int G = g.gqa, HD = g.hd, NKV = g.nkv;
  if (tid < 64) {
    const int64_t TT = stream_tiles(g, a, tid);
    int64_t before = 0;
    for (int base = 0; base < b; base += 64) {
      int T = 0, ov, n;
      if (base + tid < b) T = seq_tiles(g, a, base + tid, &ov, &n);
      before += wave_sum_i(T);
    }
    int ov, n;
    const int Tb = seq_tiles(g, a, b, &ov, &n);
    if (tid == 0) {
      span_s[0] = before * NKV;
      span_s[1] = TT;
      span_s[2] = Tb;
    }
  }
  __syncthreads();
  const int64_t TT = span_s[1], Tb = span_s[2];
  const int64_t W = stream_waves(TT, a.waves);
  const int64_t s = span_s[0] + (int64_t)h * Tb, e = s + Tb;
  auto wave_of = [&](int64_t x) -> int64_t { return ((x + 1) * W - 1) / TT; };
  const int64_t w0 = wave_of(s), w1 = wave_of(e - 1);
  if (w0 == w1) return;  // one wavefront covered it and wrote O
  const int64_t seg = (int64_t)b * NKV + h;
  if (tid < G) {
    float M = -INFINITY;
    for (int64_t w = w0; w <= w1; ++w) M = fmaxf(M, a.ws_ml[((seg + w) * G + tid) * 2]);
    float L = 0.f;
    for (int64_t w = w0; w <= w1; ++w) {
      const int64_t p = (seg + w) * G + tid;
      L += a.ws_ml[p * 2 + 1] * __builtin_amdgcn_exp2f(a.ws_ml[p * 2] - M);
    }
    mx_s[tid] = M;
    inv_s[tid] = 1.0f / fmaxf(L, 1.0e-30f);
  }
  __syncthreads();
  for (int e2 = tid; e2 < G * HD; e2 += 256) {
    const int gi = e2 / HD, d = e2 % HD;
    const float M = mx_s[gi];
    float acc = 0.f;
    for (int64_t w = w0; w <= w1; ++w) {
      const int64_t p = (seg + w) * G + gi;
      acc += a.ws_acc[p * HD + d] * __builtin_amdgcn_exp2f(a.ws_ml[p * 2] - M);
    }
    a.out[(int64_t)b * a.out_stride + ((int64_t)h * G + gi) * HD + d] = acc * inv_s[gi];
  }
}

template <int HD, int P>
static void launch_one(const KiviGeo& g, const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((kivi_decode_stream_kernel<HD, P>), dim3(a.waves), dim3(64), 0, stream, g, a);
}

hipError_t launch_decode_mfma(const KiviGeo& g, const DecodeArgs& a, int batch,
                              hipStream_t stream) {
  if (g.hd == 128 && g.page == 16)
    launch_one<128, 16>(g, a, stream);
  else if (g.hd == 128)
    launch_one<128, 32>(g, a, stream);
  else if (g.page == 16)
    launch_one<64, 16>(g, a, stream);
  else
    launch_one<64, 32>(g, a, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kivi_combine_stream_kernel, dim3(g.nkv, batch), dim3(256), 0, stream, g, a);
  return hipGetLastError();
}

int decode_stream_waves(int cus) { return cus * 8; }

}  // namespace jacq
