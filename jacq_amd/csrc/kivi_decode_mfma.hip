// kivi_decode_mfma.hip -- paged int4-KIVI decode attention on CDNA4 matrix cores.
//
// One workgroup (4 waves) owns one split of one (sequence, kv head): a run of
// whole 32-token groups.  The G query heads of the kv head form the 16-wide
// N (QK) / M (PV) side of v_mfma_f32_16x16x32_f16 tiles, so each KV byte is
// read from HBM once per step for all G heads (the reference reads it G
// times, decode_attention_kivi_paged_library_flash.cu:51-60).  Waves take
// groups round-robin, keep their own online-softmax state, and merge in LDS;
// splits of a sequence merge through the workspace, the last split to finish
// doing the log-sum-exp combine (variants.rs:3548-3565) -- one launch total.
//
// Per 32-token group and wave (lane l: c = l % 16, j = l / 16):
//   QK^T   S^T[t, g] = sum_d K[t, d] Q[g, d]   (M = tokens, N = heads, K = d)
//          K = code * s_d + z_d is never dequantised: the A operand holds the
//          codes as exact fp16 (1024 + c, or 1024 + 16c, made by OR-ing a nibble
//          into the exponent field 0x6400), the B operand holds q_gd * s_d
//          (an fp16 hi + lo pair, rebuilt per group because K scales are per
//          group), and the
//          accumulator starts from sum_d q_gd z_d - 1024 sum_d B_gd, which two
//          more MFMAs against broadcast operands compute.
//   softmax  in registers: lane (c, j) holds S for head g = c and tokens
//          8j..8j+7 -- exactly the A-operand layout PV needs for P, so P never
//          leaves registers.  Rescaling is lazy (only when a head's running max
//          grows by more than 2^8).
//   PV     O[g, ch] = sum_t P[g, t] V[t, ch]  (M = heads, N = channels, K = t)
//          lane c owns channels CPL*c .. CPL*c+CPL-1 (one V scale group), so
//          V = code * s_t + z_t is dequantised in packed fp16 with the per-
//          token scale, and sum_t P z_t accumulates in one extra MFMA per group.
#include <type_traits>

#include "kivi_kernels.h"

namespace jacq {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMfmaThreads = 256;
constexpr int kWaves = kMfmaThreads / 64;
constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)
constexpr float kRescaleThreshold = 8.0f;  // log2 units

__device__ inline floatx4 mfma(half8_t a, half8_t b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline half8_t as_h8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }
__device__ inline u32x4 as_u4(half8_t v) { return __builtin_bit_cast(u32x4, v); }
__device__ inline half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ inline uint32_t as_u(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// 8 int4 codes of one dword (channel k at bits 4k..4k+3) -> A operand of one
// k-step in the order [c0, c4, c1, c5, c2, c6, c3, c7]; odd channels carry a
// factor 16 (nibble left in bits 4..7 of the mantissa).
__device__ inline u32x4 unpack_codes(uint32_t x) {
  const uint32_t x8 = x >> 8;
  u32x4 r;
  r[0] = (x & 0x000F000Fu) | kMagic;
  r[1] = (x & 0x00F000F0u) | kMagic;
  r[2] = (x8 & 0x000F000Fu) | kMagic;
  r[3] = (x8 & 0x00F000F0u) | kMagic;
  return r;
}

// Natural fp16 pairs (v0,v1),(v2,v3),(v4,v5),(v6,v7) -> the unpack order above.
__device__ inline u32x4 perm_pairs(u32x4 d) {
  u32x4 r;
  r[0] = (d[0] & 0xFFFFu) | (d[2] << 16);
  r[1] = (d[0] >> 16) | (d[2] & 0xFFFF0000u);
  r[2] = (d[1] & 0xFFFFu) | (d[3] << 16);
  r[3] = (d[1] >> 16) | (d[3] & 0xFFFF0000u);
  return r;
}

template <int HD>
struct Cfg {
  static constexpr int KS = HD / 32;       // k-steps of the QK^T product
  static constexpr int CPL = HD / 16;      // V channels per lane = PV N-tiles
  static constexpr int HDP = HD / 2;       // packed bytes per token row
  static constexpr int HDG = HD / kGroup;  // V scale groups per token
  static constexpr int KCB = HD / 8;       // K code bytes per lane per token
};

template <int HD>
struct WaveState {
  floatx4 o[Cfg<HD>::CPL];  // O tiles: lane holds O[4j+i][CPL*c + nt]
  floatx4 ob;               // sum_t P z_t: applies to every channel of lane c
  float m;                  // running max (log2 domain) of head c
  float l;                  // this lane's share of the running denominator
};

template <int HD>
__device__ inline void rescale(WaveState<HD>& st, float corr) {
  // corr of head c lives in lanes c, c+16, ...; O rows are heads 4j+i.
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4;
  float ci[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ci[i] = __shfl(corr, 4 * j + i, 64);
#pragma unroll
  for (int nt = 0; nt < Cfg<HD>::CPL; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) st.o[nt][i] *= ci[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) st.ob[i] *= ci[i];
  st.l *= corr;
}

// Online-softmax update of one 32-token tile pair; s[tt][i] are log2-domain
// scores of tokens 8j + 4tt + i for head c.  Returns P as the PV A operand.
template <int HD>
__device__ inline half8_t softmax_tile(WaveState<HD>& st, floatx4 s0, floatx4 s1) {
  float mx = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                   fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const bool grow = mx > st.m + kRescaleThreshold;
  if (__builtin_amdgcn_ballot_w64(grow)) {
    const float m_new = fmaxf(st.m, mx);
    const float corr = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
    rescale<HD>(st, corr);
  }
  float p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = __builtin_amdgcn_exp2f(s0[i] - st.m);
    p[4 + i] = __builtin_amdgcn_exp2f(s1[i] - st.m);
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

// 4 codes (a: byte k of tokens 2q, b: byte k of token 2q+1) -> fp16 pairs of
// the low / high nibble (value 1024 + c / 1024 + 16c).
__device__ inline uint32_t byte_pair(uint32_t a, uint32_t b, int k) {
  return ((a >> (8 * k)) & 0xFFu) | (((b >> (8 * k)) & 0xFFu) << 16);
}

constexpr int kMaxSplitPages = 256;  // split_plan keeps a split within 4096 tokens
constexpr int kMaxCombineSplits = 64;  // the host rejects geometries needing more

// Raw bytes of one quantised 32-token group as one lane loads them; filled
// one group ahead of the compute so two groups are in flight per wave.
template <int HD>
struct Stage {
  typedef typename std::conditional<HD == 128, u32x4, u32x2>::type kvec;
  typedef typename std::conditional<HD == 128, u32x2, uint32_t>::type pvec;
  kvec kc[2];      // K codes of row c of tiles 0/1, channels j*HD/4 ..
  uint32_t vc[8];  // V codes of rows 8j..8j+7, channels CPL*c ..
  pvec ksz;        // K scale (lanes < 32) / zero (lanes >= 32), channels (HD/32)*(lane%32) ..
  pvec vsz;        // V scale / zero of token lane%32, all HD/32 channel groups
};

template <int HD>
__device__ inline void load_stage(Stage<HD>& st, const DecodeArgs& a, const int* pages,
                                  int first_lp, int t0, int h, int nkv, int P, int lane) {
  using C = Cfg<HD>;
  using S = Stage<HD>;
  const int c = lane & 15, j = lane >> 4;
  auto token_row = [&](int tok) -> int64_t {  // (phys page, kv head, slot) row index
    const int phys = pages[tok / P - first_lp];
    return ((int64_t)phys * nkv + h) * P + (tok % P);
  };
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tok = t0 + 8 * (c >> 2) + 4 * tt + (c & 3);
    st.kc[tt] = *(const typename S::kvec*)(a.k_code + token_row(tok) * C::HDP + j * C::KCB);
  }
  {
    const uint8_t* base = a.v_code + token_row(t0 + 8 * j) * C::HDP + c * (C::CPL / 2);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if constexpr (C::CPL == 8)
        st.vc[r] = *(const uint32_t*)(base + r * C::HDP);
      else
        st.vc[r] = *(const uint16_t*)(base + r * C::HDP);
    }
  }
  const int which = lane >> 5, t = lane & 31;
  {
    const int phys = pages[t0 / P - first_lp];  // the group's first page holds its K params
    const uint16_t* src = (which ? a.k_zero : a.k_scale) + ((int64_t)phys * nkv + h) * HD +
                          (HD / 32) * t;
    st.ksz = *(const typename S::pvec*)src;
  }
  {
    const uint16_t* src = (which ? a.v_zero : a.v_scale) + token_row(t0 + t) * C::HDG;
    st.vsz = *(const typename S::pvec*)src;
  }
}

template <int HD>
__global__ __launch_bounds__(kMfmaThreads) void kivi_decode_mfma_kernel(KiviGeo g, DecodeArgs a) {
  using C = Cfg<HD>;
  constexpr int KS = C::KS, CPL = C::CPL, HDP = C::HDP, HDG = C::HDG;
  // per-wave V scale/zero staging [wave][s|z][group][token] and the merge area
  __shared__ __attribute__((aligned(16))) uint16_t vsz_s[kWaves][2][HDG][kGroup];
  __shared__ __attribute__((aligned(16))) uint16_t ksz_s[kWaves][2][HD];
  __shared__ int pages_s[kMaxSplitPages];
  __shared__ float m_s[kWaves][16], l_s[kWaves][16];
  __shared__ float o_s[kWaves][16][HD + 4];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, j = lane >> 4;
  const int G = g.gqa, P = g.page, NKV = g.nkv;

  int ov, rv;
  decode_window(g, a.seq_lens ? a.seq_lens[b] : a.seq_len, &ov, &rv);
  const int n = ov + rv;
  int nsplit, chunk;
  split_plan(n, &nsplit, &chunk);
  if (split >= nsplit) return;
  const int t_begin = split * chunk;
  const int t_end = min(n, t_begin + chunk);

  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
  const uint16_t* qh = a.q + (int64_t)b * a.q_stride + (int64_t)h * G * HD;

  // B operands of Q: natural order (bias / residual tiles) and the unpack
  // order with odd channels divided by 16 (quantised tiles).  Lane (c, j)
  // covers channels j*HD/4 + 8*ks + e of head c.
  half8_t qn[KS], qp[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (c < G) v = *(const u32x4*)(qh + c * HD + j * (HD / 4) + 8 * ks);
    qn[ks] = as_h8(v);
    half8_t pp = as_h8(perm_pairs(v));
    const half8_t div = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f,
                         (_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f};
    qp[ks] = pp * div;
  }
  const half8_t neg1024 = {(_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                           (_Float16)-1024.f, (_Float16)-1024.f, (_Float16)-1024.f,
                           (_Float16)-1024.f, (_Float16)-1024.f};
  const float sscale = 1.4426950408889634f / __builtin_sqrtf((float)HD);  // log2(e)/sqrt(HD)

  WaveState<HD> st;
#pragma unroll
  for (int nt = 0; nt < CPL; ++nt) st.o[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.ob = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -1.0e30f;
  st.l = 0.0f;

  // ---------------- quantised groups ----------------
  // physical pages of this split's old tokens, once per workgroup
  const int old_end = min(t_end, ov);
  const int first_lp = t_begin / P;
  if (t_begin < old_end) {
    const int np = (old_end - 1) / P - first_lp + 1;
    for (int i = tid; i < np; i += kMfmaThreads) pages_s[i] = bt[first_lp + i];
  }
  __syncthreads();

  Stage<HD> cur, nxt;
  int t0 = t_begin + wave * kGroup;
  if (t0 < old_end) load_stage<HD>(cur, a, pages_s, first_lp, t0, h, NKV, P, lane);
  for (; t0 < old_end; t0 += kWaves * kGroup) {
    const int t1 = t0 + kWaves * kGroup;
    if (t1 < old_end) load_stage<HD>(nxt, a, pages_s, first_lp, t1, h, NKV, P, lane);
    // stage this group's scales / zeros through LDS
    {
      const int t = lane & 31, which = lane >> 5;
      *(typename Stage<HD>::pvec*)&ksz_s[wave][which][(HD / 32) * t] = cur.ksz;
      if constexpr (HDG == 4) {
        vsz_s[wave][which][0][t] = (uint16_t)cur.vsz[0];
        vsz_s[wave][which][1][t] = (uint16_t)(cur.vsz[0] >> 16);
        vsz_s[wave][which][2][t] = (uint16_t)cur.vsz[1];
        vsz_s[wave][which][3][t] = (uint16_t)(cur.vsz[1] >> 16);
      } else {
        vsz_s[wave][which][0][t] = (uint16_t)cur.vsz;
        vsz_s[wave][which][1][t] = (uint16_t)(cur.vsz >> 16);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();
    u32x4 ksv[KS], kzv[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      ksv[ks] = *(const u32x4*)&ksz_s[wave][0][j * (HD / 4) + 8 * ks];
      kzv[ks] = *(const u32x4*)&ksz_s[wave][1][j * (HD / 4) + 8 * ks];
    }
    const auto& kc = cur.kc;
    const auto& vc = cur.vc;

    // ---- S^T = K Q^T, accumulator seeded with the per-head bias ----
    // B = q*s as an unevaluated fp16 sum hi + lo (lo = fma(q, s, -hi) is the
    // rounding error of hi), so the QK^T product keeps ~22 bits.
    half8_t qs[KS], ql[KS];
    floatx4 bias = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const half8_t sp = as_h8(perm_pairs(ksv[ks]));
      qs[ks] = qp[ks] * sp;
      ql[ks] = __builtin_elementwise_fma(qp[ks], sp, -qs[ks]);
      bias = mfma(as_h8(kzv[ks]), qn[ks], bias);  // sum_d z_d q_gd
      bias = mfma(neg1024, qs[ks], bias);          // -1024 sum_d B_gd
      bias = mfma(neg1024, ql[ks], bias);
    }
    floatx4 s[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      s[tt] = bias;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8_t x = as_h8(unpack_codes(kc[tt][ks]));
        s[tt] = mfma(x, qs[ks], s[tt]);
        s[tt] = mfma(x, ql[ks], s[tt]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) s[tt][i] *= sscale;
    }
    const half8_t pa = softmax_tile<HD>(st, s[0], s[1]);

    // ---- V dequant (packed fp16) and PV ----
    const int vg = (CPL * c) / kGroup;
    const u32x4 vs4 = *(const u32x4*)&vsz_s[wave][0][vg][8 * j];
    const u32x4 vz4 = *(const u32x4*)&vsz_s[wave][1][vg][8 * j];
    st.ob = mfma(pa, as_h8(vz4), st.ob);
    u32x4 s_lo, s_hi, n_lo, n_hi;
    {
      const half8_t sv = as_h8(vs4);
      const half8_t c16 = {(_Float16)0.0625f, (_Float16)0.0625f, (_Float16)0.0625f,
                           (_Float16)0.0625f, (_Float16)0.0625f, (_Float16)0.0625f,
                           (_Float16)0.0625f, (_Float16)0.0625f};
      const half8_t sh = sv * c16;
      s_lo = as_u4(sv);
      s_hi = as_u4(sh);
      n_lo = as_u4(sv * neg1024);
      n_hi = as_u4(sh * neg1024);
    }
    // -1024*s overflows fp16 for s >= 64: then dequantise in two steps.
    float smax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) smax = fmaxf(smax, __builtin_fabsf((float)as_h8(vs4)[e]));
    const bool big = __builtin_amdgcn_ballot_w64(!(smax < 64.0f)) != 0;
#pragma unroll
    for (int k = 0; k < CPL / 2; ++k) {
      u32x4 lo, hi;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t y = byte_pair(vc[2 * q], vc[2 * q + 1], k);
        const uint32_t xl = (y & 0x000F000Fu) | kMagic;
        const uint32_t xh = (y & 0x00F000F0u) | kMagic;
        if (!big) {
          lo[q] = as_u(__builtin_elementwise_fma(as_h2(xl), as_h2(s_lo[q]), as_h2(n_lo[q])));
          hi[q] = as_u(__builtin_elementwise_fma(as_h2(xh), as_h2(s_hi[q]), as_h2(n_hi[q])));
        } else {
          const half2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
          lo[q] = as_u((as_h2(xl) + m1024) * as_h2(s_lo[q]));
          hi[q] = as_u((as_h2(xh) + m1024) * as_h2(s_hi[q]));
        }
      }
      st.o[2 * k] = mfma(pa, as_h8(lo), st.o[2 * k]);
      st.o[2 * k + 1] = mfma(pa, as_h8(hi), st.o[2 * k + 1]);
    }
    __builtin_amdgcn_wave_barrier();  // LDS reads above precede the next group's writes
    cur = nxt;
  }

  // ---------------- fp16 residual tiles ----------------
  const int res_begin = max(t_begin, ov);
  for (int t0 = res_begin + wave * kGroup; t0 < t_end; t0 += kWaves * kGroup) {
    const int tn = min(kGroup, t_end - t0);
    const int r0 = t0 - ov;  // scratch row of token t0
    const uint16_t* kscr = a.k_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
    const uint16_t* vscr = a.v_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
    floatx4 s[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tl = 8 * (c >> 2) + 4 * tt + (c & 3);
      s[tt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u32x4 kv = {0u, 0u, 0u, 0u};
        if (tl < tn) kv = *(const u32x4*)(kscr + (int64_t)(r0 + tl) * HD + j * (HD / 4) + 8 * ks);
        s[tt] = mfma(as_h8(kv), qn[ks], s[tt]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 8 * j + 4 * tt + i;
        s[tt][i] = tok < tn ? s[tt][i] * sscale : -INFINITY;
      }
    }
    const half8_t pa = softmax_tile<HD>(st, s[0], s[1]);
    // V rows 8j..8j+7, channels CPL*c.. : fp16 values straight from scratch
    uint32_t vr[8][CPL / 2];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int tl = 8 * j + r;
#pragma unroll
      for (int w = 0; w < CPL / 2; ++w) vr[r][w] = 0u;
      if (tl < tn) {
        const uint32_t* src = (const uint32_t*)(vscr + (int64_t)(r0 + tl) * HD + CPL * c);
#pragma unroll
        for (int w = 0; w < CPL / 2; ++w) vr[r][w] = src[w];
      }
    }
#pragma unroll
    for (int nt = 0; nt < CPL; ++nt) {
      u32x4 vb;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t va = vr[2 * q][nt >> 1], vb2 = vr[2 * q + 1][nt >> 1];
        vb[q] = (nt & 1) ? ((va >> 16) | (vb2 & 0xFFFF0000u)) : ((va & 0xFFFFu) | (vb2 << 16));
      }
      st.o[nt] = mfma(pa, as_h8(vb), st.o[nt]);
    }
  }

  // ---------------- merge the 4 waves in LDS ----------------
  float lsum = st.l;
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (j == 0) {
    m_s[wave][c] = st.m;
    l_s[wave][c] = lsum;
  }
#pragma unroll
  for (int nt = 0; nt < CPL; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) o_s[wave][4 * j + i][CPL * c + nt] = st.o[nt][i] + st.ob[i];
  __syncthreads();

  const int64_t slot0 = ((int64_t)b * NKV + h) * a.max_splits;
  for (int e = tid; e < G * HD; e += kMfmaThreads) {
    const int gi = e / HD, d = e % HD;
    float M = m_s[0][gi];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, m_s[w][gi]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(m_s[w][gi] - M);
      L += l_s[w][gi] * f;
      acc += o_s[w][gi][d] * f;
    }
    if (nsplit == 1) {
      a.out[(int64_t)b * a.out_stride + ((int64_t)h * G + gi) * HD + d] = acc / fmaxf(L, 1.0e-30f);
    } else {
      a.ws_acc[((slot0 + split) * G + gi) * HD + d] = acc;
      if (d == 0) {
        a.ws_ml[((slot0 + split) * G + gi) * 2] = M;
        a.ws_ml[((slot0 + split) * G + gi) * 2 + 1] = L;
      }
    }
  }
}

// LSE merge of the split partials (variants.rs:3548-3565), one workgroup per
// (kv head, sequence).  A separate launch: the kernel boundary makes every
// split's partials visible across the GPU's L2 slices without device-scope
// fences inside the decode kernel.
__global__ __launch_bounds__(kMfmaThreads) void kivi_combine_mfma_kernel(KiviGeo g, DecodeArgs a) {
  __shared__ float w_s[kMaxCombineSplits][16];
  __shared__ float l_s[kMaxCombineSplits][16];
  __shared__ float inv_s[16];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int G = g.gqa, HD = g.hd;
  int ov, rv;
  decode_window(g, a.seq_lens ? a.seq_lens[b] : a.seq_len, &ov, &rv);
  int nsplit, chunk;
  split_plan(ov + rv, &nsplit, &chunk);
  if (nsplit <= 1) return;  // the decode kernel wrote O directly
  const int64_t slot0 = ((int64_t)b * g.nkv + h) * a.max_splits;
  for (int e = tid; e < nsplit * G; e += kMfmaThreads) {
    const int sp = e / G, gi = e % G;
    w_s[sp][gi] = a.ws_ml[((slot0 + sp) * G + gi) * 2];
    l_s[sp][gi] = a.ws_ml[((slot0 + sp) * G + gi) * 2 + 1];
  }
  __syncthreads();
  if (tid < G) {
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, w_s[sp][tid]);
    float L = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float f = __builtin_amdgcn_exp2f(w_s[sp][tid] - M);
      w_s[sp][tid] = f;
      L += l_s[sp][tid] * f;
    }
    inv_s[tid] = 1.0f / fmaxf(L, 1.0e-30f);
  }
  __syncthreads();
  const int64_t stride = (int64_t)G * HD;
  for (int e = tid; e < G * HD; e += kMfmaThreads) {
    const int gi = e / HD, d = e % HD;
    const float* src = a.ws_acc + (slot0 * G + gi) * HD + d;
    float acc = 0.f;
    int sp = 0;
    for (; sp + 4 <= nsplit; sp += 4) {  // four independent loads in flight
      const float x0 = src[(sp + 0) * stride], x1 = src[(sp + 1) * stride];
      const float x2 = src[(sp + 2) * stride], x3 = src[(sp + 3) * stride];
      acc += x0 * w_s[sp][gi] + x1 * w_s[sp + 1][gi] + x2 * w_s[sp + 2][gi] +
             x3 * w_s[sp + 3][gi];
    }
    for (; sp < nsplit; ++sp) acc += src[sp * stride] * w_s[sp][gi];
    a.out[(int64_t)b * a.out_stride + ((int64_t)h * G + gi) * HD + d] = acc * inv_s[gi];
  }
}

hipError_t launch_decode_mfma(const KiviGeo& g, const DecodeArgs& a, int batch,
                              hipStream_t stream) {
  const dim3 grid(a.max_splits, g.nkv, batch);
  if (g.hd == 128)
    hipLaunchKernelGGL(kivi_decode_mfma_kernel<128>, grid, dim3(kMfmaThreads), 0, stream, g, a);
  else
    hipLaunchKernelGGL(kivi_decode_mfma_kernel<64>, grid, dim3(kMfmaThreads), 0, stream, g, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.max_splits <= 1) return e;
  hipLaunchKernelGGL(kivi_combine_mfma_kernel, dim3(g.nkv, batch), dim3(kMfmaThreads), 0, stream,
                     g, a);
  return hipGetLastError();
}

}  // namespace jacq
