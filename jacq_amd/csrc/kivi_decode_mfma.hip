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
// directly; otherwise it leaves an online-softmax partial (m, l, acc) that the
// merge workgroups of the same launch combine with the log-sum-exp rule of the
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
#include <hip/hip_ext.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <random>
#include <type_traits>
#include <utility>

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

// fp32 16x16x4: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16].  Its
// i-th use over a tile takes element i of a lane's 16x16x32 f16 operand (k =
// 8 (l / 16) + i), so eight of them cover the same 32 k.
__device__ inline floatx4 mfma32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ inline half8_t as_h8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }
__device__ inline u32x4 as_u4(half8_t v) { return __builtin_bit_cast(u32x4, v); }
__device__ inline half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ inline uint32_t as_u(half2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ inline _Float16 as_f16(uint16_t v) { return __builtin_bit_cast(_Float16, v); }

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
// factor 16 (their nibble sits in bits 4..7 of the mantissa).  The codes
// enter as exact fp16 integers: (1024 + c) - 1024.  Leaving the 1024 in (and
// subtracting 1024 sum B afterwards) cancels large fp32 sums; the masked bits
// alone (c * 2^-24, subnormal) are exact too, but the matrix cores' sums of
// subnormal products over operands of mixed magnitude are off by up to ~2^-16
// relative -- either costs the scores about 1e-3 absolute, which large values
// turn into output errors above 2e-3 + 1e-2 |O|.
__device__ inline u32x4 unpack_codes(uint32_t x, const Nibble& nb) {
  const uint32_t x8 = x >> 8;
  const half2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
  u32x4 r;
  r[0] = as_u(as_h2((x & nb.lo) | nb.magic) + m1024);
  r[1] = as_u(as_h2((x & nb.hi) | nb.magic) + m1024);
  r[2] = as_u(as_h2((x8 & nb.lo) | nb.magic) + m1024);
  r[3] = as_u(as_h2((x8 & nb.hi) | nb.magic) + m1024);
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

// Token <-> MFMA position maps of a quantised group.  The QK^T A operand
// row c of tile tt holds token tok_k(tt, c); the PV K index 8j + e (lane
// quarter j, element e) is token tok_v(j, e).  They agree -- S^T row 4j + i of
// tile tt lands in lane quarter j, element 4tt + i -- so P leaves the softmax
// already in PV A-operand order.  Within a 32-lane half the 16 rows a V read
// touches alternate in parity, which keeps ds_read_b32 free of bank conflicts
// on the row-major LDS image of the codes.
__device__ constexpr int tok_k(int tt, int c) {
  return 8 * tt + 2 * (c & 3) + ((c >> 2) & 1) + 16 * (c >> 3);
}
__device__ constexpr int tok_v(int j, int e) { return 2 * e + (j & 1) + 16 * (j >> 1); }

template <int HD>
struct StageBuf {
  uint8_t k[32 * HD / 2];
  uint8_t v[32 * HD / 2];
  uint8_t s[4 * HD + 128 * (HD / kGroup)];
  uint8_t ones[128];  // fp16 1.0, written once: the row-sum lanes read it as V zeros
};

// The lanes whose column of the Sigma P z tile carries Sigma P: the last
// column of each 32-channel group (lane c covers channels CPL*c ..).
template <int HD>
__device__ inline bool sum_lane(int c) {
  constexpr int per = kGroup / (HD / 16);  // columns per V group
  return c % per == per - 1;
}

// Per-lane LDS read offsets inside a stage, fixed for the whole kernel.
struct LaneMap {
  int kread[2];  // K codes of tile tt: row tok_k(tt, c), channel block j
  int vread;     // V codes: row tok_v(j, 0), channels CPL*c..; element e adds 2e rows
  int vsread;    // V scale of (token tok_v(j, 0), group of channel CPL*c)
  int vzread;    // V zeros of the same (from the stage start); the ones block in
                 // the last lane of each group's columns, whose Sigma P z column
                 // then carries the row sum Sigma P instead
};

template <int HD, int P>
__device__ inline LaneMap lane_map(int lane) {
  using C = Cfg<HD, P>;
  const int c = lane & 15, j = lane >> 4;
  LaneMap m;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) m.kread[tt] = tok_k(tt, c) * C::HDP + j * C::KCB;
  m.vread = tok_v(j, 0) * C::HDP + c * (C::CPL / 2);
  m.vsread = 2 * (tok_v(j, 0) * C::HDG + (C::CPL * c) / kGroup);
  m.vzread = sum_lane<HD>(c) ? (int)offsetof(StageBuf<HD>, ones)
                             : (int)offsetof(StageBuf<HD>, s) + 4 * HD + m.vsread + 64 * C::HDG;
  return m;
}

// One quantised 32-token group of one kv head in LDS.  Codes keep the cache's
// row-major order (token rows of HD/2 bytes); scales and zeros arrive as
//   s[0, 2HD)        K scale of channel d at 2d
//   s[2HD, 4HD)      K zero
//   s[4HD, ..)       V scale of (token t, group g) at 2(t*HDG + g), then V zero.
// Everything comes by LDS DMA with 16 bytes per lane (global_load_lds_dwordx4
// puts lane i's bytes at 16i): an LDS DMA costs about the same issue time
// whatever its width, so a group is 2 * 32*HD/2 / 1024 + 1 of them.  The DMAs
// are issued from inline asm and waited for with explicit vmcnt counts: a
// ring of stages keeps S - 1 groups in flight while one is computed.

template <int HD>
constexpr int code_dmas() {  // 1 KiB DMAs per K or V code block
  return 32 * HD / 2 / 1024;
}

// vector memory instructions one stage issues (vmcnt units)
template <int HD>
constexpr int stage_loads() {
  return 2 * code_dmas<HD>() + 1;
}

// Per-segment DMA sources.  Codes: wave-uniform bases (kv head folded in);
// scales: the lane's own 16-byte word of page 0 and the page stride of its
// array (K scales live once per group, in its first page).
struct StageBases {
  uint64_t kc, vc;     // k_code / v_code + head offset (uniform)
  uint32_t code_page;  // bytes per physical page of K or V codes (all kv heads)
  uint64_t sc;         // lane's scale / zero source in page 0
  uint32_t sc_page;    // lane's page stride in bytes
  bool sc_p1;          // lane's word lies in the group's second page
  bool sc_on;          // lane takes part in the scale DMA
};

template <int HD, int P>
__device__ inline StageBases stage_bases(const DecodeArgs& a, int nkv, int h, int lane) {
  using C = Cfg<HD, P>;
  asm volatile("" : "+v"(lane));  // per segment, not hoisted into the whole run
  constexpr int KL = HD / 8;          // lanes per K scale (or zero) row
  constexpr int VL = 4 * C::HDG;      // lanes per V scale (or zero) block of 32 tokens
  StageBases sb;
  sb.code_page = (uint32_t)(nkv * P * C::HDP);
  sb.kc = (uint64_t)(a.k_code + (int64_t)h * P * C::HDP);
  sb.vc = (uint64_t)(a.v_code + (int64_t)h * P * C::HDP);
  sb.sc_on = lane < 2 * KL + 2 * VL;
  sb.sc_p1 = false;
  if (lane < 2 * KL) {
    const uint16_t* arr = lane < KL ? a.k_scale : a.k_zero;
    sb.sc = (uint64_t)(arr + (int64_t)h * HD + 8 * (lane % KL));
    sb.sc_page = (uint32_t)(nkv * HD * 2);
  } else {
    const int l = (lane - 2 * KL) % VL;
    const uint16_t* arr = lane < 2 * KL + VL ? a.v_scale : a.v_zero;
    const int t = 8 * l / C::HDG;  // first token of the lane's word
    sb.sc_p1 = t >= P;
    sb.sc = (uint64_t)(arr + ((int64_t)h * P + t % P) * C::HDG);
    sb.sc_page = (uint32_t)(nkv * P * C::HDG * 2);
  }
  return sb;
}

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS DMA of SZ bytes per lane from addr + OFF to LDS byte dst + lane * max(SZ, 4),
// non-temporal: every cache byte is read once per decode step, and streaming
// it past the caches sustains a markedly higher HBM read rate.
// The instruction's immediate offset moves the LDS address as well as the
// global one, so M0 gets dst - OFF.  M0 is set inside the same asm statement,
// so nothing the compiler keeps in M0 is live across it.  An LDS DMA must not
// read M0 in the instruction right after the SALU write of it (the GFX9
// M0 / LDS-DMA hazard: one wait state); the compiler's hazard recognizer does
// not look inside asm, so the s_nop is written here.
// COH: device-scope load (sc1) instead of the non-temporal hint -- for data
// another wavefront of the same launch stored with device-scope stores (the
// fused step's age-outs), which a non-temporal load could find stale in this
// XCD's L2.
template <int SZ, int OFF, bool COH = false>
__device__ inline void dma(uint64_t addr, uint32_t dst) {
  static_assert(OFF >= 0 && OFF < 4096, "global immediate offset range");
  const uint32_t m0 = dst - OFF;
  if constexpr (COH) {
    static_assert(SZ == 16, "device-scope LDS DMA: 16 bytes per lane");
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:%2 sc1"
                 :: "s"(m0), "v"(addr), "n"(OFF) : "memory", "m0");
  } else if constexpr (SZ == 16)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:%2 nt"
                 :: "s"(m0), "v"(addr), "n"(OFF) : "memory", "m0");
  else if constexpr (SZ == 4)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off offset:%2 nt"
                 :: "s"(m0), "v"(addr), "n"(OFF) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_ushort %1, off offset:%2 nt"
                 :: "s"(m0), "v"(addr), "n"(OFF) : "memory", "m0");
}

// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit lane offset.
template <int OFF, bool COH = false>
__device__ inline void dma16s(uint64_t sbase, uint32_t voff, uint32_t dst) {
  static_assert(OFF >= 0 && OFF < 4096, "global immediate offset range");
  const uint32_t m0 = dst - OFF;
  if constexpr (COH)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3 sc1"
                 :: "s"(m0), "v"(voff), "s"(sbase), "n"(OFF) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3 nt"
                 :: "s"(m0), "v"(voff), "s"(sbase), "n"(OFF) : "memory", "m0");
}

template <int N>
__device__ inline void wait_vm() {  // at most N vector memory ops outstanding
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

template <class F, int... I>
__device__ inline void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Wait until `later` stages (issued after the one about to be read) remain.
template <int L, int S>
__device__ inline void wait_stages(int later) {
  if constexpr (S >= 4) {
    if (later >= 2) {
      wait_vm<2 * L>();
      return;
    }
  }
  if (later >= 1)
    wait_vm<L>();
  else
    wait_vm<0>();
}

// LDS stages per wave: S - 1 groups in flight while one is computed.
// LDS stages and waves per SIMD of each kernel.  Two waves per SIMD do not
// hide one wave's dependency chain (LDS read, unpack, QK MFMA chain, max, exp,
// PV), so the packed HD=128 kernel (G <= 8, the common GQA shapes) runs three
// per SIMD: at most 168 VGPRs, and two 5 KiB stages per wave so that 12 waves'
// rings fit the CU's 160 KiB of LDS (one group in flight while one is
// computed: the memory latency is below a group's compute time).  The other
// kernels keep three stages; their register use already allows three waves
// (HD=64) or would spill at three (HD=128, G > 8).
template <int HD, bool PACK>
constexpr int stages() {
  return (HD == 128 && PACK) ? 2 : 3;
}
template <int HD, bool PACK>
constexpr int min_waves_per_simd() {
  return (HD == 128 && PACK) ? 3 : 1;
}

// Issue the DMAs of one group whose tokens 0..P-1 sit in page p0 and the
// rest (page size 16) in p1.
template <int HD, int P, bool COH = false>
__device__ inline void load_stage(StageBuf<HD>* buf, const StageBases& sb, uint32_t p0,
                                  uint32_t p1, int lane) {
  const uint32_t base = lds_addr(buf);
  const uint32_t kd = base + (uint32_t)offsetof(StageBuf<HD>, k);
  const uint32_t vd = base + (uint32_t)offsetof(StageBuf<HD>, v);
  const uint32_t lo = 16u * (uint32_t)lane;
  if constexpr (HD == 128) {
    // 1 KiB = 16 token rows per DMA: rows 0-15 and 16-31
    const uint64_t o0 = (uint64_t)p0 * sb.code_page;
    const uint64_t o1 = P == 16 ? (uint64_t)p1 * sb.code_page : o0 + 1024;
    dma16s<0, COH>(sb.kc + o0, lo, kd);
    dma16s<0, COH>(sb.kc + o1, lo, kd + 1024);
    dma16s<0, COH>(sb.vc + o0, lo, vd);
    dma16s<0, COH>(sb.vc + o1, lo, vd + 1024);
  } else if constexpr (P == 32) {
    const uint64_t o0 = (uint64_t)p0 * sb.code_page;
    dma16s<0, COH>(sb.kc + o0, lo, kd);
    dma16s<0, COH>(sb.vc + o0, lo, vd);
  } else {
    // one DMA spans both pages: lanes 0-31 rows 0-15 of p0, lanes 32-63 of p1
    const uint64_t o = (uint64_t)(lane < 32 ? p0 : p1) * sb.code_page + (lo & 511u);
    dma<16, 0, COH>(sb.kc + o, kd);
    dma<16, 0, COH>(sb.vc + o, vd);
  }
  const uint32_t sd = base + (uint32_t)offsetof(StageBuf<HD>, s);
  const uint64_t sa = sb.sc + (uint64_t)(sb.sc_p1 ? p1 : p0) * sb.sc_page;
  if (sb.sc_on) dma<16, 0, COH>(sa, sd);
}

// IEEE maximum (llvm.maximum): lowers to v_maximum3_f32 without the
// canonicalising moves that fmaxf needs in IEEE mode.
__device__ inline float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ inline float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// max with lane l ^ 16 / l ^ 32 by v_permlane16_swap / v_permlane32_swap
// (all VALU, no LDS round trip).  Both operands start as x; after the swap one
// holds this lane's row value and the other the partner row's.  Written as
// asm with both operands read-write: the compiler's lowering of the builtin
// reads the first result register for both results.  The s_nop gives the
// VALU write of x the wait states the swap needs.
__device__ inline float max_xor16(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return max2f(a, b);
}
__device__ inline float max_xor32(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return max2f(a, b);
}

template <int HD>
struct WaveState {
  floatx4 o[HD / 16];  // O tiles: lane holds O[4j+i][CPL*c + nt]
  floatx4 ob;          // sum_t P z_t of lane c's group; sum_t P in the sum lanes
  float m;             // running max (log2 domain) of head c
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
}

// The fp32 P of a tile whose values need the exact PV steps, parked in LDS
// in the k and v bytes of a ring slot whose contents are already in
// registers or consumed (no DMA targets the slot until the next group): kept
// in VGPRs from the softmax to the PV step it costs the common path's
// schedule.  Element i of lane l (k = 8 (l / 16) + i) sits at float 64 i + l;
// each lane reads back only what it wrote, so a one-wave workgroup needs no
// barrier.  get() takes an opaque copy of the lane's offset, so every read is
// a fresh ds_read, not a register kept live from the store.
struct PStash {
  float* base;
  __device__ explicit PStash(uint8_t* bytes) : base((float*)bytes) {}
  __device__ void put(const float (&p)[8]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) base[64 * i + threadIdx.x] = p[i];
  }
  __device__ float get(int i) const {
    int o = threadIdx.x;
    asm volatile("" : "+v"(o));
    return base[64 * i + o];
  }
};

// Online-softmax update for raw scores s[tt][i] of tokens 8j + 4tt + i and
// head c; the log2-domain score is fma(s, kscale, kbias).  Returns P as the
// fp16 PV A operand; with `precise` (wave-uniform) it also stores P in fp32
// to `stash`.
template <int HD>
__device__ inline half8_t softmax_tile(WaveState<HD>& st, floatx4 s0, floatx4 s1, float kscale,
                                       float kbias, int j, bool precise, const PStash& stash) {
  // max over the lane's 8 scores, then over the 4 lanes of head c (lanes
  // c, c+16, c+32, c+48) with the row-swap permutes (no LDS round trip)
  const float raw = max3f(max3f(s0[0], s0[1], s0[2]), max3f(s0[3], s1[0], s1[1]), max2f(s1[2], s1[3]));
  float mx = __builtin_fmaf(raw, kscale, kbias);
  mx = max_xor16(mx);
  mx = max_xor32(mx);
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
  if (__builtin_expect(precise, 0)) stash.put(p);
  half8_t pa;
#pragma unroll
  for (int i = 0; i < 8; ++i) pa[i] = (_Float16)p[i];
  return pa;
}

// V operands of one group kept in registers until its PV step: codes of rows
// tok_v(j, e), and the scale / zero pairs of the lane's channel group for
// tokens (tok_v(j, 2q), tok_v(j, 2q + 1)).
struct VData {
  uint32_t vc[8];
  u32x4 vs4, vz4;
};

template <int HD, int P>
__device__ inline VData load_v(const StageBuf<HD>* buf, const LaneMap& lm) {
  using C = Cfg<HD, P>;
  constexpr int HDG = C::HDG;
  VData d;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint8_t* vp = &buf->v[lm.vread + 2 * e * C::HDP];
    if constexpr (C::CPL == 8)
      d.vc[e] = *(const uint32_t*)vp;
    else
      d.vc[e] = *(const uint16_t*)vp;
  }
  const uint8_t* vp = &buf->s[4 * HD + lm.vsread];
  const uint8_t* zp = (const uint8_t*)buf + lm.vzread;
#pragma unroll
  for (int e = 0; e < 4; ++e) {  // pair q = e: tokens two rows apart
    const uint8_t* p0 = vp + 8 * HDG * e;
    const uint8_t* z0 = zp + 8 * HDG * e;
    // element inserts: the compiler pairs the two halves with one v_perm,
    // not a shift and an or
    half2_t sv, zv;
    sv[0] = *(const _Float16*)p0;
    sv[1] = *(const _Float16*)(p0 + 4 * HDG);
    zv[0] = *(const _Float16*)z0;
    zv[1] = *(const _Float16*)(z0 + 4 * HDG);
    d.vs4[e] = as_u(sv);
    d.vz4[e] = as_u(zv);
  }
  return d;
}

// |s| >= 64 somewhere in the wave's V scales (fp16 exponent field >= 0x15).
// The OR of the bit patterns reaches the bound whenever one value does (and,
// rarely, when none does, which only selects the slower exact arithmetic).
__device__ inline uint64_t big_scales(const VData& d) {
  const uint32_t sor = (d.vs4[0] | d.vs4[1] | d.vs4[2] | d.vs4[3]) & 0x7FFF7FFFu;
  const bool big = (sor & 0xFFFFu) >= 0x5400u || sor >= 0x54000000u;
  return __builtin_amdgcn_ballot_w64(big);  // nonzero: some lane holds a big scale
}

// The fp16 PV step rounds P and code * s to 11 bits and sums the zero-point
// terms P z apart from the P code * s terms, so a token group's error scales
// with |z| + 15 s (s >= 0), the larger of the two terms' magnitudes: up to
// 2^-11 (|z| + 15 s) in the worst case.  Groups above kFastRange get the
// exact correction (exact_fix_group), fp16 residual tiles with some |V| above
// it (their values are exact) the fp32 path; N(0,1) data, whose |z| + 15 s
// stays below ~11, never do.
constexpr float kFastRange = 16.0f;

// Some token group of the quantised group in `buf` has |z| + 15 s above
// kFastRange.  The V scales and zeros are 16 HDG dwords each (two groups per
// dword): each lane tests one of each, so the test costs two LDS reads and a
// few packed operations, not a pass over the lane's redundant copies in VData.
template <int HD>
__device__ inline bool wide_group(const StageBuf<HD>* buf, int lane) {
  constexpr int W = 16 * (HD / kGroup);  // dwords of V scales (and of zeros)
  const uint8_t* vs = &buf->s[4 * HD];
  const int o = 4 * (lane & (W - 1));
  const half2_t sc = as_h2(*(const uint32_t*)(vs + o));
  const half2_t z = as_h2(*(const uint32_t*)(vs + 4 * W + o) & 0x7FFF7FFFu);
  const half2_t k15 = {(_Float16)15.0f, (_Float16)15.0f};
  const half2_t r = __builtin_elementwise_fma(sc, k15, z);
  return __builtin_amdgcn_ballot_w64((float)r[0] > kFastRange || (float)r[1] > kFastRange) != 0;
}

// PV of one group, dequantising the lane's V channels CPL*c + 2k (low
// nibbles) and + 2k + 1 (high nibbles) for its 8 tokens.  x = 1024 + code is
// exact in fp16, so code * s = fma(x, s, -1024 s) with one rounding; the high
// nibble carries 16x and uses s / 16.  When some |s| >= 64 (`big`,
// wave-uniform) -1024 s and even code * s can leave the fp16 range.  Such a
// group always takes the exact correction (15 s > kFastRange), so the fp16
// step only has to stay finite and be repeatable: by scalar selects, with no
// branch to split the loop body, it contributes exactly zero (scales and
// offsets 0: fma(1024 + c, 0, 0)).
//
// `precise` (wave-uniform; exact_fix_group): fp32 MFMAs (16x16x4) of the
// fp32 P (from the stash `ps`) against code * s in fp32, which is exact (4 by
// 11 significant bits), and against z for the zero-point sums (the row sums
// in the sum columns); the caller adds none.  Only the fp32 products and
// sums round, about 2^-24 relative; eight MFMAs cover what one f16 MFMA does.
template <int HD>
__device__ inline void pv_group(WaveState<HD>& st, half8_t ph, const VData& d,
                                const Nibble& nb, uint64_t bigmask, bool precise,
                                const PStash& ps) {
  constexpr int CPL = HD / 16;
  if (__builtin_expect(precise, 0)) {
    // fp32 P against fp32 values: code * s is exact in fp32 (4 x 11 bits), so
    // the products carry fp32 rounding only
    const half8_t zh = as_h8(d.vz4), sh = as_h8(d.vs4);
#pragma unroll
    for (int i = 0; i < 8; ++i) st.ob = mfma32(ps.get(i), (float)zh[i], st.ob);  // sum_t P z_t
#pragma unroll
    for (int k = 0; k < CPL / 2; ++k) {
#pragma unroll
      for (int nib = 0; nib < 2; ++nib) {  // low nibbles (channel 2k), then high (2k + 1)
        floatx4& o = st.o[2 * k + nib];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t y = __builtin_amdgcn_perm(d.vc[2 * q + 1], d.vc[2 * q], nb.sel[k]);
          const half2_t x = as_h2((y & (nib ? nb.hi : nb.lo)) | nb.magic);  // 1024 + c (16c)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float sc = (float)sh[2 * q + e] * (nib ? 0.0625f : 1.0f);
            o = mfma32(ps.get(2 * q + e), ((float)x[e] - 1024.0f) * sc, o);
          }
        }
      }
    }
    return;
  }
  const half8_t sv = as_h8(d.vs4);
  // wave-uniform constants chosen by scalar selects on the ballot mask
  const bool big = bigmask != 0;
  const uint32_t fs2 = __builtin_amdgcn_readfirstlane(big ? 0u : 0x3C003C00u);   // 0 or 1
  const uint32_t fh2 = __builtin_amdgcn_readfirstlane(big ? 0u : 0x2C002C00u);   // 0 or 1/16
  const uint32_t fn2 = __builtin_amdgcn_readfirstlane(big ? 0u : 0xE400E400u);   // 0 or -1024
  const _Float16 f_s = as_h2(fs2)[0], f_h = as_h2(fh2)[0], f_n = as_h2(fn2)[0];
  const half8_t slo = sv * f_s, shi = sv * f_h;  // s, s / 16 (exact) or 0
  const u32x4 s_lo = as_u4(slo), s_hi = as_u4(shi);
  const u32x4 n_lo = as_u4(slo * f_n), n_hi = as_u4(shi * f_n);  // -1024 s (exact) or 0
  const half8_t pv = ph;
  const uint32_t magic = nb.magic;
#pragma unroll
  for (int k = 0; k < CPL / 2; ++k) {
    uint32_t xl[4], xh[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t y = __builtin_amdgcn_perm(d.vc[2 * q + 1], d.vc[2 * q], nb.sel[k]);
      xl[q] = (y & nb.lo) | magic;  // (1024 + c, 1024 + c')
      xh[q] = (y & nb.hi) | magic;  // (1024 + 16c, 1024 + 16c')
    }
    u32x4 lo, hi;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lo[q] = as_u(__builtin_elementwise_fma(as_h2(xl[q]), as_h2(s_lo[q]), as_h2(n_lo[q])));
      hi[q] = as_u(__builtin_elementwise_fma(as_h2(xh[q]), as_h2(s_hi[q]), as_h2(n_hi[q])));
    }
    st.o[2 * k] = mfma(pv, as_h8(lo), st.o[2 * k]);
    st.o[2 * k + 1] = mfma(pv, as_h8(hi), st.o[2 * k + 1]);
  }
}

// Everything one (sequence, kv head) needs while its tiles are processed.
template <int HD>
struct SegCtx {
  // B operand of Q in natural channel order (bias, residual tiles): the
  // segment's Q rows sit in the wave's LDS block; the lane's 16 bytes of k-step
  // ks at qn + 16 ks (zero rows for the columns past G).  In registers they
  // would hold 16 VGPRs through every group.
  const uint8_t* qn;
  half8_t qp[HD / 32];  // B operand of Q in the unpack order, odd channels / 16
  __device__ half8_t n(int ks) const { return *(const half8_t*)(qn + 16 * ks); }
};

// QK^T of one quantised group (already in LDS) and its online-softmax update:
// S^T = K Q^T with B = q*s as fp16 hi + lo (lo = fma(q, s, -hi)); returns P
// as the PV A operand (and stashes it in fp32 when `precise`).
struct Scores {
  floatx4 s0, s1;      // raw scores of tiles tt = 0, 1
  float kscale, kbias;  // log2-domain score = fma(s, kscale, kbias)
};

template <int HD, int P, bool PACK>
__device__ inline Scores qk_scores(const SegCtx<HD>& q, const StageBuf<HD>* buf,
                                   const LaneMap& lm, const Nibble& nb, float sscale, int lane) {
  using C = Cfg<HD, P>;
  constexpr int KS = C::KS;
  const int j = lane >> 4;
  typename C::kvec kc[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) kc[tt] = *(const typename C::kvec*)&buf->k[lm.kread[tt]];
  floatx4 bz = {0.f, 0.f, 0.f, 0.f}, s0 = bz, s1 = bz;
  if constexpr (PACK) {
    // G <= 8: columns 0-7 carry q*s (hi) of heads 0-7, columns 8-15 the
    // rounding remainder (lo) of the same heads, so one MFMA does both; a
    // row_ror:8 add merges the halves (and leaves the sum in both lanes).
    // fma(q, s, 0) = round(q * s) in the hi columns, fma(q, s, -round(q * s))
    // = the exact remainder in the lo columns
    const bool lo_col = (lane & 15) >= 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint8_t* kp = &buf->s[2 * (j * (HD / 4) + 8 * ks)];
      const u32x4 sv = *(const u32x4*)kp;
      const u32x4 zv = *(const u32x4*)(kp + 2 * HD);
      const half8_t sp = as_h8(perm_pairs(sv));
      const half8_t qs = q.qp[ks] * sp;
      const half8_t bq = __builtin_elementwise_fma(q.qp[ks], sp, lo_col ? -qs : half8_t(0));
      bz = mfma(as_h8(zv), q.n(ks), bz);  // sum_d z_d q_gd
      s0 = mfma(as_h8(unpack_codes(kc[0][ks], nb)), bq, s0);
      s1 = mfma(as_h8(unpack_codes(kc[1][ks], nb)), bq, s1);
    }
    // the score scale is applied before the hi/lo merge: a DPP add whose
    // source is an MFMA result register is miscompiled (the DPP combiner
    // reads the tuple's first register for every element), one on a VALU
    // result is not
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t0 = s0[i] * sscale, t1 = s1[i] * sscale;
      s0[i] = t0 + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                       0, __builtin_bit_cast(int, t0), 0x128, 0xF, 0xF, false));
      s1[i] = t1 + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                       0, __builtin_bit_cast(int, t1), 0x128, 0xF, 0xF, false));
    }
    return Scores{s0, s1, 1.0f, bz[0] * sscale};
  }
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const uint8_t* kp = &buf->s[2 * (j * (HD / 4) + 8 * ks)];
    const u32x4 sv = *(const u32x4*)kp;
    const u32x4 zv = *(const u32x4*)(kp + 2 * HD);
    const half8_t sp = as_h8(perm_pairs(sv));
    const half8_t qs = q.qp[ks] * sp;
    const half8_t ql = __builtin_elementwise_fma(q.qp[ks], sp, -qs);
    bz = mfma(as_h8(zv), q.n(ks), bz);  // sum_d z_d q_gd
    const half8_t x0 = as_h8(unpack_codes(kc[0][ks], nb));
    const half8_t x1 = as_h8(unpack_codes(kc[1][ks], nb));
    s0 = mfma(x0, qs, s0);
    s1 = mfma(x1, qs, s1);
    s0 = mfma(x0, ql, s0);
    s1 = mfma(x1, ql, s1);
  }
  // every row of the bias tile holds the same per-head constant
  return Scores{s0, s1, sscale, bz[0] * sscale};
}

template <int HD, int P, bool PACK>
__device__ inline half8_t qk_softmax(WaveState<HD>& st, const SegCtx<HD>& q,
                                     const StageBuf<HD>* buf, const LaneMap& lm, const Nibble& nb,
                                     float sscale, int lane) {
  const Scores sc = qk_scores<HD, P, PACK>(q, buf, lm, nb, sscale, lane);
  return softmax_tile<HD>(st, sc.s0, sc.s1, sc.kscale, sc.kbias, lane >> 4, false, PStash(nullptr));
}

// The exact correction of a quantised group whose fast PV step already ran
// with P16 = pa: the same products with -P16 take that contribution out again
// (fp16 products are exact in fp32, so this leaves only fp32 rounding), then
// P in fp32 -- from the scores recomputed off the K codes still in the slot,
// with the softmax state the fast step left -- meets fp32 values (pv_group's
// exact branch), P parked in the slot's k and v bytes (V is in registers).
template <int HD, int P, bool PACK>
__device__ inline void exact_fix_group(WaveState<HD>& st, const SegCtx<HD>& q, StageBuf<HD>* buf,
                                       const LaneMap& lm, const Nibble& nb, float sscale,
                                       int lane, half8_t pa, const VData& vd) {
  static_assert(sizeof(buf->k) + sizeof(buf->v) >= 64 * 8 * sizeof(float), "P stash");
  // HD = 128: the stash fits in the k bytes and V is read again afterwards
  // (kept in registers through the score step it would spill); HD = 64 keeps
  // V and stashes over the k and v bytes
  constexpr bool kReload = sizeof(buf->k) >= 64 * 8 * sizeof(float);
  st.ob = mfma(-pa, as_h8(vd.vz4), st.ob);
  pv_group<HD>(st, -pa, vd, nb, big_scales(vd), false, PStash(nullptr));
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const Scores sc = qk_scores<HD, P, PACK>(q, buf, lane_map<HD, P>(ln), nb, sscale, ln);
  const float off = sc.kbias - st.m;
  float p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc.s0[i], sc.kscale, off));
    p[4 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc.s1[i], sc.kscale, off));
  }
  const PStash ps(buf->k);  // after the score reads: LDS serves one wave in order
  ps.put(p);
  if constexpr (kReload) {
    int l2 = lane;
    asm volatile("" : "+v"(l2));
    pv_group<HD>(st, pa, load_v<HD, P>(buf, lane_map<HD, P>(l2)), nb, 0, true, ps);
  } else {
    pv_group<HD>(st, pa, vd, nb, 0, true, ps);
  }
}

// Tiles of one sequence: 32-token tiles of its decode window, at least one so
// that an empty sequence still produces its (zero) output.
__device__ inline int seq_tiles(const KiviGeo& g, const DecodeArgs& a, int b, int* ov, int* n) {
  int o, r;
  window_of(g, a.retained_pages,
            a.seq_lens ? ((const __attribute__((address_space(4))) int32_t*)a.seq_lens)[b]
                       : a.seq_len,
            &o, &r);
  *ov = o;
  *n = o + r;
  return max(1, (o + r + kGroup - 1) / kGroup);
}

// Work units of the stream-K split.  An fp16 residual tile moves 16 KiB per
// kv head at HD=128 with its load latency exposed, a quantised group 5 KiB
// from the LDS ring, so a residual tile weighs kResidualUnits: the split then
// gives every wavefront about the same bytes (by tile count, the waves that
// end a sequence finished last).
constexpr int kResidualUnits = 3;
__device__ inline int seq_units(const KiviGeo& g, const DecodeArgs& a, int b) {
  int ov, n;
  const int T = seq_tiles(g, a, b, &ov, &n);
  const int nq = ov / kGroup;
  return nq + kResidualUnits * (T - nq);
}
// First tile of a segment (nq quantised groups, then residual tiles) whose
// first unit is at or after unit u: the tiles owned by a unit range [u0, u1)
// are [tile_at(u0), tile_at(u1)).
__device__ inline int tile_at(int u, int nq) {
  return u <= nq ? u : nq + (u - nq + kResidualUnits - 1) / kResidualUnits;
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
__device__ inline int64_t stream_units(const KiviGeo& g, const DecodeArgs& a, int lane) {
  int64_t tot = 0;
  for (int base = 0; base < a.batch; base += 64) {
    int U = 0;
    if (base + lane < a.batch) U = seq_units(g, a, base + lane);
    tot += __builtin_amdgcn_readfirstlane(wave_sum_i(U));
  }
  return tot * g.nkv;
}

// Wavefronts that share the stream: at most the resident ones, and at least
// kMinUnitsPerWave units each, so that small batches spread over enough
// wavefronts to hide the per-group latency chain without cutting every
// segment into pieces the merge must fold (4: TinyLlama 17.9 -> 15.6 us,
// Qwen0.5B 19.6 -> 18.5 us against 8; 2 was slower at Qwen0.5B).  A whole
// call's stream of fewer than kTinyStream units (TinyLlama's 72) takes 2 per
// wavefront (0.9 us faster there; 1 was slower).  The per-query split keeps
// 4: the host sizes its partial slots from that.
constexpr int kMinUnitsPerWave = 4, kTinyStream = 256;
__device__ inline int64_t stream_waves(int64_t units, int grid, bool whole_call = false) {
  const int per = whole_call && units < kTinyStream ? 2 : kMinUnitsPerWave;
  int64_t w = (units + per - 1) / per;
  if (w < 1) w = 1;
  return w < grid ? w : grid;
}

// Start of a sequence's stream (in units, times NKV) and its unit count.
struct SeqSpan {
  int b;
  int64_t start;  // global unit index of (b, kv head 0)
  int units;      // units per kv head
};

// The sequence whose streams contain global tile x.
__device__ inline SeqSpan locate(const KiviGeo& g, const DecodeArgs& a, int64_t x, int lane) {
  int64_t run = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int bb = base + lane;
    int T = 0;
    if (bb < a.batch) T = seq_units(g, a, bb);
    const int incl = wave_incl_scan(T, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(bb < a.batch && run + (int64_t)g.nkv * incl > x);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      const int Tf = __builtin_amdgcn_readlane(T, f), If = __builtin_amdgcn_readlane(incl, f);
      return {base + f, run + (int64_t)g.nkv * (If - Tf), Tf};
    }
    run += (int64_t)g.nkv * __builtin_amdgcn_readlane(incl, 63);
  }
  return {a.batch, run, 1};
}

// One 32-token fp16 residual tile in registers: K rows of MFMA row c of tile
// tt (tokens 8(c/4) + 4tt + c%4, channel block j) and V rows 8j..8j+7
// (channels CPL*c..).  Rows past the end read row 0 of the tile (a valid
// scratch row) and are masked by the caller.
template <int HD>
struct ResTile {
  typedef typename std::conditional<HD == 128, u32x4, u32x2>::type vrow_t;
  u32x4 kv[2][HD / 32];
  vrow_t vr[8];
};

// FUSED: residual row new_row (>= 0) is the step's new token, read from
// NEW_K / NEW_V.
// Rows of a residual tile: non-temporal loads, or (COH) device-scope loads
// of eight bytes at a time, for rows the fused step's writer just shifted.
template <typename V, bool COH>
__device__ inline V ld_rows(const uint16_t* p) {
  if constexpr (COH) {
    constexpr int N = sizeof(V) / 8;
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      w[i] = __hip_atomic_load((const uint64_t*)p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(V, w);
  } else {
    return __builtin_nontemporal_load((const V*)p);
  }
}

template <int HD, bool FUSED, bool COH>
__device__ inline ResTile<HD> load_res(const DecodeArgs& a, const KiviGeo& g, int b, int h,
                                       int ov, int n, int tile, int lane, int new_row) {
  constexpr int KS = HD / 32, CPL = HD / 16;
  // lane offsets from an opaque copy of the lane id: hoisted out of the
  // loops they would hold 64-bit registers through the whole run
  asm volatile("" : "+v"(lane));
  const int c = lane & 15, j = lane >> 4;
  const uint16_t* kscr = a.k_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const uint16_t* vscr = a.v_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const int t0 = tile * kGroup;
  const int tn = min(kGroup, n - t0);
  const int r0 = t0 - ov;  // scratch row of token t0
  // the row pointers of K and V (FUSED: the new token's row from NEW_K / NEW_V)
  auto krow = [&](int row) -> const uint16_t* {
    if constexpr (FUSED) {
      if (row == new_row) return a.wr.new_k + (int64_t)b * a.wr.new_stride + (int64_t)h * HD;
    }
    return kscr + (int64_t)row * HD;
  };
  auto vrow = [&](int row) -> const uint16_t* {
    if constexpr (FUSED) {
      if (row == new_row) return a.wr.new_v + (int64_t)b * a.wr.new_stride + (int64_t)h * HD;
    }
    return vscr + (int64_t)row * HD;
  };
  ResTile<HD> rt;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tl = 8 * (c >> 2) + 4 * tt + (c & 3);
    const uint16_t* kr = krow(r0 + (tl < tn ? tl : 0)) + j * (HD / 4);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      rt.kv[tt][ks] = ld_rows<u32x4, COH>(kr + 8 * ks);
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int tl = 8 * j + r;
    rt.vr[r] = ld_rows<typename ResTile<HD>::vrow_t, COH>(vrow(r0 + (tl < tn ? tl : 0)) + CPL * c);
  }
  return rt;
}

// ---- per-query split (the v1 symbols) ----
//
// Each query's streams (NKV x its units) are cut into stream_waves(its units)
// equal runs by its own length alone, exactly as a call with that query alone
// cuts them, whatever the other queries of the call are: every query decodes
// to the same bits in a batched call as in a single one (variants.rs:1211-1213
// expects the batched kernel to match the single-token one bit for bit).  The
// runs of all queries are numbered query by query; the stream wavefronts take
// them in turn.
struct RunLoc {
  int q;       // query, or -1 past the last run
  int units;   // units per kv head of the query
  int runs;    // runs of the query
  int64_t r0;  // global index of the query's first run
};

__device__ inline int query_runs(const KiviGeo& g, const DecodeArgs& a, int units) {
  return (int)stream_waves((int64_t)g.nkv * units, a.waves);
}

__device__ inline RunLoc locate_run(const KiviGeo& g, const DecodeArgs& a, int64_t r, int lane) {
  int64_t acc = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int bb = base + lane;
    int U = 0, R = 0;
    if (bb < a.batch) {
      U = seq_units(g, a, bb);
      R = query_runs(g, a, U);
    }
    const int incl = wave_incl_scan(R, lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(bb < a.batch && acc + incl > r);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      const int Rf = __builtin_amdgcn_readlane(R, f);
      return {base + f, __builtin_amdgcn_readlane(U, f), Rf,
              acc + __builtin_amdgcn_readlane(incl, f) - Rf};
    }
    acc += __builtin_amdgcn_readlane(incl, 63);
  }
  return {-1, 0, 0, acc};
}

// Global index of query b's first run.
__device__ inline int64_t query_run_start(const KiviGeo& g, const DecodeArgs& a, int b, int lane) {
  int64_t run = 0;
  for (int base = 0; base < b; base += 64) {
    const int bb = base + lane;
    const int R = bb < b ? query_runs(g, a, seq_units(g, a, bb)) : 0;
    run += __builtin_amdgcn_readfirstlane(wave_sum_i(R));
  }
  return run;
}

// The step's sequence b ages a group out: its old-token count grows.
__device__ inline bool step_ages(const KiviGeo& g, int len_after) {
  return len_after >= 1 &&
         split_old_tokens(len_after, g.residual) > split_old_tokens(len_after - 1, g.residual);
}

__device__ inline int step_len(const DecodeArgs& a, int b) {
  return ((const __attribute__((address_space(4))) int32_t*)a.seq_lens)[b];
}

// ---- split-K merge, run by workgroups of the same launch ----
//
// The stream wavefronts fill every slot of the device, so the merge
// workgroups (block ids past a.waves) start as stream wavefronts finish, on
// the CUs the end of the launch leaves idle.  A wavefront that leaves a
// partial stores it with agent-scope stores (they reach the point of
// coherence of all XCDs without an L2 write-back), waits for them, and then
// stores the launch's 64-bit epoch in the partial's flag.  A merge wavefront
// reads a partial only after it has read that epoch from the flag, with
// agent-scope loads, and then clears the flag.  Every flag is therefore zero
// when a launch starts -- also when a replayed graph repeats the epoch --
// except in a fresh buffer, whose contents match a 64-bit epoch with
// probability 2^-64; the workspace needs no reset.  The merge does not hold
// anything a stream wavefront waits for, and there are at most half as many
// merge workgroups as stream slots, so the stream wavefronts always run; a
// merge wavefront that still waits after kMergeTimeoutTicks (s_memrealtime,
// 100 MHz) writes NaN for its segments and ends, so the launch always drains.
constexpr uint64_t kMergeTimeoutTicks = 100000000;  // 1 s
// Value of a workspace's poison word (its first 8 bytes) after a merge on it
// timed out; anything else means clean (a fresh buffer matches with
// probability 2^-64).
constexpr uint64_t kWorkspacePoison = 0x4A4B49564954494Dull;

// Test-only (jacq_kivi_test_force_merge_timeout): when nonzero, every merge
// waits for an epoch no stream wave stores and gives up after this many
// s_memrealtime ticks, so a test can check from the host that a launch whose
// merges time out still drains and reports it.  Zero in normal use.
static std::atomic<uint64_t> g_test_merge_timeout_ticks{0};
void set_test_merge_timeout_us(uint32_t us) {
  g_test_merge_timeout_ticks.store((uint64_t)us * 100, std::memory_order_relaxed);  // 100 MHz
}

// Global unit index of (b, kv head 0): NKV times the units of the sequences before b.
__device__ inline int64_t seq_start(const KiviGeo& g, const DecodeArgs& a, int b, int lane) {
  int64_t run = 0;
  for (int base = 0; base < b; base += 64) {
    const int bb = base + lane;
    const int U = bb < b ? seq_units(g, a, bb) : 0;
    run += __builtin_amdgcn_readfirstlane(wave_sum_i(U));
  }
  return run * g.nkv;
}

// Run weights, in sixteenths: a run of the fused step's writer wavefronts
// (the first nw runs) weighs kWriterRun, every other run kRun, so the waves
// that first do the writer's age-outs take shorter runs of the stream (by
// per-wave stamps at 14B, a writer's items take about a quarter of a run).
constexpr int kRun = 16, kWriterRun = 13;
__device__ inline int64_t run_weight_sum(int64_t w, int64_t nw) {
  return kRun * w - (kRun - kWriterRun) * (w < nw ? w : nw);
}
// First unit of wavefront w's run, and the wavefront whose run holds unit x
// (W runs over TT units, the first nw of them writer runs).
__device__ inline int64_t run_begin(int64_t w, int64_t TT, int64_t W, int64_t nw = 0) {
  return TT * run_weight_sum(w, nw) / run_weight_sum(W, nw);
}
__device__ inline int64_t wave_of(int64_t x, int64_t TT, int64_t W, int64_t nw = 0) {
  const int64_t c = x * run_weight_sum(W, nw) / TT;  // the weight sum at x, rounded down
  const int64_t n = nw < W ? nw : W;
  int64_t w = c < kWriterRun * n ? c / kWriterRun : n + (c - kWriterRun * n) / kRun;
  if (w > W - 1) w = W - 1;
  while (w > 0 && run_begin(w, TT, W, nw) > x) --w;
  while (w + 1 < W && run_begin(w + 1, TT, W, nw) <= x) ++w;
  return w;
}

__device__ inline uint64_t ld_agent(const void* p) {
  return __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(void* p, float lo, float hi) {
  const uint64_t v = (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte agent-scope store (the bits the compiler gives an agent-scope
// relaxed atomic store, sc1, on a four-dword store); waited for by the
// explicit vmcnt(0) before the partial's flag.  A VALU write of the data
// VGPRs of a store wider than 8 bytes needs one wait state after it (a GFX9
// hazard the compiler's recognizer cannot see inside asm): without the s_nop
// the next instruction may overwrite data the store has not read yet, and a
// lane's 16 bytes of a partial were now and then stored wrong.
__device__ inline void st_agent4(float* p, floatx4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}
// 16-byte agent-scope load; the caller waits with an explicit vmcnt(0) and
// then passes the value through keep() so no use moves above the wait
__device__ inline floatx4 ld_agent4(const float* p) {
  floatx4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ inline void keep(floatx4& v) { asm volatile("" : "+v"(v)); }
// Device-scope (sc1) store of one to eight bytes: the fused step's writer
// stores what decode wavefronts of the same launch, on any XCD, read next.
template <typename T>
__device__ inline void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float lo_f(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ inline float hi_f(uint64_t v) { return __uint_as_float((uint32_t)(v >> 32)); }

// ---- profiling: per-workgroup stamps (jacq_kivi_profile_wave_stamps) ----
static std::atomic<uint64_t*> g_stamps{nullptr};
static std::atomic<int> g_stamp_cap{0};
void set_wave_stamps(uint64_t* buf, int cap) {
  g_stamp_cap.store(buf ? cap : 0, std::memory_order_relaxed);
  g_stamps.store(buf, std::memory_order_relaxed);
}
// start and end (s_memrealtime, 100 MHz), HW_ID | XCC_ID << 32 and `info`,
// written by lane 0 with plain vector stores
__device__ inline void write_stamp(const DecodeArgs& a, uint64_t t0, uint64_t info, int lane) {
  const int b = blockIdx.x;
  if (!a.stamps || b >= a.stamp_cap || lane != 0) return;
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  const uint32_t hw = __builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11));    // HW_ID
  const uint32_t xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11));  // XCC_ID
  uint64_t* p = a.stamps + 4 * (int64_t)b;
  p[0] = t0;
  p[1] = t1;
  p[2] = (uint64_t)hw | ((uint64_t)xcc << 32);
  p[3] = info;
}

// Log-sum-exp merge of the partials of every (sequence, kv head) whose run was
// cut (variants.rs:3548-3565): M = max m_w, L = sum l_w e^(m_w - M), acc
// likewise, O = acc / max(L, 1e-30), in the log2 domain of the decode loop.
// The pieces of a segment are recomputed from the same split the stream
// wavefronts used; a segment with a single non-empty piece was written whole.
template <int HD, bool PACK, bool PQ, bool FUSED>
__device__ __attribute__((always_inline)) inline uint64_t merge_segments(const KiviGeo& g,
                                                                       const DecodeArgs& a,
                                                                       int lane) {
  constexpr int K = (PACK ? 8 : 16) * HD / 256;  // float4 outputs per lane: G * HD <= 256 K
  constexpr int U = K <= 2 ? 8 : K > 4 ? 1 : 2;  // partials whose loads are in flight together
  const int G = g.gqa, NKV = g.nkv, n4 = G * HD / 4;
  // the whole call's stream (per-query split: each segment's own query, below)
  const int64_t TT = PQ ? 0 : stream_units(g, a, lane);
  const int64_t W = PQ ? 0 : stream_waves(TT, a.waves, true);
  const int64_t nw = FUSED ? a.writer_waves : 0;  // writer runs (PQ: none)
  const int nseg = a.batch * NKV;
  const uint64_t epoch = a.epoch + a.merge_skew, t_start = __builtin_amdgcn_s_memrealtime();
  // wave-uniform: the wait ran out.  A merge of an earlier launch on this
  // workspace that timed out left the poison word set: flags its stream
  // wavefronts stored after it gave up may carry the epoch a replayed graph
  // repeats, so until the host resets the workspace every merged segment is
  // NaN and no flag is consumed.
  bool late = a.ws_poison && ld_agent(a.ws_poison) == kWorkspacePoison;
  uint64_t t_land = t_start;  // profiling: when the last wait ended
  uint32_t rounds_after = 0;  // profiling: load rounds after it
  int gi[K], d[K];
  bool on[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int e = lane + 64 * k;  // outputs 4e .. 4e + 3 of head gi
    on[k] = e < n4;
    gi[k] = 4 * e / HD;
    d[k] = 4 * e - gi[k] * HD;
  }
  for (int seg = (int)blockIdx.x - a.waves; seg < nseg; seg += a.merge_wgs) {
    const int b = seg / NKV, h = seg - b * NKV;
    int ov, n;
    const int T = seq_tiles(g, a, b, &ov, &n);
    const int nq = ov / kGroup;
    const int units = nq + kResidualUnits * (T - nq);
    // the stream the segment's runs cut (sq units in wq runs), the segment's
    // first unit in it, and the global index of that stream's first run
    int64_t sq = TT, wq = W, S0, roff = 0;
    if constexpr (PQ) {
      sq = (int64_t)NKV * units;
      wq = stream_waves(sq, a.waves);
      S0 = (int64_t)h * units;
      roff = query_run_start(g, a, b, lane);
    } else {
      S0 = seq_start(g, a, b, lane) + (int64_t)h * units;
    }
    const int64_t S1 = S0 + units;
    const int64_t w0 = wave_of(S0, sq, wq, nw), w1 = wave_of(S1 - 1, sq, wq, nw);
    // non-empty pieces: the runs that own at least one tile of the segment
    auto owns = [&](int64_t w) {
      const int64_t x0 = max(run_begin(w, sq, wq, nw), S0),
                    x1 = min(run_begin(w + 1, sq, wq, nw), S1);
      return tile_at((int)(x0 - S0), nq) < tile_at((int)(x1 - S0), nq);
    };
    int pieces = 0;
    for (int64_t wb = w0; wb <= w1; wb += 64)
      pieces += __builtin_popcountll(
          __builtin_amdgcn_ballot_w64(wb + lane <= w1 && owns(wb + lane)));
    if (pieces <= 1) continue;  // written whole by its wavefront

    float M[K], Lsum[K];
    floatx4 acc[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      M[k] = -INFINITY;
      Lsum[k] = 0.0f;
      acc[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    for (int64_t wb = w0; wb <= w1 && !late; wb += 64) {
      const int64_t wl = wb + lane;
      const bool mine = wl <= w1 && owns(wl);
      const uint64_t* flag = a.ws_flag + seg + roff + wl;
      uint64_t todo = __builtin_amdgcn_ballot_w64(mine);
      // fold the partials in piece order (the result does not depend on
      // timing), each run of them as soon as its flags show this launch's
      // epoch: after the last one lands, only those behind it remain
      while (todo) {
        const uint64_t bit = 1ull << lane;
        // one lane waits for the first piece in order ...
        if (lane == __builtin_ctzll(todo)) {
          while (ld_agent(flag) != epoch &&
                 __builtin_amdgcn_s_memrealtime() - t_start <= a.merge_timeout)
            __builtin_amdgcn_s_sleep(4);
        }
        // ... then one round finds how many after it have landed too
        const uint64_t landed =
            __builtin_amdgcn_ballot_w64((todo & bit) && ld_agent(flag) == epoch);
        if (a.stamps) {
          t_land = __builtin_amdgcn_s_memrealtime();
          rounds_after = 0;
        }
        // the ready prefix: pieces of todo below its first one not yet stored
        const uint64_t waiting = todo & ~landed;
        uint64_t ready = waiting ? todo & ((waiting & (0 - waiting)) - 1) : todo;
        if (!ready) {  // the first piece's wait ran out
          late = true;
          break;
        }
        todo &= ~ready;
        while (ready) {
          int64_t slot[U];
          uint64_t consumed = ready;  // after the loop below: the bits this round takes
#pragma unroll
          for (int u = 0; u < U; ++u) {
            slot[u] = -1;
            if (ready) {
              slot[u] = seg + roff + wb + __builtin_ctzll(ready);
              ready &= ready - 1;
            }
          }
          consumed &= ~ready;
          ++rounds_after;
          uint64_t ml[U][K];
          floatx4 vv[U][K];
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
              ml[u][k] = 0xff800000u;  // (m, l) = (-inf, 0): folded with weight 0
              vv[u][k] = floatx4{0.f, 0.f, 0.f, 0.f};
              if (slot[u] >= 0 && on[k]) {
                const int64_t p = slot[u] * G + gi[k];
                ml[u][k] = ld_agent(a.ws_ml + 2 * p);
                vv[u][k] = ld_agent4(a.ws_acc + p * HD + d[k]);
              }
            }
          }
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < K; ++k) keep(vv[u][k]);
          }
          // read: clear the flags, so the next launch starts from zero even
          // when it carries the same epoch (a replayed graph does)
          if (consumed & bit)
            __hip_atomic_store(a.ws_flag + seg + roff + wl, 0ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
              const float m = lo_f(ml[u][k]), l = hi_f(ml[u][k]);
              const float mn = fmaxf(M[k], m);
              const float fo = __builtin_amdgcn_exp2f(M[k] - mn);
              const float fn = __builtin_amdgcn_exp2f(m - mn);
              const floatx4 v = vv[u][k];
              acc[k] = acc[k] * fo + v * fn;
              Lsum[k] = Lsum[k] * fo + l * fn;
              M[k] = mn;
            }
          }
        }
      }
    }
    float* out = a.out + (int64_t)b * a.out_stride + (int64_t)h * G * HD;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (on[k])
        *(floatx4*)(out + (int64_t)gi[k] * HD + d[k]) =
            late ? floatx4{NAN, NAN, NAN, NAN} : acc[k] / fmaxf(Lsum[k], 1.0e-30f);
    // fused step: every piece of the segment has landed, so its readers of
    // the writer's age-out are done; its flags start the next launch at zero
    if constexpr (FUSED) {
      if (lane < 2 * (HD / kGroup) && step_ages(g, step_len(a, b)))
        __hip_atomic_store(a.ws_wflag + 2 * (HD / kGroup) * (int64_t)seg + lane, 0ull,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // a wait ran out (or an earlier one poisoned the workspace): the workspace
  // stays poisoned, and the host sees it in the device's status word
  if (late && lane == 0) {
    if (a.ws_poison)
      __hip_atomic_store(a.ws_poison, kWorkspacePoison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.status) __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  return ((t_land - t_start) & ((1ull << 24) - 1)) | ((uint64_t)(rounds_after & 63) << 24);
}

// ---- fused write + decode: the writer wavefronts ----
//
// jacq_kivi_write_decode appends one token per sequence (length seq_lens - 1
// before, seq_lens after) and decodes the new state in one launch.  The
// writer's work rides on the first stream wavefronts of the grid, which are
// dispatched before the others, do it first (waiting for nothing) and then
// decode a run of the stream shorter than the others' (kWriterRun):
//  - a plain append stores the new token in scratch row r0.  No decode
//    wavefront of this launch reads that row from the scratch: the residual
//    tile that holds it takes the row from NEW_K / NEW_V instead;
//  - a sequence that ages a group out (its 32 oldest scratch rows become int4
//    pages) is one item per (kv head, K or V, 32-channel slice): quantise
//    rows 0..31 into the group's pages, shift the scratch down 32 rows, store
//    the new token in rows R - 1 and r0 (the writer's final state, stale copy
//    included), all with device-scope stores, then wait for them and store
//    the launch's epoch in the item's flag.  Decode wavefronts that read the
//    new group or the residual tiles of such a segment wait for all of its
//    flags before their first (device-scope) load of them; the wavefront or
//    merge that finishes the segment clears them.
// The arithmetic is the writer kernel's (kivi_append_kernel), so pages and
// scratch end bit for bit as a separate write would leave them.

// Flags per (sequence, kv head): K and V, one per 32-channel slice each.
template <int HD>
constexpr int step_flags() {
  return 2 * (HD / kGroup);
}

// One age-out item: channels [32 q, 32 q + 32) of K or V of (sequence b, kv
// head h).  The slice is self-contained: K is quantised per channel (over the
// group's 32 tokens) and V per (token, 32-channel group), so the slice's codes
// and scales need only its own rows, and the slice's shift touches no other
// item's bytes -- items need no ordering among themselves.
template <int HD>
__device__ __attribute__((always_inline)) inline void step_age_out(const KiviGeo& g,
                                                                   const DecodeArgs& a, int b,
                                                                   int h, bool is_v, int q,
                                                                   int lane) {
#pragma clang fp contract(off)
  constexpr int HDP = HD / 2, HDG = HD / kGroup;
  const AppendArgs& w = a.wr;
  const int P = g.page, ppg = kGroup / P;
  const int start = step_len(a, b) - 1;
  const int old0 = split_old_tokens(start, g.residual), r0 = start - old0;  // r0 = R + 31
  uint16_t* xs = (is_v ? w.v_scr : w.k_scr) + (int64_t)b * w.scr_stride + (int64_t)h * g.rs * HD +
                 kGroup * q;
  const uint16_t* nx =
      (is_v ? w.new_v : w.new_k) + (int64_t)b * w.new_stride + (int64_t)h * HD + kGroup * q;
  const int fp = (old0 / kGroup) * ppg;  // the group's first logical page
  const bool table_ok = fp + ppg <= g.max_pages;
  int p0 = -1, p1 = -1;
  if (table_ok) {
    const int32_t* bt = w.block_tables + (int64_t)b * w.bt_stride;
    p0 = bt[fp];
    p1 = ppg == 2 ? bt[fp + 1] : p0;
  }
  auto phys_ok = [&](int p) { return table_ok && p >= 0 && p < g.num_pages; };
  if (!is_v) {
    // K: lane = (channel pair pr of the slice's 16, token quarter tq): the
    // pair's min / max over its 8 tokens, merged over the 4 quarters
    const int pr = lane >> 2, tq = lane & 3, t0 = 8 * tq;
    uint32_t x[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) x[t] = *(const uint32_t*)(xs + (t0 + t) * HD + 2 * pr);
    float mn0 = h2f((uint16_t)x[0]), mx0 = mn0, mn1 = h2f((uint16_t)(x[0] >> 16)), mx1 = mn1;
#pragma unroll
    for (int t = 1; t < 8; ++t) {
      const float v0 = h2f((uint16_t)x[t]), v1 = h2f((uint16_t)(x[t] >> 16));
      mn0 = min_num(mn0, v0);
      mx0 = max_num(mx0, v0);
      mn1 = min_num(mn1, v1);
      mx1 = max_num(mx1, v1);
    }
#pragma unroll
    for (int off = 1; off < 4; off <<= 1) {
      mn0 = min_num(mn0, __shfl_xor(mn0, off, 64));
      mx0 = max_num(mx0, __shfl_xor(mx0, off, 64));
      mn1 = min_num(mn1, __shfl_xor(mn1, off, 64));
      mx1 = max_num(mx1, __shfl_xor(mx1, off, 64));
    }
    float s0 = (mx0 - mn0) / 15.0f, s1 = (mx1 - mn1) / 15.0f;
    if (!(s0 > 0.0f)) s0 = 1.0f;
    if (!(s1 > 0.0f)) s1 = 1.0f;
    const int d0 = kGroup * q + 2 * pr;  // channel of the pair's low nibble
    if (tq == 0) {
      const uint32_t sc = (uint32_t)f2h(s0) | ((uint32_t)f2h(s1) << 16);
      const uint32_t zr = (uint32_t)f2h(mn0) | ((uint32_t)f2h(mn1) << 16);
      for (int pg = 0; pg < ppg; ++pg) {  // K scales live in every page of the group
        const int phys = pg == 0 ? p0 : p1;
        if (!phys_ok(phys)) continue;
        const int64_t base = ((int64_t)phys * g.nkv + h) * HD + d0;
        st_dev((uint32_t*)(w.k_scale + base), sc);
        st_dev((uint32_t*)(w.k_zero + base), zr);
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int tok = t0 + t, phys = tok < P ? p0 : p1;
      const int c0 = clamp_code((h2f((uint16_t)x[t]) - mn0) / s0);
      const int c1 = clamp_code((h2f((uint16_t)(x[t] >> 16)) - mn1) / s1);
      if (phys_ok(phys))
        st_dev(w.k_code + (((int64_t)phys * g.nkv + h) * P + tok % P) * HDP + d0 / 2,
               (uint8_t)((c0 & 0x0f) | ((c1 & 0x0f) << 4)));
    }
  } else {
    // V: lane = (token t, half hf of the slice's 32 channels); min / max over
    // 16 channels, merged with the other half
    const int t = lane >> 1, hf = lane & 1;
    const uint16_t* row = xs + t * HD + 16 * hf;
    const u32x4 v0 = *(const u32x4*)row, v1 = *(const u32x4*)(row + 8);
    auto ch = [&](int k) -> float {  // channel k of the lane's 16
      const u32x4& v = k < 8 ? v0 : v1;
      return h2f((uint16_t)(v[(k % 8) / 2] >> (16 * (k & 1))));
    };
    float mn = ch(0), mx = mn;
#pragma unroll
    for (int k = 1; k < 16; ++k) {
      mn = min_num(mn, ch(k));
      mx = max_num(mx, ch(k));
    }
    mn = min_num(mn, __shfl_xor(mn, 1, 64));
    mx = max_num(mx, __shfl_xor(mx, 1, 64));
    float sv = (mx - mn) / 15.0f;
    if (!(sv > 0.0f)) sv = 1.0f;
    u32x2 codes;
#pragma unroll
    for (int wd = 0; wd < 2; ++wd) {
      uint32_t word = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) word |= (uint32_t)clamp_code((ch(8 * wd + k) - mn) / sv) << (4 * k);
      codes[wd] = word;
    }
    const int phys = t < P ? p0 : p1;
    if (phys_ok(phys)) {
      const int64_t tok = ((int64_t)phys * g.nkv + h) * P + t % P;
      st_dev((uint64_t*)(w.v_code + tok * HDP + q * (kGroup / 2) + 8 * hf),
             __builtin_bit_cast(uint64_t, codes));
      if (hf == 0) {
        st_dev(w.v_scale + tok * HDG + q, f2h(sv));
        st_dev(w.v_zero + tok * HDG + q, f2h(mn));
      }
    }
  }
  // shift the slice: rows [0, R - 1) <- rows [32, R + 31), four 16-byte
  // pieces per row, in chunks of 8 pieces per lane.  Within a chunk store k
  // writes rows that no later load of any chunk reads (sources lie 32 rows
  // above), and the quantisation above read rows 0..31 first.
  const int units = (g.residual - 1) * 4;
  for (int u0 = 0; u0 < units; u0 += 64 * 8) {
    u32x4 buf[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int u = min(u0 + lane + 64 * k, units - 1);
      buf[k] = *(const u32x4*)(xs + (int64_t)(u / 4 + kGroup) * HD + 8 * (u % 4));
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int u = u0 + lane + 64 * k;
      if (u < units)
        st_agent4((float*)(xs + (int64_t)(u / 4) * HD + 8 * (u % 4)),
                  __builtin_bit_cast(floatx4, buf[k]));
    }
  }
  // the new token's slice: row R - 1 (live) and row r0 (the reference's stale copy)
  if (lane < 8) {
    const int row = lane < 4 ? g.residual - 1 : r0, piece = lane % 4;
    st_agent4((float*)(xs + (int64_t)row * HD + 8 * piece),
              __builtin_bit_cast(floatx4, *(const u32x4*)(nx + 8 * piece)));
  }
  // every store above is device-scope (the readers' loads are too): complete
  // before the flag
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane == 0)
    __hip_atomic_store(a.ws_wflag + step_flags<HD>() * ((int64_t)b * g.nkv + h) +
                           (is_v ? HDG : 0) + q,
                       a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Writer wavefront wi of a.writer_waves: first the age-out items (sequence
// rank among the aging ones, kv head, K | V) in turn, then the plain appends
// of the other (sequence, kv head) pairs.
template <int HD>
__device__ __attribute__((always_inline)) inline uint64_t step_writer(const KiviGeo& g, const DecodeArgs& a, int wi,
                                                                int lane) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint64_t tf = t0;  // profiling: the end of its last age-out item
  const int NW = a.writer_waves, NKV = g.nkv;
  int rank0 = 0;  // aging sequences before this 64-sequence window
  for (int base = 0; base < a.batch; base += 64) {
    const int bb = base + lane;
    const bool ag = bb < a.batch && step_ages(g, step_len(a, bb));
    uint64_t m = __builtin_amdgcn_ballot_w64(ag);
    int rank = rank0;
    while (m) {
      const int b = base + __builtin_ctzll(m);
      m &= m - 1;
      constexpr int F = step_flags<HD>();  // items per (sequence, kv head)
      for (int k = 0; k < F * NKV; ++k) {
        const int item = rank * F * NKV + k;
        if (item % NW == wi) {
          const int hh = k / F, f = k % F;
          step_age_out<HD>(g, a, b, hh, f >= F / 2, f % (F / 2), lane);
          tf = __builtin_amdgcn_s_memrealtime();
        }
      }
      ++rank;
    }
    rank0 = rank;
  }
  constexpr int V16 = HD / 8;
  const AppendArgs& w = a.wr;
  for (int p = wi; p < a.batch * NKV; p += NW) {
    const int b = p / NKV, h = p - b * NKV;
    const int L = step_len(a, b);
    if (L < 1 || step_ages(g, L)) continue;
    const int start = L - 1, r0 = start - split_old_tokens(start, g.residual);
    if (r0 >= g.rs) continue;  // the writer's bound (in-scratch appends only)
    if (lane < 2 * V16) {
      const bool v = lane >= V16;
      const int piece = lane % V16;
      uint16_t* xs = (v ? w.v_scr : w.k_scr) + (int64_t)b * w.scr_stride + (int64_t)h * g.rs * HD;
      const uint16_t* nx = (v ? w.new_v : w.new_k) + (int64_t)b * w.new_stride + (int64_t)h * HD;
      *(u32x4*)(xs + (int64_t)r0 * HD + 8 * piece) = *(const u32x4*)(nx + 8 * piece);
    }
  }
  return tf - t0;
}

// One run of the stream: units [x0, x1) of the concatenated (sequence, kv
// head) streams, starting in sequence sp.b.  `first_seg` with first_* gives
// the first segment's window when the caller has it already.  Partials of cut
// segments go to slot b * NKV + h + w (w: the run's index), their flags after
// the run.  Returns the s_memrealtime of the first group in LDS (profiling).
template <int HD, int P, bool PACK, bool FUSED>
__device__ __attribute__((always_inline)) inline uint64_t stream_run(
    const KiviGeo& g, const DecodeArgs& a, StageBuf<HD>* ring, uint16_t* qrows, const Nibble& nb,
    float sscale, int lane, int64_t x0, int64_t x1, SeqSpan sp, bool first_seg, int first_T,
    int first_ov, int first_n, int w) {
  using C = Cfg<HD, P>;
  constexpr int KS = C::KS, CPL = C::CPL;
  constexpr int L = stage_loads<HD>(), S = stages<HD, PACK>();
  constexpr int QROW = HD + 8;
  const int c = lane & 15, j = lane >> 4;
  const int G = g.gqa, NKV = g.nkv;
  const bool sum_col = sum_lane<HD>(c);
  constexpr int C1 = kGroup / CPL - 1;  // a sum column (the first group's)
  // Issue arbitration favours the oldest of the waves sharing a SIMD, which left
  // alone finishes its run well before the younger ones.  Each wave drops its
  // priority at 1/2, 4/5 and 19/20 of its own run, so a wave behind its
  // partners outranks them and they reach each mark close together; the last
  // band, where age alone decides again, is short.
  const int n_run = (int)(x1 - x0), q1 = n_run / 2, q2 = 4 * n_run / 5, q3 = 19 * n_run / 20;
  int done = 0, level = 3;
  __builtin_amdgcn_s_setprio(3);
  auto progress = [&](int units) {
    done += units;
    if (level == 3 && done >= q1) {
      __builtin_amdgcn_s_setprio(2);
      level = 2;
    }
    if (level == 2 && done >= q2) {
      __builtin_amdgcn_s_setprio(1);
      level = 1;
    }
    if (level == 1 && done >= q3) {
      __builtin_amdgcn_s_setprio(0);
      level = 0;
    }
  };
  int kvh = (int)((x0 - sp.start) / sp.units);
  int u = (int)((x0 - sp.start) % sp.units);  // unit offset inside the segment
  int64_t x = x0, xe = x1;                  // the current pass: [x, xe)
  // fused step: a run whose first segment ages a group out would wait for the
  // writer at its very start; when the run goes on into further segments it
  // decodes those first and that segment last (two passes), by which time
  // the writer is done
  int64_t x_rot = -1;
  SeqSpan sp_rot = sp;
  int kvh_rot = kvh, u_rot = u;
  if constexpr (FUSED) {
    const int64_t seg_end = x0 + (sp.units - u);
    if (seg_end < x1) {
      int ov0, n0_;
      seq_tiles(g, a, sp.b, &ov0, &n0_);
      const int L0 = step_len(a, sp.b);
      if (step_ages(g, L0) && ov0 == split_old_tokens(L0, g.residual)) {
        x_rot = x0;
        xe = seg_end;  // the end of the rotated-away pass, kept below
        x = seg_end;
        u = 0;
        if (++kvh == NKV) {
          kvh = 0;
          sp.b += 1;
        }
        first_seg = false;
      }
    }
  }
  const int64_t x_rot_end = xe;
  if (x_rot >= 0) xe = x1;
  int64_t cut_first = -1, cut_last = -1;  // pieces this run leaves as partials
  uint64_t t_first = 0;                   // profiling: first group in LDS
  uint64_t t_wait = 0;                    // profiling (fused step): ticks waited for the writer
  for (;;) {
    while (x < xe) {
      const int b = sp.b, h = kvh;
      int ov = first_ov, n = first_n, T = first_T;
      if (!first_seg) T = seq_tiles(g, a, b, &ov, &n);
      first_seg = false;
      const int nq = ov / kGroup;
      const int u_end = (int)min((int64_t)(nq + kResidualUnits * (T - nq)), u + (xe - x));
      const int t_beg = tile_at(u, nq), t_fin = tile_at(u_end, nq);
      x += u_end - u;
      u = 0;
      if (++kvh == NKV) {
        kvh = 0;
        sp.b += 1;
      }
      // the run starts inside this segment's last residual tile, which the
      // previous wavefront owns: nothing here (no partial, no map entry)
      if (t_beg >= t_fin) continue;

      // fused step: a segment whose sequence ages a group out reads its new
      // group (tile g_age) and its residual rows only after the writer's two
      // flags; in the others the residual row new_row (the new token) comes
      // from NEW_K / NEW_V, never from the scratch the writer is storing to
      int g_age = 0x7fffffff, new_row = -1;
      bool ages = false, aging = false, waited = false;
      if constexpr (FUSED) {
        const int Lb = step_len(a, b);
        ages = step_ages(g, Lb);
        aging = ages && ov == split_old_tokens(Lb, g.residual);
        if (aging)
          g_age = ov / kGroup - 1;
        else if (Lb == n && n > ov)
          new_row = n - ov - 1;
      }
      auto wait_new = [&]() {
        if (waited) return;
        waited = true;
        if (lane == 0) {
          constexpr int F = step_flags<HD>();
          const uint64_t* f = a.ws_wflag + F * ((int64_t)b * NKV + h);
          const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
          bool late = false;
          auto ready = [&]() {
            bool r = true;
#pragma unroll
            for (int k = 0; k < F; ++k) r = r && ld_agent(f + k) == a.epoch;
            return r;
          };
          while (!ready()) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > a.merge_timeout) {
              late = true;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          if (a.stamps) t_wait += __builtin_amdgcn_s_memrealtime() - t0;
          if (late && a.status)
            __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        // the writer stored with device-scope stores; the segment's new group
        // and residual rows are read with device-scope loads (COH)
      };

      // ---- quantised groups: a ring of S LDS stages, S - 1 in flight ----
      const int tq_end = min(t_fin, ov / kGroup);
      // read-only for the whole launch: the constant address space lets the
      // wave-uniform page reads be scalar loads (lgkmcnt, not vmcnt)
      const __attribute__((address_space(4))) int32_t* bt =
          (const __attribute__((address_space(4))) int32_t*)(a.block_tables +
                                                             (int64_t)b * a.bt_stride);
      const StageBases sb = stage_bases<HD, P>(a, NKV, h, lane);
      auto page = [&](int tile, int k) -> uint32_t {
        return (uint32_t)bt[tile * C::PPG + (C::PPG == 2 ? k : 0)];
      };
      uint32_t n0 = 0, n1 = 0;  // pages of group i + S - 1, read one group early
      if (t_beg < tq_end) {
        if constexpr (FUSED) {
          if (g_age >= t_beg && g_age < t_beg + S - 1 && g_age < tq_end) wait_new();
        }
        wait_vm<0>();  // the counts below see only this segment's DMAs
#pragma unroll
        for (int k = 0; k < S - 1; ++k)
          if (t_beg + k < tq_end)
            if (FUSED && t_beg + k == g_age)
              load_stage<HD, P, true>(&ring[k], sb, page(t_beg + k, 0), page(t_beg + k, 1), lane);
            else
              load_stage<HD, P>(&ring[k], sb, page(t_beg + k, 0), page(t_beg + k, 1), lane);
        if (t_beg + S - 1 < tq_end) {
          n0 = page(t_beg + S - 1, 0);
          n1 = page(t_beg + S - 1, 1);
        }
      }

      // ---- Q operands and softmax state (the loads overlap the first DMAs) ----
      SegCtx<HD> q;
      const uint16_t* qh = a.q + (int64_t)b * a.q_stride + (int64_t)h * G * HD;
      // lane offsets from an opaque lane id (hoisted out of the segment loop,
      // they would hold 64-bit registers through the whole run)
      int lq = lane;
      asm volatile("" : "+v"(lq));
      const int hq = PACK ? (lq & 7) : (lq & 15);  // packed: columns c and c + 8 share head c
      const int jq = lq >> 4;
      uint16_t* qrow = &qrows[hq * QROW + jq * (HD / 4)];
      q.qn = (const uint8_t*)qrow;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (hq < G) {
          v = *(const u32x4*)(qh + hq * HD + jq * (HD / 4) + 8 * ks);
          *(u32x4*)(qrow + 8 * ks) = v;  // the same words from columns c and c + 8
        }
        const half8_t div = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f,
                             (_Float16)1.0f, (_Float16)1.0f, (_Float16)0.0625f, (_Float16)0.0625f};
        q.qp[ks] = as_h8(perm_pairs(v)) * div;
      }
      WaveState<HD> st;
#pragma unroll
      for (int nt = 0; nt < CPL; ++nt) st.o[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
      st.ob = floatx4{0.f, 0.f, 0.f, 0.f};
      st.m = -1.0e30f;

      const int r_beg = max(t_beg, ov / kGroup);  // first fp16 residual tile
      if (t_beg < tq_end) {
        const LaneMap lm = lane_map<HD, P>(lane);
        int slot = 0;
        for (int i = t_beg; i < tq_end; ++i) {
          const int ahead = slot == 0 ? S - 1 : slot - 1;  // (slot + S - 1) % S
          if (i + S - 1 < tq_end) {
            if (FUSED && i + S - 1 == g_age) {
              wait_new();
              load_stage<HD, P, true>(&ring[ahead], sb, n0, n1, lane);
            } else {
              load_stage<HD, P>(&ring[ahead], sb, n0, n1, lane);
            }
            if (i + S < tq_end) {
              n0 = page(i + S, 0);
              n1 = page(i + S, 1);
            }
            wait_vm<(S - 1) * L>();
          } else {
            wait_stages<L, S>(tq_end - 1 - i);
          }
          if (a.stamps && t_first == 0) t_first = __builtin_amdgcn_s_memrealtime();
          const VData vd = load_v<HD, P>(&ring[slot], lm);
          const half8_t pa = qk_softmax<HD, P, PACK>(st, q, &ring[slot], lm, nb, sscale, lane);
          st.ob = mfma(pa, as_h8(vd.vz4), st.ob);  // sum_t P z_t
          pv_group<HD>(st, pa, vd, nb, big_scales(vd), false, PStash(nullptr));
          // the range test comes last, so the steps above stay one block for
          // the scheduler (a branch between them costs the common case ~15%)
          if (__builtin_expect(wide_group<HD>(&ring[slot], lane), 0))
            exact_fix_group<HD, P, PACK>(st, q, &ring[slot], lm, nb, sscale, lane, pa, vd);
          slot = slot == S - 1 ? 0 : slot + 1;
          progress(1);
        }
      }

      // ---- fp16 residual tiles (all loads of a tile issued before its first use) ----
      if constexpr (FUSED) {
        if (aging && r_beg < t_fin) wait_new();
      }
      for (int i = r_beg; i < t_fin; ++i) {
        ResTile<HD> cur =
            (FUSED && aging) ? load_res<HD, FUSED, true>(a, g, b, h, ov, n, i, lane, new_row)
                             : load_res<HD, FUSED, false>(a, g, b, h, ov, n, i, lane, new_row);
        const int tn = min(kGroup, n - i * kGroup);  // 0 only for an empty sequence
        floatx4 sres[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          sres[tt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) sres[tt] = mfma(as_h8(cur.kv[tt][ks]), q.n(ks), sres[tt]);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
            if (8 * j + 4 * tt + ii >= tn) sres[tt][ii] = -INFINITY;
        }
        // rows past the end carry P = 0 but must not carry NaN/Inf garbage
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (8 * j + r >= tn) cur.vr[r] = typename ResTile<HD>::vrow_t(0u);
        // P also goes to LDS in fp32 (slot 0 is idle: every stage DMA has
        // landed), for the exact correction of values above kFastRange
        const PStash ps(ring[0].k);
        const half8_t prh = softmax_tile<HD>(st, sres[0], sres[1], sscale, 0.0f, j, true, ps);
        half2_t vmax = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
          for (int e = 0; e < (int)(sizeof(cur.vr[0]) / 4); ++e)
            vmax = __builtin_elementwise_max(vmax, __builtin_elementwise_abs(as_h2(cur.vr[r][e])));
        const bool wide = __builtin_amdgcn_ballot_w64((float)vmax[0] > kFastRange ||
                                                      (float)vmax[1] > kFastRange) != 0;
        // B operand of output columns nt: the tile rows' channels 16 nt + c
        auto cols = [&](int nt) {
          u32x4 vb;
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            const uint32_t va = cur.vr[2 * qq][nt >> 1], vb2 = cur.vr[2 * qq + 1][nt >> 1];
            vb[qq] = (nt & 1) ? __builtin_amdgcn_perm(vb2, va, 0x07060302u)
                              : __builtin_amdgcn_perm(vb2, va, 0x05040100u);
          }
          return as_h8(vb);
        };
        // A residual tile (a few per segment, not the hot loop) takes one
        // arithmetic or the other, chosen before its PV step: a correction
        // after the fp16 step would turn an infinite value into inf - inf.
        if (__builtin_expect(wide, 0)) {  // fp32 P against the (exact) fp16 values
#pragma unroll
          for (int nt = 0; nt < CPL; ++nt) {
            const half8_t vh = cols(nt);
#pragma unroll
            for (int i = 0; i < 8; ++i) st.o[nt] = mfma32(ps.get(i), (float)vh[i], st.o[nt]);
          }
          // Sigma P into the sum columns; the column test is redone from an
          // opaque lane id, not kept live
          int ln = lane;
          asm volatile("" : "+v"(ln));
          const float one = sum_lane<HD>(ln & 15) ? 1.0f : 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) st.ob = mfma32(ps.get(i), one, st.ob);
        } else {
#pragma unroll
          for (int nt = 0; nt < CPL; ++nt) st.o[nt] = mfma(prh, cols(nt), st.o[nt]);
          const uint32_t one2 = sum_col ? 0x3C003C00u : 0u;  // Sigma P into the sum columns
          st.ob = mfma(prh, as_h8(u32x4{one2, one2, one2, one2}), st.ob);
        }
        progress(kResidualUnits);
      }

      // ---- segment output: O directly, or a partial for the merge workgroups ----
      // row sums: Sigma P of O row 4j + i sits in the sum column C1 of row
      // block j; a sum lane takes its group's Sigma P z from its left neighbour
      const bool whole = (t_beg == 0 && t_fin == T);
      const int64_t piece = (int64_t)b * NKV + h + w;
      float rowscale[4], zsum[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float li = __shfl(st.ob[i], 16 * j + C1, 64);
        const float left = __shfl(st.ob[i], lane - 1, 64);
        zsum[i] = sum_col ? left : st.ob[i];
        rowscale[i] = whole ? 1.0f / fmaxf(li, 1.0e-30f) : 1.0f;
      }
      float* dst = whole ? a.out + (int64_t)b * a.out_stride + (int64_t)h * G * HD
                         : a.ws_acc + piece * G * HD;
      // the lane's output offset, computed here: hoisted out of the segment
      // loop it would hold two registers for the whole run
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int lane_off = (ln >> 4) * 4 * HD + CPL * (ln & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * j + i;
        if (row < G) {
          float v[CPL];
#pragma unroll
          for (int nt = 0; nt < CPL; ++nt) v[nt] = (st.o[nt][i] + zsum[i]) * rowscale[i];
          float* p = dst + lane_off + i * HD;
          if (whole) {
#pragma unroll
            for (int q4 = 0; q4 < CPL / 4; ++q4)
              *(floatx4*)(p + 4 * q4) =
                  floatx4{v[4 * q4], v[4 * q4 + 1], v[4 * q4 + 2], v[4 * q4 + 3]};
          } else if (CPL == 4) {  // read by a merge wavefront, possibly on another XCD
            st_agent4(p, floatx4{v[0], v[1], v[2], v[3]});
          } else {
            // agent-scope stores bypass the L2, so each instruction should
            // write whole sectors: lane c of the row's 16 takes floats
            // 4c .. 4c + 3 and then 64 + 4c .. 64 + 4c + 3 (held by lanes c / 2
            // and 8 + c / 2, half c % 2), two 256-byte contiguous stores
            float* row_base = dst + (((ln >> 4) << 2) + i) * HD;
            const int cl = ln & 15, src0 = (ln & 48) + (cl >> 1), hi = cl & 1;
#pragma unroll
            for (int part = 0; part < 2; ++part) {
              const int src = src0 + 8 * part;
              floatx4 o;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float lo_half = __shfl(v[e], src, 64), hi_half = __shfl(v[4 + e], src, 64);
                o[e] = hi ? hi_half : lo_half;
              }
              st_agent4(row_base + 64 * part + 4 * cl, o);
            }
          }
        }
      }
      if (!whole) {
        float lh[4];  // Sigma P of head c (rows 4 (c >> 2) + i)
#pragma unroll
        for (int i = 0; i < 4; ++i) lh[i] = __shfl(st.ob[i], 16 * (c >> 2) + C1, 64);
        if (j == 0 && c < G) {
          const int ci = c & 3;
          st_agent(a.ws_ml + (piece * G + c) * 2, st.m,
                   ci == 0 ? lh[0] : ci == 1 ? lh[1] : ci == 2 ? lh[2] : lh[3]);
        }
        // only a run's first and last segments can be cut
        (t_beg == 0 ? cut_last : cut_first) = piece;
      }
      // fused step: the wavefront that decoded the whole aging segment was its
      // only reader; it clears the writer's flags (a cut one: its merge)
      if constexpr (FUSED) {
        if (ages && whole && lane < step_flags<HD>())
          __hip_atomic_store(a.ws_wflag + step_flags<HD>() * ((int64_t)b * NKV + h) + lane, 0ull,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (x_rot < 0) break;
    // the second pass: the rotated-away first segment
    x = x_rot;
    xe = x_rot_end;
    sp = sp_rot;
    kvh = kvh_rot;
    u = u_rot;
    x_rot = -1;
  }
  // flags after the run: the partials are complete at the point of coherence
  // before their flags are
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane == 0) {
    if (cut_first >= 0)
      __hip_atomic_store(a.ws_flag + cut_first, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (cut_last >= 0)
      __hip_atomic_store(a.ws_flag + cut_last, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (FUSED) return t_wait;  // profiling: the wait, not t_first
  return t_first;
}



// The per-query kernels (PQ) keep one more run's state live across their run
// loop, which at three waves per SIMD spills; they run with the register
// budget of two (the v1 symbols decode one sequence, or the causal prefixes
// of one, far from filling the device).
template <int HD, int P, bool PACK, bool PQ, bool FUSED>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(
    PQ ? 1 : min_waves_per_simd<HD, PACK>()))) void kivi_decode_stream_kernel(KiviGeo g,
                                                                              DecodeArgs a) {
  constexpr int S = stages<HD, PACK>();
  static_assert(S >= 2 && S <= 4, "wait_stages covers up to 3 stages in flight");
  __shared__ __attribute__((aligned(16))) StageBuf<HD> ring[S];
  // Q rows of the current segment, one per MFMA column head (rows past G stay zero)
  // Q rows padded by 16 bytes: at a 2 HD-byte stride (a multiple of the 256
  // bytes the LDS banks span) the rows' k-step reads would all hit the same
  // banks, an 8-way conflict on every read
  constexpr int QROW = HD + 8;
  __shared__ __attribute__((aligned(16))) uint16_t qrows[(PACK ? 8 : 16) * QROW];

  const int lane = threadIdx.x;
  const uint64_t t_start = a.stamps ? __builtin_amdgcn_s_memrealtime() : 0;
  // the stream wavefronts (in the fused step the first writer_waves of them
  // do the writer's work first), then the merges
  const int bid = (int)blockIdx.x;
  uint64_t writer_bit = 0;  // profiling: marks a writer wavefront's stamp
  if constexpr (FUSED) {
    if (bid < a.writer_waves) {
      // top issue priority: the stream wavefronts start at 3 too, and a
      // writer left below them ran for about 100 us while decode wavefronts
      // waited for its age-outs
      __builtin_amdgcn_s_setprio(3);
      step_writer<HD>(g, a, bid, lane);
      writer_bit = 1ull << 62;
    }
  }
  if (bid >= a.waves) {
    // profiling: the ticks from the merge's start to the end of its last wait
    // (bits 32-55) and the load rounds after that wait (bits 56-61)
    const uint64_t t_wait = merge_segments<HD, PACK, PQ, FUSED>(g, a, lane);
    write_stamp(a, t_start, t_wait << 32, lane);
    return;
  }
  if constexpr (PQ) {
    const Nibble nb;
    // the ones block of every stage (the DMAs never write it)
    if (lane < 32) {
#pragma unroll
      for (int s_ = 0; s_ < S; ++s_) ((uint32_t*)ring[s_].ones)[lane] = 0x3C003C00u;
    }
    // rows past G are read as zeros by the columns that carry no head
    for (int i = lane; i < (int)(sizeof(qrows) / 16); i += 64)
      ((u32x4*)qrows)[i] = u32x4{0u, 0u, 0u, 0u};
    const float sscale = 1.4426950408889634f / __builtin_sqrtf((float)HD);  // log2(e)/sqrt(HD)
    for (int64_t r = bid;; r += a.waves) {
      const RunLoc rl = locate_run(g, a, r, lane);
      if (rl.q < 0) break;
      const int64_t TTq = (int64_t)g.nkv * rl.units, wl = r - rl.r0;
      const int64_t x0 = wl * TTq / rl.runs, x1 = (wl + 1) * TTq / rl.runs;
      if (x0 >= x1) continue;
      stream_run<HD, P, PACK, false>(g, a, ring, qrows, nb, sscale, lane, x0, x1,
                                     SeqSpan{rl.q, 0, rl.units}, false, 0, 0, 0, (int)r);
    }
    return;
  }
  const int G = g.gqa, NKV = g.nkv;
  // Up to 64 sequences, one length load per lane serves the stream's total,
  // the run's first sequence and that sequence's window: the first block-table
  // read waits for one memory round, not three.
  const bool one_pass = a.batch <= 64;
  int lane_T = 0, lane_ov = 0, lane_n = 0, lane_U = 0;
  if (one_pass && lane < a.batch) {
    lane_T = seq_tiles(g, a, lane, &lane_ov, &lane_n);
    lane_U = lane_ov / kGroup + kResidualUnits * (lane_T - lane_ov / kGroup);
  }
  const int lane_incl = wave_incl_scan(lane_U, lane);
  const int64_t TT = one_pass ? (int64_t)NKV * __builtin_amdgcn_readlane(lane_incl, 63)
                              : stream_units(g, a, lane);
  const int64_t W = stream_waves(TT, a.waves, true);
  const int w = bid;
  const int64_t nw = FUSED ? a.writer_waves : 0;
  if (w >= W) return;
  const int64_t x0 = run_begin(w, TT, W, nw), x1 = run_begin(w + 1, TT, W, nw);
  if (x0 >= x1) return;

  const Nibble nb;
  // the ones block of every stage (the DMAs never write it)
  if (lane < 32) {
#pragma unroll
    for (int s_ = 0; s_ < S; ++s_) ((uint32_t*)ring[s_].ones)[lane] = 0x3C003C00u;
  }
  // rows past G are read as zeros by the columns that carry no head
  for (int i = lane; i < (int)(sizeof(qrows) / 16); i += 64) ((u32x4*)qrows)[i] = u32x4{0u, 0u, 0u, 0u};
  const float sscale = 1.4426950408889634f / __builtin_sqrtf((float)HD);  // log2(e)/sqrt(HD)

  SeqSpan sp;
  int first_T = 0, first_ov = 0, first_n = 0;  // the first segment's window (one_pass)
  if (one_pass) {
    const uint64_t hit =
        __builtin_amdgcn_ballot_w64(lane < a.batch && (int64_t)NKV * lane_incl > x0);
    const int f = __builtin_ctzll(hit);  // x0 < TT: some lane hits
    const int Uf = __builtin_amdgcn_readlane(lane_U, f);
    sp = {f, (int64_t)NKV * (__builtin_amdgcn_readlane(lane_incl, f) - Uf), Uf};
    first_T = __builtin_amdgcn_readlane(lane_T, f);
    first_ov = __builtin_amdgcn_readlane(lane_ov, f);
    first_n = __builtin_amdgcn_readlane(lane_n, f);
  } else {
    sp = locate(g, a, x0, lane);
  }
  const uint64_t t_first = stream_run<HD, P, PACK, FUSED>(
      g, a, ring, qrows, nb, sscale, lane, x0, x1, sp, one_pass, first_T, first_ov, first_n, w);
  // profiling: the run's units (bits 0-31) and the ticks to its first group (32-63)
  if constexpr (FUSED) {  // profiling: the run's units and the ticks it waited for the writer
    write_stamp(a, t_start,
                writer_bit | (uint64_t)(x1 - x0) | ((t_first & ((1ull << 30) - 1)) << 32), lane);
    return;
  }
  write_stamp(a, t_start, (uint64_t)(x1 - x0) | ((t_first ? t_first - t_start : 0) << 32), lane);
}

template <int HD, int P>
static void launch_one(const KiviGeo& g, const DecodeArgs& a, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
  const dim3 grid(a.waves + a.merge_wgs);
  const dim3 block(64);
  if (a.writer_waves > 0) {
    if (g.gqa <= 8)
      hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, true, false, true>), grid, block, 0,
                            stream, start, stop, 0, g, a);
    else
      hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, false, false, true>), grid, block,
                            0, stream, start, stop, 0, g, a);
  } else if (g.gqa <= 8 && a.per_query) {
    hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, true, true, false>), grid, block, 0,
                          stream, start, stop, 0, g, a);
  } else if (g.gqa <= 8) {
    hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, true, false, false>), grid, block, 0,
                          stream, start, stop, 0, g, a);
  } else if (a.per_query) {
    hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, false, true, false>), grid, block, 0,
                          stream, start, stop, 0, g, a);
  } else {
    hipExtLaunchKernelGGL((kivi_decode_stream_kernel<HD, P, false, false, false>), grid, block,
                          0, stream, start, stop, 0, g, a);
  }
}

hipError_t launch_decode_mfma(const KiviGeo& g, const DecodeArgs& args, int batch,
                              hipStream_t stream, const LaunchEvents& ev) {
  // One launch: the stream wavefronts, then the merge workgroups (at most
  // half as many as stream slots, each taking segments in turn).  Every
  // launch gets its own epoch, which marks the partials it stores.
  // Epochs start from a random 64-bit value with the top bit set, so that
  // leftover workspace contents (zeros, small integers, earlier epochs of
  // other processes) are unlikely to match one.
  static std::atomic<uint64_t> epochs{[] {
    std::random_device rd;
    const uint64_t t = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
    const uint64_t r = ((uint64_t)rd() << 32) ^ rd() ^ (t * 0x9E3779B97F4A7C15ull);
    return (r >> 2) | (1ull << 63);  // room for 2^62 launches before the top bit clears
  }()};
  DecodeArgs a = args;
  a.epoch = epochs.fetch_add(1, std::memory_order_relaxed);
  a.stamps = g_stamps.load(std::memory_order_relaxed);
  a.stamp_cap = g_stamp_cap.load(std::memory_order_relaxed);
  a.merge_wgs = std::max(1, std::min(batch * g.nkv, a.waves / 2));
  a.merge_timeout = kMergeTimeoutTicks;
  a.merge_skew = 0;
  if (const uint64_t t = g_test_merge_timeout_ticks.load(std::memory_order_relaxed)) {
    a.merge_timeout = t;
    a.merge_skew = 1;
  }
  // Profiling only.  With main_end, the kernel's start and end are stamped by
  // the command processor (its own duration, as a kernel trace reads it);
  // that launch form delays the next kernel by a few microseconds, so without
  // main_end a plain record precedes the launch instead.
  hipError_t e;
  const bool split = ev.main_end != nullptr;
  if (!split && ev.start && (e = hipEventRecord(ev.start, stream)) != hipSuccess) return e;
  hipEvent_t s0 = split ? ev.start : nullptr, s1 = split ? ev.main_end : nullptr;
  if (g.hd == 128 && g.page == 16)
    launch_one<128, 16>(g, a, stream, s0, s1);
  else if (g.hd == 128)
    launch_one<128, 32>(g, a, stream, s0, s1);
  else if (g.page == 16)
    launch_one<64, 16>(g, a, stream, s0, s1);
  else
    launch_one<64, 32>(g, a, stream, s0, s1);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  return ev.end ? hipEventRecord(ev.end, stream) : hipSuccess;
}

// One resident wavefront per slot: the tile stream is cut into as many runs as
// the device holds waves of this kernel at once (registers and LDS decide how
// many fit on a CU), so no CU idles and none runs a second round.
template <int HD, int P, bool PACK>
static int resident_per_cu() {
  static int n = 0;
  if (n == 0) {
    int k = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, kivi_decode_stream_kernel<HD, P, PACK, false, false>,
                                                     64, 0) != hipSuccess ||
        k < 1)
      k = 8;
    n = k;
  }
  return n;
}

template <int HD, int P>
static int resident_per_cu(const KiviGeo& g) {
  return g.gqa <= 8 ? resident_per_cu<HD, P, true>() : resident_per_cu<HD, P, false>();
}

int decode_stream_waves(const KiviGeo& g, int cus) {
  int per = 8;
  if (g.hd == 128 && g.page == 16)
    per = resident_per_cu<128, 16>(g);
  else if (g.hd == 128)
    per = resident_per_cu<128, 32>(g);
  else if (g.page == 16)
    per = resident_per_cu<64, 16>(g);
  else
    per = resident_per_cu<64, 32>(g);
  return cus * per;
}

}  // namespace jacq
