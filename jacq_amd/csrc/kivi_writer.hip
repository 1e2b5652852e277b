// kivi_writer.hip -- KIVI cache writer for gfx950.
//
// One workgroup per (kv head, sequence, K or V) performs that array's whole
// write in a single launch: append the new fp16 tokens to the residual
// scratch, quantise every 32-token group that ages out (K per channel over
// the group's tokens, V per token over 32-channel groups), and shift the
// scratch.  K and V share nothing, so splitting them halves the latency of the
// workgroups that age a group out, which set the launch's time.  The reference does
// the same in up to four launches, two of them with one thread per block
// (integrations/vllm_kivi/source_patch.py:1532-1697, batched :1705-1775).
//
// Arithmetic is kept bit-exact with the reference: fp32 fminf/fmaxf over fp16
// inputs, scale = (max - min) / 15 with
// IEEE division, scale <= 0 -> 1, codes = clamp(rint((x - min) / scale)),
// scale and min stored as fp16 with round-to-nearest-even.
#include "kivi_kernels.h"

namespace jacq {


constexpr int kWriterThreads = 256;

// 16-byte vector as a native vector type: arrays of it stay in registers
// (HIP's uint4 class does not).
typedef uint32_t w4 __attribute__((ext_vector_type(4)));
typedef uint32_t w2 __attribute__((ext_vector_type(2)));

#pragma clang fp contract(off)

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, not for its global stores (those have no reader in the kernel).
// The memory clobber keeps the compiler from moving LDS accesses across it.
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__global__ __launch_bounds__(kWriterThreads) __attribute__((amdgpu_waves_per_eu(2))) void kivi_append_kernel(KiviGeo g, AppendArgs a) {
  __shared__ w4 x_tile[kGroup * 128 / 8];       // 32 tokens x HD fp16, HD <= 128
  __shared__ w4 x_code_tile[kGroup * 64 / 16];  // 32 tokens x HD/2 code bytes

  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const bool is_v = blockIdx.z != 0;  // this workgroup writes V (else K)
  const int tid = threadIdx.x;
  const int HD = g.hd;
  const int VPR = HD / 8;  // 16-byte vectors per fp16 row
  const int HDP = HD / 2;
  const int HDG = HD / kGroup;
  const int P = g.page;
  const int ppg = kGroup / P;

  const int start = a.start_lens ? a.start_lens[b] : a.start_len;
  const int n = a.num_new;
  if (start < 0 || n < 1) return;
  const int old0 = split_old_tokens(start, g.residual);
  const int r0 = start - old0;
  const int end = start + n;
  const int old1 = split_old_tokens(end, g.residual);
  const int r1 = end - old1;
  const int D = old1 - old0;
  const bool in_scratch = (r0 + n <= g.rs);

  uint16_t* xs = (is_v ? a.v_scr : a.k_scr) + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const int64_t tok_stride = (int64_t)g.nkv * HD;
  const uint16_t* nx = (is_v ? a.new_v : a.new_k) + (int64_t)b * a.new_stride + (int64_t)h * HD;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  // Row p of the concatenated stream [scratch rows 0..r0) ++ [new tokens].
  // Appended rows are always read from NEW_K / NEW_V, so nothing below reads
  // what this kernel writes to the scratch.
  auto xrow = [&](int p) -> const uint16_t* {
    if (p < r0) return xs + (int64_t)p * HD;
    return nx + (int64_t)(p - r0) * tok_stride;
  };

  // The first aged group's 32 rows go to LDS (the stores below cannot touch
  // them: phase 1 writes rows >= r0, the shift only after its barrier).  All
  // of a thread's loads are issued before its LDS stores: one memory latency.
  constexpr int kTilePer = kGroup * 128 / 8 / kWriterThreads;  // w4 per thread, HD <= 128
  w4 tx[kTilePer];
  auto load_tile = [&](int gi) {
#pragma unroll
    for (int j = 0; j < kTilePer; ++j) {
      const int i = min(tid + j * kWriterThreads, kGroup * VPR - 1);
      const int t = i / VPR, c = i % VPR;
      tx[j] = *(const w4*)(xrow(gi * kGroup + t) + c * 8);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < kTilePer; ++j) {
      const int i = tid + j * kWriterThreads;
      if (i < kGroup * VPR) x_tile[i] = tx[j];
    }
  };
  // Physical pages of an aged group (first_page, first_page + 1 at page 16),
  // read through the constant address space: wave-uniform scalar loads,
  // issued for the first group together with its tile.
  const __attribute__((address_space(4))) int32_t* btc =
      (const __attribute__((address_space(4))) int32_t*)bt;
  auto group_pages = [&](int gi, int* p0, int* p1) {
    const int fp = (old0 / kGroup + gi) * ppg;
    *p0 = *p1 = -1;
    if (fp + ppg <= g.max_pages) {
      *p0 = btc[fp];
      if (ppg == 2) *p1 = btc[fp + 1];
    }
  };
  int gp0 = -1, gp1 = -1;
  if (D > 0) {
    group_pages(0, &gp0, &gp1);
    load_tile(0);
  }

  // Shift sources of the first pass (phase 3), loaded now so that their
  // latency overlaps the quantisation.
  constexpr int kShiftRows = 128;
  constexpr int kPer = kShiftRows * 16 / kWriterThreads;  // w4 per thread per array, HD <= 128
  const bool shift = !(in_scratch && D == 0);
  w4 shx[kPer];
  const int rows0 = shift ? min(kShiftRows, r1) : 0;
  // every load unconditional (a lane past the last row re-reads the last
  // row): under a per-lane branch the compiler waited for each load before
  // issuing the next
  if (rows0 > 0) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = min(tid + j * kWriterThreads, rows0 * VPR - 1);
      const int r = i / VPR, c = i % VPR;
      shx[j] = *(const w4*)(xrow(D + r) + c * 8);
    }
  }

  if (D > 0) store_tile();

  // Every load above lands before any store below (wait + barrier).
  __syncthreads();

  // Phase 1 (reference order: append, then age out, then shift): in the
  // in-scratch case the appended rows [r0, r0+n) that the shift does not
  // overwrite, i.e. [max(r0, r1'), r0+n) with r1' = r1 when a group ages out,
  // stay visible (as live rows or as the reference's stale rows).  The shift
  // rewrites the others, so they are not stored and no store of this kernel
  // is ordered against another (append_scratch_token_kernel /
  // append_scratch_tokens_batched_kernel).
  if (in_scratch) {
    const int keep_from = D > 0 ? max(r0, r1) : r0;
    for (int i = tid; i < (r0 + n - keep_from) * VPR; i += kWriterThreads) {
      const int r = keep_from + i / VPR, c = i % VPR;
      *(w4*)(xs + (int64_t)r * HD + c * 8) = *(const w4*)(xrow(r) + c * 8);
    }
  }

  // Phase 2: quantise each aged group (pack_key/pack_value_age_out_page_kernel).
  // Every thread works: a K workgroup uses four threads per channel pair (8
  // tokens each), a V workgroup two per (token, 32-channel group) (16
  // channels each); the partial min / max merge through shuffles, in any
  // order since min_num / max_num are associative.  Codes are packed into LDS and stored as whole 16-byte row pieces.
  uint8_t* const code_tile = (uint8_t*)x_code_tile;
  for (int gi = 0; gi < D / kGroup; ++gi) {
    const int lg = old0 / kGroup + gi;
    const int first_page = lg * ppg;
    if (gi > 0) {
      group_pages(gi, &gp0, &gp1);
      load_tile(gi);
      store_tile();
      lds_barrier();
    }
    const bool table_ok = first_page + ppg <= g.max_pages;
    auto phys_of = [&](int k) { return k == 0 ? gp0 : gp1; };  // page k of the group
    const uint16_t* kt = (const uint16_t*)x_tile;
    const uint16_t* vt = (const uint16_t*)x_tile;
    if (!is_v && tid < 2 * HD) {
      // K: channel pair p = tid / 4 (channels 2p, 2p + 1), tokens 8q..8q+7.
      const int pr = tid >> 2, q = tid & 3, d0 = 2 * pr, t0 = 8 * q;
      float mn0 = h2f(kt[t0 * HD + d0]), mx0 = mn0;
      float mn1 = h2f(kt[t0 * HD + d0 + 1]), mx1 = mn1;
#pragma unroll
      for (int t = t0 + 1; t < t0 + 8; ++t) {
        const float x0 = h2f(kt[t * HD + d0]), x1 = h2f(kt[t * HD + d0 + 1]);
        mn0 = min_num(mn0, x0);
        mx0 = max_num(mx0, x0);
        mn1 = min_num(mn1, x1);
        mx1 = max_num(mx1, x1);
      }
#pragma unroll
      for (int off = 1; off < 4; off <<= 1) {  // merge the four quarters
        mn0 = min_num(mn0, __shfl_xor(mn0, off, 64));
        mx0 = max_num(mx0, __shfl_xor(mx0, off, 64));
        mn1 = min_num(mn1, __shfl_xor(mn1, off, 64));
        mx1 = max_num(mx1, __shfl_xor(mx1, off, 64));
      }
      float s0 = (mx0 - mn0) / 15.0f;
      float s1 = (mx1 - mn1) / 15.0f;
      if (!(s0 > 0.0f)) s0 = 1.0f;
      if (!(s1 > 0.0f)) s1 = 1.0f;
      if (q == 0 && table_ok) {
        const uint32_t sc = (uint32_t)f2h(s0) | ((uint32_t)f2h(s1) << 16);
        const uint32_t zr = (uint32_t)f2h(mn0) | ((uint32_t)f2h(mn1) << 16);
        for (int pg = 0; pg < ppg; ++pg) {
          const int phys = phys_of(pg);
          if (phys < 0 || phys >= g.num_pages) continue;
          const int64_t base = ((int64_t)phys * g.nkv + h) * HD + d0;
          *(uint32_t*)(a.k_scale + base) = sc;
          *(uint32_t*)(a.k_zero + base) = zr;
        }
      }
#pragma unroll
      for (int t = t0; t < t0 + 8; ++t) {
        const int c0 = clamp_code((h2f(kt[t * HD + d0]) - mn0) / s0);
        const int c1 = clamp_code((h2f(kt[t * HD + d0 + 1]) - mn1) / s1);
        code_tile[t * HDP + pr] = (uint8_t)((c0 & 0x0f) | ((c1 & 0x0f) << 4));
      }
    }
    if (is_v && tid < 2 * kGroup * HDG) {
      // V: (token t, channel group cg) = tid / 2, channels 16 * (tid % 2) .. + 15.
      const int pr = tid >> 1, hf = tid & 1;
      const int t = pr / HDG, cg = pr % HDG;
      const uint16_t* row = vt + t * HD + cg * kGroup + 16 * hf;
      float mn = h2f(row[0]), mx = mn;
#pragma unroll
      for (int c = 1; c < 16; ++c) {
        const float x = h2f(row[c]);
        mn = min_num(mn, x);
        mx = max_num(mx, x);
      }
      mn = min_num(mn, __shfl_xor(mn, 1, 64));
      mx = max_num(mx, __shfl_xor(mx, 1, 64));
      float sv = (mx - mn) / 15.0f;
      if (!(sv > 0.0f)) sv = 1.0f;
      uint32_t packed[2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int code = clamp_code((h2f(row[w * 8 + k]) - mn) / sv);
          word |= (uint32_t)code << (4 * k);
        }
        packed[w] = word;
      }
      *(w2*)(code_tile + t * HDP + cg * (kGroup / 2) + 8 * hf) = w2{packed[0], packed[1]};
      if (hf == 0 && table_ok) {
        const int phys = phys_of(t / P);
        if (phys >= 0 && phys < g.num_pages) {
          const int64_t tok = ((int64_t)phys * g.nkv + h) * P + (t % P);
          a.v_scale[tok * HDG + cg] = f2h(sv);
          a.v_zero[tok * HDG + cg] = f2h(mn);
        }
      }
    }
    lds_barrier();
    // packed codes: 32 rows of HD/2 bytes, 16 bytes per thread
    if (table_ok) {
      const int RPC = HDP / 16;  // 16-byte pieces per code row
      for (int i = tid; i < kGroup * RPC; i += kWriterThreads) {
        const int r = i / RPC, c = i % RPC;
        const int phys = phys_of(r / P);
        if (phys < 0 || phys >= g.num_pages) continue;
        uint8_t* dst = (is_v ? a.v_code : a.k_code) +
                       (((int64_t)phys * g.nkv + h) * P + (r % P)) * HDP + 16 * c;
        *(w4*)dst = *(const w4*)(code_tile + r * HDP + 16 * c);
      }
    }
    lds_barrier();  // the tiles are rewritten by the next group
  }

  // Phase 3: scratch rows [0, r1) <- stream rows [D, D + r1)
  // (shift_scratch_after_age_out_kernel; nothing to do without an age-out in
  // the in-scratch case, where phase 1 already placed the new rows).  Up to
  // 128 rows per pass: every load of a pass (and every scratch read of phase
  // 2) lands before any of its stores (wait + barrier), and a later pass's
  // stores follow every earlier load.
  if (!shift) return;
  for (int r_base = 0; r_base < r1; r_base += kShiftRows) {
    const int rows = min(kShiftRows, r1 - r_base);
    if (r_base > 0) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = tid + j * kWriterThreads;
        if (i < rows * VPR) {
          const int r = r_base + i / VPR, c = i % VPR;
          shx[j] = *(const w4*)(xrow(D + r) + c * 8);
        }
      }
      __syncthreads();  // this pass's loads, in every thread, before its stores
    } else {
      // the first pass's sources were waited for before the first barrier;
      // the aged-group reads of every thread finished before their LDS
      // barriers, so only arrival is needed here
      lds_barrier();
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * kWriterThreads;
      if (i < rows * VPR) {
        const int r = r_base + i / VPR, c = i % VPR;
        *(w4*)(xs + (int64_t)r * HD + c * 8) = shx[j];
      }
    }
  }
}

hipError_t launch_append(const KiviGeo& g, const AppendArgs& a, int batch, hipStream_t stream) {
  hipLaunchKernelGGL(kivi_append_kernel, dim3(g.nkv, batch, 2), dim3(kWriterThreads), 0, stream,
                     g, a);
  return hipGetLastError();
}

}  // namespace jacq
