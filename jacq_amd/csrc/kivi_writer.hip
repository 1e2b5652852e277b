// kivi_writer.hip -- KIVI cache writer for gfx950.
//
// One workgroup per (kv head, sequence) performs the whole write in a single
// launch: append the new fp16 tokens to the residual scratch, quantise every
// 32-token group that ages out (K per channel over the group's tokens, V per
// token over 32-channel groups), and shift the scratch.  The reference does
// the same in up to four launches, two of them with one thread per block
// (integrations/vllm_kivi/source_patch.py:1532-1697, batched :1705-1775).
//
// Arithmetic is kept bit-exact with the reference: fp32 min/max over fp16
// inputs in token (K) or channel (V) order, scale = (max - min) / 15 with
// IEEE division, scale <= 0 -> 1, codes = clamp(rint((x - min) / scale)),
// scale and min stored as fp16 with round-to-nearest-even.
#include "kivi_kernels.h"

namespace jacq {


constexpr int kWriterThreads = 256;

#pragma clang fp contract(off)

__device__ inline int clamp_code(float x) {  // source_patch.py:1517-1522
  const int code = (int)__builtin_rintf(x);
  if (code < 0) return 0;
  if (code > 15) return 15;
  return code;
}

// Compare-and-select running min/max: ties (+0 / -0) keep the earlier value.
__device__ inline float min_keep(float cur, float x) { return x < cur ? x : cur; }
__device__ inline float max_keep(float cur, float x) { return x > cur ? x : cur; }

__global__ __launch_bounds__(kWriterThreads) void kivi_append_kernel(KiviGeo g, AppendArgs a) {
  __shared__ uint4 k_tile[kGroup * 128 / 8];  // 32 tokens x HD fp16, HD <= 128
  __shared__ uint4 v_tile[kGroup * 128 / 8];

  const int h = blockIdx.x;
  const int b = blockIdx.y;
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

  uint16_t* ks = a.k_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  uint16_t* vs = a.v_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const int64_t tok_stride = (int64_t)g.nkv * HD;
  const uint16_t* nk = a.new_k + (int64_t)b * a.new_stride + (int64_t)h * HD;
  const uint16_t* nv = a.new_v + (int64_t)b * a.new_stride + (int64_t)h * HD;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  // Phase 1 (reference order): append rows [r0, r0+n) of the scratch
  // (append_scratch_token_kernel / append_scratch_tokens_batched_kernel).
  if (in_scratch) {
    for (int i = tid; i < n * VPR; i += kWriterThreads) {
      const int r = i / VPR, c = i % VPR;
      *(uint4*)(ks + (int64_t)(r0 + r) * HD + c * 8) = *(const uint4*)(nk + r * tok_stride + c * 8);
      *(uint4*)(vs + (int64_t)(r0 + r) * HD + c * 8) = *(const uint4*)(nv + r * tok_stride + c * 8);
    }
    __syncthreads();
  }

  // Row p of the concatenated stream [scratch rows 0..r0) ++ [new tokens].
  auto krow = [&](int p) -> const uint16_t* {
    if (in_scratch || p < r0) return ks + (int64_t)p * HD;
    return nk + (int64_t)(p - r0) * tok_stride;
  };
  auto vrow = [&](int p) -> const uint16_t* {
    if (in_scratch || p < r0) return vs + (int64_t)p * HD;
    return nv + (int64_t)(p - r0) * tok_stride;
  };

  // Phase 2: quantise each aged group (pack_key/pack_value_age_out_page_kernel).
  for (int gi = 0; gi < D / kGroup; ++gi) {
    const int lg = old0 / kGroup + gi;
    const int first_page = lg * ppg;
    for (int i = tid; i < kGroup * VPR; i += kWriterThreads) {
      const int t = i / VPR, c = i % VPR;
      k_tile[i] = *(const uint4*)(krow(gi * kGroup + t) + c * 8);
      v_tile[i] = *(const uint4*)(vrow(gi * kGroup + t) + c * 8);
    }
    __syncthreads();
    const bool table_ok = first_page + ppg <= g.max_pages;
    const uint16_t* kt = (const uint16_t*)k_tile;
    const uint16_t* vt = (const uint16_t*)v_tile;
    if (table_ok && tid < HDP) {
      // K: channels d0 = 2*tid, d1 = d0 + 1 over the group's 32 tokens.
      const int d0 = 2 * tid;
      float mn0 = h2f(kt[d0]), mx0 = mn0, mn1 = h2f(kt[d0 + 1]), mx1 = mn1;
      for (int t = 1; t < kGroup; ++t) {
        const float x0 = h2f(kt[t * HD + d0]), x1 = h2f(kt[t * HD + d0 + 1]);
        mn0 = min_keep(mn0, x0);
        mx0 = max_keep(mx0, x0);
        mn1 = min_keep(mn1, x1);
        mx1 = max_keep(mx1, x1);
      }
      float s0 = (mx0 - mn0) / 15.0f;
      float s1 = (mx1 - mn1) / 15.0f;
      if (!(s0 > 0.0f)) s0 = 1.0f;
      if (!(s1 > 0.0f)) s1 = 1.0f;
      const uint32_t sc = (uint32_t)f2h(s0) | ((uint32_t)f2h(s1) << 16);
      const uint32_t zr = (uint32_t)f2h(mn0) | ((uint32_t)f2h(mn1) << 16);
      for (int pg = 0; pg < ppg; ++pg) {
        const int phys = bt[first_page + pg];
        if (phys < 0 || phys >= g.num_pages) continue;
        const int64_t base = ((int64_t)phys * g.nkv + h) * HD + d0;
        *(uint32_t*)(a.k_scale + base) = sc;
        *(uint32_t*)(a.k_zero + base) = zr;
      }
      for (int t = 0; t < kGroup; ++t) {
        const int phys = bt[first_page + t / P];
        if (phys < 0 || phys >= g.num_pages) continue;
        const int c0 = clamp_code((h2f(kt[t * HD + d0]) - mn0) / s0);
        const int c1 = clamp_code((h2f(kt[t * HD + d0 + 1]) - mn1) / s1);
        a.k_code[(((int64_t)phys * g.nkv + h) * P + (t % P)) * HDP + tid] =
            (uint8_t)((c0 & 0x0f) | ((c1 & 0x0f) << 4));
      }
    } else if (table_ok && tid >= HDP && tid < HDP + kGroup * HDG) {
      // V: token t, channel group cg, over 32 channels.
      const int j = tid - HDP;
      const int t = j / HDG, cg = j % HDG;
      const uint16_t* row = vt + t * HD + cg * kGroup;
      float mn = h2f(row[0]), mx = mn;
      for (int c = 1; c < kGroup; ++c) {
        const float x = h2f(row[c]);
        mn = min_keep(mn, x);
        mx = max_keep(mx, x);
      }
      float s = (mx - mn) / 15.0f;
      if (!(s > 0.0f)) s = 1.0f;
      uint32_t packed[4];
      for (int w = 0; w < 4; ++w) {
        uint32_t word = 0;
        for (int k = 0; k < 8; ++k) {
          const int code = clamp_code((h2f(row[w * 8 + k]) - mn) / s);
          word |= (uint32_t)code << (4 * k);
        }
        packed[w] = word;
      }
      const int phys = bt[first_page + t / P];
      if (phys >= 0 && phys < g.num_pages) {
        const int64_t tok = ((int64_t)phys * g.nkv + h) * P + (t % P);
        *(uint4*)(a.v_code + tok * HDP + cg * (kGroup / 2)) =
            make_uint4(packed[0], packed[1], packed[2], packed[3]);
        a.v_scale[tok * HDG + cg] = f2h(s);
        a.v_zero[tok * HDG + cg] = f2h(mn);
      }
    }
    __syncthreads();
  }

  // Phase 3: scratch rows [0, r1) <- stream rows [D, D + r1)
  // (shift_scratch_after_age_out_kernel; nothing to do without an age-out in
  // the in-scratch case, where phase 1 already placed the new rows).
  if (in_scratch && D == 0) return;
  for (int blk = 0; blk * kGroup < r1; ++blk) {
    const int rows = min(kGroup, r1 - blk * kGroup);
    uint4 kv[2], vv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * kWriterThreads;
      if (i < rows * VPR) {
        const int r = blk * kGroup + i / VPR, c = i % VPR;
        kv[j] = *(const uint4*)(krow(D + r) + c * 8);
        vv[j] = *(const uint4*)(vrow(D + r) + c * 8);
      }
    }
    // Sources of this block never overlap its destinations (D >= 32), but the
    // previous block's sources may be this block's destinations.
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + j * kWriterThreads;
      if (i < rows * VPR) {
        const int r = blk * kGroup + i / VPR, c = i % VPR;
        *(uint4*)(ks + (int64_t)r * HD + c * 8) = kv[j];
        *(uint4*)(vs + (int64_t)r * HD + c * 8) = vv[j];
      }
    }
  }
}

hipError_t launch_append(const KiviGeo& g, const AppendArgs& a, int batch, hipStream_t stream) {
  hipLaunchKernelGGL(kivi_append_kernel, dim3(g.nkv, batch), dim3(kWriterThreads), 0, stream, g,
                     a);
  return hipGetLastError();
}

}  // namespace jacq
