// kivi_decode.hip -- paged int4-KIVI decode attention for gfx950.
//
// Work decomposition (both kernels in this file):
//   grid = (split, kv head, sequence); one workgroup owns one split -- a
//   contiguous chunk of whole 32-token groups (split_plan) --
//   for ALL G query heads of its kv head, so every KV byte is read from HBM
//   once per step (the reference reads it G times, one warp per query head,
//   decode_attention_kivi_paged_library_flash.cu:51-60).
//   A sequence with one split writes O directly; otherwise the split's
//   online-softmax partials (m, l, acc[HD]) go to the workspace and
//   kivi_combine_kernel merges them with the log-sum-exp rule of
//   crates/jac-codegen-cuda/src/variants.rs:3548-3565.
//
// Per-token math is the reference's (snapshot :85-156): dequant
// code * fp16 scale + fp16 zero in fp32, score = q.k / sqrt(HD), online
// softmax m0 = -1e30, O = acc / max(l, 1e-30).
#include "kivi_kernels.h"

namespace jacq {

constexpr int kDecThreads = 256;
constexpr int kMaxG = 16;

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Straightforward VALU decode: scores with 8 threads per token, softmax with
// one wave per query head, PV with one thread per (channel pair, head set).
__global__ __launch_bounds__(kDecThreads) void kivi_decode_simple_kernel(KiviGeo g,
                                                                          DecodeArgs a) {
  __shared__ float q_s[kMaxG * 128];
  __shared__ float p_s[kMaxG * kGroup];
  __shared__ float ks_s[128], kz_s[128];
  __shared__ float m_s[kMaxG], l_s[kMaxG], corr_s[kMaxG];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int HD = g.hd, HDP = HD / 2, HDG = HD / kGroup, G = g.gqa, P = g.page;
  const int ppg = kGroup / P;

  int ov, rv;
  window_of(g, a.retained_pages, a.seq_lens ? a.seq_lens[b] : a.seq_len, &ov, &rv);
  const int n = ov + rv;
  int nsplit, chunk;
  split_plan(n, &nsplit, &chunk);
  if (split >= nsplit) return;
  const int t_begin = split * chunk;
  const int t_end = min(n, t_begin + chunk);

  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
  const uint16_t* ksr = a.k_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const uint16_t* vsr = a.v_scr + (int64_t)b * a.scr_stride + (int64_t)h * g.rs * HD;
  const uint16_t* qh = a.q + (int64_t)b * a.q_stride + (int64_t)h * G * HD;
  for (int i = tid; i < G * HD; i += kDecThreads) q_s[i] = h2f(qh[i]);
  if (tid < G) {
    m_s[tid] = -1.0e30f;
    l_s[tid] = 0.0f;
  }
  const float scale_attn = 1.0f / sqrtf((float)HD);

  // PV ownership: channel pair cp, heads hs, hs + nhs, ...
  const int cp = tid % HDP;
  const int hs = tid / HDP;
  const int nhs = kDecThreads / HDP;
  float acc[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
  __syncthreads();

  for (int t0 = t_begin; t0 < t_end; t0 += kGroup) {
    const int tn = min(kGroup, t_end - t0);
    const bool is_old = t0 < ov;
    if (is_old && tid < HD) {
      const int kp = bt[(t0 / kGroup) * ppg];
      const int64_t base = ((int64_t)kp * g.nkv + h) * HD + tid;
      ks_s[tid] = h2f(a.k_scale[base]);
      kz_s[tid] = h2f(a.k_zero[base]);
    }
    __syncthreads();

    // Scores: token t = tid / 8, channels [part*CPT, part*CPT + CPT).
    {
      const int t = tid >> 3, part = tid & 7, CPT = HD / 8;
      float kf[16];
      const bool valid = t < tn;
      if (valid) {
        if (is_old) {
          const int s = t0 + t;
          const int phys = bt[s / P];
          const uint8_t* kc =
              a.k_code + (((int64_t)phys * g.nkv + h) * P + (s % P)) * HDP + part * (CPT / 2);
          for (int i = 0; i < CPT / 2; ++i) {
            const uint32_t byte = kc[i];
            const int d = part * CPT + 2 * i;
            kf[2 * i] = (float)(byte & 15u) * ks_s[d] + kz_s[d];
            kf[2 * i + 1] = (float)(byte >> 4) * ks_s[d + 1] + kz_s[d + 1];
          }
        } else {
          const uint16_t* kr = ksr + (int64_t)(t0 - ov + t) * HD + part * CPT;
          for (int i = 0; i < CPT; ++i) kf[i] = h2f(kr[i]);
        }
      }
      for (int gi = 0; gi < G; ++gi) {
        float dot = 0.0f;
        if (valid) {
          const float* qg = q_s + gi * HD + part * CPT;
          for (int i = 0; i < CPT; ++i) dot += qg[i] * kf[i];
        }
        dot += __shfl_xor(dot, 1, 64);
        dot += __shfl_xor(dot, 2, 64);
        dot += __shfl_xor(dot, 4, 64);
        if (valid && part == 0) p_s[gi * kGroup + t] = dot * scale_attn;
      }
    }
    __syncthreads();

    // Online softmax, one wave per query head.
    for (int gi = wave; gi < G; gi += kDecThreads / 64) {
      const float s = lane < tn ? p_s[gi * kGroup + lane] : -INFINITY;
      const float mt = wave_max(s);
      const float m_old = m_s[gi];
      const float m_new = fmaxf(m_old, mt);
      const float p = lane < tn ? __expf(s - m_new) : 0.0f;
      const float lt = wave_sum(p);
      if (lane < tn) p_s[gi * kGroup + lane] = p;
      if (lane == 0) {
        const float corr = __expf(m_old - m_new);
        corr_s[gi] = corr;
        l_s[gi] = l_s[gi] * corr + lt;
        m_s[gi] = m_new;
      }
    }
    __syncthreads();

    // PV.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int gi = hs + k * nhs;
      if (gi < G) {
        acc[k][0] *= corr_s[gi];
        acc[k][1] *= corr_s[gi];
      }
    }
    for (int t = 0; t < tn; ++t) {
      float v0, v1;
      if (is_old) {
        const int s = t0 + t;
        const int phys = bt[s / P];
        const int64_t tok = ((int64_t)phys * g.nkv + h) * P + (s % P);
        const uint32_t byte = a.v_code[tok * HDP + cp];
        const float vs = h2f(a.v_scale[tok * HDG + (2 * cp) / kGroup]);
        const float vz = h2f(a.v_zero[tok * HDG + (2 * cp) / kGroup]);
        v0 = (float)(byte & 15u) * vs + vz;
        v1 = (float)(byte >> 4) * vs + vz;
      } else {
        const uint16_t* vr = vsr + (int64_t)(t0 - ov + t) * HD + 2 * cp;
        v0 = h2f(vr[0]);
        v1 = h2f(vr[1]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int gi = hs + k * nhs;
        if (gi < G) {
          const float p = p_s[gi * kGroup + t];
          acc[k][0] += p * v0;
          acc[k][1] += p * v1;
        }
      }
    }
    __syncthreads();
  }

  if (nsplit == 1) {
    float* o = a.out + (int64_t)b * a.out_stride + (int64_t)h * G * HD;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int gi = hs + k * nhs;
      if (gi < G) {
        const float inv_l = 1.0f / fmaxf(l_s[gi], 1.0e-30f);
        o[gi * HD + 2 * cp] = acc[k][0] * inv_l;
        o[gi * HD + 2 * cp + 1] = acc[k][1] * inv_l;
      }
    }
  } else {
    const int64_t slot = ((int64_t)b * g.nkv + h) * a.max_splits + split;
    float* wacc = a.ws_acc + slot * G * HD;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int gi = hs + k * nhs;
      if (gi < G) {
        wacc[gi * HD + 2 * cp] = acc[k][0];
        wacc[gi * HD + 2 * cp + 1] = acc[k][1];
      }
    }
    if (tid < G) {
      a.ws_ml[(slot * G + tid) * 2] = m_s[tid];
      a.ws_ml[(slot * G + tid) * 2 + 1] = l_s[tid];
    }
  }
}

// LSE merge of a sequence's split partials (variants.rs:3548-3565), one
// workgroup per (query head, sequence), one thread per channel.
__global__ __launch_bounds__(128) void kivi_combine_kernel(KiviGeo g, DecodeArgs a) {
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int ov, rv;
  window_of(g, a.retained_pages, a.seq_lens ? a.seq_lens[b] : a.seq_len, &ov, &rv);
  int nsplit, chunk;
  split_plan(ov + rv, &nsplit, &chunk);
  if (nsplit <= 1 || d >= g.hd) return;
  const int G = g.gqa, h = hq / G, gi = hq % G;
  const int64_t slot0 = ((int64_t)b * g.nkv + h) * a.max_splits;
  float gm = -1.0e30f;
  for (int c = 0; c < nsplit; ++c) gm = fmaxf(gm, a.ws_ml[((slot0 + c) * G + gi) * 2]);
  float gl = 0.0f, acc = 0.0f;
  for (int c = 0; c < nsplit; ++c) {
    const float m = a.ws_ml[((slot0 + c) * G + gi) * 2];
    const float l = a.ws_ml[((slot0 + c) * G + gi) * 2 + 1];
    const float corr = __expf(m - gm);
    gl += l * corr;
    acc += a.ws_acc[((slot0 + c) * G + gi) * g.hd + d] * corr;
  }
  a.out[(int64_t)b * a.out_stride + (int64_t)hq * g.hd + d] = acc * (1.0f / fmaxf(gl, 1.0e-30f));
}

hipError_t launch_decode(const KiviGeo& g, const DecodeArgs& a, int batch, hipStream_t stream,
                         hipEvent_t between) {
  hipLaunchKernelGGL(kivi_decode_simple_kernel, dim3(a.max_splits, g.nkv, batch),
                     dim3(kDecThreads), 0, stream, g, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (between && (e = hipEventRecord(between, stream)) != hipSuccess) return e;
  if (a.max_splits > 1) {
    hipLaunchKernelGGL(kivi_combine_kernel, dim3(g.nh, batch), dim3(128), 0, stream, g, a);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace jacq
