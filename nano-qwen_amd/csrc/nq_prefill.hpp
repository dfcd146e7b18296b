// Parameters shared by the prefill kernels (bf16 MFMA and fp32 MFMA forms).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nq {

struct PrefillParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  const float* qw;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int max_pos;
  const int32_t* q_pos;
  const int32_t* q_pos_base;
  int q_pos0;
  int B, Hq, Hkv, G, S, T, BM, nqb;
  float scale_log2;  // sm_scale * log2(e)
  // Per-sequence key counts (key padding, ragged or paged caches): sequence
  // b holds keys [0, kv_lens[b] + kv_extra), or none if kv_lens[b] lies
  // outside [0, kv_max - kv_extra] (its rows then come out NaN; a sequence
  // with no keys gives zeros); NULL = every sequence holds T.  With kv_lens
  // and neither q_pos nor q_pos0 >= 0 (decode), a query sits at position
  // keys - 1.
  const int32_t* kv_lens;
  int kv_extra, kv_max;
  // paged K/V (NULL bt = dense): key t of sequence b is row t % page of page
  // bt[b * bts + t / page], strides (ksb, ksh, kss) = (page, head, row)
  const int32_t* bt;
  int64_t bts;
  int page;
  // additive attention bias (SDPA's attn_mask: a bool mask as 0 / -inf, or a
  // float mask), in the kernel's element type: bias[b, h, i, j] at
  // b * bsb + h * bsh + i * bss + j (0 strides broadcast), each row's keys
  // contiguous and readable up to T rounded up to a multiple of 8
  const void* bias;
  int64_t bsb, bsh, bss;
};

// Keys of sequence b (-1: a length out of range).
__device__ __forceinline__ int pf_keys(const PrefillParams& p, int b) {
  if (!p.kv_lens) return p.T;
  const int l = ld_uniform(p.kv_lens, b);
  return (l < 0 || l > p.kv_max - p.kv_extra) ? -1 : l + p.kv_extra;
}

// The fp32 prefill (q, k, v, o all fp32; products on v_mfma_f32_32x32x2_f32).
// p.BM must be 128 / G (4 waves of 32 query rows).
hipError_t launch_prefill_f32(const PrefillParams& p, int D, bool causal, bool fuse, hipStream_t st);

// Plain bf16 attention at head_dim 256 (no fusion, key lengths, bias or
// pages); p.nqb counts 64-row query blocks.
hipError_t launch_prefill_wide(const PrefillParams& p, bool causal, hipStream_t st);

}  // namespace nq
