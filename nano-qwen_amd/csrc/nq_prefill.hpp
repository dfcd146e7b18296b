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
  // fp32 kernel only (decode against a ragged or paged cache): sequence b
  // holds kv_lens[b] + kv_extra keys, or none if that count lies outside
  // [kv_extra, kv_max] (its rows then come out NaN; a sequence with no keys
  // gives zeros); NULL = every sequence holds T.  With kv_lens and neither
  // q_pos nor q_pos0 >= 0, a query sits at position keys - 1.
  const int32_t* kv_lens;
  int kv_extra, kv_max;
  // paged K/V: key t of sequence b is row t % page of page
  // bt[b * bts + t / page], strides (ksb, ksh, kss) = (page, head, row)
  const int32_t* bt;
  int64_t bts;
  int page;
};

// The fp32 prefill (q, k, v, o all fp32; products on v_mfma_f32_32x32x2_f32).
// p.BM must be 128 / G (4 waves of 32 query rows).
hipError_t launch_prefill_f32(const PrefillParams& p, int D, bool causal, bool fuse, hipStream_t st);

}  // namespace nq
