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
};

// The fp32 prefill (q, k, v, o all fp32; products on v_mfma_f32_32x32x2_f32).
// p.BM must be 128 / G (4 waves of 32 query rows).
hipError_t launch_prefill_f32(const PrefillParams& p, int D, bool causal, bool fuse, hipStream_t st);

}  // namespace nq
