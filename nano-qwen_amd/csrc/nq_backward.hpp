// Parameters shared by the attention backward kernels (bf16 MFMA and fp32
// MFMA forms).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nq {

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;  // (B, Hq, S) natural log
  // scratch written by bwd_dq_kernel: per (batch, head) and 32-row query
  // tile, 64 floats = [32 x LSE * log2(e) | 32 x Delta], rows past S zero
  float* ws;
  int nst;           // 32-row tiles per (batch, head)
  void* dq;
  void* dk;
  void* dv;
  int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss;
  int64_t osb, osh, oss, dosb, dosh, doss;
  int64_t dqsb, dqsh, dqss, dksb, dksh, dkss, dvsb, dvsh, dvss;
  int B, Hq, Hkv, G, S, T, BM, nqb, coff;
  float scale, scale_log2;
  // key padding: sequence b attends keys [0, kv_lens[b]) (clamped to
  // [0, T]; the rest get zero gradients); NULL = all T keys
  const int32_t* kv_lens;
  // additive attention bias as in the forward (bias[b, h, i, j], keys
  // contiguous, rows readable up to T rounded up to 8), and its transpose
  // bias_t[b, h, j, i] (queries contiguous, rows readable up to S rounded up
  // to 8) for the dK/dV kernel, whose lanes hold keys; NULL = no bias
  const void* bias;
  int64_t bsb, bsh, bss;
  const void* bias_t;
  int64_t btsb, btsh, btss;
};

// Keys sequence b attends.
__device__ __forceinline__ int bw_keys(const BwdParams& p, int b) {
  if (!p.kv_lens) return p.T;
  const int l = p.kv_lens[b];
  return l < 0 ? 0 : (l > p.T ? p.T : l);
}

// Scratch slot of query row s of (batch b, head h): LSE * log2(e) at the
// returned index, Delta 32 floats later.
__device__ __forceinline__ int64_t bw_ws_index(const BwdParams& p, int b, int h, int s) {
  return (((int64_t)b * p.Hq + h) * p.nst + s / 32) * 64 + (s & 31);
}

// The fp32 backward (every tensor fp32; products on v_mfma_f32_32x32x2_f32).
hipError_t launch_bwd_f32(const BwdParams& p, int D, bool causal, hipStream_t st);

// The head_dim 256 backward (bf16, no key lengths or bias): dQ with Delta,
// then dK/dV; p.nqb counts 64-row query blocks.
hipError_t launch_bwd_wide(const BwdParams& p, bool causal, hipStream_t st);

}  // namespace nq
