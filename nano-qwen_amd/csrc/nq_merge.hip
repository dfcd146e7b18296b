// Merge of attention partials computed over disjoint key sets.
//
// Replaces the online-softmax combine of ring attention
// (distributed/context_parallel.py:120-127, 133-134: running max, rescaled
// sum and output across the K/V chunks that arrive round the ring).  Each
// part is a normalised output O_i with the natural-log sum-exp L_i of its
// scaled scores (what nq_attn_prefill_fwd writes), so the merge is
//   L = log(exp(L_a) + exp(L_b)),  O = O_a * exp(L_a - L) + O_b * exp(L_b - L)
// applied in place to the accumulator.  A part with L = -inf holds no keys
// and contributes nothing; if both are -inf the row stays empty (O = 0).
//
// HBM-bound elementwise work: per row, two D-element reads, one write and
// three fp32 LSE words.  D/8 lanes hold a row, 8 elements each.

#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

struct MergeParams {
  void* o;                 // accumulator (B, H, S, D), updated in place
  int64_t osb, osh, oss;
  float* lse;              // (B, H, S) contiguous, updated in place
  const void* op;          // part
  int64_t psb, psh, pss;
  const float* lsep;
  int B, H, S;
};

constexpr int MERGE_MAX_BLOCKS = 2048;

template <typename T, int D>
__global__ __launch_bounds__(256) void merge_kernel(MergeParams p) {
  constexpr int LPR = D / 8;          // lanes per row
  constexpr int RPB = 256 / LPR;      // rows per block step
  const int sub = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.H * p.S;
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < nrows;
       row += (int64_t)gridDim.x * RPB) {
    const int s = (int)(row % p.S);
    const int h = (int)((row / p.S) % p.H);
    const int b = (int)(row / ((int64_t)p.S * p.H));
    T* o = reinterpret_cast<T*>(p.o) + b * p.osb + h * p.osh + s * p.oss + sub * 8;
    const T* op = reinterpret_cast<const T*>(p.op) + b * p.psb + h * p.psh + s * p.pss + sub * 8;
    const float la = p.lse[row], lb = p.lsep[row];
    const float m = fmaxf(la, lb);
    floatx8 out{};
    float L = -INFINITY;
    if (m != -INFINITY) {
      const float wa = __expf(la - m), wb = __expf(lb - m);
      const float sum = wa + wb;
      L = m + __logf(sum);
      const float ca = wa / sum, cb = wb / sum;
      // a part without keys may hold anything (it is never read)
      const floatx8 xa = ca > 0.f ? Vec8<T>::load_f32(o) : floatx8{};
      const floatx8 xb = cb > 0.f ? Vec8<T>::load_f32(op) : floatx8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = xa[e] * ca + xb[e] * cb;
    }
    store8<T>(o, out);
    if (sub == 0) p.lse[row] = L;
  }
}

template <typename T, int D>
static hipError_t launch_merge(const MergeParams& p, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t rows = (int64_t)p.B * p.H * p.S;
  const int64_t blocks = (rows + RPB - 1) / RPB;
  hipLaunchKernelGGL((merge_kernel<T, D>), dim3((unsigned)(blocks < MERGE_MAX_BLOCKS ? blocks : MERGE_MAX_BLOCKS)),
                     dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace nq

using namespace nq;

extern "C" int nq_attn_merge(void* o, const int64_t* o_strides, float* lse, const void* o_part,
                             const int64_t* part_strides, const float* lse_part, int B, int H, int S,
                             int D, int dtype, void* stream) {
  nq_clear_error();
  if (!head_dim_ok(D)) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || H <= 0 || S <= 0) return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d H=%d S=%d)", B, H, S);
  if (!o || !lse || !o_part || !lse_part || !o_strides || !part_strides)
    return nq_fail(NQ_ERR_INVALID, "outputs, parts, their LSEs and strides are required");
  if (!nq_aligned16(o) || !nq_aligned16(o_part))
    return nq_fail(NQ_ERR_INVALID, "o and o_part must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  for (int i = 0; i < 3; ++i)
    if ((o_strides[i] * esz) % 16 || (part_strides[i] * esz) % 16)
      return nq_fail(NQ_ERR_INVALID, "strides must be multiples of 16 bytes");
  MergeParams p{};
  p.o = o; p.osb = o_strides[0]; p.osh = o_strides[1]; p.oss = o_strides[2];
  p.lse = lse;
  p.op = o_part; p.psb = part_strides[0]; p.psh = part_strides[1]; p.pss = part_strides[2];
  p.lsep = lse_part;
  p.B = B; p.H = H; p.S = S;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == NQ_DTYPE_BF16)
    e = with_head_dim(D, [&](auto dc) { return launch_merge<bf16, decltype(dc)::value>(p, st); });
  else
    e = with_head_dim(D, [&](auto dc) { return launch_merge<float, decltype(dc)::value>(p, st); });
  return nq_check_launch(e);
}
