// fp32 attention backward for gfx950: the gradient of
// F.scaled_dot_product_attention (model/attention.py:110-115) for fp32
// tensors, with every product on v_mfma_f32_32x32x2_f32 (fp32 operands, fp32
// accumulate), as torch's autograd of the reference computes it in fp32.
//
// Given Q-hat, K-hat, V, O, dO and the forward's LSE:
//   P = exp(scale * Q K^T - LSE),  Delta = rowsum(dO * O),
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - Delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
// Two kernels, the decomposition of the bf16 backward:
//   bwd_dq_f32_kernel: a workgroup owns the G heads x 128/G positions of one
//     kv head (4 waves x 32 rows) and walks the 32-key tiles.  Lane (query
//     column, half hh) as in the fp32 forward: S^T = K Q^T and dP^T = V dO^T
//     (k-slot hh of step t = head dim hh*D/2 + t), then dQ^T += K^T dS^T, whose
//     k-slot hh of step t is key (t/4)*8 + hh*4 + t%4 = the lane's own dS^T
//     element t.  It also forms each row's Delta and stores it with LSE*log2(e)
//     in the scratch for the next kernel.
//   bwd_dkdv_f32_kernel: a workgroup owns 128 keys (32 per wave, one key column
//     per lane) and walks every 32-row query tile of its G heads, so the GQA
//     sum over heads stays in registers.  S = Q K^T and dP = dO V^T (A from the
//     LDS Q / dO tile, B = the lane's K / V row held in registers), then
//     dV^T += dO^T P and dK^T += Q^T dS, again with the lane's own elements as
//     the B operand.
// Tiles travel HBM -> registers -> LDS (XOR-swizzled 16-byte chunks: the row
// reads are conflict-free, the column reads at most 2-way).

#include "nq_backward.hpp"
#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

constexpr int BF32_NW = 4;    // waves per workgroup
constexpr int BF32_TILE = 32; // keys (dQ) or query rows (dK/dV) per tile

__device__ __forceinline__ floatx16 mfma_f32x2(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
struct BwF32 {
  static constexpr int CPR = D / 4;        // 16-byte chunks per fp32 row
  static constexpr int TILE4 = BF32_TILE * CPR;
  static constexpr int LPT = TILE4 / (64 * BF32_NW);
  __device__ static int swz(int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); }
  // float4 slot of (row, 16-byte chunk c) in a tile
  __device__ static int slot(int r, int c) { return r * CPR + (c ^ swz(r)); }
  // one fp32 element (row, column) of a tile viewed as floats
  __device__ static float at(const floatx4* t, int r, int col) { return t[slot(r, col / 4)][col % 4]; }
};

// Copy rows [r0, r0 + 32) of a strided fp32 tensor into a swizzled LDS tile
// through registers; rows at or past `nrows` become zeros.
template <int D>
struct TileCopy {
  using L = BwF32<D>;
  floatx4 r[L::LPT];
  __device__ void fetch(const float* base, int64_t row_stride, int r0, int nrows) {
#pragma unroll
    for (int u = 0; u < L::LPT; ++u) {
      const int i = threadIdx.x + 64 * BF32_NW * u;
      const int row = r0 + i / L::CPR, c = i % L::CPR;
      r[u] = row < nrows ? *reinterpret_cast<const floatx4*>(base + (int64_t)row * row_stride + c * 4) : floatx4{};
    }
  }
  __device__ void stash(floatx4* t) {
#pragma unroll
    for (int u = 0; u < L::LPT; ++u) {
      const int i = threadIdx.x + 64 * BF32_NW * u;
      t[L::slot(i / L::CPR, i % L::CPR)] = r[u];
    }
  }
};

// ---------------------------------------------------------------------------
// BIAS: the forward's additive bias (p.bias) enters every score; a row the
// bias masks entirely has LSE -inf and P = 0 (its scratch LSE is stored +inf).
template <int D, bool CAUSAL, bool BIAS = false>
__global__ void __launch_bounds__(64 * BF32_NW) bwd_dq_f32_kernel(BwdParams p) {
  using L = BwF32<D>;
  constexpr int NT = D / 2, NDO = D / 32;
  __shared__ floatx4 kt[L::TILE4];
  __shared__ floatx4 vt[L::TILE4];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r32 = lane & 31, hh = lane >> 5;
  const int npairs = p.B * p.Hkv;
  const int pair = blockIdx.x % npairs, qrank = blockIdx.x / npairs;
  const int qblk = CAUSAL ? (p.nqb - 1 - qrank) : qrank;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  const int Tk = bw_keys(p, b);  // keys this sequence attends
  const int kv_end = CAUSAL ? min(Tk, q0 + p.BM + p.coff) : Tk;
  const int ntiles = (kv_end + BF32_TILE - 1) / BF32_TILE;
  const float* kbase = reinterpret_cast<const float*>(p.k) + b * p.ksb + kvh * p.ksh;
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.vsb + kvh * p.vsh;
  TileCopy<D> kc, vc;  // rows past the sequence's keys read as zeros (padding is never read)
  kc.fetch(kbase, p.kss, 0, Tk);
  vc.fetch(vbase, p.vss, 0, Tk);

  const int R = wave * 32 + r32;
  const int g = R / p.BM, pr = R - g * p.BM;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  // this lane's halves of the query row: Q, dO (B operands) and Delta
  float x[NT], dov[NT];
  float dlt;
  {
    const int64_t boff = (int64_t)b, hoff = (int64_t)head;
    const float* qrow = reinterpret_cast<const float*>(p.q) + boff * p.qsb + hoff * p.qsh + (int64_t)qi_c * p.qss + hh * NT;
    const float* drow = reinterpret_cast<const float*>(p.dout) + boff * p.dosb + hoff * p.dosh + (int64_t)qi_c * p.doss + hh * NT;
    const float* orow = reinterpret_cast<const float*>(p.o) + boff * p.osb + hoff * p.osh + (int64_t)qi_c * p.oss + hh * NT;
    float acc = 0.f;
#pragma unroll
    for (int t4 = 0; t4 < NT / 4; ++t4) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(qrow + 4 * t4);
      const floatx4 d = *reinterpret_cast<const floatx4*>(drow + 4 * t4);
      const floatx4 o = *reinterpret_cast<const floatx4*>(orow + 4 * t4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[4 * t4 + e] = a[e];
        dov[4 * t4 + e] = d[e];
        acc = __builtin_fmaf(d[e], o[e], acc);
      }
    }
    dlt = xor32_sum(acc);
  }
  float lse2 = p.lse[((int64_t)b * p.Hq + head) * p.S + qi_c] * kLog2e;
  if (BIAS && !(lse2 > -INFINITY)) lse2 = INFINITY;  // no key kept: P = exp2(s - inf) = 0
  if (qvalid && hh == 0) {
    const int64_t wi = bw_ws_index(p, b, head, qi);
    p.ws[wi] = lse2;
    p.ws[wi + 32] = dlt;
  }
  const float* brow = BIAS ? reinterpret_cast<const float*>(p.bias) + b * p.bsb + head * p.bsh +
                                 (int64_t)qi_c * p.bss
                           : nullptr;
  if (qblk == p.nqb - 1) {  // scratch slots past S: zero
    const int pad = p.nst * 32 - p.S;
    for (int t = threadIdx.x; t < p.G * 32; t += 64 * BF32_NW) {
      if (t % 32 < pad) {
        const int64_t w2 = bw_ws_index(p, b, kvh * p.G + t / 32, p.S + t % 32);
        p.ws[w2] = 0.f;
        p.ws[w2 + 32] = 0.f;
      }
    }
  }

  floatx16 dqacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) dqacc[dd] = floatx16{};
  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();
    kc.stash(kt);
    vc.stash(vt);
    __syncthreads();
    if (j + 1 < ntiles) {
      kc.fetch(kbase, p.kss, (j + 1) * BF32_TILE, Tk);
      vc.fetch(vbase, p.vss, (j + 1) * BF32_TILE, Tk);
    }
    // S^T = K Q^T and dP^T = V dO^T (MFMA row = key r32 of the tile)
    floatx16 s = floatx16{}, dp = floatx16{};
#pragma unroll
    for (int t4 = 0; t4 < NT / 4; ++t4) {
      const floatx4 a = kt[L::slot(r32, hh * (NT / 4) + t4)];
      const floatx4 c = vt[L::slot(r32, hh * (NT / 4) + t4)];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = mfma_f32x2(a[e], x[4 * t4 + e], s);
        dp = mfma_f32x2(c[e], dov[4 * t4 + e], dp);
      }
    }
    const int n0 = j * BF32_TILE;
    const int lim = CAUSAL ? min(Tk - 1, qi + p.coff) : Tk - 1;
    float bsv[16];
    if constexpr (BIAS) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k4 = n0 + r * 8 + hh * 4;
        const floatx4 bv = k4 < Tk ? *reinterpret_cast<const floatx4*>(brow + k4) : floatx4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) bsv[r * 4 + e] = bv[e] * kLog2e;
      }
    }
    float ds[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = n0 + (i / 4) * 8 + hh * 4 + (i % 4);
      const float x = BIAS ? __builtin_fmaf(s[i], p.scale_log2, bsv[i]) - lse2 : s[i] * p.scale_log2 - lse2;
      const float pe = key <= lim ? fast_exp2(x) : 0.f;
      ds[i] = pe * (dp[i] - dlt);
    }
    // dQ^T += K^T dS^T: step t, k-slot hh = key (t/4)*8 + hh*4 + t%4
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int key = (t / 4) * 8 + hh * 4 + (t % 4);
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd)
        dqacc[dd] = mfma_f32x2(L::at(kt, key, dd * 32 + r32), ds[t], dqacc[dd]);
    }
  }
  if (!qvalid) return;
  float* dqrow = reinterpret_cast<float*>(p.dq) + b * p.dqsb + head * p.dqsh + (int64_t)qi * p.dqss;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const floatx4 t = {dqacc[dd][gq * 4 + 0] * p.scale, dqacc[dd][gq * 4 + 1] * p.scale,
                         dqacc[dd][gq * 4 + 2] * p.scale, dqacc[dd][gq * 4 + 3] * p.scale};
      *reinterpret_cast<floatx4*>(dqrow + dd * 32 + gq * 8 + hh * 4) = t;
    }
}

// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool BIAS = false>
__global__ void __launch_bounds__(64 * BF32_NW) bwd_dkdv_f32_kernel(BwdParams p) {
  using L = BwF32<D>;
  constexpr int NT = D / 2, NDO = D / 32;
  constexpr int KEYS = 32 * BF32_NW;  // keys per workgroup
  __shared__ floatx4 qt[L::TILE4];
  __shared__ floatx4 dot[L::TILE4];
  __shared__ float lse2s[BF32_TILE], dlts[BF32_TILE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r32 = lane & 31, hh = lane >> 5;
  const int npairs = p.B * p.Hkv;
  const int pair = blockIdx.x % npairs, kblk = blockIdx.x / npairs;  // lowest keys (most work) first
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int k0 = kblk * KEYS;
  const int key = k0 + wave * 32 + r32;  // this lane's key column
  const bool kvalid = key < p.T;
  const bool kattend = key < bw_keys(p, b);  // keys past the sequence's count: zero gradients

  // this lane's halves of its K and V rows (B operands of S and dP); zeros for
  // keys past T or the sequence's count (padding rows are never read)
  float kr[NT], vr[NT];
  {
    const int kc = kattend ? key : 0;
    const float* krow = reinterpret_cast<const float*>(p.k) + b * p.ksb + kvh * p.ksh + (int64_t)kc * p.kss + hh * NT;
    const float* vrow = reinterpret_cast<const float*>(p.v) + b * p.vsb + kvh * p.vsh + (int64_t)kc * p.vss + hh * NT;
#pragma unroll
    for (int t4 = 0; t4 < NT / 4; ++t4) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(krow + 4 * t4);
      const floatx4 c = *reinterpret_cast<const floatx4*>(vrow + 4 * t4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[4 * t4 + e] = kattend ? a[e] : 0.f;
        vr[4 * t4 + e] = kattend ? c[e] : 0.f;
      }
    }
  }

  floatx16 dkacc[NDO], dvacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) dkacc[dd] = dvacc[dd] = floatx16{};

  // query rows that see any of this workgroup's keys: s + coff >= k0
  const int sbeg = CAUSAL ? max(0, k0 - p.coff) / BF32_TILE * BF32_TILE : 0;
  TileCopy<D> qc, dc;
  for (int g = 0; g < p.G; ++g) {
    const int head = kvh * p.G + g;
    const float* qbase = reinterpret_cast<const float*>(p.q) + b * p.qsb + head * p.qsh;
    const float* dbase = reinterpret_cast<const float*>(p.dout) + b * p.dosb + head * p.dosh;
    for (int s0 = sbeg; s0 < p.S; s0 += BF32_TILE) {
      qc.fetch(qbase, p.qss, s0, p.S);
      dc.fetch(dbase, p.doss, s0, p.S);
      __syncthreads();  // every wave is done with the previous tile
      qc.stash(qt);
      dc.stash(dot);
      if (threadIdx.x < BF32_TILE) {
        const int s = s0 + threadIdx.x;
        const int64_t wi = bw_ws_index(p, b, head, s);
        lse2s[threadIdx.x] = s < p.S ? p.ws[wi] : INFINITY;  // rows past S: P = 0
        dlts[threadIdx.x] = s < p.S ? p.ws[wi + 32] : 0.f;
      }
      __syncthreads();
      // S = Q K^T and dP = dO V^T (MFMA row = query row r32 of the tile)
      floatx16 s = floatx16{}, dp = floatx16{};
#pragma unroll
      for (int t4 = 0; t4 < NT / 4; ++t4) {
        const floatx4 a = qt[L::slot(r32, hh * (NT / 4) + t4)];
        const floatx4 c = dot[L::slot(r32, hh * (NT / 4) + t4)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma_f32x2(a[e], kr[4 * t4 + e], s);
          dp = mfma_f32x2(c[e], vr[4 * t4 + e], dp);
        }
      }
      float bsv[16];
      if constexpr (BIAS) {
        // the transposed bias: this key's row, the tile's queries in runs of 4
        const float* brow = reinterpret_cast<const float*>(p.bias_t) + b * p.btsb + head * p.btsh +
                            (int64_t)(kattend ? key : 0) * p.btss;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q4 = s0 + r * 8 + hh * 4;
          const floatx4 bv = (kattend && q4 < p.S) ? *reinterpret_cast<const floatx4*>(brow + q4) : floatx4{};
#pragma unroll
          for (int e = 0; e < 4; ++e) bsv[r * 4 + e] = bv[e] * kLog2e;
        }
      }
      float pe[16], ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int ql = (i / 4) * 8 + hh * 4 + (i % 4);
        const bool keep = kattend && (!CAUSAL || key <= s0 + ql + p.coff);
        const float x = BIAS ? __builtin_fmaf(s[i], p.scale_log2, bsv[i]) - lse2s[ql] : s[i] * p.scale_log2 - lse2s[ql];
        pe[i] = keep ? fast_exp2(x) : 0.f;
        ds[i] = pe[i] * (dp[i] - dlts[ql]);
      }
      // dV^T += dO^T P and dK^T += Q^T dS: step t, k-slot hh = query row
      // (t/4)*8 + hh*4 + t%4 of the tile = the lane's own element t
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int ql = (t / 4) * 8 + hh * 4 + (t % 4);
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) {
          dvacc[dd] = mfma_f32x2(L::at(dot, ql, dd * 32 + r32), pe[t], dvacc[dd]);
          dkacc[dd] = mfma_f32x2(L::at(qt, ql, dd * 32 + r32), ds[t], dkacc[dd]);
        }
      }
    }
  }
  if (!kvalid) return;
  float* dkrow = reinterpret_cast<float*>(p.dk) + b * p.dksb + kvh * p.dksh + (int64_t)key * p.dkss;
  float* dvrow = reinterpret_cast<float*>(p.dv) + b * p.dvsb + kvh * p.dvsh + (int64_t)key * p.dvss;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const floatx4 tk = {dkacc[dd][gq * 4 + 0] * p.scale, dkacc[dd][gq * 4 + 1] * p.scale,
                          dkacc[dd][gq * 4 + 2] * p.scale, dkacc[dd][gq * 4 + 3] * p.scale};
      const floatx4 tv = {dvacc[dd][gq * 4 + 0], dvacc[dd][gq * 4 + 1], dvacc[dd][gq * 4 + 2],
                          dvacc[dd][gq * 4 + 3]};
      *reinterpret_cast<floatx4*>(dkrow + dd * 32 + gq * 8 + hh * 4) = tk;
      *reinterpret_cast<floatx4*>(dvrow + dd * 32 + gq * 8 + hh * 4) = tv;
    }
}

template <int D>
static hipError_t launch_f32(const BwdParams& p, bool causal, hipStream_t st) {
  const dim3 block(64 * BF32_NW);
  const dim3 gq((unsigned)(p.nqb * p.B * p.Hkv));
  const dim3 gk((unsigned)(((p.T + 32 * BF32_NW - 1) / (32 * BF32_NW)) * p.B * p.Hkv));
  if (p.bias) {
    if (causal) {
      hipLaunchKernelGGL((bwd_dq_f32_kernel<D, true, true>), gq, block, 0, st, p);
      hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, true, true>), gk, block, 0, st, p);
    } else {
      hipLaunchKernelGGL((bwd_dq_f32_kernel<D, false, true>), gq, block, 0, st, p);
      hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, false, true>), gk, block, 0, st, p);
    }
    return hipGetLastError();
  }
  if (causal) {
    hipLaunchKernelGGL((bwd_dq_f32_kernel<D, true>), gq, block, 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, true>), gk, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((bwd_dq_f32_kernel<D, false>), gq, block, 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, false>), gk, block, 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_bwd_f32(const BwdParams& p, int D, bool causal, hipStream_t st) {
  return with_head_dim(D, [&](auto dc) { return launch_f32<decltype(dc)::value>(p, causal, st); });
}

}  // namespace nq
