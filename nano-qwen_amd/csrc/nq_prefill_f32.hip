// fp32 GQA prefill attention for gfx950: the arithmetic the reference's SDPA
// does for fp32 inputs (model/attention.py:110-115 keeps the input dtype), with
// every product on v_mfma_f32_32x32x2_f32 (fp32 operands, fp32 accumulate) and
// the norm, rotation and softmax in fp32.  QK-Norm + RoPE of Q
// (attention.py:95-100) are fused into the Q load as in the bf16 kernel.
//
// Layout (one workgroup = 4 waves = 128 query rows of one kv head: the G heads
// of a GQA group times 128/G positions; each K/V tile in LDS serves all G):
//   S^T = K Q^T.  The MFMA's k-slot hh of step t is head dim hh*D/2 + t, so a
//   lane (key row r, half hh) reads K[r][hh*D/2 + 4u .. +4] as one float4 and
//   holds Q[q][hh*D/2 + t] for all t in registers.  The result gives each
//   lane one query column and 16 keys, (i/4)*8 + hh*4 + i%4.
//   O^T += V^T P^T.  Step t takes key (t/4)*8 + hh*4 + t%4 in k-slot hh: that
//   is the lane's own score element t, so P never moves between lanes; V^T
//   comes from the row-major V tile one float per lane.
// Tiles of 32 keys go HBM -> registers (one tile ahead) -> LDS; rows past T
// are zero-filled (their scores are masked).  LDS rows are XOR-swizzled by
// 16-byte chunk: the 16 rows one ds_read_b128 of K serves, and the two rows
// (k, k+4) one V^T read touches, land on distinct banks (D = 32: the V read
// is 2-way).
// The same kernel serves the fp32 decode (S = 1): per-sequence key counts and
// a paged cache (block table) replace the uniform T and dense strides.

#include "nq_common.hpp"
#include "nq_internal.hpp"
#include "nq_prefill.hpp"

namespace nq {

constexpr int PF32_BN = 32;  // keys per tile
constexpr int PF32_NW = 4;   // waves per workgroup, 32 query rows each

__device__ __forceinline__ floatx16 mfma32_f32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
struct F32Tile {
  static constexpr int CPR = D / 4;  // 16-byte chunks per fp32 row
  __device__ static int kswz(int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); }
  __device__ static int vswz(int r) { return CPR >= 16 ? (((r >> 2) & 1) << 3) : 0; }
};

// BIAS: p.bias (fp32) is added to every score; a row may then see no finite
// score in a tile, or in any (zeros out, LSE -inf, as SDPA gives).
template <int D, bool CAUSAL, bool FUSE_Q, bool BIAS = false>
__global__ void __launch_bounds__(64 * PF32_NW) prefill_f32_kernel(PrefillParams p) {
  using Tl = F32Tile<D>;
  constexpr int CPR = Tl::CPR;
  constexpr int NT = D / 2;   // QK steps (two head dims each)
  constexpr int NDO = D / 32; // 32-row output blocks
  constexpr int TILE4 = PF32_BN * CPR;           // float4 slots per tile
  constexpr int LPT = TILE4 / (64 * PF32_NW);    // slots per thread per tile
  static_assert(LPT >= 1 && TILE4 % (64 * PF32_NW) == 0, "tile must split over the workgroup");
  __shared__ floatx4 kt[TILE4];
  __shared__ floatx4 vt[TILE4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int r32 = lane & 31, hh = lane >> 5;

  const int npairs = p.B * p.Hkv;
  const int L = blockIdx.x;
  const int pair = L % npairs, qrank = L / npairs;
  const int qblk = CAUSAL ? (p.nqb - 1 - qrank) : qrank;  // heaviest first
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  // keys of this sequence (-1: a length out of range, no keys and NaN rows)
  const int T = pf_keys(p, b);
  // the causal frontier is bottom-right against the launch's T (query i keeps
  // keys j <= i + p.T - p.S); key_lens only shortens the key range, as in the
  // bf16 kernel and the backward
  const int coff = p.T - p.S;
  const int kv_end = max(0, CAUSAL ? min(T, q0 + p.BM + coff) : T);
  const int ntiles = (kv_end + PF32_BN - 1) / PF32_BN;

  // row `key` of this (batch, kv head): dense strides, or through the block table
  auto krow = [&](const void* base, int64_t sb, int64_t sh, int64_t ss, int key) {
    const float* f = reinterpret_cast<const float*>(base) + kvh * sh;
    if (p.bt) return f + (int64_t)p.bt[b * p.bts + key / p.page] * sb + (int64_t)(key % p.page) * ss;
    return f + b * sb + (int64_t)key * ss;
  };

  // slot i = tid + 256u of a tile: row i / CPR, chunk i % CPR (coalesced rows)
  floatx4 kr[LPT], vr[LPT];
  auto fetch = [&](int tile) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int i = tid + 64 * PF32_NW * u;
      const int key = tile * PF32_BN + i / CPR, c = i % CPR;
      if (key < T) {
        kr[u] = *reinterpret_cast<const floatx4*>(krow(p.k, p.ksb, p.ksh, p.kss, key) + c * 4);
        vr[u] = *reinterpret_cast<const floatx4*>(krow(p.v, p.vsb, p.vsh, p.vss, key) + c * 4);
      } else {
        kr[u] = floatx4{};
        vr[u] = floatx4{};
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int i = tid + 64 * PF32_NW * u;
      const int row = i / CPR, c = i % CPR;
      kt[row * CPR + (c ^ Tl::kswz(row))] = kr[u];
      vt[row * CPR + (c ^ Tl::vswz(row))] = vr[u];
    }
  };
  if (ntiles > 0) fetch(0);

  // this lane's query row: column r32 of this wave's 32 rows
  const int R = wave * 32 + r32;
  const int g = R / p.BM, pr = R - g * p.BM;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  // ---- Q operand: x[t] = Q[row][hh*D/2 + t]
  float x[NT];
  {
    const float* qrow = reinterpret_cast<const float*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qi_c * p.qss + hh * NT;
#pragma unroll
    for (int t4 = 0; t4 < NT / 4; ++t4) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(qrow + 4 * t4);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * t4 + e] = v[e];
    }
    if (FUSE_Q) {
      if (p.qw) {  // model/norm.py:17-22: (x * rsqrt(mean(x^2) + eps)) * w, fp32
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) ss = __builtin_fmaf(x[t], x[t], ss);
        ss = xor32_sum(ss);
        const float r = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
        for (int t8 = 0; t8 < NT / 8; ++t8) {
          const floatx8 w = Vec8<float>::load_f32(p.qw + hh * NT + 8 * t8);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[8 * t8 + e] = (x[8 * t8 + e] * r) * w[e];
        }
      }
      if (p.cos_tab) {  // model/rope.py:133-161, rotate-half pairs (t, t + D/2)
        const bool from_len = p.kv_lens && !p.q_pos && p.q_pos0 < 0;  // decode: the newest key's position
        const int pos = table_row(from_len ? T - 1 : row_position(p.q_pos, p.q_pos_base, p.q_pos0, b, qi_c, p.S),
                                  p.max_pos);
#pragma unroll
        for (int t8 = 0; t8 < NT / 8; ++t8) {
          const floatx8 c = load_tab8(p.cos_tab, pos, D / 2, 8 * t8);
          const floatx8 sn = load_tab8(p.sin_tab, pos, D / 2, 8 * t8);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t = 8 * t8 + e;
            const float partner = __shfl_xor(x[t], 32, 64);  // the other half of the pair
            x[t] = hh ? (x[t] * c[e] + partner * sn[e]) : (x[t] * c[e] - partner * sn[e]);
          }
        }
      }
    }
  }

  float m_i = -INFINITY, l_i = 0.f;
  floatx16 oacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx16{};

  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();  // every wave is done with the previous tile
    stash();
    __syncthreads();
    if (j + 1 < ntiles) fetch(j + 1);

    // S^T = K Q^T for this tile's 32 keys (MFMA row = key r32)
    floatx16 s = floatx16{};
#pragma unroll
    for (int t4 = 0; t4 < NT / 4; ++t4) {
      const floatx4 a = kt[r32 * CPR + ((hh * (NT / 4) + t4) ^ Tl::kswz(r32))];
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma32_f32(a[e], x[4 * t4 + e], s);
    }

    const int n0 = j * PF32_BN;
    if constexpr (BIAS) {
      // scores to log2 units plus the bias (the lane's keys: 4 runs of 4)
      const float* brow = reinterpret_cast<const float*>(p.bias) + b * p.bsb + head * p.bsh + (int64_t)qi_c * p.bss;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k4 = n0 + r * 8 + hh * 4;
        const floatx4 bv = k4 < T ? *reinterpret_cast<const floatx4*>(brow + k4) : floatx4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) s[r * 4 + e] = __builtin_fmaf(bv[e], kLog2e, s[r * 4 + e] * p.scale_log2);
      }
    }
    // keys past T, and (causal) keys past this row's frontier
    if (BIAS || n0 + PF32_BN > T || (CAUSAL && n0 + PF32_BN - 1 > q0 + coff)) {
      const int lim = CAUSAL ? min(T - 1, qi + coff) : T - 1;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (n0 + (i / 4) * 8 + hh * 4 + (i % 4) > lim) s[i] = -INFINITY;
    }

    // online softmax in the log2 domain (tile 0 holds key 0 for every row,
    // so m_i is finite from the first tile on, unless a bias masks it: a row
    // with no finite score yet keeps m_i = -inf and exponentiates against 0)
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
    const float m_new = fmaxf(m_i, xor32_max(mx) * (BIAS ? 1.f : p.scale_log2));
    const float m_use = (BIAS && !(m_new > -INFINITY)) ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    l_i *= alpha;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) oacc[dd] *= alpha;
    m_i = m_new;
    float pv[16];
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      pv[i] = BIAS ? fast_exp2(s[i] - m_use) : fast_exp2(s[i] * p.scale_log2 - m_i);
      ls += pv[i];
    }
    l_i += ls;

    // O^T += V^T P^T: step t, k-slot hh = key (t/4)*8 + hh*4 + t%4
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int key = (t / 4) * 8 + hh * 4 + (t % 4);
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) {
        const int col = dd * 32 + r32;
        const float a = vt[key * CPR + ((col / 4) ^ Tl::vswz(key))][col % 4];
        oacc[dd] = mfma32_f32(a, pv[t], oacc[dd]);
      }
    }
  }

  l_i = xor32_sum(l_i);
  if (!qvalid) return;
  float* orow = reinterpret_cast<float*>(p.o) + b * p.osb + head * p.osh + (int64_t)qi * p.oss;
  if (kv_end == 0) {  // no keys: zeros; a length out of range: NaN
    const float f = T < 0 ? __builtin_nanf("") : 0.f;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        *reinterpret_cast<floatx4*>(orow + dd * 32 + gq * 8 + hh * 4) = floatx4{f, f, f, f};
    if (p.lse && hh == 0) p.lse[((int64_t)b * p.Hq + head) * p.S + qi] = -INFINITY;
    return;
  }
  const bool none = BIAS && !(l_i > 0.f);  // every key masked by the bias: zeros, as SDPA gives
  const float inv_l = none ? 0.f : 1.f / l_i;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const floatx4 t = {oacc[dd][gq * 4 + 0] * inv_l, oacc[dd][gq * 4 + 1] * inv_l,
                         oacc[dd][gq * 4 + 2] * inv_l, oacc[dd][gq * 4 + 3] * inv_l};
      *reinterpret_cast<floatx4*>(orow + dd * 32 + gq * 8 + hh * 4) = t;
    }
  if (p.lse && hh == 0)
    p.lse[((int64_t)b * p.Hq + head) * p.S + qi] = none ? -INFINITY : (m_i + __log2f(l_i)) * kLn2;
}

template <int D>
static hipError_t launch_f32(const PrefillParams& p, bool causal, bool fuse, hipStream_t st) {
  dim3 grid((unsigned)(p.nqb * p.B * p.Hkv));
  dim3 block(64 * PF32_NW);
  if (p.bias) {
    if (causal) hipLaunchKernelGGL((prefill_f32_kernel<D, true, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_f32_kernel<D, false, true, true>), grid, block, 0, st, p);
    return hipGetLastError();
  }
  if (causal) {
    if (fuse) hipLaunchKernelGGL((prefill_f32_kernel<D, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_f32_kernel<D, true, false>), grid, block, 0, st, p);
  } else {
    if (fuse) hipLaunchKernelGGL((prefill_f32_kernel<D, false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_f32_kernel<D, false, false>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_prefill_f32(const PrefillParams& p, int D, bool causal, bool fuse, hipStream_t st) {
  return with_head_dim(D, [&](auto dc) { return launch_f32<decltype(dc)::value>(p, causal, fuse, st); });
}

}  // namespace nq
