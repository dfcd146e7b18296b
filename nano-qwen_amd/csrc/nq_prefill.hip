// Causal / full GQA prefill attention for gfx950 (FlashAttention-2 forward).
//
// Replaces kernels/flash_attn.py:28-143 and the SDPA call of
// model/attention.py:105-115; QK-Norm + RoPE of Q (attention.py:95-100) are
// fused into the Q load.
//
// Work decomposition
//   A workgroup (4 waves, 256 lanes) owns 128 query rows that all read the
//   same kv head: the G = Hq/Hkv query heads of one GQA group times
//   BM = 128/G consecutive positions.  Every K/V tile it stages in LDS is
//   therefore used by all G heads (the repeat_interleave of
//   attention.py:106-108 never materialises).  All 128 rows share one causal
//   frontier, so the whole workgroup walks the same key range.
//
// Per wave: 32 query rows.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_bf16 (A = K tile from LDS, B = Q from registers).  In
// the result each lane owns one query column and 16 of its 32 keys, so the
// row max / row sum of the online softmax need no cross-lane traffic except a
// single xor-32 exchange.  The output is kept transposed too,
// O^T += V^T P^T, so the per-row rescale applies lane-locally.  K rows enter
// MFMA rows through a bit permutation (swap bits 2 and 3 of the row index)
// chosen so each lane's 8 consecutive P values are 8 consecutive keys; the
// V^T operand is then read from the row-major V tile with
// ds_read_b64_tr_b16 (two transpose reads per operand), so V is never
// transposed on the way into LDS.
//
// LDS (64 banks on gfx950): K rows are padded by 16 bytes so the 16 rows one
// ds_read_b128 touches fall on distinct banks; V rows are padded by 64 bytes
// so the 4 rows x 64 bytes one transpose read touches do.
//
// Softmax: log2 domain (exp2 with log2(e) folded into the scale).  The
// running max is only raised when some row's tile max exceeds it by more than
// 2^8 (then O and l are rescaled); otherwise P values up to 256 are
// accumulated against the stale max.  The final O/l is exact either way.
//
// Pipeline: the next K/V tile is fetched from HBM into registers while the
// current tile's MFMAs run, then written to the other LDS buffer; one barrier
// per 64-key tile.  Causal workgroups are issued heaviest (last q-block)
// first.

#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

constexpr int PF_THREADS = 256;
constexpr int PF_ROWS = 128;  // query rows per workgroup
constexpr int PF_BN = 64;     // keys per tile
constexpr float PF_RESCALE_LOG2 = 8.0f;

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

// MFMA row r of a 32-key block holds key sigma(r): bits 2 and 3 swapped.
__device__ __forceinline__ int key_perm32(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

template <int D>
struct PrefillLds {
  static constexpr int KS = D + 8;        // K row stride (elements): +16 B
  static constexpr int VS = D + 32;       // V row stride (elements): +64 B
  static constexpr int K_TILE = PF_BN * KS;
  static constexpr int V_TILE = PF_BN * VS;
  static constexpr int BUF = K_TILE + V_TILE;
};

template <int D, typename T, bool CAUSAL, bool FUSE_Q>
__global__ void __attribute__((amdgpu_flat_work_group_size(PF_THREADS, PF_THREADS),
                               amdgpu_waves_per_eu(2, 2)))
prefill_kernel(PrefillParams p) {
  using Lds = PrefillLds<D>;
  constexpr int KS = Lds::KS, VS = Lds::VS, K_TILE = Lds::K_TILE, BUF = Lds::BUF;
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int NDB = D / 16;        // 16-wide d blocks (QK^T k-steps)
  constexpr int NDO = D / 32;        // 32-wide d blocks (output tiles)
  constexpr int LOADS = PF_BN * CPR / PF_THREADS;  // per tensor per thread
  static_assert(LOADS * PF_THREADS == PF_BN * CPR, "tile must split evenly");

  __shared__ __attribute__((aligned(16))) bf16 smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, hh = lane >> 5;

  // workgroup -> (batch, kv head, q-block); causal: heaviest q-blocks first
  const int npairs = p.B * p.Hkv;
  const int L = blockIdx.x;
  const int qblk = CAUSAL ? (p.nqb - 1 - L / npairs) : (L / npairs);
  const int pair = L % npairs;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  const int coff = p.T - p.S;

  // this lane's query row: column r32 of this wave's 32 rows
  const int R = wave * 32 + r32;
  const int g = R / p.BM, pr = R - g * p.BM;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[row][dblk*16 + hh*8 + e]
  bf16x8 qop[NDB];
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qi_c * p.qss;
    floatx8 xf[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) xf[db] = Vec8<T>::load_f32(qrow + db * 16 + hh * 8);
    if (FUSE_Q) {
      if (p.qw) {
        float ss = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += xf[db][e] * xf[db][e];
        ss += shfl_xor_f(ss, 32);
        const float r = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          floatx8 w = Vec8<float>::load_f32(p.qw + db * 16 + hh * 8);
#pragma unroll
          for (int e = 0; e < 8; ++e) xf[db][e] = xf[db][e] * r * w[e];
        }
      }
      if (p.cos_tab) {
        const int pos = clamp_pos(row_position(p.q_pos, p.q_pos_base, p.q_pos0, b, qi_c, p.S), p.max_pos);
        const float* ct = p.cos_tab + (int64_t)pos * (D / 2);
        const float* st = p.sin_tab + (int64_t)pos * (D / 2);
#pragma unroll
        for (int db = 0; db < NDB / 2; ++db) {
          floatx8 c = Vec8<float>::load_f32(ct + db * 16 + hh * 8);
          floatx8 s = Vec8<float>::load_f32(st + db * 16 + hh * 8);
          floatx8 x1 = xf[db], x2 = xf[db + NDB / 2];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            xf[db][e] = x1[e] * c[e] - x2[e] * s[e];
            xf[db + NDB / 2][e] = x2[e] * c[e] + x1[e] * s[e];
          }
        }
      }
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) qop[db] = to_bf16x8(xf[db]);
  }

  const int kv_end = CAUSAL ? min(p.T, q0 + p.BM + coff) : p.T;
  const int ntiles = (kv_end + PF_BN - 1) / PF_BN;
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.ksb + kvh * p.ksh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.vsb + kvh * p.vsh;

  // global -> register staging: thread owns 16-byte chunks c = tid + 256*i
  bf16x8 kreg[LOADS], vreg[LOADS];
  const bf16x8 zero8 = {};
  auto load_tile = [&](int n0) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * PF_THREADS;
      const int key = n0 + c / CPR, ch = c % CPR;
      const bool ok = key < p.T;
      kreg[i] = ok ? Vec8<T>::load_bf16(kbase + (int64_t)key * p.kss + ch * 8) : zero8;
      vreg[i] = ok ? Vec8<T>::load_bf16(vbase + (int64_t)key * p.vss + ch * 8) : zero8;
    }
  };
  auto store_tile = [&](int buf) {
    bf16* Ks = smem + buf * BUF;
    bf16* Vs = Ks + K_TILE;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * PF_THREADS;
      *reinterpret_cast<bf16x8*>(Ks + (c / CPR) * KS + (c % CPR) * 8) = kreg[i];
      *reinterpret_cast<bf16x8*>(Vs + (c / CPR) * VS + (c % CPR) * 8) = vreg[i];
    }
  };

  // per-lane LDS offsets (elements within a buffer)
  const int k_off = key_perm32(r32) * KS + hh * 8;
  // V^T operand via transpose reads: lane group gi = lane/16, j = lane%16;
  // source row hh*8 + j/4 (+ks*16 + 4*half), column (gi&1)*16 + 4*(j%4) (+dd*32)
  const int gi = lane >> 4, jj = lane & 15;
  const int v_off = K_TILE + (hh * 8 + (jj >> 2)) * VS + (gi & 1) * 16 + 4 * (jj & 3);

  float m_i = -INFINITY, l_i = 0.f;
  floatx16 oacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx16{};

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    const int n0 = j * PF_BN;
    const int buf = j & 1;
    if (j + 1 < ntiles) load_tile(n0 + PF_BN);
    const bf16* Bs = smem + buf * BUF;

    // S^T = K Q^T for two 32-key blocks (chains interleaved)
    floatx16 s[2] = {floatx16{}, floatx16{}};
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bf16x8 a = *reinterpret_cast<const bf16x8*>(Bs + k_off + kb * 32 * KS + db * 16);
        s[kb] = mfma32(a, qop[db], s[kb]);
      }

    // masking: keys past T, and (causal) keys past this row's frontier
    const bool need_mask = (n0 + PF_BN > p.T) || (CAUSAL && n0 + PF_BN - 1 > q0 + coff);
    if (need_mask) {
      const int lim = CAUSAL ? min(p.T - 1, qi + coff) : p.T - 1;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = n0 + kb * 32 + (i >> 3) * 16 + hh * 8 + (i & 7);
          if (key > lim) s[kb][i] = -INFINITY;
        }
    }

    // online softmax (log2 domain); each lane owns one query row
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = fmaxf(mx, shfl_xor_f(mx, 32)) * p.scale_log2;
    if (wave_any(mx > m_i + PF_RESCALE_LOG2)) {
      const float m_new = fmaxf(m_i, mx);
      const float alpha = fast_exp2(m_i - m_new);  // 0 on the first tile
      l_i *= alpha;
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) oacc[dd] *= alpha;
      m_i = m_new;
    }
    // every row has seen key 0 by now, so m_i is finite
    float rs = 0.f;
    bf16x8 pop[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        floatx8 t;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = fast_exp2(s[kb][half * 8 + e] * p.scale_log2 - m_i);
          rs += pe;
          t[e] = pe;
        }
        pop[kb * 2 + half] = to_bf16x8(t);
      }
    l_i += rs;

    // O^T += V^T P^T
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) {
        const bf16* src = Bs + v_off + ks * 16 * VS + dd * 32;
        bf16x8 a = lds_read_tr8(src, src + 4 * VS);
        oacc[dd] = mfma32(a, pop[ks], oacc[dd]);
      }

    if (j + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  l_i += shfl_xor_f(l_i, 32);
  if (!qvalid) return;
  const float inv_l = 1.f / l_i;
  T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + head * p.osh + (int64_t)qi * p.oss;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      floatx4 t = {oacc[dd][gq * 4 + 0] * inv_l, oacc[dd][gq * 4 + 1] * inv_l,
                   oacc[dd][gq * 4 + 2] * inv_l, oacc[dd][gq * 4 + 3] * inv_l};
      store4<T>(orow + dd * 32 + gq * 8 + hh * 4, t);
    }
  if (p.lse && hh == 0) p.lse[((int64_t)b * p.Hq + head) * p.S + qi] = (m_i + __log2f(l_i)) * kLn2;
}

template <int D, typename T>
static hipError_t launch_prefill(const PrefillParams& p, bool causal, bool fuse, hipStream_t st) {
  dim3 grid((unsigned)(p.nqb * p.B * p.Hkv));
  dim3 block(PF_THREADS);
  if (causal) {
    if (fuse) hipLaunchKernelGGL((prefill_kernel<D, T, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_kernel<D, T, true, false>), grid, block, 0, st, p);
  } else {
    if (fuse) hipLaunchKernelGGL((prefill_kernel<D, T, false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_kernel<D, T, false, false>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace nq

using namespace nq;

extern "C" int nq_attn_prefill_fwd(const void* q, const int64_t* q_strides, const void* k,
                                   const int64_t* k_strides, const void* v,
                                   const int64_t* v_strides, void* o, const int64_t* o_strides,
                                   float* lse, int B, int Hq, int Hkv, int S, int T, int D,
                                   int dtype, const float* q_weight, float eps,
                                   const float* cos_tab, const float* sin_tab, int max_pos,
                                   const int32_t* q_pos, const int32_t* q_pos_base, int q_pos0,
                                   int causal, float sm_scale, void* stream) {
  nq_clear_error();
  if (D != 64 && D != 128) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || T <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d S=%d T=%d)", B, Hq, Hkv, S, T);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  const int G = Hq / Hkv;
  if (PF_ROWS % G) return nq_fail(NQ_ERR_UNSUPPORTED, "GQA group size %d must divide 128", G);
  if (causal && S > T) return nq_fail(NQ_ERR_INVALID, "causal attention needs S <= T (S=%d T=%d)", S, T);
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return nq_fail(NQ_ERR_INVALID, "q, k, v, o and their strides are required");
  if (!nq_aligned16(q) || !nq_aligned16(k) || !nq_aligned16(v) || !nq_aligned16(o))
    return nq_fail(NQ_ERR_INVALID, "base pointers must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  const int64_t* all[4] = {q_strides, k_strides, v_strides, o_strides};
  for (const int64_t* s : all)
    for (int i = 0; i < 3; ++i)
      if ((s[i] * esz) % 16) return nq_fail(NQ_ERR_INVALID, "strides must be multiples of 16 bytes");
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  PrefillParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse;
  p.qsb = q_strides[0]; p.qsh = q_strides[1]; p.qss = q_strides[2];
  p.ksb = k_strides[0]; p.ksh = k_strides[1]; p.kss = k_strides[2];
  p.vsb = v_strides[0]; p.vsh = v_strides[1]; p.vss = v_strides[2];
  p.osb = o_strides[0]; p.osh = o_strides[1]; p.oss = o_strides[2];
  p.qw = q_weight; p.eps = eps; p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.q_pos = q_pos; p.q_pos_base = q_pos_base; p.q_pos0 = q_pos0;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = G; p.S = S; p.T = T;
  p.BM = PF_ROWS / G;
  p.nqb = (S + p.BM - 1) / p.BM;
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;
  const bool fuse = q_weight != nullptr || cos_tab != nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == NQ_DTYPE_BF16)
    e = (D == 128) ? launch_prefill<128, bf16>(p, causal, fuse, st) : launch_prefill<64, bf16>(p, causal, fuse, st);
  else
    e = (D == 128) ? launch_prefill<128, float>(p, causal, fuse, st) : launch_prefill<64, float>(p, causal, fuse, st);
  return nq_check_launch(e);
}
