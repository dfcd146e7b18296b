// FlashAttention-2 backward for gfx950, and the backward of QK-Norm + RoPE.
//
// Replaces the autograd of the attention path that training runs today:
// F.scaled_dot_product_attention's backward (model/attention.py:110-115,
// driven by the training loops' loss.backward()), the backward of the
// rotate-half RoPE (model/rope.py:133-161) and of RMSNorm as QK-Norm
// (model/norm.py:17-22, applied at attention.py:95-97).
//
// Attention backward, given Q-hat, K-hat, V, O, dO and the forward's LSE
// (natural log of the row sums of exp(scale * S)):
//   P = exp(scale * Q K^T - LSE),  Delta = rowsum(dO * O),
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - Delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
// Three kernels: Delta (one row per D/8 lanes); dQ per query block (the
// forward's decomposition: a workgroup owns the G heads x BM positions of one
// kv head and walks the key tiles); dK/dV per key block (a workgroup owns 128
// keys of one kv head and walks every query row of its G heads, so the GQA sum
// over heads happens in registers, with no atomics).
//
// MFMA layouts (v_mfma_f32_32x32x16_bf16): A lane l holds row l%32, k = 8*(l/32)..+7;
// B lane l holds column l%32, the same k; C lane l holds column l%32, rows
// 8*(i/4) + 4*(l/32) + i%4.  As in the forward, the operand that becomes the
// C rows (keys in the dQ kernel, queries in the dK/dV kernel) enters through
// the bit-2<->3 row permutation, so that each lane's 8 consecutive C values
// are 8 consecutive keys (queries): the next MFMA takes them as its B operand
// with no data movement, and its A operand (K^T, dO^T or Q^T) is read from the
// row-major LDS tile with ds_read_b64_tr_b16.
//
// This version stages every tile through LDS with one buffer and a barrier on
// each side (the second resident workgroup of the CU overlaps the loads).

#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;  // (B, Hq, S) natural log
  float* delta;      // (B, Hq, S) scratch, written by bwd_delta_kernel
  void* dq;
  void* dk;
  void* dv;
  int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss;
  int64_t osb, osh, oss, dosb, dosh, doss;
  int64_t dqsb, dqsh, dqss, dksb, dksh, dkss, dvsb, dvsh, dvss;
  int B, Hq, Hkv, G, S, T, BM, nqb, coff;
  float scale, scale_log2;
};

constexpr int BW_BN = 64;     // keys per tile (dQ kernel)
constexpr int BW_BQ = 32;     // query rows per tile (dK/dV kernel)
constexpr int BW_KEYS = 128;  // keys per dK/dV workgroup (32 per wave)

__device__ __forceinline__ int bw_perm32(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
// C element i of a lane in half hh -> index (key or query) within its 32-block
__device__ __forceinline__ int bw_cidx(int i, int hh) { return (i < 8 ? 0 : 16) + hh * 8 + (i & 7); }

template <int D>
struct BwTile {
  static constexpr int RB = 2 * D;         // bytes per row
  static constexpr int CPR = D / 8;        // 16-byte chunks per row
  static constexpr int RPL = 256 / RB;     // rows per 256-byte bank line
  // row-chunk reads of 16 consecutive rows hit distinct banks
  __device__ static int rsw(int r, int c) { return c ^ ((r / RPL) & (CPR - 1)); }
  // transpose reads (4 rows x 64 bytes) hit distinct banks
  __device__ static int tsw(int r, int c) { return c ^ (4 * ((r / RPL) & (D / 32 - 1))); }
};

// Stage rows [r0, r0 + NR) of a strided (row stride `rs` elements) source into
// a row-major LDS tile with chunk swizzle SW; rows >= nvalid are zero.
template <int D, typename T, int NR, bool TRANSPOSE_SW>
__device__ __forceinline__ void bw_stage(unsigned char* tile, const T* src, int64_t rs, int r0, int nvalid) {
  using L = BwTile<D>;
  constexpr int CH = NR * L::CPR;  // 16-byte chunks in the tile
  for (int c = threadIdx.x; c < CH; c += 256) {
    const int r = c / L::CPR, ch = c % L::CPR;
    const int row = r0 + r;
    bf16x8 val = row < nvalid ? to_bf16x8(Vec8<T>::load_f32(src + (int64_t)row * rs + ch * 8)) : bf16x8{};
    const int pc = TRANSPOSE_SW ? L::tsw(r, ch) : L::rsw(r, ch);
    *reinterpret_cast<bf16x8*>(tile + r * L::RB + pc * 16) = val;
  }
}

// ---------------------------------------------------------------- Delta
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdParams p) {
  constexpr int LPR = D / 8;
  constexpr int RPB = 256 / LPR;
  const int sub = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.Hq * p.S;
  for (int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR; row < nrows; row += (int64_t)gridDim.x * RPB) {
    const int s = (int)(row % p.S);
    const int h = (int)((row / p.S) % p.Hq);
    const int b = (int)(row / ((int64_t)p.S * p.Hq));
    const floatx8 o = Vec8<T>::load_f32(reinterpret_cast<const T*>(p.o) + b * p.osb + h * p.osh + s * p.oss + sub * 8);
    const floatx8 d =
        Vec8<T>::load_f32(reinterpret_cast<const T*>(p.dout) + b * p.dosb + h * p.dosh + s * p.doss + sub * 8);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(o[e], d[e], acc);
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) acc += shfl_xor_f(acc, m);
    if (sub == 0) p.delta[row] = acc;
  }
}

// ---------------------------------------------------------------- dQ
template <int D, typename T, bool CAUSAL>
__global__ void __launch_bounds__(256, 2) bwd_dq_kernel(BwdParams p) {
  using L = BwTile<D>;
  constexpr int NDB = D / 16, NDO = D / 32;
  constexpr int TB = BW_BN * L::RB;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * TB];  // K (transpose swizzle), V
  unsigned char* Kt = smem;
  unsigned char* Vt = smem + TB;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r32 = lane & 31, hh = lane >> 5;
  const int npairs = p.B * p.Hkv;
  const int qrank = blockIdx.x / npairs, pair = blockIdx.x % npairs;
  const int qblk = CAUSAL ? (p.nqb - 1 - qrank) : qrank;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  const int kv_end = CAUSAL ? min(p.T, q0 + p.BM + p.coff) : p.T;
  const int ntiles = (kv_end + BW_BN - 1) / BW_BN;

  const int R = wave * 32 + r32;
  const int g = R / p.BM, pr = R - g * p.BM;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  bf16x8 qop[NDB], dop[NDB];
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qi_c * p.qss;
    const T* drow = reinterpret_cast<const T*>(p.dout) + b * p.dosb + head * p.dosh + (int64_t)qi_c * p.doss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      qop[db] = to_bf16x8(Vec8<T>::load_f32(qrow + db * 16 + hh * 8));
      dop[db] = to_bf16x8(Vec8<T>::load_f32(drow + db * 16 + hh * 8));
    }
  }
  const int64_t srow = ((int64_t)b * p.Hq + head) * p.S + qi_c;
  const float lse2 = qvalid ? p.lse[srow] * kLog2e : INFINITY;  // invalid rows: P = 0
  const float dlt = p.delta[srow];

  // LDS offsets: K / V rows through the key permutation (A of S^T and dP^T);
  // K^T through transpose reads (A of dQ^T)
  const int prow = bw_perm32(r32);
  int kro[NDB], vro[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    kro[db] = prow * L::RB + L::tsw(prow, 2 * db + hh) * 16;
    vro[db] = prow * L::RB + L::rsw(prow, 2 * db + hh) * 16;
  }
  int kto[NDO];
  {
    const int gi = lane >> 4, jj = lane & 15;
    const int row = hh * 8 + (jj >> 2);
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      const int col = dd * 32 + (gi & 1) * 16 + 4 * (jj & 3);
      kto[dd] = row * L::RB + L::tsw(row, col / 8) * 16 + (col % 8) * 2;
    }
  }

  floatx16 dqacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) dqacc[dd] = floatx16{};

  const T* kb0 = reinterpret_cast<const T*>(p.k) + b * p.ksb + kvh * p.ksh;
  const T* vb0 = reinterpret_cast<const T*>(p.v) + b * p.vsb + kvh * p.vsh;
  const int lim = CAUSAL ? qi + p.coff : p.T - 1;  // last key this row sees

  for (int j = 0; j < ntiles; ++j) {
    const int n0 = j * BW_BN;
    __syncthreads();
    bw_stage<D, T, BW_BN, true>(Kt, kb0 + (int64_t)n0 * p.kss, p.kss, 0, p.T - n0);
    bw_stage<D, T, BW_BN, false>(Vt, vb0 + (int64_t)n0 * p.vss, p.vss, 0, p.T - n0);
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      floatx16 s = floatx16{}, dp = floatx16{};
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const bf16x8 ak = *reinterpret_cast<const bf16x8*>(Kt + kro[db] + kb * 32 * L::RB);
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(Vt + vro[db] + kb * 32 * L::RB);
        s = mfma32(ak, qop[db], s);
        dp = mfma32(av, dop[db], dp);
      }
      floatx8 ds[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = n0 + kb * 32 + bw_cidx(i, hh);
        const float pe = key <= lim && key < p.T ? fast_exp2(s[i] * p.scale_log2 - lse2) : 0.f;
        ds[i / 8][i % 8] = pe * (dp[i] - dlt);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 bds = to_bf16x8(ds[ks]);
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) {
          const bf16* a = reinterpret_cast<const bf16*>(Kt + kto[dd] + (kb * 32 + ks * 16) * L::RB);
          const bf16x8 ak = lds_read_tr8(a, a + 4 * D);  // rows +0..3 and +4..7 (4 rows = 4 * D elements)
          dqacc[dd] = mfma32(ak, bds, dqacc[dd]);
        }
      }
    }
  }

  if (!qvalid || g >= p.G) return;
  T* out = reinterpret_cast<T*>(p.dq) + b * p.dqsb + head * p.dqsh + (int64_t)qi * p.dqss;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      floatx4 t = {dqacc[dd][gq * 4] * p.scale, dqacc[dd][gq * 4 + 1] * p.scale, dqacc[dd][gq * 4 + 2] * p.scale,
                   dqacc[dd][gq * 4 + 3] * p.scale};
      store4<T>(out + dd * 32 + gq * 8 + hh * 4, t);
    }
}

// ---------------------------------------------------------------- dK, dV
template <int D, typename T, bool CAUSAL>
__global__ void __launch_bounds__(256, 2) bwd_dkdv_kernel(BwdParams p) {
  using L = BwTile<D>;
  constexpr int NDB = D / 16, NDO = D / 32;
  constexpr int TB = BW_BQ * L::RB;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * TB + 2 * BW_BQ * 4];
  unsigned char* Qt = smem;        // transpose swizzle (row reads and transpose reads)
  unsigned char* Dt = smem + TB;   // dO, likewise
  float* lse_t = reinterpret_cast<float*>(smem + 2 * TB);
  float* dlt_t = lse_t + BW_BQ;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r32 = lane & 31, hh = lane >> 5;
  const int nkb = (p.T + BW_KEYS - 1) / BW_KEYS;
  const int kblk = blockIdx.x % nkb, pair = blockIdx.x / nkb;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int k0 = kblk * BW_KEYS;
  const int key = k0 + wave * 32 + r32;  // this lane's key (C column)
  const int key_c = key < p.T ? key : p.T - 1;

  // K and V of the lane's key as B operands (column = key, k = head dims)
  bf16x8 kop[NDB], vop[NDB];
  {
    const T* krow = reinterpret_cast<const T*>(p.k) + b * p.ksb + kvh * p.ksh + (int64_t)key_c * p.kss;
    const T* vrow = reinterpret_cast<const T*>(p.v) + b * p.vsb + kvh * p.vsh + (int64_t)key_c * p.vss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      kop[db] = to_bf16x8(Vec8<T>::load_f32(krow + db * 16 + hh * 8));
      vop[db] = to_bf16x8(Vec8<T>::load_f32(vrow + db * 16 + hh * 8));
    }
  }
  const int prow = bw_perm32(r32);
  int rro[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) rro[db] = prow * L::RB + L::tsw(prow, 2 * db + hh) * 16;
  int tro[NDO];
  {
    const int gi = lane >> 4, jj = lane & 15;
    const int row = hh * 8 + (jj >> 2);
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      const int col = dd * 32 + (gi & 1) * 16 + 4 * (jj & 3);
      tro[dd] = row * L::RB + L::tsw(row, col / 8) * 16 + (col % 8) * 2;
    }
  }

  floatx16 dkacc[NDO], dvacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) dkacc[dd] = dvacc[dd] = floatx16{};

  // queries that see any key of this block: q + coff >= k0
  const int qstart = CAUSAL ? max(0, k0 - p.coff) / BW_BQ * BW_BQ : 0;
  for (int g = 0; g < p.G; ++g) {
    const int head = kvh * p.G + g;
    const T* qh = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh;
    const T* dh = reinterpret_cast<const T*>(p.dout) + b * p.dosb + head * p.dosh;
    const int64_t sbase = ((int64_t)b * p.Hq + head) * p.S;
    for (int qt = qstart; qt < p.S; qt += BW_BQ) {
      __syncthreads();
      bw_stage<D, T, BW_BQ, true>(Qt, qh + (int64_t)qt * p.qss, p.qss, 0, p.S - qt);
      bw_stage<D, T, BW_BQ, true>(Dt, dh + (int64_t)qt * p.doss, p.doss, 0, p.S - qt);
      if (threadIdx.x < BW_BQ) {
        const int q = qt + threadIdx.x;
        lse_t[threadIdx.x] = q < p.S ? p.lse[sbase + q] * kLog2e : INFINITY;  // padding rows: P = 0
        dlt_t[threadIdx.x] = q < p.S ? p.delta[sbase + q] : 0.f;
      }
      __syncthreads();
      floatx16 s = floatx16{}, dp = floatx16{};
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const bf16x8 aq = *reinterpret_cast<const bf16x8*>(Qt + rro[db]);
        const bf16x8 ad = *reinterpret_cast<const bf16x8*>(Dt + rro[db]);
        s = mfma32(aq, kop[db], s);
        dp = mfma32(ad, vop[db], dp);
      }
      floatx8 pv[2], ds[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qr = bw_cidx(i, hh);
        const int q = qt + qr;
        const bool keep = key < p.T && (!CAUSAL || key <= q + p.coff);
        const float pe = keep ? fast_exp2(s[i] * p.scale_log2 - lse_t[qr]) : 0.f;
        pv[i / 8][i % 8] = pe;
        ds[i / 8][i % 8] = pe * (dp[i] - dlt_t[qr]);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 bp = to_bf16x8(pv[ks]);
        const bf16x8 bds = to_bf16x8(ds[ks]);
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) {
          const bf16* ad = reinterpret_cast<const bf16*>(Dt + tro[dd] + ks * 16 * L::RB);
          const bf16* aq = reinterpret_cast<const bf16*>(Qt + tro[dd] + ks * 16 * L::RB);
          dvacc[dd] = mfma32(lds_read_tr8(ad, ad + 4 * D), bp, dvacc[dd]);
          dkacc[dd] = mfma32(lds_read_tr8(aq, aq + 4 * D), bds, dkacc[dd]);
        }
      }
    }
  }

  if (key >= p.T) return;
  T* dko = reinterpret_cast<T*>(p.dk) + b * p.dksb + kvh * p.dksh + (int64_t)key * p.dkss;
  T* dvo = reinterpret_cast<T*>(p.dv) + b * p.dvsb + kvh * p.dvsh + (int64_t)key * p.dvss;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      floatx4 tk = {dkacc[dd][gq * 4] * p.scale, dkacc[dd][gq * 4 + 1] * p.scale, dkacc[dd][gq * 4 + 2] * p.scale,
                    dkacc[dd][gq * 4 + 3] * p.scale};
      floatx4 tv = {dvacc[dd][gq * 4], dvacc[dd][gq * 4 + 1], dvacc[dd][gq * 4 + 2], dvacc[dd][gq * 4 + 3]};
      store4<T>(dko + dd * 32 + gq * 8 + hh * 4, tk);
      store4<T>(dvo + dd * 32 + gq * 8 + hh * 4, tv);
    }
}

template <int D, typename T>
static hipError_t launch_bwd(const BwdParams& p, bool causal, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.S;
  constexpr int RPB = 256 / (D / 8);
  const int64_t dblocks = (rows + RPB - 1) / RPB;
  hipLaunchKernelGGL((bwd_delta_kernel<T, D>), dim3((unsigned)(dblocks < 2048 ? dblocks : 2048)), dim3(256), 0, st,
                     p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 gq((unsigned)(p.nqb * p.B * p.Hkv));
  const dim3 gk((unsigned)(((p.T + BW_KEYS - 1) / BW_KEYS) * p.B * p.Hkv));
  if (causal) {
    hipLaunchKernelGGL((bwd_dq_kernel<D, T, true>), gq, dim3(256), 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, true>), gk, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((bwd_dq_kernel<D, T, false>), gq, dim3(256), 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, false>), gk, dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- QK-Norm + RoPE backward
// y = rope(x * r * w), r = rsqrt(mean(x^2) + eps).  With g = rope^T(dy) (the
// rotation by -theta): dw += g * x * r (summed over rows), and with
// u = g * w: dx = r * u - x * (r^3 / D) * sum(u * x).  Rows are held as in
// the forward row kernel (D/16 lanes, a lane owns 8 elements and their
// rotate-half partners).  dw is accumulated per block in LDS, then one atomic
// add per block and element into the caller's zeroed fp32 buffer.
struct NormBwdParams {
  const void* x;
  int64_t xsb, xsh, xss;
  const void* dy;
  int64_t ysb, ysh, yss;
  void* dx;
  int64_t dsb, dsh, dss;
  const float* w;
  float* dw;
  int B, H, S;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int max_pos;
  const int32_t* pos;
  const int32_t* pos_base;
  int pos0;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void norm_rope_bwd_kernel(NormBwdParams p) {
  constexpr int LPR = D / 16;
  constexpr int RPB = 256 / LPR;
  __shared__ float dws[256 / LPR][D];  // per-row-slot partial dw
  const int sub = threadIdx.x % LPR, slot = threadIdx.x / LPR;
  const int64_t nrows = (int64_t)p.B * p.H * p.S;
  floatx8 w1{}, w2{}, a1{}, a2{};
  if (p.w) {
    w1 = Vec8<float>::load_f32(p.w + sub * 8);
    w2 = Vec8<float>::load_f32(p.w + D / 2 + sub * 8);
  }
  for (int64_t row = (int64_t)blockIdx.x * RPB + slot; row < nrows; row += (int64_t)gridDim.x * RPB) {
    const int s = (int)(row % p.S);
    const int h = (int)((row / p.S) % p.H);
    const int b = (int)(row / ((int64_t)p.S * p.H));
    const T* xr = reinterpret_cast<const T*>(p.x) + b * p.xsb + h * p.xsh + s * p.xss + sub * 8;
    const T* yr = reinterpret_cast<const T*>(p.dy) + b * p.ysb + h * p.ysh + s * p.yss + sub * 8;
    floatx8 x1 = Vec8<T>::load_f32(xr), x2 = Vec8<T>::load_f32(xr + D / 2);
    floatx8 g1 = Vec8<T>::load_f32(yr), g2 = Vec8<T>::load_f32(yr + D / 2);
    if (p.cos_tab) {
      const int ps = clamp_pos(row_position(p.pos, p.pos_base, p.pos0, b, s, p.S), p.max_pos);
      const floatx8 c = Vec8<float>::load_f32(p.cos_tab + (int64_t)ps * (D / 2) + sub * 8);
      const floatx8 sn = Vec8<float>::load_f32(p.sin_tab + (int64_t)ps * (D / 2) + sub * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d1 = g1[e], d2 = g2[e];
        g1[e] = d1 * c[e] + d2 * sn[e];
        g2[e] = d2 * c[e] - d1 * sn[e];
      }
    }
    floatx8 r1 = g1, r2 = g2;
    if (p.w) {
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sq += x1[e] * x1[e] + x2[e] * x2[e];
      sq = row_sum<LPR>(sq);
      const float r = rsqrtf(sq / (float)D + p.eps);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a1[e] += g1[e] * x1[e] * r;
        a2[e] += g2[e] * x2[e] * r;
        dot += g1[e] * w1[e] * x1[e] + g2[e] * w2[e] * x2[e];
      }
      dot = row_sum<LPR>(dot);
      const float c3 = r * r * r * dot / (float)D;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        r1[e] = r * g1[e] * w1[e] - x1[e] * c3;
        r2[e] = r * g2[e] * w2[e] - x2[e] * c3;
      }
    }
    T* dr = reinterpret_cast<T*>(p.dx) + b * p.dsb + h * p.dsh + s * p.dss + sub * 8;
    store8<T>(dr, r1);
    store8<T>(dr + D / 2, r2);
  }
  if (!p.w) return;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dws[slot][sub * 8 + e] = a1[e];
    dws[slot][D / 2 + sub * 8 + e] = a2[e];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    float t = 0.f;
    for (int i = 0; i < RPB; ++i) t += dws[i][d];
    atomicAdd(p.dw + d, t);
  }
}

}  // namespace nq

using namespace nq;

extern "C" int64_t nq_attn_bwd_workspace_bytes(int B, int Hq, int S) {
  if (B <= 0 || Hq <= 0 || S <= 0) return 0;
  return (int64_t)B * Hq * S * (int64_t)sizeof(float);
}

extern "C" int nq_attn_bwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                           const void* dout, const int64_t* do_strides, const float* lse, void* dq,
                           const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                           const int64_t* dv_strides, void* workspace, int64_t workspace_bytes, int B, int Hq,
                           int Hkv, int S, int T, int D, int dtype, int causal, float sm_scale, void* stream) {
  nq_clear_error();
  if (D != 64 && D != 128) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || T <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d S=%d T=%d)", B, Hq, Hkv, S, T);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  const int G = Hq / Hkv;
  if (128 % G) return nq_fail(NQ_ERR_UNSUPPORTED, "the backward needs 128 %% (Hq/Hkv) == 0, got G=%d", G);
  if (causal && S > T) return nq_fail(NQ_ERR_INVALID, "causal attention needs S <= T (S=%d T=%d)", S, T);
  const void* ptrs[] = {q, k, v, o, dout, dq, dk, dv};
  const int64_t* strs[] = {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides};
  const int esz = nq_dtype_size(dtype);
  for (int i = 0; i < 8; ++i) {
    if (!ptrs[i] || !strs[i]) return nq_fail(NQ_ERR_INVALID, "q, k, v, o, dout, dq, dk, dv and strides are required");
    if (!nq_aligned16(ptrs[i])) return nq_fail(NQ_ERR_INVALID, "tensor base pointers must be 16-byte aligned");
    for (int a = 0; a < 3; ++a)
      if ((strs[i][a] * esz) % 16) return nq_fail(NQ_ERR_INVALID, "strides must be multiples of 16 bytes");
  }
  if (!lse) return nq_fail(NQ_ERR_INVALID, "the forward's LSE is required");
  const int64_t need = (int64_t)B * Hq * S * (int64_t)sizeof(float);
  if (!workspace || workspace_bytes < need)
    return nq_fail(NQ_ERR_WORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                   (long long)workspace_bytes);
  BwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.lse = lse;
  p.delta = reinterpret_cast<float*>(workspace);
  p.dq = dq; p.dk = dk; p.dv = dv;
  p.qsb = q_strides[0]; p.qsh = q_strides[1]; p.qss = q_strides[2];
  p.ksb = k_strides[0]; p.ksh = k_strides[1]; p.kss = k_strides[2];
  p.vsb = v_strides[0]; p.vsh = v_strides[1]; p.vss = v_strides[2];
  p.osb = o_strides[0]; p.osh = o_strides[1]; p.oss = o_strides[2];
  p.dosb = do_strides[0]; p.dosh = do_strides[1]; p.doss = do_strides[2];
  p.dqsb = dq_strides[0]; p.dqsh = dq_strides[1]; p.dqss = dq_strides[2];
  p.dksb = dk_strides[0]; p.dksh = dk_strides[1]; p.dkss = dk_strides[2];
  p.dvsb = dv_strides[0]; p.dvsh = dv_strides[1]; p.dvss = dv_strides[2];
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = G; p.S = S; p.T = T;
  p.BM = 128 / G;
  p.nqb = (S + p.BM - 1) / p.BM;
  p.coff = T - S;
  p.scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = p.scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == NQ_DTYPE_BF16)
    e = D == 128 ? launch_bwd<128, bf16>(p, causal != 0, st) : launch_bwd<64, bf16>(p, causal != 0, st);
  else
    e = D == 128 ? launch_bwd<128, float>(p, causal != 0, st) : launch_bwd<64, float>(p, causal != 0, st);
  return nq_check_launch(e);
}

extern "C" int nq_qk_norm_rope_bwd(const void* x, const int64_t* x_strides, const void* dy,
                                   const int64_t* dy_strides, void* dx, const int64_t* dx_strides,
                                   const float* weight, float* dweight, int B, int S, int H, int D, int dtype,
                                   float eps, const float* cos_tab, const float* sin_tab, int max_pos,
                                   const int32_t* pos, const int32_t* pos_base, int pos0, void* stream) {
  nq_clear_error();
  if (D != 64 && D != 128) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || S <= 0 || H <= 0) return nq_fail(NQ_ERR_INVALID, "sizes must be positive");
  if (!x || !dy || !dx || !x_strides || !dy_strides || !dx_strides)
    return nq_fail(NQ_ERR_INVALID, "x, dy, dx and their strides are required");
  if ((weight == nullptr) != (dweight == nullptr))
    return nq_fail(NQ_ERR_INVALID, "weight and dweight go together");
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  if (!nq_aligned16(x) || !nq_aligned16(dy) || !nq_aligned16(dx))
    return nq_fail(NQ_ERR_INVALID, "base pointers must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  for (int a = 0; a < 3; ++a)
    if ((x_strides[a] * esz) % 16 || (dy_strides[a] * esz) % 16 || (dx_strides[a] * esz) % 16)
      return nq_fail(NQ_ERR_INVALID, "strides must be multiples of 16 bytes");
  NormBwdParams p{};
  p.x = x; p.xsb = x_strides[0]; p.xsh = x_strides[1]; p.xss = x_strides[2];
  p.dy = dy; p.ysb = dy_strides[0]; p.ysh = dy_strides[1]; p.yss = dy_strides[2];
  p.dx = dx; p.dsb = dx_strides[0]; p.dsh = dx_strides[1]; p.dss = dx_strides[2];
  p.w = weight; p.dw = dweight;
  p.B = B; p.H = H; p.S = S; p.eps = eps;
  p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.pos = pos; p.pos_base = pos_base; p.pos0 = pos0;
  const int64_t rows = (int64_t)B * H * S;
  const int rpb = 256 / (D / 16);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == NQ_DTYPE_BF16) {
    if (D == 128) hipLaunchKernelGGL((norm_rope_bwd_kernel<bf16, 128>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((norm_rope_bwd_kernel<bf16, 64>), grid, dim3(256), 0, st, p);
  } else {
    if (D == 128) hipLaunchKernelGGL((norm_rope_bwd_kernel<float, 128>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((norm_rope_bwd_kernel<float, 64>), grid, dim3(256), 0, st, p);
  }
  return nq_check_launch(hipGetLastError());
}
