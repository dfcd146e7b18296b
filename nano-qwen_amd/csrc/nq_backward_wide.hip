// Attention backward at head_dim 256, for gfx950: the gradient of
// nq_prefill_wide.hip's forward (kernels/flash_attn.py:106 takes head_dim
// 256; under autograd the reference differentiates SDPA, model/attention.py:
// 110-115).  bf16 q, k, v, o, dO; GQA (kv-head gradients summed over their G
// query heads in registers, no atomics); causal with the bottom-right
// frontier.  The same tiles, operands and products as the forward
// (nq_wide.hpp, v_mfma_f32_16x16x32_bf16):
//
// bwd_dq_wide_kernel: 4 waves x 16 query rows of one head.  Per row it forms
//   Delta = rowsum(dO * O) and writes LSE * log2 e and Delta to the scratch
//   (the layout of the head_dim 32-128 backward: per (batch, head) and 32-row
//   tile, 64 floats, rows past S zero).  Per 32-key step: S^T = K Q^T and
//   dP^T = V dO^T (A = K, V rows from LDS; B = the row's scaled Q and its dO
//   in registers), P = exp2(S - LSE), dS = P (dP - Delta), and
//   dQ^T += K^T dS^T (A = K^T by transpose reads).
// bwd_dkdv_wide_kernel: 4 waves x 16 keys of one kv head, K and V rows in
//   registers.  Per 32-row query tile of each of the G heads: S = Q K^T and
//   dP = dO V^T (rows on M: each lane holds 8 rows of one key, in the order
//   that packs into the B operand of the next products), then
//   dV^T += dO^T P and dK^T += Q^T dS (A = dO^T, Q^T by transpose reads).
// dQ = scale dS K and dK = scale dS^T Q; the scores run in log2 units.

#include "nq_backward.hpp"
#include "nq_common.hpp"
#include "nq_internal.hpp"
#include "nq_wide.hpp"

namespace nq {

constexpr int BWW_ROWS = 64;  // query rows (dQ) or keys (dK/dV) per workgroup

template <bool CAUSAL>
__global__ void __launch_bounds__(256) bwd_dq_wide_kernel(BwdParams p) {
  constexpr int NDQ = PW_D / 32, NDO = PW_D / 16;
  __shared__ __attribute__((aligned(16))) unsigned char kt[PW_TILE_BYTES];   // K, row layout
  __shared__ __attribute__((aligned(16))) unsigned char ktt[PW_TILE_BYTES];  // K, tr layout
  __shared__ __attribute__((aligned(16))) unsigned char vt[PW_TILE_BYTES];   // V, row layout

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, grp = lane >> 4;
  const int nbh = p.B * p.Hq;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / nbh);  // heaviest q-blocks first
  const int bh = (int)(blockIdx.x % nbh);
  const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.G;
  const int q0 = qb * BWW_ROWS;
  const int row = q0 + wave * 16 + c16;
  const int rowc = row < p.S ? row : p.S - 1;

  // the row's scaled Q and dO as B operands, and Delta = rowsum(dO * O)
  const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)rowc * p.qss;
  const bf16* dorow = reinterpret_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh + (int64_t)rowc * p.doss;
  const bf16* orow = reinterpret_cast<const bf16*>(p.o) + b * p.osb + h * p.osh + (int64_t)rowc * p.oss;
  bf16x8 qop[NDQ], doop[NDQ];
  float dsum = 0.f;
#pragma unroll
  for (int dq = 0; dq < NDQ; ++dq) {
    floatx8 x = Vec8<bf16>::load_f32(qrow + dq * 32 + grp * 8);
    const floatx8 d = Vec8<bf16>::load_f32(dorow + dq * 32 + grp * 8);
    const floatx8 o = Vec8<bf16>::load_f32(orow + dq * 32 + grp * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] *= p.scale_log2;
      dsum += d[e] * o[e];
    }
    qop[dq] = to_bf16x8(x);
    doop[dq] = to_bf16x8(d);
  }
  dsum += shfl_xor_f(dsum, 16);
  dsum += shfl_xor_f(dsum, 32);
  const bool rv = row < p.S;
  const float delta = rv ? dsum : 0.f;
  const float lse2 = rv ? p.lse[((int64_t)b * p.Hq + h) * p.S + row] * kLog2e : 0.f;
  if (grp == 0 && (row >> 5) < p.nst) {
    float* w = p.ws + ((int64_t)bh * p.nst + (row >> 5)) * 64;
    w[row & 31] = lse2;
    w[32 + (row & 31)] = delta;
  }

  const int coff = p.coff;
  const int kv_end = CAUSAL ? min(p.T, q0 + BWW_ROWS + coff) : p.T;
  const int nsteps = (kv_end + PW_TILE - 1) / PW_TILE;
  const int lim = CAUSAL ? min(p.T - 1, row + coff) : p.T - 1;
  const bf16* kbase = reinterpret_cast<const bf16*>(p.k) + b * p.ksb + kvh * p.ksh;
  const bf16* vbase = reinterpret_cast<const bf16*>(p.v) + b * p.vsb + kvh * p.vsh;
  bf16x8 kr[PW_PIECES], vr[PW_PIECES];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PW_PIECES; ++i) {
      const int pc = threadIdx.x + 256 * i;
      const int key = min(k0 + (pc >> 5), p.T - 1);
      kr[i] = Vec8<bf16>::load_bf16(kbase + (int64_t)key * p.kss + (pc & 31) * 8);
      vr[i] = Vec8<bf16>::load_bf16(vbase + (int64_t)key * p.vss + (pc & 31) * 8);
    }
  };
  load(0);

  floatx4 acc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) acc[dd] = floatx4{};
  for (int s = 0; s < nsteps; ++s) {
    const int k0 = s * PW_TILE;
    __syncthreads();  // every wave is done with the previous tiles
#pragma unroll
    for (int i = 0; i < PW_PIECES; ++i) {
      const int pc = threadIdx.x + 256 * i;
      pw_store_row(kt, pc, kr[i]);
      pw_store_tr(ktt, pc, kr[i]);
      pw_store_row(vt, pc, vr[i]);
    }
    __syncthreads();
    if (s + 1 < nsteps) load(k0 + PW_TILE);

    floatx4 st[2], dpt[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      st[kb] = floatx4{};
      dpt[kb] = floatx4{};
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) {
        st[kb] = mfma16(pw_row_operand(kt, kb * 16, dq, lane), qop[dq], st[kb]);
        dpt[kb] = mfma16(pw_row_operand(vt, kb * 16, dq, lane), doop[dq], dpt[kb]);
      }
    }
    // lane: keys k0 + 16 kb + 4 grp + i of its row
    floatx8 dsf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool keep = k0 + kb * 16 + grp * 4 + i <= lim;
        const float pe = keep ? fast_exp2(st[kb][i] - lse2) : 0.f;
        dsf[kb * 4 + i] = pe * (dpt[kb][i] - delta);
      }
    const bf16x8 dsop = to_bf16x8(dsf);
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) acc[dd] = mfma16(pw_tr_operand(ktt, dd, lane), dsop, acc[dd]);
  }
  if (rv) {
    bf16* dqrow = reinterpret_cast<bf16*>(p.dq) + b * p.dqsb + h * p.dqsh + (int64_t)row * p.dqss;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) store4<bf16>(dqrow + dd * 16 + grp * 4, acc[dd] * p.scale);
  }
}

template <bool CAUSAL>
__global__ void __launch_bounds__(256) bwd_dkdv_wide_kernel(BwdParams p) {
  constexpr int NDQ = PW_D / 32, NDO = PW_D / 16;
  __shared__ __attribute__((aligned(16))) unsigned char qt[PW_TILE_BYTES];    // Q, row layout
  __shared__ __attribute__((aligned(16))) unsigned char qtt[PW_TILE_BYTES];   // Q, tr layout
  __shared__ __attribute__((aligned(16))) unsigned char dt[PW_TILE_BYTES];    // dO, row layout
  __shared__ __attribute__((aligned(16))) unsigned char dtt[PW_TILE_BYTES];   // dO, tr layout
  __shared__ float ld[64];  // the tile's LSE * log2 e and Delta

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, grp = lane >> 4;
  const int nbk = p.B * p.Hkv;
  const int kblk = (int)(blockIdx.x / nbk);  // low keys (most queries) first
  const int bk = (int)(blockIdx.x % nbk);
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  const int kb0 = kblk * BWW_ROWS;
  const int key = kb0 + wave * 16 + c16;  // this lane's key
  const int keyc = key < p.T ? key : p.T - 1;

  // the key's K and V rows as B operands
  const bf16* krow = reinterpret_cast<const bf16*>(p.k) + b * p.ksb + kvh * p.ksh + (int64_t)keyc * p.kss;
  const bf16* vrow = reinterpret_cast<const bf16*>(p.v) + b * p.vsb + kvh * p.vsh + (int64_t)keyc * p.vss;
  bf16x8 kop[NDQ], vop[NDQ];
#pragma unroll
  for (int dq = 0; dq < NDQ; ++dq) {
    kop[dq] = Vec8<bf16>::load_bf16(krow + dq * 32 + grp * 8);
    vop[dq] = Vec8<bf16>::load_bf16(vrow + dq * 32 + grp * 8);
  }

  // query tiles of each of the G heads; causal: only rows i >= kb0 - coff see this block
  const int coff = p.coff;
  const int t0 = CAUSAL ? max(0, kb0 - coff) / PW_TILE : 0;
  const int ntl = t0 < p.nst ? p.nst - t0 : 0;
  const int nsteps = ntl * p.G;
  bf16x8 qr[PW_PIECES], dr[PW_PIECES];
  float wv = 0.f;
  auto load = [&](int s) {
    const int g = s / ntl, t = t0 + s % ntl;
    const int h = kvh * p.G + g;
    const bf16* qb = reinterpret_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh;
    const bf16* db = reinterpret_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh;
#pragma unroll
    for (int i = 0; i < PW_PIECES; ++i) {
      const int pc = threadIdx.x + 256 * i;
      const int r = min(t * PW_TILE + (pc >> 5), p.S - 1);
      qr[i] = Vec8<bf16>::load_bf16(qb + (int64_t)r * p.qss + (pc & 31) * 8);
      dr[i] = Vec8<bf16>::load_bf16(db + (int64_t)r * p.doss + (pc & 31) * 8);
    }
    if (threadIdx.x < 64) wv = p.ws[(((int64_t)b * p.Hq + h) * p.nst + t) * 64 + threadIdx.x];
  };
  if (nsteps > 0) load(0);

  floatx4 dk[NDO], dv[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) {
    dk[dd] = floatx4{};
    dv[dd] = floatx4{};
  }
  for (int s = 0; s < nsteps; ++s) {
    const int row0 = (t0 + s % ntl) * PW_TILE;
    __syncthreads();  // every wave is done with the previous tiles
#pragma unroll
    for (int i = 0; i < PW_PIECES; ++i) {
      const int pc = threadIdx.x + 256 * i;
      pw_store_row(qt, pc, qr[i]);
      pw_store_tr(qtt, pc, qr[i]);
      pw_store_row(dt, pc, dr[i]);
      pw_store_tr(dtt, pc, dr[i]);
    }
    if (threadIdx.x < 64) ld[threadIdx.x] = wv;
    __syncthreads();
    if (s + 1 < nsteps) load(s + 1);

    // S and dP (rows x keys): lane holds rows 16 mb + 4 grp + i of its key
    floatx4 st[2], dpt[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      st[mb] = floatx4{};
      dpt[mb] = floatx4{};
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) {
        st[mb] = mfma16(pw_row_operand(qt, mb * 16, dq, lane), kop[dq], st[mb]);
        dpt[mb] = mfma16(pw_row_operand(dt, mb * 16, dq, lane), vop[dq], dpt[mb]);
      }
    }
    floatx8 pf, dsf;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rl = mb * 16 + grp * 4 + i, r = row0 + rl;
        const bool keep = r < p.S && key < p.T && (!CAUSAL || key <= r + coff);
        const float pe = keep ? fast_exp2(st[mb][i] * p.scale_log2 - ld[rl]) : 0.f;
        pf[mb * 4 + i] = pe;
        dsf[mb * 4 + i] = pe * (dpt[mb][i] - ld[32 + rl]);
      }
    const bf16x8 pop = to_bf16x8(pf), dsop = to_bf16x8(dsf);
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      dv[dd] = mfma16(pw_tr_operand(dtt, dd, lane), pop, dv[dd]);
      dk[dd] = mfma16(pw_tr_operand(qtt, dd, lane), dsop, dk[dd]);
    }
  }
  if (key < p.T) {
    bf16* dkrow = reinterpret_cast<bf16*>(p.dk) + b * p.dksb + kvh * p.dksh + (int64_t)key * p.dkss;
    bf16* dvrow = reinterpret_cast<bf16*>(p.dv) + b * p.dvsb + kvh * p.dvsh + (int64_t)key * p.dvss;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      store4<bf16>(dkrow + dd * 16 + grp * 4, dk[dd] * p.scale);
      store4<bf16>(dvrow + dd * 16 + grp * 4, dv[dd]);
    }
  }
}

hipError_t launch_bwd_wide(const BwdParams& p, bool causal, hipStream_t st) {
  const dim3 block(256);
  const dim3 gq((unsigned)((int64_t)p.nqb * p.B * p.Hq));
  const dim3 gk((unsigned)((int64_t)((p.T + BWW_ROWS - 1) / BWW_ROWS) * p.B * p.Hkv));
  if (causal) hipLaunchKernelGGL(bwd_dq_wide_kernel<true>, gq, block, 0, st, p);
  else hipLaunchKernelGGL(bwd_dq_wide_kernel<false>, gq, block, 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (causal) hipLaunchKernelGGL(bwd_dkdv_wide_kernel<true>, gk, block, 0, st, p);
  else hipLaunchKernelGGL(bwd_dkdv_wide_kernel<false>, gk, block, 0, st, p);
  return hipGetLastError();
}

}  // namespace nq
