// Prefill at head_dim 256, for gfx950.
//
// kernels/flash_attn.py:106 accepts head_dim 256 (no reference model config
// uses it).  This is plain attention: bf16 q, k, v, o with (b, h, s) strides
// and contiguous head dims, GQA by indexing (kv head = h / G), causal with
// the bottom-right frontier (query i keeps keys j <= i + T - S), optional LSE
// output.  QK-Norm / RoPE fusion, key lengths, biases and paged caches stay
// with the head_dim 32-128 kernels.
//
// Decomposition: a workgroup of 4 waves takes 64 query rows of one head, 16
// per wave, and walks the keys 32 at a time.  K and V tiles (32 rows x 512 B)
// are loaded cooperatively, one step ahead into registers, and stored to LDS
// (K in the row layout, V in the tr layout of nq_wide.hpp); every wave reads
// them as MFMA operands:
//   S^T (keys x rows) = K Q^T on v_mfma_f32_16x16x32_bf16 (A = K from LDS,
//   ds_read_b128; B = Q in registers, pre-scaled by sm_scale * log2 e), and
//   O^T (dims x rows) += V^T P^T (A = V^T by transpose reads, B = P in
//   registers), 16 output blocks of 16 dims.
// A lane owns 8 scores of one query row (its column), so the online softmax
// is lane-local plus two xor shuffles, as in the decode kernel.

#include "nq_common.hpp"
#include "nq_internal.hpp"
#include "nq_prefill.hpp"
#include "nq_wide.hpp"

namespace nq {

constexpr int PW_KEYS = PW_TILE;   // keys per step
constexpr int PW_ROWS = 64;        // query rows per workgroup (16 per wave)

// Two workgroups per CU (the compiler fits 220 registers, no spills): one
// hides the other's tile stores and barriers (+57% over one per CU, which
// the compiler's default of 264 registers gave).
template <bool CAUSAL>
__global__ void __launch_bounds__(256, 2) prefill_wide_kernel(PrefillParams p) {
  constexpr int NDQ = PW_D / 32;  // 32-wide k-steps of S^T
  constexpr int NDO = PW_D / 16;  // 16-wide output blocks
  __shared__ __attribute__((aligned(16))) unsigned char kt[PW_TILE_BYTES];  // row layout
  __shared__ __attribute__((aligned(16))) unsigned char vt[PW_TILE_BYTES];  // tr layout

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, grp = lane >> 4;

  // workgroup -> (q-block, batch, head), heaviest q-blocks of every head first
  const int nbh = p.B * p.Hq;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / nbh);
  const int bh = (int)(blockIdx.x % nbh);
  const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.G;
  const int q0 = qb * PW_ROWS;
  const int coff = p.T - p.S;
  const int row = q0 + wave * 16 + c16;  // this lane's query row
  const int rowc = row < p.S ? row : p.S - 1;
  const int kv_end = CAUSAL ? min(p.T, q0 + PW_ROWS + coff) : p.T;
  const int nsteps = (kv_end + PW_KEYS - 1) / PW_KEYS;

  // Q operand (B of S^T): lane holds Q[row][dq*32 + grp*8 + e], scaled
  const bf16* qrow = reinterpret_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)rowc * p.qss;
  bf16x8 qop[NDQ];
#pragma unroll
  for (int dq = 0; dq < NDQ; ++dq) {
    floatx8 x = Vec8<bf16>::load_f32(qrow + dq * 32 + grp * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= p.scale_log2;
    qop[dq] = to_bf16x8(x);
  }

  // tile pieces: thread t moves pieces t + 256 i (row = piece / 32, chunk = piece % 32);
  // rows past T read row T - 1 (finite values; their scores are masked)
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

  const int lim = CAUSAL ? min(p.T - 1, row + coff) : p.T - 1;  // last key this row keeps

  float m_i = -INFINITY, l_i = 0.f;
  floatx4 oacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx4{};

  for (int s = 0; s < nsteps; ++s) {
    const int k0 = s * PW_KEYS;
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int i = 0; i < PW_PIECES; ++i) {
      pw_store_row(kt, threadIdx.x + 256 * i, kr[i]);
      pw_store_tr(vt, threadIdx.x + 256 * i, vr[i]);
    }
    __syncthreads();
    if (s + 1 < nsteps) load(k0 + PW_KEYS);

    floatx4 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = floatx4{};
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) sc[kb] = mfma16(pw_row_operand(kt, kb * 16, dq, lane), qop[dq], sc[kb]);
    }
    if (k0 + PW_KEYS - 1 > lim) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + kb * 16 + grp * 4 + i > lim) sc[kb][i] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][i]);
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    // key 0 is in every row's first step (T >= S), so m_new is finite from step 0 on
    const float m_new = fmaxf(m_i, mx);
    const float alpha = fast_exp2(m_i - m_new);
    floatx8 pf;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pe = fast_exp2(sc[kb][i] - m_new);
        pf[kb * 4 + i] = pe;
        rs += pe;
      }
    const bf16x8 pop = to_bf16x8(pf);
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      oacc[dd] *= alpha;
      oacc[dd] = mfma16(pw_tr_operand(vt, dd, lane), pop, oacc[dd]);
    }
  }

  l_i += shfl_xor_f(l_i, 16);
  l_i += shfl_xor_f(l_i, 32);
  if (row < p.S) {
    const float inv = 1.0f / l_i;
    bf16* orow = reinterpret_cast<bf16*>(p.o) + b * p.osb + h * p.osh + (int64_t)row * p.oss;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) store4<bf16>(orow + dd * 16 + grp * 4, oacc[dd] * inv);
    if (p.lse && grp == 0) p.lse[((int64_t)b * p.Hq + h) * p.S + row] = (m_i + __log2f(l_i)) * kLn2;
  }
}

hipError_t launch_prefill_wide(const PrefillParams& p, bool causal, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)p.nqb * p.B * p.Hq)), block(256);
  if (causal) hipLaunchKernelGGL(prefill_wide_kernel<true>, grid, block, 0, st, p);
  else hipLaunchKernelGGL(prefill_wide_kernel<false>, grid, block, 0, st, p);
  return hipGetLastError();
}

}  // namespace nq
