// Single-token GQA decode against a ragged KV cache, split-K, for gfx950.
//
// Replaces model/attention.py:95-115 at S == 1 with a KVCache (the decode
// step driven by eval/generate.py:135): QK-Norm + RoPE of the new query
// (fused into its load), attention over keys [0, lens[b]) with no mask
// (attention.py:113: is_causal=False when a cache is present), and the GQA
// expansion of attention.py:106-108 done by indexing, never materialised.
//
// Work decomposition
//   grid (split, kv-head x head-group, batch).  A workgroup (4 waves) takes
//   `chunk` consecutive keys of one (batch, kv head) and up to 16 query heads
//   of that kv head's group; those 16 heads form the N side of
//   v_mfma_f32_16x16x32_bf16 for both S^T = K Q^T (A = 16 keys x 32 dims,
//   loaded straight from HBM in 16-byte pieces) and O^T += V^T P^T (A = V^T,
//   staged through a per-wave LDS transpose).  Waves stride over 32-key steps
//   of the chunk.  Each lane owns one head column, so the softmax reductions
//   are two xor shuffles.  The four waves merge in LDS; a workgroup writes
//   either the final row (single split) or an fp32 partial (O/l, m, l) that
//   decode_merge_kernel combines.  Workgroups whose chunk starts past
//   lens[b] exit at once, so the grid can be sized from max_len.
//
// The cache is read exactly once: HBM-bound at 16 FLOP/byte for G = 16.

#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

constexpr int DC_THREADS = 256;
constexpr int DC_STEP = 32;             // keys per wave step
constexpr int DC_DEFAULT_CHUNK = 1024;  // keys per split

struct DecodeParams {
  const void* q;
  int64_t qsb, qsh;
  const void* kc;
  int64_t ksb, ksh, kst;
  const void* vc;
  int64_t vsb, vsh, vst;
  const int32_t* lens;
  void* o;
  int64_t osb, osh;
  float* ws_o;   // (B, Hq, nsplit, D) normalised partial outputs
  float* ws_ml;  // (B, Hq, nsplit, 2)  (m in log2 units, l)
  const float* qw;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int max_pos;
  const int32_t* q_pos;
  int q_pos0;
  int B, Hq, Hkv, G, NG, nsplit, chunk, max_len;
  float scale_log2;
};

template <int D, typename T>
__global__ void __attribute__((amdgpu_flat_work_group_size(DC_THREADS, DC_THREADS)))
decode_split_kernel(DecodeParams p) {
  constexpr int NDQ = D / 32;         // 32-wide d blocks (QK^T k-steps)
  constexpr int NDO = D / 16;         // 16-wide d blocks (output tiles)
  constexpr int CPR = D / 8;          // 16-byte chunks per V row
  constexpr int VS = D + 16;          // V row stride (elements) in LDS: +32 B
  constexpr int V_LOADS = DC_STEP * CPR / 64;  // 16-byte V loads per lane per step
  constexpr int WAVE_LDS = DC_STEP * VS;       // bf16 elements per wave
  constexpr int COMB_F = 4 * 16 * D + 2 * 4 * 16;  // floats for the wave merge
  constexpr int LDS_BYTES = (4 * WAVE_LDS * 2 > COMB_F * 4) ? 4 * WAVE_LDS * 2 : COMB_F * 4;
  __shared__ __attribute__((aligned(16))) unsigned char smem_raw[LDS_BYTES];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y / p.NG, hgi = blockIdx.y % p.NG;
  const int b = blockIdx.z;
  // lens[b] is clamped to max_len (the caller guarantees max_len <= T_cap), so
  // no key past the cache capacity is ever read.
  const int len = p.lens ? min(p.lens[b], p.max_len) : p.max_len;
  const int s0 = split * p.chunk;
  if (len <= 0) {
    // empty row: defined output (zeros) instead of an unwritten buffer
    if (split == 0) {
      for (int idx = threadIdx.x; idx < 16 * D; idx += DC_THREADS) {
        const int ghq = hgi * 16 + idx / D;
        if (ghq < p.G)
          (reinterpret_cast<T*>(p.o) + b * p.osb + (kvh * p.G + ghq) * p.osh)[idx % D] = static_cast<T>(0.f);
      }
    }
    return;
  }
  if (s0 >= len) return;
  const int s1 = min(len, s0 + p.chunk);
  const int nsplit_b = (len + p.chunk - 1) / p.chunk;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, grp = lane >> 4;
  const int gh = hgi * 16 + c16;
  const bool hvalid = gh < p.G;
  const int head = kvh * p.G + (hvalid ? gh : 0);

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[head c16][dq*32 + grp*8 + e]
  bf16x8 qop[NDQ];
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh;
    floatx8 xf[NDQ];
#pragma unroll
    for (int dq = 0; dq < NDQ; ++dq) xf[dq] = Vec8<T>::load_f32(qrow + dq * 32 + grp * 8);
    if (p.qw) {
      float ss = 0.f;
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xf[dq][e] * xf[dq][e];
      ss += shfl_xor_f(ss, 16);
      ss += shfl_xor_f(ss, 32);
      const float r = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) {
        floatx8 w = Vec8<float>::load_f32(p.qw + dq * 32 + grp * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[dq][e] = xf[dq][e] * r * w[e];
      }
    }
    if (p.cos_tab) {
      const int pos = clamp_pos(p.q_pos ? p.q_pos[b] : (p.q_pos0 >= 0 ? p.q_pos0 : len - 1), p.max_pos);
      const float* ct = p.cos_tab + (int64_t)pos * (D / 2);
      const float* st = p.sin_tab + (int64_t)pos * (D / 2);
#pragma unroll
      for (int dq = 0; dq < NDQ / 2; ++dq) {
        floatx8 c = Vec8<float>::load_f32(ct + dq * 32 + grp * 8);
        floatx8 s = Vec8<float>::load_f32(st + dq * 32 + grp * 8);
        floatx8 x1 = xf[dq], x2 = xf[dq + NDQ / 2];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xf[dq][e] = x1[e] * c[e] - x2[e] * s[e];
          xf[dq + NDQ / 2][e] = x2[e] * c[e] + x1[e] * s[e];
        }
      }
    }
#pragma unroll
    for (int dq = 0; dq < NDQ; ++dq) qop[dq] = hvalid ? to_bf16x8(xf[dq]) : bf16x8{};
  }

  const T* kbase = reinterpret_cast<const T*>(p.kc) + b * p.ksb + kvh * p.ksh;
  const T* vbase = reinterpret_cast<const T*>(p.vc) + b * p.vsb + kvh * p.vsh;
  bf16* Vs = reinterpret_cast<bf16*>(smem_raw) + wave * WAVE_LDS;
  const bf16x8 zero8 = {};
  // V^T operand via transpose reads: lane group grp, j = lane%16: source row
  // 4*grp + j/4 (+16 for the second half), column 4*(j%4) (+dd*16).  Rows
  // 16*half + 4*grp + [0,4) are exactly the keys of this lane's P values.
  const int jj = lane & 15;
  const int v_off = (4 * grp + (jj >> 2)) * VS + 4 * (jj & 3);

  float m_i = -INFINITY, l_i = 0.f;
  floatx4 oacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx4{};

  const int nsteps = (s1 - s0 + DC_STEP - 1) / DC_STEP;
  for (int t = wave; t < nsteps; t += 4) {
    const int k0 = s0 + t * DC_STEP;
    // K as MFMA A operand: block kb, row r holds key kb*16 + r
    bf16x8 ka[2][NDQ];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key = k0 + kb * 16 + c16;
      const bool ok = key < s1;
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq)
        ka[kb][dq] = ok ? Vec8<T>::load_bf16(kbase + (int64_t)key * p.kst + dq * 32 + grp * 8) : zero8;
    }
    // V rows, whole rows per 16 lanes: chunk c = lane + 64*i
    bf16x8 vr[V_LOADS];
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int c = lane + 64 * i;
      const int key = k0 + c / CPR;
      vr[i] = key < s1 ? Vec8<T>::load_bf16(vbase + (int64_t)key * p.vst + (c % CPR) * 8) : zero8;
    }

    floatx4 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = floatx4{};
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) sc[kb] = mfma16(ka[kb][dq], qop[dq], sc[kb]);
    }
    if (k0 + DC_STEP > s1) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + kb * 16 + grp * 4 + i >= s1) sc[kb][i] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][i]);
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float m_new = fmaxf(m_i, mx * p.scale_log2);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    floatx8 pf;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pe = fast_exp2(sc[kb][i] * p.scale_log2 - m_use);
        pf[kb * 4 + i] = pe;
        rs += pe;
      }
    const bf16x8 pop = to_bf16x8(pf);
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) oacc[dd] *= alpha;

    // V rows into this wave's LDS slab (row-major), read back transposed
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int c = lane + 64 * i;
      *reinterpret_cast<bf16x8*>(Vs + (c / CPR) * VS + (c % CPR) * 8) = vr[i];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      const bf16* src = Vs + v_off + dd * 16;
      bf16x8 a = lds_read_tr8(src, src + 16 * VS);
      oacc[dd] = mfma16(a, pop, oacc[dd]);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the four waves through LDS
  l_i += shfl_xor_f(l_i, 16);
  l_i += shfl_xor_f(l_i, 32);
  __syncthreads();
  float* co = reinterpret_cast<float*>(smem_raw);        // [wave][16][D]
  float* cm = co + 4 * 16 * D;                          // [wave][16]
  float* cl = cm + 4 * 16;                              // [wave][16]
  if (grp == 0) {
    cm[wave * 16 + c16] = m_i;
    cl[wave * 16 + c16] = l_i;
  }
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int i = 0; i < 4; ++i) co[(wave * 16 + c16) * D + dd * 16 + grp * 4 + i] = oacc[dd][i];
  __syncthreads();

  const bool single = nsplit_b == 1;
  for (int idx = tid; idx < 16 * D; idx += DC_THREADS) {
    const int hq = idx / D, d = idx - hq * D;
    const int ghq = hgi * 16 + hq;
    if (ghq >= p.G) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, cm[w * 16 + hq]);
    float wsum = 0.f, osum = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = fast_exp2(cm[w * 16 + hq] - M);
      wsum += cl[w * 16 + hq] * sc;
      osum += co[(w * 16 + hq) * D + d] * sc;
    }
    const int hglob = kvh * p.G + ghq;
    if (single) {
      T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + hglob * p.osh;
      orow[d] = static_cast<T>(osum / wsum);
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + hglob) * p.nsplit + split;
      p.ws_o[slot * D + d] = osum / wsum;
      if (d == 0) {
        p.ws_ml[slot * 2 + 0] = M;
        p.ws_ml[slot * 2 + 1] = wsum;
      }
    }
  }
}

// One workgroup per (batch, query head); one lane per output element.
template <int D, typename T>
__global__ void __launch_bounds__(D) decode_merge_kernel(DecodeParams p) {
  const int b = blockIdx.y, h = blockIdx.x, d = threadIdx.x;
  const int len = p.lens ? min(p.lens[b], p.max_len) : p.max_len;
  const int ns = (len + p.chunk - 1) / p.chunk;
  if (ns <= 1) return;
  const int64_t base = ((int64_t)b * p.Hq + h) * p.nsplit;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, p.ws_ml[(base + s) * 2]);
  float wsum = 0.f, osum = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float w = p.ws_ml[(base + s) * 2 + 1] * fast_exp2(p.ws_ml[(base + s) * 2] - M);
    wsum += w;
    osum += w * p.ws_o[(base + s) * D + d];
  }
  T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + h * p.osh;
  orow[d] = static_cast<T>(osum / wsum);
}

template <int D, typename T>
static hipError_t launch_decode(const DecodeParams& p, hipStream_t st) {
  dim3 grid((unsigned)p.nsplit, (unsigned)(p.Hkv * p.NG), (unsigned)p.B);
  hipLaunchKernelGGL((decode_split_kernel<D, T>), grid, dim3(DC_THREADS), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.nsplit <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<D, T>), dim3((unsigned)p.Hq, (unsigned)p.B), dim3(D), 0, st, p);
  return hipGetLastError();
}

static int decode_chunk(int chunk) {
  if (chunk <= 0) return DC_DEFAULT_CHUNK;
  return ((chunk + DC_STEP - 1) / DC_STEP) * DC_STEP;
}

}  // namespace nq

using namespace nq;

extern "C" int64_t nq_attn_decode_workspace_bytes(int B, int Hq, int D, int max_len, int chunk) {
  if (B <= 0 || Hq <= 0 || D <= 0 || max_len <= 0) return 0;
  const int c = decode_chunk(chunk);
  const int64_t nsplit = (max_len + c - 1) / c;
  if (nsplit <= 1) return 0;
  return (int64_t)B * Hq * nsplit * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int nq_attn_decode_fwd(const void* q, const int64_t* q_strides, const void* k_cache,
                                  const int64_t* k_strides, const void* v_cache,
                                  const int64_t* v_strides, const int32_t* lens, void* o,
                                  const int64_t* o_strides, void* workspace,
                                  int64_t workspace_bytes, int B, int Hq, int Hkv, int D,
                                  int max_len, int chunk, int dtype, const float* q_weight,
                                  float eps, const float* cos_tab, const float* sin_tab,
                                  int max_pos, const int32_t* q_pos, int q_pos0, float sm_scale,
                                  void* stream) {
  nq_clear_error();
  if (D != 64 && D != 128) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d max_len=%d)", B, Hq, Hkv, max_len);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  if (!q || !k_cache || !v_cache || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return nq_fail(NQ_ERR_INVALID, "q, caches, o and their strides are required");
  if (!nq_aligned16(q) || !nq_aligned16(k_cache) || !nq_aligned16(v_cache))
    return nq_fail(NQ_ERR_INVALID, "q and cache base pointers must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  for (int i = 0; i < 2; ++i)
    if ((q_strides[i] * esz) % 16) return nq_fail(NQ_ERR_INVALID, "q strides must be multiples of 16 bytes");
  for (int i = 0; i < 3; ++i)
    if ((k_strides[i] * esz) % 16 || (v_strides[i] * esz) % 16)
      return nq_fail(NQ_ERR_INVALID, "cache strides must be multiples of 16 bytes");
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  const int c = decode_chunk(chunk);
  const int64_t need = nq_attn_decode_workspace_bytes(B, Hq, D, max_len, c);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return nq_fail(NQ_ERR_WORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                   (long long)workspace_bytes);
  DecodeParams p{};
  p.q = q; p.qsb = q_strides[0]; p.qsh = q_strides[1];
  p.kc = k_cache; p.ksb = k_strides[0]; p.ksh = k_strides[1]; p.kst = k_strides[2];
  p.vc = v_cache; p.vsb = v_strides[0]; p.vsh = v_strides[1]; p.vst = v_strides[2];
  p.lens = lens; p.o = o; p.osb = o_strides[0]; p.osh = o_strides[1];
  p.qw = q_weight; p.eps = eps; p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.q_pos = q_pos; p.q_pos0 = q_pos0;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = Hq / Hkv; p.NG = (p.G + 15) / 16;
  p.chunk = c;
  p.max_len = max_len;
  p.nsplit = (max_len + c - 1) / c;
  if (p.nsplit > 1) {
    p.ws_o = reinterpret_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (int64_t)B * Hq * p.nsplit * D;
  }
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == NQ_DTYPE_BF16)
    e = (D == 128) ? launch_decode<128, bf16>(p, st) : launch_decode<64, bf16>(p, st);
  else
    e = (D == 128) ? launch_decode<128, float>(p, st) : launch_decode<64, float>(p, st);
  return nq_check_launch(e);
}
