// Single-token GQA decode against a ragged KV cache, for gfx950.
//
// Replaces model/attention.py:95-115 at S == 1 with a KVCache (the decode
// step driven by eval/generate.py:135): QK-Norm + RoPE of the new query
// (fused into its load), attention over keys [0, lens[b]) with no mask
// (attention.py:113: is_causal=False when a cache is present), and the GQA
// expansion of attention.py:106-108 done by indexing, never materialised.
//
// Work decomposition (a balanced partition of the whole cache)
//   A "row" is one (batch b, kv head, group of up to 16 query heads); rows are
//   ordered r = (b * Hkv + kv head) * NG + group and row r is cut into
//   ceil(lens[b] / 32) steps of 32 keys.  Concatenating the steps of all rows
//   gives N steps.  Each wave of the grid takes one contiguous range of that
//   sequence: with chunk == 0 the N steps are split evenly over the resident
//   waves (a persistent grid sized to the device), otherwise every wave takes
//   chunk/32 steps.  Either way every wave streams the same number of bytes
//   (to one step), whatever the spread of lens, and no workgroup is launched
//   only to find its keys past lens[b].
//
//   A wave walks its range row by row.  For each row segment it QK-Norms and
//   rotates the row's query heads (the N side of v_mfma_f32_16x16x32_bf16),
//   then streams K and V 32 keys at a time: full 256-byte rows, nontemporal,
//   one step ahead into registers, then into a wave-private LDS tile with an
//   XOR swizzle, read back as the MFMA A operand (K, ds_read_b128) and as V^T
//   (ds_read_b64_tr_b16); both read patterns are free of bank conflicts.  The
//   online softmax is lane-local per head plus two xor shuffles.
//
//   A wave that covers a whole row writes the output row itself.  Otherwise
//   it writes an fp32 partial (unnormalised O, running max m, sum l) to slot
//   (wave + row) of the workspace: because ranges are contiguous and ordered,
//   two (wave, row) pairs with the same sum cannot both occur, so at most
//   waves + rows slots are used.  The waves holding a row's first and last
//   step record their index for it; decode_merge_kernel reads the two and
//   combines the partials in between (and writes zeros for rows with no
//   keys).
//
// The cache is read exactly once: HBM-bound at 16 FLOP/byte for G = 16.

#include <type_traits>

#include "nq_common.hpp"
#include "nq_internal.hpp"
#include "nq_prefill.hpp"

#include <mutex>

namespace nq {

constexpr int DC_THREADS = 256;  // four independent waves
constexpr int DC_WAVES = DC_THREADS / 64;
constexpr int DC_STEP = 32;      // keys per wave step
constexpr int DC_WG_PER_CU = 1;  // resident workgroups per CU for the persistent grid
constexpr int DC_MAX_WAVES = 1024;  // persistent grid cap: 256 CUs x 1 workgroup x 4 waves

struct DecodeParams {
  const void* q;
  int64_t qsb, qsh;
  // dense: (batch, kv head, row) strides of a (B, Hkv, T, D) cache;
  // paged: (page, kv head, row) strides of a (pages, Hkv, page_size, D) pool
  void* kc;
  int64_t ksb, ksh, kst;
  void* vc;
  int64_t vsb, vsh, vst;
  const int32_t* lens;
  void* o;
  int64_t osb, osh;
  float* ws_o;   // (slots, 16, D) unnormalised partial outputs
  float* ws_ml;  // (slots, 16, 2) running max (log2 units) and sum
  int32_t* ws_rw;  // (rows, 2) first and last wave that covered each row
  const float* qw;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int max_pos;
  const int32_t* q_pos;
  int q_pos0;
  int B, Hq, Hkv, G, NG, max_len;
  int rows_per_batch;  // Hkv * NG
  int nwaves;          // waves launched
  int span;            // steps per wave; 0 = split N evenly over nwaves
  float scale_log2;
  int append;          // 1: a new key per batch row is appended (see kn)
  // paged: block table (row b at bt + b * bts) and rows per page (a multiple
  // of DC_STEP)
  const int32_t* bt;
  int64_t bts;
  int page;
  // fused append: the new token's raw K (normed with kw, rotated) and V go to
  // row lens[b] of the cache and are attended
  const void* kn;
  int64_t knsb, knsh;
  const void* vn;
  int64_t vnsb, vnsh;
  const float* kw;
  int32_t* lens_out;  // lens[b] + 1 after an append (never aliases lens)
};

// LDS tile of DC_STEP rows (keys) x D bf16, 16-byte chunks XOR-swizzled per row.
template <int D>
struct DcTile {
  static constexpr int RB = 2 * D;                 // bytes per row
  static constexpr int CPR = D / 8;                // 16-byte chunks per row
  static constexpr int RPB = 256 / RB;             // rows per 256-byte bank row
  static constexpr int BYTES = DC_STEP * RB;       // one K or V tile
  static constexpr int RPI = 64 / CPR;             // rows per 64-lane load
  static constexpr int LOADS = DC_STEP / RPI;      // 16-byte pieces per lane per tile
  // K: a ds_read_b128 of one chunk from 16 consecutive rows hits 16 distinct
  // 16-byte bank groups.
  __device__ static int kswz(int row) { return (row / RPB) % CPR; }
  // V: a transpose read of 32 bytes from 8 consecutive rows hits 8 distinct
  // 32-byte bank groups.
  __device__ static int vswz(int row) { return ((row / RPB) % (CPR / 2)) * 2; }
};

// K/V pieces come through buffer loads: the descriptor's range ends after the
// last key of the segment, so the hardware returns zeros for keys past it (no
// per-lane branches, and NaN-poisoned or unallocated rows are never read).
// aux = 2 marks the loads nontemporal (each cache byte is read once).
constexpr int DC_BUF_FLAGS = 0x00020000;  // gfx9 raw-buffer descriptor word 3
constexpr int DC_AUX_NT = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dc_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, DC_BUF_FLAGS);
}

// Storage type -> 8-element piece held between the HBM load and the LDS store.
template <typename T> struct Piece;
template <> struct Piece<bf16> {
  typedef bf16x8 type;
  __device__ __forceinline__ static type load(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, DC_AUX_NT));
  }
  __device__ __forceinline__ static bf16x8 to_bf16(type v) { return v; }
};

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------- schedule
// Keys attended by batch row b (the appended key included), or -1 for a row
// whose length lies outside [0, max_len - append]: such a row attends
// nothing, appends nothing and its output is NaN (a cache row past max_len is
// not the caller's to give).
__device__ __forceinline__ int batch_len(const DecodeParams& p, int b) {
  if (!p.lens) return p.max_len;
  const int l = p.lens[b];
  return (l < 0 || l > p.max_len - p.append) ? -1 : l + p.append;
}
__device__ __forceinline__ int batch_steps(const DecodeParams& p, int b) {
  const int len = batch_len(p, b);
  return len > 0 ? (len + DC_STEP - 1) / DC_STEP : 0;
}
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ int64_t lane_value_i64(int64_t v, int src) {
  const int lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, src);
  const int hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Total number of steps N over all rows (same value in every lane).
__device__ int64_t total_steps(const DecodeParams& p, int lane) {
  int64_t acc = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    if (b < p.B) acc += batch_steps(p, b);
  }
  return wave_sum_i64(acc) * p.rows_per_batch;
}

// The batch whose rows hold global step q (q < N), and the steps before it.
__device__ void find_batch(const DecodeParams& p, int lane, int64_t q, int& b_out, int64_t& before) {
  int64_t run = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    const int64_t v = b < p.B ? (int64_t)batch_steps(p, b) * p.rows_per_batch : 0;
    int64_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const int64_t excl = run + incl - v;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(v > 0 && excl <= q && q < excl + v);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      b_out = base + src;
      before = lane_value_i64(excl, src);
      return;
    }
    run += lane_value_i64(incl, 63);
  }
  b_out = p.B - 1;  // not reached for q < N
  before = run;
}

// Effective number of waves of the balanced split (never more than N).
__device__ __forceinline__ int64_t waves_used(const DecodeParams& p, int64_t N) {
  return p.span > 0 ? (N + p.span - 1) / p.span : min((int64_t)p.nwaves, N);
}
// The persistent split weights the waves by the XCD they run on (workgroup i
// runs on XCD i mod 8): a wave on an odd XCD takes DC_ODD_W / DC_EVEN_W of the
// steps of one on an even XCD.  Timestamps per wave on MI355X put the odd XCDs'
// waves 12-15% behind the even ones' over the same number of steps, whichever
// rows they stream (their share of the memory system is smaller), so an even
// split left the even XCDs idle for the last tenth of the kernel.
constexpr int DC_EVEN_W = 25, DC_ODD_W = 22;
// Total weight of waves [0, w).
__device__ __forceinline__ int64_t split_weight(int64_t w) {
  constexpr int GW = DC_WAVES * 8;  // the waves of one workgroup on each XCD
  const int64_t rounds = w / GW;
  const int k = (int)(w % GW), g = k / DC_WAVES, r = k % DC_WAVES;
  return rounds * (DC_WAVES * 4) * (DC_EVEN_W + DC_ODD_W) +
         ((int64_t)((g + 1) / 2) * DC_EVEN_W + (int64_t)(g / 2) * DC_ODD_W) * DC_WAVES +
         (int64_t)r * ((g & 1) ? DC_ODD_W : DC_EVEN_W);
}
// First global step of wave w (the chunked form: span steps per wave).  The
// weighted split applies when it still gives every wave at least one step (a
// wave with none would leave a gap in a row's run of partials); otherwise the
// steps are split evenly.
__device__ __forceinline__ int64_t wave_begin(const DecodeParams& p, int64_t N, int64_t We, int64_t w) {
  if (p.span > 0) return min(N, w * p.span);
  const int64_t total = split_weight(We);
  return N * DC_ODD_W >= total ? split_weight(w) * N / total : w * N / We;
}
// ---------------------------------------------------------------- kernels
// bf16 caches (fp32 caches run the fp32 prefill kernel at S = 1)
template <int D, typename T, bool PAGED, bool APPEND>
__global__ void __attribute__((amdgpu_flat_work_group_size(DC_THREADS, DC_THREADS), amdgpu_waves_per_eu(DC_WG_PER_CU)))
decode_stream_kernel(DecodeParams p) {
  static_assert(std::is_same<T, bf16>::value, "bf16 cache");
  using L = DcTile<D>;
  using P8 = Piece<T>;
  constexpr int NDQ = D / 32;  // 32-wide d blocks (QK^T k-steps)
  constexpr int NDO = D / 16;  // 16-wide d blocks (output tiles)
  constexpr int LPR = D / 16;  // lanes holding one appended row
  __shared__ __attribute__((aligned(16))) unsigned char smem[DC_WAVES * 2 * L::BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t w = (int64_t)blockIdx.x * DC_WAVES + wave;

  const int64_t N = lane_value_i64(total_steps(p, lane), 0);
  if (N == 0) return;
  const int64_t We = waves_used(p, N);
  if (w >= We) return;
  const int64_t q0 = wave_begin(p, N, We, w), q1 = wave_begin(p, N, We, w + 1);
  if (q0 >= q1) return;

  // lens of up to 64 batch rows kept in a register: no memory round trip at a
  // row boundary
  const bool lens_in_reg = p.B <= 64;
  const int lens_lane = lens_in_reg && lane < p.B ? batch_len(p, lane) : 0;
  auto len_of = [&](int bb) {
    return lens_in_reg ? __builtin_amdgcn_readlane(lens_lane, bb) : uniform(batch_len(p, bb));
  };
  auto steps_of = [&](int bb) {
    const int l = len_of(bb);
    return l > 0 ? (l + DC_STEP - 1) / DC_STEP : 0;
  };

  int b;
  int64_t before;
  find_batch(p, lane, q0, b, before);
  int nb = steps_of(b);
  int j = (int)((q0 - before) / nb);   // row within the batch
  int ls = (int)((q0 - before) % nb);  // first step within the row

  const int c16 = lane & 15, grp = lane >> 4;
  unsigned char* kt = smem + wave * 2 * L::BYTES;
  unsigned char* vt = kt + L::BYTES;

  // loop-invariant LDS offsets
  const int lrow = lane / L::CPR, lc = lane % L::CPR;  // piece (row, chunk) for loads
  int kwa[L::LOADS], vwa[L::LOADS];
#pragma unroll
  for (int i = 0; i < L::LOADS; ++i) {
    const int row = i * L::RPI + lrow;
    kwa[i] = row * L::RB + ((lc ^ L::kswz(row)) << 4);
    vwa[i] = row * L::RB + ((lc ^ L::vswz(row)) << 4);
  }
  // K operand (kb, dq): row kb*16 + c16, chunk dq*4 + grp -> koff ^ (dq << 6) + kb*16*RB
  const int koff = c16 * L::RB + ((grp ^ L::kswz(c16)) << 4);
  // V^T operand (half h, dd): source row 16h + 4grp + jj/4, column dd*16 + 4*(jj%4)
  const int jj = lane & 15;
  const int vrow = 4 * grp + (jj >> 2);
  const int voff = vrow * L::RB + ((L::vswz(vrow) >> 1) << 5) + (jj & 3) * 8;

  int64_t q = q0;
  while (true) {
    const int len = len_of(b);
    const int kvh = j / p.NG, hg = j % p.NG;
    const int nseg = (int)min((int64_t)(nb - ls), q1 - q);
    const bool whole = ls == 0 && nseg == nb;
    const int kbeg = ls * DC_STEP;
    const int kend = min(len, (ls + nseg) * DC_STEP);

    // ---- K/V of this (batch, kv head).  Keys [0, kend_ld) come from the
    // cache; with an append, key len - 1 is the new one (built in registers),
    // so its cache row is not read.  Keys past the range read as zeros.
    const bool tail = APPEND && kend == len;  // this segment holds the appended key
    const int kend_ld = tail ? kend - 1 : kend;
    const int esz = (int)sizeof(T);
    const T* kbase = reinterpret_cast<const T*>(p.kc) + kvh * p.ksh;
    const T* vbase = reinterpret_cast<const T*>(p.vc) + kvh * p.vsh;
    auto span_bytes = [&](int n, int64_t st) {
      return n > 0 ? (uint32_t)(((int64_t)(n - 1) * st + D) * esz) : 0u;
    };
    __amdgpu_buffer_rsrc_t krs, vrs;
    // paged: block-table entries [wbase, wbase + 64) of this row, one per lane;
    // loaded before everything else so the first K/V loads wait on it alone
    int wbase = 0, win = 0;
    auto load_window = [&](int first) {
      const int npg = (kend + p.page - 1) / p.page;
      wbase = first;
      win = first + lane < npg ? p.bt[b * p.bts + first + lane] : 0;
    };
    if constexpr (PAGED) {
      load_window(kbeg / p.page);
    } else {
      krs = dc_buffer(kbase + b * p.ksb, span_bytes(kend_ld, p.kst));
      vrs = dc_buffer(vbase + b * p.vsb, span_bytes(kend_ld, p.vst));
    }

    // ---- the appended row's operands, in the row layout of norm_row /
    // rope_row: lane `sub` of each group of LPR lanes holds chunks sub and
    // sub + D/16 of the row
    const int sub = lane % LPR;
    floatx8 ka1{}, ka2{}, va1{}, va2{}, kw1{}, kw2{}, kc1{}, ks1{};
    if (tail) {
      const T* ks = reinterpret_cast<const T*>(p.kn) + b * p.knsb + kvh * p.knsh + sub * 8;
      const T* vs = reinterpret_cast<const T*>(p.vn) + b * p.vnsb + kvh * p.vnsh + sub * 8;
      ka1 = Vec8<T>::load_f32(ks);
      ka2 = Vec8<T>::load_f32(ks + D / 2);
      va1 = Vec8<T>::load_f32(vs);
      va2 = Vec8<T>::load_f32(vs + D / 2);
      if (p.kw) {
        kw1 = Vec8<float>::load_f32(p.kw + sub * 8);
        kw2 = Vec8<float>::load_f32(p.kw + D / 2 + sub * 8);
      }
    }

    // ---- query-side loads (before K/V, so waiting for them does not wait for K/V)
    const int gh = hg * 16 + c16;
    const bool hvalid = gh < p.G;
    const int head = kvh * p.G + (hvalid ? gh : 0);
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh;
    // cos/sin of this lane's elements: for D >= 64 the rotate-half partners sit
    // in the same lane (d blocks dq and dq + NDQ/2); for D = 32 (one d block)
    // element d of lanes 0..31 pairs with d + 16 of lanes 32..63
    constexpr int NCS = NDQ >= 2 ? NDQ / 2 : 1;
    floatx8 xf[NDQ], wq[NDQ], cs[NCS], sn[NCS];
#pragma unroll
    for (int dq = 0; dq < NDQ; ++dq) xf[dq] = Vec8<T>::load_f32(qrow + dq * 32 + grp * 8);
    if (p.qw) {
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) wq[dq] = Vec8<float>::load_f32(p.qw + dq * 32 + grp * 8);
    }
    const int pos =
        p.cos_tab ? table_row(p.q_pos ? ld_uniform(p.q_pos, b) : (p.q_pos0 >= 0 ? p.q_pos0 : len - 1), p.max_pos) : 0;
    if (p.cos_tab) {
#pragma unroll
      for (int dq = 0; dq < NCS; ++dq) {
        const int col = NDQ >= 2 ? dq * 32 + grp * 8 : (grp & 1) * 8;
        cs[dq] = load_tab8(p.cos_tab, pos, D / 2, col);
        sn[dq] = load_tab8(p.sin_tab, pos, D / 2, col);
      }
      if (tail) {  // the appended key is rotated at the query's position
        kc1 = load_tab8(p.cos_tab, pos, D / 2, sub * 8);
        ks1 = load_tab8(p.sin_tab, pos, D / 2, sub * 8);
      }
    }

    const int kvo = (int)(lrow * p.kst * esz) + lc * 8 * esz;
    const int vvo = (int)(lrow * p.vst * esz) + lc * 8 * esz;
    const int kstep = (int)(L::RPI * p.kst * esz), vstep = (int)(L::RPI * p.vst * esz);
    typename P8::type kr[L::LOADS], vr[L::LOADS];
    auto load = [&](int k0) {
      int ks, vs;
      if constexpr (PAGED) {
        // a step never crosses a page: page_size is a multiple of DC_STEP
        const int pg = k0 / p.page;
        if (pg - wbase >= 64) load_window(pg);
        const int64_t pid = __builtin_amdgcn_readlane(win, pg - wbase);
        const int rel = k0 - pg * p.page;
        const int nval = min(kend_ld, k0 + DC_STEP) - k0;
        krs = dc_buffer(kbase + pid * p.ksb + (int64_t)rel * p.kst, span_bytes(nval, p.kst));
        vrs = dc_buffer(vbase + pid * p.vsb + (int64_t)rel * p.vst, span_bytes(nval, p.vst));
        ks = vs = 0;
      } else {
        ks = (int)(k0 * p.kst * esz);
        vs = (int)(k0 * p.vst * esz);
      }
#pragma unroll
      for (int i = 0; i < L::LOADS; ++i) {
        kr[i] = P8::load(krs, kvo, ks + i * kstep);
        vr[i] = P8::load(vrs, vvo, vs + i * vstep);
      }
    };
    load(kbeg);

    // ---- the appended key: QK-Norm, then RoPE (the arithmetic of the row
    // kernel, so the cached row matches its K-hat bit for bit), written back
    // by one wave per (batch, kv head); no wave of this launch reads that row
    if (tail) {
      if (p.kw) norm_row<D>(ka1, ka2, kw1, kw2, p.eps);
      if (p.cos_tab) rope_row(ka1, ka2, kc1, ks1);
      if (hg == 0 && lane < LPR) {
        const int t = len - 1;
        int64_t slab = b, row = t;
        if constexpr (PAGED) {
          slab = p.bt[b * p.bts + t / p.page];
          row = t % p.page;
        }
        T* kd = reinterpret_cast<T*>(p.kc) + slab * p.ksb + kvh * p.ksh + row * p.kst + sub * 8;
        T* vd = reinterpret_cast<T*>(p.vc) + slab * p.vsb + kvh * p.vsh + row * p.vst + sub * 8;
        store8<T>(kd, ka1);
        store8<T>(kd + D / 2, ka2);
        store8<T>(vd, va1);
        store8<T>(vd + D / 2, va2);
      }
    }

    // ---- Q operand (B of S^T = K Q^T): lane holds Q[head c16][dq*32 + grp*8 + e]
    bf16x8 qop[NDQ];
    {
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
        for (int dq = 0; dq < NDQ; ++dq)
#pragma unroll
          for (int e = 0; e < 8; ++e) xf[dq][e] = xf[dq][e] * r * wq[dq][e];
      }
      if (p.cos_tab) {
        if constexpr (NDQ >= 2) {
#pragma unroll
          for (int dq = 0; dq < NDQ / 2; ++dq) {
            floatx8 x1 = xf[dq], x2 = xf[dq + NDQ / 2];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              xf[dq][e] = x1[e] * cs[dq][e] - x2[e] * sn[dq][e];
              xf[dq + NDQ / 2][e] = x2[e] * cs[dq][e] + x1[e] * sn[dq][e];
            }
          }
        } else {
          // first half (lanes < 32): x1 c - x2 s; second half: x2 c + x1 s
          const float sg = lane < 32 ? -1.f : 1.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float partner = __shfl_xor(xf[0][e], 32, 64);
            xf[0][e] = xf[0][e] * cs[0][e] + sg * (partner * sn[0][e]);
          }
        }
      }
#pragma unroll
      for (int dq = 0; dq < NDQ; ++dq) qop[dq] = hvalid ? to_bf16x8(xf[dq]) : bf16x8{};
    }

    float m_i = -INFINITY, l_i = 0.f;
    floatx4 oacc[NDO];
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx4{};

    for (int s = 0; s < nseg; ++s) {
      const int k0 = kbeg + s * DC_STEP;
      // registers -> LDS (in-order LDS within the wave: the previous step's
      // reads of this tile have been served before these writes)
#pragma unroll
      for (int i = 0; i < L::LOADS; ++i) {
        *reinterpret_cast<bf16x8*>(kt + kwa[i]) = P8::to_bf16(kr[i]);
        *reinterpret_cast<bf16x8*>(vt + vwa[i]) = P8::to_bf16(vr[i]);
      }
      if (tail && s == nseg - 1 && lane < LPR) {
        // the appended row replaces the zeros loaded for it
        const int rr = len - 1 - k0;
        const int c2 = sub + L::CPR / 2;
        *reinterpret_cast<bf16x8*>(kt + rr * L::RB + ((sub ^ L::kswz(rr)) << 4)) = to_bf16x8(ka1);
        *reinterpret_cast<bf16x8*>(kt + rr * L::RB + ((c2 ^ L::kswz(rr)) << 4)) = to_bf16x8(ka2);
        *reinterpret_cast<bf16x8*>(vt + rr * L::RB + ((sub ^ L::vswz(rr)) << 4)) = to_bf16x8(va1);
        *reinterpret_cast<bf16x8*>(vt + rr * L::RB + ((c2 ^ L::vswz(rr)) << 4)) = to_bf16x8(va2);
      }
      if (s + 1 < nseg) load(k0 + DC_STEP);

      floatx4 sc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sc[kb] = floatx4{};
#pragma unroll
        for (int dq = 0; dq < NDQ; ++dq) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(kt + ((koff ^ (dq << 6)) + kb * 16 * L::RB));
          sc[kb] = mfma16(a, qop[dq], sc[kb]);
        }
      }
      if (k0 + DC_STEP > kend) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + kb * 16 + grp * 4 + i >= kend) sc[kb][i] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][i]);
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      // every step holds at least one key < kend, so m_new is finite
      const float m_new = fmaxf(m_i, mx * p.scale_log2);
      const float alpha = fast_exp2(m_i - m_new);
      floatx8 pf;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pe = fast_exp2(sc[kb][i] * p.scale_log2 - m_new);
          pf[kb * 4 + i] = pe;
          rs += pe;
        }
      const bf16x8 pop = to_bf16x8(pf);
      l_i = l_i * alpha + rs;
      m_i = m_new;
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) {
        oacc[dd] *= alpha;
        const unsigned char* src = vt + (voff ^ (dd << 5));
        const bf16x8 a = lds_read_tr8(reinterpret_cast<const bf16*>(src),
                                      reinterpret_cast<const bf16*>(src + 16 * L::RB));
        oacc[dd] = mfma16(a, pop, oacc[dd]);
      }
    }

    // ---- flush the segment
    l_i += shfl_xor_f(l_i, 16);
    l_i += shfl_xor_f(l_i, 32);
    const int64_t r = ((int64_t)b * p.Hkv + kvh) * p.NG + hg;
    if (lane == 0) {
      if (ls == 0) p.ws_rw[r * 2] = (int32_t)w;
      if (ls + nseg == nb) p.ws_rw[r * 2 + 1] = (int32_t)w;
    }
    if (whole) {
      if (hvalid) {
        T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + (int64_t)(kvh * p.G + gh) * p.osh;
        const float inv = 1.0f / l_i;
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) store4<T>(orow + dd * 16 + grp * 4, oacc[dd] * inv);
      }
    } else {
      const int64_t slot = w + r;
      float* so = p.ws_o + (slot * 16 + c16) * D;
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) *reinterpret_cast<floatx4*>(so + dd * 16 + grp * 4) = oacc[dd];
      if (grp == 0) *reinterpret_cast<floatx2*>(p.ws_ml + (slot * 16 + c16) * 2) = floatx2{m_i, l_i};
    }

    q += nseg;
    if (q >= q1) break;
    ls = 0;
    if (++j == p.rows_per_batch) {
      j = 0;
      do nb = steps_of(++b); while (nb == 0 && b + 1 < p.B);  // q < N: a batch with keys follows
    }
  }
}

// One workgroup per row (batch, kv head, head group): combines the partials
// of the waves that covered the row, or writes zeros for a row without keys.
// Thread t owns head t / 16 of the group and DPT consecutive dims.
template <int D, typename T>
__global__ void __launch_bounds__(DC_THREADS) decode_merge_kernel(DecodeParams p) {
  constexpr int DPT = D / 16;  // dims per thread (8, 4 or 2)
  const int64_t r = blockIdx.x;
  const int b = (int)(r / p.rows_per_batch), j = (int)(r % p.rows_per_batch);
  const int kvh = j / p.NG, hg = j % p.NG;
  const int hq = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * DPT;
  const int gh = hg * 16 + hq;
  // the row's first and last covering wave, read through the scalar path
  // alongside lens[b] (a row without keys never uses them)
  const int64_t wf = ld_uniform(p.ws_rw, r * 2), wl = ld_uniform(p.ws_rw, r * 2 + 1);
  const int len = uniform(batch_len(p, b));
  if (p.lens_out && j == 0 && threadIdx.x == 0) p.lens_out[b] = len < 0 ? p.lens[b] : p.lens[b] + 1;
  T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + (int64_t)(kvh * p.G + (gh < p.G ? gh : 0)) * p.osh + d0;
  if (len <= 0) {  // no keys: zeros; a length out of range: NaN
    if (gh < p.G) {
      const float f = len < 0 ? __builtin_nanf("") : 0.f;
      if constexpr (DPT == 8) store8<T>(orow, floatx8{f, f, f, f, f, f, f, f});
      else if constexpr (DPT == 4) store4<T>(orow, floatx4{f, f, f, f});
      else store2<T>(orow, f, f);
    }
    return;
  }
  if (wf == wl || gh >= p.G) return;  // one wave covered the row and wrote it
  const float* ml = p.ws_ml + ((wf + r) * 16 + hq) * 2;
  const float* po = p.ws_o + ((wf + r) * 16 + hq) * D + d0;
  const int ns = (int)(wl - wf + 1);
  // one pass with a running max, so every partial's (m, l) and outputs are
  // loaded together (every partial holds at least one key: its m is finite)
  float M = -INFINITY, wsum = 0.f;
  float acc[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) acc[e] = 0.f;
#pragma unroll 4
  for (int i = 0; i < ns; ++i) {
    const floatx2 m_l = *reinterpret_cast<const floatx2*>(ml + i * 32);
    float o[DPT];
    if constexpr (DPT == 2) {
      const floatx2 o2 = *reinterpret_cast<const floatx2*>(po + (int64_t)i * 16 * D);
      o[0] = o2[0];
      o[1] = o2[1];
    } else {
#pragma unroll
      for (int e = 0; e < DPT; e += 4) {
        const floatx4 o4 = *reinterpret_cast<const floatx4*>(po + (int64_t)i * 16 * D + e);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[e + k] = o4[k];
      }
    }
    const float Mn = fmaxf(M, m_l[0]);
    const float a = fast_exp2(M - Mn);  // 0 for the first partial
    const float sc = fast_exp2(m_l[0] - Mn);
    wsum = wsum * a + m_l[1] * sc;
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] = acc[e] * a + o[e] * sc;
    M = Mn;
  }
  const float inv = 1.0f / wsum;
  if constexpr (DPT == 8) {
    store8<T>(orow, floatx8{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv,
                            acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv});
  } else if constexpr (DPT == 4) {
    store4<T>(orow, floatx4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv});
  } else {
    store2<T>(orow, acc[0] * inv, acc[1] * inv);
  }
}

static int dc_span(int chunk) { return chunk > 0 ? (chunk + DC_STEP - 1) / DC_STEP : 0; }

// Waves the grid launches (an upper bound of the waves that take steps).
static int64_t dc_waves(int B, int Hkv, int NG, int max_len, int chunk) {
  const int span = dc_span(chunk);
  if (span == 0) return DC_MAX_WAVES;
  const int64_t upper = (int64_t)B * Hkv * NG * ((max_len + DC_STEP - 1) / DC_STEP);
  return ((upper + span - 1) / span + DC_WAVES - 1) / DC_WAVES * DC_WAVES;
}

static int64_t dc_workspace(int B, int Hq, int Hkv, int D, int max_len, int chunk) {
  const int NG = (Hq / Hkv + 15) / 16;
  const int64_t rows = (int64_t)B * Hkv * NG;
  const int64_t slots = dc_waves(B, Hkv, NG, max_len, chunk) + rows;
  return slots * 16 * (D + 2) * (int64_t)sizeof(float) + rows * 2 * (int64_t)sizeof(int32_t);
}

template <int D, typename T, bool PAGED, bool APPEND>
static hipError_t launch_decode(DecodeParams p, hipStream_t st) {
  auto kern = decode_stream_kernel<D, T, PAGED, APPEND>;
  if (p.span == 0) {
    // persistent grid: as many waves as stay resident at once (<= DC_MAX_WAVES),
    // worked out once per device and kernel variant
    static int resident[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int waves = (dev >= 0 && dev < 64) ? __atomic_load_n(&resident[dev], __ATOMIC_RELAXED) : 0;
    if (waves == 0) {
      int cus = 0, per_cu = 0;
      e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), DC_THREADS, 0);
      if (e != hipSuccess) return e;
      const int64_t per = per_cu < 1 ? 1 : (per_cu > DC_WG_PER_CU ? DC_WG_PER_CU : per_cu);
      const int64_t all = (int64_t)cus * per * DC_WAVES;
      waves = (int)(all < DC_MAX_WAVES ? all : DC_MAX_WAVES);
      if (dev >= 0 && dev < 64) __atomic_store_n(&resident[dev], waves, __ATOMIC_RELAXED);
    }
    p.nwaves = waves;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(p.nwaves / DC_WAVES)), dim3(DC_THREADS), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)p.B * p.rows_per_batch;
  hipLaunchKernelGGL((decode_merge_kernel<D, T>), dim3((unsigned)rows), dim3(DC_THREADS), 0, st, p);
  return hipGetLastError();
}

// Checks shared by both entry points, then the parameters that do not
// depend on the cache layout.  Returns NQ_OK or the failure code.
static int decode_setup(DecodeParams& p, const void* q, const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, void* o, const int64_t* o_strides, void* workspace,
                        int64_t workspace_bytes, int B, int Hq, int Hkv, int D, int max_len, int chunk,
                        int dtype, const float* q_weight, float eps, const float* cos_tab,
                        const float* sin_tab, int max_pos, const int32_t* q_pos, int q_pos0, float sm_scale) {
  if (!head_dim_ok(D)) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d max_len=%d)", B, Hq, Hkv, max_len);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  if (!q || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return nq_fail(NQ_ERR_INVALID, "q, caches, o and their strides are required");
  if (!nq_aligned16(q) || !nq_aligned16(o))
    return nq_fail(NQ_ERR_INVALID, "q, o and cache base pointers must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  for (int i = 0; i < 2; ++i)
    if ((q_strides[i] * esz) % 16 || (o_strides[i] * esz) % 16)
      return nq_fail(NQ_ERR_INVALID, "q and o strides must be multiples of 16 bytes");
  for (int i = 0; i < 3; ++i)
    if ((k_strides[i] * esz) % 16 || (v_strides[i] * esz) % 16)
      return nq_fail(NQ_ERR_INVALID, "cache strides must be multiples of 16 bytes");
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  if (k_strides[2] < D || v_strides[2] < D)
    return nq_fail(NQ_ERR_INVALID, "cache rows must not overlap (seq stride >= head_dim)");
  // fp32 caches run the fp32 prefill kernel at S = 1, which keeps no partials:
  // the workspace is neither required nor read there
  const bool f32 = dtype == NQ_DTYPE_F32;
  const int64_t need = dc_workspace(B, Hq, Hkv, D, max_len, chunk);
  if (!f32 && (workspace == nullptr || workspace_bytes < need))
    return nq_fail(NQ_ERR_WORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                   (long long)workspace_bytes);
  p.q = q; p.qsb = q_strides[0]; p.qsh = q_strides[1];
  p.ksb = k_strides[0]; p.ksh = k_strides[1]; p.kst = k_strides[2];
  p.vsb = v_strides[0]; p.vsh = v_strides[1]; p.vst = v_strides[2];
  p.o = o; p.osb = o_strides[0]; p.osh = o_strides[1];
  p.qw = q_weight; p.eps = eps; p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.q_pos = q_pos; p.q_pos0 = q_pos0;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = Hq / Hkv; p.NG = (p.G + 15) / 16;
  p.max_len = max_len;
  p.rows_per_batch = Hkv * p.NG;
  p.span = dc_span(chunk);
  const int64_t nw = dc_waves(B, Hkv, p.NG, max_len, chunk);
  if (nw / DC_WAVES > 0x7fffffff) return nq_fail(NQ_ERR_INVALID, "chunk %d too small for these sizes", chunk);
  p.nwaves = (int)nw;
  if (!f32) {
    p.ws_o = reinterpret_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (nw + (int64_t)B * p.rows_per_batch) * 16 * D;
    p.ws_rw = reinterpret_cast<int32_t*>(p.ws_ml + (nw + (int64_t)B * p.rows_per_batch) * 16 * 2);
  }
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;
  return NQ_OK;
}

// ---------------------------------------------------------------- fp32 caches
// An fp32 cache keeps fp32 arithmetic (the reference's SDPA runs in the input
// dtype): the append, when fused, is its own launch, then the fp32 MFMA
// attention kernel of the prefill runs with S = 1 over each sequence's keys
// (its per-sequence lengths and block table), with the same length, position
// and NaN rules as the bf16 path.  The workspace is not used.

// The new token's K (QK-Normed with kw, rotated at the query's position) and
// V to row lens[b] of the paged cache, and lens_out[b] = lens[b] + 1; a
// sequence whose length is out of range appends nothing and keeps lens[b].
// D/16 lanes per (batch, kv head) row, as the row kernel.
template <int D>
__global__ void __launch_bounds__(256) decode_append_f32_kernel(DecodeParams p) {
  constexpr int LPR = D / 16;
  const int64_t gl = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gl / LPR;  // whole groups of LPR lanes leave together
  const int sub = (int)(gl % LPR);
  if (row >= (int64_t)p.B * p.Hkv) return;
  const int b = (int)(row / p.Hkv), kvh = (int)(row % p.Hkv);
  const int len = batch_len(p, b);
  if (kvh == 0 && sub == 0 && p.lens_out) p.lens_out[b] = len < 0 ? p.lens[b] : p.lens[b] + 1;
  if (len < 0) return;
  const int t = len - 1;  // the new key's row
  const int pos = table_row(p.q_pos ? p.q_pos[b] : (p.q_pos0 >= 0 ? p.q_pos0 : len - 1), p.max_pos);
  const float* kn = reinterpret_cast<const float*>(p.kn) + b * p.knsb + kvh * p.knsh;
  const float* vn = reinterpret_cast<const float*>(p.vn) + b * p.vnsb + kvh * p.vnsh;
  floatx8 x1 = Vec8<float>::load_f32(kn + sub * 8), x2 = Vec8<float>::load_f32(kn + D / 2 + sub * 8);
  floatx8 w1, w2;
  if (p.kw) {
    w1 = Vec8<float>::load_f32(p.kw + sub * 8);
    w2 = Vec8<float>::load_f32(p.kw + D / 2 + sub * 8);
  }
  norm_rope_row<D>(x1, x2, p.kw ? &w1 : nullptr, &w2, p.eps, p.cos_tab, p.sin_tab, pos, sub);
  const int64_t pg = p.bt[b * p.bts + t / p.page];
  float* kd = reinterpret_cast<float*>(p.kc) + pg * p.ksb + kvh * p.ksh + (int64_t)(t % p.page) * p.kst;
  float* vd = reinterpret_cast<float*>(p.vc) + pg * p.vsb + kvh * p.vsh + (int64_t)(t % p.page) * p.vst;
  store8<float>(kd + sub * 8, x1);
  store8<float>(kd + D / 2 + sub * 8, x2);
  store8<float>(vd + sub * 8, Vec8<float>::load_f32(vn + sub * 8));
  store8<float>(vd + D / 2 + sub * 8, Vec8<float>::load_f32(vn + D / 2 + sub * 8));
}

static int decode_launch_f32(const DecodeParams& d, int D, bool paged, bool append, void* stream) {
  if (128 % d.G) return nq_fail(NQ_ERR_UNSUPPORTED, "fp32 decode: GQA group size %d must divide 128", d.G);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (append) {
    const int64_t threads = (int64_t)d.B * d.Hkv * (D / 16);
    const dim3 grid((unsigned)((threads + 255) / 256));
    with_head_dim(D, [&](auto dc) {
      hipLaunchKernelGGL((decode_append_f32_kernel<decltype(dc)::value>), grid, dim3(256), 0, st, d);
      return 0;
    });
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return nq_check_launch(e);
  }
  PrefillParams p{};
  p.q = d.q; p.qsb = d.qsb; p.qsh = d.qsh; p.qss = 0;
  p.k = d.kc; p.ksb = d.ksb; p.ksh = d.ksh; p.kss = d.kst;
  p.v = d.vc; p.vsb = d.vsb; p.vsh = d.vsh; p.vss = d.vst;
  p.o = d.o; p.osb = d.osb; p.osh = d.osh; p.oss = 0;
  p.qw = d.qw; p.eps = d.eps; p.cos_tab = d.cos_tab; p.sin_tab = d.sin_tab; p.max_pos = d.max_pos;
  p.q_pos = d.q_pos;
  // no lens: every sequence holds max_len keys, the query at max_len - 1
  p.q_pos0 = (!d.lens && !d.q_pos && d.q_pos0 < 0) ? d.max_len - 1 : d.q_pos0;
  p.B = d.B; p.Hq = d.Hq; p.Hkv = d.Hkv; p.G = d.G; p.S = 1; p.T = d.max_len;
  p.BM = 128 / d.G; p.nqb = 1;
  p.scale_log2 = d.scale_log2;
  p.kv_lens = d.lens; p.kv_extra = d.append; p.kv_max = d.max_len;
  if (paged) { p.bt = d.bt; p.bts = d.bts; p.page = d.page; }
  const bool fuse = d.qw != nullptr || d.cos_tab != nullptr;
  return nq_check_launch(launch_prefill_f32(p, D, false, fuse, st));
}

template <bool PAGED, bool APPEND>
static int decode_launch(const DecodeParams& p, int D, int dtype, void* stream) {
  if (dtype == NQ_DTYPE_F32) return decode_launch_f32(p, D, PAGED, APPEND, stream);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const hipError_t e =
      with_head_dim(D, [&](auto dc) { return launch_decode<decltype(dc)::value, bf16, PAGED, APPEND>(p, st); });
  return nq_check_launch(e);
}

}  // namespace nq

using namespace nq;

extern "C" int64_t nq_attn_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int max_len, int chunk) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_len <= 0 || Hq % Hkv) return 0;
  return dc_workspace(B, Hq, Hkv, D, max_len, chunk);
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
  DecodeParams p{};
  int rc = decode_setup(p, q, q_strides, k_strides, v_strides, o, o_strides, workspace, workspace_bytes, B, Hq,
                        Hkv, D, max_len, chunk, dtype, q_weight, eps, cos_tab, sin_tab, max_pos, q_pos, q_pos0,
                        sm_scale);
  if (rc != NQ_OK) return rc;
  if (!k_cache || !v_cache) return nq_fail(NQ_ERR_INVALID, "q, caches, o and their strides are required");
  if (!nq_aligned16(k_cache) || !nq_aligned16(v_cache))
    return nq_fail(NQ_ERR_INVALID, "q, o and cache base pointers must be 16-byte aligned");
  // one (batch, kv head) slab of max_len rows is addressed with 32-bit byte offsets
  const int esz = nq_dtype_size(dtype);
  if ((int64_t)max_len * k_strides[2] * esz > 0x7fffffff || (int64_t)max_len * v_strides[2] * esz > 0x7fffffff)
    return nq_fail(NQ_ERR_UNSUPPORTED, "max_len x seq stride exceeds 2 GiB per (batch, kv head)");
  p.kc = const_cast<void*>(k_cache);
  p.vc = const_cast<void*>(v_cache);
  p.lens = lens;
  return decode_launch<false, false>(p, D, dtype, stream);
}

extern "C" int nq_attn_decode_paged_fwd(const void* q, const int64_t* q_strides, const void* k_new,
                                        const int64_t* k_new_strides, const void* v_new,
                                        const int64_t* v_new_strides, const float* k_weight,
                                        void* k_pool, const int64_t* k_pool_strides, void* v_pool,
                                        const int64_t* v_pool_strides, const int32_t* block_table,
                                        int64_t bt_stride, int page_size, const int32_t* lens,
                                        int32_t* lens_out, void* o, const int64_t* o_strides,
                                        void* workspace, int64_t workspace_bytes, int B, int Hq,
                                        int Hkv, int D, int max_len, int chunk, int dtype,
                                        const float* q_weight, float eps, const float* cos_tab,
                                        const float* sin_tab, int max_pos, const int32_t* q_pos,
                                        int q_pos0, float sm_scale, void* stream) {
  nq_clear_error();
  DecodeParams p{};
  int rc = decode_setup(p, q, q_strides, k_pool_strides, v_pool_strides, o, o_strides, workspace,
                        workspace_bytes, B, Hq, Hkv, D, max_len, chunk, dtype, q_weight, eps, cos_tab, sin_tab,
                        max_pos, q_pos, q_pos0, sm_scale);
  if (rc != NQ_OK) return rc;
  if (!k_pool || !v_pool) return nq_fail(NQ_ERR_INVALID, "q, caches, o and their strides are required");
  if (!nq_aligned16(k_pool) || !nq_aligned16(v_pool))
    return nq_fail(NQ_ERR_INVALID, "q, o and cache base pointers must be 16-byte aligned");
  if (!block_table || !lens) return nq_fail(NQ_ERR_INVALID, "a paged cache needs the block table and lens");
  if (page_size <= 0 || page_size % DC_STEP)
    return nq_fail(NQ_ERR_UNSUPPORTED, "page_size must be a positive multiple of %d, got %d", DC_STEP, page_size);
  if (bt_stride < (max_len + page_size - 1) / page_size)
    return nq_fail(NQ_ERR_INVALID, "bt_stride %lld holds fewer than the %d pages of max_len %d",
                   (long long)bt_stride, (max_len + page_size - 1) / page_size, max_len);
  if ((k_new == nullptr) != (v_new == nullptr))
    return nq_fail(NQ_ERR_INVALID, "k_new and v_new go together");
  const int esz = nq_dtype_size(dtype);
  if (k_new) {
    if (!k_new_strides || !v_new_strides)
      return nq_fail(NQ_ERR_INVALID, "k_new and v_new need their strides");
    if (!nq_aligned16(k_new) || !nq_aligned16(v_new))
      return nq_fail(NQ_ERR_INVALID, "k_new and v_new must be 16-byte aligned");
    for (int i = 0; i < 2; ++i)
      if ((k_new_strides[i] * esz) % 16 || (v_new_strides[i] * esz) % 16)
        return nq_fail(NQ_ERR_INVALID, "k_new and v_new strides must be multiples of 16 bytes");
    if (lens_out == lens) return nq_fail(NQ_ERR_INVALID, "lens_out must not alias lens");
  } else if (lens_out) {
    return nq_fail(NQ_ERR_INVALID, "lens_out is written only with an append (k_new/v_new)");
  }
  p.kc = k_pool; p.vc = v_pool;
  p.bt = block_table; p.bts = bt_stride; p.page = page_size;
  p.lens = lens;
  if (k_new) {
    p.append = 1;
    p.kn = k_new; p.knsb = k_new_strides[0]; p.knsh = k_new_strides[1];
    p.vn = v_new; p.vnsb = v_new_strides[0]; p.vnsh = v_new_strides[1];
    p.kw = k_weight;
    p.lens_out = lens_out;
  }
  return p.append ? decode_launch<true, true>(p, D, dtype, stream) : decode_launch<true, false>(p, D, dtype, stream);
}

// ---------------------------------------------------------------- no allocation
// nq_attn_decode_paged_fwd for callers that cannot allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc): the
// workspace is this file-scope device array, one copy per GPU, held until the
// process ends.  In host code `scratch` only names the symbol; its device
// address (one per GPU) comes from hipGetSymbolAddress on the first call on
// each device and is what the kernels receive.  Nothing in the workspace has
// to start at zero: every partial slot and wave index a launch reads, the
// same launch wrote.  Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[NQ_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this GPU's scratch array (resolved once per device, with
// that device current), or null with the error recorded.
void* scratch_address(int* rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = nq_check_launch(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = nq_fail(NQ_ERR_UNSUPPORTED, "device ordinal %d beyond the %d the scratch table holds", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = nq_fail(NQ_ERR_WORKSPACE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int nq_attn_decode_paged_fwd_noalloc(
    const void* q, const int64_t* q_strides, const void* k_new, const int64_t* k_new_strides,
    const void* v_new, const int64_t* v_new_strides, const float* k_weight, void* k_pool,
    const int64_t* k_pool_strides, void* v_pool, const int64_t* v_pool_strides, const int32_t* block_table,
    int64_t bt_stride, int page_size, const int32_t* lens, int32_t* lens_out, void* o,
    const int64_t* o_strides, int B, int Hq, int Hkv, int D, int max_len, int chunk, int dtype,
    const float* q_weight, float eps, const float* cos_tab, const float* sin_tab, int max_pos,
    const int32_t* q_pos, int q_pos0, float sm_scale, void* stream) {
  nq_clear_error();
  if (!head_dim_ok(D)) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128, got %d", D);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0 || Hq % Hkv)
    return nq_fail(NQ_ERR_INVALID, "invalid sizes (B=%d Hq=%d Hkv=%d max_len=%d)", B, Hq, Hkv, max_len);
  // fp32 caches keep no partials (the workspace is unused), so any size is served
  const int64_t need = dtype == NQ_DTYPE_F32 ? 0 : dc_workspace(B, Hq, Hkv, D, max_len, chunk);
  if (need > NQ_DECODE_SCRATCH_BYTES)
    return nq_fail(NQ_ERR_WORKSPACE,
                   "these sizes need %lld bytes of workspace, more than the %lld of the static scratch; "
                   "use nq_attn_decode_paged_fwd with a caller-owned workspace",
                   (long long)need, (long long)NQ_DECODE_SCRATCH_BYTES);
  int rc = NQ_OK;
  void* ws = scratch_address(&rc);
  if (!ws) return rc;
  return nq_attn_decode_paged_fwd(q, q_strides, k_new, k_new_strides, v_new, v_new_strides, k_weight, k_pool,
                                  k_pool_strides, v_pool, v_pool_strides, block_table, bt_stride, page_size, lens,
                                  lens_out, o, o_strides, ws, NQ_DECODE_SCRATCH_BYTES, B, Hq, Hkv, D, max_len,
                                  chunk, dtype, q_weight, eps, cos_tab, sin_tab, max_pos, q_pos, q_pos0, sm_scale,
                                  stream);
}
