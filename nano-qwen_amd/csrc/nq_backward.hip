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
// Two kernels: dQ per query block (the forward's decomposition: a workgroup
// owns the G heads x BM positions of one kv head and walks the key tiles; it
// also forms each row's Delta and stores it with the row's LSE for the next
// kernel); dK/dV per key block (a workgroup owns 128 keys of one kv head and
// walks every query row of its G heads, last query tile first, so the GQA sum
// over heads happens in registers, with no atomics, and the key blocks of a
// pair stream Q / dO through L2 together).
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
// Tiles are double-buffered in LDS: bf16 tiles travel HBM -> LDS with
// global_load_lds (one tile ahead), one barrier per tile; the transpose reads
// are issued as inline asm so that the loads in flight are not waited for.

#include <type_traits>

#include "nq_backward.hpp"
#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {


constexpr int BW_BN = 64;     // keys per tile (dQ kernel)
constexpr int BW_BQ = 32;     // query rows per tile (dK/dV kernel)
constexpr int BW_KEYS = 128;  // keys per dK/dV workgroup (32 per wave)
constexpr int64_t BW_DQ_WIDE_MIN_WGS = 2048;  // 8-wave dQ workgroups needed to prefer them
constexpr int BW_XCD_MIN_BLOCKS = 64;  // blocks per pair from which each XCD takes whole pairs

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

// ---------------------------------------------------------------- scratch
// Index of (batch b, head h, query s) in the scratch: its LSE; Delta is 32 on.

// Stage a tile of NR rows (rows >= nvalid clamp to the last valid row; their
// scores are masked) into LDS, swizzled.  bf16 storage: global_load_lds
// (HBM -> LDS, no registers): instruction m of the tile fills LDS bytes
// [m*1024, m*1024+1024), lane t the 16 bytes at +16t, so the lane loads the
// logical chunk that belongs in that physical slot (the swizzle is an XOR,
// its own inverse).  fp32 storage: loads converted in registers.
template <int D, typename T, int NR, bool TSW, int NW = 4>
__device__ __forceinline__ void bw_tile(unsigned char* tile, const T* src, int64_t rs, int nvalid, int wave,
                                        int lane) {
  using L = BwTile<D>;
  if constexpr (sizeof(T) == 2) {
    constexpr int NI = NR * L::RB / 1024;
    static_assert(NI % NW == 0 || NI < NW, "tile size");
    for (int m = wave; m < NI; m += NW) {
      const int pbyte = m * 1024 + lane * 16;
      const int r = pbyte / L::RB, pc = (pbyte % L::RB) / 16;
      const int lc = TSW ? L::tsw(r, pc) : L::rsw(r, pc);
      const int row = r < nvalid ? r : nvalid - 1;
      global_load_lds16(src + (int64_t)row * rs + lc * 8, tile + m * 1024);
    }
  } else {
    constexpr int CH = NR * L::CPR;
    for (int c = threadIdx.x; c < CH; c += 64 * NW) {
      const int r = c / L::CPR, ch = c % L::CPR;
      const int row = r < nvalid ? r : nvalid - 1;
      const bf16x8 val = to_bf16x8(Vec8<T>::load_f32(src + (int64_t)row * rs + ch * 8));
      const int pc = TSW ? L::tsw(r, ch) : L::rsw(r, ch);
      *reinterpret_cast<bf16x8*>(tile + r * L::RB + pc * 16) = val;
    }
  }
}

// The same staging of a full bf16 tile (all NR rows valid) with buffer loads:
// the tile in a scalar descriptor, the lane's offset in one VGPR and each
// instruction's row step as a scalar offset.  Instruction m = wave + NW*i
// covers rows 4m.. (D = 128; 1024 / (2D) rows per instruction in general):
// the lane's row moves by a multiple of the swizzle period with i, so its
// chunk, and hence its offset, is the same for every i.
template <int D, int NR, bool TSW, int NW = 4>
__device__ __forceinline__ void bw_tile_full(unsigned char* tile, const bf16* src, int64_t rs, int wave,
                                             int lane) {
  using L = BwTile<D>;
  constexpr int NI = NR * L::RB / 1024;
  constexpr int RPI = 1024 / L::RB;
  static_assert(NI % NW == 0 || NI < NW, "tile size");
  if (NI < NW && wave >= NI) return;
  const int r0 = (wave * 1024 + lane * 16) / L::RB, pc = (lane * 16 % L::RB) / 16;
  const int lc = TSW ? L::tsw(r0, pc) : L::rsw(r0, pc);
  const uint32_t rb = (uint32_t)(rs * 2);
  const BufRsrc r = make_rsrc(src, NR * rb);
  const uint32_t off = r0 * rb + lc * 16;
#pragma unroll
  for (int i = 0; i < (NI < NW ? 1 : NI / NW); ++i)
    buffer_load_lds16(r, tile + (wave + NW * i) * 1024, off, i * NW * RPI * rb);
}

// Transpose-read operand: rows r0..r0+3 at `addr`, r0+4..r0+7 four rows on.
template <int D>
__device__ __forceinline__ bf16x8 bw_tr8(const unsigned char* p) {
  return lds_read_tr8_nowait<8 * D>(lds_addr(p));
}

// ---------------------------------------------------------------- dQ
// BIAS: the forward's additive bias (p.bias) enters every score (every tile
// takes the masked path); a row the bias masks entirely has LSE -inf and
// P = 0 (its scratch LSE is stored +inf for the dK/dV kernel).
template <int D, typename T, bool CAUSAL, int NW, bool BIAS = false>
__global__ void __launch_bounds__(64 * NW, 8 / NW) bwd_dq_kernel(BwdParams p) {
  using L = BwTile<D>;
  constexpr int NDB = D / 16, NDO = D / 32;
  constexpr int TB = BW_BN * L::RB;
  // two buffers of (K tile with the transpose swizzle, V tile)
  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * TB];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31, hh = lane >> 5;
  const int npairs = p.B * p.Hkv;
  // workgroup -> (pair, q-block), heaviest q-blocks first.  Dispatch deals
  // workgroups to the 8 XCDs round-robin; when the pairs split evenly over
  // them and each pair has many q-blocks, XCD x works through its own pairs
  // one after another, so a pair's K/V stream stays in that XCD's L2
  // (8B-like shape: HBM fetch 1.97 -> 1.15 GB per launch, time unchanged).
  int qrank, pair;
  if (npairs % 8 == 0 && p.nqb >= BW_XCD_MIN_BLOCKS) {
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
    pair = (k / p.nqb) * 8 + x;
    qrank = k % p.nqb;
  } else {
    qrank = blockIdx.x / npairs;
    pair = blockIdx.x % npairs;
  }
  const int qblk = CAUSAL ? (p.nqb - 1 - qrank) : qrank;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  const int Tk = bw_keys(p, b);  // keys this sequence attends
  const int kv_end = CAUSAL ? min(Tk, q0 + p.BM + p.coff) : Tk;
  const int ntiles = (kv_end + BW_BN - 1) / BW_BN;

  const T* kb0 = reinterpret_cast<const T*>(p.k) + b * p.ksb + kvh * p.ksh;
  const T* vb0 = reinterpret_cast<const T*>(p.v) + b * p.vsb + kvh * p.vsh;
  auto stage = [&](int j, int buf) {
    const int n0 = j * BW_BN;
    if (sizeof(T) == 2 && n0 + BW_BN <= Tk) {
      bw_tile_full<D, BW_BN, true, NW>(smem + buf * 2 * TB, reinterpret_cast<const bf16*>(kb0 + (int64_t)n0 * p.kss),
                                       p.kss, wave, lane);
      bw_tile_full<D, BW_BN, false, NW>(smem + buf * 2 * TB + TB,
                                        reinterpret_cast<const bf16*>(vb0 + (int64_t)n0 * p.vss), p.vss, wave, lane);
      return;
    }
    // rows past the sequence's keys clamp to its last key (masked; padding
    // rows are never read)
    bw_tile<D, T, BW_BN, true, NW>(smem + buf * 2 * TB, kb0 + (int64_t)n0 * p.kss, p.kss, Tk - n0, wave, lane);
    bw_tile<D, T, BW_BN, false, NW>(smem + buf * 2 * TB + TB, vb0 + (int64_t)n0 * p.vss, p.vss, Tk - n0, wave,
                                    lane);
  };
  if (ntiles > 0) stage(0, 0);  // its latency overlaps the Q / dO loads below

  const int R = wave * 32 + r32;
  const int g = R / p.BM, pr = R - g * p.BM;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  // the row's Q and dO (B operands), and Delta = rowsum(dO * O): the two
  // lanes of a row (hh = 0, 1) each hold half of it
  bf16x8 qop[NDB], dop[NDB];
  float dlt;
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qi_c * p.qss;
    const T* drow = reinterpret_cast<const T*>(p.dout) + b * p.dosb + head * p.dosh + (int64_t)qi_c * p.doss;
    const T* orow = reinterpret_cast<const T*>(p.o) + b * p.osb + head * p.osh + (int64_t)qi_c * p.oss;
    float acc = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      qop[db] = to_bf16x8(Vec8<T>::load_f32(qrow + db * 16 + hh * 8));
      const floatx8 d = Vec8<T>::load_f32(drow + db * 16 + hh * 8);
      const floatx8 o = Vec8<T>::load_f32(orow + db * 16 + hh * 8);
      dop[db] = to_bf16x8(d);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(o[e], d[e], acc);
    }
    dlt = xor32_sum(acc);
  }
  float lse2 = p.lse[((int64_t)b * p.Hq + head) * p.S + qi_c] * kLog2e;
  if (BIAS && !(lse2 > -INFINITY)) lse2 = INFINITY;  // no key kept: P = exp2(s - inf) = 0
  // the dK/dV kernel reads both per 32-row tile from the scratch; the
  // workgroup of the last q-block also zeroes its heads' slots past S (the
  // dK/dV kernel's masked rows then see finite values)
  if (qvalid && hh == 0) {
    const int64_t wi = bw_ws_index(p, b, head, qi);
    p.ws[wi] = lse2;
    p.ws[wi + 32] = dlt;
  }
  if (qblk == p.nqb - 1) {
    const int pad = p.nst * 32 - p.S;  // 0..31 slots per head
    for (int t = threadIdx.x; t < p.G * 32; t += 64 * NW) {
      const int g2 = t / 32, s2 = p.S + t % 32;
      if (t % 32 < pad) {
        const int64_t w2 = bw_ws_index(p, b, kvh * p.G + g2, s2);
        p.ws[w2] = 0.f;
        p.ws[w2 + 32] = 0.f;
      }
    }
  }

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
  // last key this row sees (rows past S see none)
  const int lim = !qvalid ? -1 : (CAUSAL ? min(qi + p.coff, Tk - 1) : Tk - 1);

  for (int j = 0; j < ntiles; ++j) {
    const int n0 = j * BW_BN;
    // tile j has landed (each wave waits for its own loads, the barrier for
    // everyone's); every wave is done with tile j-1, whose buffer is refilled
    if constexpr (sizeof(T) == 2) wait_vmcnt0();
    __syncthreads();
    if (j + 1 < ntiles) stage(j + 1, (j + 1) & 1);
    const unsigned char* Kt = smem + (j & 1) * 2 * TB;
    const uint32_t ka = lds_addr(Kt);  // the V tile is TB bytes on
    // a tile inside every row's bounds (all keys below T and at or before
    // the block's first query's frontier, no rows past S) skips the mask
    const bool full = !BIAS && n0 + BW_BN <= Tk && q0 + p.BM <= p.S && (!CAUSAL || n0 + BW_BN - 1 <= q0 + p.coff);
    // the two 32-key blocks of the tile (kb a compile-time constant, so its
    // LDS offset goes into the read instructions)
    auto key_block = [&](auto KB) {
      constexpr int kb = decltype(KB)::value;
      // S^T and dP^T over the d chunks, the next chunk's K and V reads in
      // flight behind the current chunk's two MFMAs
      floatx16 s = floatx16{}, dp = floatx16{};
      bf16x8 ak[2], av[2];
      auto rd_sdp = [&](int db, int slot) {
        ak[slot] = lds_read_b128_nowait<kb * 32 * L::RB>(ka + kro[db]);
        av[slot] = lds_read_b128_nowait<TB + kb * 32 * L::RB>(ka + vro[db]);
      };
      rd_sdp(0, 0);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        if (db + 1 < NDB) {
          rd_sdp(db + 1, (db + 1) & 1);
          lgkm_wait<2>();
        } else {
          lgkm_wait<0>();
        }
        s = mfma32(ak[db & 1], qop[db], s);
        dp = mfma32(av[db & 1], dop[db], dp);
      }
      bf16x8 bds[2];
      auto grads = [&](auto masked) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          floatx8 ds;
          // the bias of the lane's 8 keys n0 + kb*32 + ks*16 + hh*8 + 0..7
          bf16x8 bv{};
          if constexpr (BIAS) {
            const int k8 = n0 + kb * 32 + ks * 16 + hh * 8;
            if (k8 < Tk)
              bv = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.bias) + b * p.bsb +
                                                    head * p.bsh + (int64_t)qi_c * p.bss + k8);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = ks * 8 + e;
            float x = __builtin_fmaf(s[i], p.scale_log2, -lse2);
            if constexpr (BIAS) x = __builtin_fmaf((float)bv[e], kLog2e, x);
            if constexpr (decltype(masked)::value) {
              // masked: exp2(-inf) = 0, selected before the exp (no branch around it)
              const int key = n0 + kb * 32 + bw_cidx(i, hh);
              x = key <= lim ? x : -INFINITY;
            }
            ds[e] = fast_exp2(x) * (dp[i] - dlt);
          }
          bds[ks] = to_bf16x8(ds);
        }
      };
      if (full)
        grads(std::false_type{});
      else
        grads(std::true_type{});
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 akt[NDO];
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) akt[dd] = bw_tr8<D>(Kt + kto[dd] + (kb * 32 + ks * 16) * L::RB);
        lgkm_wait<0>();
#pragma unroll
        for (int dd = 0; dd < NDO; ++dd) dqacc[dd] = mfma32(akt[dd], bds[ks], dqacc[dd]);
      }
    };
    key_block(std::integral_constant<int, 0>{});
    key_block(std::integral_constant<int, 1>{});
  }

  if (!qvalid) return;
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
// D = 64 fits three workgroups per CU (168 VGPRs), D = 128 two
template <int D, typename T, bool CAUSAL, bool BIAS = false>
__global__ void __launch_bounds__(256, D == 64 ? 3 : 2) bwd_dkdv_kernel(BwdParams p) {
  using L = BwTile<D>;
  constexpr int NDB = D / 16, NDO = D / 32;
  constexpr int TB = BW_BQ * L::RB;
  constexpr int BUF = 2 * TB + 2 * BW_BQ * 4;  // Q tile, dO tile, LSE*log2e, Delta
  constexpr int VB = BW_KEYS * L::RB;          // the block's V rows (B operand of dP)
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * BUF + VB];
  unsigned char* Vs = smem + 2 * BUF;

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31, hh = lane >> 5;
  // key blocks in launch order: under the causal mask the first keys see the
  // most queries, so the heaviest blocks start first.  Dispatch deals
  // workgroups to the 8 XCDs round-robin.  When the pairs split evenly over
  // the XCDs and each has many key blocks, XCD x works through its own pairs
  // one at a time, so the blocks of one pair are co-resident and walk the
  // query tiles together, sharing its L2 for the Q / dO stream (8B-like
  // shape: HBM fetch 7.3 -> 3.7 GB per launch, time unchanged).  Otherwise
  // consecutive blocks are different pairs, heaviest blocks of every pair
  // first; with a pair count that is a multiple of 8 a pair's blocks still
  // land on one XCD.
  const int npairs = p.B * p.Hkv;
  int kblk, pair;
  const int nkb = gridDim.x / npairs;
  if (npairs % 8 == 0 && nkb >= BW_XCD_MIN_BLOCKS) {
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
    pair = (k / nkb) * 8 + x;
    kblk = k % nkb;
  } else {
    kblk = blockIdx.x / npairs;
    pair = blockIdx.x % npairs;
  }
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int k0 = kblk * BW_KEYS;
  const int key = k0 + wave * 32 + r32;  // this lane's key (C column)
  const int Tk = bw_keys(p, b);  // keys past Tk are padding: zero gradients, rows never read
  const int key_c = key < Tk ? key : k0;  // a padded key's K row: the block's first (read only if < Tk)

  // the work list: (query tile qt, head g) for queries that see a key of this
  // block (q + coff >= k0); none when the whole block is padding
  const int qstart = CAUSAL ? max(0, k0 - p.coff) / BW_BQ * BW_BQ : 0;
  const int nqt = (qstart < p.S && k0 < Tk) ? (p.S - qstart + BW_BQ - 1) / BW_BQ : 0;
  const int niter = p.G * nqt;
  // bf16 Q / dO tiles: this wave's DMA instruction i fills LDS bytes
  // [(wave + 4i) * 1024, +1024), the lane's 16 bytes lying in tile row
  // dr0 + i * DSTEP at the same swizzled chunk for every i (the swizzle
  // repeats every 4 * 1024 bytes), so two lane constants cover the tile
  // (a D = 32 tile is 2 KiB: waves 0 and 1 issue one instruction each)
  constexpr int NI = BW_BQ * L::RB / 1024;  // load instructions per tile
  constexpr int NPW = NI >= 4 ? NI / 4 : 1;
  constexpr int DSTEP = 4 * 1024 / L::RB;
  static_assert(NI % 4 == 0 || NI < 4, "tile size");
  const int dr0 = (wave * 1024 + lane * 16) / L::RB;
  const int dlc = L::tsw(dr0, (lane * 16 % L::RB) / 16) * 8;
  // stage the (head g, query tile qt) step into buffer buf
  auto stage = [&](int g, int qt, int buf) {
    const int head = kvh * p.G + g;
    unsigned char* base = smem + buf * BUF;
    const T* qsrc = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qt * p.qss;
    const T* dsrc = reinterpret_cast<const T*>(p.dout) + b * p.dosb + head * p.dosh + (int64_t)qt * p.doss;
    if constexpr (sizeof(T) == 2) {
      // (per-instruction addresses even for full tiles: the buffer-descriptor
      // form of the dQ kernel raised this kernel's HBM fetch at the 8B-like
      // shape from 3.65 to 5.45 GB per launch, at equal time)
      const int last = p.S - qt - 1;  // rows past S clamp to the last row (masked)
#pragma unroll
      for (int i = 0; i < NPW; ++i) {
        if (NI < 4 && wave >= NI) break;
        const int row = min(dr0 + i * DSTEP, last);
        global_load_lds16(qsrc + (int64_t)row * p.qss + dlc, base + (wave + 4 * i) * 1024);
        global_load_lds16(dsrc + (int64_t)row * p.doss + dlc, base + TB + (wave + 4 * i) * 1024);
      }
    } else {
      bw_tile<D, T, BW_BQ, true>(base, qsrc, p.qss, p.S - qt, wave, lane);
      bw_tile<D, T, BW_BQ, true>(base + TB, dsrc, p.doss, p.S - qt, wave, lane);
    }
    // LSE (log2 units) and Delta of the tile's 32 rows: 256 contiguous bytes
    // of the scratch, one 16-byte piece per lane of the last wave's first 16
    if (wave == 3 && lane < 16)
      global_load_lds16(p.ws + bw_ws_index(p, b, head, qt) + lane * 4, base + 2 * TB);
  };
  // Steps run query tile by query tile from the LAST tile down to qstart, the
  // G heads of a tile back to back.  Every key block of a pair then starts at
  // the same tile and walks down in step with the others (they only differ in
  // where they stop), so the workgroups of one pair that are resident on an
  // XCD read each Q / dO tile at about the same time and share it in L2,
  // instead of streaming windows of the pair offset by their key blocks.
  auto advance = [&](int& g, int& qt) {
    if (++g == p.G) {
      g = 0;
      qt -= BW_BQ;
    }
  };
  const int qtop = qstart + (nqt - 1) * BW_BQ;  // the last query tile
  int gn = 0, qtn = qtop;  // the next step to stage
  // V of the block's keys stays in LDS (read as the B operand of dP each
  // step); K of the lane's key is held in registers (B operand of S).  Both
  // stagings are waited for at the top of the first iteration (a workgroup
  // without work issues none, so none is left in flight at exit).
  if (niter > 0) {
    bw_tile<D, T, BW_KEYS, false>(Vs, reinterpret_cast<const T*>(p.v) + b * p.vsb + kvh * p.vsh + (int64_t)k0 * p.vss,
                                  p.vss, Tk - k0, wave, lane);
    stage(gn, qtn, 0);
    advance(gn, qtn);
  }

  bf16x8 kop[NDB];
  {
    const T* krow = reinterpret_cast<const T*>(p.k) + b * p.ksb + kvh * p.ksh + (int64_t)key_c * p.kss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) kop[db] = to_bf16x8(Vec8<T>::load_f32(krow + db * 16 + hh * 8));
  }
  // V row of the lane's key in the block tile, chunk (2 db + hh) swizzled
  const int vrow_l = wave * 32 + r32;
  const int vrow_o = vrow_l * L::RB;
  const int prow = bw_perm32(r32);
  // Q / dO rows as the A operand of S^T / dP^T: chunk 2 db + hh of row
  // prow.  The swizzle XORs chunk bits 2 and up, so chunks 4m + hh and
  // 4m + 2 + hh lie 32 bytes apart: one offset per d-chunk pair
  int rro[NDB / 2];
#pragma unroll
  for (int m = 0; m < NDB / 2; ++m) rro[m] = prow * L::RB + L::tsw(prow, 4 * m + hh) * 16;
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

  int gcur = 0, qnext = qtop;
  for (int it = 0; it < niter; ++it) {
    const int qt = qnext;  // this step's query tile
    const int gstep = gcur;  // and head
    (void)gstep;
    advance(gcur, qnext);
    wait_vmcnt0();  // the LSE / Delta rows always come through global_load_lds
    __syncthreads();
    if (it + 1 < niter) {
      stage(gn, qtn, (it + 1) & 1);
      advance(gn, qtn);
    }
    // a wave whose keys all lie past T, or (causal) after every query of the
    // step, has P = 0 there: nothing to add
    const int kw0 = k0 + wave * 32;
    if (kw0 >= Tk || (CAUSAL && kw0 > qt + BW_BQ - 1 + p.coff)) continue;
    const unsigned char* Qt = smem + (it & 1) * BUF;
    const unsigned char* Dt = Qt + TB;
    const float* lse_t = reinterpret_cast<const float*>(Qt + 2 * TB);
    const float* dlt_t = lse_t + BW_BQ;
    // S^T and dP^T over the d chunks, the next chunk's three reads (Q, dO, V)
    // in flight behind the current chunk's two MFMAs
    const uint32_t qa = lds_addr(Qt), va = lds_addr(Vs) + vrow_o;
    floatx16 s = floatx16{}, dp = floatx16{};
    bf16x8 aq[2], ad[2], bv[2];
    auto rd_sdp = [&](int db, int slot) {
      if (db & 1) {
        aq[slot] = lds_read_b128_nowait<32>(qa + rro[db / 2]);
        ad[slot] = lds_read_b128_nowait<TB + 32>(qa + rro[db / 2]);
      } else {
        aq[slot] = lds_read_b128_nowait<0>(qa + rro[db / 2]);
        ad[slot] = lds_read_b128_nowait<TB>(qa + rro[db / 2]);
      }
      bv[slot] = lds_read_b128_nowait<0>(va + L::rsw(vrow_l, 2 * db + hh) * 16);
    };
    rd_sdp(0, 0);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      if (db + 1 < NDB) {
        rd_sdp(db + 1, (db + 1) & 1);
        lgkm_wait<3>();
      } else {
        lgkm_wait<0>();
      }
      s = mfma32(aq[db & 1], kop[db], s);
      dp = mfma32(ad[db & 1], bv[db & 1], dp);
    }
    // this lane's 16 query rows: hh*8 + 0..7 and 16 + hh*8 + 0..7, four at a
    // time; P and dS go to bf16 (the B operands below) as soon as they exist.
    // A step whose 32 x 32 (key, query) square lies inside every bound skips
    // the per-element mask (a wave-uniform test).
    bf16x8 bpv[2], bdsv[2];
    auto probs = [&](auto masked) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        floatx8 pv, ds;
#pragma unroll
        for (int i4h = 0; i4h < 2; ++i4h) {
          const int r0 = ks * 16 + hh * 8 + i4h * 4;
          const floatx4 lv = *reinterpret_cast<const floatx4*>(lse_t + r0);
          const floatx4 dv4 = *reinterpret_cast<const floatx4*>(dlt_t + r0);
          // the transposed bias of this key for queries qt + r0 + 0..3
          bf16x4 bv{};
          if constexpr (BIAS) {
            if (key < Tk && qt + r0 < p.S)
              bv = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16*>(p.bias_t) + b * p.btsb +
                                                    (kvh * p.G + gstep) * p.btsh + (int64_t)key * p.btss + qt + r0);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int i = ks * 8 + i4h * 4 + u;
            float x = __builtin_fmaf(s[i], p.scale_log2, -lv[u]);
            if constexpr (BIAS) x = __builtin_fmaf((float)bv[u], kLog2e, x);
            if constexpr (decltype(masked)::value) {
              // masked: exp2(-inf) = 0, selected before the exp (no branch around it)
              const int q = qt + r0 + u;
              const bool keep = key < Tk && q < p.S && (!CAUSAL || key <= q + p.coff);
              x = keep ? x : -INFINITY;
            }
            const float pe = fast_exp2(x);
            pv[i4h * 4 + u] = pe;
            ds[i4h * 4 + u] = pe * (dp[i] - dv4[u]);
          }
        }
        bpv[ks] = to_bf16x8(pv);
        bdsv[ks] = to_bf16x8(ds);
      }
    };
    const int kw1 = kw0 + 31;  // the wave's last key
    if (!BIAS && kw1 < Tk && qt + BW_BQ <= p.S && (!CAUSAL || kw1 <= qt + p.coff))
      probs(std::false_type{});
    else
      probs(std::true_type{});
    // dV += dO^T P^T and dK += Q^T dS^T, one (16-query step ks, 32-wide d
    // block dd) at a time, the next pair's transpose reads in flight
    bf16x8 td[2], tq[2];
    auto rd_t = [&](int t, int slot) {
      const int ks = t / NDO, dd = t % NDO;
      td[slot] = bw_tr8<D>(Dt + tro[dd] + ks * 16 * L::RB);
      tq[slot] = bw_tr8<D>(Qt + tro[dd] + ks * 16 * L::RB);
    };
    rd_t(0, 0);
#pragma unroll
    for (int t = 0; t < 2 * NDO; ++t) {
      if (t + 1 < 2 * NDO) {
        rd_t(t + 1, (t + 1) & 1);
        lgkm_wait<4>();
      } else {
        lgkm_wait<0>();
      }
      const int ks = t / NDO, dd = t % NDO;
      dvacc[dd] = mfma32(td[t & 1], bpv[ks], dvacc[dd]);
      dkacc[dd] = mfma32(tq[t & 1], bdsv[ks], dkacc[dd]);
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
static hipError_t launch_bwd(const BwdParams& p, int nw, bool causal, hipStream_t st) {
  const dim3 gq((unsigned)(p.nqb * p.B * p.Hkv));
  const dim3 gk((unsigned)(((p.T + BW_KEYS - 1) / BW_KEYS) * p.B * p.Hkv));
  const dim3 bq(64 * nw);
  if (p.bias) {  // 4-wave dQ workgroups
    if (nw != 4) return hipErrorInvalidValue;
    if (causal) {
      hipLaunchKernelGGL((bwd_dq_kernel<D, T, true, 4, true>), gq, bq, 0, st, p);
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, true, true>), gk, dim3(256), 0, st, p);
    } else {
      hipLaunchKernelGGL((bwd_dq_kernel<D, T, false, 4, true>), gq, bq, 0, st, p);
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, false, true>), gk, dim3(256), 0, st, p);
    }
    return hipGetLastError();
  }
  if (causal) {
    if (nw == 8) hipLaunchKernelGGL((bwd_dq_kernel<D, T, true, 8>), gq, bq, 0, st, p);
    else hipLaunchKernelGGL((bwd_dq_kernel<D, T, true, 4>), gq, bq, 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, true>), gk, dim3(256), 0, st, p);
  } else {
    if (nw == 8) hipLaunchKernelGGL((bwd_dq_kernel<D, T, false, 8>), gq, bq, 0, st, p);
    else hipLaunchKernelGGL((bwd_dq_kernel<D, T, false, 4>), gq, bq, 0, st, p);
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, T, false>), gk, dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- QK-Norm + RoPE backward
// y = rope(x * r * w), r = rsqrt(mean(x^2) + eps).  With g = rope^T(dy) (the
// rotation by -theta): dw += g * x * r (summed over rows), and with
// u = g * w: dx = r * u - x * (r^3 / D) * sum(u * x).  Rows are held as in
// the forward row kernel (D/16 lanes, a lane owns 8 elements and their
// rotate-half partners).  dw is accumulated per block in LDS and each block
// stores its partial sum in the workspace; a second launch adds the partials
// in block order, so dw is the same bit for bit on every run (no atomics).
struct NormBwdParams {
  const void* x;
  int64_t xsb, xsh, xss;
  const void* dy;
  int64_t ysb, ysh, yss;
  void* dx;
  int64_t dsb, dsh, dss;
  const float* w;
  float* dw;
  float* ws;  // per-block partial dw, gridDim.x x D
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
      const int ps = table_row(row_position(p.pos, p.pos_base, p.pos0, b, s, p.S), p.max_pos);
      const floatx8 c = load_tab8(p.cos_tab, ps, D / 2, sub * 8);
      const floatx8 sn = load_tab8(p.sin_tab, ps, D / 2, sub * 8);
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
    p.ws[(int64_t)blockIdx.x * D + d] = t;
  }
}

// dw[d] = sum of the nblk partials in block order: 256 threads, thread t adds
// blocks t / D, t / D + 256 / D, ... of column t % D, then the 256 / D column
// sums are added in thread order.
template <int D>
__global__ __launch_bounds__(256) void norm_dw_reduce_kernel(const float* ws, int nblk, float* dw) {
  constexpr int LANES = 256 / D;
  __shared__ float part[LANES][D];
  const int d = threadIdx.x % D, l = threadIdx.x / D;
  float t = 0.f;
  for (int i = l; i < nblk; i += LANES) t += ws[(int64_t)i * D + d];
  part[l][d] = t;
  __syncthreads();
  if (l == 0) {
    float s = 0.f;
    for (int i = 0; i < LANES; ++i) s += part[i][d];
    dw[d] = s;
  }
}

}  // namespace nq

using namespace nq;

extern "C" int64_t nq_attn_bwd_workspace_bytes(int B, int Hq, int S) {
  if (B <= 0 || Hq <= 0 || S <= 0) return 0;
  return (int64_t)B * Hq * ((S + 31) / 32) * 64 * (int64_t)sizeof(float);
}

// Shared by nq_attn_bwd and nq_attn_bwd_bias (bias == NULL: none).
static int bwd_entry(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                     const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                     const void* dout, const int64_t* do_strides, const float* lse, const int32_t* key_lens,
                     const void* bias, const int64_t* bias_strides, const void* bias_t,
                     const int64_t* bias_t_strides, void* dq, const int64_t* dq_strides, void* dk,
                     const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* workspace,
                     int64_t workspace_bytes, int B, int Hq, int Hkv, int S, int T, int D, int dtype, int causal,
                     float sm_scale, void* stream) {
  // head_dim 256 (kernels/flash_attn.py:106): the gradient of the plain bf16 forward
  const bool wide = D == 256;
  if (wide && (dtype != NQ_DTYPE_BF16 || bias || key_lens))
    return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim 256 takes bf16 tensors without key lengths or bias");
  if (!wide && !head_dim_ok(D))
    return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || T <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d S=%d T=%d)", B, Hq, Hkv, S, T);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  const int G = Hq / Hkv;
  if (!wide && 128 % G)
    return nq_fail(NQ_ERR_UNSUPPORTED, "the backward needs 128 %% (Hq/Hkv) == 0, got G=%d", G);
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
  // the dK/dV kernel addresses a 32-row query tile with 32-bit lane offsets
  for (const int64_t rs : {q_strides[2], do_strides[2]})
    if (rs < 0 || rs * esz * 32 >= (int64_t(1) << 31))
      return nq_fail(NQ_ERR_UNSUPPORTED, "q and dout position strides must lie in [0, 2^26 / element size)");
  // the dQ kernel stages 64-key K/V tiles through a buffer descriptor whose
  // range and lane offsets are 32-bit (as the prefill's tiles)
  for (const int64_t rs : {k_strides[2], v_strides[2]})
    if (rs < 0 || rs * esz * BW_BN >= (int64_t(1) << 31))
      return nq_fail(NQ_ERR_UNSUPPORTED, "k/v sequence stride %lld too large", (long long)rs);
  if (!lse) return nq_fail(NQ_ERR_INVALID, "the forward's LSE is required");
  if (bias) {
    if (!bias_strides || !bias_t || !bias_t_strides)
      return nq_fail(NQ_ERR_INVALID, "the bias needs its strides and its transpose");
    for (const int64_t* bs : {bias_strides, bias_t_strides})
      for (int a = 0; a < 3; ++a)
        if (bs[a] < 0 || bs[a] % 8)
          return nq_fail(NQ_ERR_INVALID, "bias strides must be non-negative multiples of 8 elements");
    if (!nq_aligned16(bias) || !nq_aligned16(bias_t))
      return nq_fail(NQ_ERR_INVALID, "the bias and its transpose must be 16-byte aligned");
  }
  const int64_t need = nq_attn_bwd_workspace_bytes(B, Hq, S);
  if (!workspace || workspace_bytes < need)
    return nq_fail(NQ_ERR_WORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                   (long long)workspace_bytes);
  BwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.lse = lse;
  p.ws = reinterpret_cast<float*>(workspace);
  p.nst = (S + 31) / 32;
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
  p.kv_lens = key_lens;
  p.bias = bias;
  p.bias_t = bias_t;
  if (bias) {
    p.bsb = bias_strides[0]; p.bsh = bias_strides[1]; p.bss = bias_strides[2];
    p.btsb = bias_t_strides[0]; p.btsh = bias_t_strides[1]; p.btss = bias_t_strides[2];
  }
  // dQ workgroups: 8 waves (256 query rows: each K/V tile load serves twice
  // the rows) when that still gives enough workgroups to fill the device
  const int64_t wide_wgs = (int64_t)B * Hkv * ((S + 256 / G - 1) / (256 / G));
  const bool f32 = dtype == NQ_DTYPE_F32;  // fp32 tensors: the fp32 MFMA kernels (4 waves)
  const int nw = (!f32 && !bias && wide_wgs >= BW_DQ_WIDE_MIN_WGS) ? 8 : 4;
  p.BM = 32 * nw / G;
  p.nqb = (S + p.BM - 1) / p.BM;
  p.coff = T - S;
  p.scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = p.scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (wide) {
    p.nqb = (S + 63) / 64;
    if ((int64_t)p.nqb * B * Hq >= (1LL << 31) || (int64_t)((T + 63) / 64) * B * Hkv >= (1LL << 31))
      return nq_fail(NQ_ERR_UNSUPPORTED, "too many blocks for one launch");
    return nq_check_launch(launch_bwd_wide(p, causal != 0, st));
  }
  if (f32) return nq_check_launch(launch_bwd_f32(p, D, causal != 0, st));
  const hipError_t e =
      with_head_dim(D, [&](auto dc) { return launch_bwd<decltype(dc)::value, bf16>(p, nw, causal != 0, st); });
  return nq_check_launch(e);
}

extern "C" int nq_attn_bwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                           const void* dout, const int64_t* do_strides, const float* lse,
                           const int32_t* key_lens, void* dq,
                           const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                           const int64_t* dv_strides, void* workspace, int64_t workspace_bytes, int B, int Hq,
                           int Hkv, int S, int T, int D, int dtype, int causal, float sm_scale, void* stream) {
  nq_clear_error();
  return bwd_entry(q, q_strides, k, k_strides, v, v_strides, o, o_strides, dout, do_strides, lse, key_lens, nullptr,
                   nullptr, nullptr, nullptr, dq, dq_strides, dk, dk_strides, dv, dv_strides, workspace,
                   workspace_bytes, B, Hq, Hkv, S, T, D, dtype, causal, sm_scale, stream);
}

extern "C" int nq_attn_bwd_bias(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                                const void* dout, const int64_t* do_strides, const float* lse,
                                const int32_t* key_lens, const void* bias, const int64_t* bias_strides,
                                const void* bias_t, const int64_t* bias_t_strides, void* dq,
                                const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                                const int64_t* dv_strides, void* workspace, int64_t workspace_bytes, int B,
                                int Hq, int Hkv, int S, int T, int D, int dtype, int causal, float sm_scale,
                                void* stream) {
  nq_clear_error();
  if (!bias) return nq_fail(NQ_ERR_INVALID, "nq_attn_bwd_bias needs the bias");
  return bwd_entry(q, q_strides, k, k_strides, v, v_strides, o, o_strides, dout, do_strides, lse, key_lens, bias,
                   bias_strides, bias_t, bias_t_strides, dq, dq_strides, dk, dk_strides, dv, dv_strides, workspace,
                   workspace_bytes, B, Hq, Hkv, S, T, D, dtype, causal, sm_scale, stream);
}

// Blocks of the QK-Norm + RoPE backward (one per 256 / (D/16) rows, at most 1024).
static int64_t norm_bwd_blocks(int B, int S, int H, int D) {
  const int64_t rows = (int64_t)B * H * S;
  const int rpb = 256 / (D / 16);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  return blocks < 1024 ? blocks : 1024;
}

extern "C" int64_t nq_qk_norm_rope_bwd_workspace_bytes(int B, int S, int H, int D) {
  if (B <= 0 || S <= 0 || H <= 0 || !head_dim_ok(D)) return 0;
  return norm_bwd_blocks(B, S, H, D) * D * (int64_t)sizeof(float);
}

extern "C" int nq_qk_norm_rope_bwd(const void* x, const int64_t* x_strides, const void* dy,
                                   const int64_t* dy_strides, void* dx, const int64_t* dx_strides,
                                   const float* weight, float* dweight, void* workspace, int64_t workspace_bytes,
                                   int B, int S, int H, int D, int dtype,
                                   float eps, const float* cos_tab, const float* sin_tab, int max_pos,
                                   const int32_t* pos, const int32_t* pos_base, int pos0, void* stream) {
  nq_clear_error();
  if (!head_dim_ok(D)) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || S <= 0 || H <= 0) return nq_fail(NQ_ERR_INVALID, "sizes must be positive");
  if (!x || !dy || !dx || !x_strides || !dy_strides || !dx_strides)
    return nq_fail(NQ_ERR_INVALID, "x, dy, dx and their strides are required");
  if ((weight == nullptr) != (dweight == nullptr))
    return nq_fail(NQ_ERR_INVALID, "weight and dweight go together");
  if (weight) {
    const int64_t need = nq_qk_norm_rope_bwd_workspace_bytes(B, S, H, D);
    if (!workspace || workspace_bytes < need)
      return nq_fail(NQ_ERR_WORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                     (long long)workspace_bytes);
  }
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
  p.w = weight; p.dw = dweight; p.ws = reinterpret_cast<float*>(workspace);
  p.B = B; p.H = H; p.S = S; p.eps = eps;
  p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.pos = pos; p.pos_base = pos_base; p.pos0 = pos0;
  const int nblk = (int)norm_bwd_blocks(B, S, H, D);
  const dim3 grid((unsigned)nblk);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  with_head_dim(D, [&](auto dc) {
    constexpr int DD = decltype(dc)::value;
    if (dtype == NQ_DTYPE_BF16) hipLaunchKernelGGL((norm_rope_bwd_kernel<bf16, DD>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((norm_rope_bwd_kernel<float, DD>), grid, dim3(256), 0, st, p);
    if (weight) hipLaunchKernelGGL((norm_dw_reduce_kernel<DD>), dim3(1), dim3(256), 0, st, p.ws, nblk, dweight);
    return 0;
  });
  return nq_check_launch(hipGetLastError());
}
