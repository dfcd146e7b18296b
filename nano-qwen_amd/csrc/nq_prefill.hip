// Causal / full GQA prefill attention for gfx950 (FlashAttention-2 forward).
//
// Replaces kernels/flash_attn.py:28-143 and the SDPA call of
// model/attention.py:105-115; QK-Norm + RoPE of Q (attention.py:95-100) are
// fused into the Q load.
//
// Work decomposition
//   A workgroup of NW waves owns 32*NW query rows that all read the same kv
//   head: the G = Hq/Hkv query heads of one GQA group times BM = 32*NW/G
//   consecutive positions.  Every K/V tile it stages in LDS is therefore used
//   by all G heads (the repeat_interleave of attention.py:106-108 never
//   materialises).  All rows share one causal frontier, so the whole
//   workgroup walks the same key range.  NW = 8 (256 rows, one workgroup per
//   CU) halves the HBM/L2 -> LDS bytes per FLOP and the load instructions per
//   wave against NW = 4 (each one stalls its wave for tens of clocks while the
//   CU's load path, about 64 bytes per clock, drains); launches that would
//   have fewer than PF_WIDE_MIN_WGS such workgroups use NW = 4 (two per CU),
//   whose smaller causal q-blocks balance the tail better.
//
// Per wave: 32 query rows.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_bf16 (A = K tile from LDS, B = Q from registers).  In
// the result each lane owns one query column and 16 of its 32 keys, so the
// row max / row sum of the online softmax need no cross-lane traffic except a
// single xor-32 exchange.  The output is kept transposed too,
// O^T += V^T P^T, so the per-row rescale applies lane-locally.  K rows enter
// MFMA rows through a bit permutation (swap bits 2 and 3 of the row index)
// chosen so each lane's 8 consecutive P values are 8 consecutive keys; the
// V^T operand is read from the row-major V tile with ds_read_b64_tr_b16.
//
// Memory pipeline: K and V tiles (64 keys) travel HBM -> LDS directly with
// global_load_lds_dwordx4 / buffer_load_dwordx4 ... lds (no staging registers,
// no LDS store instructions).  K and V are double-buffered separately and K
// runs one tile ahead: iteration j issues the loads of K[j+2] and V[j+1], then
// one stream of MFMAs: S[j+1] = K[j+1] Q^T (the softmax VALU work of tile j
// interleaved between them) and O += V[j] P[j] (the row max of S[j+1] between
// those), every LDS operand read two MFMAs ahead of its use.  Every load has
// one full iteration to land; one barrier per tile.
//
// LDS (64 banks on gfx950): rows are unpadded and their 16-byte chunks are
// XOR-swizzled by row, so the 16 rows one ds_read_b128 of K touches, and the
// 4 rows x 64 bytes one transpose read of V touches, fall on distinct banks.
//
// Softmax: log2 domain (sm_scale * log2(e) folded into Q before its bf16
// rounding).  The score MFMAs start from -m (m = running row max), so exp2
// takes their output as is; the row sum adds the bf16 P values that feed the
// PV MFMAs (v_dot2 against ones), so numerator and denominator use the same
// weights.  The running max is only raised when some row's tile max exceeds
// it by more than 2^8 (then O, l and the pending scores are shifted);
// otherwise P values up to 256 accumulate against the stale max.  The final
// O/l is exact either way.
// Causal workgroups are issued heaviest (last q-block) first.

#include <type_traits>

#include "nq_common.hpp"
#include "nq_internal.hpp"
#include "nq_prefill.hpp"

namespace nq {

// A workgroup has NW waves (8, or 4 for launches too small to fill the GPU
// with 8-wave workgroups) and 32 query rows per wave.
constexpr int PF_MAX_ROWS = 256;
constexpr int64_t PF_WIDE_MIN_WGS = 2048;  // 8-wave workgroups needed to prefer them
constexpr int PF_BN = 64;     // keys per tile
constexpr float PF_RESCALE_LOG2 = 8.0f;
// LDS operand reads in flight ahead of their MFMA.  They are inline asm waited
// for by count, so no compiler-made copy or spill may touch their registers
// before the wait: at 3 the 8-wave D = 128 instance spills a pending operand
// (wrong results); tests/test_asm_waits.py checks the built assembly.
constexpr int PF_READ_AHEAD = 2;

// LDS reads still in flight when op i of a step's MFMA stream waits for its
// own: those of ops i+1 .. min(i+pd, nops-1); a K operand (op < nqk) is one
// ds_read_b128, a V^T operand two transpose reads.
constexpr int stream_younger(int i, int nops, int nqk, int pd) {
  int c = 0;
  const int last = (i + pd < nops - 1) ? i + pd : nops - 1;
  for (int k = i + 1; k <= last; ++k) c += (k < nqk ? 1 : 2);
  return c;
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}


// This lane's index (0..63), computed afresh (volatile, so the compiler cannot
// reuse an earlier value): code after the main loop derives its lane-dependent
// values from it instead of keeping them live through the loop, where they
// would be spilled and reloaded (and a reload, counted by vmcnt like the tile
// loads in flight, waits for those loads too).
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// MFMA row r of a 32-key block holds key sigma(r): bits 2 and 3 swapped.
__device__ __forceinline__ int key_perm32(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

template <int D, int NW>
struct PfTile {
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int CPR = D / 8;                   // 16-byte chunks per row
  static constexpr int RPL = 256 / ROW_BYTES;         // rows per 256-byte bank line
  static constexpr int TILE_BYTES = PF_BN * ROW_BYTES;
  static constexpr int LOADS = TILE_BYTES / 1024 / NW; // 1 KiB load instructions per wave
  // physical chunk of logical chunk c in row r
  __device__ static int k_chunk(int r, int c) { return c ^ ((r / RPL) & (CPR - 1)); }
  __device__ static int v_chunk(int r, int c) { return c ^ (4 * ((r / RPL) & (D / 32 - 1))); }
};

// PAGED: K and V rows come from paged pools through the block table (key t of
// sequence b is row t % page of page bt[b * bts + t / page], pool strides
// (ksb, ksh, kss) = (page, head, row)); page % 32 == 0, so each 32-row half of
// a 64-key tile lies in one page.
// BIAS: an additive bias per (query, key) (p.bias, SDPA's attn_mask) is added
// to every score tile before the row max, so every step takes the masked
// path; a row may then see no finite score in its first tiles (or in none),
// which the running max starts from a placeholder for (below).
template <int D, typename T, bool CAUSAL, bool FUSE_Q, int NW, bool PAGED = false, bool BIAS = false>
__global__ void __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW),
                               amdgpu_waves_per_eu(2, 2)))
prefill_kernel(PrefillParams p) {
  using Tl = PfTile<D, NW>;
  constexpr int NDB = D / 16;        // 16-wide d blocks (QK^T k-steps)
  constexpr int NDO = D / 32;        // 32-wide d blocks (output tiles)
  constexpr int TB = Tl::TILE_BYTES;
  // LDS: K0 K1 V0 V1, and one more tile's worth for the staged sin rows
  __shared__ __attribute__((aligned(1024))) unsigned char smem[5 * TB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int r32 = lane & 31, hh = lane >> 5;

  // workgroup -> (batch, kv head, q-block).  Workgroups are dealt to the 8
  // XCDs round-robin (id % 8).  When the (batch, kv head) pairs split evenly
  // over the XCDs and each pair has many q-blocks, XCD x works through its own
  // pairs one after another, so the K/V of one pair (its L2 working set) is
  // shared by all of that XCD's CUs; otherwise pairs are interleaved and the
  // heaviest q-blocks of all pairs go first (better tail balance when each
  // pair is only a few rounds of work).
  const int npairs = p.B * p.Hkv;
  const int L = blockIdx.x;
  int qrank, pair;
  if (npairs % 8 == 0 && p.nqb >= 128) {
    const int xcd = L & 7, k = L >> 3;
    pair = (k / p.nqb) * 8 + xcd;
    qrank = k % p.nqb;
  } else {
    pair = L % npairs;
    qrank = L / npairs;
  }
  const int qblk = CAUSAL ? (p.nqb - 1 - qrank) : qrank;
  const int b = pair / p.Hkv, kvh = pair % p.Hkv;
  const int q0 = qblk * p.BM;
  const int coff = p.T - p.S;
  // keys of this sequence (key padding: fewer than T)
  const int Tk = pf_keys(p, b);
  if (Tk <= 0) {  // no keys: zeros; a length out of range: NaN
    const float f = Tk < 0 ? __builtin_nanf("") : 0.f;
    for (int r = threadIdx.x; r < 32 * NW; r += 64 * NW) {
      const int g = r % p.G, qi = q0 + r / p.G;
      if (qi >= p.S) continue;
      T* orow = reinterpret_cast<T*>(p.o) + b * p.osb + (kvh * p.G + g) * p.osh + (int64_t)qi * p.oss;
      for (int d = 0; d < D; ++d) orow[d] = (T)f;
      if (p.lse) p.lse[((int64_t)b * p.Hq + kvh * p.G + g) * p.S + qi] = -INFINITY;
    }
    return;
  }

  const int kv_end = CAUSAL ? min(Tk, q0 + p.BM + coff) : Tk;
  const int ntiles = (kv_end + PF_BN - 1) / PF_BN;
  // K/V are bf16 in memory: they go to LDS unconverted.  A paged pool's base
  // is its kv head's slice of page 0 (pages are added per tile).
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(
      reinterpret_cast<const bf16*>(p.k) + (PAGED ? 0 : b * p.ksb) + kvh * p.ksh);
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(
      reinterpret_cast<const bf16*>(p.v) + (PAGED ? 0 : b * p.vsb) + kvh * p.vsh);
  const int64_t krow_bytes = p.kss * 2, vrow_bytes = p.vss * 2;
  const int64_t kpage_bytes = p.ksb * 2, vpage_bytes = p.vsb * 2;

  // ---- tile loads: load instruction G (0 <= G < NW*LOADS) fills LDS
  // bytes [G*1024, G*1024+1024) of the tile, lane t the 16 bytes at +16*t;
  // wave w issues G = NW*m + w.  With that interleave a lane's row
  // offset within its 16-row (D=128) or 8-row (D=64) swizzle period, and so
  // its chunk swizzle, is the same for every m: the address is a wave-uniform
  // base (tile, m) in SGPRs plus one loop-invariant 32-bit lane offset.  In a tile that runs past T the rows
  // are clamped to T-1 instead (their scores are masked, so P = 0 there).
  constexpr int RPI = 64 / Tl::CPR;  // rows per load instruction
  const int row0 = wave * RPI + lane / Tl::CPR;  // row of instruction m: row0 + NW*RPI*m
  const int pc0 = lane % Tl::CPR;
  const uint32_t koff = (uint32_t)(row0 * krow_bytes) + Tl::k_chunk(row0, pc0) * 16;
  const uint32_t voff = (uint32_t)(row0 * vrow_bytes) + Tl::v_chunk(row0, pc0) * 16;
  auto load_tile = [&](const unsigned char* base, int64_t row_bytes, int64_t page_bytes, uint32_t off,
                       int lds_off, int tile) {
    const int lds_w = lds_off + wave * 1024;
    if constexpr (PAGED) {
      // rows key0 .. key0+31 lie in page pi0 from row r0, rows key0+32 .. +63
      // in page pi1 from row r1 (page % 32 == 0, key0 % 64 == 0); the block
      // table is read through the scalar path, only for rows below Tk
      const int key0 = tile * PF_BN;
      const int pi0 = key0 / p.page, r0 = key0 - pi0 * p.page;
      const bool same = r0 + 32 < p.page;
      const int r1 = same ? r0 + 32 : 0;
      const int64_t btb = (int64_t)b * p.bts;
      const int64_t pg0 = ld_uniform(p.bt, btb + pi0);
      const int64_t pg1 = (same || key0 + 32 >= Tk) ? pg0 : (int64_t)ld_uniform(p.bt, btb + pi0 + 1);
      if (key0 + PF_BN <= Tk) {
        // one descriptor per instruction over its RPI rows; the lane's offset
        // within them is its offset less the wave's rows
        const uint32_t loff = off - (uint32_t)(wave * RPI * row_bytes);
#pragma unroll
        for (int m = 0; m < Tl::LOADS; ++m) {
          const int rr = m * NW * RPI + wave * RPI;  // first tile row of instruction m
          const unsigned char* rb = base + (rr < 32 ? pg0 : pg1) * page_bytes +
                                    (int64_t)((rr < 32 ? r0 : r1) + (rr & 31)) * row_bytes;
          buffer_load_lds16(make_rsrc(rb, (uint32_t)(RPI * row_bytes)), smem + lds_w + m * NW * 1024, loff, 0u);
        }
      } else {
        const uint32_t chunk_off = off - (uint32_t)(row0 * row_bytes);
#pragma unroll
        for (int m = 0; m < Tl::LOADS; ++m) {
          const int kr = min(row0 + m * NW * RPI, Tk - 1 - key0);  // tile row, clamped to the last key
          const unsigned char* rb = base + (kr < 32 ? pg0 : pg1) * page_bytes +
                                    (int64_t)((kr < 32 ? r0 : r1) + (kr & 31)) * row_bytes;
          global_load_lds16(rb + chunk_off, smem + lds_w + m * NW * 1024);
        }
      }
      return;
    }
    if (tile * PF_BN + PF_BN <= Tk) {
      // buffer loads: the tile's base in a scalar descriptor, the lane offset
      // in one 32-bit VGPR, the instruction's row step as a scalar offset (no
      // 64-bit per-instruction address VGPRs; the 8-wave kernel ran 1.1-1.5%
      // faster than with global_load_lds, outputs bit-identical)
      const BufRsrc r = make_rsrc(base + (int64_t)tile * PF_BN * row_bytes, (uint32_t)(PF_BN * row_bytes));
#pragma unroll
      for (int m = 0; m < Tl::LOADS; ++m)
        buffer_load_lds16(r, smem + lds_w + m * NW * 1024, off, (uint32_t)(m * NW * RPI * row_bytes));
    } else {
      const uint32_t chunk_off = off - (uint32_t)(row0 * row_bytes);
#pragma unroll
      for (int m = 0; m < Tl::LOADS; ++m) {
        const int key = min(tile * PF_BN + row0 + m * NW * RPI, Tk - 1);
        global_load_lds16(base + key * row_bytes + chunk_off, smem + lds_w + m * NW * 1024);
      }
    }
  };
  auto load_k = [&](int tile, int buf) { load_tile(kbase, krow_bytes, kpage_bytes, koff, buf * TB, tile); };
  auto load_v = [&](int tile, int buf) { load_tile(vbase, vrow_bytes, vpage_bytes, voff, (2 + buf) * TB, tile); };
  // this lane's query row: column r32 of this wave's 32 rows.  Row R of the
  // workgroup is head R % G at position q0 + R / G: the G heads of a position
  // sit in adjacent lanes, so a wave's rows span 32 / G positions and their
  // cos/sin table rows (and, in the projections' (B, S, H, D) storage, their
  // Q and O rows) share cache lines.
  const int R = wave * 32 + r32;
  const int g = R % p.G, pr = R / p.G;
  const int head = kvh * p.G + g;
  const int qi = q0 + pr;
  const bool qvalid = qi < p.S;
  const int qi_c = qvalid ? qi : p.S - 1;

  // ---- prologue loads.  The first K/V tiles go first, then every register
  // load of the Q work (the Q row, the norm weight, the row's cos/sin) back to
  // back, so that a single memory round trip covers all of them before the Q
  // work starts (each load depending on an earlier one's result would cost a
  // round trip of its own).  The table row is resolved before anything is in
  // flight: only explicit per-token positions need a load for it.
  const bool do_norm = FUSE_Q && p.qw != nullptr;
  const bool do_rope = FUSE_Q && p.cos_tab != nullptr;
  int tab_row = 0;
  if (do_rope) tab_row = table_row(row_position(p.q_pos, p.q_pos_base, p.q_pos0, b, qi_c, p.S), p.max_pos);
  // The cos/sin rows of the workgroup's BM consecutive positions are staged in
  // LDS (cos in the V1 buffer, idle until step 0, sin in the extra tile) with
  // coalesced 1 KiB DMA instructions, instead of every lane loading its own
  // row's 64 values: a table row (D/2 fp32) is as long as a K row, so BM <= 64
  // rows fit one tile.  Explicit per-token positions keep the per-lane loads.
  const bool stage_tab = do_rope && p.q_pos == nullptr && p.BM <= PF_BN;
  load_k(0, 0);
  load_v(0, 0);
  if (ntiles > 1) load_k(1, 1);
  // A wave reads the table rows of its own 32 / G positions.  When those fill
  // whole DMA instructions the wave stages exactly them and then waits for its
  // own loads only; otherwise the instructions are spread over the waves and a
  // barrier follows (8B-like shape: that barrier waited ~1.7 us for the
  // slowest wave).
  constexpr int TROW = D * 2;  // bytes per table row
  const int tab_rpw = 32 / p.G;
  const bool tab_own = stage_tab && tab_rpw > 0 && tab_rpw % (1024 / TROW) == 0;  // G = 64: 0 rows
  if (stage_tab) {
    const int pos0 = (p.q_pos_base ? ld_uniform(p.q_pos_base, b) : p.q_pos0) + q0;
    const int ninst = (p.BM * TROW + 1023) / 1024;
    const int m0 = tab_own ? wave * tab_rpw * TROW / 1024 : wave;
    const int m1 = tab_own ? (wave + 1) * tab_rpw * TROW / 1024 : ninst;
    for (int m = m0; m < m1; m += tab_own ? 1 : NW) {
      const int pb = m * 1024 + lane * 16;
      const int row = pb / TROW;
      const int c = Tl::k_chunk(row, (pb % TROW) / 16);  // logical 16-byte chunk (4 values)
      const int tr = min(max(pos0 + min(row, p.BM - 1), 0), p.max_pos - 1);
      global_load_lds16(p.cos_tab + (int64_t)tr * (D / 2) + c * 4, smem + 3 * TB + m * 1024);
      global_load_lds16(p.sin_tab + (int64_t)tr * (D / 2) + c * 4, smem + 4 * TB + m * 1024);
    }
  }
  floatx8 xf[NDB];
  floatx8 tc[NDB / 2], ts[NDB / 2];
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + head * p.qsh + (int64_t)qi_c * p.qss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) xf[db] = Vec8<T>::load_f32(qrow + db * 16 + hh * 8);
    if (do_rope) {
      if (stage_tab) {
        wait_vmcnt0();
        if (!tab_own) __syncthreads();
        // row pr of the stage; a position outside the tables gives NaN, as the
        // per-lane loads do
        const float bad = tab_row < 0 ? __builtin_nanf("") : 0.f;
#pragma unroll
        for (int db = 0; db < NDB / 2; ++db) {
          const int c0 = db * 4 + hh * 2;
          const floatx4 c_lo = *reinterpret_cast<const floatx4*>(smem + 3 * TB + pr * Tl::ROW_BYTES + Tl::k_chunk(pr, c0) * 16);
          const floatx4 c_hi = *reinterpret_cast<const floatx4*>(smem + 3 * TB + pr * Tl::ROW_BYTES + Tl::k_chunk(pr, c0 + 1) * 16);
          const floatx4 s_lo = *reinterpret_cast<const floatx4*>(smem + 4 * TB + pr * Tl::ROW_BYTES + Tl::k_chunk(pr, c0) * 16);
          const floatx4 s_hi = *reinterpret_cast<const floatx4*>(smem + 4 * TB + pr * Tl::ROW_BYTES + Tl::k_chunk(pr, c0 + 1) * 16);
          tc[db] = floatx8{c_lo[0], c_lo[1], c_lo[2], c_lo[3], c_hi[0], c_hi[1], c_hi[2], c_hi[3]} + bad;
          ts[db] = floatx8{s_lo[0], s_lo[1], s_lo[2], s_lo[3], s_hi[0], s_hi[1], s_hi[2], s_hi[3]} + bad;
        }
      } else {
#pragma unroll
        for (int db = 0; db < NDB / 2; ++db) {
          tc[db] = load_tab8(p.cos_tab, tab_row, D / 2, db * 16 + hh * 8);
          ts[db] = load_tab8(p.sin_tab, tab_row, D / 2, db * 16 + hh * 8);
        }
      }
    }
  }

  // ---- Q operand (B of S^T = K Q^T): lane holds Q[row][dblk*16 + hh*8 + e]
  bf16x8 qop[NDB];
  {
    if (do_norm) {
      float ss = 0.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xf[db][e] * xf[db][e];
      ss = xor32_sum(ss);
      const float r = rsqrtf(ss / (float)D + p.eps);
      // the weights through the scalar path: the 32 lanes of a half-wave need
      // the same 8, so both halves' values come as wave-uniform loads and each
      // lane selects its own (as vector loads, 16 of them issued at ~220
      // clocks each: 1.8 us of a ~7.5 us prologue at the 1.7B-like shape)
      const auto* wc = (const __attribute__((address_space(4))) float*)p.qw;  // read-only
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float w0 = wc[db * 16 + e], w1 = wc[db * 16 + 8 + e];
          xf[db][e] = xf[db][e] * r * (hh ? w1 : w0);
        }
    }
    if (do_rope) {
#pragma unroll
      for (int db = 0; db < NDB / 2; ++db) {
        floatx8 x1 = xf[db], x2 = xf[db + NDB / 2];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xf[db][e] = x1[e] * tc[db][e] - x2[e] * ts[db][e];
          xf[db + NDB / 2][e] = x2[e] * tc[db][e] + x1[e] * ts[db][e];
        }
      }
    }
    // the softmax scale (times log2 e) rides on Q, so S comes out in log2 units
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[db][e] *= p.scale_log2;
      qop[db] = to_bf16x8(xf[db]);
    }
  }

  // ---- per-lane LDS read offsets (bytes within a tile)
  // K: MFMA row sigma(r32) (+32 for the second key block), chunk 2*db + hh
  static_assert(Tl::CPR * 16 == Tl::ROW_BYTES && NDB * 2 <= Tl::CPR && NDO * 4 <= Tl::CPR,
                "k_off[db] == k_off[0] ^ (db << 5), v_off[dd] == v_off[0] ^ (dd << 6): "
                "the swizzled chunk bits stay below the row bits");
  int k_off[NDB];
  {
    const int row = key_perm32(r32);
#pragma unroll
    for (int db = 0; db < NDB; ++db) k_off[db] = row * Tl::ROW_BYTES + Tl::k_chunk(row, 2 * db + hh) * 16;
  }
  // V^T via transpose reads: lane group gi = lane/16, j = lane%16 reads row
  // hh*8 + j/4 (+16*ks + 4*half), column dd*32 + (gi&1)*16 + 4*(j%4)
  int v_off[NDO];
  {
    const int gi = lane >> 4, jj = lane & 15;
    const int row = hh * 8 + (jj >> 2);
#pragma unroll
    for (int dd = 0; dd < NDO; ++dd) {
      const int col = dd * 32 + (gi & 1) * 16 + 4 * (jj & 3);
      v_off[dd] = row * Tl::ROW_BYTES + Tl::v_chunk(row, col / 8) * 16 + (col % 8) * 2;
    }
  }

  auto qk = [&](int buf, floatx16& s0, floatx16& s1) {
    s0 = floatx16{};
    s1 = floatx16{};
    const unsigned char* Kt = smem + buf * TB;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      bf16x8 a0 = *reinterpret_cast<const bf16x8*>(Kt + k_off[db]);
      bf16x8 a1 = *reinterpret_cast<const bf16x8*>(Kt + k_off[db] + 32 * Tl::ROW_BYTES);
      s0 = mfma32(a0, qop[db], s0);
      s1 = mfma32(a1, qop[db], s1);
    }
  };

  // Running row max m_i is kept as the sum of two bf16 values, so that -m_i
  // enters the score MFMAs exactly: S^T = [1 1 0..] x [-m_hi -m_lo 0..]^T
  // (one extra MFMA per 32-key block, k-slots 0 and 1) + K Q^T.  Every score
  // then leaves the MFMA already offset by the row max, and exp2 takes it as is.
  float m_i = 0.f, l_i = 0.f;
  bf16x8 qaug;
  // [1 1 0 ..] in the lanes of k-slots 0..7 (hh = 0), zeros in the others.
  // 4-wave workgroups build it where it is used, from a fresh lane index:
  // held through the loop, it is what their register allocation spills (and
  // reloads every step); 8-wave workgroups keep it in registers.
  bf16x8 ones_held;
  {
    const bf16 one = hh == 0 ? (bf16)1.0f : (bf16)0.0f;
    const bf16 z = (bf16)0.0f;
    ones_held = bf16x8{one, one, z, z, z, z, z, z};
  }
  auto ones_op = [&]() {
    if constexpr (NW == 4) {
      const bf16 one = (fresh_lane() >> 5) == 0 ? (bf16)1.0f : (bf16)0.0f;
      const bf16 z = (bf16)0.0f;
      return bf16x8{one, one, z, z, z, z, z, z};
    } else {
      return ones_held;
    }
  };
  // m_i <- m rounded to the nearest hi + lo bf16 pair; qaug <- (-hi, -lo)
  auto set_max = [&](float m) {
    const bf16 mh = (bf16)m;
    const bf16 ml = (bf16)(m - (float)mh);
    m_i = (float)mh + (float)ml;
    const bf16 z = (bf16)0.0f;
    qaug = hh == 0 ? bf16x8{(bf16)(-(float)mh), (bf16)(-(float)ml), z, z, z, z, z, z}
                   : bf16x8{z, z, z, z, z, z, z, z};
  };
  floatx16 oacc[NDO];
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd) oacc[dd] = floatx16{};

  // prologue: K0, V0 (and K1) in flight; S0
  wait_vmcnt0();
  __syncthreads();
  // S[j] lives in sA for even j and in sB for odd j (the loop is unrolled by
  // two so neither the S registers nor the LDS buffer offsets need moving)
  floatx16 sA[2], sB[2];
  qk(0, sA[0], sA[1]);

  // masking of tile n0: keys past T, and (causal) keys past this row's frontier
  // 1/G as a wave-uniform float: (R + 0.5) / G rounds down to R / G exactly
  // for R < 2^16, without the integer-division sequence and its constants
  const float inv_g = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, 1.0f / (float)p.G)));
  auto mask_tile = [&](floatx16* s, int n0) {
    if (BIAS || (n0 + PF_BN > Tk) || (CAUSAL && n0 + PF_BN - 1 > q0 + coff)) {
      const int ml = fresh_lane();
      const int mhh = ml >> 5;
      const int mR = wave * 32 + (ml & 31);
      const int mqi = q0 + (int)(((float)mR + 0.5f) * inv_g);
      if constexpr (BIAS) {
        // the lane's 32 scores are 4 runs of 8 consecutive keys: one 16-byte
        // read each (runs starting past the keys are masked below anyway)
        const int mg = mR - (mqi - q0) * p.G;
        const bf16* brow = reinterpret_cast<const bf16*>(p.bias) + b * p.bsb + (kvh * p.G + mg) * p.bsh +
                           (int64_t)min(mqi, p.S - 1) * p.bss;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int k8 = n0 + kb * 32 + h2 * 16 + mhh * 8;
            if (k8 < Tk) {
              const bf16x8 bv = *reinterpret_cast<const bf16x8*>(brow + k8);
#pragma unroll
              for (int e = 0; e < 8; ++e) s[kb][h2 * 8 + e] += (float)bv[e] * kLog2e;
            }
          }
      }
      const int lim = CAUSAL ? min(Tk - 1, mqi + coff) : Tk - 1;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = n0 + kb * 32 + (i >> 3) * 16 + mhh * 8 + (i & 7);
          if (key > lim) s[kb][i] = -INFINITY;
        }
    }
  };
  // row max of the current tile in log2 units (tile 0 holds key 0 for every
  // row, so it is finite there; later tiles compare against a finite m_i)
  // (S0 was computed without the offset: its max sets m_i and is subtracted
  // here; later tiles carry the offset from their MFMAs.)  mx_cur is the row
  // max of the next tile to be exponentiated, relative to m_i.
  float mx_cur = 0.f;
  // BIAS: a row with no finite score yet holds the placeholder max 0 (ph);
  // its first finite tile max then replaces it outright (O and l are still 0)
  bool ph = false;
  {
    mask_tile(sA, 0);
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) mx = fmaxf(mx, fmaxf(sA[kb][i], sA[kb][i + 1]));
    mx = xor32_max(mx);
    if constexpr (BIAS) {
      ph = !(mx > -INFINITY);
      if (ph) mx = 0.f;
      // S[0] relative to the placeholder is all -inf: no max to take from it
      if (ph) mx_cur = -INFINITY;
    }
    set_max(mx);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sA[kb] -= m_i;
  }

  // One 64-key tile.  Order inside a step: barrier + next loads; rescale
  // against the row max of S[j] (found in the previous step); then one
  // fixed-order stream in which the MFMAs of S[j+1] = K[j+1] Q^T are
  // interleaved with the exp/pack/sum of P[j] (sched_barrier keeps them
  // interleaved, since a wave issues in order); then, in the steps that may
  // need it, the mask of S[j+1]; then O += V[j]^T P[j], with the row max of
  // S[j+1] taken alongside those MFMAs.
  auto step = [&](auto parity, auto has_next, auto may_mask, int j) {
    constexpr int P = decltype(parity)::value;       // == j & 1
    constexpr bool NEXT = decltype(has_next)::value;  // j + 1 < ntiles
    constexpr bool MASKN = decltype(may_mask)::value; // tile j + 1 may need masking
    floatx16* s_cur = P ? sB : sA;
    floatx16* s_next = P ? sA : sB;
    const int n0 = j * PF_BN;
    // loads issued last step (K[j+1], V[j]) have landed; every wave is done
    // with K[j] and V[j-1], so their buffers can be refilled
    wait_vmcnt0();
    __syncthreads();
    if (NEXT) {
      if (j + 2 < ntiles) load_k(j + 2, P);
      load_v(j + 1, P ^ 1);
    }

    // online softmax (log2 domain); each lane owns one query row
    (void)n0;
    bool raise = mx_cur > PF_RESCALE_LOG2;
    if constexpr (BIAS) raise = raise || (ph && mx_cur > -INFINITY);
    if (wave_any(raise)) {
      const float m_old = m_i;
      float inc = fmaxf(mx_cur, 0.f);
      if constexpr (BIAS) {
        if (ph) inc = mx_cur > -INFINITY ? mx_cur : 0.f;
      }
      set_max(m_i + inc);
      const float delta = m_i - m_old;
      float alpha = fast_exp2(-delta);
      if constexpr (BIAS) {
        if (ph) alpha = 0.f;  // nothing accumulated yet (avoids 0 * inf)
        ph = ph && !(mx_cur > -INFINITY);
      }
      l_i *= alpha;
#pragma unroll
      for (int dd = 0; dd < NDO; ++dd) oacc[dd] *= alpha;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s_cur[kb] -= delta;
    }

    // ---- one fixed-order stream of MFMAs (sched_barrier fences; a wave
    // issues in order).  Op i < NQK: S[j+1] for k-block i/2, key half i%2
    // (A = K[j+1] from LDS, B = Q), after one op that loads -m_i into both
    // halves' accumulators; op NQK + t: O^T[t % NDO] += V[j]^T (keys 16*(t/NDO)..)
    // P[j]^T.  LDS operands are read PD ops ahead (K: one ds_read_b128, V^T:
    // two transpose reads), issued as inline asm so the HBM->LDS loads just
    // issued keep flying (the compiler would wait for them before an LDS read
    // it can see), with lgkmcnt counting this stream's reads only.  Between
    // the QK MFMAs go the exp2 / bf16 pack / row sum of P[j] (two values per
    // op), between the PV MFMAs the row max of S[j+1].
    constexpr int NQK = NEXT ? 2 * NDB : 0;
    constexpr int NPV = 4 * NDO;
    constexpr int NOPS = NQK + NPV;
    constexpr int PD = PF_READ_AHEAD;
    const uint32_t Kt = lds_addr(smem + (P ^ 1) * TB);
    const uint32_t Vt = lds_addr(smem + (2 + P) * TB);
    float acc[2] = {0.f, 0.f};
    floatx8 tv[4];
    bf16x8 pop[4];
    bf16x8 opnd[PD + 1];
    floatx16 sn[2];
    float mxn = -INFINITY;
    auto issue = [&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (i < NQK) {
        // k_off[db] = k_off[0] ^ (db << 5) (the XOR swizzle moves the chunk
        // index, whose bits sit below the row's).  The masked steps, which come
        // last, derive it so the other seven offsets die after the unmasked
        // loop instead of being spilled and reloaded around the masked steps.
        const uint32_t ko = MASKN ? (uint32_t)(k_off[0] ^ ((i / 2) << 5)) : (uint32_t)k_off[i / 2];
        opnd[i % (PD + 1)] = lds_read_b128_nowait<(i % 2) * 32 * Tl::ROW_BYTES>(Kt + ko);
      } else {
        constexpr int t = i - NQK;
        // likewise v_off[dd] = v_off[0] ^ (dd << 6)
        const uint32_t vo = MASKN ? (uint32_t)(v_off[0] ^ ((t % NDO) << 6)) : (uint32_t)v_off[t % NDO];
        opnd[i % (PD + 1)] = lds_read_tr8_nowait<8 * D>(Vt + vo + (t / NDO) * 16 * Tl::ROW_BYTES);
      }
    };
    // P[j] values e: exp2, and per 8 values a bf16 pack and its row sum
    auto pwork = [&](int e) {
      tv[e / 8][e % 8] = fast_exp2(s_cur[e / 16][e % 16]);
      if (e % 8 == 7) {
        pop[e / 8] = to_bf16x8(tv[e / 8]);
        acc[(e / 8) & 1] = rowsum_bf16x8(pop[e / 8], acc[(e / 8) & 1]);
      }
    };
    static_for<0, (PD < NOPS ? PD : NOPS)>(issue);
    floatx16 s_init;  // -m_i in every element; the first MFMA of each key half starts from it
    if (NEXT) s_init = mfma32(ones_op(), qaug, floatx16{});
    if (NQK == 0) {  // last tile: all of P[j] before the PV stream
#pragma unroll
      for (int e = 0; e < 32; ++e) pwork(e);
    }
    static_for<0, NOPS>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (i + PD < NOPS) issue(std::integral_constant<int, i + PD>{});
      lgkm_wait<stream_younger(i, NOPS, NQK, PD)>();
      if constexpr (i < NQK) {
        sn[i % 2] = mfma32(opnd[i % (PD + 1)], qop[i / 2], i < 2 ? s_init : sn[i % 2]);
        constexpr int per = NQK ? 32 / NQK : 1;  // P values per QK op
#pragma unroll
        for (int u = 0; u < per; ++u) pwork(i * per + u);
      } else {
        constexpr int t = i - NQK;
        if constexpr (t == 0 && NEXT) {
          s_next[0] = sn[0];
          s_next[1] = sn[1];
          if (MASKN) mask_tile(s_next, n0 + PF_BN);  // diagonal / last tiles only
        }
        oacc[t % NDO] = mfma32(opnd[i % (PD + 1)], pop[t / NDO], oacc[t % NDO]);
        if (NEXT) {
          constexpr int mper = 32 / NPV;  // S[j+1] elements folded into the max per op
#pragma unroll
          for (int u = 0; u < mper; ++u) {
            const int e = t * mper + u;
            mxn = fmaxf(mxn, s_next[e / 16][e % 16]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    l_i += acc[0] + acc[1];
    if (NEXT) mx_cur = xor32_max(mxn);
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using Yes = std::integral_constant<bool, true>;
  using No = std::integral_constant<bool, false>;
  // Tiles below jfree lie inside T and before every row's causal frontier, so a
  // step whose next tile is one of them carries no mask branch.  That branch would
  // split the step into basic blocks, and the compiler would then sink the exp2
  // work of P[j] below the S[j+1] MFMAs it is meant to interleave with.
  const int jfree = BIAS ? 0 : min(ntiles, min(Tk / PF_BN, CAUSAL ? (q0 + coff + 1) / PF_BN : ntiles));
  int j = 0;
  for (; j + 2 < jfree; j += 2) {
    step(I0{}, Yes{}, No{}, j);
    step(I1{}, Yes{}, No{}, j + 1);
  }
  for (; j + 2 < ntiles; j += 2) {
    step(I0{}, Yes{}, Yes{}, j);
    step(I1{}, Yes{}, Yes{}, j + 1);
  }
  if (ntiles - j == 2) {
    step(I0{}, Yes{}, Yes{}, j);
    step(I1{}, No{}, Yes{}, j + 1);
  } else {
    step(I0{}, No{}, Yes{}, j);
  }

  l_i = xor32_sum(l_i);
  // (BIAS: a row the bias masks entirely has l = 0 and gets zeros, as SDPA gives)
  const float inv_l = (BIAS && !(l_i > 0.f)) ? 0.f : 1.f / l_i;

  // ---- epilogue: O goes through LDS, so that every store instruction writes
  // whole rows (16 lanes x 16 contiguous bytes per row) instead of 8-byte
  // pieces of 32 rows, which leave L2 as partly written lines.  Each wave
  // stages its own 32 rows in its own slice of the (now idle) tile buffers,
  // with the K tile's chunk swizzle, and reads them back row-major.
  static_assert(std::is_same<T, bf16>::value, "bf16 output");
  constexpr int OCH = D / 8;  // 16-byte chunks per output row
  static_assert(32 * NW * Tl::ROW_BYTES <= 4 * TB, "output stage fits the tile buffers");
  __syncthreads();  // every wave is done with the last K/V tiles
  unsigned char* const ostage = smem + wave * 32 * Tl::ROW_BYTES;
  const int el = fresh_lane(), er32 = el & 31, ehh = el >> 5;
#pragma unroll
  for (int dd = 0; dd < NDO; ++dd)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const floatx4 t = {oacc[dd][gq * 4 + 0] * inv_l, oacc[dd][gq * 4 + 1] * inv_l,
                         oacc[dd][gq * 4 + 2] * inv_l, oacc[dd][gq * 4 + 3] * inv_l};
      *reinterpret_cast<bf16x4*>(ostage + er32 * Tl::ROW_BYTES + Tl::k_chunk(er32, dd * 4 + gq) * 16 + ehh * 8) =
          __builtin_convertvector(t, bf16x4);
    }
  {
    constexpr int RPR = 64 / OCH;  // rows per read-back instruction
#pragma unroll
    for (int i = 0; i < 32 / RPR; ++i) {
      const int r = i * RPR + el / OCH, c = el % OCH;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(ostage + r * Tl::ROW_BYTES + Tl::k_chunk(r, c) * 16);
      const int Rw = wave * 32 + r;
      const int qr = q0 + Rw / p.G;
      if (qr < p.S)
        *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.o) + b * p.osb + (kvh * p.G + Rw % p.G) * p.osh +
                                   (int64_t)qr * p.oss + c * 8) = v;
    }
  }
  if (p.lse && ehh == 0) {
    const int eR = wave * 32 + er32;
    const int eq = q0 + eR / p.G;
    if (eq < p.S)
      p.lse[((int64_t)b * p.Hq + kvh * p.G + eR % p.G) * p.S + eq] =
          (BIAS && !(l_i > 0.f)) ? -INFINITY : (m_i + __log2f(l_i)) * kLn2;
  }
}

template <int D, typename T, int NW>
static hipError_t launch_prefill_nw(const PrefillParams& p, bool causal, bool fuse, hipStream_t st) {
  dim3 grid((unsigned)(p.nqb * p.B * p.Hkv));
  dim3 block(64 * NW);
  if (p.bias) {  // an attention bias: 4-wave workgroups, the fused-Q instance, dense K/V
    if constexpr (NW == 4) {
      if (causal) hipLaunchKernelGGL((prefill_kernel<D, T, true, true, 4, false, true>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((prefill_kernel<D, T, false, true, 4, false, true>), grid, block, 0, st, p);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (p.bt) {  // paged pools: the fused-Q instance (its norm and rotation are skipped when not given)
    if (causal) hipLaunchKernelGGL((prefill_kernel<D, T, true, true, NW, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_kernel<D, T, false, true, NW, true>), grid, block, 0, st, p);
    return hipGetLastError();
  }
  if (causal) {
    if (fuse) hipLaunchKernelGGL((prefill_kernel<D, T, true, true, NW>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_kernel<D, T, true, false, NW>), grid, block, 0, st, p);
  } else {
    if (fuse) hipLaunchKernelGGL((prefill_kernel<D, T, false, true, NW>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((prefill_kernel<D, T, false, false, NW>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

template <int D, typename T>
static hipError_t launch_prefill(const PrefillParams& p, int nw, bool causal, bool fuse, hipStream_t st) {
  if constexpr (D == 32) {
    if (nw != 4) return hipErrorInvalidValue;  // one 1 KiB tile load per wave needs 4 waves
    return launch_prefill_nw<D, T, 4>(p, causal, fuse, st);
  } else {
    return nw == 8 ? launch_prefill_nw<D, T, 8>(p, causal, fuse, st) : launch_prefill_nw<D, T, 4>(p, causal, fuse, st);
  }
}

}  // namespace nq

using namespace nq;

// Shared by the dense, paged and bias entry points: bt == NULL for dense K/V,
// bias == NULL for none.
static int prefill_entry(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, const int32_t* bt, int64_t bts, int page,
                         const void* bias, const int64_t* bias_strides,
                         void* o, const int64_t* o_strides, float* lse, const int32_t* key_lens, int B, int Hq,
                         int Hkv, int S, int T, int D, int dtype, const float* q_weight, float eps,
                         const float* cos_tab, const float* sin_tab, int max_pos, const int32_t* q_pos,
                         const int32_t* q_pos_base, int q_pos0, int causal, float sm_scale, void* stream) {
  // head_dim 256 (kernels/flash_attn.py:106): plain bf16 attention only
  const bool wide = D == 256;
  if (wide && (dtype != NQ_DTYPE_BF16 || q_weight || cos_tab || key_lens || bias || bt))
    return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim 256 takes bf16 q/k/v without QK-Norm/RoPE fusion, key lengths, "
                   "bias or paging");
  if (!wide && !head_dim_ok(D))
    return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256, got %d", D);
  if (!nq_dtype_ok(dtype)) return nq_fail(NQ_ERR_UNSUPPORTED, "unknown dtype code %d", dtype);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || T <= 0)
    return nq_fail(NQ_ERR_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d S=%d T=%d)", B, Hq, Hkv, S, T);
  if (Hq % Hkv) return nq_fail(NQ_ERR_INVALID, "num_heads %d not divisible by num_kv_heads %d", Hq, Hkv);
  const int G = Hq / Hkv;
  const bool f32 = dtype == NQ_DTYPE_F32;  // fp32 q, k, v, o: the fp32 MFMA kernel
  if (f32 && 128 % G) return nq_fail(NQ_ERR_UNSUPPORTED, "fp32: GQA group size %d must divide 128", G);
  if (!wide && PF_MAX_ROWS % G) return nq_fail(NQ_ERR_UNSUPPORTED, "GQA group size %d must divide %d", G, PF_MAX_ROWS);
  if (D == 32 && 128 % G)
    return nq_fail(NQ_ERR_UNSUPPORTED, "at head_dim 32 the GQA group size %d must divide 128", G);
  if (causal && S > T) return nq_fail(NQ_ERR_INVALID, "causal attention needs S <= T (S=%d T=%d)", S, T);
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return nq_fail(NQ_ERR_INVALID, "q, k, v, o and their strides are required");
  if (!nq_aligned16(q) || !nq_aligned16(k) || !nq_aligned16(v) || !nq_aligned16(o))
    return nq_fail(NQ_ERR_INVALID, "base pointers must be 16-byte aligned");
  const int esz = nq_dtype_size(dtype);
  for (const int64_t* s : {q_strides, k_strides, v_strides, o_strides})
    for (int i = 0; i < 3; ++i)
      if ((s[i] * esz) % 16) return nq_fail(NQ_ERR_INVALID, "strides must be multiples of 16 bytes");
  for (const int64_t* s : {k_strides, v_strides})  // a bf16 tile's lane offsets (64 rows) are 32-bit
    if (s[2] < 0 || (int64_t)PF_BN * s[2] * esz >= (1LL << 31))
      return nq_fail(NQ_ERR_UNSUPPORTED, "k/v sequence stride %lld too large", (long long)s[2]);
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  if (!nq_aligned16(cos_tab) || !nq_aligned16(sin_tab))  // their rows are DMA'd to LDS in 16-byte pieces
    return nq_fail(NQ_ERR_INVALID, "cos/sin tables must be 16-byte aligned");
  if (bias) {
    if (bt) return nq_fail(NQ_ERR_UNSUPPORTED, "an attention bias is taken with dense K/V only");
    if (!bias_strides) return nq_fail(NQ_ERR_INVALID, "the bias needs its strides");
    if (!f32 && 128 % G) return nq_fail(NQ_ERR_UNSUPPORTED, "with a bias the GQA group size %d must divide 128", G);
    // 8 consecutive keys per vector read
    if (!nq_aligned16(bias) || bias_strides[0] % 8 || bias_strides[1] % 8 || bias_strides[2] % 8 ||
        bias_strides[0] < 0 || bias_strides[1] < 0 || bias_strides[2] < 0)
      return nq_fail(NQ_ERR_INVALID, "the bias must be 16-byte aligned with non-negative strides that are multiples "
                     "of 8 elements");
  }
  PrefillParams p{};
  p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse;
  p.qsb = q_strides[0]; p.qsh = q_strides[1]; p.qss = q_strides[2];
  p.ksb = k_strides[0]; p.ksh = k_strides[1]; p.kss = k_strides[2];
  p.vsb = v_strides[0]; p.vsh = v_strides[1]; p.vss = v_strides[2];
  p.osb = o_strides[0]; p.osh = o_strides[1]; p.oss = o_strides[2];
  p.qw = q_weight; p.eps = eps; p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.q_pos = q_pos; p.q_pos_base = q_pos_base; p.q_pos0 = q_pos0;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = G; p.S = S; p.T = T;
  p.kv_lens = key_lens; p.kv_extra = 0; p.kv_max = T;
  p.bt = bt; p.bts = bts; p.page = page;
  p.bias = bias;
  if (bias) { p.bsb = bias_strides[0]; p.bsh = bias_strides[1]; p.bss = bias_strides[2]; }
  const float scale = sm_scale > 0.f ? sm_scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;
  const bool fuse = q_weight != nullptr || cos_tab != nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (wide) {
    p.BM = 64;
    p.nqb = (S + 63) / 64;
    if ((int64_t)p.nqb * B * Hq >= (1LL << 31))
      return nq_fail(NQ_ERR_UNSUPPORTED, "too many query blocks for one launch");
    return nq_check_launch(launch_prefill_wide(p, causal != 0, st));
  }
  if (f32) {
    p.BM = 128 / G;
    p.nqb = (S + p.BM - 1) / p.BM;
    return nq_check_launch(launch_prefill_f32(p, D, causal != 0, fuse, st));
  }
  // 256 rows per workgroup when that still gives enough workgroups, else 128
  const int64_t wide_wgs = (int64_t)B * Hkv * ((S + PF_MAX_ROWS / G - 1) / (PF_MAX_ROWS / G));
  // (a D = 32 tile is 4 KiB: one 1 KiB load per wave of a 4-wave workgroup,
  // too few for eight waves)
  const int nw = (128 % G == 0 && (wide_wgs < PF_WIDE_MIN_WGS || D == 32 || bias)) ? 4 : 8;
  p.BM = 32 * nw / G;
  p.nqb = (S + p.BM - 1) / p.BM;
  const hipError_t e =
      with_head_dim(D, [&](auto dc) { return launch_prefill<decltype(dc)::value, bf16>(p, nw, causal, fuse, st); });
  return nq_check_launch(e);
}

extern "C" int nq_attn_prefill_fwd(const void* q, const int64_t* q_strides, const void* k,
                                   const int64_t* k_strides, const void* v,
                                   const int64_t* v_strides, void* o, const int64_t* o_strides,
                                   float* lse, const int32_t* key_lens, int B, int Hq, int Hkv, int S,
                                   int T, int D,
                                   int dtype, const float* q_weight, float eps,
                                   const float* cos_tab, const float* sin_tab, int max_pos,
                                   const int32_t* q_pos, const int32_t* q_pos_base, int q_pos0,
                                   int causal, float sm_scale, void* stream) {
  nq_clear_error();
  return prefill_entry(q, q_strides, k, k_strides, v, v_strides, nullptr, 0, 0, nullptr, nullptr, o, o_strides, lse,
                       key_lens, B, Hq, Hkv, S, T, D, dtype, q_weight, eps, cos_tab, sin_tab, max_pos, q_pos,
                       q_pos_base, q_pos0, causal, sm_scale, stream);
}

extern "C" int nq_attn_prefill_bias_fwd(const void* q, const int64_t* q_strides, const void* k,
                                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                        void* o, const int64_t* o_strides, float* lse, const int32_t* key_lens,
                                        const void* bias, const int64_t* bias_strides, int B, int Hq, int Hkv,
                                        int S, int T, int D, int dtype, const float* q_weight, float eps,
                                        const float* cos_tab, const float* sin_tab, int max_pos,
                                        const int32_t* q_pos, const int32_t* q_pos_base, int q_pos0, int causal,
                                        float sm_scale, void* stream) {
  nq_clear_error();
  if (!bias) return nq_fail(NQ_ERR_INVALID, "nq_attn_prefill_bias_fwd needs the bias");
  return prefill_entry(q, q_strides, k, k_strides, v, v_strides, nullptr, 0, 0, bias, bias_strides, o, o_strides,
                       lse, key_lens, B, Hq, Hkv, S, T, D, dtype, q_weight, eps, cos_tab, sin_tab, max_pos, q_pos,
                       q_pos_base, q_pos0, causal, sm_scale, stream);
}

extern "C" int nq_attn_prefill_paged_fwd(const void* q, const int64_t* q_strides, const void* k_pool,
                                         const int64_t* k_pool_strides, const void* v_pool,
                                         const int64_t* v_pool_strides, const int32_t* block_table,
                                         int64_t bt_stride, int page_size, void* o,
                                         const int64_t* o_strides, float* lse, int B, int Hq, int Hkv,
                                         int S, int T, int D, int dtype, const float* q_weight,
                                         float eps, const float* cos_tab, const float* sin_tab,
                                         int max_pos, const int32_t* q_pos, const int32_t* q_pos_base,
                                         int q_pos0, int causal, float sm_scale, void* stream) {
  nq_clear_error();
  if (!block_table) return nq_fail(NQ_ERR_INVALID, "a paged prefill needs the block table");
  if (page_size <= 0 || page_size % 32)
    return nq_fail(NQ_ERR_UNSUPPORTED, "page_size must be a positive multiple of 32, got %d", page_size);
  if (T > 0 && bt_stride < (T + page_size - 1) / page_size)
    return nq_fail(NQ_ERR_INVALID, "bt_stride %lld holds fewer than the %d pages of T %d", (long long)bt_stride,
                   (T + page_size - 1) / page_size, T);
  return prefill_entry(q, q_strides, k_pool, k_pool_strides, v_pool, v_pool_strides, block_table, bt_stride,
                       page_size, nullptr, nullptr, o, o_strides, lse, nullptr, B, Hq, Hkv, S, T, D, dtype, q_weight,
                       eps, cos_tab, sin_tab, max_pos, q_pos, q_pos_base, q_pos0, causal, sm_scale, stream);
}
