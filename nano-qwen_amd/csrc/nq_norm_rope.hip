// Row kernel: RMSNorm over head_dim + rotate-half RoPE from an fp32 table,
// written to an arbitrary strided destination (a KV-cache slot or a buffer).
//
// Replaces, for the attention path of nano-qwen:
//   model/norm.py:17-22           RMSNorm used as QK-Norm (attention.py:95-97)
//   model/rope.py:133-161         apply_rotary_pos_emb (rotate-half pairing)
//   kernels/rope.py:99-108        apply_rope (in-place when src == dst)
//   model/attention.py:31-38      KVCache.update (rows land at row_base[b] + s)
//
// One launch processes up to three jobs (Q, K, V); V rows are copied (and
// converted) without arithmetic.  Layout: a row is D contiguous elements;
// (b, h, s) strides are free.  A row is handled by D/16 lanes: lane s of the
// row owns elements [8s, 8s+8) and their RoPE partners [D/2+8s, D/2+8s+8)
// (two 16-byte bf16 loads), so the rotation needs no cross-lane traffic; the
// norm's sum of squares is reduced over the row's lanes with DPP adds
// (row_half_mirror, then quad swaps), all VALU.  Rows are enumerated with the
// heads of one position adjacent when the source stores them so (a wave then
// reads contiguous memory and its rows share their cos/sin table rows, which
// matters when the tables outgrow the L2), else position-fastest.  The grid
// is persistent (as many blocks as stay resident) and loops over rows, one
// row per thread per pass; the weight and each row's table chunks reach the
// lanes through LDS by DMA.  HBM-bound: one read and one write per element;
// the weight and table reads hit the caches.

#include "nq_common.hpp"
#include "nq_internal.hpp"

namespace nq {

struct RowJob {
  const void* src;
  void* dst;
  int64_t sb, sh, ss;   // source strides (elements)
  int64_t db, dh, ds;   // destination strides (elements)
  const float* weight;  // RMSNorm weight (D) or null
  int H;
  int rope;             // apply RoPE
  int norm;             // apply RMSNorm
  int use_row_base;     // destination row = row_base[b] + s
  int heads_inner;      // source heads closer in memory than positions: rows run (b, s, h), h fastest
};

struct RowParams {
  RowJob job[3];
  int njobs;
  int B, S, D;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int max_pos;
  const int32_t* pos;
  const int32_t* pos_base;
  int pos0;
  const int32_t* row_base;
  int row0;
  // paged destination for row-base jobs: row t of sequence b lands in page
  // block_table[b * bt_stride + t / page_size], row t % page_size; the job's
  // destination strides are then (page, head, row)
  const int32_t* block_table;
  int64_t bt_stride;
  int page_size;
};

// An opaque zero (a VALU move the compiler cannot see through): added to the
// addresses of the per-row LDS reads so they stay inside the row loop;
// hoisted, the weight reads would hold 16 registers across every row's wait.
__device__ __forceinline__ int row_opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// LDS per wave: the norm weight (D fp32, staged once, 1 KiB slot), then the
// lanes' table chunks (cos lo / cos hi / sin lo / sin hi, 16 bytes per lane
// each: 4 KiB), refilled every row.
constexpr int ROW_WAVE_LDS = 5 * 1024;

// A persistent grid: as many blocks as stay resident (the occupancy of the
// instance times the CUs), each looping over rows, one row per thread per
// pass.  Per row a thread issues its two 16-byte row loads, then its table
// chunks as DMA into its wave's LDS slice, and waits once: the row and table
// latencies overlap, and the tables (and the weights) occupy no registers
// while in flight, which keeps the kernel at 7-8 waves per SIMD.
template <typename TI, typename TO, int D>
__global__ __launch_bounds__(256) void norm_rope_rows_kernel(RowParams p) {
  constexpr int LPR = D / 16;         // lanes per row
  constexpr int RPW = 64 / LPR;       // rows per wave
  constexpr int RPB = RPW * 4;        // rows per 256-thread block
  static_assert(LPR == 2 || LPR == 4 || LPR == 8, "D must be 32, 64 or 128");
  static_assert(D * 4 <= 1024, "the weight fits its 1 KiB slot");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[4 * ROW_WAVE_LDS];
  const RowJob& jb = p.job[blockIdx.y];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % LPR;         // chunk pair: [8sub, 8sub+8) and [D/2 + 8sub, ...)
  unsigned char* const wslot = smem + wave * ROW_WAVE_LDS;  // weight
  unsigned char* const tslot = wslot + 1024;                // table chunks
  const int64_t nrows = (int64_t)p.B * jb.H * p.S;
  // lane l stages weight values [4 (l % (D/4)), +4): the slot holds the
  // weight (repeated for D < 256); waited for with the first row
  if (jb.norm) global_load_lds16(jb.weight + (lane % (D / 4)) * 4, wslot);
  // explicit or per-batch positions need a load before the table row is known;
  // the plain pos0 + s form needs none (a separate loop, so no merged path
  // waits on a position load that was never issued)
  auto rows = [&](auto pos_arrays) {
    constexpr bool PA = decltype(pos_arrays)::value;
    for (int64_t row = (int64_t)blockIdx.x * RPB + wave * RPW + lane / LPR; row < nrows;
         row += (int64_t)gridDim.x * RPB) {
      // row -> (b, h, s): s fastest, or h fastest when the heads of one
      // position are adjacent in memory (the projections' (B, S, H, D)
      // storage): a wave then reads contiguous bytes and its rows share table rows
      const uint32_t rr = (uint32_t)row;
      int b, h, s;
      if (jb.heads_inner) {
        h = (int)(rr % (uint32_t)jb.H);
        const uint32_t t = rr / (uint32_t)jb.H;
        s = (int)(t % (uint32_t)p.S);
        b = (int)(t / (uint32_t)p.S);
      } else {
        s = (int)(rr % (uint32_t)p.S);
        const uint32_t t = rr / (uint32_t)p.S;
        h = (int)(t % (uint32_t)jb.H);
        b = (int)(t / (uint32_t)jb.H);
      }
      const int pos = jb.rope ? table_row(PA ? row_position(p.pos, p.pos_base, p.pos0, b, s, p.S) : p.pos0 + s,
                                          p.max_pos)
                              : 0;
      // destination (a cache row base or a page is a load of its own)
      const int drow = jb.use_row_base ? ((p.row_base ? p.row_base[b] : p.row0) + s) : s;
      int64_t slab = b, prow = drow;
      if (jb.use_row_base && p.block_table) {
        slab = p.block_table[b * p.bt_stride + drow / p.page_size];
        prow = drow % p.page_size;
      }
      const TI* src = reinterpret_cast<const TI*>(jb.src) + b * jb.sb + h * jb.sh + s * jb.ss + sub * 8;
      floatx8 x1 = Vec8<TI>::load_f32(src);
      floatx8 x2 = Vec8<TI>::load_f32(src + D / 2);
      if (jb.rope) {
        // a position outside the tables reads row 0 and gives NaN (below)
        const int64_t toff = (int64_t)(pos < 0 ? 0 : pos) * (D / 2) + sub * 8;
        global_load_lds16(p.cos_tab + toff, tslot);
        global_load_lds16(p.cos_tab + toff + 4, tslot + 1024);
        global_load_lds16(p.sin_tab + toff, tslot + 2048);
        global_load_lds16(p.sin_tab + toff + 4, tslot + 3072);
      }
      wait_vmcnt0();
      const int z = row_opaque_zero();
      if (jb.norm) {
        const unsigned char* w = wslot + z + sub * 32;
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(w);
        const floatx4 a1 = *reinterpret_cast<const floatx4*>(w + 16);
        const floatx4 b0 = *reinterpret_cast<const floatx4*>(w + D * 2);
        const floatx4 b1 = *reinterpret_cast<const floatx4*>(w + D * 2 + 16);
        const floatx8 w1{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const floatx8 w2{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        norm_row<D>(x1, x2, w1, w2, p.eps);
      }
      if (jb.rope) {
        const unsigned char* t = tslot + z + lane * 16;
        const floatx4 c0 = *reinterpret_cast<const floatx4*>(t);
        const floatx4 c1 = *reinterpret_cast<const floatx4*>(t + 1024);
        const floatx4 s0 = *reinterpret_cast<const floatx4*>(t + 2048);
        const floatx4 s1 = *reinterpret_cast<const floatx4*>(t + 3072);
        const float nan = __builtin_nanf("");
        floatx8 c, sn;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c[e] = pos < 0 ? nan : c0[e];
          c[e + 4] = pos < 0 ? nan : c1[e];
          sn[e] = pos < 0 ? nan : s0[e];
          sn[e + 4] = pos < 0 ? nan : s1[e];
        }
        rope_row(x1, x2, c, sn);
      }
      TO* dst = reinterpret_cast<TO*>(jb.dst) + slab * jb.db + h * jb.dh + prow * jb.ds + sub * 8;
      store8<TO>(dst, x1);
      store8<TO>(dst + D / 2, x2);
    }
  };
  if (p.pos || p.pos_base) rows(std::true_type{});
  else rows(std::false_type{});
}

template <typename TI, typename TO, int D>
static hipError_t launch_rows(const RowParams& p, int max_h, hipStream_t st) {
  constexpr int RPB = (64 / (D / 16)) * 4;  // rows per block and pass
  auto kern = norm_rope_rows_kernel<TI, TO, D>;
  // resident blocks of this instance, worked out once per device
  static int resident[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int cap = (dev >= 0 && dev < 64) ? __atomic_load_n(&resident[dev], __ATOMIC_RELAXED) : 0;
  if (cap == 0) {
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), 256, 0);
    if (e != hipSuccess) return e;
    cap = (cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
    if (dev >= 0 && dev < 64) __atomic_store_n(&resident[dev], cap, __ATOMIC_RELAXED);
  }
  const int64_t nrows = (int64_t)p.B * max_h * p.S;
  const int64_t blocks = (nrows + RPB - 1) / RPB;
  dim3 grid((unsigned)(blocks < cap ? blocks : cap), (unsigned)p.njobs);
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace nq

using namespace nq;

static int qk_norm_rope_impl(const void* q, const int64_t* q_strides, void* q_out,
                             const int64_t* q_out_strides, const void* k, const int64_t* k_strides,
                             void* k_out, const int64_t* k_out_strides, const void* v,
                             const int64_t* v_strides, void* v_out, const int64_t* v_out_strides,
                             int B, int S, int Hq, int Hkv, int D, int dtype_in, int dtype_out,
                             const float* q_weight, const float* k_weight, float eps,
                             const float* cos_tab, const float* sin_tab, int max_pos,
                             const int32_t* pos, const int32_t* pos_base, int pos0,
                             const int32_t* kv_row_base, int kv_row0, const int32_t* block_table,
                             int64_t bt_stride, int page_size, void* stream) {
  nq_clear_error();
  if (!head_dim_ok(D)) return nq_fail(NQ_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128, got %d", D);
  if (B <= 0 || S <= 0) return nq_fail(NQ_ERR_INVALID, "B and S must be positive (B=%d S=%d)", B, S);
  if (!nq_dtype_ok(dtype_in) || !nq_dtype_ok(dtype_out))
    return nq_fail(NQ_ERR_UNSUPPORTED, "dtype codes must be NQ_DTYPE_BF16 or NQ_DTYPE_F32");
  if ((cos_tab == nullptr) != (sin_tab == nullptr) || (cos_tab && max_pos <= 0))
    return nq_fail(NQ_ERR_INVALID, "cos and sin tables go together, with max_pos > 0");
  // the tables and the norm weights reach LDS in 16-byte DMA pieces
  if (!nq_aligned16(cos_tab) || !nq_aligned16(sin_tab) || !nq_aligned16(q_weight) || !nq_aligned16(k_weight))
    return nq_fail(NQ_ERR_INVALID, "cos/sin tables and norm weights must be 16-byte aligned");
  const int esz_in = nq_dtype_size(dtype_in), esz_out = nq_dtype_size(dtype_out);
  RowParams p{};
  p.B = B; p.S = S; p.D = D; p.eps = eps;
  p.block_table = block_table; p.bt_stride = bt_stride; p.page_size = page_size;
  p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.max_pos = max_pos;
  p.pos = pos; p.pos_base = pos_base; p.pos0 = pos0;
  p.row_base = kv_row_base; p.row0 = kv_row0;
  int nj = 0, max_h = 0;
  struct In { const void* s; const int64_t* ss; void* d; const int64_t* ds; int H; const float* w; int rope; int rb; const char* name; };
  In ins[3] = {{q, q_strides, q_out, q_out_strides, Hq, q_weight, 1, 0, "q"},
               {k, k_strides, k_out, k_out_strides, Hkv, k_weight, 1, 1, "k"},
               {v, v_strides, v_out, v_out_strides, Hkv, nullptr, 0, 1, "v"}};
  for (const In& in : ins) {
    if (!in.s) continue;
    if (!in.d || !in.ss || !in.ds) return nq_fail(NQ_ERR_INVALID, "%s: output and strides required", in.name);
    if (in.H <= 0) return nq_fail(NQ_ERR_INVALID, "%s: head count must be positive", in.name);
    if (!nq_aligned16(in.s) || !nq_aligned16(in.d))
      return nq_fail(NQ_ERR_INVALID, "%s: base pointers must be 16-byte aligned", in.name);
    for (int i = 0; i < 3; ++i) {
      if ((in.ss[i] * esz_in) % 16 || (in.ds[i] * esz_out) % 16)
        return nq_fail(NQ_ERR_INVALID, "%s: strides must be multiples of 16 bytes", in.name);
    }
    RowJob& j = p.job[nj++];
    j.src = in.s; j.dst = in.d;
    j.sb = in.ss[0]; j.sh = in.ss[1]; j.ss = in.ss[2];
    j.db = in.ds[0]; j.dh = in.ds[1]; j.ds = in.ds[2];
    j.weight = in.w; j.H = in.H; j.rope = in.rope && cos_tab != nullptr; j.norm = in.w != nullptr;
    j.use_row_base = in.rb;
    j.heads_inner = in.H > 1 && S > 1 && (in.ss[1] < 0 ? -in.ss[1] : in.ss[1]) < (in.ss[2] < 0 ? -in.ss[2] : in.ss[2]);
    if (in.H > max_h) max_h = in.H;
  }
  if (nj == 0) return NQ_OK;
  if ((int64_t)B * max_h * S >= (1LL << 31))
    return nq_fail(NQ_ERR_UNSUPPORTED, "B * heads * S must stay below 2^31 rows");
  p.njobs = nj;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool bi = dtype_in == NQ_DTYPE_BF16, bo = dtype_out == NQ_DTYPE_BF16;
#define NQ_ROWS(TI, TO) \
  e = with_head_dim(D, [&](auto dc) { return launch_rows<TI, TO, decltype(dc)::value>(p, max_h, st); })
  if (bi && bo) NQ_ROWS(bf16, bf16);
  else if (bi && !bo) NQ_ROWS(bf16, float);
  else if (!bi && bo) NQ_ROWS(float, bf16);
  else NQ_ROWS(float, float);
#undef NQ_ROWS
  return nq_check_launch(e);
}

extern "C" int nq_qk_norm_rope(const void* q, const int64_t* q_strides, void* q_out,
                               const int64_t* q_out_strides, const void* k,
                               const int64_t* k_strides, void* k_out,
                               const int64_t* k_out_strides, const void* v,
                               const int64_t* v_strides, void* v_out,
                               const int64_t* v_out_strides, int B, int S, int Hq, int Hkv,
                               int D, int dtype_in, int dtype_out, const float* q_weight,
                               const float* k_weight, float eps, const float* cos_tab,
                               const float* sin_tab, int max_pos, const int32_t* pos,
                               const int32_t* pos_base, int pos0,
                               const int32_t* kv_row_base, int kv_row0, void* stream) {
  return qk_norm_rope_impl(q, q_strides, q_out, q_out_strides, k, k_strides, k_out, k_out_strides, v,
                           v_strides, v_out, v_out_strides, B, S, Hq, Hkv, D, dtype_in, dtype_out,
                           q_weight, k_weight, eps, cos_tab, sin_tab, max_pos, pos, pos_base, pos0,
                           kv_row_base, kv_row0, nullptr, 0, 0, stream);
}

extern "C" int nq_kv_append_paged(const void* k, const int64_t* k_strides, const void* v,
                                  const int64_t* v_strides, void* k_pool,
                                  const int64_t* k_pool_strides, void* v_pool,
                                  const int64_t* v_pool_strides, const int32_t* block_table,
                                  int64_t bt_stride, int page_size, int B, int S, int Hkv, int D,
                                  int dtype_in, int dtype_out, const float* k_weight, float eps,
                                  const float* cos_tab, const float* sin_tab, int max_pos,
                                  const int32_t* pos, const int32_t* pos_base, int pos0,
                                  const int32_t* row_base, int row0, void* stream) {
  if (!block_table || page_size <= 0 || bt_stride <= 0) {
    nq_clear_error();
    return nq_fail(NQ_ERR_INVALID, "a block table, bt_stride > 0 and page_size > 0 are required");
  }
  if (!k && !v) {
    nq_clear_error();
    return nq_fail(NQ_ERR_INVALID, "nothing to append (k and v are both null)");
  }
  return qk_norm_rope_impl(nullptr, nullptr, nullptr, nullptr, k, k_strides, k_pool, k_pool_strides, v,
                           v_strides, v_pool, v_pool_strides, B, S, 0, Hkv, D, dtype_in, dtype_out,
                           nullptr, k_weight, eps, cos_tab, sin_tab, max_pos, pos, pos_base, pos0,
                           row_base, row0, block_table, bt_stride, page_size, stream);
}

// ---------------------------------------------------------------- RMSNorm
// RMSNorm.forward of model/norm.py:17-22 over rows of any width (a multiple
// of 8): y = round_x(x * rsqrt(mean(x^2) + eps)) * w, where round_x is the
// cast back to the input dtype (`.type_as(x)`) and the product is formed in
// fp32 and stored in the promoted dtype of x and w -- the reference's cast
// order and dtype promotion.  One wave per row; lane l holds the 8-element
// chunks l, l + 64, ...; the sum of squares is a wave reduction.
namespace nq {

struct RmsParams {
  const void* x;
  int64_t xs;  // row stride (elements)
  const void* w;
  void* y;
  int64_t ys;
  int64_t rows;
  int width;
  float eps;
};

template <typename T>
__device__ __forceinline__ float round_to(float v) {
  return (float)(T)v;
}

template <typename TI, typename TW, typename TO>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(RmsParams p) {
  const int lane = threadIdx.x & 63;
  const int nch = p.width / 8;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += (int64_t)gridDim.x * 4) {
    const TI* xr = reinterpret_cast<const TI*>(p.x) + row * p.xs;
    float ss = 0.f;
    for (int c = lane; c < nch; c += 64) {
      const floatx8 v = Vec8<TI>::load_f32(xr + c * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float r = rsqrtf(ss / (float)p.width + p.eps);
    TO* yr = reinterpret_cast<TO*>(p.y) + row * p.ys;
    for (int c = lane; c < nch; c += 64) {
      const floatx8 v = Vec8<TI>::load_f32(xr + c * 8);
      const floatx8 wv = Vec8<TW>::load_f32(reinterpret_cast<const TW*>(p.w) + c * 8);
      floatx8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = round_to<TI>(v[e] * r) * wv[e];
      store8<TO>(yr + c * 8, o);
    }
  }
}

}  // namespace nq

extern "C" int nq_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, void* y,
                          int64_t y_row_stride, int64_t rows, int width, int dtype_x, int dtype_w,
                          int dtype_y, float eps, void* stream) {
  nq_clear_error();
  if (!nq_dtype_ok(dtype_x) || !nq_dtype_ok(dtype_w) || !nq_dtype_ok(dtype_y))
    return nq_fail(NQ_ERR_UNSUPPORTED, "dtype codes must be NQ_DTYPE_BF16 or NQ_DTYPE_F32");
  // the promoted dtype: fp32 unless both x and w are bf16
  const int promoted = (dtype_x == NQ_DTYPE_BF16 && dtype_w == NQ_DTYPE_BF16) ? NQ_DTYPE_BF16 : NQ_DTYPE_F32;
  if (dtype_y != promoted)
    return nq_fail(NQ_ERR_INVALID, "y must have the promoted dtype of x and weight (code %d)", promoted);
  if (rows < 0 || width <= 0 || width % 8)
    return nq_fail(NQ_ERR_UNSUPPORTED, "width must be a positive multiple of 8, got %d", width);
  if (rows == 0) return NQ_OK;
  if (!x || !weight || !y) return nq_fail(NQ_ERR_INVALID, "x, weight and y are required");
  if (!nq_aligned16(x) || !nq_aligned16(weight) || !nq_aligned16(y))
    return nq_fail(NQ_ERR_INVALID, "base pointers must be 16-byte aligned");
  if ((x_row_stride * nq_dtype_size(dtype_x)) % 16 || (y_row_stride * nq_dtype_size(dtype_y)) % 16)
    return nq_fail(NQ_ERR_INVALID, "row strides must be multiples of 16 bytes");
  RmsParams p{x, x_row_stride, weight, y, y_row_stride, rows, width, eps};
  const int64_t blocks = (rows + 3) / 4;
  const dim3 grid((unsigned)(blocks < 2048 ? blocks : 2048));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool bx = dtype_x == NQ_DTYPE_BF16, bw = dtype_w == NQ_DTYPE_BF16;
  if (bx && bw) hipLaunchKernelGGL((rmsnorm_rows_kernel<bf16, bf16, bf16>), grid, dim3(256), 0, st, p);
  else if (bx) hipLaunchKernelGGL((rmsnorm_rows_kernel<bf16, float, float>), grid, dim3(256), 0, st, p);
  else if (bw) hipLaunchKernelGGL((rmsnorm_rows_kernel<float, bf16, float>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((rmsnorm_rows_kernel<float, float, float>), grid, dim3(256), 0, st, p);
  return nq_check_launch(hipGetLastError());
}
