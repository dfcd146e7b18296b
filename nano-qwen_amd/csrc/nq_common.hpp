// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Storage types are bf16 (clang __bf16) or fp32; all arithmetic that is not
// an MFMA runs in fp32.  Vector loads are 16 bytes per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace nq {

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- MFMA
// v_mfma_f32_32x32x16_bf16: A 32x16, B 16x32, C/D 32x32 fp32.
//   A: lane l holds row (l % 32), k = (l / 32) * 8 + [0, 8)
//   B: lane l holds col (l % 32), k = (l / 32) * 8 + [0, 8)
//   D: lane l holds col (l % 32), rows (i / 4) * 8 + (l / 32) * 4 + (i % 4), i < 16
__device__ __forceinline__ floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x32_bf16: A 16x32, B 32x16, C/D 16x16 fp32.
//   A: lane l holds row (l % 16), k = (l / 16) * 8 + [0, 8)
//   B: lane l holds col (l % 16), k = (l / 16) * 8 + [0, 8)
//   D: lane l holds col (l % 16), rows (l / 16) * 4 + i, i < 4
__device__ __forceinline__ floatx4 mfma16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- loads
// 8 consecutive elements starting at p (16-byte aligned for bf16, 32 for fp32).
template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  __device__ __forceinline__ static floatx8 load_f32(const bf16* p) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
    return __builtin_convertvector(v, floatx8);
  }
  __device__ __forceinline__ static bf16x8 load_bf16(const bf16* p) {
    return *reinterpret_cast<const bf16x8*>(p);
  }
  // streaming (read-once) data: nontemporal load
  __device__ __forceinline__ static bf16x8 load_bf16_nt(const bf16* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
  }
};
template <> struct Vec8<float> {
  __device__ __forceinline__ static floatx8 load_f32(const float* p) {
    floatx4 a = *reinterpret_cast<const floatx4*>(p);
    floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
    return floatx8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
  __device__ __forceinline__ static bf16x8 load_bf16(const float* p) {
    return __builtin_convertvector(load_f32(p), bf16x8);
  }
  __device__ __forceinline__ static bf16x8 load_bf16_nt(const float* p) {
    floatx4 a = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p));
    floatx4 b = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p + 4));
    return __builtin_convertvector((floatx8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}), bf16x8);
  }
};

__device__ __forceinline__ bf16x8 to_bf16x8(floatx8 v) { return __builtin_convertvector(v, bf16x8); }

// ---------------------------------------------------------------- LDS
// gfx950 LDS: 64 banks x 4 bytes (256 B per clock).  A ds_read_b128 serves 16
// lanes per clock, a ds_read_b64 (and the transpose read) 32 lanes per clock.
typedef short shortx4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16.  Within each group of 16 lanes, source lane j supplies
// the address of 4 consecutive 16-bit values M[j][0..3]; destination lane i
// receives (M[i/4][i%4], M[4+i/4][i%4], M[8+i/4][i%4], M[12+i/4][i%4]).
// Pointing source lane j at row r0 + j/4, column c0 + 4*(j%4) of a row-major
// tile hands destination lane i the column c0 + i of rows r0 .. r0+3.
__device__ __forceinline__ shortx4 lds_read_tr4(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) shortx4*)(const_cast<bf16*>(p)));
}

// Two transpose reads (rows r0..r0+3 and r0+4..r0+7 of one column) as one
// 8-element MFMA operand.
__device__ __forceinline__ bf16x8 lds_read_tr8(const bf16* p_lo, const bf16* p_hi) {
  shortx4 a = lds_read_tr4(p_lo);
  shortx4 b = lds_read_tr4(p_hi);
  typedef short shortx8 __attribute__((ext_vector_type(8)));
  shortx8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, ab);
}

// The same transpose read issued as inline asm.  The compiler treats the
// builtin as an LDS access it cannot tell apart from pending HBM->LDS loads
// (global_load_lds) and puts s_waitcnt vmcnt(0) in front of it; a caller that
// knows the tile it reads has landed uses this form and waits for the result
// itself with lgkm_wait (the compiler does not track these reads).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char*)(p)));
}
template <int OFF>
__device__ __forceinline__ shortx4 lds_read_tr4_nowait(uint32_t addr) {
  shortx4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}
// A plain 16-byte LDS read issued the same way (waited for with lgkm_wait).
template <int OFF>
__device__ __forceinline__ bf16x8 lds_read_b128_nowait(uint32_t addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}
// rows r0..r0+3 at addr and r0+4..r0+7 at addr + HI bytes, as one operand
template <int HI>
__device__ __forceinline__ bf16x8 lds_read_tr8_nowait(uint32_t addr) {
  shortx4 a = lds_read_tr4_nowait<0>(addr);
  shortx4 b = lds_read_tr4_nowait<HI>(addr);
  typedef short shortx8 __attribute__((ext_vector_type(8)));
  shortx8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, ab);
}
// s_waitcnt lgkmcnt(N) (gfx9 encoding: vmcnt and expcnt left at their
// maximum), fenced so that nothing is scheduled across it.  Valid when every
// LDS access still outstanding is younger than the reads being waited for.
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// global_load_lds_dwordx4: lane t copies 16 bytes from its global address to
// LDS at lds + 16*t (lds must be wave-uniform; it is passed through M0).
// Completion is tracked by vmcnt.  (Kept in a non-template function: naming
// the builtin directly inside a kernel template made the host pass drop that
// kernel's launch stubs.)
__device__ __forceinline__ void global_load_lds16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// Raw buffer descriptor over `bytes` bytes at `base` (stride 0; gfx9 word 3).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// buffer_load_dwordx4 ... lds: lane t copies 16 bytes from the descriptor's
// base + soff + voff to LDS at lds + 16*t (lds wave-uniform, through M0).
// Completion is tracked by vmcnt, like global_load_lds.
__device__ __forceinline__ void buffer_load_lds16(BufRsrc r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// s_waitcnt vmcnt(0): all of this wave's vector-memory loads (including
// global_load_lds) have completed.
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x3f70); }
// s_waitcnt vmcnt(N): all but this wave's N most recent vector-memory
// instructions have completed (loads complete in order).  gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt and lgkmcnt left at their maximum.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

template <typename T>
__device__ __forceinline__ void store8(T* p, floatx8 v);
template <>
__device__ __forceinline__ void store8<bf16>(bf16* p, floatx8 v) {
  *reinterpret_cast<bf16x8*>(p) = __builtin_convertvector(v, bf16x8);
}
template <>
__device__ __forceinline__ void store8<float>(float* p, floatx8 v) {
  *reinterpret_cast<floatx4*>(p) = floatx4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<floatx4*>(p + 4) = floatx4{v[4], v[5], v[6], v[7]};
}

template <typename T>
__device__ __forceinline__ void store2(T* p, float a, float b) {
  p[0] = (T)a;
  p[1] = (T)b;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, floatx4 v);
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, floatx4 v) {
  *reinterpret_cast<bf16x4*>(p) = __builtin_convertvector(v, bf16x4);
}
template <>
__device__ __forceinline__ void store4<float>(float* p, floatx4 v) {
  *reinterpret_cast<floatx4*>(p) = v;
}

// ---------------------------------------------------------------- lanes
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// max / sum of lanes l and l^32 with v_permlane32_swap (a VALU op; __shfl_xor
// goes through the LDS crossbar).  swap(x, x) leaves (x[l], x[l+32]) in lanes
// l < 32 and (x[l-32], x[l]) in lanes l >= 32.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// c + the sum of the 8 bf16 values of v, in fp32, with v_dot2_f32_bf16 against
// (1, 1): four VALU ops for 8 values, exact products, fp32 sums.
__device__ __forceinline__ float rowsum_bf16x8(bf16x8 v, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), ones, c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), ones, c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), ones, c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), ones, c, false);
  return c;
}

// Sum over groups of LPR = 2, 4 or 8 consecutive lanes with DPP (all VALU).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  static_assert(LPR == 2 || LPR == 4 || LPR == 8, "groups of 2, 4 or 8 lanes");
  if (LPR == 8) {  // lane i <- lane 7-i within each group of 8
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  }
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad xor 1
  if (LPR >= 4)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad xor 2
  return v;
}

// Head dims every kernel is built for, and the host-side switch that calls
// f(std::integral_constant<int, D>) for the one asked for.
constexpr bool head_dim_ok(int D) { return D == 32 || D == 64 || D == 128; }
template <typename F>
inline auto with_head_dim(int D, F&& f) {
  if (D == 32) return f(std::integral_constant<int, 32>{});
  if (D == 64) return f(std::integral_constant<int, 64>{});
  return f(std::integral_constant<int, 128>{});
}

// RoPE table row of position p: p itself when 0 <= p < max_pos, else -1.
// Rows at an out-of-range position rotate with NaN cos/sin, so every value
// they reach comes out NaN (the reference's table lookup, model/rope.py:128,
// fails on such positions; callers that know positions on the host check them
// there).
__device__ __forceinline__ int table_row(int p, int max_pos) { return (p >= 0 && p < max_pos) ? p : -1; }
// 8 consecutive table values of row `row` (from table_row) at column `col`
// of a table with `width` columns; NaN for row -1.
__device__ __forceinline__ floatx8 load_tab8(const float* tab, int row, int width, int col) {
  if (row < 0) {
    const float n = __builtin_nanf("");
    return floatx8{n, n, n, n, n, n, n, n};
  }
  return Vec8<float>::load_f32(tab + (int64_t)row * width + col);
}

// One head_dim row held by D/16 lanes: lane `sub` owns elements [8sub, 8sub+8)
// (x1) and their rotate-half partners [D/2 + 8sub, D/2 + 8sub + 8) (x2).
// RMSNorm with weight halves w1/w2 (when w1 is given), then RoPE with the
// fp32 table row at `pos` (when cos_tab is given).  The same arithmetic, in
// the same order, serves every kernel that writes a K-hat row.
// The fused multiply-adds are written out so that every kernel that inlines
// these rounds exactly alike (the compiler's own contraction may differ from
// one context to the next).
template <int D>
__device__ __forceinline__ void norm_row(floatx8& x1, floatx8& x2, const floatx8& w1, const floatx8& w2,
                                         float eps) {
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sq = __builtin_fmaf(x1[e], x1[e], sq);
    sq = __builtin_fmaf(x2[e], x2[e], sq);
  }
  sq = row_sum<D / 16>(sq);
  const float r = rsqrtf(sq / (float)D + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x1[e] = x1[e] * r * w1[e];
    x2[e] = x2[e] * r * w2[e];
  }
}
__device__ __forceinline__ void rope_row(floatx8& x1, floatx8& x2, const floatx8& c, const floatx8& sn) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = x1[e], b = x2[e];
    x1[e] = __builtin_fmaf(a, c[e], -(b * sn[e]));
    x2[e] = __builtin_fmaf(b, c[e], a * sn[e]);
  }
}
template <int D>
__device__ __forceinline__ void norm_rope_row(floatx8& x1, floatx8& x2, const floatx8* w1, const floatx8* w2,
                                              float eps, const float* cos_tab, const float* sin_tab, int pos,
                                              int sub) {
  if (w1) norm_row<D>(x1, x2, *w1, *w2, eps);
  if (cos_tab) {
    const floatx8 c = load_tab8(cos_tab, pos, D / 2, sub * 8);
    const floatx8 sn = load_tab8(sin_tab, pos, D / 2, sub * 8);
    rope_row(x1, x2, c, sn);
  }
}

// An element of a read-only input (the address space says the kernel never
// writes it): a wave-uniform index reads through the scalar path (s_load), a
// per-lane one still becomes a vector load.  As a vector load, a conditional
// wave-uniform read like pos_base[b] left an s_waitcnt vmcnt(0) where its
// paths merged, which drained every tile load issued before it.
__device__ __forceinline__ int32_t ld_uniform(const int32_t* base, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)base)[i];
}

// Position of (b, s): explicit positions win, else base[b] + s, else pos0 + s.
__device__ __forceinline__ int row_position(const int32_t* pos, const int32_t* pos_base, int pos0,
                                            int b, int s, int S) {
  if (pos) return pos[(int64_t)b * S + s];
  return (pos_base ? ld_uniform(pos_base, b) : pos0) + s;
}


}  // namespace nq
