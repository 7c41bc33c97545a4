// Shared device helpers for the gfx950 paged-attention kernels.
//
// Lane layouts of the bf16 MFMA instructions used here (checked on gfx950 by
// comparing against a host matmul):
//   v_mfma_f32_16x16x32_bf16: A[m][k]: lane l holds m = l%16, k = 8*(l/16)+i
//                             B[k][n]: lane l holds n = l%16, k = 8*(l/16)+i
//                             C[m][n]: lane l holds n = l%16, m = 4*(l/16)+i
//   v_mfma_f32_32x32x16_bf16: A: m = l%32, k = 8*(l/32)+i
//                             B: n = l%32, k = 8*(l/32)+i
//                             C: n = l%32, m = 8*(i/4) + 4*(l/32) + i%4
// The reduction index k only has to agree between A and B, so kernels are
// free to permute which data sits in which k slot.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 16-byte global load / store through plain vector memory instructions.
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ u32x2 ld8(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}

// Two OCP float8 e4m3fn codes (bytes 0,1 of x, or bytes 2,3 with hi) to two
// bf16 in one dword, low byte to the low half; exact (every e4m3 value is a
// bf16 value).
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t x, bool hi) {
  const auto r = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)x, 1.0f, true)
                    : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)x, 1.0f, false);
  return __builtin_bit_cast(uint32_t, r);
}

// Eight e4m3 codes (one u32x2) to eight bf16 (one u32x4), in order.
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(const u32x2& c) {
  return u32x4{fp8x2_to_bf16x2(c[0], false), fp8x2_to_bf16x2(c[0], true), fp8x2_to_bf16x2(c[1], false),
               fp8x2_to_bf16x2(c[1], true)};
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) {
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ u32x4 as_u32x4(const bf16x8& v) {
  return __builtin_bit_cast(u32x4, v);
}

// bf16 bit pattern <-> float.  The float->bf16 direction rounds to nearest
// even (the hardware conversion of the __bf16 type on gfx950).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

// Two floats -> one packed bf16 pair (a single v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Codes of 1-byte quantized pages (the code_type argument of pa_decode_quant
// and pa_prefill_quant): OCP float8 e4m3fn, or integers.  The reference casts
// pages of any dtype to q's dtype before the dot (decode_paged_attention.py:
// 72-75, prefill_paged_attention.py:84-85), so int8 / uint8 codes are the
// integers -128..127 / 0..255, exact in bf16.
constexpr int kCodeE4M3 = 0;
constexpr int kCodeI8 = 1;
constexpr int kCodeU8 = 2;

// Eight 1-byte codes (one u32x2, byte 0 first) to eight bf16 (one u32x4), in
// order, exactly.  Integers: v_cvt_f32_ubyte per byte (int8 flips the sign
// bit first, so the byte reads code + 128, then subtracts 128), two per pack.
template <int kCode>
__device__ __forceinline__ u32x4 codes8_to_bf16x8(const u32x2& c) {
  if constexpr (kCode == kCodeE4M3) {
    return fp8x8_to_bf16x8(c);
  } else {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t w = kCode == kCodeI8 ? c[i] ^ 0x80808080u : c[i];
      const float bias = kCode == kCodeI8 ? 128.f : 0.f;
      const float f0 = (float)(w & 0xffu) - bias, f1 = (float)((w >> 8) & 0xffu) - bias;
      const float f2 = (float)((w >> 16) & 0xffu) - bias, f3 = (float)(w >> 24) - bias;
      r[2 * i] = pack_bf16x2(f0, f1);
      r[2 * i + 1] = pack_bf16x2(f2, f3);
    }
    return r;
  }
}

// Value of `x` in lane l^32 / l^16 combined with the own value.  permlane
// swaps exchange halves of two registers; passing the same register twice
// yields (own, partner) in some order in every lane.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Soft-capped logit in log2 units, cap * log2 e * tanh(x * scale / cap),
// from tanh(y) = 1 - 2 / (e^(2y) + 1): c - 2c / (2^(x * s2) + 1) with
// s2 = 2 log2(e) scale / cap and c = cap log2 e (soft_cap_s2, soft_cap_c).  One
// v_exp_f32 and one v_rcp_f32 (about 1 ulp each) instead of the library
// tanhf; for large |y| the power is +inf or 0 and the result exactly +-c.
// The absolute error is a few 2^-24 c, below the bf16 rounding of P.
__device__ __forceinline__ float soft_cap_log2(float x, float s2, float c) {
  return c - (2.f * c) * __builtin_amdgcn_rcpf(fast_exp2(x * s2) + 1.f);
}
// The same minus an offset m: (c - m) - 2c / (2^(x * s2) + 1), with
// two_c = 2c and cm = c - m, so that logits relative to a reference max
// cost no extra subtraction.
__device__ __forceinline__ float soft_cap_log2_rel(float x, float s2, float two_c, float cm) {
  return cm - two_c * __builtin_amdgcn_rcpf(fast_exp2(x * s2) + 1.f);
}
__device__ __forceinline__ float soft_cap_s2(float logit_scale, float cap) {
  return 2.f * kLog2e * logit_scale / cap;
}
__device__ __forceinline__ float soft_cap_c(float cap) { return cap * kLog2e; }

// Exclusive scan over the workgroup (blockDim.x == kScanThreads) of one
// value per thread; `tmp` is kScanThreads ints of LDS.  Returns the sum of
// the values of lower threads; `total` receives the sum of all.
template <int kScanThreads>
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int& total) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  for (int o = 1; o < kScanThreads; o <<= 1) {
    __syncthreads();
    const int u = tid >= o ? tmp[tid - o] : 0;
    __syncthreads();
    tmp[tid] += u;
  }
  __syncthreads();
  total = tmp[kScanThreads - 1];
  const int excl = tmp[tid] - v;
  __syncthreads();
  return excl;
}

// Max and min of `mx` / `mn` over the 32 lanes of each wave half (lanes i
// and i ^ k, k < 32), in VALU: two quad permutations, the 8- and 16-lane
// row mirrors (DPP), then one permlane16 swap.  Every lane ends with the
// result of its half.
template <int kCtrl>
__device__ __forceinline__ void minmax_dpp(int& mx, int& mn) {
  mx = max(mx, __builtin_amdgcn_update_dpp(mx, mx, kCtrl, 0xF, 0xF, false));
  mn = min(mn, __builtin_amdgcn_update_dpp(mn, mn, kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ void minmax32(int& mx, int& mn) {
  minmax_dpp<0xB1>(mx, mn);   // quad_perm(1, 0, 3, 2)
  minmax_dpp<0x4E>(mx, mn);   // quad_perm(2, 3, 0, 1)
  minmax_dpp<0x141>(mx, mn);  // row_half_mirror
  minmax_dpp<0x140>(mx, mn);  // row_mirror
  const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)mx, (uint32_t)mx, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap((uint32_t)mn, (uint32_t)mn, false, false);
  mx = max((int)a[0], (int)a[1]);
  mn = min((int)b[0], (int)b[1]);
}

// acc + lo + hi of a packed bf16 pair (v_dot2c_f32_bf16 against (1, 1)).
__device__ __forceinline__ float dot2_bf16_ones(uint32_t pair, float acc) {
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), ones, acc, false);
}

// Physical page of logical page `lp` of a sequence: negative ids (padding
// entries of the block table) read page 0, ids past the pool are clamped so
// that no access leaves the pool.
__device__ __forceinline__ int32_t safe_page(const int32_t* __restrict__ bt_row, int lp, int num_pages) {
  int32_t p = bt_row[lp];
  p = p < 0 ? 0 : p;
  return p >= num_pages ? num_pages - 1 : p;
}

// safe_page through the scalar cache: for a wave-uniform `lp` this is an
// s_load (counted by lgkmcnt), so it never waits behind outstanding vector
// loads.  The block table is read-only for the duration of every kernel.
__device__ __forceinline__ int32_t safe_page_scalar(const int32_t* __restrict__ bt_row, int lp, int num_pages) {
  const __attribute__((address_space(4))) int32_t* c = (const __attribute__((address_space(4))) int32_t*)bt_row;
  int32_t p = c[lp];
  p = p < 0 ? 0 : p;
  return p >= num_pages ? num_pages - 1 : p;
}

}  // namespace pa
