// Shared device helpers for the gfx950 W4A16 kernels: vector types, the
// exact int4 -> bf16/fp16 dequantization used in every GEMM regime, and the
// host-side error plumbing of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "int4_hip.h"

namespace w4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Activation element type per dtype code and the matching 8-wide MFMA operand.
template <int DT> struct Act;
template <> struct Act<W4_DTYPE_BF16> {
  typedef __bf16 scalar;
  typedef bf16x8 frag;
};
template <> struct Act<W4_DTYPE_FP16> {
  typedef _Float16 scalar;
  typedef f16x8 frag;
};

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ float act_bits_to_float(uint16_t b, int dt) {
  if (dt == W4_DTYPE_BF16) return __builtin_bit_cast(float, (uint32_t)b << 16);
  return half_bits_to_float(b);
}

template <int DT>
__device__ __forceinline__ uint16_t float_to_act_bits(float v) {
  typedef typename Act<DT>::scalar S;
  return __builtin_bit_cast(uint16_t, (S)v);
}

// Per (group, column) constants of the exact dequantization.
//
// A nibble q is placed in the mantissa of an fp16 whose exponent is fixed:
//   0x6400 | q        = 1024 + q         (nibbles 0, 2, 4, 6)
//   0x6400 | (q << 4) = 1024 + 16 q      (nibbles 1, 3, 5, 7)
// and w_hat = (q - z) * s comes out of ONE fused multiply-add in fp32:
//   (1024 + q)   * s      + (-(1024 + z) * s) = (q - z) * s
//   (1024 + 16q) * (s/16) + (-(64 + z) * s)   = (q - z) * s
// Every term is exact in fp32: (1024 + z) * s has <= 22 significant bits,
// s/16 is a power-of-two scaling and the fma rounds once from the exact
// (q - z) * s, which has <= 15 significant bits, so w_hat is bit-identical to
// the reference's fp32 (q - z) * s (int4_triton/quantize.py:135,
// int4_triton/gemm.py:139,211) for every finite s and integer z in [0, 15].
// It is then rounded once (RNE) to the activation dtype, as the reference's
// kernels do before the product.
struct GroupConst {
  float s, c0, s16, c1;
};

__device__ __forceinline__ GroupConst make_group_const(uint16_t s_bits, uint16_t z_bits) {
  const float s = half_bits_to_float(s_bits);
  const float z = half_bits_to_float(z_bits);
  GroupConst g;
  g.s = s;
  g.c0 = -((1024.0f + z) * s);
  g.s16 = s * 0.0625f;
  g.c1 = -((64.0f + z) * s);
  return g;
}

// 0x64006400 kept in a VGPR so that the nibble insertion compiles to one
// v_and_or_b32 (mask from an SGPR, magic from this VGPR) per two nibbles.
__device__ __forceinline__ uint32_t fp16_magic_vgpr() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

// Eight int4 values of one packed word -> eight dequantized activation-dtype
// values in k order (element i = nibble i = row 8*k8 + i).
template <int DT>
__device__ __forceinline__ typename Act<DT>::frag dequant_word(uint32_t w, const GroupConst& g,
                                                               uint32_t magic) {
  typedef typename Act<DT>::scalar S;
  const uint32_t w8 = w >> 8;
  const f16x2 t0 = __builtin_bit_cast(f16x2, (w & 0x000F000Fu) | magic);   // q0, q4
  const f16x2 t1 = __builtin_bit_cast(f16x2, (w & 0x00F000F0u) | magic);   // 16q1, 16q5
  const f16x2 t2 = __builtin_bit_cast(f16x2, (w8 & 0x000F000Fu) | magic);  // q2, q6
  const f16x2 t3 = __builtin_bit_cast(f16x2, (w8 & 0x00F000F0u) | magic);  // 16q3, 16q7
  typename Act<DT>::frag r;
  r[0] = (S)__builtin_fmaf((float)t0[0], g.s, g.c0);
  r[1] = (S)__builtin_fmaf((float)t1[0], g.s16, g.c1);
  r[2] = (S)__builtin_fmaf((float)t2[0], g.s, g.c0);
  r[3] = (S)__builtin_fmaf((float)t3[0], g.s16, g.c1);
  r[4] = (S)__builtin_fmaf((float)t0[1], g.s, g.c0);
  r[5] = (S)__builtin_fmaf((float)t1[1], g.s16, g.c1);
  r[6] = (S)__builtin_fmaf((float)t2[1], g.s, g.c0);
  r[7] = (S)__builtin_fmaf((float)t3[1], g.s16, g.c1);
  return r;
}

template <int DT> struct Mfma;
template <> struct Mfma<W4_DTYPE_BF16> {
  __device__ __forceinline__ static f32x4 m16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x16 m32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<W4_DTYPE_FP16> {
  __device__ __forceinline__ static f32x4 m16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x16 m32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Load 8 consecutive activation elements x[k .. k+7] of one row (zero past K).
template <int DT, bool CONTIG>
__device__ __forceinline__ typename Act<DT>::frag load_x8(const uint16_t* __restrict__ row,
                                                          int64_t k, int64_t K, int64_t sxk) {
  typedef typename Act<DT>::frag F;
  if (CONTIG && k + 8 <= K) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + k);
    return __builtin_bit_cast(F, v);
  }
  uint16_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (k + i < K) ? row[(k + i) * sxk] : (uint16_t)0;
  u32x4 v;
  v[0] = e[0] | ((uint32_t)e[1] << 16);
  v[1] = e[2] | ((uint32_t)e[3] << 16);
  v[2] = e[4] | ((uint32_t)e[5] << 16);
  v[3] = e[6] | ((uint32_t)e[7] << 16);
  return __builtin_bit_cast(F, v);
}

}  // namespace w4

// ---------------------------------------------------------------- host side
namespace w4host {

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
void clear_error();
int device_cu_count();

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}

}  // namespace w4host
