// Shared device helpers and host-side argument checking for the kx355 kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kx355.h"

namespace kx {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;

// ---- bf16 <-> fp32 -----------------------------------------------------------------------------
// Widening is exact. Narrowing uses gfx950's v_cvt_pk_bf16_f32: round to nearest even.
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
// Two values in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

__device__ __forceinline__ void unpack8(const uint4& w, float* v) {
  v[0] = lo_f(w.x); v[1] = hi_f(w.x);
  v[2] = lo_f(w.y); v[3] = hi_f(w.y);
  v[4] = lo_f(w.z); v[5] = hi_f(w.z);
  v[6] = lo_f(w.w); v[7] = hi_f(w.w);
}
__device__ __forceinline__ uint4 pack8(const float* v) {
  uint4 w;
  w.x = pack2(v[0], v[1]);
  w.y = pack2(v[2], v[3]);
  w.z = pack2(v[4], v[5]);
  w.w = pack2(v[6], v[7]);
  return w;
}

// ---- 16-bit activations: bf16 (H = false) or fp16 (H = true) ------------------------------------
// Widening is exact for both. Narrowing rounds to nearest even (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32); an fp16 result beyond 65504 becomes infinity, as an fp16 cast does.
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
template <bool H>
__device__ __forceinline__ float e2f(uint16_t b) {
  if constexpr (H) return (float)__builtin_bit_cast(_Float16, b);
  else return bf2f(b);
}
template <bool H>
__device__ __forceinline__ float e_lo(uint32_t w) { return e2f<H>((uint16_t)(w & 0xffffu)); }
template <bool H>
__device__ __forceinline__ float e_hi(uint32_t w) {
  if constexpr (H) return e2f<H>((uint16_t)(w >> 16));
  else return hi_f(w);
}
template <bool H>
__device__ __forceinline__ uint16_t f2e(float f) {
  if constexpr (H) return __builtin_bit_cast(uint16_t, (_Float16)f);
  else return f2bf(f);
}
template <bool H>
__device__ __forceinline__ uint32_t e_pack2(float lo, float hi) {
  if constexpr (H) return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2));
  else return pack2(lo, hi);
}
template <bool H>
__device__ __forceinline__ void e_unpack8(const uint4& w, float* v) {
  v[0] = e_lo<H>(w.x); v[1] = e_hi<H>(w.x);
  v[2] = e_lo<H>(w.y); v[3] = e_hi<H>(w.y);
  v[4] = e_lo<H>(w.z); v[5] = e_hi<H>(w.z);
  v[6] = e_lo<H>(w.w); v[7] = e_hi<H>(w.w);
}
template <bool H>
__device__ __forceinline__ uint4 e_pack8(const float* v) {
  uint4 w;
  w.x = e_pack2<H>(v[0], v[1]);
  w.y = e_pack2<H>(v[2], v[3]);
  w.z = e_pack2<H>(v[4], v[5]);
  w.w = e_pack2<H>(v[6], v[7]);
  return w;
}
// One 32x32x16 MFMA on 16-bit operands held as 8 x 16-bit lanes (the bits of bf16 or fp16).
template <bool H>
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (H)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One fp32 value rounded to the 16-bit type, as the bits of a __bf16 vector lane.
template <bool H>
__device__ __forceinline__ __bf16 e16(float f) {
  if constexpr (H) return __builtin_bit_cast(__bf16, (_Float16)f);
  else return (__bf16)f;
}

// The entry point's name for a launch of element type H (names end in _bf16 / _f16).
template <bool H>
constexpr const char* ename(const char* bf16_name, const char* f16_name) { return H ? f16_name : bf16_name; }

// ---- activations (fp32 opmath) -----------------------------------------------------------------
// tanh GELU with the inner argument clamped to +-10 (kinomlx/kernels/fused_ops.py:27-35), through
// the identity 0.5 x (1 + tanh(u)) = x * sigmoid(2u) = x / (1 + e^(-2u)). The tanh form cancels in
// 1 + tanh(u) for negative u (at x = -3 an ulp of tanh is ~70 ulps of the result, so last-bit
// differences between tanh implementations flip bf16 roundings); the sigmoid form has no
// cancellation and stays within a few fp32 ulps of the exact function everywhere.
__device__ __forceinline__ float gelu_inner(float x) {
  const float inner = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
  return fminf(fmaxf(inner, -10.0f), 10.0f);
}
__device__ __forceinline__ float gelu_tanh(float x) {
  return x / (1.0f + expf(-2.0f * gelu_inner(x)));
}
// x / (1 + exp(-x)) (kinomlx/kernels/fused_ops.py:40-45).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Call-free forms for epilogues that hold many live accumulators: a libm call there would force
// every live register to be saved around it. exp via v_exp_f32 (exp2), division via v_rcp_f32.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// The same function with -2 log2(e) folded into the inner polynomial and the clamp (+-10 on the
// inner argument is +-20 log2(e) on the exp2 argument): 7 VALU per value instead of 11. Its error
// against the exact clamped tanh GELU is the same as the unfolded form's (both <= 2.5e-6 relative
// over [-12, 12], set by the exp at large negative x).
__device__ __forceinline__ float fast_gelu_tanh(float x) {
  constexpr float A = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
  constexpr float B = A * 0.044715f;
  constexpr float LIM = 20.0f * 1.4426950408889634f;
  const float z = fminf(fmaxf(x * fmaf(B, x * x, A), -LIM), LIM);
  return x * fast_rcp(1.0f + __builtin_amdgcn_exp2f(z));
}
__device__ __forceinline__ float fast_silu(float x) { return x * fast_rcp(1.0f + fast_exp(-x)); }
__device__ __forceinline__ float fast_sigmoid2(float x) { return 2.0f * fast_rcp(1.0f + fast_exp(-x)); }
__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + fast_exp(-x)); }

// ---- wave reductions (wave64) -------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), the same in every lane of the row, by
// VALU lane permutes instead of LDS round trips: swap neighbours, swap pairs (quad_perm [1,0,3,2]
// and [2,3,0,1]), then the half-row mirror (lane i <- 7 - i) and the row mirror (i <- 15 - i), which
// after the quad steps add the other quad and the other half-row. The adds are the ones of an
// xor-1, 2, 4, 8 butterfly, in that order.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// ---- host side ----------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Maps a workgroup id to a logical tile id so that each of the 8 XCDs (which receive workgroups
// round-robin) walks a contiguous range of logical tiles: neighbouring tiles then share the
// same XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, local = bid / 8;
  return (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

}  // namespace kx

#define KX_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return ::kx::set_error(KX_ERR_INVALID, __VA_ARGS__); \
  } while (0)
