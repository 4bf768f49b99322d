// Quantize-on-load: a bf16 (out, in) weight -> the packed group-wise affine format the quantized
// GEMMs read (uint32 words holding 32 / bits codes each, lowest bits first; one bf16 scale and
// bias per group of 64 along K).
//
// Per group: lo, hi = min, max (exact in fp32); scale = bf16((hi - lo) / (2^bits - 1)), 1 when
// that is not positive; bias = bf16(lo); code = clamp(rint((w - bias) / scale), 0, 2^bits - 1)
// with the fp32 subtraction and correctly rounded division. The dequantized weight is then
// bf16(scale * code + bias) (kx_dequant_affine_bf16). HBM-bound: one read of the weight, an
// eighth (int4) or a quarter (int8) of it written back. The mxfp8 quantizer (OCP MX) follows.
#include <math.h>

#include "common.h"

namespace kx {
namespace {

constexpr int QGROUP = 64;

// Eight lanes per (row, group): lane `sub` holds values 8 sub .. 8 sub + 7 (one 16-byte load), so a
// wave reads eight whole groups = 1 KB of contiguous weight per load; min / max are reduced over
// the eight lanes with three xor shuffles. Each lane packs its own eight codes: one word (int4) or
// two (int8), written contiguously across the group's lanes.
template <int BITS>
__global__ __launch_bounds__(256) void quantize_affine_kernel(const uint16_t* __restrict__ w, int64_t ldw,
                                                              uint32_t* __restrict__ words,
                                                              uint16_t* __restrict__ scales,
                                                              uint16_t* __restrict__ biases, int64_t groups,
                                                              int64_t groups_per_row) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = t >> 3;
  const int sub = (int)(t & 7);
  // the grid covers whole groups (8 lanes each) and every lane of a partial last wave is out of
  // range together, so the shuffles below only ever read lanes of the same group
  if (g >= groups) return;
  const int64_t row = g / groups_per_row, col = g - row * groups_per_row;
  float v[8];
  unpack8(*reinterpret_cast<const uint4*>(w + row * ldw + col * QGROUP + sub * 8), v);
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, o, 8));
    hi = fmaxf(hi, __shfl_xor(hi, o, 8));
  }
  constexpr int LEVELS = (1 << BITS) - 1;
  float scale = (hi - lo) / (float)LEVELS;
  if (!(scale > 0.0f)) scale = 1.0f;
  uint16_t scale_bits = f2bf(scale);
  float s = bf2f(scale_bits);
  if (!(s > 0.0f)) {
    scale_bits = f2bf(1.0f);
    s = 1.0f;
  }
  const uint16_t bias_bits = f2bf(lo);
  const float b = bf2f(bias_bits);
  uint32_t code[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) code[i] = (uint32_t)fminf(fmaxf(rintf((v[i] - b) / s), 0.0f), (float)LEVELS);
  if constexpr (BITS == 4) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= code[i] << (4 * i);
    words[g * 8 + sub] = word;
  } else {
    uint2 pair;
    pair.x = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
    pair.y = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    reinterpret_cast<uint2*>(words)[g * 8 + sub] = pair;
  }
  if (sub == 0) {
    scales[g] = scale_bits;
    biases[g] = bias_bits;
  }
}

// ---- mxfp8 (OCP MX: FP8 E4M3 elements, one E8M0 scale per 32 along K) ---------------------------
//
// Per group: X = floor(log2(max |w|)) - 8 (8: the exponent of E4M3's largest normal, 448), clamped
// to [-127, 127], and -127 for an all-zero group; scale byte X + 127; element code = E4M3 of
// w * 2^-X rounded to nearest even and saturated at +-448. Every step is exact in fp32 except the
// one rounding to E4M3.

// |v| -> E4M3 code (sign from v's sign bit; NaN -> 0x7F).
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
  if (v != v) return 0x7Fu;
  const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  uint32_t code;
  if (a >= 448.0f) {
    code = 0x7Eu;
  } else if (a < 0.015625f) {
    code = (uint32_t)rintf(a * 512.0f);  // subnormal steps of 2^-9; 8 steps is 2^-6 (code 8)
  } else {
    int e;
    frexpf(a, &e);
    const int ex = e - 1;  // a in [2^ex, 2^(ex+1)), ex in [-6, 8]: 8 steps of 2^(ex-3) per binade
    code = (uint32_t)(((ex + 7) << 3) + (int)rintf(ldexpf(a, 3 - ex)) - 8);  // 16 steps carry to ex+1
  }
  return sign | code;
}

// Four lanes per group of 32: lane `sub` holds values 8 sub .. 8 sub + 7 (one 16-byte load) and
// writes their two packed words; the group maximum is reduced over the four lanes.
__global__ __launch_bounds__(256) void quantize_mx8_kernel(const uint16_t* __restrict__ w, int64_t ldw,
                                                           uint32_t* __restrict__ words, uint8_t* __restrict__ scales,
                                                           int64_t groups, int64_t groups_per_row) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = t >> 2;
  const int sub = (int)(t & 3);
  // whole groups of four lanes are in or out of range together, so the shuffles stay in a group
  if (g >= groups) return;
  const int64_t row = g / groups_per_row, col = g - row * groups_per_row;
  float v[8];
  unpack8(*reinterpret_cast<const uint4*>(w + row * ldw + col * 32 + sub * 8), v);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 4));
  int x = -127;
  if (amax > 0.0f) {
    int e;
    frexpf(amax, &e);
    x = min(max(e - 1 - 8, -127), 127);
  }
  uint32_t code[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) code[i] = e4m3_rne(ldexpf(v[i], -x));
  uint2 pair;
  pair.x = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
  pair.y = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
  reinterpret_cast<uint2*>(words)[g * 4 + sub] = pair;
  if (sub == 0) scales[g] = (uint8_t)(x + 127);
}

// ---- mxfp4 / nvfp4 (FP4 E2M1 elements) ---------------------------------------------------------
//
// E2M1 (OCP MX v1.0): sign in bit 3, exponent bits 2-1 (bias 1), mantissa bit 0: magnitudes 0, 0.5,
// 1, 1.5, 2, 3, 4, 6; eight codes per little-endian uint32 (element j at bits [4j, 4j + 4)).
// mxfp4: one E8M0 scale per 32 along K, X = floor(log2(max |w|)) - 2 (2: the exponent of E2M1's
// largest normal, 6 = 1.5 * 2^2), clamped to [-127, 127] (-127 for an all-zero group); element =
// E2M1 of w * 2^-X (an exact scaling). nvfp4: one E4M3 scale per 16, s = E4M3(max |w| / 6) (IEEE
// fp32 division, round to nearest even, saturating at 448); element = E2M1 of fp32(w / s); a
// group whose s is zero stores zero codes. E2M1 rounds to nearest even and saturates at +-6.

// |v| -> E2M1 code (sign from v's sign bit): the round-to-nearest-even decision boundaries of the
// grid 0, 0.5, 1, 1.5, 2, 3, 4, 6 (a tie goes to the even mantissa: 0.25 -> 0, 0.75 -> 1, 1.25 -> 1,
// 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4); NaN gives zero.
__device__ __forceinline__ uint32_t e2m1_rne(float v) {
  if (v != v) return 0u;
  const uint32_t sign = (__float_as_uint(v) >> 28) & 8u;
  const float a = fabsf(v);
  uint32_t code;
  if (a <= 0.25f) code = 0;
  else if (a < 0.75f) code = 1;
  else if (a <= 1.25f) code = 2;
  else if (a < 1.75f) code = 3;
  else if (a <= 2.5f) code = 4;
  else if (a < 3.5f) code = 5;
  else if (a <= 5.0f) code = 6;
  else code = 7;
  return sign | code;
}

// An E4M3 byte (OCP, no infinities) as fp32, exactly.
__device__ __forceinline__ float e4m3_value(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  const float mag = e == 0 ? (float)m * 0.001953125f : ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  return (b & 0x80u) ? -mag : mag;
}

// G / 8 lanes per group (mxfp4: G = 32, nvfp4: G = 16): lane `sub` holds values 8 sub .. 8 sub + 7
// (one 16-byte load) and writes their packed word; the group maximum is reduced over the lanes.
template <bool NV>
__global__ __launch_bounds__(256) void quantize_fp4_kernel(const uint16_t* __restrict__ w, int64_t ldw,
                                                           uint32_t* __restrict__ words, uint8_t* __restrict__ scales,
                                                           int64_t groups, int64_t groups_per_row) {
  constexpr int G = NV ? 16 : 32, LPG = G / 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = t / LPG;
  const int sub = (int)(t % LPG);
  // whole groups of lanes are in or out of range together, so the shuffles stay in a group
  if (g >= groups) return;
  const int64_t row = g / groups_per_row, col = g - row * groups_per_row;
  float v[8];
  unpack8(*reinterpret_cast<const uint4*>(w + row * ldw + col * G + sub * 8), v);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int o = 1; o < LPG; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, LPG));
  uint32_t word = 0, sbyte;
  if constexpr (NV) {
    sbyte = e4m3_rne(amax / 6.0f) & 0x7Fu;
    const float sc = e4m3_value(sbyte);
    if (sc > 0.0f) {
#pragma unroll
      for (int i = 0; i < 8; ++i) word |= e2m1_rne(v[i] / sc) << (4 * i);
    }
  } else {
    int x = -127;
    if (amax > 0.0f) {
      int e;
      frexpf(amax, &e);
      x = min(max(e - 1 - 2, -127), 127);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= e2m1_rne(ldexpf(v[i], -x)) << (4 * i);
    sbyte = (uint32_t)(x + 127);
  }
  words[g * LPG + sub] = word;
  if (sub == 0) scales[g] = (uint8_t)sbyte;
}

}  // namespace
}  // namespace kx

using namespace kx;

extern "C" int kx_quantize_mxfp8_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, int64_t n, int64_t k,
                                      int group_size, kx_stream_t stream) {
  const char* what = "kx_quantize_mxfp8_bf16";
  KX_REQUIRE(w && wq && scales, "%s: null tensor", what);
  KX_REQUIRE(group_size == 32, "%s: group_size must be 32, got %d", what, group_size);
  KX_REQUIRE(n >= 0 && k > 0 && k % 32 == 0 && ldw >= k && ldw % 8 == 0 && aligned16(w),
             "%s: bad shape (n=%lld k=%lld ldw=%lld; k %% 32 == 0, 16-byte rows)", what, (long long)n, (long long)k,
             (long long)ldw);
  KX_REQUIRE(aligned8(wq), "%s: wq must be 8-byte aligned", what);
  const int64_t groups = n * (k / 32);
  KX_REQUIRE(groups * 4 / 256 < (1ll << 31), "%s: too many groups", what);
  if (groups == 0) return KX_OK;
  quantize_mx8_kernel<<<(unsigned)((groups * 4 + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)w, ldw, wq, (uint8_t*)scales, groups, k / 32);
  return check_launch(what);
}

extern "C" int kx_quantize_affine_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, void* biases,
                                       int64_t n, int64_t k, int group_size, int bits, kx_stream_t stream) {
  KX_REQUIRE(w && wq && scales && biases, "kx_quantize_affine_bf16: null tensor");
  KX_REQUIRE(bits == 4 || bits == 8, "kx_quantize_affine_bf16: bits must be 4 or 8, got %d", bits);
  KX_REQUIRE(group_size == QGROUP, "kx_quantize_affine_bf16: group_size must be 64, got %d", group_size);
  KX_REQUIRE(n >= 0 && k > 0 && k % QGROUP == 0 && ldw >= k && ldw % 8 == 0 && aligned16(w),
             "kx_quantize_affine_bf16: bad shape (n=%lld k=%lld ldw=%lld; k %% 64 == 0, 16-byte rows)",
             (long long)n, (long long)k, (long long)ldw);
  KX_REQUIRE(aligned8(wq), "kx_quantize_affine_bf16: wq must be 8-byte aligned");
  const int64_t groups = n * (k / QGROUP);
  KX_REQUIRE(groups * 8 / 256 < (1ll << 31), "kx_quantize_affine_bf16: too many groups");
  if (groups == 0) return KX_OK;
  const unsigned grid = (unsigned)((groups * 8 + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4)
    quantize_affine_kernel<4><<<grid, 256, 0, s>>>((const uint16_t*)w, ldw, wq, (uint16_t*)scales,
                                                   (uint16_t*)biases, groups, k / QGROUP);
  else
    quantize_affine_kernel<8><<<grid, 256, 0, s>>>((const uint16_t*)w, ldw, wq, (uint16_t*)scales,
                                                   (uint16_t*)biases, groups, k / QGROUP);
  return check_launch("kx_quantize_affine_bf16");
}

extern "C" int kx_quantize_fp4_bf16(const void* w, int64_t ldw, uint32_t* wq, void* scales, int64_t n, int64_t k,
                                    int group_size, int scale_kind, kx_stream_t stream) {
  const char* what = "kx_quantize_fp4_bf16";
  KX_REQUIRE(w && wq && scales, "%s: null tensor", what);
  KX_REQUIRE(scale_kind == KX_FP4_MX || scale_kind == KX_FP4_NV, "%s: bad scale kind %d", what, scale_kind);
  const int gs = scale_kind == KX_FP4_NV ? 16 : 32;
  KX_REQUIRE(group_size == gs, "%s: group_size must be %d for this scale kind, got %d", what, gs, group_size);
  KX_REQUIRE(n >= 0 && k > 0 && k % gs == 0 && ldw >= k && ldw % 8 == 0 && aligned16(w),
             "%s: bad shape (n=%lld k=%lld ldw=%lld; k %% %d == 0, 16-byte rows)", what, (long long)n, (long long)k,
             (long long)ldw, gs);
  KX_REQUIRE(aligned8(wq), "%s: wq must be 8-byte aligned", what);
  const int64_t groups = n * (k / gs);
  KX_REQUIRE(groups * (gs / 8) / 256 < (1ll << 31), "%s: too many groups", what);
  if (groups == 0) return KX_OK;
  const unsigned grid = (unsigned)((groups * (gs / 8) + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
  if (scale_kind == KX_FP4_NV)
    quantize_fp4_kernel<true><<<grid, 256, 0, s>>>((const uint16_t*)w, ldw, wq, (uint8_t*)scales, groups, k / gs);
  else
    quantize_fp4_kernel<false><<<grid, 256, 0, s>>>((const uint16_t*)w, ldw, wq, (uint8_t*)scales, groups, k / gs);
  return check_launch(what);
}
