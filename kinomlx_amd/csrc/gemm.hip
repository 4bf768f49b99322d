// Dense bf16 and affine int4/int8 weight-quantized linear layers on gfx950 MFMA.
//
// c[m, n] = epilogue(sum_k a[m, k] * w[n, k]) — both operands K-contiguous (the reference's
// (out, in) weight layout), fp32 accumulation in v_mfma_f32_32x32x16_bf16 (or _f16: the dense
// kernels take bf16 or fp16 operands, template H), one rounding to the 16-bit type.
//
// Tiling: a BM x BN output tile per workgroup of WM x WN waves; each wave owns a
// (BM/WM) x (BN/WN) sub-tile as a grid of 32x32 MFMA blocks. K advances in stages of 64: the
// next stage's global loads are issued into registers before the current stage's MFMAs and
// written to the other half of a double-buffered LDS tile afterwards, so one barrier per stage
// suffices. LDS rows are 128 bytes (64 bf16) with the 16-byte chunk index XOR-swizzled by the
// row, so the 32-row fragment reads of an MFMA operand are bank-conflict free.
//
// The MFMA A operand is the weight tile and the B operand the activation tile, so that the
// accumulator's lane holds one output row m and runs of 4 consecutive columns n: the epilogue
// stores 8-byte vectors along the output row.
//
// Quantized weights: the stage's packed words and per-group bf16 scale/bias are loaded instead,
// and dequantized (bf16(fp32(scale) * q + fp32(bias))) inside the mainloop. mxfp8 weights (OCP
// MX: FP8 E4M3 elements, one E8M0 scale byte per 32 along K) take the same route: each element is
// converted to fp32 exactly (v_cvt_pk_f32_fp8) and multiplied by its power-of-two scale (exact),
// so the bf16 operand equals the format's value.
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace kx {
namespace {

constexpr int BK = 64;        // K per stage
constexpr int ROWB = BK * 2;  // bytes per LDS tile row

struct Epilogue {
  const uint16_t* bias;
  const void* resid;  // bf16, or fp32 with KX_EPI_RESID_F32
  int64_t ldr;
  const float* gate;
  int64_t gate_div;
  int64_t gate_stride;
  int flags;
  // KX_EPI_QK_NORM_ROPE: columns [0, q_end) are query heads and [q_end, k_end) key heads of 128;
  // each row's head is RMS-normalized (weights nq / nk, fp32 or bf16, plus w_off; eps), then
  // rotated in adjacent pairs by the row's cos / sin table row:
  // tables + (m / t_rows) * t_bs + (m % t_rows) * t_ld + head * t_hs + d.
  const void* nq;
  const void* nk;
  int n_bf16;
  float n_eps, n_off;
  int64_t q_end, k_end;
  // set by the launcher, not part of the C ABI: visit the tile rows last to first (see
  // rows_last_first)
  int rows_desc;
  const float* cosp;
  const float* sinp;
  int64_t t_ld, t_hs, t_rows, t_bs;
  uint32_t t_magic;  // m / t_rows = (umulhi(m, t_magic) + m) >> t_shift for m < 2^31
  int t_shift;
};

struct QuantW {
  const uint32_t* words;  // (n, k * bits / 32)
  const uint16_t* scales;  // (n, k / 64)
  const uint16_t* biases;  // (n, k / 64)
  const uint8_t* e8m0;     // mxfp8: (n, k / 32) scale bytes
};

// Weight-mode template code: 0 dense bf16, 4 / 8 affine int4 / int8, QMX8 mxfp8 (8-bit codes).
constexpr int QMX8 = 9;
template <int QB>
constexpr int qbits() { return QB == QMX8 ? 8 : QB; }

// 2^(s - 127) for an E8M0 scale byte (s = 0: 2^-127, an fp32 subnormal; s = 255: NaN).
__device__ __forceinline__ float e8m0_f32(uint32_t s) {
  const uint32_t bits = s == 0 ? 0x00400000u : (s == 255 ? 0x7FC00000u : s << 23);
  return __uint_as_float(bits);
}

// Four E4M3 bytes of w (lowest first) times a power-of-two scale, as four bf16 (two words). The
// fp8 -> fp32 conversion is exact, and so is the product while it stays in the fp32 normal range.
__device__ __forceinline__ uint2 mx8_quad(uint32_t w, float scale) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  return make_uint2(pack2(lo.x * scale, lo.y * scale), pack2(hi.x * scale, hi.y * scale));
}

__device__ __forceinline__ int lds_off(int r, int c) { return r * ROWB + ((c ^ (r & 7)) << 4); }

__device__ __forceinline__ float apply_act(float v, int act) {
  switch (act) {
    case 1: return fast_gelu_tanh(v);
    case 2: return fast_silu(v);
    case 3: return fast_sigmoid2(v);
    case 4: return fast_sigmoid(v);
    default: return v;
  }
}

template <int BITS>
__device__ __forceinline__ uint4 dequant8(const uint32_t* wd, float s, float b) {
  if constexpr (BITS == QMX8) {
    const uint2 q0 = mx8_quad(wd[0], s), q1 = mx8_quad(wd[1], s);
    return make_uint4(q0.x, q0.y, q1.x, q1.y);
  }
  float v[8];
  if (BITS == 4) {
    const uint32_t w = wd[0];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = fmaf(s, (float)((w >> (4 * j)) & 15u), b);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = fmaf(s, (float)((wd[0] >> (8 * j)) & 255u), b);
      v[4 + j] = fmaf(s, (float)((wd[1] >> (8 * j)) & 255u), b);
    }
  }
  return pack8(v);
}

// QB = 0: dense bf16 weights; QB = 4 / 8: affine quantized weights of that many bits; QMX8: mxfp8.
template <int BM, int BN, int WM, int WN, int QB, bool H = false>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ W, int64_t ldw,
    QuantW qw, void* __restrict__ C, int64_t ldc, int M, int N, int K, Epilogue epi) {
  constexpr int NT = WM * WN * 64;
  constexpr int WT_M = BM / WM, WT_N = BN / WN;
  constexpr int MB = WT_M / 32, NB = WT_N / 32;
  constexpr int A_PER = BM * (BK / 8) / NT;
  constexpr int W_PER = BN * (BK / 8) / NT;
  constexpr int QBITS = qbits<QB>();
  constexpr int QWORDS = QBITS == 8 ? 2 : 1;
  static_assert(A_PER * NT == BM * (BK / 8) && W_PER * NT == BN * (BK / 8), "tile/threads");
  static_assert(MB >= 1 && NB >= 1, "wave tile");
  constexpr int STAGE = (BM + BN) * ROWB;

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;

  // ---- tile coordinates: XCD-contiguous, then grouped by 8 tile rows for L2 reuse
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  constexpr int GM = 8;
  const int group_width = GM * tiles_n;
  const int first_m = (t / group_width) * GM;
  const int gsz = min(tiles_m - first_m, GM);
  const int tm = first_m + (t % group_width) % gsz;
  const int tn = (t % group_width) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;

  // ---- global -> register prefetch
  uint4 ra[A_PER];
  uint4 rw[QB == 0 ? W_PER : 1];
  uint32_t rq[QB == 0 ? 1 : W_PER][QWORDS];
  float rs[QB == 0 ? 1 : W_PER], rb[QB == 0 ? 1 : W_PER];

  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, c = q & 7;
      const int gm = min(m0 + r, M - 1);
      const int gk = k0 + c * 8;
      // Branch-free K tail: read a valid chunk, then zero it (K % 8 == 0, so K - 8 >= 0).
      uint4 v = *reinterpret_cast<const uint4*>(A + (int64_t)gm * lda + min(gk, K - 8));
      if (gk >= K) v = make_uint4(0, 0, 0, 0);
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < W_PER; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, c = q & 7;
      const int gn = min(n0 + r, N - 1);
      const int gk = k0 + c * 8;
      if (QB == 0) {
        uint4 v = *reinterpret_cast<const uint4*>(W + (int64_t)gn * ldw + min(gk, K - 8));
        if (gk >= K) v = make_uint4(0, 0, 0, 0);
        rw[i] = v;
      } else if constexpr (QB == QMX8) {
        // K % 32 == 0: a stage's second 32-wide half may lie past K; it reads the last group and
        // is zeroed (zero codes dequantize to zero)
        const int gkc = min(gk, K - 8);
        const int64_t wrow = (int64_t)gn * (K / 4);
#pragma unroll
        for (int j = 0; j < 2; ++j) rq[i][j] = gk < K ? qw.words[wrow + gkc / 4 + j] : 0u;
        rs[i] = e8m0_f32(qw.e8m0[(int64_t)gn * (K / 32) + gkc / 32]);
        rb[i] = 0.0f;
      } else {
        const int64_t wrow = (int64_t)gn * (K * QB / 32);
#pragma unroll
        for (int j = 0; j < QWORDS; ++j) rq[i][j] = qw.words[wrow + gk * QB / 32 + j];
        const int64_t g = (int64_t)gn * (K / 64) + k0 / 64;
        rs[i] = bf2f(qw.scales[g]);
        rb[i] = bf2f(qw.biases[g]);
      }
    }
  };

  auto store_stage = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<uint4*>(buf + lds_off(q >> 3, q & 7)) = ra[i];
    }
    uint8_t* wbuf = buf + BM * ROWB;
#pragma unroll
    for (int i = 0; i < W_PER; ++i) {
      const int q = tid + i * NT;
      uint4 v;
      if (QB == 0)
        v = rw[i];
      else
        v = dequant8<QB>(rq[i], rs[i], rb[i]);
      *reinterpret_cast<uint4*>(wbuf + lds_off(q >> 3, q & 7)) = v;
    }
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int stages = (K + BK - 1) / BK;
  load_stage(0);
  store_stage(smem);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < stages; ++kt) {
    uint8_t* cur = smem + (kt & 1) * STAGE;
    const bool more = kt + 1 < stages;
    if (more) load_stage((kt + 1) * BK);
    const uint8_t* tA = cur;
    const uint8_t* tW = cur + BM * ROWB;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int c = 2 * s + lhalf;
      bf16x8 af[MB], wf[NB];
#pragma unroll
      for (int j = 0; j < MB; ++j)
        af[j] = *reinterpret_cast<const bf16x8*>(tA + lds_off(wm * WT_M + j * 32 + lrow, c));
#pragma unroll
      for (int i = 0; i < NB; ++i)
        wf[i] = *reinterpret_cast<const bf16x8*>(tW + lds_off(wn * WT_N + i * 32 + lrow, c));
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j)
          acc[i][j] = mfma32x32x16<H>(wf[i], af[j], acc[i][j]);
    }
    if (more) store_stage(smem + ((kt + 1) & 1) * STAGE);
    __syncthreads();
  }

  // ---- epilogue, staged through LDS one 32-column block at a time. The unrolled part only
  // moves accumulators (static indices, so they stay in registers); bias, activation and the
  // gated residual run in a plain loop over rows with each lane on 4 consecutive columns.
  constexpr int EP_LD = 36;  // padded fp32 row: 16-byte writes from 16 rows hit distinct banks
  static_assert(WM * WN * WT_M * EP_LD * 4 <= 2 * STAGE, "epilogue staging must fit in LDS");
  float* ep = reinterpret_cast<float*>(smem) + wave * (WT_M * EP_LD);
  const int act = (epi.flags >> 4) & 15;
  const bool has_bias = epi.flags & KX_EPI_BIAS;
  const bool gated = epi.flags & KX_EPI_GATED_RESIDUAL;
  const bool resid_f32 = epi.flags & KX_EPI_RESID_F32;
  const bool out_f32 = epi.flags & KX_EPI_OUT_F32;
  const bool vec_store = (ldc % 4 == 0) && (!gated || epi.ldr % 4 == 0);
  const int col4 = (lane & 7) * 4;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
#pragma unroll
    for (int j = 0; j < MB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 v;
        v.x = acc[i][j][g * 4 + 0];
        v.y = acc[i][j][g * 4 + 1];
        v.z = acc[i][j][g * 4 + 2];
        v.w = acc[i][j][g * 4 + 3];
        *reinterpret_cast<float4*>(ep + (j * 32 + lrow) * EP_LD + g * 8 + lhalf * 4) = v;
      }
    __syncthreads();
    const int n = n0 + wn * WT_N + i * 32 + col4;
    float bias4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (has_bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bias4[e] = n + e < N ? e2f<H>(epi.bias[n + e]) : 0.0f;
    }
#pragma unroll 2
    for (int r = lane >> 3; r < WT_M; r += 8) {
      const int m = m0 + wm * WT_M + r;
      if (m >= M || n >= N) continue;
      const float4 a4 = *reinterpret_cast<const float4*>(ep + r * EP_LD + col4);
      float v[4] = {a4.x + bias4[0], a4.y + bias4[1], a4.z + bias4[2], a4.w + bias4[3]};
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = apply_act(v[e], act);
      const int64_t ro = (int64_t)m * epi.ldr + n;
      const int64_t co = (int64_t)m * ldc + n;
      if (vec_store && n + 3 < N) {
        if (gated) {
          const float* grow = epi.gate + (m / epi.gate_div) * epi.gate_stride;
          const float4 gv = *reinterpret_cast<const float4*>(grow + n);
          float rv[4];
          if (resid_f32) {
            const float4 rr = *reinterpret_cast<const float4*>(static_cast<const float*>(epi.resid) + ro);
            rv[0] = rr.x; rv[1] = rr.y; rv[2] = rr.z; rv[3] = rr.w;
          } else {
            const uint2 rr = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(epi.resid) + ro);
            rv[0] = e_lo<H>(rr.x); rv[1] = e_hi<H>(rr.x); rv[2] = e_lo<H>(rr.y); rv[3] = e_hi<H>(rr.y);
          }
          v[0] = rv[0] + gv.x * v[0];
          v[1] = rv[1] + gv.y * v[1];
          v[2] = rv[2] + gv.z * v[2];
          v[3] = rv[3] + gv.w * v[3];
        }
        if (out_f32) {
          *reinterpret_cast<float4*>(static_cast<float*>(C) + co) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          uint2 o;
          o.x = e_pack2<H>(v[0], v[1]);
          o.y = e_pack2<H>(v[2], v[3]);
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + co) = o;
        }
      } else {
        for (int e = 0; e < 4 && n + e < N; ++e) {
          float x = v[e];
          if (gated) {
            const float rv = resid_f32 ? static_cast<const float*>(epi.resid)[ro + e]
                                       : e2f<H>(static_cast<const uint16_t*>(epi.resid)[ro + e]);
            x = rv + epi.gate[(m / epi.gate_div) * epi.gate_stride + n + e] * x;
          }
          if (out_f32)
            static_cast<float*>(C)[co + e] = x;
          else
            static_cast<uint16_t*>(C)[co + e] = f2e<H>(x);
        }
      }
    }
    __syncthreads();
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ words,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      uint16_t* __restrict__ out, int64_t n,
                                                      int64_t k, int group) {
  const int64_t chunks_per_row = k / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * chunks_per_row) return;
  const int64_t r = idx / chunks_per_row, c = idx - r * chunks_per_row;
  const int64_t kk = c * 8;
  const int64_t g = r * (k / group) + kk / group;
  const uint32_t* wd = words + r * (k * BITS / 32) + kk * BITS / 32;
  uint32_t tmp[2] = {wd[0], BITS == 8 ? wd[1] : 0u};
  *reinterpret_cast<uint4*>(out + r * k + kk) = dequant8<BITS>(tmp, bf2f(scales[g]), bf2f(biases[g]));
}

// mxfp8 in the reference layout: (n, k / 4) words and (n, k / 32) scale bytes -> (n, k) bf16, eight
// values per thread.
__global__ __launch_bounds__(256) void dequant_mx8_kernel(const uint32_t* __restrict__ words,
                                                          const uint8_t* __restrict__ scales,
                                                          uint16_t* __restrict__ out, int64_t n, int64_t k) {
  const int64_t chunks_per_row = k / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * chunks_per_row) return;
  const int64_t r = idx / chunks_per_row, c = idx - r * chunks_per_row;
  const uint2 w = *reinterpret_cast<const uint2*>(words + r * (k / 4) + 2 * c);
  uint32_t tmp[2] = {w.x, w.y};
  *reinterpret_cast<uint4*>(out + r * k + 8 * c) =
      dequant8<QMX8>(tmp, e8m0_f32(scales[r * (k / 32) + c / 4]), 0.0f);
}

// mxfp4 / nvfp4: (n, k / 8) words of eight E2M1 codes and (n, k / G) scale bytes (G = 32: E8M0,
// G = 16: E4M3) -> (n, k) bf16, eight values (one word) per thread. Every value is exact: an E2M1
// magnitude has at most 2 significant bits and the scale at most 4.
__device__ __forceinline__ float e2m1_f32(uint32_t c) {
  const uint32_t m3 = c & 7u;
  // 0, 0.5, then 1, 1.5, 2, 3, 4, 6: from code 2 on, the fp32 bits step by 2^22 from 1.0
  const float mag = m3 < 2u ? 0.5f * (float)m3 : __uint_as_float(0x3F800000u + ((m3 - 2u) << 22));
  return __uint_as_float(__float_as_uint(mag) | ((c & 8u) << 28));
}
__device__ __forceinline__ float e4m3_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  const float mag = e == 0 ? (float)m * 0.001953125f : ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  return (b & 0x80u) ? -mag : mag;
}
template <bool NV>
__global__ __launch_bounds__(256) void dequant_fp4_kernel(const uint32_t* __restrict__ words,
                                                          const uint8_t* __restrict__ scales,
                                                          uint16_t* __restrict__ out, int64_t n, int64_t k) {
  constexpr int G = NV ? 16 : 32;
  const int64_t words_per_row = k / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * words_per_row) return;
  const int64_t r = idx / words_per_row, c = idx - r * words_per_row;
  const uint32_t w = words[idx];
  const uint32_t sb = scales[r * (k / G) + (8 * c) / G];
  const float sc = NV ? e4m3_f32(sb) : e8m0_f32(sb);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = e2m1_f32((w >> (4 * j)) & 15u) * sc;
  *reinterpret_cast<uint4*>(out + r * k + 8 * c) = pack8(v);
}

// mxfp8 in the pretransposed layout (quantized from weight.T: (k, n / 4) words and (k, n / 32)
// scale bytes, groups along n) -> the (n, k) bf16 weight, through 64 x 64 LDS tiles: a thread
// dequantizes 16 consecutive n of one k row and writes them transposed into the tile, then
// writes 16 consecutive k of one n row. n % 32 == 0 and k % 8 == 0 keep every 16-run of n and
// every 8-run of k either wholly inside the matrix or wholly outside.
__global__ __launch_bounds__(256) void dequant_mx8_t_kernel(const uint32_t* __restrict__ words,
                                                            const uint8_t* __restrict__ scales,
                                                            uint16_t* __restrict__ out, int64_t n, int64_t k) {
  __shared__ uint16_t tile[64][64 + 2];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  {
    const int kl = t >> 2, nl = (t & 3) * 16;
    const int64_t kk = k0 + kl, nn = n0 + nl;
    if (kk < k && nn < n) {
      const uint4 w = *reinterpret_cast<const uint4*>(words + kk * (n / 4) + nn / 4);
      const float sc = e8m0_f32(scales[kk * (n / 32) + nn / 32]);
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint2 q = mx8_quad(wv[j], sc);
        tile[nl + 4 * j][kl] = (uint16_t)(q.x & 0xffffu);
        tile[nl + 4 * j + 1][kl] = (uint16_t)(q.x >> 16);
        tile[nl + 4 * j + 2][kl] = (uint16_t)(q.y & 0xffffu);
        tile[nl + 4 * j + 3][kl] = (uint16_t)(q.y >> 16);
      }
    }
  }
  __syncthreads();
  const int nl = t >> 2, kl = (t & 3) * 16;
  const int64_t nn = n0 + nl;
  if (nn >= n) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t kk = k0 + kl + 8 * h;
    if (kk >= k) break;
    const uint16_t* src = &tile[nl][kl + 8 * h];
    uint4 v;
    v.x = src[0] | ((uint32_t)src[1] << 16);
    v.y = src[2] | ((uint32_t)src[3] << 16);
    v.z = src[4] | ((uint32_t)src[5] << 16);
    v.w = src[6] | ((uint32_t)src[7] << 16);
    *reinterpret_cast<uint4*>(out + nn * k + kk) = v;
  }
}

// Tile of workgroup `bid` for the direct-to-LDS kernel, as (tile row, tile column). The 256
// workgroups of a round run at once, 32 per XCD, and the XCDs' L2s are separate. When the tile
// columns divide a round (8, 16, 32 or 64 of them) and the rows fill whole rounds, each round
// covers R = 256 / tiles_n whole tile rows, and each XCD an a x b block of them with the fewest
// operand panels (a + b = 12 for 32 tiles): every activation panel is then read in one round
// only, so a product whose operands exceed the last-level cache re-reads them from HBM once per
// round rather than once per round and XCD pair (the 9216 x 4096 x 16384 down projection: mean
// L1 -> L2 request latency 688 -> 505 cycles, 2.5 % faster). Otherwise: XCD-contiguous tiles,
// grouped by 8 tile rows.
__device__ __forceinline__ int2 lds_tile_of(int bid, int tiles_m, int tiles_n) {
  const int rows = 256 / tiles_n;
  if ((tiles_n == 8 || tiles_n == 16 || tiles_n == 32 || tiles_n == 64) && tiles_m % rows == 0) {
    // XCD x: block (x % ra, x / ra) of an ra x cb grid over the round, ra * cb = 8
    const int ra = tiles_n >= 32 ? 1 : tiles_n == 16 ? 2 : 8, cb = 8 / ra;
    const int a = rows / ra, b = tiles_n / cb;  // block rows x columns, a * b = 32
    const int x = bid % 8, i = bid / 8, r = i / 32, j = i % 32;
    return make_int2(r * rows + (x % ra) * a + j % a, (x / ra) * b + j / a);
  }
  const int t = xcd_remap(bid, tiles_m * tiles_n);
  constexpr int GM = 8;
  const int group_width = GM * tiles_n;
  const int first_m = (t / group_width) * GM;
  const int gsz = min(tiles_m - first_m, GM);
  return make_int2(first_m + (t % group_width) % gsz, (t % group_width) / gsz);
}

// ---- direct-to-LDS pipelined kernel (dense: K % 64 == 0; quantized: K % 128 == 0) ------------
//
// Operand tiles go from global memory straight into LDS with global_load_lds_dwordx4 (no VGPR
// staging): one wave instruction fills 64 lanes x 16 B = DRPI rows of DBK bf16, from a scalar tile
// base plus a loop-invariant 32-bit lane offset. Dense products use stages of DBK = 64 along K: a row's 128 bytes of a stage are one full cache line, so each row makes one
// 128-byte L1 -> L2 request. The per-CU operand stream is bounded by the requests it keeps in
// flight times their latency, so 128-byte requests carry twice the bytes of the 64-byte ones
// that 32-wide stages make. The 256 x 256 and 192 x 256 tiles keep two stages in LDS: stage kt+2
// goes into stage kt's buffer, half of its DMA instructions right after the barrier of stage
// kt's last k16 step and half during stage kt+1's first step. The small tiles (whose few MFMAs
// per stage cannot hide a one-stage prefetch) keep a ring of four, and so do the quantized
// products with 32-wide stages: their DMA for stage kt+3 goes out between the MFMAs of stage kt. Every k16 step is one scheduling region: wait for this step's
// fragments (read one step earlier), issue the fragment reads of the next step, then the step's
// MFMAs, so LDS latency hides under a full step of MFMAs and never more than MB + NB reads are
// outstanding (lgkmcnt counts to 15). The last step of a stage holds the stage's only workgroup
// barrier. The 16-byte slots of a row are XOR-swizzled so that both the DMA writes and the
// 32-row fragment reads are bank-conflict free.
//
// Epilogue: each wave stages half of its fp32 tile in LDS at a time and writes it back in rows,
// 4 columns per lane, so bias / gate / residual loads and the stores are contiguous runs. Full,
// aligned tiles take a compile-time specialisation per residual mode (GMODE 0: none, 1: bf16
// residual, 2: fp32 residual) and output type; edge tiles take the generic masked path.

// K per LDS stage of a dense product: a row's 128 bytes per stage are one full cache line, so
// every DMA lane group of a row makes one 128-byte request (32-wide stages made two 64-byte
// requests per line, twice the L1 -> L2 requests for the same bytes)
constexpr int DENSE_BK = 64;
// 8-bit packed weight rows (32 bytes per stage): chunk swizzle of row r
__device__ __forceinline__ int qswz(int r) { return (r >> 3) & 1; }
#define KX_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// Raw buffer resource over `base` (stride 0, 4 GiB range; dword 3 as for every gfx9 raw buffer)
// and a 16-byte-per-lane buffer load into LDS (M0 + lane * 16) from base + voff + soff: the
// offsets are one loop-invariant 32-bit lane offset and a scalar K offset, so a DMA issue needs
// no 64-bit address arithmetic (3 % on the block GEMMs against global_load_lds with per-issue
// 64-bit VALU adds). The host compilation pass has no buffer builtins; kernels only run on the
// device.
#if defined(__HIP_DEVICE_COMPILE__)
using rsrc_t = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ void buffer_lds16(rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, KX_LDS(lds), 16, voff, soff, 0, 0);
}
#else
struct rsrc_t {};
__device__ inline rsrc_t raw_rsrc(const void*) { return {}; }
__device__ inline void buffer_lds16(rsrc_t, void*, uint32_t, uint32_t) {}
#endif
// A workgroup barrier that the compiler may not move memory accesses across.
#define KX_BARRIER() asm volatile("s_barrier" ::: "memory")

// gfx9 s_waitcnt immediate that waits for vmcnt <= N only.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// gfx9 s_waitcnt immediate that waits for lgkmcnt <= N only (LDS reads complete in order).
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// bias + activation + gated residual on 4 consecutive columns n..n+3 of row m, then the store.
template <bool H>
__device__ __forceinline__ void epilogue_store4(float v[4], int m, int n, int N, const Epilogue& epi,
                                                void* __restrict__ C, int64_t ldc, bool vec_ok) {
  const int act = (epi.flags >> 4) & 15;
  const bool gated = epi.flags & KX_EPI_GATED_RESIDUAL;
  const bool resid_f32 = epi.flags & KX_EPI_RESID_F32;
  const bool out_f32 = epi.flags & KX_EPI_OUT_F32;
  const int64_t ro = (int64_t)m * epi.ldr + n;
  const int64_t co = (int64_t)m * ldc + n;
  if (vec_ok && n + 3 < N) {
    if (epi.flags & KX_EPI_BIAS) {
      const uint2 bb = *reinterpret_cast<const uint2*>(epi.bias + n);
      v[0] += e_lo<H>(bb.x); v[1] += e_hi<H>(bb.x); v[2] += e_lo<H>(bb.y); v[3] += e_hi<H>(bb.y);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = apply_act(v[e], act);
    if (gated) {
      const float4 gv = *reinterpret_cast<const float4*>(epi.gate + (m / epi.gate_div) * epi.gate_stride + n);
      float rv[4];
      if (resid_f32) {
        const float4 rr = *reinterpret_cast<const float4*>(static_cast<const float*>(epi.resid) + ro);
        rv[0] = rr.x; rv[1] = rr.y; rv[2] = rr.z; rv[3] = rr.w;
      } else {
        const uint2 rr = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(epi.resid) + ro);
        rv[0] = e_lo<H>(rr.x); rv[1] = e_hi<H>(rr.x); rv[2] = e_lo<H>(rr.y); rv[3] = e_hi<H>(rr.y);
      }
      v[0] = rv[0] + gv.x * v[0];
      v[1] = rv[1] + gv.y * v[1];
      v[2] = rv[2] + gv.z * v[2];
      v[3] = rv[3] + gv.w * v[3];
    }
    if (out_f32) {
      *reinterpret_cast<float4*>(static_cast<float*>(C) + co) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint2 o;
      o.x = e_pack2<H>(v[0], v[1]);
      o.y = e_pack2<H>(v[2], v[3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + co) = o;
    }
    return;
  }
  for (int e = 0; e < 4 && n + e < N; ++e) {
    float x = v[e];
    if (epi.flags & KX_EPI_BIAS) x += e2f<H>(epi.bias[n + e]);
    x = apply_act(x, act);
    if (gated) {
      const float rv = resid_f32 ? static_cast<const float*>(epi.resid)[ro + e]
                                 : e2f<H>(static_cast<const uint16_t*>(epi.resid)[ro + e]);
      x = rv + epi.gate[(m / epi.gate_div) * epi.gate_stride + n + e] * x;
    }
    if (out_f32)
      static_cast<float*>(C)[co + e] = x;
    else
      static_cast<uint16_t*>(C)[co + e] = f2e<H>(x);
  }
}

// The activation as a compile-time choice (ACT = the epilogue's activation code; -1: chosen at
// run time per value).
template <int ACT>
__device__ __forceinline__ float act_c(float v, int act) {
  if constexpr (ACT == 1) return fast_gelu_tanh(v);
  else if constexpr (ACT == 2) return fast_silu(v);
  else if constexpr (ACT == 0) return v;
  else return apply_act(v, act);
}

// One full-tile epilogue row piece: bias + activation (+ gated residual), then the store of 4
// consecutive columns. Values by value so that nothing of the caller's frame is addressed.
template <bool H, int GMODE, bool OUTF32, int ACT, typename ResidT>
__device__ __forceinline__ void epi_row4(float4 a4, ResidT res, float b0, float b1, float b2, float b3,
                                         int act, float4 gv, char* dst) {
  float v[4] = {a4.x + b0, a4.y + b1, a4.z + b2, a4.w + b3};
  if (ACT != 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = act_c<ACT>(v[e], act);
  }
  if constexpr (GMODE != 0) {
    float rv[4];
    if constexpr (GMODE == 2) {
      rv[0] = res.x; rv[1] = res.y; rv[2] = res.z; rv[3] = res.w;
    } else {
      rv[0] = e_lo<H>(res.x); rv[1] = e_hi<H>(res.x); rv[2] = e_lo<H>(res.y); rv[3] = e_hi<H>(res.y);
    }
    v[0] = rv[0] + gv.x * v[0];
    v[1] = rv[1] + gv.y * v[1];
    v[2] = rv[2] + gv.z * v[2];
    v[3] = rv[3] + gv.w * v[3];
  }
  if constexpr (OUTF32) {
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint2 o;
    o.x = e_pack2<H>(v[0], v[1]);
    o.y = e_pack2<H>(v[2], v[3]);
    *reinterpret_cast<uint2*>(dst) = o;
  }
}

// QB = 0: bf16 weights, DMA'd like the activations. QB = 4 / 8 (affine) and QMX8 (mxfp8): each
// stage DMAs the packed weight bytes and the scale (/ bias) words of its group, and every wave
// dequantizes its own weight fragments in registers (bit-exact, the arithmetic of dequant8)
// between the MFMAs of the previous k16 step: the stage's weights cross LDS once, packed, and no
// bf16 copy of them is written. TL: the affine weights are in the tiled layout (one contiguous
// block per 256-row tile and stage, see kx_qweight_tile_affine), else in the reference layout
// (one 16- or 32-byte piece per row).
template <int BM, int BN, int QB, bool TL, int GMODE, bool OUTF32, bool NR = false, bool H = false>
__global__ __launch_bounds__(256) void gemm_lds_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ W, int64_t ldw,
    QuantW qw, void* __restrict__ C, int64_t ldc, int M, int N, int K, Epilogue epi) {
  // stage geometry: dense products, 64-wide stages, in a 2-stage ring for the 256 x 256 and
  // 192 x 256 tiles and a 4-stage ring for the small tiles (whose few MFMAs per stage cannot
  // cover a one-stage prefetch); quantized products, 32-wide stages in a 4-stage ring. A row's
  // 16-byte slots are XOR-swizzled (by (r >> 1) & 7, resp. (r >> 2) & 3) so that the DMA writes
  // and the 32-row fragment reads are bank-conflict free.
  constexpr bool D64 = QB == 0;
  constexpr bool RING2 = D64 && BM * BN >= 192 * 256;
  constexpr int DBK = D64 ? DENSE_BK : 32;  // K per LDS stage
  constexpr int DROW = DBK * 2;             // bytes per LDS row
  constexpr int DCPR = DBK / 8;             // 16-byte chunks per row
  constexpr int DRPI = 64 / DCPR;           // rows one DMA instruction fills
  constexpr int DNS = RING2 ? 2 : 4;        // stages in the ring
  const auto dswz = [](int r) { return D64 ? (r >> 1) & 7 : (r >> 2) & 3; };
  constexpr int A_INST = BM / DRPI / 4;
  constexpr int QROW = DBK * qbits<QB>() / 8;                         // packed bytes per row
  constexpr int WQ_INST = QB ? BN * QROW / 1024 / 4 : 0;              // packed words, per wave
  constexpr int SB_BYTES = QB == QMX8 ? 4 : 8;                        // scale (bias) bytes per row
  constexpr int SB_INST = QB ? SB_BYTES * BN / 256 / 4 : 0;           // scale and bias pairs
  constexpr int W_INST = QB ? WQ_INST + SB_INST : BN / DRPI / 4;
  constexpr int PER = A_INST + W_INST;  // DMA instructions per wave per stage
  constexpr int W_BYTES = QB ? BN * QROW + BN * SB_BYTES : BN * DROW;
  constexpr int STAGE = BM * DROW + W_BYTES;
  constexpr int RING = DNS * STAGE;
  // wave layout: dense products 2 x 2 waves of (BM / 2) x (BN / 2); quantized weights 1 x 4 waves
  // of BM x (BN / 4), so that each weight column is dequantized by one wave only (a 2 x 2 layout
  // dequantizes every column twice) for the same LDS fragment traffic per MFMA as the dense form
  constexpr int WGM = QB ? 1 : 2, WGN = 4 / WGM;
  constexpr int WT_M = BM / WGM, WT_N = BN / WGN;
  constexpr int MB = WT_M / 32, NB = WT_N / 32;
  constexpr int KS = DBK / 16;
  static_assert(KS == (D64 ? 4 : 2), "k16 steps per stage");
  constexpr int DPS = (PER + KS - 1) / KS;  // DMA instructions per k16 step
  // At the wait in the last k16 step, stages kt+2 .. kt+NS-2 and the DMA of this iteration's
  // earlier steps may stay in flight: stage kt+1 is then complete.
  constexpr int NBEFORE = (KS - 1) * DPS < PER ? (KS - 1) * DPS : PER;
  constexpr int WAITN = RING2 ? 0 : (DNS - 3) * PER + NBEFORE;
  constexpr int PITCH = WT_N / 2 + 4;  // staged epilogue row, floats
  constexpr int EP_BYTES = 4 * WT_M * PITCH * 4;
  constexpr int SMEM = RING > EP_BYTES ? RING : EP_BYTES;
  static_assert(A_INST * DRPI * 4 == BM && MB >= 1 && NB >= 2, "tile");
  static_assert(QB == 0 ? (BN / DRPI / 4) * DRPI * 4 == BN : (BN == 256 && WQ_INST >= 1), "weight tile");
  static_assert(MB + NB <= 15 && WAITN >= 0, "pipeline");
  static_assert(!(TL && QB == QMX8), "mxfp8 weights are read in the reference layout only");
  static_assert(!H || (QB == 0 && !NR), "fp16 operands: the dense product without the norm epilogue");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WGM, wn = wave / WGM;
  const int lrow = lane & 31, lhalf = lane >> 5;
  if constexpr (QB == 0 && GMODE == 0 && OUTF32) {
    // split-K (grid.y > 1): workgroup row y multiplies K slice y (K is the slice length) and
    // writes its fp32 partial product to plane y of C (planes M * ldc floats apart)
    const int64_t y = blockIdx.y;
    A += y * K;
    W += y * K;
    C = static_cast<float*>(C) + y * (int64_t)M * ldc;
  }

  // tile coordinates (see lds_tile_of)
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int2 tile = lds_tile_of(blockIdx.x, tiles_m, tiles_n);
  if (epi.rows_desc) tile.x = tiles_m - 1 - tile.x;
  const int m0 = tile.x * BM, n0 = tile.y * BN;

  // per-lane DMA sources: lane -> row lane / DCPR of the instruction's rows, slot lane % DCPR;
  // rows past the end re-read the last row (in bounds; their results are never stored)
  const int r_in = lane / DCPR, slot = lane % DCPR;
  uint32_t vo[PER];
#pragma unroll
  for (int i = 0; i < A_INST; ++i) {
    const int r = (wave * A_INST + i) * DRPI + r_in;
    vo[i] = (uint32_t)(((int64_t)(min(m0 + r, M - 1) - m0) * lda + (slot ^ dswz(r)) * 8) * 2);
  }
  const char* a_base = reinterpret_cast<const char*>(A + (int64_t)m0 * lda);
  const char* w_base;   // bf16 weights, or the packed words
  const char* s_base = nullptr;  // scale pairs (bias pairs follow at b_base)
  const char* b_base = nullptr;
  const int64_t qrow_bytes = (int64_t)K * qbits<QB>() / 8, groups = K / 64;
  if constexpr (QB == 0) {
#pragma unroll
    for (int i = 0; i < W_INST; ++i) {
      const int r = (wave * W_INST + i) * DRPI + r_in;
      vo[A_INST + i] = (uint32_t)(((int64_t)(min(n0 + r, N - 1) - n0) * ldw + (slot ^ dswz(r)) * 8) * 2);
    }
    w_base = reinterpret_cast<const char*>(W + (int64_t)n0 * ldw);
  } else if constexpr (TL) {
    // tiled: the stage's packed words (BN * QROW bytes) and scale / bias pairs (BN * 8 bytes of
    // its 128-wide window) are contiguous blocks (8-bit rows: chunk swizzle as below)
#pragma unroll
    for (int i = 0; i < WQ_INST; ++i) {
      const int r = (wave * WQ_INST + i) * (1024 / QROW) + lane / (QROW / 16);
      const int chunk = QROW == 32 ? (lane & 1) ^ qswz(r) : 0;
      vo[A_INST + i] = (uint32_t)(r * QROW + chunk * 16);
    }
#pragma unroll
    for (int i = 0; i < SB_INST; ++i) vo[A_INST + WQ_INST + i] = (uint32_t)((wave * SB_INST + i) * 256 + lane * 4);
    const int64_t nb = n0 / BN;
    w_base = reinterpret_cast<const char*>(qw.words) + nb * (K / DBK) * (int64_t)(BN * QROW);
    s_base = reinterpret_cast<const char*>(qw.scales) + nb * (K / 128) * (int64_t)(BN * 8);
  } else {
    // packed words: RPW rows per instruction, QROW / 16 chunks per row; an 8-bit row's two
    // chunks trade places when (r >> 3) & 1, so that the 16-byte fragment reads of 16 rows
    // cover every bank once
    constexpr int RPW = 1024 / QROW;
#pragma unroll
    for (int i = 0; i < WQ_INST; ++i) {
      const int r = (wave * WQ_INST + i) * RPW + lane / (QROW / 16);
      const int chunk = QROW == 32 ? (lane & 1) ^ qswz(r) : 0;
      vo[A_INST + i] = (uint32_t)((int64_t)(min(n0 + r, N - 1) - n0) * qrow_bytes + chunk * 16);
    }
    // scale / bias pairs (mxfp8: scale-byte quads): 64 rows x 4 bytes per instruction
    const int64_t sb_row = QB == QMX8 ? K / 32 : groups * 2;  // bytes per row of the scale array
#pragma unroll
    for (int i = 0; i < SB_INST; ++i) {
      const int g = wave * SB_INST + i;
      const int r = (g % (BN / 64)) * 64 + lane;
      vo[A_INST + WQ_INST + i] = (uint32_t)((int64_t)(min(n0 + r, N - 1) - n0) * sb_row);
    }
    w_base = reinterpret_cast<const char*>(qw.words) + (int64_t)n0 * qrow_bytes;
    if constexpr (QB == QMX8) {
      s_base = reinterpret_cast<const char*>(qw.e8m0) + (int64_t)n0 * sb_row;
    } else {
      s_base = reinterpret_cast<const char*>(qw.scales) + (int64_t)n0 * sb_row;
      b_base = reinterpret_cast<const char*>(qw.biases) + (int64_t)n0 * sb_row;
    }
  }
  // dense operands: buffer loads (the tile bases as resources; lane offsets < 2^31, K offsets
  // < 2^23 by the dispatch's stride limits)
  const rsrc_t a_rsrc = raw_rsrc(a_base), w_rsrc = raw_rsrc(w_base);
  auto dma = [&](int i, uint8_t* buf, int k0) {
    if (i < A_INST) {
      buffer_lds16(a_rsrc, buf + (wave * A_INST + i) * DRPI * DROW, vo[i], (uint32_t)k0 * 2);
    } else if constexpr (QB == 0) {
      buffer_lds16(w_rsrc, buf + (BM + (wave * W_INST + i - A_INST) * DRPI) * DROW, vo[i], (uint32_t)k0 * 2);
    } else if (TL && i < A_INST + WQ_INST) {
      __builtin_amdgcn_global_load_lds((const void*)(w_base + (int64_t)(k0 / DBK) * (BN * QROW) + vo[i]),
                                       KX_LDS(buf + BM * DROW + (wave * WQ_INST + i - A_INST) * 1024), 16, 0, 0);
    } else if (TL) {
      const int g = wave * SB_INST + (i - A_INST - WQ_INST);
      __builtin_amdgcn_global_load_lds((const void*)(s_base + (int64_t)(k0 / 128) * (BN * 8) + vo[i]),
                                       KX_LDS(buf + BM * DROW + BN * QROW + g * 256), 4, 0, 0);
    } else if (i < A_INST + WQ_INST) {
      __builtin_amdgcn_global_load_lds((const void*)(w_base + (int64_t)k0 * qbits<QB>() / 8 + vo[i]),
                                       KX_LDS(buf + BM * DROW + (wave * WQ_INST + i - A_INST) * 1024), 16, 0, 0);
    } else if constexpr (QB == QMX8) {
      // the scale-byte quad holding group k0 / 32 (k0 / 32 rounded down to a multiple of 4)
      const int g = wave * SB_INST + (i - A_INST - WQ_INST);
      __builtin_amdgcn_global_load_lds((const void*)(s_base + (int64_t)((k0 >> 5) & ~3) + vo[i]),
                                       KX_LDS(buf + BM * DROW + BN * QROW + g * 256), 4, 0, 0);
    } else {
      // the pair of groups holding group k0 / 64 (k0 / 64 rounded down to even)
      const int g = wave * SB_INST + (i - A_INST - WQ_INST);
      const char* src = (g < BN / 64 ? s_base : b_base) + (int64_t)((k0 >> 6) & ~1) * 2 + vo[i];
      __builtin_amdgcn_global_load_lds((const void*)src, KX_LDS(buf + BM * DROW + BN * QROW + g * 256), 4, 0, 0);
    }
  };

  // fragment byte offsets, per k16 step (the MFMA A operand is the weight tile). Dense: step s
  // of lane half h covers k = 16 s + 8 h .. + 7 of the stage. Quantized: k = 16 h + 8 s .. + 7
  // (the same permutation of the sum on both operands), so that a lane's packed weight bytes of
  // both steps are contiguous and come in one read per stage.
  int a_off[KS][MB], w_off[KS][NB];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int c = QB ? 2 * lhalf + s : 2 * s + lhalf;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int r = wm * WT_M + j * 32 + lrow;
      a_off[s][j] = r * DROW + ((c ^ dswz(r)) << 4);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = wn * WT_N + i * 32 + lrow;
      w_off[s][i] = BM * DROW + r * DROW + ((c ^ dswz(r)) << 4);
    }
  }
  auto load_frags = [&](const uint8_t* buf, int s, bf16x8* af, bf16x8* wf) {
#pragma unroll
    for (int j = 0; j < MB; ++j) af[j] = *reinterpret_cast<const bf16x8*>(buf + a_off[s][j]);
    if constexpr (QB == 0) {
#pragma unroll
      for (int i = 0; i < NB; ++i) wf[i] = *reinterpret_cast<const bf16x8*>(buf + w_off[s][i]);
    }
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int stages = K / DBK;
  // dense: stage 0, and the first DH1 DMA instructions of stage 1 (the rest go out in stage 0's
  // first step); quantized: stages 0 .. NS-2
  constexpr int DH1 = (PER + 1) / 2;
  if constexpr (RING2) {
#pragma unroll
    for (int i = 0; i < PER; ++i) dma(i, smem, 0);
#pragma unroll
    for (int i = 0; i < DH1; ++i) dma(i, smem + STAGE, min(1, stages - 1) * DBK);
    wait_vmcnt<DH1>();
  } else {
#pragma unroll
    for (int p = 0; p < DNS - 1; ++p)
#pragma unroll
      for (int i = 0; i < PER; ++i) dma(i, smem + p * STAGE, min(p, stages - 1) * DBK);
    wait_vmcnt<(DNS - 2) * PER>();
  }
  KX_BARRIER();
  bf16x8 fa[2][MB], fw[2][NB];
  int cur_i = 0;
  if constexpr (QB != 0) {
    // ---- quantized mainloop: every wave dequantizes its own weight fragments in registers ----
    // A lane's packed bytes of weight block i for the whole stage (both k16 steps of its row)
    // and the row's scale (and bias) word; read once per stage, right after the stage's barrier.
    using Raw = typename std::conditional<qbits<QB>() == 4, uint2, uint4>::type;
    Raw raw[NB];
    uint32_t rsw[NB], rbw[NB];
    int wr_off[NB], ws_off[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = wn * WT_N + i * 32 + lrow;
      wr_off[i] = BM * DROW + (QROW == 16 ? r * 16 + 8 * lhalf : r * 32 + ((lhalf ^ qswz(r)) << 4));
      ws_off[i] = BM * DROW + BN * QROW + (TL && QB != QMX8 ? 8 * r : 4 * r);
    }
    // scale (and bias) of each block's rows for stage kt: affine, group kt / 2 of the pair (64-wide
    // groups); mxfp8, scale byte kt % 4 of the word (32-wide groups)
    float scl[NB], bia[NB];
    auto stage_scales = [&](int kt) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if constexpr (QB == QMX8) {
          scl[i] = e8m0_f32((rsw[i] >> (8 * (kt & 3))) & 255u);
          bia[i] = 0.0f;
        } else {
          const bool half = (kt >> 1) & 1;
          scl[i] = half ? hi_f(rsw[i]) : lo_f(rsw[i]);
          bia[i] = half ? hi_f(rbw[i]) : lo_f(rbw[i]);
        }
      }
    };
    // values 2p, 2p+1 of block i's fragment for k16 step s, as two bf16 (dequant8's arithmetic)
    auto dq_pair = [&](int i, int s, int p) -> uint32_t {
      if constexpr (QB == QMX8) {
        const uint32_t w = (2 * s + (p >> 1)) == 0 ? raw[i].x : (2 * s + (p >> 1)) == 1 ? raw[i].y
                           : (2 * s + (p >> 1)) == 2 ? raw[i].z : raw[i].w;
        const f32x2 v = (p & 1) ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
        return pack2(v.x * scl[i], v.y * scl[i]);
      } else if constexpr (QB == 8) {
        const uint32_t w = (2 * s + (p >> 1)) == 0 ? raw[i].x : (2 * s + (p >> 1)) == 1 ? raw[i].y
                           : (2 * s + (p >> 1)) == 2 ? raw[i].z : raw[i].w;
        const int b = 2 * (p & 1);
        return pack2(fmaf(scl[i], (float)((w >> (8 * b)) & 255u), bia[i]),
                     fmaf(scl[i], (float)((w >> (8 * b + 8)) & 255u), bia[i]));
      } else {
        // even nibbles in the low halves of the bytes of lo, odd ones in hi: each value is one
        // byte conversion (v_cvt_f32_ubyte), the masks are shared by the word's four pairs
        const uint32_t w = s ? raw[i].y : raw[i].x;
        uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        // the masked words opaque to the optimizer, which would otherwise fold the masks back
        // into one bit-field extract per value
        asm("" : "+v"(lo));
        asm("" : "+v"(hi));
        return pack2(fmaf(scl[i], (float)((lo >> (8 * p)) & 255u), bia[i]),
                     fmaf(scl[i], (float)((hi >> (8 * p)) & 255u), bia[i]));
      }
    };
    // the fragment under construction, four pairs
    uint32_t part[NB][4];
    auto dq_step = [&](int idx, int s) {  // pair idx of the step's NB * 4 pairs
      const int i = idx >> 2, p = idx & 3;
      part[i][p] = dq_pair(i, s, p);
    };
    auto dq_commit = [&](bf16x8* wf) {
#pragma unroll
      for (int i = 0; i < NB; ++i) wf[i] = __builtin_bit_cast(bf16x8, make_uint4(part[i][0], part[i][1], part[i][2], part[i][3]));
    };
    constexpr int NMF = NB * MB;
    constexpr int NPAIR = NB * 4;
    constexpr int SB_RD = QB == QMX8 || TL ? 1 : 2;  // scale (bias) reads per block
    constexpr int NRD1 = MB + NB * (1 + SB_RD);      // LDS reads at a stage's start
    constexpr int NRQ = NB * (1 + SB_RD);             // of which the packed weights and scales
    constexpr int QSPLIT = 4;                         // MFMAs before the wait for those
    static_assert(NMF > QSPLIT, "MFMAs per step");
    // LDS read r of a stage's start: the raw blocks and scale words (needed first, by the
    // dequantization of the stage's step 0), then the A fragments of its step 0
    auto stage_read = [&](int r, const uint8_t* buf) {
      if (r >= NRQ) {
        fa[0][r - NRQ] = *reinterpret_cast<const bf16x8*>(buf + a_off[0][r - NRQ]);
      } else if (r < NB) {
        raw[r] = *reinterpret_cast<const Raw*>(buf + wr_off[r]);
      } else {
        const int q = r - NB, i = q % NB;
        if constexpr (QB == QMX8) {
          rsw[i] = *reinterpret_cast<const uint32_t*>(buf + ws_off[i]);
        } else if constexpr (TL) {
          const uint2 pr = *reinterpret_cast<const uint2*>(buf + ws_off[i]);
          rsw[i] = pr.x;
          rbw[i] = pr.y;
        } else if (q < NB) {
          rsw[i] = *reinterpret_cast<const uint32_t*>(buf + ws_off[i]);
        } else {
          rbw[i] = *reinterpret_cast<const uint32_t*>(buf + ws_off[i] + 4 * BN);
        }
      }
    };

#pragma unroll
    for (int r = 0; r < NRD1; ++r) stage_read(r, smem);
    wait_lgkmcnt0();
    stage_scales(0);
#pragma unroll
    for (int q = 0; q < NPAIR; ++q) dq_step(q, 0);
    dq_commit(fw[0]);
    for (int kt = 0; kt < stages; ++kt) {
      const uint8_t* cur = smem + cur_i * STAGE;
      const int nxt_i = cur_i + 1 == DNS ? 0 : cur_i + 1;
      const uint8_t* nxt = smem + nxt_i * STAGE;
      uint8_t* iss = smem + (cur_i == 0 ? DNS - 1 : cur_i - 1) * STAGE;
      const int k_iss = min(kt + DNS - 1, stages - 1) * DBK;
      // step 0, in a fixed order: each MFMA, then its share of the pairs of step 1's weight
      // fragments (the arithmetic runs while the MFMA executes); the A fragments of step 1 and
      // the first DMA issues ride along the first MFMAs
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkmcnt0();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < NMF; ++q) {
        const int i = q / MB, j = q % MB;
        acc[i][j] = mfma32x32x16<H>(fw[0][i], fa[0][j], acc[i][j]);
        if (q < MB) fa[1][q] = *reinterpret_cast<const bf16x8*>(cur + a_off[1][q]);
        if (q < DPS && q < PER) dma(q, iss, k_iss);
#pragma unroll
        for (int idx = q * NPAIR / NMF; idx < (q + 1) * NPAIR / NMF; ++idx) dq_step(idx, 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      dq_commit(fw[1]);
      // step 1: stage kt+1 has landed for this wave and its reads of stage kt-1's buffer ended
      // one step ago; after the barrier this holds for every wave. The stage-start reads of stage
      // kt+1 and the remaining DMA issues ride along the first QSPLIT MFMAs; after the wait for
      // those reads, each further MFMA is followed by pairs of stage kt+1's step-0 fragments.
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkmcnt0();
      wait_vmcnt<WAITN>();
      KX_BARRIER();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < QSPLIT; ++q) {
        const int i = q / MB, j = q % MB;
        acc[i][j] = mfma32x32x16<H>(fw[1][i], fa[1][j], acc[i][j]);
#pragma unroll
        for (int r = q * NRD1 / QSPLIT; r < (q + 1) * NRD1 / QSPLIT; ++r) stage_read(r, nxt);
#pragma unroll
        for (int d = DPS + q * (PER - DPS) / QSPLIT; d < DPS + (q + 1) * (PER - DPS) / QSPLIT; ++d)
          dma(d, iss, k_iss);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_lgkmcnt<MB>();
      stage_scales(kt + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = QSPLIT; q < NMF; ++q) {
        const int i = q / MB, j = q % MB;
        acc[i][j] = mfma32x32x16<H>(fw[1][i], fa[1][j], acc[i][j]);
#pragma unroll
        for (int idx = (q - QSPLIT) * NPAIR / (NMF - QSPLIT); idx < (q - QSPLIT + 1) * NPAIR / (NMF - QSPLIT); ++idx)
          dq_step(idx, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      dq_commit(fw[0]);
      cur_i = nxt_i;
    }
  } else if constexpr (!RING2) {
    load_frags(smem, 0, fa[0], fw[0]);
    for (int kt = 0; kt < stages; ++kt) {
      const uint8_t* cur = smem + cur_i * STAGE;
      const int nxt_i = cur_i + 1 == DNS ? 0 : cur_i + 1;
      // stage kt+NS-1 goes into the buffer stage kt-1 used; past the end the last stage is
      // re-read into it, which keeps the loop free of branches and the vmcnt arithmetic uniform
      uint8_t* iss = smem + (cur_i == 0 ? DNS - 1 : cur_i - 1) * STAGE;
      const int k_iss = min(kt + DNS - 1, stages - 1) * DBK;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int b = s & 1;
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        if (s + 1 == KS) {
          // stage kt+1 has landed for this wave and its reads of cur are done; after the barrier
          // this holds for every wave, and nobody reads cur again before it is refilled
          wait_vmcnt<WAITN>();
          KX_BARRIER();
        }
        __builtin_amdgcn_sched_barrier(0);
        // after each MFMA, its share of the next step's fragment reads (after the last step:
        // stage kt+1's first) and of this step's DMA issues, in source order
        const uint8_t* rbuf = s + 1 < KS ? cur : smem + nxt_i * STAGE;
        const int rs = s + 1 < KS ? s + 1 : 0;
        constexpr int NRD = MB + NB, NMF = NB * MB;
        const int d0 = s * DPS, nd = PER - d0 < DPS ? (PER - d0 > 0 ? PER - d0 : 0) : DPS;
#pragma unroll
        for (int q = 0; q < NMF; ++q) {
          const int i = q / MB, j = q % MB;
          acc[i][j] = mfma32x32x16<H>(fw[b][i], fa[b][j], acc[i][j]);
#pragma unroll
          for (int r = q * NRD / NMF; r < (q + 1) * NRD / NMF; ++r) {
            if (r < MB) {
              fa[b ^ 1][r] = *reinterpret_cast<const bf16x8*>(rbuf + a_off[rs][r]);
            } else {
              fw[b ^ 1][r - MB] = *reinterpret_cast<const bf16x8*>(rbuf + w_off[rs][r - MB]);
            }
          }
#pragma unroll
          for (int d = q * nd / NMF; d < (q + 1) * nd / NMF; ++d) dma(d0 + d, iss, k_iss);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      cur_i = nxt_i;
    }
  } else {
    // Two 64-wide stages. Stage kt+2 goes into stage kt's buffer: its first DH1 DMA instructions
    // right after the barrier of stage kt's last k16 step (every wave has read that buffer's
    // last fragments by then), the rest during step 0 of stage kt+1; the barrier of stage
    // kt+1's last step waits for all of them. Past the end the last stage is re-read, which
    // keeps the loop free of branches and the vmcnt arithmetic uniform. Each MFMA is followed by
    // its share of the fragment reads and DMA issues, in source order (the compiler's own
    // placement bunched the DMA issues, ~10 VALU / SALU / VMEM instructions each, between two
    // MFMAs and left the matrix core idle: 5 % on every block shape).
    load_frags(smem, 0, fa[0], fw[0]);
    for (int kt = 0; kt < stages; ++kt) {
      uint8_t* cur = smem + (kt & 1) * STAGE;
      uint8_t* oth = smem + ((kt & 1) ^ 1) * STAGE;
      const int k1 = min(kt + 1, stages - 1) * DBK;
      const int k2 = min(kt + 2, stages - 1) * DBK;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int b = s & 1;
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        if (s + 1 == KS) {
          wait_vmcnt<0>();
          KX_BARRIER();
        }
        __builtin_amdgcn_sched_barrier(0);
        // the next step's fragments (after the last step: stage kt+1's first) and this step's
        // DMA issues, one group after each MFMA, in a fixed order
        const uint8_t* rbuf = s + 1 < KS ? cur : oth;
        const int rs = s + 1 < KS ? s + 1 : 0;
        constexpr int NRD = MB + NB, NMF = NB * MB;
        const int nd = s == 0 ? PER - DH1 : s + 1 == KS ? DH1 : 0;
        const int d0 = s == 0 ? DH1 : 0;
        uint8_t* dbuf = s == 0 ? oth : cur;
        const int dk = s == 0 ? k1 : k2;
#pragma unroll
        for (int q = 0; q < NMF; ++q) {
          const int i = q / MB, j = q % MB;
          acc[i][j] = mfma32x32x16<H>(fw[b][i], fa[b][j], acc[i][j]);
          if (q < MB) {
            fa[b ^ 1][q] = *reinterpret_cast<const bf16x8*>(rbuf + a_off[rs][q]);
          } else if (q < NRD) {
            fw[b ^ 1][q - MB] = *reinterpret_cast<const bf16x8*>(rbuf + w_off[rs][q - MB]);
          }
#pragma unroll
          for (int d = q * nd / NMF; d < (q + 1) * nd / NMF; ++d) dma(d0 + d, dbuf, dk);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  wait_vmcnt<0>();

  // ---- KX_EPI_QK_NORM_ROPE (NR): a wave's 128 columns are one head. A query or key head's wave
  // stages its two halves twice: the first time its store-loop lanes sum the squares of bias +
  // accumulator, rounded to bf16 as the projection's output would be, over their rows (each
  // row's 128 columns spread over 16 lanes and both halves), the second time they apply the
  // same rounded values' weighted RMSNorm and the adjacent-pair rotation in fp32
  // (each product of the rotation rounded before the sum, as the standalone norm + RoPE kernel
  // does) and store. Reading the accumulators only through the staging keeps them in place.
  bool bias_done = false;  // a norm wave: its store loop adds the bias
  int64_t nr_head = 0;
  const void* nr_w = nullptr;
  if constexpr (NR) {
    static_assert(WT_N == 128 && GMODE == 0 && !OUTF32 && QB == 0, "one 128-wide head per wave");
    const int64_t ncol0 = (int64_t)n0 + wn * WT_N;
    if (ncol0 < epi.k_end) {
      const bool isq = ncol0 < epi.q_end;
      nr_w = isq ? epi.nq : epi.nk;
      nr_head = isq ? ncol0 / 128 : (ncol0 - epi.q_end) / 128;
      bias_done = true;
    }
  }

  // ---- epilogue: the accumulator lane holds row m = j*32 + lrow and columns 8g + 4 lhalf + e of
  // block i; staged per half of the wave's columns into a private LDS region.
  const bool vec_ok = (ldc % 4 == 0) && (!(epi.flags & KX_EPI_GATED_RESIDUAL) || epi.ldr % 4 == 0);
  const bool full = vec_ok && m0 + BM <= M && n0 + BN <= N;
  float* ep = reinterpret_cast<float*>(smem) + wave * (WT_M * PITCH);
  constexpr int HALF_N = WT_N / 2;
  constexpr int LPR = HALF_N / 4;  // lanes per staged row
  constexpr int RPI_EP = 64 / LPR;   // rows per read-back iteration
  const int q = lane % LPR, rr = lane / LPR;
  const int act = (epi.flags >> 4) & 15;
  const bool has_bias = epi.flags & KX_EPI_BIAS;
  const int mrow0 = m0 + wm * WT_M;
  // Full tiles read the residual of all of a lane's rows of a half before any compute or store:
  // the loads are in flight together (C may alias the residual, so loads issued after a store
  // would wait for it), and the half's LDS staging and barrier run under their latency.
  constexpr int NROW = WT_M / RPI_EP;  // rows per lane per half
  static_assert(NROW * RPI_EP == WT_M, "epilogue rows");
  // residual rows are prefetched in chunks of PF rows. 256-row tiles hold all 256 accumulator
  // registers through the epilogue and have no room for the prefetch: they read the residual
  // row by row (PREF false); so do the 1 x 4 quantized layouts, whose lanes hold 192 or 256 rows.
  constexpr bool PREF = GMODE != 0 && BM <= 192 && WGM == 2;
  constexpr int PF = NROW > 24 ? NROW / 2 : NROW;
  constexpr int NCH = NROW / PF;
  static_assert(NCH * PF == NROW && PF % 4 == 0, "epilogue chunks");
  using ResidT = typename std::conditional<GMODE == 2, float4, uint2>::type;
  ResidT rpre[PREF ? PF : 1];
  const int64_t resid_es = GMODE == 2 ? 4 : 2;
  const char* rbase = GMODE == 0 ? nullptr
      : reinterpret_cast<const char*>(epi.resid) + ((int64_t)mrow0 * epi.ldr + n0 + wn * WT_N + 4 * q) * resid_es;
#define KX_PREFETCH_RESID(h, c)                                                                    \
  _Pragma("unroll") for (int k = 0; k < PF; ++k) rpre[k] = *reinterpret_cast<const ResidT*>(       \
      rbase + ((int64_t)(rr + ((c) * PF + k) * RPI_EP) * epi.ldr + (h) * HALF_N) * resid_es);
  if constexpr (PREF) {
    if (full) { KX_PREFETCH_RESID(0, 0) }
  }
  KX_BARRIER();  // every wave is done with the main loop's LDS
  // The half loop is not unrolled (its body is large); each half stages its accumulator blocks
  // under its own branch so that every accumulator index stays a compile-time constant.
#define KX_STAGE_BLOCK(ii, i)                                                                     \
  _Pragma("unroll") for (int j = 0; j < MB; ++j)                                                  \
  _Pragma("unroll") for (int g = 0; g < 4; ++g)                                                   \
      *reinterpret_cast<float4*>(ep + (j * 32 + lrow) * PITCH + (ii) * 32 + 8 * g + 4 * lhalf) =  \
          make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
  float nr_ss[NR ? NROW : 1], nr_inv[NR ? NROW : 1];  // NR: per row of this lane
#pragma unroll
  for (int k = 0; k < (NR ? NROW : 1); ++k) nr_ss[k] = 0.0f;
  const int passes = NR && bias_done ? 4 : 2;  // norm waves: two summing passes, then two storing
#pragma unroll 1
  for (int hp = 0; hp < passes; ++hp) {
    const int h = hp & 1;
    if constexpr (PREF) {
      if (h == 1 && full) { KX_PREFETCH_RESID(1, 0) }
    }
    if (h == 0) {
#pragma unroll
      for (int ii = 0; ii < NB / 2; ++ii) { KX_STAGE_BLOCK(ii, ii) }
    } else {
#pragma unroll
      for (int ii = 0; ii < NB / 2; ++ii) { KX_STAGE_BLOCK(ii, NB / 2 + ii) }
    }
#undef KX_STAGE_BLOCK
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int n = n0 + wn * WT_N + h * HALF_N + 4 * q;
    if (NR && bias_done && hp < 2) {
      // summing pass: this lane's 4 columns of each of its rows
      float b4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (has_bias) {
        const uint2 bb = *reinterpret_cast<const uint2*>(epi.bias + n);
        b4[0] = e_lo<H>(bb.x); b4[1] = e_hi<H>(bb.x); b4[2] = e_lo<H>(bb.y); b4[3] = e_hi<H>(bb.y);
      }
#pragma unroll
      for (int k = 0; k < (NR ? NROW : 1); ++k) {
        const float4 a4 = *reinterpret_cast<const float4*>(ep + (rr + k * RPI_EP) * PITCH + 4 * q);
        const float v0 = bf2f(f2bf(a4.x + b4[0])), v1 = bf2f(f2bf(a4.y + b4[1]));
        const float v2 = bf2f(f2bf(a4.z + b4[2])), v3 = bf2f(f2bf(a4.w + b4[3]));
        nr_ss[k] = fmaf(v3, v3, fmaf(v2, v2, fmaf(v1, v1, fmaf(v0, v0, nr_ss[k]))));
      }
      if (hp == 1) {
        // a row's 16 lanes (lane / LPR is the row slot) add their sums; then 1 / rms
#pragma unroll
        for (int k = 0; k < (NR ? NROW : 1); ++k) {
          static_assert(!NR || LPR == 16, "a staged row's lanes are one DPP row");
          nr_inv[k] = rsqrtf(row16_sum(nr_ss[k]) * (1.0f / 128.0f) + epi.n_eps);
        }
      }
    } else if (NR && bias_done) {
      // storing pass: bias, norm and rotation of 4 columns per lane of a query / key head (whole
      // inside N)
      const int d = h * HALF_N + 4 * q;  // column within the head; pairs (d, d+1), (d+2, d+3)
      float b4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, w4[4];
      if (has_bias) {
        const uint2 bb = *reinterpret_cast<const uint2*>(epi.bias + n);
        b4[0] = e_lo<H>(bb.x); b4[1] = e_hi<H>(bb.x); b4[2] = e_lo<H>(bb.y); b4[3] = e_hi<H>(bb.y);
      }
      if (epi.n_bf16) {
        const uint2 ww = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(nr_w) + d);
        w4[0] = lo_f(ww.x); w4[1] = hi_f(ww.x); w4[2] = lo_f(ww.y); w4[3] = hi_f(ww.y);
      } else {
        const float4 ww = *reinterpret_cast<const float4*>(static_cast<const float*>(nr_w) + d);
        w4[0] = ww.x; w4[1] = ww.y; w4[2] = ww.z; w4[3] = ww.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) w4[e] += epi.n_off;
      // Rows go in groups of GR: the group's table rows (a row clamped to M - 1 past the end) are
      // loaded together, so one memory latency covers GR rows. Table row of output row m: m / t_rows
      // by the host's magic number (m < 2^31: umulhi(m, magic) + m fits 32 bits).
      if constexpr (NR) {
        constexpr int GR = 8, NG = NROW / GR;
        static_assert(NROW % GR == 0, "NR row groups");
        const float* ct = epi.cosp + nr_head * epi.t_hs + d;
        const float* st = epi.sinp + nr_head * epi.t_hs + d;
        const uint32_t t_rows = (uint32_t)epi.t_rows, t_bs = (uint32_t)epi.t_bs, t_ld = (uint32_t)epi.t_ld;
        // the rows' offsets are the same in both storing passes: opaque here, so that they are
        // computed per pass and group rather than held in registers across the epilogue
        int mb = mrow0 + rr;
        asm volatile("" : "+v"(mb));
        uint16_t* crow = static_cast<uint16_t*>(C) + (int64_t)mb * ldc + n;
        // two groups of table rows in flight: group g + 1's loads are issued before group g's math
        float4 c4[2][GR], s4[2][GR];
        auto load_group = [&](int g0, float4* cg, float4* sg) {
#pragma unroll
          for (int j = 0; j < GR; ++j) {
            const uint32_t m = (uint32_t)min(mb + (g0 + j) * RPI_EP, M - 1);
            const uint32_t seq = (__umulhi(m, epi.t_magic) + m) >> epi.t_shift;
            const uint32_t trow = seq * t_bs + (m - seq * t_rows) * t_ld;  // < 2^31 (host check)
            cg[j] = *reinterpret_cast<const float4*>(ct + trow);
            sg[j] = *reinterpret_cast<const float4*>(st + trow);
          }
        };
        load_group(0, c4[0], s4[0]);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          if (gi + 1 < NG) load_group((gi + 1) * GR, c4[(gi + 1) & 1], s4[(gi + 1) & 1]);
          const float4* cg = c4[gi & 1];
          const float4* sg = s4[gi & 1];
#pragma unroll
          for (int j = 0; j < GR; ++j) {
            const int k = gi * GR + j;
            const int r = rr + k * RPI_EP;
            const int m = mb + k * RPI_EP;
            const float4 a4 = *reinterpret_cast<const float4*>(ep + r * PITCH + 4 * q);
            const float iv = nr_inv[k];
            const float av[4] = {a4.x, a4.y, a4.z, a4.w};
            const float c[4] = {cg[j].x, cg[j].y, cg[j].z, cg[j].w}, sn[4] = {sg[j].x, sg[j].y, sg[j].z, sg[j].w};
            float nv[4], o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) nv[e] = bf2f(f2bf(av[e] + b4[e])) * iv * w4[e];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
#pragma clang fp contract(off)
              const float a0 = nv[e] * c[e];
              const float b0 = (-nv[e + 1]) * sn[e];
              const float a1 = nv[e + 1] * c[e + 1];
              const float b1 = nv[e] * sn[e + 1];
              o[e] = a0 + b0;
              o[e + 1] = a1 + b1;
            }
            uint2 sv;
            sv.x = pack2(o[0], o[1]);
            sv.y = pack2(o[2], o[3]);
            if (m < M) *reinterpret_cast<uint2*>(crow + (int64_t)(k * RPI_EP) * ldc) = sv;
          }
          // keeps group g + 2's loads (and their address arithmetic) below this group's math
          asm volatile("" ::: "memory");
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if (full) {
      // column data is fixed per lane: bias, and the gate when one gate row covers the rows
      float b4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (has_bias) {
        const uint2 bb = *reinterpret_cast<const uint2*>(epi.bias + n);
        b4[0] = e_lo<H>(bb.x); b4[1] = e_hi<H>(bb.x); b4[2] = e_lo<H>(bb.y); b4[3] = e_hi<H>(bb.y);
      }
      const int64_t gstride = epi.gate_stride, gdiv = epi.gate_div;
      const bool gate_const = GMODE == 0 || gstride == 0 || (mrow0 / gdiv) == ((mrow0 + WT_M - 1) / gdiv);
      float4 g4c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (GMODE != 0 && gate_const) g4c = *reinterpret_cast<const float4*>(epi.gate + (mrow0 / gdiv) * gstride + n);
      char* cbase = reinterpret_cast<char*>(C) + ((int64_t)mrow0 * ldc + n) * (OUTF32 ? 4 : 2);
      // the rows with the activation fixed at compile time (a run-time choice per value put a
      // chain of scalar branches around every value and serialised them)
      auto full_rows = [&](auto act_tag, auto gate_tag) {
        constexpr int ACT = decltype(act_tag)::value;
        constexpr bool GC = decltype(gate_tag)::value;  // one gate row covers the wave's rows
        if constexpr (!PREF) {
#pragma unroll 4
          for (int r = rr; r < WT_M; r += RPI_EP) {
            ResidT res{};
            float4 gv = g4c;
            if constexpr (GMODE != 0) {
              res = *reinterpret_cast<const ResidT*>(rbase + ((int64_t)r * epi.ldr + h * HALF_N) * resid_es);
              if constexpr (!GC) {
                const int64_t grow = gdiv == 1 ? (int64_t)(mrow0 + r) : (int64_t)(mrow0 + r) / gdiv;
                gv = *reinterpret_cast<const float4*>(epi.gate + grow * gstride + n);
              }
            }
            epi_row4<H, GMODE, OUTF32, ACT>(*reinterpret_cast<const float4*>(ep + r * PITCH + 4 * q), res, b4[0],
                                         b4[1], b4[2], b4[3], act, gv, cbase + (int64_t)r * ldc * (OUTF32 ? 4 : 2));
          }
        } else {
          // groups of 4 rows: their staged reads together, then their stores (bounded registers:
          // the prefetched residual stays live, the staged values of one group at a time)
          constexpr int GR = 4;
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
            if (c > 0) { KX_PREFETCH_RESID(h, c) }
#pragma unroll
            for (int k0 = 0; k0 < PF; k0 += GR) {
              float4 a4[GR];
#pragma unroll
              for (int k = 0; k < GR; ++k)
                a4[k] = *reinterpret_cast<const float4*>(ep + (rr + (c * PF + k0 + k) * RPI_EP) * PITCH + 4 * q);
#pragma unroll
              for (int k = 0; k < GR; ++k) {
                const int r = rr + (c * PF + k0 + k) * RPI_EP;
                float4 gv = g4c;
                if constexpr (!GC) {
                  const int64_t grow = gdiv == 1 ? (int64_t)(mrow0 + r) : (int64_t)(mrow0 + r) / gdiv;
                  gv = *reinterpret_cast<const float4*>(epi.gate + grow * gstride + n);
                }
                epi_row4<H, GMODE, OUTF32, ACT>(a4[k], rpre[k0 + k], b4[0], b4[1], b4[2], b4[3], act, gv,
                                             cbase + (int64_t)r * ldc * (OUTF32 ? 4 : 2));
              }
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
      };
      using Const = std::true_type;
      using PerRow = std::integral_constant<bool, GMODE == 0>;  // GMODE 0 reads no gate
      if (act == 0 && gate_const) full_rows(std::integral_constant<int, 0>{}, Const{});
      else if (act == 0) full_rows(std::integral_constant<int, 0>{}, PerRow{});
      else if (GMODE == 0 && act == 1) full_rows(std::integral_constant<int, GMODE == 0 ? 1 : -1>{}, Const{});
      else if (GMODE == 0 && act == 2) full_rows(std::integral_constant<int, GMODE == 0 ? 2 : -1>{}, Const{});
      else full_rows(std::integral_constant<int, -1>{}, PerRow{});
    } else {
#pragma unroll 2
      for (int r = rr; r < WT_M; r += RPI_EP) {
        const int m = mrow0 + r;
        const float4 a4 = *reinterpret_cast<const float4*>(ep + r * PITCH + 4 * q);
        if (m < M && n < N) {
          float v[4] = {a4.x, a4.y, a4.z, a4.w};
          epilogue_store4<H>(v, m, n, N, epi, C, ldc, vec_ok);
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
#undef KX_PREFETCH_RESID
}

// ---- skinny kernel (N <= 64: the gate-logit projections) ------------------------------------
//
// One workgroup per R rows x 32 columns, R = ceil(M / 256) (at least 16, at most 128), so that the
// rows spread evenly over the 256 CUs: the kernel is bound by each CU's operand stream, and 32-row
// workgroups (288 of them at 9216 rows) left 32 CUs with twice the rows of the others. The R rows
// are RB = ceil(R / 16) MFMA row blocks; rows past R or M re-read the last valid row (the same
// cache lines as its own lanes) and are not stored. The NWK waves split K into NWK slices and
// read both MFMA operands straight from global memory (the weight is a few hundred KB and stays
// in L2, each activation row is read once), then add their partial tiles through LDS. The products are
// 16x16x32 MFMAs: a 16-byte operand load then spans 16 rows (four lanes of 64 contiguous bytes per
// row) instead of the 32 rows of a 32x32x16 operand, which halves the cache lines each load
// instruction touches, the limit of this kernel.
// Quantized weights are dequantized in registers with the arithmetic of the other kernels.
// One 16x16x32 MFMA on 16-bit operands (bf16, or fp16 with H).
template <bool H>
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (H)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int QB, int NWK, int RB, bool H = false>
__global__ __launch_bounds__(NWK * 64) void gemm_skinny_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ W, int64_t ldw,
    QuantW qw, void* __restrict__ C, int64_t ldc, int M, int N, int K, int R, Epilogue epi) {
  __shared__ __attribute__((aligned(16))) float part[NWK][2 * RB * 4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int m0 = blockIdx.x * R, n0 = blockIdx.y * 32;
  const int mend = min(m0 + R, M);
  // operand rows of this lane: activation rows m0 + 16 rb + l16 (clamped to the last valid row),
  // weight rows n0 + 16 cb + l16
  int wrow_i[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) wrow_i[b] = min(n0 + 16 * b + l16, N - 1);
  const uint16_t* arow[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) arow[b] = A + (int64_t)min(m0 + 16 * b + l16, mend - 1) * lda + 8 * lq;
  const int kq = K / NWK, kbeg = wave * kq;
  // accumulator (cb, rb): lane holds weight rows n0 + 16 cb + 4 lq + e, activation row m0 + 16 rb + l16
  f32x4 acc[2][RB];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[cb][rb][e] = 0.0f;
  auto wfrag = [&](int n, int k) -> bf16x8 {  // row n, this lane's 8 values start at k (k % 8 == 0)
    if constexpr (QB == 0) {
      return *reinterpret_cast<const bf16x8*>(W + (int64_t)n * ldw + k);
    } else if constexpr (QB == QMX8) {
      const float sc = e8m0_f32(qw.e8m0[(int64_t)n * (K / 32) + k / 32]);
      const uint32_t* wd = qw.words + (int64_t)n * (K / 4) + k / 4;
      uint32_t tmp[2] = {wd[0], wd[1]};
      return __builtin_bit_cast(bf16x8, dequant8<QMX8>(tmp, sc, 0.0f));
    } else {
      const int64_t g = (int64_t)n * (K / 64) + k / 64;
      const float sc = bf2f(qw.scales[g]), bi = bf2f(qw.biases[g]);
      const uint32_t* wd = qw.words + (int64_t)n * (K * QB / 32) + k * QB / 32;
      uint32_t tmp[2] = {wd[0], QB == 8 ? wd[1] : 0u};
      return __builtin_bit_cast(bf16x8, dequant8<QB>(tmp, sc, bi));
    }
  };
#pragma unroll 2
  for (int k = kbeg; k < kbeg + kq; k += 32) {
    const bf16x8 w0 = wfrag(wrow_i[0], k + 8 * lq), w1 = wfrag(wrow_i[1], k + 8 * lq);
    bf16x8 x[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) x[b] = *reinterpret_cast<const bf16x8*>(arow[b] + k);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      acc[0][b] = mfma16x16x32<H>(w0, x[b], acc[0][b]);
      acc[1][b] = mfma16x16x32<H>(w1, x[b], acc[1][b]);
    }
  }
#pragma unroll
  for (int a = 0; a < 2 * RB; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) part[wave][4 * a + e][lane] = acc[a / RB][a % RB][e];
  __syncthreads();
  // wave w finishes accumulators a = w, w + NWK, ...: (cb, rb) = (a / RB, a % RB), 4 consecutive
  // columns of one row per lane
  const bool vec_ok = (ldc % 4 == 0) && (!(epi.flags & KX_EPI_GATED_RESIDUAL) || epi.ldr % 4 == 0);
  for (int a = wave; a < 2 * RB; a += NWK) {
    const int cb = a / RB, rb = a % RB;
    const int row = m0 + 16 * rb + l16;
    const int col = n0 + 16 * cb + 4 * lq;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int p = 0; p < NWK; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += part[p][4 * a + e][lane];
    if (row < mend && col < N) epilogue_store4<H>(v, row, col, N, epi, C, ldc, vec_ok);
  }
}

// LDS-staged form for bf16 / fp16 weights and K % 256 == 0. The register form's 16-byte operand
// loads cover four lanes (64 bytes) of a row: every L1 -> L2 request is half a cache line, and the
// per-CU stream (requests in flight x latency) holds the activation read to ~2.4 TB/s. Here each
// wave streams its K quarter through a private ring of SKS stages in LDS: per stage its R
// activation rows and 32 weight rows x 64 K, DMA'd by buffer loads of 8 rows x 128 bytes (one
// full-line request per row), slots XOR-swizzled by (row >> 1) & 7 so that the 16-row fragment
// reads are conflict free. A wave only reads stages it copied itself, so the ring needs its own
// vmcnt waits and no barrier.
template <int A_I, bool H>
__global__ __launch_bounds__(256) void gemm_skinny_lds_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ W, int64_t ldw,
    void* __restrict__ C, int64_t ldc, int M, int N, int K, int R, Epilogue epi) {
  constexpr int SKS = 3;                          // stages per wave ring
  constexpr int AROWS = A_I * 8;                  // activation rows per stage (R <= AROWS)
  constexpr int RB = (AROWS + 15) / 16;           // MFMA row blocks; rows past AROWS read the
                                                  // weight rows that follow (never stored)
  constexpr int W_I = 4;                          // weight DMA instructions per stage
  constexpr int STG = (AROWS + 32) * 128;         // bytes per stage
  constexpr int RING_W = SKS * STG;               // bytes per wave
  constexpr int PART = 4 * 2 * RB * 4 * 64 * 4;   // partial tiles of the 4 waves
  constexpr int SMEM = 4 * RING_W > PART ? 4 * RING_W : PART;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int m0 = blockIdx.x * R, n0 = blockIdx.y * 32;
  const int mend = min(m0 + R, M);
  uint8_t* ring = smem + wave * RING_W;
  // DMA lanes: row lane / 8 of the instruction's 8, 16-byte slot lane % 8 (global chunk slot ^ swz)
  const int r8 = lane >> 3, slot = lane & 7;
  const int kq = K / 4, kbeg = wave * kq, nst = kq / 64;
  uint32_t av[A_I], wv[W_I];
#pragma unroll
  for (int i = 0; i < A_I; ++i) {
    const int r = 8 * i + r8;
    av[i] = (uint32_t)(((int64_t)(min(m0 + r, mend - 1) - m0) * lda + kbeg + 8 * (slot ^ ((r >> 1) & 7))) * 2);
  }
#pragma unroll
  for (int i = 0; i < W_I; ++i) {
    const int r = 8 * i + r8;
    wv[i] = (uint32_t)(((int64_t)(min(n0 + r, N - 1) - n0) * ldw + kbeg + 8 * (slot ^ ((r >> 1) & 7))) * 2);
  }
  const rsrc_t a_rsrc = raw_rsrc(A + (int64_t)m0 * lda), w_rsrc = raw_rsrc(W + (int64_t)n0 * ldw);
  auto issue = [&](int st) {  // stage st of this wave's K quarter (clamped: re-reads the last)
    uint8_t* buf = ring + (st % SKS) * STG;
    const uint32_t ko = (uint32_t)(min(st, nst - 1) * 64 * 2);
#pragma unroll
    for (int i = 0; i < A_I; ++i) buffer_lds16(a_rsrc, buf + i * 1024, av[i], ko);
#pragma unroll
    for (int i = 0; i < W_I; ++i) buffer_lds16(w_rsrc, buf + AROWS * 128 + i * 1024, wv[i], ko);
  };
  // fragment offsets: row r, 16-byte chunk c = 4 h + lq of k32 half h
  int fo[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) fo[h] = l16 * 128 + (((4 * h + lq) ^ ((l16 >> 1) & 7)) << 4);
  f32x4 acc[2][RB];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[cb][rb][e] = 0.0f;
#pragma unroll
  for (int st = 0; st < SKS - 1; ++st) issue(st);
  for (int st = 0; st < nst; ++st) {
    // stage st landed (stage st + 1 may still be in flight)
    wait_vmcnt<(SKS - 2) * (A_I + W_I)>();
    const uint8_t* buf = ring + (st % SKS) * STG;
    bf16x8 wf[2][2], xf[2][RB];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // 16-row blocks are 2 KB apart; the swizzle depends on the row within its block only
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        wf[h][cb] = *reinterpret_cast<const bf16x8*>(buf + AROWS * 128 + cb * 2048 + fo[h]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) xf[h][rb] = *reinterpret_cast<const bf16x8*>(buf + rb * 2048 + fo[h]);
    }
    wait_lgkmcnt0();
    // the slot of stage st + SKS - 1 is stage st - 1's: read out one iteration ago
    issue(st + SKS - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        acc[0][rb] = mfma16x16x32<H>(wf[h][0], xf[h][rb], acc[0][rb]);
        acc[1][rb] = mfma16x16x32<H>(wf[h][1], xf[h][rb], acc[1][rb]);
      }
  }
  wait_vmcnt<0>();
  __syncthreads();
  float* part = reinterpret_cast<float*>(smem);  // [wave][2 RB * 4][64]
#pragma unroll
  for (int a = 0; a < 2 * RB; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) part[(wave * 2 * RB * 4 + 4 * a + e) * 64 + lane] = acc[a / RB][a % RB][e];
  __syncthreads();
  const bool vec_ok = (ldc % 4 == 0) && (!(epi.flags & KX_EPI_GATED_RESIDUAL) || epi.ldr % 4 == 0);
  for (int a = wave; a < 2 * RB; a += 4) {
    const int cb = a / RB, rb = a % RB;
    const int row = m0 + 16 * rb + l16;
    const int col = n0 + 16 * cb + 4 * lq;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += part[(p * 2 * RB * 4 + 4 * a + e) * 64 + lane];
    if (row < mend && col < N) epilogue_store4<H>(v, row, col, N, epi, C, ldc, vec_ok);
  }
}

template <bool H, int AI>
void launch_skinny_lds_ai(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, void* c, int64_t ldc,
                          int m, int n, int k, int r, const Epilogue& epi, hipStream_t s) {
  const dim3 grid((unsigned)((m + r - 1) / r), (unsigned)((n + 31) / 32));
  gemm_skinny_lds_kernel<AI, H><<<grid, 256, 0, s>>>(a, lda, w, ldw, c, ldc, m, n, k, r, epi);
}

// Rows per skinny workgroup (see above) and its launch.
template <int QB, bool H, int RB>
void launch_skinny_rb(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw, void* c,
                      int64_t ldc, int m, int n, int k, int r, const Epilogue& epi, hipStream_t s) {
  const dim3 grid((unsigned)((m + r - 1) / r), (unsigned)((n + 31) / 32));
  gemm_skinny_kernel<QB, 4, RB, H><<<grid, 256, 0, s>>>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi);
}

template <int QB, bool H>
void launch_skinny(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw, void* c,
                   int64_t ldc, int m, int n, int k, const Epilogue& epi, hipStream_t s) {
  if (QB == 0 && k % 256 == 0 && lda <= (1 << 22) && ldw <= (1 << 22)) {
    // rows per workgroup: the rows spread over the 256 CUs in the fewest rounds of at most 64
    // rows (at least 16)
    const int per_cu = (m + 255) / 256, rounds = (per_cu + 63) / 64;
    const int r = std::max((m + 256 * rounds - 1) / (256 * rounds), 16);
    switch ((r + 7) / 8) {
      case 2: return launch_skinny_lds_ai<H, 2>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      case 3: return launch_skinny_lds_ai<H, 3>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      case 4: return launch_skinny_lds_ai<H, 4>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      case 5: return launch_skinny_lds_ai<H, 5>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      case 6: return launch_skinny_lds_ai<H, 6>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      case 7: return launch_skinny_lds_ai<H, 7>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
      default: return launch_skinny_lds_ai<H, 8>(a, lda, w, ldw, c, ldc, m, n, k, r, epi, s);
    }
  }
  const int r = std::min(std::max((m + 255) / 256, 16), 128);
  switch ((r + 15) / 16) {
    case 1: return launch_skinny_rb<QB, H, 1>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
    case 2: return launch_skinny_rb<QB, H, 2>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
    case 3: return launch_skinny_rb<QB, H, 3>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
    case 4: return launch_skinny_rb<QB, H, 4>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
    case 5:
    case 6: return launch_skinny_rb<QB, H, 6>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
    default: return launch_skinny_rb<QB, H, 8>(a, lda, w, ldw, qw, c, ldc, m, n, k, r, epi, s);
  }
}

// ---- dispatch ---------------------------------------------------------------------------------

enum TileCfg { T256x256 = 0, T256x128 = 1, T128x128 = 2, T64x64 = 3, T128x64 = 4 };

template <int BM, int BN, int WM, int WN, int QB, bool H = false>
int launch_cfg(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw,
               void* c, int64_t ldc, int m, int n, int k, const Epilogue& epi,
               hipStream_t s) {
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  gemm_kernel<BM, BN, WM, WN, QB, H><<<tiles, WM * WN * 64, 0, s>>>(a, lda, w, ldw, qw, c, ldc, m, n,
                                                                k, epi);
  return KX_OK;
}

int pick_cfg(int64_t m, int64_t n) {
  const char* env = getenv("KX355_GEMM_TILE");
  if (env && *env) {
    const int v = atoi(env);
    if (v >= 0 && v <= 4) return v;
  }
  if (m < 512 || n < 512) return (m * n >= 256 * 1024) ? T128x64 : T64x64;
  // Prefer the largest tile whose last wave of workgroups keeps the 256 CUs mostly busy.
  auto eff = [](int64_t tiles) {
    const int64_t waves = (tiles + 255) / 256;
    return (double)tiles / (double)(waves * 256);
  };
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256);
  const int64_t t128 = ((m + 255) / 256) * ((n + 127) / 128);
  if (eff(t256) >= 0.85) return T256x256;
  if (eff(t128) >= 0.85 || t128 >= 1024) return T256x128;
  return T128x128;
}

// Whether a product visits its tile rows last to first. Every producer of an activation in
// this library writes its rows in ascending order, so the last rows written are the ones most
// likely still in the 256 MB memory-side cache. When the input is too large for that cache to
// hold whole (above 128 MiB: the 9216 x 16384 feed-forward hidden state, 302 MB, read by the
// down projection right after the up projection wrote it), reading its rows newest first turns
// part of the operand stream into cache hits (down projection 964 -> 927 us in the config-3
// block). The order of tiles does not change any result.
bool rows_last_first(int64_t m, int64_t k) { return m * k * 2 > (128ll << 20); }

template <int BM, int BN, int QB, bool TL, int GMODE, bool OUTF32, bool NR = false, bool H = false>
int launch_lds_t(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw, void* c,
                 int64_t ldc, int m, int n, int k, const Epilogue& epi, hipStream_t s) {
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  Epilogue e = epi;
  e.rows_desc = rows_last_first(m, k);
  gemm_lds_kernel<BM, BN, QB, TL, GMODE, OUTF32, NR, H><<<tiles, 256, 0, s>>>(a, lda, w, ldw, qw, c, ldc, m, n, k, e);
  return KX_OK;
}

// Residual mode (none / bf16 / fp32) and output type select the epilogue specialisation.
template <int BM, int BN, int QB, bool TL = false, bool H = false>
int launch_lds(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw, void* c,
               int64_t ldc, int m, int n, int k, const Epilogue& epi, hipStream_t s) {
  const int gmode = (epi.flags & KX_EPI_GATED_RESIDUAL) ? ((epi.flags & KX_EPI_RESID_F32) ? 2 : 1) : 0;
  const bool out32 = epi.flags & KX_EPI_OUT_F32;
  switch (gmode * 2 + (out32 ? 1 : 0)) {
    case 0: return launch_lds_t<BM, BN, QB, TL, 0, false, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
    case 1: return launch_lds_t<BM, BN, QB, TL, 0, true, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
    case 2: return launch_lds_t<BM, BN, QB, TL, 1, false, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
    case 3: return launch_lds_t<BM, BN, QB, TL, 1, true, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
    case 4: return launch_lds_t<BM, BN, QB, TL, 2, false, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
    default: return launch_lds_t<BM, BN, QB, TL, 2, true, false, H>(a, lda, w, ldw, qw, c, ldc, m, n, k, epi, s);
  }
}

// Tile for the direct-to-LDS kernel: the fewest rounds of 256 workgroups, weighted by the
// tile's relative speed (a bigger tile reuses each LDS byte more). 0: 256x256, 1: 192x256,
// 2: 128x128.
int pick_lds_cfg(int64_t m, int64_t n) {
  const char* env = getenv("KX355_GEMM_LDS_TILE");
  if (env && *env) {
    const int v = atoi(env);
    if (v >= 0 && v <= 3) return v;
  }
  // tiles 256x256, 192x256, 128x128 and (for a few hundred rows, e.g. the text K/V projection)
  // 64x128, which fills the CUs where 128x128 leaves half of them idle. Speeds per unit of tile
  // area relative to 256x256, measured: 192x256 runs 3-5 % slower per FLOP at 9216 and 27 280
  // rows (it moves 17 % more bytes per FLOP through L2 and LDS)
  const int64_t bm[4] = {256, 192, 128, 64}, bn[4] = {256, 256, 128, 128};
  const double speed[4] = {1.0, 0.93, 0.8, 0.6};
  int best = 0;
  double best_cost = 0.0;
  for (int i = 0; i < 4; ++i) {
    const int64_t tiles = ((m + bm[i] - 1) / bm[i]) * ((n + bn[i] - 1) / bn[i]);
    const double cost = (double)((tiles + 255) / 256) * (double)(bm[i] * bn[i]) / speed[i];
    if (i == 0 || cost < best_cost) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

template <int QB, bool H = false>
int dispatch(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, QuantW qw,
             void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, const Epilogue& epi,
             hipStream_t s) {
  const char* legacy = getenv("KX355_GEMM_TILE");
  const bool use_legacy = legacy && *legacy;
  if (n <= 64 && k % 128 == 0 && !use_legacy) {
    launch_skinny<QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
    return KX_OK;
  }
  // the direct-to-LDS kernel keeps per-lane 32-bit byte offsets within a 256-row tile
  if (QB == 0 && k % DENSE_BK == 0 && lda <= (1 << 22) && ldw <= (1 << 22) && !use_legacy) {
    switch (pick_lds_cfg(m, n)) {
      case 0: return launch_lds<256, 256, 0, false, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
      case 1: return launch_lds<192, 256, 0, false, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
      case 2: return launch_lds<128, 128, 0, false, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
      default: return launch_lds<64, 128, 0, false, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
    }
  }
  // quantized weights: the direct-to-LDS kernel with in-LDS dequantization needs whole 128-wide
  // K blocks (scale / bias pairs of two groups), 16-byte aligned packed rows and 4-byte aligned
  // scale / bias rows; tile 2 (or a narrow N) selects the register-staged kernel
  // (a few hundred rows leave most CUs idle with its 192 / 256-row tiles: they take the
  // register-staged kernel's small tiles instead)
  const bool sb_aligned = QB == QMX8 ? (reinterpret_cast<uintptr_t>(qw.e8m0) & 3) == 0
                                     : (reinterpret_cast<uintptr_t>(qw.scales) & 3) == 0 &&
                                           (reinterpret_cast<uintptr_t>(qw.biases) & 3) == 0;
  if (QB != 0 && k % 128 == 0 && lda <= (1 << 22) && n >= 128 && m >= 512 && !use_legacy &&
      aligned16(qw.words) && sb_aligned) {
    const int cfg = pick_lds_cfg(m, n);
    const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256), t192 = ((m + 191) / 192) * ((n + 255) / 256);
    const bool tall = cfg == 0 || (cfg != 1 && (t256 + 255) / 256 * 256 <= (t192 + 255) / 256 * 192);
    if (cfg != 2 || !getenv("KX355_GEMM_LDS_TILE")) {
      if (tall) return launch_lds<256, 256, QB>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
      return launch_lds<192, 256, QB>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
    }
  }
  switch (pick_cfg(m, n)) {
    case T256x256:
      return launch_cfg<256, 256, 2, 2, QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k,
                                            epi, s);
    case T256x128:
      return launch_cfg<256, 128, 2, 2, QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k,
                                            epi, s);
    case T128x128:
      return launch_cfg<128, 128, 2, 2, QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k,
                                            epi, s);
    case T128x64:
      return launch_cfg<128, 64, 2, 2, QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k,
                                           epi, s);
    default:
      return launch_cfg<64, 64, 2, 2, QB, H>(a, lda, w, ldw, qw, c, ldc, (int)m, (int)n, (int)k, epi,
                                          s);
  }
}

// Split-K reduction: c = epilogue(sum over the planes of the fp32 partial products), 4 columns
// of one row per thread (the planes are (M, N) fp32, N a multiple of 4).
template <bool H>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ parts, int splits,
                                                            int M, int N, void* __restrict__ C, int64_t ldc,
                                                            Epilogue epi, bool vec_ok) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = N / 4;
  if (idx >= (int64_t)M * per_row) return;
  const int m = (int)(idx / per_row), n = (int)(idx - m * per_row) * 4;
  const int64_t plane = (int64_t)M * N;
  float4 acc = *reinterpret_cast<const float4*>(parts + (int64_t)m * N + n);
  for (int y = 1; y < splits; ++y) {
    const float4 p = *reinterpret_cast<const float4*>(parts + y * plane + (int64_t)m * N + n);
    acc.x += p.x;
    acc.y += p.y;
    acc.z += p.z;
    acc.w += p.w;
  }
  float v[4] = {acc.x, acc.y, acc.z, acc.w};
  epilogue_store4<H>(v, m, n, N, epi, C, ldc, vec_ok);
}

template <int BM, int BN, bool H>
int launch_splitk(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, float* parts, int m, int n,
                  int k, int splits, hipStream_t s) {
  const dim3 grid((unsigned)(((m + BM - 1) / BM) * ((n + BN - 1) / BN)), (unsigned)splits);
  const Epilogue plain{nullptr, nullptr, 0, nullptr, 1, 0, KX_EPI_OUT_F32};
  gemm_lds_kernel<BM, BN, 0, false, 0, true, false, H><<<grid, 256, 0, s>>>(a, lda, w, ldw, QuantW{}, parts, n, m, n,
                                                                   k / splits, plain);
  return KX_OK;
}

// Tiled affine weights: for 256-row tile nb and 32-wide K stage kb, the rows' packed bytes of the
// stage are one block of 256 * (32 * bits / 8) bytes; for the 128-wide window p, the rows'
// (scale 2p, scale 2p+1, bias 2p, bias 2p+1) are one block of 256 * 8 bytes. Rows past n repeat
// row n - 1 (their products are never stored).
template <int BITS>
__global__ __launch_bounds__(256) void tile_weights_kernel(const uint32_t* __restrict__ words,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint16_t* __restrict__ biases,
                                                           uint8_t* __restrict__ wt, uint8_t* __restrict__ sbt,
                                                           int64_t n, int64_t k) {
  constexpr int QROW = 32 * BITS / 8;
  const int64_t npad = (n + 255) / 256 * 256;
  const int64_t kb_count = k / 32, p_count = k / 128;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows_x_kb = npad * kb_count;
  if (idx < rows_x_kb) {
    const int64_t r = idx % npad, kb = idx / npad;  // consecutive threads: consecutive rows
    const int64_t src_row = r < n ? r : n - 1;
    const uint32_t* src = words + src_row * (k * BITS / 32) + kb * (QROW / 4);
    uint32_t* dst = reinterpret_cast<uint32_t*>(wt + (((r / 256) * kb_count + kb) * 256 + (r % 256)) * QROW);
#pragma unroll
    for (int j = 0; j < QROW / 4; ++j) dst[j] = src[j];
  }
  if (idx < npad * p_count) {
    const int64_t r = idx % npad, p = idx / npad;
    const int64_t src_row = r < n ? r : n - 1;
    const int64_t g = src_row * (k / 64) + 2 * p;
    uint16_t* dst = reinterpret_cast<uint16_t*>(sbt + (((r / 256) * p_count + p) * 256 + (r % 256)) * 8);
    dst[0] = scales[g];
    dst[1] = scales[g + 1];
    dst[2] = biases[g];
    dst[3] = biases[g + 1];
  }
}

int check_epilogue(const char* name, int epilogue, const void* bias, const void* c,
                   int64_t ldc, const void* resid, int64_t ldr, int64_t n, const float* gate,
                   int64_t gate_div, int64_t gate_stride) {
  const int act = (epilogue >> 4) & 15;
  const int known = KX_EPI_BIAS | (15 << 4) | KX_EPI_GATED_RESIDUAL | KX_EPI_RESID_F32 |
                    KX_EPI_OUT_F32;
  KX_REQUIRE((epilogue & ~known) == 0 && act <= 4, "%s: bad epilogue flags %d", name, epilogue);
  KX_REQUIRE(!(epilogue & KX_EPI_BIAS) || (bias && aligned8(bias)), "%s: bias missing or unaligned",
             name);
  KX_REQUIRE(!(epilogue & KX_EPI_OUT_F32) || (aligned16(c) && ldc % 4 == 0),
             "%s: an fp32 output needs 16-byte aligned rows", name);
  KX_REQUIRE(!(epilogue & KX_EPI_RESID_F32) || (epilogue & KX_EPI_GATED_RESIDUAL),
             "%s: KX_EPI_RESID_F32 without a gated residual", name);
  if (epilogue & KX_EPI_GATED_RESIDUAL) {
    KX_REQUIRE(resid && gate && ldr >= n && gate_div > 0 && gate_stride >= 0,
               "%s: gated residual needs resid, ldr >= n and gate rows", name);
    KX_REQUIRE(aligned16(gate) && gate_stride % 4 == 0, "%s: gate must be 16-byte aligned", name);
    if (epilogue & KX_EPI_RESID_F32)
      KX_REQUIRE(aligned16(resid) && ldr % 4 == 0, "%s: an fp32 residual needs 16-byte aligned rows",
                 name);
    else
      KX_REQUIRE(aligned8(resid), "%s: resid must be 8-byte aligned", name);
  }
  return KX_OK;
}

}  // namespace
}  // namespace kx

using namespace kx;

namespace {
template <bool H>
int gemm_entry(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc,
               int64_t m, int64_t n, int64_t k, int epilogue, const void* resid, int64_t ldr, const float* gate,
               int64_t gate_div, int64_t gate_stride, hipStream_t s) {
  const char* what = ename<H>("kx_gemm_bf16", "kx_gemm_f16");
  KX_REQUIRE(a && w && c, "%s: null tensor", what);
  KX_REQUIRE(m >= 0 && n >= 0 && k > 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 30),
             "%s: bad shape (%lld, %lld, %lld)", what, (long long)m, (long long)n, (long long)k);
  KX_REQUIRE(k % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0 && lda >= k && ldw >= k && ldc >= n,
             "%s: k, lda and ldw must be multiples of 8 (k=%lld lda=%lld ldw=%lld)", what, (long long)k,
             (long long)lda, (long long)ldw);
  KX_REQUIRE(aligned16(a) && aligned16(w) && aligned8(c), "%s: a/w must be 16-byte and c 8-byte aligned", what);
  const int rc = check_epilogue(what, epilogue, bias, c, ldc, resid, ldr, n, gate, gate_div, gate_stride);
  if (rc) return rc;
  if (m == 0 || n == 0) return KX_OK;
  const Epilogue epi{(const uint16_t*)bias, resid, ldr, gate, gate_div, gate_stride, epilogue};
  dispatch<0, H>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, QuantW{}, c, ldc, m, n, k, epi, s);
  return check_launch(what);
}
}  // namespace

extern "C" int kx_gemm_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                            int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid,
                            int64_t ldr, const float* gate, int64_t gate_div, int64_t gate_stride,
                            kx_stream_t stream) {
  return gemm_entry<false>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div, gate_stride,
                           (hipStream_t)stream);
}

extern "C" int kx_gemm_f16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c,
                           int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid,
                           int64_t ldr, const float* gate, int64_t gate_div, int64_t gate_stride,
                           kx_stream_t stream) {
  return gemm_entry<true>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div, gate_stride,
                          (hipStream_t)stream);
}

extern "C" int kx_gemm_qknorm_rope_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                                        void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t q_end,
                                        int64_t k_end, const void* norm_q, const void* norm_k, int norm_dtype,
                                        float eps, float weight_offset, const float* cos, const float* sin,
                                        int64_t table_ld, int64_t table_hs, int64_t table_rows, int64_t table_bs,
                                        kx_stream_t stream) {
  const char* what = "kx_gemm_qknorm_rope_bf16";
  KX_REQUIRE(a && w && c && norm_q && norm_k && cos && sin, "%s: null tensor", what);
  KX_REQUIRE(m >= 0 && n > 0 && k > 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 30) &&
                 k % DENSE_BK == 0,
             "%s: bad shape (m=%lld n=%lld k=%lld; k %% 64 == 0)", what, (long long)m, (long long)n, (long long)k);
  KX_REQUIRE(q_end >= 0 && q_end % 128 == 0 && k_end >= q_end && k_end % 128 == 0 && k_end <= n,
             "%s: the query and key columns must be whole 128-wide heads inside n (q_end=%lld k_end=%lld)", what,
             (long long)q_end, (long long)k_end);
  KX_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= k && ldw >= k && ldc >= n && ldc % 4 == 0 && lda <= (1 << 22) &&
                 ldw <= (1 << 22),
             "%s: bad strides", what);
  KX_REQUIRE(aligned16(a) && aligned16(w) && aligned8(c) && (!bias || aligned8(bias)), "%s: misaligned tensor", what);
  KX_REQUIRE(norm_dtype == KX_F32 || norm_dtype == KX_BF16, "%s: norm weights must be KX_F32 or KX_BF16", what);
  KX_REQUIRE(norm_dtype == KX_BF16 ? (aligned8(norm_q) && aligned8(norm_k)) : (aligned16(norm_q) && aligned16(norm_k)),
             "%s: misaligned norm weights", what);
  KX_REQUIRE(aligned16(cos) && aligned16(sin) && table_ld % 4 == 0 && table_hs % 4 == 0 && table_bs % 4 == 0 &&
                 table_rows > 0 && table_rows < (1ll << 31),
             "%s: tables need 16-byte aligned rows (table_ld, table_hs, table_bs multiples of 4)", what);
  {
    // the kernel indexes the tables with 32-bit offsets
    const int64_t heads = std::max(q_end, k_end - q_end) / 128;
    const int64_t last = (m > 0 ? (m - 1) / table_rows : 0) * table_bs + std::min(m, table_rows) * table_ld +
                         std::max<int64_t>(heads - 1, 0) * table_hs + 128;
    KX_REQUIRE(table_ld >= 0 && table_hs >= 0 && table_bs >= 0 && last < (1ll << 31),
               "%s: table offsets must be non-negative and below 2^31 elements", what);
  }
  if (m == 0) return KX_OK;
  Epilogue epi{(const uint16_t*)bias, nullptr, 0, nullptr, 1, 0, bias ? KX_EPI_BIAS : 0};
  epi.nq = norm_q;
  epi.nk = norm_k;
  epi.n_bf16 = norm_dtype == KX_BF16;
  epi.n_eps = eps;
  epi.n_off = weight_offset;
  epi.q_end = q_end;
  epi.k_end = k_end;
  epi.cosp = cos;
  epi.sinp = sin;
  epi.t_ld = table_ld;
  epi.t_hs = table_hs;
  epi.t_rows = table_rows;
  epi.t_bs = table_bs;
  // division by the invariant table_rows (round-up method): shift = ceil(log2 d),
  // magic = floor(2^32 (2^shift - d) / d) + 1
  int shift = 0;
  while ((1ll << shift) < table_rows) ++shift;
  epi.t_shift = shift;
  epi.t_magic = (uint32_t)(((((unsigned __int128)1 << 32) * (uint64_t)((1ll << shift) - table_rows)) /
                            (uint64_t)table_rows) + 1);
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256), t192 = ((m + 191) / 192) * ((n + 255) / 256);
  const bool tall = (t256 + 255) / 256 * 256 <= (t192 + 255) / 256 * 192;
  hipStream_t s = (hipStream_t)stream;
  if (tall)
    launch_lds_t<256, 256, 0, false, 0, false, true>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, QuantW{}, c,
                                                     ldc, (int)m, (int)n, (int)k, epi, s);
  else
    launch_lds_t<192, 256, 0, false, 0, false, true>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, QuantW{}, c,
                                                     ldc, (int)m, (int)n, (int)k, epi, s);
  return check_launch(what);
}

extern "C" int kx_qgemm_affine_bf16(const void* a, int64_t lda, const uint32_t* wq,
                                    const void* scales, const void* biases, const void* bias,
                                    void* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                                    int group_size, int bits, int epilogue, const void* resid,
                                    int64_t ldr, const float* gate, int64_t gate_div,
                                    int64_t gate_stride, kx_stream_t stream) {
  KX_REQUIRE(a && wq && scales && biases && c, "kx_qgemm_affine_bf16: null tensor");
  KX_REQUIRE(bits == 4 || bits == 8, "kx_qgemm_affine_bf16: bits must be 4 or 8, got %d", bits);
  KX_REQUIRE(group_size == 64, "kx_qgemm_affine_bf16: group_size must be 64, got %d", group_size);
  KX_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 64 == 0 && m < (1ll << 31) && n < (1ll << 31) &&
                 k < (1ll << 30),
             "kx_qgemm_affine_bf16: bad shape (k must be a multiple of 64)");
  KX_REQUIRE(lda % 8 == 0 && lda >= k && ldc >= n && aligned16(a) && aligned8(c),
             "kx_qgemm_affine_bf16: bad stride or alignment");
  const int rc = check_epilogue("kx_qgemm_affine_bf16", epilogue, bias, c, ldc, resid, ldr, n,
                                gate, gate_div, gate_stride);
  if (rc) return rc;
  if (m == 0 || n == 0) return KX_OK;
  const Epilogue epi{(const uint16_t*)bias, resid, ldr, gate, gate_div, gate_stride, epilogue};
  const QuantW qw{wq, (const uint16_t*)scales, (const uint16_t*)biases};
  if (bits == 4)
    dispatch<4>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, m, n, k, epi, (hipStream_t)stream);
  else
    dispatch<8>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, m, n, k, epi, (hipStream_t)stream);
  return check_launch("kx_qgemm_affine_bf16");
}

extern "C" int kx_dequant_affine_bf16(const uint32_t* wq, const void* scales, const void* biases,
                                      void* out, int64_t n, int64_t k, int group_size, int bits,
                                      kx_stream_t stream) {
  KX_REQUIRE(wq && scales && biases && out, "kx_dequant_affine_bf16: null tensor");
  KX_REQUIRE(bits == 4 || bits == 8, "kx_dequant_affine_bf16: bits must be 4 or 8");
  KX_REQUIRE(group_size > 0 && group_size % 8 == 0 && n >= 0 && k > 0 && k % group_size == 0,
             "kx_dequant_affine_bf16: k must be a multiple of group_size (a multiple of 8)");
  KX_REQUIRE(aligned16(out), "kx_dequant_affine_bf16: out must be 16-byte aligned");
  const int64_t total = n * (k / 8);
  if (total == 0) return KX_OK;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (bits == 4)
    dequant_kernel<4><<<blocks, 256, 0, (hipStream_t)stream>>>(
        wq, (const uint16_t*)scales, (const uint16_t*)biases, (uint16_t*)out, n, k, group_size);
  else
    dequant_kernel<8><<<blocks, 256, 0, (hipStream_t)stream>>>(
        wq, (const uint16_t*)scales, (const uint16_t*)biases, (uint16_t*)out, n, k, group_size);
  return check_launch("kx_dequant_affine_bf16");
}

extern "C" int kx_qgemm_mxfp8_bf16(const void* a, int64_t lda, const uint32_t* wq, const void* scales,
                                   const void* bias, void* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                                   int group_size, int epilogue, const void* resid, int64_t ldr, const float* gate,
                                   int64_t gate_div, int64_t gate_stride, kx_stream_t stream) {
  const char* what = "kx_qgemm_mxfp8_bf16";
  KX_REQUIRE(a && wq && scales && c, "%s: null tensor", what);
  KX_REQUIRE(group_size == 32, "%s: group_size must be 32, got %d", what, group_size);
  KX_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 32 == 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 30),
             "%s: bad shape (m=%lld n=%lld k=%lld; k must be a multiple of 32)", what, (long long)m, (long long)n,
             (long long)k);
  KX_REQUIRE(lda % 8 == 0 && lda >= k && ldc >= n && aligned16(a) && aligned8(c) && aligned8(wq),
             "%s: bad stride or alignment", what);
  const int rc = check_epilogue(what, epilogue, bias, c, ldc, resid, ldr, n, gate, gate_div, gate_stride);
  if (rc) return rc;
  if (m == 0 || n == 0) return KX_OK;
  const Epilogue epi{(const uint16_t*)bias, resid, ldr, gate, gate_div, gate_stride, epilogue};
  const QuantW qw{wq, nullptr, nullptr, (const uint8_t*)scales};
  dispatch<QMX8>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, m, n, k, epi, (hipStream_t)stream);
  return check_launch(what);
}

extern "C" int kx_dequant_mxfp8_bf16(const uint32_t* wq, const void* scales, void* out, int64_t n, int64_t k,
                                     int group_size, int transposed, kx_stream_t stream) {
  const char* what = "kx_dequant_mxfp8_bf16";
  KX_REQUIRE(wq && scales && out, "%s: null tensor", what);
  KX_REQUIRE(group_size == 32, "%s: group_size must be 32, got %d", what, group_size);
  KX_REQUIRE(n >= 0 && k >= 0 && n < (1ll << 31) && k < (1ll << 31), "%s: bad shape", what);
  KX_REQUIRE(transposed ? (n % 32 == 0 && k % 8 == 0) : k % 32 == 0,
             "%s: the grouped axis must be a multiple of 32 (and k of 8 when transposed): n=%lld k=%lld", what,
             (long long)n, (long long)k);
  KX_REQUIRE(aligned16(out) && (transposed ? aligned16(wq) : aligned8(wq)), "%s: out (and wq) misaligned", what);
  if (n == 0 || k == 0) return KX_OK;
  hipStream_t s = (hipStream_t)stream;
  if (transposed) {
    const dim3 grid((unsigned)((n + 63) / 64), (unsigned)((k + 63) / 64));
    dequant_mx8_t_kernel<<<grid, 256, 0, s>>>(wq, (const uint8_t*)scales, (uint16_t*)out, n, k);
  } else {
    const int64_t total = n * (k / 8);
    dequant_mx8_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(wq, (const uint8_t*)scales, (uint16_t*)out,
                                                                       n, k);
  }
  return check_launch(what);
}

extern "C" int kx_dequant_fp4_bf16(const uint32_t* wq, const void* scales, void* out, int64_t n, int64_t k,
                                   int group_size, int scale_kind, kx_stream_t stream) {
  const char* what = "kx_dequant_fp4_bf16";
  KX_REQUIRE(wq && scales && out, "%s: null tensor", what);
  KX_REQUIRE(scale_kind == KX_FP4_MX || scale_kind == KX_FP4_NV, "%s: bad scale kind %d", what, scale_kind);
  const int gs = scale_kind == KX_FP4_NV ? 16 : 32;
  KX_REQUIRE(group_size == gs, "%s: group_size must be %d for this scale kind, got %d", what, gs, group_size);
  KX_REQUIRE(n >= 0 && k > 0 && k % gs == 0, "%s: k must be a multiple of the group size (n=%lld k=%lld)", what,
             (long long)n, (long long)k);
  KX_REQUIRE(aligned16(out), "%s: out must be 16-byte aligned", what);
  const int64_t total = n * (k / 8);
  KX_REQUIRE(total / 256 < (1ll << 31), "%s: too many elements", what);
  if (total == 0) return KX_OK;
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (scale_kind == KX_FP4_NV)
    dequant_fp4_kernel<true><<<grid, 256, 0, (hipStream_t)stream>>>(wq, (const uint8_t*)scales, (uint16_t*)out, n, k);
  else
    dequant_fp4_kernel<false><<<grid, 256, 0, (hipStream_t)stream>>>(wq, (const uint8_t*)scales, (uint16_t*)out, n, k);
  return check_launch(what);
}

extern "C" int kx_qweight_tile_affine(const uint32_t* wq, const void* scales, const void* biases,
                                      void* wt, void* sbt, int64_t n, int64_t k, int group_size,
                                      int bits, kx_stream_t stream) {
  KX_REQUIRE(wq && scales && biases && wt && sbt, "kx_qweight_tile_affine: null tensor");
  KX_REQUIRE(bits == 4 || bits == 8, "kx_qweight_tile_affine: bits must be 4 or 8, got %d", bits);
  KX_REQUIRE(group_size == 64, "kx_qweight_tile_affine: group_size must be 64, got %d", group_size);
  KX_REQUIRE(n > 0 && k > 0 && k % 128 == 0 && n < (1ll << 31) && k < (1ll << 30),
             "kx_qweight_tile_affine: k must be a positive multiple of 128");
  KX_REQUIRE(aligned16(wt) && aligned8(sbt), "kx_qweight_tile_affine: wt must be 16-byte and sbt 8-byte aligned");
  const int64_t npad = (n + 255) / 256 * 256;
  const int64_t work = npad * (k / 32);
  const unsigned blocks = (unsigned)((work + 255) / 256);
  if (bits == 4)
    tile_weights_kernel<4><<<blocks, 256, 0, (hipStream_t)stream>>>(
        wq, (const uint16_t*)scales, (const uint16_t*)biases, (uint8_t*)wt, (uint8_t*)sbt, n, k);
  else
    tile_weights_kernel<8><<<blocks, 256, 0, (hipStream_t)stream>>>(
        wq, (const uint16_t*)scales, (const uint16_t*)biases, (uint8_t*)wt, (uint8_t*)sbt, n, k);
  return check_launch("kx_qweight_tile_affine");
}

extern "C" int kx_qgemm_affine_tiled_bf16(const void* a, int64_t lda, const void* wt, const void* sbt,
                                          const void* bias, void* c, int64_t ldc, int64_t m, int64_t n,
                                          int64_t k, int bits, int epilogue, const void* resid,
                                          int64_t ldr, const float* gate, int64_t gate_div,
                                          int64_t gate_stride, kx_stream_t stream) {
  KX_REQUIRE(a && wt && sbt && c, "kx_qgemm_affine_tiled_bf16: null tensor");
  KX_REQUIRE(bits == 4 || bits == 8, "kx_qgemm_affine_tiled_bf16: bits must be 4 or 8, got %d", bits);
  KX_REQUIRE(m >= 0 && n > 0 && k > 0 && k % 128 == 0 && m < (1ll << 31) && n < (1ll << 31) &&
                 k < (1ll << 30),
             "kx_qgemm_affine_tiled_bf16: bad shape (k must be a multiple of 128)");
  KX_REQUIRE(lda % 8 == 0 && lda >= k && lda <= (1 << 22) && ldc >= n && aligned16(a) && aligned8(c) &&
                 aligned16(wt) && aligned8(sbt),
             "kx_qgemm_affine_tiled_bf16: bad stride or alignment");
  const int rc = check_epilogue("kx_qgemm_affine_tiled_bf16", epilogue, bias, c, ldc, resid, ldr, n,
                                gate, gate_div, gate_stride);
  if (rc) return rc;
  if (m == 0) return KX_OK;
  const Epilogue epi{(const uint16_t*)bias, resid, ldr, gate, gate_div, gate_stride, epilogue};
  const QuantW qw{(const uint32_t*)wt, (const uint16_t*)sbt, nullptr};
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256), t192 = ((m + 191) / 192) * ((n + 255) / 256);
  const char* env = getenv("KX355_GEMM_LDS_TILE");
  const bool tall = (env && *env) ? atoi(env) == 0 : (t256 + 255) / 256 * 256 <= (t192 + 255) / 256 * 192;
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4) {
    if (tall) launch_lds<256, 256, 4, true>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
    else launch_lds<192, 256, 4, true>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
  } else {
    if (tall) launch_lds<256, 256, 8, true>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
    else launch_lds<192, 256, 8, true>((const uint16_t*)a, lda, nullptr, 0, qw, c, ldc, (int)m, (int)n, (int)k, epi, s);
  }
  return check_launch("kx_qgemm_affine_tiled_bf16");
}

namespace {

// Argument checks shared by the two split-K entry points (no GPU call).
int check_splitk(const char* what, const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                 void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid,
                 int64_t ldr, const float* gate, int64_t gate_div, int64_t gate_stride, int splits) {
  KX_REQUIRE(a && w && c, "%s: null tensor", what);
  KX_REQUIRE(splits >= 2 && splits <= 64, "%s: splits must be 2..64, got %d", what, splits);
  KX_REQUIRE(m > 0 && n > 0 && k > 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 30) && n % 4 == 0 &&
                 k % (splits * DENSE_BK) == 0,
             "%s: bad shape (m=%lld n=%lld k=%lld; n %% 4 == 0, k %% (64 splits) == 0)", what, (long long)m,
             (long long)n, (long long)k);
  KX_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= k && ldw >= k && ldc >= n && lda <= (1 << 22) &&
                 ldw <= (1 << 22),
             "%s: bad strides", what);
  KX_REQUIRE(aligned16(a) && aligned16(w) && aligned8(c), "%s: a/w must be 16-byte and c 8-byte aligned", what);
  return check_epilogue(what, epilogue, bias, c, ldc, resid, ldr, n, gate, gate_div, gate_stride);
}

// Both passes of a split-K product on `parts` (splits * m * n floats): every slice writes all of its
// (m, n) plane before the reduction reads it, so `parts` needs no clearing between calls.
template <bool H>
int run_splitk(const char* what, const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
               void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue, const void* resid,
               int64_t ldr, const float* gate, int64_t gate_div, int64_t gate_stride, float* parts, int splits,
               hipStream_t s) {
  // slices of 256x256 tiles for the tail rows of a large product (a few 256-row tiles across a wide
  // N, each slice a quarter or less of K); up to 512 rows keep the 64x128 / 128x128 tiles
  if (m > 512 && n >= 1024)
    launch_splitk<256, 256, H>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, parts, (int)m, (int)n, (int)k, splits,
                            s);
  else if (pick_lds_cfg(m, n) == 3)
    launch_splitk<64, 128, H>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, parts, (int)m, (int)n, (int)k, splits, s);
  else
    launch_splitk<128, 128, H>((const uint16_t*)a, lda, (const uint16_t*)w, ldw, parts, (int)m, (int)n, (int)k, splits,
                            s);
  const Epilogue epi{(const uint16_t*)bias, resid, ldr, gate, gate_div, gate_stride, epilogue};
  const bool vec_ok = (ldc % 4 == 0) && (!(epilogue & KX_EPI_GATED_RESIDUAL) || ldr % 4 == 0);
  const int64_t threads = m * (n / 4);
  splitk_reduce_kernel<H><<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(parts, splits, (int)m, (int)n, c, ldc, epi,
                                                                         vec_ok);
  return check_launch(what);
}

// The no-allocation variant's partial products: one static array per device (the HIP runtime
// places a copy on each device that loads this code object, for the life of the process). Host
// code never passes `scratch` itself to a kernel (on the host it names a stand-in, not a device
// address); it passes the device address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float scratch[KX_SPLITK_SCRATCH_BYTES / 4];

constexpr int KX_MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[KX_MAX_DEVICES] = {};

// The current device's address of `scratch`, looked up on the first call on that device (with the
// device current) and kept per device.
int scratch_address(const char* what, float** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_error(KX_ERR_LAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(err));
  if (dev < 0 || dev >= KX_MAX_DEVICES) return set_error(KX_ERR_UNSUPPORTED, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return set_error(KX_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                       hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return KX_OK;
}

}  // namespace

namespace {
template <bool H>
int splitk_entry(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, void* c, int64_t ldc,
                 int64_t m, int64_t n, int64_t k, int epilogue, const void* resid, int64_t ldr, const float* gate,
                 int64_t gate_div, int64_t gate_stride, void* workspace, int64_t workspace_bytes, int splits,
                 hipStream_t s) {
  const char* what = ename<H>("kx_gemm_splitk_bf16", "kx_gemm_splitk_f16");
  KX_REQUIRE(workspace, "%s: null tensor", what);
  const int rc = check_splitk(what, a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div,
                              gate_stride, splits);
  if (rc) return rc;
  KX_REQUIRE(aligned16(workspace), "%s: workspace must be 16-byte aligned", what);
  KX_REQUIRE(workspace_bytes >= (int64_t)splits * m * n * 4,
             "%s: workspace of %lld bytes is below splits * m * n * 4 = %lld", what, (long long)workspace_bytes,
             (long long)splits * m * n * 4);
  return run_splitk<H>(what, a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div,
                       gate_stride, static_cast<float*>(workspace), splits, s);
}
}  // namespace

#define KX_SPLITK_ENTRY(SUFFIX, H)                                                                                \
  extern "C" int kx_gemm_splitk_##SUFFIX(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, \
                                         void* c, int64_t ldc, int64_t m, int64_t n, int64_t k, int epilogue,     \
                                         const void* resid, int64_t ldr, const float* gate, int64_t gate_div,     \
                                         int64_t gate_stride, void* workspace, int64_t workspace_bytes,           \
                                         int splits, kx_stream_t stream) {                                        \
    return splitk_entry<H>(a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div,          \
                           gate_stride, workspace, workspace_bytes, splits, (hipStream_t)stream);                \
  }

KX_SPLITK_ENTRY(bf16, false)
KX_SPLITK_ENTRY(f16, true)

extern "C" int kx_gemm_splitk_noalloc_bf16(const void* a, int64_t lda, const void* w, int64_t ldw,
                                           const void* bias, void* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                                           int epilogue, const void* resid, int64_t ldr, const float* gate,
                                           int64_t gate_div, int64_t gate_stride, int splits, kx_stream_t stream) {
  const char* what = "kx_gemm_splitk_noalloc_bf16";
  const int rc = check_splitk(what, a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div,
                              gate_stride, splits);
  if (rc) return rc;
  KX_REQUIRE((int64_t)splits * m * n * 4 <= KX_SPLITK_SCRATCH_BYTES,
             "%s: splits * m * n * 4 = %lld bytes exceeds the %lld-byte static scratch", what,
             (long long)splits * m * n * 4, (long long)KX_SPLITK_SCRATCH_BYTES);
  float* parts = nullptr;
  const int arc = scratch_address(what, &parts);
  if (arc) return arc;
  return run_splitk<false>(what, a, lda, w, ldw, bias, c, ldc, m, n, k, epilogue, resid, ldr, gate, gate_div,
                           gate_stride, parts, splits, (hipStream_t)stream);
}
