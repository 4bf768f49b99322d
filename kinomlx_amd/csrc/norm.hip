// Row norms of the DiT block on gfx950: HBM-bound, one wavefront per row.
//
// Fast path: a row of DIM = 512 * VPL bf16 values is held in registers, VPL 16-byte vectors per
// lane, lane l's vector i covering columns [(64 i + l) * 8, +8). Every load and store is a
// 16-byte access and a wave's access of one vector index is 1 KiB contiguous. The reduction is
// a wave64 butterfly; nothing goes through LDS. Generic path (any width or alignment): one wave
// per row (or norm group) with a strided scalar loop.
#include "common.h"

namespace kx {
namespace {

constexpr int kWaves = 4;  // rows per 256-thread workgroup

// ----------------------------------------------------------------------------------------------
// Modulated RMSNorm / LayerNorm: y = norm(x) * (1 + scale) + shift.

// Loads 8 consecutive elements of a 16-bit (bf16 / fp16 by H) or fp32 row (16-byte aligned) as
// fp32.
template <bool H, bool XF32>
__device__ __forceinline__ void load8(const void* row, int64_t col, float* v) {
  if (XF32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + col);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + col + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    e_unpack8<H>(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(row) + col), v);
  }
}

template <bool H, bool XF32>
__device__ __forceinline__ float load1(const void* row, int64_t col) {
  return XF32 ? static_cast<const float*>(row)[col] : e2f<H>(static_cast<const uint16_t*>(row)[col]);
}

// H: the 16-bit element type is fp16 (else bf16). XF32: x is fp32 (a residual stream carried in
// fp32); y is always the 16-bit type.
template <bool H, int VPL, int KIND, bool MOD, bool XF32>
__global__ __launch_bounds__(256) void adaln_norm_kernel(
    const void* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, const float* __restrict__ shift, const float* __restrict__ scale,
    int64_t mod_div, int64_t mod_stride, float eps) {
  constexpr int DIM = VPL * 512;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const void* xr = XF32 ? (const void*)(static_cast<const float*>(x) + row * ldx)
                        : (const void*)(static_cast<const uint16_t*>(x) + row * ldx);
  float v[VPL][8];
#pragma unroll
  for (int i = 0; i < VPL; ++i) load8<H, XF32>(xr, (i * 64 + lane) * 8, v[i]);
  float mean = 0.0f;
  if (KIND == KX_NORM_LAYER) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[i][j];
    mean = wave_sum<64>(s) * (1.0f / DIM);
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = v[i][j] - mean;
      ss = fmaf(d, d, ss);
    }
  const float inv = rsqrtf(wave_sum<64>(ss) * (1.0f / DIM) + eps);
  const int64_t mrow = MOD ? (row / mod_div) * mod_stride : 0;
  uint16_t* yr = y + row * ldy;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int col = (i * 64 + lane) * 8;
    float o[8];
    if (MOD) {
      const float4 sc0 = *reinterpret_cast<const float4*>(scale + mrow + col);
      const float4 sc1 = *reinterpret_cast<const float4*>(scale + mrow + col + 4);
      const float4 sh0 = *reinterpret_cast<const float4*>(shift + mrow + col);
      const float4 sh1 = *reinterpret_cast<const float4*>(shift + mrow + col + 4);
      const float sc[8] = {sc0.x, sc0.y, sc0.z, sc0.w, sc1.x, sc1.y, sc1.z, sc1.w};
      const float sh[8] = {sh0.x, sh0.y, sh0.z, sh0.w, sh1.x, sh1.y, sh1.z, sh1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (v[i][j] - mean) * inv * (1.0f + sc[j]) + sh[j];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (v[i][j] - mean) * inv;
    }
    *reinterpret_cast<uint4*>(yr + col) = e_pack8<H>(o);
  }
}

template <bool H, int KIND, bool XF32>
__global__ __launch_bounds__(256) void adaln_norm_generic(
    const void* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, int64_t dim, const float* __restrict__ shift, const float* __restrict__ scale,
    int64_t mod_div, int64_t mod_stride, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const void* xr = XF32 ? (const void*)(static_cast<const float*>(x) + row * ldx)
                        : (const void*)(static_cast<const uint16_t*>(x) + row * ldx);
  float mean = 0.0f;
  if (KIND == KX_NORM_LAYER) {
    float s = 0.0f;
    for (int64_t c = lane; c < dim; c += 64) s += load1<H, XF32>(xr, c);
    mean = wave_sum<64>(s) / (float)dim;
  }
  float ss = 0.0f;
  for (int64_t c = lane; c < dim; c += 64) {
    const float d = load1<H, XF32>(xr, c) - mean;
    ss = fmaf(d, d, ss);
  }
  const float inv = rsqrtf(wave_sum<64>(ss) / (float)dim + eps);
  const bool mod = shift != nullptr;
  const int64_t mrow = mod ? (row / mod_div) * mod_stride : 0;
  uint16_t* yr = y + row * ldy;
  for (int64_t c = lane; c < dim; c += 64) {
    float o = (load1<H, XF32>(xr, c) - mean) * inv;
    if (mod) o = o * (1.0f + scale[mrow + c]) + shift[mrow + c];
    yr[c] = f2e<H>(o);
  }
}

// ----------------------------------------------------------------------------------------------
// Weighted RMSNorm (+ optional RoPE on the normalized value).
//
// G == 0: one norm over the whole row. G > 0: norm groups of 8 * G columns (G lanes of one
// vector), e.g. per-head norms of 128 columns with G = 16.
// SPLIT RoPE pairs column d < half of a head with d + half, held by lane l ^ (half / 8).
// PAIR RoPE pairs columns 2i and 2i + 1, both in the same lane.

// Norm weights: WT = KX_F32, KX_BF16 or KX_F16.
template <int WT>
__device__ __forceinline__ float load_w(const void* w, int64_t i) {
  if constexpr (WT == KX_BF16) return bf2f(reinterpret_cast<const uint16_t*>(w)[i]);
  else if constexpr (WT == KX_F16) return e2f<true>(reinterpret_cast<const uint16_t*>(w)[i]);
  else return reinterpret_cast<const float*>(w)[i];
}

template <bool H, int VPL, int G, int ROPE, int WT>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, int norm_width, const void* __restrict__ w, float eps, float weight_offset,
    const float* __restrict__ cosp, const float* __restrict__ sinp, int64_t table_ld,
    int64_t table_hs, int64_t tokens, int table_batched, int head_dim) {
  constexpr int DIM = VPL * 512;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * ldx;
  float v[VPL][8];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const uint4 q = *reinterpret_cast<const uint4*>(xr + (i * 64 + lane) * 8);
    e_unpack8<H>(q, v[i]);
  }
  float inv[VPL];
  if (G == 0) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[i][j], v[i][j], ss);
    const float r = rsqrtf(wave_sum<64>(ss) * (1.0f / DIM) + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) inv[i] = r;
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[i][j], v[i][j], ss);
      inv[i] = rsqrtf(wave_sum<G>(ss) * (1.0f / (8 * G)) + eps);
    }
  }
  // normalized, weighted values (fp32, not rounded)
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int col = (i * 64 + lane) * 8;
    const int wcol = (G == 0) ? col : (col % norm_width);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[i][j] = v[i][j] * inv[i] * (load_w<WT>(w, wcol + j) + weight_offset);
  }
  uint16_t* yr = y + row * ldy;
  if (ROPE == KX_ROPE_NONE) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) *reinterpret_cast<uint4*>(yr + (i * 64 + lane) * 8) = e_pack8<H>(v[i]);
    return;
  }
  const int64_t tok = table_batched ? row : (row % tokens);
  const float* ct = cosp + tok * table_ld;
  const float* st = sinp + tok * table_ld;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int col = (i * 64 + lane) * 8;
    const int h = col / head_dim;
    const int d = col - h * head_dim;
    float o[8];
    if (ROPE == KX_ROPE_SPLIT) {
      const int half = head_dim >> 1;
      const int partner_mask = half >> 3;  // lanes between d and d + half
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = __shfl_xor(v[i][j], partner_mask, 64);
      const bool first = d < half;
      const int ti = first ? d : d - half;
      const float* cr = ct + h * table_hs + ti;
      const float* sr = st + h * table_hs + ti;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma clang fp contract(off)
        const float c = cr[j], s = sr[j];
        if (first) {
          const float a = v[i][j] * c;  // first * c
          const float b = p[j] * s;     // second * s
          o[j] = a - b;
        } else {
          const float a = p[j] * s;     // first * s
          const float b = v[i][j] * c;  // second * c
          o[j] = a + b;
        }
      }
    } else {  // PAIR
      const float* cr = ct + h * table_hs + d;
      const float* sr = st + h * table_hs + d;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
#pragma clang fp contract(off)
        const float x0 = v[i][j], x1 = v[i][j + 1];
        const float a0 = x0 * cr[j];
        const float b0 = (-x1) * sr[j];
        const float a1 = x1 * cr[j + 1];
        const float b1 = x0 * sr[j + 1];
        o[j] = a0 + b0;
        o[j + 1] = a1 + b1;
      }
    }
    *reinterpret_cast<uint4*>(yr + col) = e_pack8<H>(o);
  }
}

// Full-width weighted RMSNorm with split-half RoPE for 128-wide heads (the LTX q/k path): each
// lane owns matching 8-value chunks of both halves of a head (dims d .. d+7 and d+64 .. d+71), so
// the rotation needs no lane exchange and every cos / sin table value is read once. All loads
// (row, both tables) are issued before the row reduction. Rounding as rmsnorm_rope_kernel: the
// normalized value stays fp32, each RoPE product is rounded before the difference / sum.
template <bool H, int VPL, int WT>
__global__ __launch_bounds__(256) void rmsnorm_rope_split128_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, const void* __restrict__ w, float eps, float weight_offset,
    const float* __restrict__ cosp, const float* __restrict__ sinp, int64_t table_ld,
    int64_t table_hs, int64_t tokens, int table_batched) {
  constexpr int DIM = VPL * 512;
  constexpr int NP = VPL / 2;  // head-half pairs of chunks per lane
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * ldx;
  const int64_t tok = table_batched ? row : (row % tokens);
  float a[NP][8], b[NP][8], c[NP][8], sn[NP][8];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = i * 64 + lane, h = p >> 3, k = p & 7;
    const int col = h * 128 + k * 8;
    e_unpack8<H>(*reinterpret_cast<const uint4*>(xr + col), a[i]);
    e_unpack8<H>(*reinterpret_cast<const uint4*>(xr + col + 64), b[i]);
    const float* cr = cosp + tok * table_ld + h * table_hs + k * 8;
    const float* sr = sinp + tok * table_ld + h * table_hs + k * 8;
    const float4 c0 = *reinterpret_cast<const float4*>(cr), c1 = *reinterpret_cast<const float4*>(cr + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sr), s1 = *reinterpret_cast<const float4*>(sr + 4);
    c[i][0] = c0.x; c[i][1] = c0.y; c[i][2] = c0.z; c[i][3] = c0.w;
    c[i][4] = c1.x; c[i][5] = c1.y; c[i][6] = c1.z; c[i][7] = c1.w;
    sn[i][0] = s0.x; sn[i][1] = s0.y; sn[i][2] = s0.z; sn[i][3] = s0.w;
    sn[i][4] = s1.x; sn[i][5] = s1.y; sn[i][6] = s1.z; sn[i][7] = s1.w;
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(b[i][j], b[i][j], fmaf(a[i][j], a[i][j], ss));
  const float r = rsqrtf(wave_sum<64>(ss) * (1.0f / DIM) + eps);
  uint16_t* yr = y + row * ldy;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = i * 64 + lane, h = p >> 3, k = p & 7;
    const int col = h * 128 + k * 8;
    float o0[8], o1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma clang fp contract(off)
      const float n0 = a[i][j] * r * (load_w<WT>(w, col + j) + weight_offset);
      const float n1 = b[i][j] * r * (load_w<WT>(w, col + 64 + j) + weight_offset);
      const float fc = n0 * c[i][j], ss2 = n1 * sn[i][j];  // first * c, second * s
      const float fs = n0 * sn[i][j], sc = n1 * c[i][j];   // first * s, second * c
      o0[j] = fc - ss2;
      o1[j] = fs + sc;
    }
    *reinterpret_cast<uint4*>(yr + col) = e_pack8<H>(o0);
    *reinterpret_cast<uint4*>(yr + col + 64) = e_pack8<H>(o1);
  }
}

// Q and K of the same tokens in one pass (self-attention q_norm / k_norm + split RoPE): a wave
// handles one token's Q row and K row with their own weights and shares the token's cos / sin
// table values between them, so the tables (as large as Q and K together at D = 4096, fp32) are
// read once instead of twice. Per row the arithmetic is exactly rmsnorm_rope_split128_kernel's.
template <bool H, int VPL, int WT>
__global__ __launch_bounds__(256) void qk_rmsnorm_rope_split128_kernel(
    const uint16_t* __restrict__ xq, int64_t ldq, const uint16_t* __restrict__ xk, int64_t ldk,
    uint16_t* __restrict__ yq, int64_t ldyq, uint16_t* __restrict__ yk, int64_t ldyk, int64_t rows,
    const void* __restrict__ wq, const void* __restrict__ wk, float eps, float weight_offset,
    const float* __restrict__ cosp, const float* __restrict__ sinp, int64_t table_ld,
    int64_t table_hs, int64_t tokens, int table_batched) {
  constexpr int DIM = VPL * 512;
  constexpr int NP = VPL / 2;  // head-half pairs of chunks per lane
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t tok = table_batched ? row : (row % tokens);
  uint4 qa[NP], qb[NP], ka[NP], kb[NP];
  float c[NP][8], sn[NP][8];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = i * 64 + lane, h = p >> 3, k = p & 7;
    const int col = h * 128 + k * 8;
    qa[i] = *reinterpret_cast<const uint4*>(xq + row * ldq + col);
    qb[i] = *reinterpret_cast<const uint4*>(xq + row * ldq + col + 64);
    ka[i] = *reinterpret_cast<const uint4*>(xk + row * ldk + col);
    kb[i] = *reinterpret_cast<const uint4*>(xk + row * ldk + col + 64);
    const float* cr = cosp + tok * table_ld + h * table_hs + k * 8;
    const float* sr = sinp + tok * table_ld + h * table_hs + k * 8;
    const float4 c0 = *reinterpret_cast<const float4*>(cr), c1 = *reinterpret_cast<const float4*>(cr + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sr), s1 = *reinterpret_cast<const float4*>(sr + 4);
    c[i][0] = c0.x; c[i][1] = c0.y; c[i][2] = c0.z; c[i][3] = c0.w;
    c[i][4] = c1.x; c[i][5] = c1.y; c[i][6] = c1.z; c[i][7] = c1.w;
    sn[i][0] = s0.x; sn[i][1] = s0.y; sn[i][2] = s0.z; sn[i][3] = s0.w;
    sn[i][4] = s1.x; sn[i][5] = s1.y; sn[i][6] = s1.z; sn[i][7] = s1.w;
  }
  float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float a[8], b[8];
    e_unpack8<H>(qa[i], a);
    e_unpack8<H>(qb[i], b);
#pragma unroll
    for (int j = 0; j < 8; ++j) ssq = fmaf(b[j], b[j], fmaf(a[j], a[j], ssq));
    e_unpack8<H>(ka[i], a);
    e_unpack8<H>(kb[i], b);
#pragma unroll
    for (int j = 0; j < 8; ++j) ssk = fmaf(b[j], b[j], fmaf(a[j], a[j], ssk));
  }
  const float rq = rsqrtf(wave_sum<64>(ssq) * (1.0f / DIM) + eps);
  const float rk = rsqrtf(wave_sum<64>(ssk) * (1.0f / DIM) + eps);
  auto finish = [&](const uint4* xa, const uint4* xb, float r, const void* w, uint16_t* yr) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int p = i * 64 + lane, h = p >> 3, k = p & 7;
      const int col = h * 128 + k * 8;
      float a[8], b[8], o0[8], o1[8];
      e_unpack8<H>(xa[i], a);
      e_unpack8<H>(xb[i], b);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma clang fp contract(off)
        const float n0 = a[j] * r * (load_w<WT>(w, col + j) + weight_offset);
        const float n1 = b[j] * r * (load_w<WT>(w, col + 64 + j) + weight_offset);
        const float fc = n0 * c[i][j], ss2 = n1 * sn[i][j];  // first * c, second * s
        const float fs = n0 * sn[i][j], sc = n1 * c[i][j];   // first * s, second * c
        o0[j] = fc - ss2;
        o1[j] = fs + sc;
      }
      *reinterpret_cast<uint4*>(yr + col) = e_pack8<H>(o0);
      *reinterpret_cast<uint4*>(yr + col + 64) = e_pack8<H>(o1);
    }
  };
  finish(qa, qb, rq, wq, yq + row * ldyq);
  finish(ka, kb, rk, wk, yk + row * ldyk);
}

// One wave per norm group, any width; weighted RMSNorm only.
template <bool H, int WT>
__global__ __launch_bounds__(256) void rmsnorm_generic(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, int64_t dim, int64_t norm_width, const void* __restrict__ w, float eps,
    float weight_offset) {
  const int lane = threadIdx.x & 63;
  const int64_t groups_per_row = dim / norm_width;
  const int64_t g = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (g >= rows * groups_per_row) return;
  const int64_t row = g / groups_per_row;
  const int64_t c0 = (g - row * groups_per_row) * norm_width;
  const uint16_t* xr = x + row * ldx + c0;
  float ss = 0.0f;
  for (int64_t c = lane; c < norm_width; c += 64) {
    const float a = e2f<H>(xr[c]);
    ss = fmaf(a, a, ss);
  }
  const float inv = rsqrtf(wave_sum<64>(ss) / (float)norm_width + eps);
  uint16_t* yr = y + row * ldy + c0;
  for (int64_t c = lane; c < norm_width; c += 64)
    yr[c] = f2e<H>(e2f<H>(xr[c]) * inv * (load_w<WT>(w, c) + weight_offset));
}

// ----------------------------------------------------------------------------------------------
// Elementwise row ops with fp32 modulation rows.

template <bool H>
__global__ __launch_bounds__(256) void modulate_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, int64_t dim, const float* __restrict__ shift, const float* __restrict__ scale,
    int64_t mod_div, int64_t mod_stride) {
  const int64_t per_row = dim;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int64_t r = idx / per_row, c = idx - r * per_row;
  const int64_t m = (r / mod_div) * mod_stride + c;
  y[r * ldy + c] = f2e<H>(e2f<H>(x[r * ldx + c]) * (1.0f + scale[m]) + shift[m]);
}

template <bool H>
__global__ __launch_bounds__(256) void gated_residual_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ r, int64_t ldr,
    uint16_t* __restrict__ y, int64_t ldy, int64_t rows, int64_t dim,
    const float* __restrict__ gate, int64_t gate_div, int64_t gate_stride) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * dim) return;
  const int64_t row = idx / dim, c = idx - row * dim;
  const float g = gate[(row / gate_div) * gate_stride + c];
  const float base = x ? e2f<H>(x[row * ldx + c]) : 0.0f;
  y[row * ldy + c] = f2e<H>(base + e2f<H>(r[row * ldr + c]) * g);
}

template <bool H, int VPL, int KIND, bool XF32>
int launch_adaln(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                 const float* shift, const float* scale, int64_t mod_div, int64_t mod_stride,
                 float eps, hipStream_t s) {
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  if (shift)
    adaln_norm_kernel<H, VPL, KIND, true, XF32><<<grid, 256, 0, s>>>(
        x, ldx, (uint16_t*)y, ldy, rows, shift, scale, mod_div, mod_stride, eps);
  else
    adaln_norm_kernel<H, VPL, KIND, false, XF32><<<grid, 256, 0, s>>>(
        x, ldx, (uint16_t*)y, ldy, rows, shift, scale, mod_div, mod_stride, eps);
  return check_launch(ename<H>("kx_adaln_norm_bf16", "kx_adaln_norm_f16"));
}

template <bool H, int KIND, bool XF32>
int dispatch_adaln(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                   const float* shift, const float* scale, int64_t mod_div, int64_t mod_stride,
                   float eps, bool vec, hipStream_t s) {
  if (vec) {
    switch (dim / 512) {
      case 1: return launch_adaln<H, 1, KIND, XF32>(x, ldx, y, ldy, rows, shift, scale, mod_div, mod_stride, eps, s);
      case 2: return launch_adaln<H, 2, KIND, XF32>(x, ldx, y, ldy, rows, shift, scale, mod_div, mod_stride, eps, s);
      case 4: return launch_adaln<H, 4, KIND, XF32>(x, ldx, y, ldy, rows, shift, scale, mod_div, mod_stride, eps, s);
      default: return launch_adaln<H, 8, KIND, XF32>(x, ldx, y, ldy, rows, shift, scale, mod_div, mod_stride, eps, s);
    }
  }
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  adaln_norm_generic<H, KIND, XF32><<<grid, 256, 0, s>>>(x, ldx, (uint16_t*)y, ldy, rows, dim, shift,
                                                         scale, mod_div, mod_stride, eps);
  return check_launch(ename<H>("kx_adaln_norm_bf16", "kx_adaln_norm_f16"));
}

template <bool H, int VPL, int G, int ROPE, int WT>
int launch_rmsnorm_rope(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                        int64_t norm_width, const void* w, float eps, float off,
                        const float* cosp, const float* sinp, int64_t table_ld, int64_t table_hs,
                        int64_t tokens, int table_batched, int64_t head_dim, hipStream_t s) {
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
  rmsnorm_rope_kernel<H, VPL, G, ROPE, WT><<<grid, 256, 0, s>>>(
      (const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, (int)norm_width, w, eps, off, cosp, sinp,
      table_ld, table_hs, tokens, table_batched, (int)head_dim);
  return check_launch(ename<H>("kx_rmsnorm_rope_bf16", "kx_rmsnorm_rope_f16"));
}

template <bool H, int VPL, int G, int WT>
int dispatch_rope(int rope, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                  int64_t nw, const void* w, float eps, float off, const float* c,
                  const float* sn, int64_t tld, int64_t ths, int64_t tokens, int tb, int64_t hd,
                  hipStream_t s) {
  switch (rope) {
    case KX_ROPE_NONE:
      return launch_rmsnorm_rope<H, VPL, G, KX_ROPE_NONE, WT>(x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld,
                                                              ths, tokens, tb, hd, s);
    case KX_ROPE_SPLIT:
      return launch_rmsnorm_rope<H, VPL, G, KX_ROPE_SPLIT, WT>(x, ldx, y, ldy, rows, nw, w, eps, off, c, sn,
                                                               tld, ths, tokens, tb, hd, s);
    default:
      return launch_rmsnorm_rope<H, VPL, G, KX_ROPE_PAIR, WT>(x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld,
                                                              ths, tokens, tb, hd, s);
  }
}

template <bool H, int VPL, int WT>
int dispatch_group(int64_t gw, int rope, const void* x, int64_t ldx, void* y, int64_t ldy,
                   int64_t rows, int64_t nw, const void* w, float eps, float off,
                   const float* c, const float* sn, int64_t tld, int64_t ths, int64_t tokens,
                   int tb, int64_t hd, hipStream_t s) {
  switch (gw) {
    case 0:
      return dispatch_rope<H, VPL, 0, WT>(rope, x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld, ths, tokens,
                                          tb, hd, s);
    case 8:
      return dispatch_rope<H, VPL, 8, WT>(rope, x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld, ths, tokens,
                                          tb, hd, s);
    case 16:
      return dispatch_rope<H, VPL, 16, WT>(rope, x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld, ths, tokens,
                                           tb, hd, s);
    default:
      return dispatch_rope<H, VPL, 32, WT>(rope, x, ldx, y, ldy, rows, nw, w, eps, off, c, sn, tld, ths, tokens,
                                           tb, hd, s);
  }
}

template <bool H>
int adaln_norm(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim, const float* shift,
               const float* scale, int64_t mod_div, int64_t mod_stride, float eps, int kind, hipStream_t s) {
  const char* name = ename<H>("kx_adaln_norm_bf16", "kx_adaln_norm_f16");
  KX_REQUIRE(x && y, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && dim > 0 && ldx >= dim && ldy >= dim, "%s: bad shape", name);
  KX_REQUIRE((shift == nullptr) == (scale == nullptr), "%s: shift and scale must both be given or both be null",
             name);
  KX_REQUIRE(!shift || (mod_div > 0 && mod_stride >= 0), "%s: bad modulation", name);
  const bool xf32 = kind & KX_NORM_IN_F32;
  kind &= ~KX_NORM_IN_F32;
  KX_REQUIRE(kind == KX_NORM_RMS || kind == KX_NORM_LAYER, "%s: bad kind", name);
  if (rows == 0) return KX_OK;
  const int64_t vpl = dim / 512;
  const bool vec = dim % 512 == 0 && (vpl == 1 || vpl == 2 || vpl == 4 || vpl == 8) &&
                   ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) && aligned16(y) &&
                   (!shift || (aligned16(shift) && aligned16(scale) && mod_stride % 4 == 0));
  if (xf32)
    return kind == KX_NORM_RMS
               ? dispatch_adaln<H, KX_NORM_RMS, true>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div, mod_stride,
                                                      eps, vec, s)
               : dispatch_adaln<H, KX_NORM_LAYER, true>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div,
                                                        mod_stride, eps, vec, s);
  return kind == KX_NORM_RMS
             ? dispatch_adaln<H, KX_NORM_RMS, false>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div, mod_stride,
                                                     eps, vec, s)
             : dispatch_adaln<H, KX_NORM_LAYER, false>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div,
                                                       mod_stride, eps, vec, s);
}

template <bool H, int WT>
int rmsnorm_rope(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim, int64_t norm_width,
                 const void* w, float eps, float weight_offset, int rope_kind, const float* cos, const float* sin,
                 int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched, int64_t head_dim,
                 hipStream_t s) {
  const char* name = ename<H>("kx_rmsnorm_rope_bf16", "kx_rmsnorm_rope_f16");
  const int64_t vpl = dim / 512;
  const int64_t group_lanes = norm_width == dim ? 0 : norm_width / 8;
  const bool shape_ok = dim % 512 == 0 && (vpl == 1 || vpl == 2 || vpl == 4 || vpl == 8) &&
                        (norm_width == dim ||
                         (norm_width % 8 == 0 &&
                          (group_lanes == 8 || group_lanes == 16 || group_lanes == 32)));
  bool rope_ok = true;
  if (rope_kind == KX_ROPE_SPLIT)
    rope_ok = head_dim >= 16 && 512 % head_dim == 0 && ((head_dim / 2) % 8 == 0);
  else if (rope_kind == KX_ROPE_PAIR)
    rope_ok = 512 % head_dim == 0 && head_dim >= 8;
  const bool align_ok = ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) && aligned16(y);
  if (shape_ok && align_ok && rope_kind == KX_ROPE_SPLIT && norm_width == dim && head_dim == 128 &&
      vpl >= 2 && table_ld % 4 == 0 && table_hs % 4 == 0 && aligned16(cos) && aligned16(sin)) {
    const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
#define KX_RS(V)                                                                                          \
  rmsnorm_rope_split128_kernel<H, V, WT><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, \
      w, eps, weight_offset, cos, sin, table_ld, table_hs, tokens, table_batched);                        \
  return check_launch(name);
    switch (vpl) {
      case 2: KX_RS(2)
      case 4: KX_RS(4)
      default: KX_RS(8)
    }
#undef KX_RS
  }
  if (shape_ok && rope_ok && align_ok) {
#define KX_RR(V)                                                                                       \
  return dispatch_group<H, V, WT>(group_lanes, rope_kind, x, ldx, y, ldy, rows, norm_width, w, eps,     \
                                  weight_offset, cos, sin, table_ld, table_hs, tokens, table_batched, head_dim, s);
    switch (vpl) {
      case 1: KX_RR(1)
      case 2: KX_RR(2)
      case 4: KX_RR(4)
      default: KX_RR(8)
    }
#undef KX_RR
  }
  if (rope_kind != KX_ROPE_NONE)
    return set_error(KX_ERR_UNSUPPORTED,
                     "%s: fused RoPE needs dim in {512,1024,2048,4096}, aligned rows and a head_dim dividing 512",
                     name);
  const int64_t groups = rows * (dim / norm_width);
  const dim3 grid((unsigned)((groups + kWaves - 1) / kWaves));
  rmsnorm_generic<H, WT><<<grid, 256, 0, s>>>((const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, dim, norm_width, w,
                                              eps, weight_offset);
  return check_launch(name);
}

template <bool H>
int rmsnorm_rope_checked(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim,
                         int64_t norm_width, const void* w, int w_dtype, float eps, float weight_offset, int rope_kind,
                         const float* cos, const float* sin, int64_t table_ld, int64_t table_hs, int64_t tokens,
                         int table_batched, int64_t head_dim, hipStream_t s) {
  const char* name = ename<H>("kx_rmsnorm_rope_bf16", "kx_rmsnorm_rope_f16");
  KX_REQUIRE(x && y && w, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && dim > 0 && ldx >= dim && ldy >= dim, "%s: bad shape", name);
  KX_REQUIRE(norm_width > 0 && dim % norm_width == 0, "%s: bad norm width", name);
  KX_REQUIRE(w_dtype == KX_F32 || w_dtype == KX_BF16 || w_dtype == KX_F16, "%s: bad weight dtype", name);
  KX_REQUIRE(rope_kind >= KX_ROPE_NONE && rope_kind <= KX_ROPE_PAIR, "%s: bad rope kind", name);
  if (rope_kind != KX_ROPE_NONE) {
    KX_REQUIRE(cos && sin, "%s: null table", name);
    KX_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && dim % head_dim == 0, "%s: bad head_dim", name);
    KX_REQUIRE(table_batched || tokens > 0, "%s: bad token count", name);
  }
  if (rows == 0) return KX_OK;
#define KX_RN(WT) \
  return rmsnorm_rope<H, WT>(x, ldx, y, ldy, rows, dim, norm_width, w, eps, weight_offset, rope_kind, cos, sin, \
                             table_ld, table_hs, tokens, table_batched, head_dim, s);
  switch (w_dtype) {
    case KX_BF16: KX_RN(KX_BF16)
    case KX_F16: KX_RN(KX_F16)
    default: KX_RN(KX_F32)
  }
#undef KX_RN
}

template <bool H>
int qk_rmsnorm_rope(const void* xq, int64_t ldq, const void* xk, int64_t ldk, void* yq, int64_t ldyq, void* yk,
                    int64_t ldyk, int64_t rows, int64_t dim, const void* wq, const void* wk, int w_dtype, float eps,
                    float weight_offset, const float* cos, const float* sin, int64_t table_ld, int64_t table_hs,
                    int64_t tokens, int table_batched, hipStream_t s) {
  const char* name = ename<H>("kx_qk_rmsnorm_rope_bf16", "kx_qk_rmsnorm_rope_f16");
  KX_REQUIRE(xq && xk && yq && yk && wq && wk && cos && sin, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && dim > 0 && ldq >= dim && ldk >= dim && ldyq >= dim && ldyk >= dim, "%s: bad shape", name);
  KX_REQUIRE(w_dtype == KX_F32 || w_dtype == KX_BF16 || w_dtype == KX_F16, "%s: bad weight dtype", name);
  KX_REQUIRE(table_batched || tokens > 0, "%s: bad token count", name);
  const int64_t vpl = dim / 512;
  const bool ok = dim % 512 == 0 && (vpl == 2 || vpl == 4 || vpl == 8) && ldq % 8 == 0 && ldk % 8 == 0 &&
                  ldyq % 8 == 0 && ldyk % 8 == 0 && aligned16(xq) && aligned16(xk) && aligned16(yq) &&
                  aligned16(yk) && table_ld % 4 == 0 && table_hs % 4 == 0 && aligned16(cos) && aligned16(sin);
  if (!ok)
    return set_error(KX_ERR_UNSUPPORTED,
                     "%s: needs dim in {1024, 2048, 4096}, 128-wide heads and 16-byte aligned rows and tables", name);
  if (rows == 0) return KX_OK;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
#define KX_QK(V, WT)                                                                                        \
  qk_rmsnorm_rope_split128_kernel<H, V, WT><<<grid, 256, 0, s>>>(                                            \
      (const uint16_t*)xq, ldq, (const uint16_t*)xk, ldk, (uint16_t*)yq, ldyq, (uint16_t*)yk, ldyk, rows, wq, wk, \
      eps, weight_offset, cos, sin, table_ld, table_hs, tokens, table_batched);                              \
  return check_launch(name);
#define KX_QKW(V)                          \
  switch (w_dtype) {                       \
    case KX_BF16: KX_QK(V, KX_BF16)        \
    case KX_F16: KX_QK(V, KX_F16)          \
    default: KX_QK(V, KX_F32)              \
  }
  switch (vpl) {
    case 2: KX_QKW(2)
    case 4: KX_QKW(4)
    default: KX_QKW(8)
  }
#undef KX_QKW
#undef KX_QK
}

template <bool H>
int modulate(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t dim, const float* shift,
             const float* scale, int64_t mod_div, int64_t mod_stride, hipStream_t s) {
  const char* name = ename<H>("kx_modulate_bf16", "kx_modulate_f16");
  KX_REQUIRE(x && y && shift && scale, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && dim > 0 && ldx >= dim && ldy >= dim && mod_div > 0 && mod_stride >= 0, "%s: bad shape",
             name);
  const int64_t total = rows * dim;
  if (total == 0) return KX_OK;
  modulate_kernel<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      (const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, dim, shift, scale, mod_div, mod_stride);
  return check_launch(name);
}

template <bool H>
int gated_residual(const void* x, int64_t ldx, const void* r, int64_t ldr, void* y, int64_t ldy, int64_t rows,
                   int64_t dim, const float* gate, int64_t gate_div, int64_t gate_stride, hipStream_t s) {
  const char* name = ename<H>("kx_gated_residual_bf16", "kx_gated_residual_f16");
  KX_REQUIRE(r && y && gate, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && dim > 0 && ldr >= dim && ldy >= dim && (!x || ldx >= dim) && gate_div > 0 &&
                 gate_stride >= 0,
             "%s: bad shape", name);
  const int64_t total = rows * dim;
  if (total == 0) return KX_OK;
  gated_residual_kernel<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      (const uint16_t*)x, ldx, (const uint16_t*)r, ldr, (uint16_t*)y, ldy, rows, dim, gate, gate_div, gate_stride);
  return check_launch(name);
}

}  // namespace
}  // namespace kx

using namespace kx;

#define KX_NORM_ENTRY(SUFFIX, H)                                                                                  \
  extern "C" int kx_adaln_norm_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,          \
                                        int64_t dim, const float* shift, const float* scale, int64_t mod_div,     \
                                        int64_t mod_stride, float eps, int kind, kx_stream_t stream) {            \
    return adaln_norm<H>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div, mod_stride, eps, kind,                 \
                         (hipStream_t)stream);                                                                    \
  }                                                                                                               \
  extern "C" int kx_rmsnorm_rope_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,        \
                                          int64_t dim, int64_t norm_width, const void* w, int w_dtype, float eps, \
                                          float weight_offset, int rope_kind, const float* cos, const float* sin, \
                                          int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,  \
                                          int64_t head_dim, kx_stream_t stream) {                                 \
    return rmsnorm_rope_checked<H>(x, ldx, y, ldy, rows, dim, norm_width, w, w_dtype, eps, weight_offset,         \
                                   rope_kind, cos, sin, table_ld, table_hs, tokens, table_batched, head_dim,      \
                                   (hipStream_t)stream);                                                          \
  }                                                                                                               \
  extern "C" int kx_qk_rmsnorm_rope_##SUFFIX(const void* xq, int64_t ldq, const void* xk, int64_t ldk, void* yq, \
                                             int64_t ldyq, void* yk, int64_t ldyk, int64_t rows, int64_t dim,     \
                                             const void* wq, const void* wk, int w_dtype, float eps,              \
                                             float weight_offset, const float* cos, const float* sin,             \
                                             int64_t table_ld, int64_t table_hs, int64_t tokens,                  \
                                             int table_batched, kx_stream_t stream) {                             \
    return qk_rmsnorm_rope<H>(xq, ldq, xk, ldk, yq, ldyq, yk, ldyk, rows, dim, wq, wk, w_dtype, eps,              \
                              weight_offset, cos, sin, table_ld, table_hs, tokens, table_batched,                 \
                              (hipStream_t)stream);                                                               \
  }                                                                                                               \
  extern "C" int kx_modulate_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,            \
                                      int64_t dim, const float* shift, const float* scale, int64_t mod_div,       \
                                      int64_t mod_stride, kx_stream_t stream) {                                   \
    return modulate<H>(x, ldx, y, ldy, rows, dim, shift, scale, mod_div, mod_stride, (hipStream_t)stream);       \
  }                                                                                                               \
  extern "C" int kx_gated_residual_##SUFFIX(const void* x, int64_t ldx, const void* r, int64_t ldr, void* y,     \
                                            int64_t ldy, int64_t rows, int64_t dim, const float* gate,            \
                                            int64_t gate_div, int64_t gate_stride, kx_stream_t stream) {          \
    return gated_residual<H>(x, ldx, r, ldr, y, ldy, rows, dim, gate, gate_div, gate_stride,                     \
                             (hipStream_t)stream);                                                                \
  }

KX_NORM_ENTRY(bf16, false)
KX_NORM_ENTRY(f16, true)
