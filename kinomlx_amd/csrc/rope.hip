// Standalone rotary embeddings (HBM-bound elementwise passes).
//
// Split-half RoPE keeps the reference's exact fp32 order: each product rounded on its own, then
// the difference or sum, then one cast (contraction into FMA is switched off for these lines).
#include "common.h"

// No FMA contraction anywhere in this file: every product is rounded on its own.
#pragma clang fp contract(off)

namespace kx {
namespace {

// Vectorized split RoPE: each thread rotates 8 consecutive pairs (i .. i+7 of one head) of one
// row; requires half % 8 == 0 and 16-byte aligned rows and tables.
template <bool H>
__global__ __launch_bounds__(256) void rope_split_vec(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t tokens, int heads, int half, const float* __restrict__ cosp,
    const float* __restrict__ sinp, int64_t rows, int table_batched) {
  const int per_row = heads * half / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int64_t row = idx / per_row;
  const int j8 = (int)(idx - row * per_row) * 8;  // pair index j = h * half + i
  const int h = j8 / half, i = j8 - h * half;
  const int64_t t = row % tokens, b = row / tokens;
  const int64_t entry = ((table_batched ? b : 0) * tokens + t) * (int64_t)(heads * half) + j8;
  const uint16_t* xr = x + row * ldx + (int64_t)h * 2 * half + i;
  float f[8], s2[8];
  e_unpack8<H>(*reinterpret_cast<const uint4*>(xr), f);
  e_unpack8<H>(*reinterpret_cast<const uint4*>(xr + half), s2);
  const float4 c0 = *reinterpret_cast<const float4*>(cosp + entry);
  const float4 c1 = *reinterpret_cast<const float4*>(cosp + entry + 4);
  const float4 n0 = *reinterpret_cast<const float4*>(sinp + entry);
  const float4 n1 = *reinterpret_cast<const float4*>(sinp + entry + 4);
  const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float s[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
  float o1[8], o2[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float first_c = f[k] * c[k];
    const float second_s = s2[k] * s[k];
    o1[k] = first_c - second_s;
    const float first_s = f[k] * s[k];
    const float second_c = s2[k] * c[k];
    o2[k] = first_s + second_c;
  }
  uint16_t* yr = y + row * ldy + (int64_t)h * 2 * half + i;
  *reinterpret_cast<uint4*>(yr) = e_pack8<H>(o1);
  *reinterpret_cast<uint4*>(yr + half) = e_pack8<H>(o2);
}

template <bool H>
__global__ __launch_bounds__(256) void rope_split_scalar(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t tokens, int heads, int half, const float* __restrict__ cosp,
    const float* __restrict__ sinp, int64_t rows, int table_batched) {
  const int per_row = heads * half;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int64_t row = idx / per_row;
  const int j = (int)(idx - row * per_row);
  const int h = j / half, i = j - h * half;
  const int64_t t = row % tokens, b = row / tokens;
  const int64_t entry = ((table_batched ? b : 0) * tokens + t) * (int64_t)per_row + j;
  const int64_t off = (int64_t)h * 2 * half + i;
  const float c = cosp[entry], s = sinp[entry];
  const float first = e2f<H>(x[row * ldx + off]);
  const float second = e2f<H>(x[row * ldx + off + half]);
  const float first_c = first * c;
  const float second_s = second * s;
  const float rotated_first = first_c - second_s;
  const float first_s = first * s;
  const float second_c = second * c;
  const float rotated_second = first_s + second_c;
  y[row * ldy + off] = f2e<H>(rotated_first);
  y[row * ldy + off + half] = f2e<H>(rotated_second);
}

template <bool H>
__global__ __launch_bounds__(256) void rope_pair_scalar(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
    int64_t rows, int heads, int head_dim, const float* __restrict__ cosp,
    const float* __restrict__ sinp, int64_t table_ld, int64_t table_hs, int64_t tokens,
    int table_batched) {
  const int pairs = heads * head_dim / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * pairs) return;
  const int64_t row = idx / pairs;
  const int p = (int)(idx - row * pairs);
  const int h = (2 * p) / head_dim, d = 2 * p - h * head_dim;
  const int64_t tok = table_batched ? row : row % tokens;
  const float* ct = cosp + tok * table_ld + (int64_t)h * table_hs + d;
  const float* st = sinp + tok * table_ld + (int64_t)h * table_hs + d;
  const int64_t off = (int64_t)h * head_dim + d;
  const float x0 = e2f<H>(x[row * ldx + off]);
  const float x1 = e2f<H>(x[row * ldx + off + 1]);
  const float a0 = x0 * ct[0];
  const float b0 = (-x1) * st[0];
  const float a1 = x1 * ct[1];
  const float b1 = x0 * st[1];
  y[row * ldy + off] = f2e<H>(a0 + b0);
  y[row * ldy + off + 1] = f2e<H>(a1 + b1);
}

// LTX split-RoPE tables (kinomlx/models/ltx2/transformer/rope.py:95-176): for token t of batch b
// and table column j < half, with pad = half - axes * n leading columns of (cos 1, sin 0), column
// pad + f * axes + a holds the angle ((p / max_pos[a]) * 2 - 1) * grid[f] of axis a, where p is
// the position (the mean of the two bounds with `middle`). Every step is one fp32 op rounded on
// its own, as the reference's array ops are.
__global__ __launch_bounds__(256) void ltx_rope_tables_kernel(
    const float* __restrict__ pos, int64_t pstride, int middle, const float* __restrict__ max_pos,
    const float* __restrict__ grid, float* __restrict__ cos_out, float* __restrict__ sin_out,
    int64_t total, int64_t tokens, int axes, int n, int half) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t bt = idx / half;
  const int j = (int)(idx - bt * half);
  const int pad = half - axes * n;
  float c = 1.0f, s = 0.0f;
  if (j >= pad) {
    const int jj = j - pad;
    const int f = jj / axes, a = jj - f * axes;
    const int64_t b = bt / tokens, t = bt - b * tokens;
    const float* p = pos + ((b * axes + a) * tokens + t) * pstride;
    const float v = middle ? (p[0] + p[1]) / 2.0f : p[0];
    const float frac = v / max_pos[a];
    const float scaled = frac * 2.0f - 1.0f;
    sincosf(scaled * grid[f], &s, &c);
  }
  cos_out[idx] = c;
  sin_out[idx] = s;
}

}  // namespace
}  // namespace kx

using namespace kx;

namespace kx {
namespace {

template <bool H>
int rope_split(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t batch, int64_t tokens, int64_t heads,
               int64_t half, const float* cos, const float* sin, int table_batched, hipStream_t s) {
  const char* name = ename<H>("kx_rope_split_bf16", "kx_rope_split_f16");
  KX_REQUIRE(x && y && cos && sin, "%s: null tensor", name);
  KX_REQUIRE(batch >= 0 && tokens >= 0 && heads > 0 && half > 0, "%s: bad shape", name);
  KX_REQUIRE(ldx >= heads * 2 * half && ldy >= heads * 2 * half, "%s: bad stride", name);
  KX_REQUIRE(heads * half < (1ll << 30), "%s: row too wide", name);
  const int64_t rows = batch * tokens;
  if (rows == 0) return KX_OK;
  const bool vec = half % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) && aligned16(y) &&
                   aligned16(cos) && aligned16(sin);
  if (vec) {
    const int64_t total = rows * heads * half / 8;
    rope_split_vec<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
        (const uint16_t*)x, ldx, (uint16_t*)y, ldy, tokens, (int)heads, (int)half, cos, sin, rows, table_batched);
  } else {
    const int64_t total = rows * heads * half;
    rope_split_scalar<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
        (const uint16_t*)x, ldx, (uint16_t*)y, ldy, tokens, (int)heads, (int)half, cos, sin, rows, table_batched);
  }
  return check_launch(name);
}

template <bool H>
int rope_pair(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t heads, int64_t head_dim,
              const float* cos, const float* sin, int64_t table_ld, int64_t table_hs, int64_t tokens,
              int table_batched, hipStream_t s) {
  const char* name = ename<H>("kx_rope_pair_bf16", "kx_rope_pair_f16");
  KX_REQUIRE(x && y && cos && sin, "%s: null tensor", name);
  KX_REQUIRE(rows >= 0 && heads > 0 && head_dim > 0 && head_dim % 2 == 0, "%s: bad shape", name);
  KX_REQUIRE(ldx >= heads * head_dim && ldy >= heads * head_dim, "%s: bad stride", name);
  KX_REQUIRE(table_batched || tokens > 0, "%s: bad token count", name);
  if (rows == 0) return KX_OK;
  const int64_t total = rows * heads * head_dim / 2;
  rope_pair_scalar<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      (const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, (int)heads, (int)head_dim, cos, sin, table_ld, table_hs,
      tokens, table_batched);
  return check_launch(name);
}

}  // namespace
}  // namespace kx

#define KX_ROPE_ENTRY(SUFFIX, H)                                                                                 \
  extern "C" int kx_rope_split_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t batch,         \
                                        int64_t tokens, int64_t heads, int64_t half, const float* cos,            \
                                        const float* sin, int table_batched, kx_stream_t stream) {                \
    return rope_split<H>(x, ldx, y, ldy, batch, tokens, heads, half, cos, sin, table_batched,                    \
                         (hipStream_t)stream);                                                                    \
  }                                                                                                               \
  extern "C" int kx_rope_pair_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,           \
                                       int64_t heads, int64_t head_dim, const float* cos, const float* sin,       \
                                       int64_t table_ld, int64_t table_hs, int64_t tokens, int table_batched,     \
                                       kx_stream_t stream) {                                                      \
    return rope_pair<H>(x, ldx, y, ldy, rows, heads, head_dim, cos, sin, table_ld, table_hs, tokens,             \
                        table_batched, (hipStream_t)stream);                                                      \
  }

KX_ROPE_ENTRY(bf16, false)
KX_ROPE_ENTRY(f16, true)

extern "C" int kx_ltx_rope_tables(const float* positions, int64_t pos_stride, int middle,
                                  const float* max_pos, const float* grid, float* cos, float* sin,
                                  int64_t batch, int64_t axes, int64_t tokens, int64_t n,
                                  int64_t half, kx_stream_t stream) {
  KX_REQUIRE(positions && max_pos && grid && cos && sin, "kx_ltx_rope_tables: null tensor");
  KX_REQUIRE(batch >= 0 && tokens >= 0 && axes > 0 && axes <= 16 && n > 0 && half > 0 &&
                 axes * n <= half && half < (1 << 24),
             "kx_ltx_rope_tables: bad shape (axes=%lld n=%lld half=%lld)", (long long)axes,
             (long long)n, (long long)half);
  KX_REQUIRE(pos_stride >= (middle ? 2 : 1), "kx_ltx_rope_tables: bad position stride");
  const int64_t total = batch * tokens * half;
  KX_REQUIRE(total / 256 < (1ll << 31), "kx_ltx_rope_tables: too many elements");
  if (total == 0) return KX_OK;
  ltx_rope_tables_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      positions, pos_stride, middle, max_pos, grid, cos, sin, total, tokens, (int)axes, (int)n,
      (int)half);
  return check_launch("kx_ltx_rope_tables");
}
