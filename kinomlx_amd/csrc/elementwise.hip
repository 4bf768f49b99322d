// FP32-opmath activations with one bf16 rounding (HBM-bound elementwise passes).
#include "common.h"

namespace kx {
namespace {

template <int OP>
__device__ __forceinline__ float act(float x) {
  return OP == 0 ? gelu_tanh(x) : silu(x);
}

template <int OP>
__global__ __launch_bounds__(256) void unary_vec(const uint16_t* __restrict__ x,
                                                 uint16_t* __restrict__ y, int64_t vecs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= vecs) return;
  float v[8];
  unpack8(reinterpret_cast<const uint4*>(x)[i], v);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = act<OP>(v[j]);
  reinterpret_cast<uint4*>(y)[i] = pack8(v);
}

template <int OP>
__global__ __launch_bounds__(256) void unary_scalar(const uint16_t* __restrict__ x,
                                                    uint16_t* __restrict__ y, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  y[i] = f2bf(act<OP>(bf2f(x[i])));
}

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                     uint16_t* __restrict__ y, int64_t ldy,
                                                     int64_t rows, int64_t hidden) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * hidden) return;
  const int64_t r = i / hidden, c = i - r * hidden;
  const float g = bf2f(x[r * ldx + c]);
  const float u = bf2f(x[r * ldx + hidden + c]);
  y[r * ldy + c] = f2bf(silu(g) * u);
}

// out[(b * tokens + t) * rows + r][c] = fp32(table[r][c]) + fp32(ts[b, t, r, c]) (ts optional).
template <bool TAB_BF16, bool TS_BF16>
__global__ __launch_bounds__(256) void table_add_kernel(const void* __restrict__ table, const void* __restrict__ ts,
                                                        int64_t ts_bs, int64_t ts_ts, int64_t ts_rs,
                                                        float* __restrict__ out, int64_t tokens, int64_t rows,
                                                        int64_t dim, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t c = i % dim, r = (i / dim) % rows, bt = i / (dim * rows);
  const int64_t t = bt % tokens, b = bt / tokens;
  float v = TAB_BF16 ? bf2f(static_cast<const uint16_t*>(table)[r * dim + c])
                     : static_cast<const float*>(table)[r * dim + c];
  if (ts) {
    const int64_t o = b * ts_bs + t * ts_ts + r * ts_rs + c;
    v += TS_BF16 ? bf2f(static_cast<const uint16_t*>(ts)[o]) : static_cast<const float*>(ts)[o];
  }
  out[i] = v;
}

template <int OP>
int launch_unary(const void* x, void* y, int64_t count, hipStream_t s, const char* name) {
  if (count == 0) return KX_OK;
  if (count % 8 == 0 && aligned16(x) && aligned16(y)) {
    const int64_t vecs = count / 8;
    unary_vec<OP><<<(unsigned)((vecs + 255) / 256), 256, 0, s>>>((const uint16_t*)x,
                                                                 (uint16_t*)y, vecs);
  } else {
    unary_scalar<OP><<<(unsigned)((count + 255) / 256), 256, 0, s>>>((const uint16_t*)x,
                                                                     (uint16_t*)y, count);
  }
  return check_launch(name);
}

}  // namespace
}  // namespace kx

using namespace kx;

extern "C" int kx_gelu_tanh_bf16(const void* x, void* y, int64_t count, kx_stream_t stream) {
  KX_REQUIRE(x && y && count >= 0, "kx_gelu_tanh_bf16: bad argument");
  return launch_unary<0>(x, y, count, (hipStream_t)stream, "kx_gelu_tanh_bf16");
}

extern "C" int kx_silu_bf16(const void* x, void* y, int64_t count, kx_stream_t stream) {
  KX_REQUIRE(x && y && count >= 0, "kx_silu_bf16: bad argument");
  return launch_unary<1>(x, y, count, (hipStream_t)stream, "kx_silu_bf16");
}

extern "C" int kx_swiglu_bf16(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                              int64_t hidden, kx_stream_t stream) {
  KX_REQUIRE(x && y && rows >= 0 && hidden > 0 && ldx >= 2 * hidden && ldy >= hidden,
             "kx_swiglu_bf16: bad argument");
  const int64_t total = rows * hidden;
  if (total == 0) return KX_OK;
  swiglu_kernel<<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, ldx, (uint16_t*)y, ldy, rows, hidden);
  return check_launch("kx_swiglu_bf16");
}

extern "C" int kx_table_add_f32(const void* table, int table_dtype, const void* ts, int ts_dtype, int64_t ts_bs,
                                int64_t ts_ts, int64_t ts_rs, float* out, int64_t batch, int64_t tokens,
                                int64_t rows, int64_t dim, kx_stream_t stream) {
  KX_REQUIRE(table && out && batch >= 0 && tokens > 0 && rows > 0 && dim > 0,
             "kx_table_add_f32: bad argument");
  KX_REQUIRE((table_dtype == KX_F32 || table_dtype == KX_BF16) && (ts_dtype == KX_F32 || ts_dtype == KX_BF16),
             "kx_table_add_f32: dtypes must be KX_F32 or KX_BF16");
  const int64_t total = batch * tokens * rows * dim;
  if (total == 0) return KX_OK;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
#define KX_TABLE_ADD(TB, SB) \
  table_add_kernel<TB, SB><<<blocks, 256, 0, s>>>(table, ts, ts_bs, ts_ts, ts_rs, out, tokens, rows, dim, total)
  if (table_dtype == KX_BF16) {
    if (ts_dtype == KX_BF16) KX_TABLE_ADD(true, true); else KX_TABLE_ADD(true, false);
  } else {
    if (ts_dtype == KX_BF16) KX_TABLE_ADD(false, true); else KX_TABLE_ADD(false, false);
  }
#undef KX_TABLE_ADD
  return check_launch("kx_table_add_f32");
}
