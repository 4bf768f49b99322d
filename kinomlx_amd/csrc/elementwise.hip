// FP32-opmath activations with one rounding to the 16-bit type, bf16 or fp16 (HBM-bound
// elementwise passes).
#include "common.h"

namespace kx {
namespace {

template <int OP>
__device__ __forceinline__ float act(float x) {
  return OP == 0 ? gelu_tanh(x) : silu(x);
}

template <bool H, int OP>
__global__ __launch_bounds__(256) void unary_vec(const uint16_t* __restrict__ x,
                                                 uint16_t* __restrict__ y, int64_t vecs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= vecs) return;
  float v[8];
  e_unpack8<H>(reinterpret_cast<const uint4*>(x)[i], v);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = act<OP>(v[j]);
  reinterpret_cast<uint4*>(y)[i] = e_pack8<H>(v);
}

template <bool H, int OP>
__global__ __launch_bounds__(256) void unary_scalar(const uint16_t* __restrict__ x,
                                                    uint16_t* __restrict__ y, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  y[i] = f2e<H>(act<OP>(e2f<H>(x[i])));
}

template <bool H>
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                     uint16_t* __restrict__ y, int64_t ldy,
                                                     int64_t rows, int64_t hidden) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * hidden) return;
  const int64_t r = i / hidden, c = i - r * hidden;
  const float g = e2f<H>(x[r * ldx + c]);
  const float u = e2f<H>(x[r * ldx + hidden + c]);
  y[r * ldy + c] = f2e<H>(silu(g) * u);
}

// fp32 of element i of an fp32, bf16 or fp16 array (dtype code DT)
template <int DT>
__device__ __forceinline__ float load_any(const void* p, int64_t i) {
  if constexpr (DT == KX_F32) return static_cast<const float*>(p)[i];
  else return e2f<DT == KX_F16>(static_cast<const uint16_t*>(p)[i]);
}

// out[(b * tokens + t) * rows + r][c] = fp32(table[r][c]) + fp32(ts[b, t, r, c]) (ts optional),
// then rounded to bf16 / fp16 (RND = KX_BF16 / KX_F16; KX_F32: kept) and stored as fp32.
template <int TAB, int TS, int RND>
__global__ __launch_bounds__(256) void table_add_kernel(const void* __restrict__ table, const void* __restrict__ ts,
                                                        int64_t ts_bs, int64_t ts_ts, int64_t ts_rs,
                                                        float* __restrict__ out, int64_t tokens, int64_t rows,
                                                        int64_t dim, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t c = i % dim, r = (i / dim) % rows, bt = i / (dim * rows);
  const int64_t t = bt % tokens, b = bt / tokens;
  float v = load_any<TAB>(table, r * dim + c);
  if (ts) v += load_any<TS>(ts, b * ts_bs + t * ts_ts + r * ts_rs + c);
  if constexpr (RND != KX_F32) v = e2f<RND == KX_F16>(f2e<RND == KX_F16>(v));
  out[i] = v;
}

template <bool H, int OP>
int launch_unary(const void* x, void* y, int64_t count, hipStream_t s, const char* name) {
  KX_REQUIRE(x && y && count >= 0, "%s: bad argument", name);
  if (count == 0) return KX_OK;
  if (count % 8 == 0 && aligned16(x) && aligned16(y)) {
    const int64_t vecs = count / 8;
    unary_vec<H, OP><<<(unsigned)((vecs + 255) / 256), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)y, vecs);
  } else {
    unary_scalar<H, OP><<<(unsigned)((count + 255) / 256), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)y, count);
  }
  return check_launch(name);
}

template <bool H>
int swiglu(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t hidden, hipStream_t s) {
  const char* name = ename<H>("kx_swiglu_bf16", "kx_swiglu_f16");
  KX_REQUIRE(x && y && rows >= 0 && hidden > 0 && ldx >= 2 * hidden && ldy >= hidden, "%s: bad argument", name);
  const int64_t total = rows * hidden;
  if (total == 0) return KX_OK;
  swiglu_kernel<H><<<(unsigned)((total + 255) / 256), 256, 0, s>>>((const uint16_t*)x, ldx, (uint16_t*)y, ldy,
                                                                  rows, hidden);
  return check_launch(name);
}

}  // namespace
}  // namespace kx

using namespace kx;

#define KX_UNARY_ENTRY(SUFFIX, H)                                                                              \
  extern "C" int kx_gelu_tanh_##SUFFIX(const void* x, void* y, int64_t count, kx_stream_t stream) {            \
    return launch_unary<H, 0>(x, y, count, (hipStream_t)stream, "kx_gelu_tanh_" #SUFFIX);                      \
  }                                                                                                            \
  extern "C" int kx_silu_##SUFFIX(const void* x, void* y, int64_t count, kx_stream_t stream) {                 \
    return launch_unary<H, 1>(x, y, count, (hipStream_t)stream, "kx_silu_" #SUFFIX);                           \
  }                                                                                                            \
  extern "C" int kx_swiglu_##SUFFIX(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,           \
                                    int64_t hidden, kx_stream_t stream) {                                      \
    return swiglu<H>(x, ldx, y, ldy, rows, hidden, (hipStream_t)stream);                                       \
  }

KX_UNARY_ENTRY(bf16, false)
KX_UNARY_ENTRY(f16, true)

extern "C" int kx_table_add_f32(const void* table, int table_dtype, const void* ts, int ts_dtype, int64_t ts_bs,
                                int64_t ts_ts, int64_t ts_rs, float* out, int64_t batch, int64_t tokens,
                                int64_t rows, int64_t dim, int round_dtype, kx_stream_t stream) {
  KX_REQUIRE(table && out && batch >= 0 && tokens > 0 && rows > 0 && dim > 0,
             "kx_table_add_f32: bad argument");
  KX_REQUIRE(table_dtype >= KX_F32 && table_dtype <= KX_F16 && ts_dtype >= KX_F32 && ts_dtype <= KX_F16 &&
                 round_dtype >= KX_F32 && round_dtype <= KX_F16,
             "kx_table_add_f32: dtypes must be KX_F32, KX_BF16 or KX_F16");
  const int64_t total = batch * tokens * rows * dim;
  if (total == 0) return KX_OK;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipStream_t s = (hipStream_t)stream;
#define KX_TABLE_ADD(TB, SB, RB) \
  table_add_kernel<TB, SB, RB><<<blocks, 256, 0, s>>>(table, ts, ts_bs, ts_ts, ts_rs, out, tokens, rows, dim, total)
#define KX_TABLE_RND(TB, SB)                                \
  switch (round_dtype) {                                    \
    case KX_BF16: KX_TABLE_ADD(TB, SB, KX_BF16); break;     \
    case KX_F16: KX_TABLE_ADD(TB, SB, KX_F16); break;       \
    default: KX_TABLE_ADD(TB, SB, KX_F32);                  \
  }
#define KX_TABLE_TS(TB)                                     \
  switch (ts_dtype) {                                       \
    case KX_BF16: KX_TABLE_RND(TB, KX_BF16) break;          \
    case KX_F16: KX_TABLE_RND(TB, KX_F16) break;            \
    default: KX_TABLE_RND(TB, KX_F32)                       \
  }
  switch (table_dtype) {
    case KX_BF16: KX_TABLE_TS(KX_BF16) break;
    case KX_F16: KX_TABLE_TS(KX_F16) break;
    default: KX_TABLE_TS(KX_F32)
  }
#undef KX_TABLE_TS
#undef KX_TABLE_RND
#undef KX_TABLE_ADD
  return check_launch("kx_table_add_f32");
}
