// The steps either side of the transformer blocks on gfx950: sinusoidal timestep features, the
// velocity -> denoised (X0) conversion, the conditioning-mask composite, the two Euler updates and
// the finite check of a latent. All are element-wise passes over HBM (memory-bound, a few MB per
// call at video shapes); the arithmetic follows the reference's op order with contraction off, so
// every result is the float32 evaluation rounded once at the same points as the reference.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace kx {
namespace {

template <bool F32>
__device__ __forceinline__ float load_x(const void* p, int64_t i) {
  if constexpr (F32) return static_cast<const float*>(p)[i];
  return bf2f(static_cast<const uint16_t*>(p)[i]);
}

template <bool F32>
__device__ __forceinline__ void store_x(void* p, int64_t i, float v) {
  if constexpr (F32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = f2bf(v);
}

template <bool F32>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (F32) return v;
  return bf2f(f2bf(v));
}

// features[i, j] = cos(t_i f_j) for j < half, sin(t_i f_(j-half)) for half <= j < 2 half, with
// t_i = t[i] * time_scale and f_j = exp((neg_log_period * j) / half) in fp32; a last odd column
// is 0 (kinomlx/models/ltx2/transformer/timestep.py:13-28; the scale is the preprocessor's
// `value * timestep_scale`, preprocessing.py:66-75).
template <bool F32>
__global__ __launch_bounds__(256) void timestep_embedding_kernel(const float* __restrict__ t,
                                                                 void* __restrict__ out, int64_t n,
                                                                 int dim, float time_scale,
                                                                 float neg_log_period) {
#pragma clang fp contract(off)
  const int half = dim / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * dim) return;
  const int64_t i = idx / dim;
  const int j = (int)(idx - i * dim);
  float v = 0.0f;
  if (j < 2 * half) {
    const int jj = j < half ? j : j - half;
    const float e = (neg_log_period * (float)jj) / (float)half;
    const float angle = (t[i] * time_scale) * expf(e);
    v = j < half ? cosf(angle) : sinf(angle);
  }
  store_x<F32>(out, idx, v);
}

// sample + dtype(delta * velocity) (kinomlx/samplers/steps.py:8-32): the scaled velocity is
// rounded to the sample dtype before the add, which rounds again.
template <bool F32>
__global__ __launch_bounds__(256) void euler_velocity_kernel(const void* __restrict__ sample,
                                                             const void* __restrict__ velocity,
                                                             void* __restrict__ out, int64_t n,
                                                             float delta) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float scaled = round_to<F32>(delta * load_x<F32>(velocity, i));
  store_x<F32>(out, i, load_x<F32>(sample, i) + scaled);
}

// denoised + ratio * (sample - denoised) in fp32, rounded once to the sample dtype
// (kinomlx/samplers/steps.py:35-72).
template <bool SF32, bool DF32>
__global__ __launch_bounds__(256) void euler_lerp_kernel(const void* __restrict__ sample,
                                                         const void* __restrict__ denoised,
                                                         void* __restrict__ out, int64_t n,
                                                         float ratio) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float s = load_x<SF32>(sample, i), d = load_x<DF32>(denoised, i);
  const float step = ratio * (s - d);
  store_x<SF32>(out, i, d + step);
}

// latent - timestep * velocity in fp32, rounded once to the latent dtype; row r (one token) uses
// timestep[r / ts_div] (kinomlx/models/ltx2/transformer/wrappers.py:48-66).
template <bool LF32, bool VF32>
__global__ __launch_bounds__(256) void to_denoised_kernel(const void* __restrict__ latent,
                                                          const void* __restrict__ velocity,
                                                          const float* __restrict__ ts,
                                                          void* __restrict__ out, int64_t rows,
                                                          int64_t dim, int64_t ts_div) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * dim) return;
  const int64_t r = i / dim;
  const float prod = ts[r / ts_div] * load_x<VF32>(velocity, i);
  store_x<LF32>(out, i, load_x<LF32>(latent, i) - prod);
}

// denoised * m + clean * (1 - m) in fp32, rounded once to the denoised dtype; row r uses mask[r]
// (kinomlx/models/ltx2/state.py:70-83).
template <bool DF32, bool CF32>
__global__ __launch_bounds__(256) void mask_composite_kernel(const void* __restrict__ denoised,
                                                             const void* __restrict__ clean,
                                                             const float* __restrict__ mask,
                                                             void* __restrict__ out, int64_t rows,
                                                             int64_t dim) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * dim) return;
  const float m = mask[i / dim];
  const float keep = load_x<DF32>(denoised, i) * m;
  const float cond = load_x<CF32>(clean, i) * (1.0f - m);
  store_x<DF32>(out, i, keep + cond);
}

__global__ void flag_init_kernel(int* flag) {
  if (threadIdx.x == 0) flag[0] = 1;
}

// Any non-finite element clears the flag; every writer stores the same 0, so the order of the
// writes does not matter. Grid-stride: the grid is capped by the host.
template <bool F32>
__global__ __launch_bounds__(256) void finite_kernel(const void* __restrict__ x, int64_t n, int* flag) {
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    bad |= !isfinite(load_x<F32>(x, i));
  if (__any(bad) && (threadIdx.x & 63) == 0) flag[0] = 0;
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

bool dtype_ok(int dtype) { return dtype == KX_F32 || dtype == KX_BF16; }

// Calls f(integral_constant<bool, dtype == KX_F32>) for one dtype.
template <typename F>
void with_dtype(int dtype, F&& f) {
  if (dtype == KX_F32) f(std::true_type{});
  else f(std::false_type{});
}

}  // namespace
}  // namespace kx

using namespace kx;

// Element counts are capped so that a grid of 256-thread blocks fits gridDim.x.
static constexpr int64_t kMaxElems = (int64_t)0x7fffffff * 256;

extern "C" int kx_timestep_embedding(const float* t, void* out, int64_t n, int64_t dim, int out_dtype,
                                     float time_scale, float neg_log_period, kx_stream_t stream) {
  KX_REQUIRE(t && out, "kx_timestep_embedding: null tensor");
  KX_REQUIRE(n >= 0 && dim > 0 && dim < (1 << 30) && n <= kMaxElems / dim,
             "kx_timestep_embedding: bad shape (n=%lld dim=%lld)", (long long)n, (long long)dim);
  KX_REQUIRE(dtype_ok(out_dtype), "kx_timestep_embedding: out_dtype must be KX_F32 or KX_BF16");
  if (n == 0) return KX_OK;
  with_dtype(out_dtype, [&](auto f32) {
    timestep_embedding_kernel<decltype(f32)::value>
        <<<blocks_for(n * dim), 256, 0, (hipStream_t)stream>>>(t, out, n, (int)dim, time_scale,
                                                                        neg_log_period);
  });
  return check_launch("kx_timestep_embedding");
}

extern "C" int kx_euler_velocity_step(const void* sample, const void* velocity, void* out, int64_t n,
                                      int dtype, float delta, kx_stream_t stream) {
  KX_REQUIRE(sample && velocity && out, "kx_euler_velocity_step: null tensor");
  KX_REQUIRE(n >= 0 && n <= kMaxElems, "kx_euler_velocity_step: bad size %lld", (long long)n);
  KX_REQUIRE(dtype_ok(dtype), "kx_euler_velocity_step: dtype must be KX_F32 or KX_BF16");
  KX_REQUIRE(isfinite(delta), "kx_euler_velocity_step: delta must be finite");
  if (n == 0) return KX_OK;
  with_dtype(dtype, [&](auto f32) {
    euler_velocity_kernel<decltype(f32)::value>
        <<<blocks_for(n), 256, 0, (hipStream_t)stream>>>(sample, velocity, out, n, delta);
  });
  return check_launch("kx_euler_velocity_step");
}

extern "C" int kx_euler_step(const void* sample, int sample_dtype, const void* denoised,
                             int denoised_dtype, void* out, int64_t n, float ratio, kx_stream_t stream) {
  KX_REQUIRE(sample && denoised && out, "kx_euler_step: null tensor");
  KX_REQUIRE(n >= 0 && n <= kMaxElems, "kx_euler_step: bad size %lld", (long long)n);
  KX_REQUIRE(dtype_ok(sample_dtype) && dtype_ok(denoised_dtype),
             "kx_euler_step: dtypes must be KX_F32 or KX_BF16");
  if (n == 0) return KX_OK;
  with_dtype(sample_dtype, [&](auto sf) {
    with_dtype(denoised_dtype, [&](auto df) {
      euler_lerp_kernel<decltype(sf)::value, decltype(df)::value>
          <<<blocks_for(n), 256, 0, (hipStream_t)stream>>>(sample, denoised, out, n, ratio);
    });
  });
  return check_launch("kx_euler_step");
}

extern "C" int kx_to_denoised(const void* latent, int latent_dtype, const void* velocity,
                              int velocity_dtype, const float* timesteps, void* out, int64_t rows,
                              int64_t dim, int64_t ts_div, kx_stream_t stream) {
  KX_REQUIRE(latent && velocity && timesteps && out, "kx_to_denoised: null tensor");
  KX_REQUIRE(rows >= 0 && dim > 0 && ts_div > 0 && rows <= kMaxElems / dim,
             "kx_to_denoised: bad shape (rows=%lld dim=%lld ts_div=%lld)", (long long)rows,
             (long long)dim, (long long)ts_div);
  KX_REQUIRE(dtype_ok(latent_dtype) && dtype_ok(velocity_dtype),
             "kx_to_denoised: dtypes must be KX_F32 or KX_BF16");
  if (rows == 0) return KX_OK;
  with_dtype(latent_dtype, [&](auto lf) {
    with_dtype(velocity_dtype, [&](auto vf) {
      to_denoised_kernel<decltype(lf)::value, decltype(vf)::value>
          <<<blocks_for(rows * dim), 256, 0, (hipStream_t)stream>>>(latent, velocity, timesteps, out,
                                                                     rows, dim, ts_div);
    });
  });
  return check_launch("kx_to_denoised");
}

extern "C" int kx_mask_composite(const void* denoised, int denoised_dtype, const void* clean,
                                 int clean_dtype, const float* mask, void* out, int64_t rows,
                                 int64_t dim, kx_stream_t stream) {
  KX_REQUIRE(denoised && clean && mask && out, "kx_mask_composite: null tensor");
  KX_REQUIRE(rows >= 0 && dim > 0 && rows <= kMaxElems / dim,
             "kx_mask_composite: bad shape (rows=%lld dim=%lld)", (long long)rows, (long long)dim);
  KX_REQUIRE(dtype_ok(denoised_dtype) && dtype_ok(clean_dtype),
             "kx_mask_composite: dtypes must be KX_F32 or KX_BF16");
  if (rows == 0) return KX_OK;
  with_dtype(denoised_dtype, [&](auto df) {
    with_dtype(clean_dtype, [&](auto cf) {
      mask_composite_kernel<decltype(df)::value, decltype(cf)::value>
          <<<blocks_for(rows * dim), 256, 0, (hipStream_t)stream>>>(denoised, clean, mask, out, rows,
                                                                     dim);
    });
  });
  return check_launch("kx_mask_composite");
}

extern "C" int kx_all_finite(const void* x, int64_t n, int dtype, int* flag, kx_stream_t stream) {
  KX_REQUIRE(flag && (x || n == 0), "kx_all_finite: null tensor");
  KX_REQUIRE(n >= 0, "kx_all_finite: bad size %lld", (long long)n);
  KX_REQUIRE(dtype_ok(dtype), "kx_all_finite: dtype must be KX_F32 or KX_BF16");
  hipStream_t s = (hipStream_t)stream;
  flag_init_kernel<<<1, 64, 0, s>>>(flag);
  if (n > 0) {
    const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 2048);
    with_dtype(dtype, [&](auto f32) {
      finite_kernel<decltype(f32)::value><<<grid, 256, 0, s>>>(x, n, flag);
    });
  }
  return check_launch("kx_all_finite");
}
