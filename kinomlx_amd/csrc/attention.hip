// Non-causal flash attention on gfx950 MFMA for token-major flattened heads.
//
// One workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries. K and V advance
// in tiles of 64 keys through a double-buffered LDS stage (global loads for tile i+1 are issued
// before tile i's MFMAs and written to the other buffer afterwards; one barrier per tile).
//
// Layout trick: scores are computed transposed, S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A =
// 32 keys from LDS, B = the wave's 32 queries held in registers for the whole loop). The
// accumulator's lane then holds one query (lane % 32) and 16 of the 32 keys, so the softmax row
// max / sum is an in-lane reduction plus one exchange with lane ^ 32. The output is accumulated
// transposed too, O^T += V^T P^T: P^T comes straight out of the S^T accumulator (converted to
// bf16) as the B operand, and V^T is the A operand read from an LDS tile that the loader writes
// transposed (rows = head dims, 64 keys per row), with keys permuted inside each 16-key group as
// {0-3, 8-11 | 4-7, 12-15} so that one 16-byte LDS read gives a lane exactly the 8 keys its P^T
// operand covers.
//
// Softmax: scores scaled into the exp2 domain (scale * log2 e folded into one multiply), running
// max per query, the O^T rescale skipped when no query's max moved in a tile, fp32 sums. Keys
// past the end are masked to -inf; queries past the end are computed on a clamped row and not
// stored. An optional per-(query, head) gate multiplies the output before the single bf16
// rounding.
#include <math.h>

#include "common.h"

namespace kx {
namespace {

constexpr int BQ = 128;  // queries per workgroup (4 waves x 32)
constexpr int BKV = 64;  // keys per LDS tile

__device__ __forceinline__ uint32_t half16(const uint4& v, int j) {
  const uint32_t w = (j >> 1) == 0 ? v.x : (j >> 1) == 1 ? v.y : (j >> 1) == 2 ? v.z : v.w;
  return (j & 1) ? (w >> 16) : (w & 0xffffu);
}

// Swizzle of 16-byte chunks in a 128-byte V^T row: distinct for 8 consecutive rows (fragment
// reads) and for rows 8 apart (the transposing writes).
__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

template <int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, int64_t ldq, const uint16_t* __restrict__ K, int64_t ldk,
    const uint16_t* __restrict__ V, int64_t ldv, uint16_t* __restrict__ O, int64_t ldo, int tq,
    int tk, int heads, float scale_log2, const uint16_t* __restrict__ gate, int64_t ld_gate,
    int qtiles) {
  constexpr int DC = D / 8;           // 16-byte chunks per K row
  constexpr int KROWB = D * 2;        // bytes per K row in LDS
  constexpr int KT_BYTES = BKV * KROWB;
  constexpr int VROWB = BKV * 2;      // bytes per V^T row (64 keys)
  constexpr int STAGE = KT_BYTES + D * VROWB;
  constexpr int QS = D / 16;          // k16 steps of Q K^T
  constexpr int DB = D / 32;          // 32-row blocks of O^T
  constexpr int K_PER = BKV * DC / 256;
  constexpr int VBLK = (BKV / 4) * DC;  // (4-key, 8-dim) transpose blocks per tile
  static_assert(K_PER >= 1 && VBLK <= 256, "tile shape");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 31, lhalf = lane >> 5;

  // Work order: XCD-contiguous so the workgroups of one XCD share few heads' K/V in its L2.
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = t % qtiles;
  const int bh = t / qtiles;
  const int h = bh % heads, b = bh / heads;
  const uint16_t* Qb = Q + (int64_t)b * tq * ldq + (int64_t)h * D;
  const uint16_t* Kb = K + (int64_t)b * tk * ldk + (int64_t)h * D;
  const uint16_t* Vb = V + (int64_t)b * tk * ldv + (int64_t)h * D;

  const int q0 = qt * BQ + wave * 32;
  const int qrow = min(q0 + lrow, tq - 1);
  bf16x8 qf[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s)
    qf[s] = *reinterpret_cast<const bf16x8*>(Qb + (int64_t)qrow * ldq + (2 * s + lhalf) * 8);

  uint4 rk[K_PER];
  uint4 rv[4];
  const int v_do = tid % DC, v_kq = tid / DC;

  auto load_kv = [&](int j0) {
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int q = tid + 256 * i;
      const int key = q / DC, c = q % DC;
      const int gk = min(j0 + key, tk - 1);
      rk[i] = *reinterpret_cast<const uint4*>(Kb + (int64_t)gk * ldk + c * 8);
    }
    if (tid < VBLK) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gk = min(j0 + 4 * v_kq + r, tk - 1);
        rv[r] = *reinterpret_cast<const uint4*>(Vb + (int64_t)gk * ldv + v_do * 8);
      }
    }
  };

  auto store_kv = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int q = tid + 256 * i;
      const int key = q / DC, c = q % DC;
      *reinterpret_cast<uint4*>(buf + key * KROWB + ((c ^ (key & 7)) << 4)) = rk[i];
    }
    if (tid < VBLK) {
      const int grp = v_kq >> 2, q4 = v_kq & 3;
      const int ch = 2 * grp + (q4 & 1);
      const int off = (q4 >> 1) * 8;
      uint8_t* vt = buf + KT_BYTES;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = v_do * 8 + j;
        uint2 w;
        w.x = half16(rv[0], j) | (half16(rv[1], j) << 16);
        w.y = half16(rv[2], j) | (half16(rv[3], j) << 16);
        *reinterpret_cast<uint2*>(vt + d * VROWB + ((ch ^ vt_swz(d)) << 4) + off) = w;
      }
    }
  };

  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  float m_run = -INFINITY;  // running max, exp2 domain
  float l_run = 0.0f;       // this lane's partial row sum

  const int ntiles = (tk + BKV - 1) / BKV;
  load_kv(0);
  store_kv(smem);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const uint8_t* cur = smem + (it & 1) * STAGE;
    const bool more = it + 1 < ntiles;
    if (more) load_kv((it + 1) * BKV);

    // S^T = K Q^T for two 32-key blocks
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
      const int krow = kb * 32 + lrow;
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(
            cur + krow * KROWB + (((2 * st + lhalf) ^ (krow & 7)) << 4));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kb], 0, 0, 0);
      }
    }

    // scale into the exp2 domain, mask keys past the end
    const int j0 = it * BKV;
    const bool tail = j0 + BKV > tk;
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = s[kb][e] * scale_log2;
        if (tail) {
          const int key = j0 + kb * 32 + 8 * (e >> 2) + 4 * lhalf + (e & 3);
          if (key >= tk) x = -INFINITY;
        }
        s[kb][e] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    if (__any(m_new != m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
      m_run = m_new;
    }

    // P^T in bf16 as the B operand: elements 8hf .. 8hf+7 of block kb
    bf16x8 pb[2][2];
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p = __builtin_amdgcn_exp2f(s[kb][8 * hf + e] - m_run);
          psum += p;
          pb[kb][hf][e] = (__bf16)p;
        }
    l_run += psum;

    // O^T += V^T P^T
    const uint8_t* vt = cur + KT_BYTES;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d = db * 32 + lrow;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int ch = 2 * (2 * kb + hf) + lhalf;
          const bf16x8 vf =
              *reinterpret_cast<const bf16x8*>(vt + d * VROWB + ((ch ^ vt_swz(d)) << 4));
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[kb][hf], o[db], 0, 0, 0);
        }
    }

    if (more) store_kv(smem + ((it + 1) & 1) * STAGE);
    __syncthreads();
  }

  // normalise, gate, store: lane holds query q0 + lrow, dims db*32 + 8g + 4*lhalf + (0..3)
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const int q = q0 + lrow;
  if (q >= tq) return;
  float scale_out = 1.0f / l_tot;
  if (gate) scale_out *= bf2f(gate[((int64_t)b * tq + q) * ld_gate + h]);
  uint16_t* orow = O + ((int64_t)b * tq + q) * ldo + (int64_t)h * D;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack2(o[db][4 * g + 0] * scale_out, o[db][4 * g + 1] * scale_out);
      w.y = pack2(o[db][4 * g + 2] * scale_out, o[db][4 * g + 3] * scale_out);
      *reinterpret_cast<uint2*>(orow + db * 32 + 8 * g + 4 * lhalf) = w;
    }
}

template <int D>
int launch_attn(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk, int64_t heads,
                float scale, const void* gate, int64_t ld_gate, hipStream_t s) {
  const int qtiles = (int)((tq + BQ - 1) / BQ);
  const int64_t blocks = (int64_t)qtiles * heads * batch;
  attn_fwd_kernel<D><<<(unsigned)blocks, 256, 0, s>>>(
      (const uint16_t*)q, ldq, (const uint16_t*)k, ldk, (const uint16_t*)v, ldv, (uint16_t*)o,
      ldo, (int)tq, (int)tk, (int)heads, scale * 1.4426950408889634f, (const uint16_t*)gate,
      ld_gate, qtiles);
  return check_launch("kx_attention_fwd_bf16");
}

}  // namespace
}  // namespace kx

using namespace kx;

extern "C" int kx_attention_fwd_bf16(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                     const void* v, int64_t ldv, void* o, int64_t ldo,
                                     int64_t batch, int64_t tq, int64_t tk, int64_t heads,
                                     int64_t head_dim, float scale, const void* gate,
                                     int64_t ld_gate, kx_stream_t stream) {
  KX_REQUIRE(q && k && v && o, "kx_attention_fwd_bf16: null tensor");
  KX_REQUIRE(head_dim == 64 || head_dim == 128,
             "kx_attention_fwd_bf16: head_dim must be 64 or 128, got %lld", (long long)head_dim);
  KX_REQUIRE(batch >= 0 && tq >= 0 && tk > 0 && heads > 0 && tq < (1ll << 30) &&
                 tk < (1ll << 30),
             "kx_attention_fwd_bf16: bad shape");
  const int64_t width = heads * head_dim;
  KX_REQUIRE(ldq >= width && ldk >= width && ldv >= width && ldo >= width,
             "kx_attention_fwd_bf16: row strides must cover heads * head_dim");
  KX_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 4 == 0 && aligned16(q) &&
                 aligned16(k) && aligned16(v) && aligned8(o),
             "kx_attention_fwd_bf16: q/k/v rows must be 16-byte and o rows 8-byte aligned");
  KX_REQUIRE(!gate || ld_gate >= heads, "kx_attention_fwd_bf16: gate stride must cover heads");
  KX_REQUIRE((int64_t)((tq + BQ - 1) / BQ) * heads * batch < (1ll << 31),
             "kx_attention_fwd_bf16: too many tiles");
  if (tq == 0 || batch == 0) return KX_OK;
  if (head_dim == 128)
    return launch_attn<128>(q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk, heads, scale, gate,
                            ld_gate, (hipStream_t)stream);
  return launch_attn<64>(q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk, heads, scale, gate,
                         ld_gate, (hipStream_t)stream);
}
