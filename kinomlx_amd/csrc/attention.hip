// Non-causal flash attention on gfx950 MFMA for token-major flattened heads.
//
// One workgroup = 12 waves = 384 queries of one head; each wave owns 32 queries and keeps them in
// registers as the MFMA B operand for the whole key loop. Three waves share each SIMD (at most 168
// VGPRs each). At 9216 tokens x 32 heads that is 768 workgroups, three full rounds of one per CU (with 8
// waves the 1152 workgroups took 4.5 rounds: 1.59 -> 1.44 ms), and each LDS K/V tile serves 384
// queries.
//
// K and V tiles of 64 keys go from global memory straight into LDS with buffer_load_dwordx4 ... lds
// (no VGPR staging) through a ring of 4 stages. Waves 0-7 each issue 1/8 of a stage's DMA
// instructions; one workgroup barrier per tile makes a tile visible and frees an older buffer.
// At D = 128 without a score bias the key loop is software-pipelined over 32-key blocks (the next
// block's score MFMAs run beside this block's exps, the P V MFMAs beside the next block's max) and
// tile i+1 becomes visible in the middle of tile i, with tile i+2 in flight; the other forms keep
// one tile per iteration with tiles i+1 .. i+3 in flight.
//
// The 16-bit type is bf16 or fp16 (template H; v_mfma_f32_32x32x16_bf16 / _f16, P rounded to the
// same type). Scores are computed transposed, S^T = K Q^T with one 32x32x16 MFMA (A = 32 keys read from
// LDS, B = the wave's 32 queries): the accumulator lane holds one query (lane % 32) and 16 of the
// 32 keys, so the row max is an in-lane reduction plus one exchange with lane ^ 32. The output
// is accumulated transposed too, O^T += V^T P^T: P^T comes straight out of the S^T accumulator
// (converted to bf16) as the B operand, with the 16 keys of an MFMA step taken in the order
// {0-3, 8-11 | 4-7, 12-15} that the accumulator layout gives; V^T is the A operand, read from the
// V tile kept in its natural key-major layout by the transposing ds_read_b64_tr_b16: a read of 16
// lanes, each addressing 4 dims of one key, hands lane i dim i of 4 consecutive keys.
//
// LDS rows are 2 * D bytes with their 16-byte chunks XOR-swizzled per row: for K so that the 32-row
// fragment reads hit distinct banks, for V so that each transposing read (4 keys x 4 chunks) does.
//
// Softmax: fp32, in the exp2 domain with the scale * log2 e folded into one FMA per score. The
// row sum adds the rounded P pairwise (v_dot2 with (1, 1)), the values the P V product uses; in
// the pipelined form the two lane halves exchange their max by v_permlane32_swap. The running max
// is lazy: it moves (and O, l are rescaled) only when a score exceeds it by more than
// 2^8 in the exp2 domain, so p stays below 256 (exact in fp32 and bf16) and rescales are rare.
// Keys past the end are masked to -inf; queries past the end run on a clamped row and are not
// stored. An optional per-(query, head) gate multiplies the output before the single bf16 rounding.
#include <math.h>

#include "common.h"

namespace kx {
namespace {

constexpr int NWAVE = 12;          // waves per workgroup (three per SIMD)
constexpr int NDMA = 8;            // waves that issue the K/V DMA
constexpr int BQ = 32 * NWAVE;     // queries per workgroup
constexpr int BKV = 64;            // keys per LDS tile
constexpr int NSTAGE = 4;          // tiles in the LDS ring
constexpr float LAZY_TH = 8.0f;    // exp2-domain slack of the running max

#define KX_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// A workgroup barrier that the compiler may not move memory accesses across.
#define KX_BARRIER() asm volatile("s_barrier" ::: "memory")
typedef short v4s __attribute__((ext_vector_type(4)));

// gfx9 s_waitcnt immediate that waits for vmcnt <= N only.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// K rows: 16 consecutive keys hit 16 distinct 16-byte slots (and the swizzle depends on the key
// modulo 16 only, so key block 1 is key block 0 plus 32 rows). V rows: the 4 keys x 4 chunks of a
// transposing read hit distinct slots.
template <int D> __device__ __forceinline__ int swz_k(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int D> __device__ __forceinline__ int swz_v(int r) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }

// A raw buffer resource over 4 GiB from a 64-bit base: the copies below address their source as
// this scalar base plus a 32-bit lane offset plus a 32-bit scalar offset, so a wave's copies of a
// tile need one vector register and no address arithmetic.
typedef __attribute__((ext_vector_type(4))) int i32x4;
__device__ __forceinline__ i32x4 dma_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return (i32x4){(int)(uint32_t)a, (int)(uint32_t)(a >> 32), -1, 0x00020000};
}

// One 16-byte-per-lane buffer -> LDS copy (buffer_load_dwordx4 ... lds; M0 holds the wave's LDS
// address). Written as inline assembly so that the compiler's wait-count pass does not see an LDS
// write pending on vmcnt: as a builtin, every transposing LDS read after it got a vmcnt(0) wait
// for the copies just issued (the pass cannot tell the ring's buffers apart), which stalled the
// issuing waves for a whole memory round trip per tile. The kernel orders the copies itself:
// wait_vmcnt for a tile's copies, then the workgroup barrier, before any wave reads the tile.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, const void* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)KX_LDS(lds);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
               "{m0}"(m0)
               : "memory");
}

__device__ __forceinline__ bf16x8 read_vt(const uint8_t* p, int second) {
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p + second));
  // whole-word casts: the operand is the two 8-byte results back to back
  const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
  return __builtin_bit_cast(bf16x8, make_uint4(lo2.x, lo2.y, hi2.x, hi2.y));
}

// The larger of the values a lane and lane ^ 32 hold, by one v_permlane32_swap (no LDS round
// trip). The scores are finite or -inf, so the max needs no NaN canonicalization.
__device__ __forceinline__ float half_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(__uint_as_float(sw[0])), "v"(__uint_as_float(sw[1])));
  return r;
}

// acc + the two 16-bit values of element pair j of v (v_dot2 with (1, 1)): the row sum of P taken
// from the rounded values the P V product uses.
template <bool H>
__device__ __forceinline__ float add_word(uint32_t w, float acc) {
  if constexpr (H)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, 0x3C003C00u), acc, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                           acc, false);
}
template <bool H>
__device__ __forceinline__ float add_pair(bf16x8 v, int j, float acc) {
  return add_word<H>(__builtin_bit_cast(uint4, v)[j], acc);
}

// One query row of O, scaled and rounded, to memory. The lane holds dims db * 32 + 8g + 4 lhalf +
// (0..3) of its query (g = 0..3); one v_permlane32_swap per word of a (g = 2p, 2p + 1) pair hands
// lane L dims 16p .. 16p + 7 and lane L + 32 dims 16p + 8 .. 16p + 15, so that each store writes 16
// contiguous bytes: half the store instructions and row pieces of 8-byte stores (which took
// 58.6 us against 51 for the 9216 x 256-key attention). Both lanes of a query pair must be active.
template <bool H, int DB>
__device__ __forceinline__ void store_o_row(uint16_t* orow, const f32x16 (&o)[DB], float s, int lhalf) {
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const uint32_t x0 = e_pack2<H>(o[db][8 * pp + 0] * s, o[db][8 * pp + 1] * s);
      const uint32_t x1 = e_pack2<H>(o[db][8 * pp + 2] * s, o[db][8 * pp + 3] * s);
      const uint32_t y0 = e_pack2<H>(o[db][8 * pp + 4] * s, o[db][8 * pp + 5] * s);
      const uint32_t y1 = e_pack2<H>(o[db][8 * pp + 6] * s, o[db][8 * pp + 7] * s);
      // lane L < 32 keeps x, takes lane L + 32's x as its y; lane L + 32 takes lane L's y as its x
      const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
      *reinterpret_cast<uint4*>(orow + db * 32 + 16 * pp + 8 * lhalf) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
    }
}

// Optional additive score bias (the reference's SDPA mask): bias[b * bs + h * hs + q * qs + key]
// in bf16, added as bias / scale to the raw score (so that the scaled score gains `bias`). A bias
// below -1e20 after that division (-inf, the bf16 minimum) removes the key: its score becomes the
// sentinel -1e30 exactly (the raw score is far below its ulp), whose p is 0 — or 1 when every key
// the row has seen is removed, so that a fully masked row averages V uniformly, as the
// reference's equal finite scores do. (The sentinel's p is selected, not computed: the FMA of
// the exp2 argument would leave the rounding error of -1e30 * scale, ~1e21, in the exponent.)
struct ScoreBias {
  const uint16_t* ptr;
  int64_t bs, hs, qs;
  float mul;  // 1 / scale
};

// Split over keys (few query tiles, many keys): grid row y takes keys [y * chunk, (y + 1) * chunk)
// and writes its unnormalized fp32 O rows and (running max in the exp2 domain, row sum) to the
// workspace; attn_combine_kernel merges the slices.
struct SplitOut {
  float* o;   // (splits, batch * heads, tq, D)
  float* ml;  // (splits, batch * heads, tq, 2)
  int chunk;  // keys per slice, a multiple of BKV
};

// RES (D = 128, no bias, no split, at most NSTAGE key tiles): every key tile is copied into LDS
// once and stays there while the workgroup runs up to qpw consecutive query tiles of its head; the
// waves need no barrier after the copy, so one wave's query load and output store overlap the
// other waves' products.
template <bool H, int D, bool BIAS, bool SPLIT, bool RES = false>
__global__ __launch_bounds__(NWAVE * 64) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, int64_t ldq, const uint16_t* __restrict__ K, int64_t ldk,
    const uint16_t* __restrict__ V, int64_t ldv, uint16_t* __restrict__ O, int64_t ldo, int tq,
    int tk_all, int heads, int kv_group, float scale_log2, const uint16_t* __restrict__ gate,
    int64_t ld_gate, int qtiles, int qpw, ScoreBias bias, SplitOut split) {
  static_assert(!RES || (D == 128 && !BIAS && !SPLIT), "resident keys: the pipelined form only");
  constexpr int ROWB = D * 2;             // bytes per K / V row
  constexpr int CPR = ROWB / 16;          // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;           // rows per DMA instruction
  constexpr int TILE = BKV * ROWB;        // one K (or V) tile
  constexpr int STAGE = 2 * TILE;
  constexpr int INST = 2 * BKV / RPI;     // DMA instructions per stage (K then V)
  constexpr int PER = INST / NDMA;        // per DMA wave
  static_assert(PER * NDMA == INST, "DMA split");
  const bool dma_wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < NDMA;
  constexpr int QS = D / 16, DB = D / 32;
  constexpr bool PIPE = D == 128 && !BIAS;  // the software-pipelined key loop
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTAGE * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, lhalf = lane >> 5;
  // work order: XCD-contiguous so the workgroups of one XCD share few heads' K/V in its L2
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int wph = RES ? (qtiles + qpw - 1) / qpw : qtiles;  // workgroups per (batch, head)
  const int qt = RES ? (t % wph) * qpw : t % qtiles, bh = t / wph;
  const int h = bh % heads, b = bh / heads;
  const uint16_t* Qb = Q + (int64_t)b * tq * ldq + (int64_t)h * D;
  const int hk = h / kv_group;  // grouped-query attention: kv_group query heads share a K/V head
  // this workgroup's keys: all of them, or one slice of the split form
  int j_begin = 0, tk = tk_all;
  if constexpr (SPLIT) {
    j_begin = blockIdx.y * split.chunk;
    tk = min(tk_all - j_begin, split.chunk);
  }
  const char* Kb = reinterpret_cast<const char*>(K + ((int64_t)b * tk_all + j_begin) * ldk + (int64_t)hk * D);
  const char* Vb = reinterpret_cast<const char*>(V + ((int64_t)b * tk_all + j_begin) * ldv + (int64_t)hk * D);

  int q0 = qt * BQ + wave * 32;
  int qrow = min(q0 + lrow, tq - 1);
  bf16x8 qf[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s)
    qf[s] = *reinterpret_cast<const bf16x8*>(Qb + (int64_t)qrow * ldq + (2 * s + lhalf) * 8);

  // DMA: waves [0, NDMA / 2) fill the K tile, the others the V tile; instruction i of the wave with
  // index wk among its kind fills rows RPI (wk + NK i) .. + RPI - 1, lane -> row lane / CPR, slot
  // lane % CPR, which holds chunk slot ^ swz(row). The row step between a wave's instructions is a
  // multiple of the swizzle period, so every copy of the wave takes the same lane offset; the row
  // step is a scalar offset and the tile's first key the resource's base. Keys past the end
  // re-read the last key (in bounds; masked below).
  constexpr int NK = NDMA / 2;
  static_assert(PER * NK == INST / 2 && (RPI * NK) % 16 == 0, "DMA row interleave");
  const bool wave_isv = wave >= NK;
  const int wk = wave_isv ? wave - NK : wave;
  const char* dma_base = wave_isv ? Vb : Kb;
  const uint32_t dma_ld = (uint32_t)((wave_isv ? ldv : ldk) * 2);  // bytes per key (< 2^25, checked on the host)
  const int dma_lds = (wave_isv ? TILE : 0) + RPI * wk * ROWB;  // the wave's first copy in a stage
  auto issue = [&](uint8_t* buf, int j0) {
    if (!dma_wave) return;
    // the lane offsets, recomputed from the lane id at each issue (a few VALU on the DMA waves):
    // held across the key loop they would take registers the loop needs, and a spilled copy
    // reloaded here would wait for every copy in flight
    uint32_t ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int r_in = (int)ln / CPR, slot = (int)ln % CPR;
    const int lrow_dma = RPI * wk + r_in;  // the lane's row in the wave's first copy
    const uint32_t chunk_off = (uint32_t)((slot ^ (wave_isv ? swz_v<D>(lrow_dma) : swz_k<D>(lrow_dma))) * 16);
    const uint32_t dma_voff = (uint32_t)lrow_dma * dma_ld + chunk_off;
    const i32x4 rsrc = dma_rsrc(dma_base + (int64_t)j0 * dma_ld);
    if (j0 + BKV <= tk) {
#pragma unroll
      for (int i = 0; i < PER; ++i)
        dma16(rsrc, dma_voff, (uint32_t)(RPI * NK * i) * dma_ld, buf + dma_lds + RPI * NK * i * ROWB);
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int r = min(lrow_dma + RPI * NK * i, tk - 1 - j0);  // rows past the last key re-read it
        dma16(rsrc, (uint32_t)r * dma_ld + chunk_off, 0u, buf + dma_lds + RPI * NK * i * ROWB);
      }
    }
  };

  // fragment offsets: one per K step (key block kb adds 32 rows) and one per V dim block (the key
  // step adds whole rows); the rest are immediate offsets of the LDS reads
  int koff[QS];
#pragma unroll
  for (int st = 0; st < QS; ++st) koff[st] = lrow * ROWB + (((2 * st + lhalf) ^ swz_k<D>(lrow)) << 4);
  // transposing read q of key step ts: lane group g16 = lane / 16, r16 = lane % 16 addresses key
  // 16 ts + 8 q + 4 (g16 >> 1) + (r16 >> 2), dims 32 db + 16 (g16 & 1) + 4 (r16 & 3) .. +3
  const int g16 = lane >> 4, r16 = lane & 15;
  const int vkey = 4 * (g16 >> 1) + (r16 >> 2);
  int voff[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int dim = 32 * db + 16 * (g16 & 1) + 4 * (r16 & 3);
    voff[db] = TILE + vkey * ROWB + (((dim >> 3) ^ swz_v<D>(vkey)) << 4) + ((dim >> 2) & 1) * 8;
  }

  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
  float m_run = -INFINITY;  // running max of the raw scores (the exp2 domain is m_run * scale_log2)
  float l_run = 0.0f;       // this lane's partial row sum

  const int ntiles = (tk + BKV - 1) / BKV;
  if constexpr (PIPE) {
    // Software pipeline over blocks of 32 keys (block c = key half c % 2 of tile c / 2): the MFMAs
    // of block c + 1's scores run between the exps of block c, and the P V MFMAs of block c between
    // the max of block c + 1, so the matrix core and the VALU of a wave work side by side instead
    // of in turns. Tile t becomes visible at a barrier before the scores of its first block (in
    // the middle of tile t - 1); that barrier also frees the buffer of tile t - 2 (every wave has
    // finished its P V products), which takes tile t + NSTAGE - 2. (A ring of 5 with a barrier per
    // two tiles measured 2-3 % slower.)
    auto buf = [&](int t) { return smem + (t % NSTAGE) * STAGE; };
    if constexpr (!RES) {
#pragma unroll
      for (int p = 0; p < NSTAGE - 2; ++p) issue(buf(p), min(p, ntiles - 1) * BKV);
    }
    auto arrive = [&](int t) {
      wait_vmcnt<(NSTAGE - 3) * PER>();  // tile t has landed (tile t + 1 may be in flight)
      KX_BARRIER();
      issue(buf(t + NSTAGE - 2), min(t + NSTAGE - 2, ntiles - 1) * BKV);
    };
    // At D = 128 the K swizzle (row & 15) and the V swizzle (4 (row & 3)) flip chunk-index bits
    // above the lane's own, so the offsets of steps st and dim blocks db are the first offset with
    // st << 5, db << 6 XORed in: one VALU per read instead of 12 registers held across the loop
    const int koff0 = koff[0], voff0 = voff[0];
    auto kfrag = [&](const uint8_t* tile, int kb, int st) {
      return *reinterpret_cast<const bf16x8*>(tile + (koff0 ^ (st << 5)) + kb * 32 * ROWB);
    };
    auto vfrag = [&](const uint8_t* tile, int db, int ts16) {
      return read_vt(tile + (voff0 ^ (db << 6)) + ts16 * 16 * ROWB, 8 * ROWB);
    };
    // keys past the end of block c score -inf
    auto mask = [&](f32x16& sc, int c) {
      if (32 * (c + 1) > tk) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (32 * c + 8 * (e >> 2) + 4 * lhalf + (e & 3) >= tk) sc[e] = -INFINITY;
      }
    };

    f32x16 sc;    // the current block's scores
    float mc;     // the running max in the exp2 domain
    bf16x8 kpre;  // the next step's first K fragment, read ahead where no barrier comes between
    // the read-ahead of kpre: the streaming forms (the resident form has no registers to spare)
    constexpr bool PRE = !RES;
    // block 0's scores and the running max they start
    auto first_block = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = 0.0f;
#pragma unroll
      for (int st = 0; st < QS; ++st)
        sc = mfma32x32x16<H>(kfrag(buf(0), 0, st), qf[st], sc);
      mask(sc, 0);
      float tmax = sc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
      m_run = half_max(tmax);  // finite: block 0 holds key 0
      mc = m_run * scale_log2;
      if constexpr (PRE) kpre = kfrag(buf(0), 1, 0);  // the first K fragment of block 1
    };
    if constexpr (!RES) {
      arrive(0);
      first_block();
    }

    // block c (key half kb of tile `cur`) with the scores of block cn (key half nkb of tile `nxt`)
    // use_pre: the first K fragment is kpre; pnxt (if not null): read block 1's first K fragment
    // of tile pnxt into kpre during the last P V MFMAs, for the step after this one
    auto step = [&](const uint8_t* cur, int kb, const uint8_t* nxt, int nkb, int cn, bool use_pre,
                    const uint8_t* pnxt) __attribute__((always_inline)) {
      uint32_t pw[2][4];  // P^T as packed pairs (one v_cvt_pk per pair in both types)
      float pe;           // the even element's p, until its odd partner is computed
      f32x16 sn;
#pragma unroll
      for (int e = 0; e < 16; ++e) sn[e] = 0.0f;
      // each exp is pinned where it is placed (the empty asm takes its result): otherwise the
      // compiler sinks the exps past the score MFMAs to their first use in the P V products
      auto pexp = [&](int e) {
        float p = __builtin_amdgcn_exp2f(fmaf(sc[e], scale_log2, -mc));
        asm volatile("" : "+v"(p));
        if ((e & 1) == 0) {
          pe = p;
        } else {
          pw[e >> 3][(e & 7) >> 1] = e_pack2<H>(pe, p);
          l_run = add_word<H>(pw[e >> 3][(e & 7) >> 1], l_run);
        }
      };
      // VALU work is spread so that each MFMA has about its own duration of it beside it: the
      // exps of elements 0..PA-1 between the 8 score MFMAs, the rest between the 4 P V MFMAs of
      // the first 16 keys (which need only elements 0..7), the max of block cn between the last 4
      // (8, 9, 12 or 14 here leave a query fragment spilled and reloaded in the loop, whose wait
      // on vmcnt also waits for the K/V copies in flight: 10 % slower; 10 and 11 fit)
      constexpr int PA = 10;
      // K fragments are read KFD MFMAs ahead, V fragments VFD ahead (the first ones during the last
      // score MFMAs)
      constexpr int KFD = 1, VFD = 1;
      bf16x8 kf[KFD + 1], vf[VFD + 1];
#pragma unroll
      for (int i = 0; i < KFD; ++i) kf[i] = i == 0 && use_pre ? kpre : kfrag(nxt, nkb, i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        if (st + KFD < QS) kf[(st + KFD) % (KFD + 1)] = kfrag(nxt, nkb, st + KFD);
        if (st + VFD >= QS) vf[st + VFD - QS] = vfrag(cur, (st + VFD - QS) % DB, 2 * kb + (st + VFD - QS) / DB);
        __builtin_amdgcn_sched_barrier(0);
        sn = mfma32x32x16<H>(kf[st % (KFD + 1)], qf[st], sn);
#pragma unroll
        for (int e = st * PA / QS; e < (st + 1) * PA / QS; ++e) pexp(e);
        __builtin_amdgcn_sched_barrier(0);
      }
      mask(sn, cn);
      // O^T += V^T P^T over the block's two 16-key steps
      float tmax = -INFINITY;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 2 * DB; ++q) {
        const int ts = q / DB, db = q % DB;
        if (q + VFD < 2 * DB)
          vf[(q + VFD) % (VFD + 1)] = vfrag(cur, (q + VFD) % DB, 2 * kb + (q + VFD) / DB);
        else if (pnxt)
          kpre = kfrag(pnxt, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        const bf16x8 pb = __builtin_bit_cast(bf16x8, make_uint4(pw[ts][0], pw[ts][1], pw[ts][2], pw[ts][3]));
        o[db] = mfma32x32x16<H>(vf[q % (VFD + 1)], pb, o[db]);
        if (q < DB) {
#pragma unroll
          for (int e = PA + q * (16 - PA) / DB; e < PA + (q + 1) * (16 - PA) / DB; ++e) pexp(e);
        } else {
#pragma unroll
          for (int e = (q - DB) * 16 / DB; e < (q - DB + 1) * 16 / DB; ++e) tmax = fmaxf(tmax, sn[e]);
          asm volatile("" : "+v"(tmax));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      tmax = half_max(tmax);
      if (__any(tmax * scale_log2 > mc + LAZY_TH)) {
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < DB; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
        m_run = m_new;
        mc = m_run * scale_log2;
      }
      sc = sn;
    };

    if constexpr (RES) {
      // every key tile, copied once (at most NSTAGE of them, checked on the host); then each query
      // tile runs the same block sequence without barriers
      for (int p = 0; p < ntiles; ++p) issue(buf(p), p * BKV);
      wait_vmcnt<0>();
      KX_BARRIER();
      const int nq = min(qpw, qtiles - qt);
      for (int qi = 0; qi < nq; ++qi) {
        if (qi > 0) {
          q0 += BQ;
          qrow = min(q0 + lrow, tq - 1);
#pragma unroll
          for (int st = 0; st < QS; ++st)
            qf[st] = *reinterpret_cast<const bf16x8*>(Qb + (int64_t)qrow * ldq + (2 * st + lhalf) * 8);
#pragma unroll
          for (int i = 0; i < DB; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
          l_run = 0.0f;
        }
        first_block();
        for (int t = 0; t < ntiles; ++t) {
          const uint8_t* cur = buf(t);
          step(cur, 0, cur, 1, 2 * t + 1, false, nullptr);
          const bool more = t + 1 < ntiles;
          step(cur, 1, more ? buf(t + 1) : cur, 0, more ? 2 * t + 2 : 2 * t, false, nullptr);
        }
        const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
        const int q = q0 + lrow;
        if (q < tq) {
          float scale_out = 1.0f / l_tot;
          if (gate) scale_out *= e2f<H>(gate[((int64_t)b * tq + q) * ld_gate + h]);
          store_o_row<H, DB>(O + ((int64_t)b * tq + q) * ldo + (int64_t)h * D, o, scale_out, lhalf);
        }
      }
      return;
    }
    for (int t = 0; t < ntiles; ++t) {
      const uint8_t* cur = buf(t);
      step(cur, 0, cur, 1, 2 * t + 1, PRE, nullptr);
      // the last block recomputes the scores of block 2t, already seen (its max cannot move the
      // running max); they are not used
      const bool more = t + 1 < ntiles;
      if (more) arrive(t + 1);
      // block 1's first K fragment of tile t + 1 (visible since the barrier above) is read during
      // this step's last P V MFMAs; after the last tile the read takes a buffer the loop no longer
      // uses and its value is dropped
      step(cur, 1, more ? buf(t + 1) : cur, 0, more ? 2 * t + 2 : 2 * t, false, PRE ? buf(t + 1) : nullptr);
    }
  } else {
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue(smem + p * STAGE, min(p, ntiles - 1) * BKV);
    int cur_i = 0;
    for (int it = 0; it < ntiles; ++it) {
      // tile it has landed for this wave; after the barrier for every wave, and every wave is done
      // with tile it-1, whose buffer takes tile it+3 (past the end the last tile is re-read, which
      // keeps the vmcnt arithmetic uniform)
      wait_vmcnt<(NSTAGE - 2) * PER>();
      KX_BARRIER();
      const uint8_t* cur = smem + cur_i * STAGE;
      issue(smem + (cur_i == 0 ? NSTAGE - 1 : cur_i - 1) * STAGE, min(it + NSTAGE - 1, ntiles - 1) * BKV);

      // S^T = K Q^T for two 32-key blocks
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
#pragma unroll
        for (int st = 0; st < QS; ++st) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(cur + koff[st] + kb * 32 * ROWB);
          s[kb] = mfma32x32x16<H>(kf, qf[st], s[kb]);
        }
      }
      const int j0 = it * BKV;
      if constexpr (BIAS) {
        // lane: query qrow, keys j0 + 32 kb + 8 g + 4 lhalf + (0..3) = elements 4 g .. 4 g + 3
        const uint16_t* brow =
            bias.ptr + (int64_t)b * bias.bs + (int64_t)h * bias.hs + (int64_t)qrow * bias.qs + j_begin;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int key = j0 + kb * 32 + 8 * g + 4 * lhalf;
            float bv[4];
            if (key + 3 < tk) {
              const uint2 w = *reinterpret_cast<const uint2*>(brow + key);
              bv[0] = e_lo<H>(w.x); bv[1] = e_hi<H>(w.x); bv[2] = e_lo<H>(w.y); bv[3] = e_hi<H>(w.y);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) bv[i] = key + i < tk ? e2f<H>(brow[key + i]) : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float add = bv[i] * bias.mul;
              s[kb][4 * g + i] += add < -1e20f ? -1e30f : add;
            }
          }
      }
      if (j0 + BKV > tk) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = j0 + kb * 32 + 8 * (e >> 2) + 4 * lhalf + (e & 3);
            if (key >= tk) s[kb][e] = -INFINITY;
          }
      }
      float tmax = s[0][0];
#pragma unroll
      for (int e = 1; e < 16; ++e) tmax = fmaxf(tmax, s[0][e]);
#pragma unroll
      for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[1][e]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      if (__any(tmax * scale_log2 > m_run * scale_log2 + LAZY_TH || m_run == -INFINITY)) {
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < DB; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
        m_run = m_new;
      }

      // P^T in bf16 as the B operand: elements 8hf .. 8hf+7 of block kb
      const float mc = m_run * scale_log2;
      const float removed_p = m_run == -1e30f ? 1.0f : 0.0f;  // p of a removed key (bias variant)
      bf16x8 pb[2][2];
      auto pexp = [&](int kb, int hf, int e) {
        float p = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * hf + e], scale_log2, -mc));
        if constexpr (BIAS) p = s[kb][8 * hf + e] == -1e30f ? removed_p : p;
        pb[kb][hf][e] = e16<H>(p);
      };
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int e = 0; e < 8; ++e) pexp(kb, hf, e);
      // the row sum of the rounded P, as in the pipelined form
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int j = 0; j < 4; ++j) l_run = add_pair<H>(pb[kb][hf], j, l_run);
      // O^T += V^T P^T, 16 keys per step; step ts = 2 kb + hf uses P^T block pb[kb][hf]
#pragma unroll
      for (int ts = 0; ts < 4; ++ts)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 vf = read_vt(cur + voff[db] + 16 * ts * ROWB, 8 * ROWB);
          o[db] = mfma32x32x16<H>(vf, pb[ts >> 1][ts & 1], o[db]);
        }
      cur_i = cur_i + 1 == NSTAGE ? 0 : cur_i + 1;
    }
  }
  wait_vmcnt<0>();  // the re-read tiles past the end have landed before the workgroup ends

  // normalise, gate, store: lane holds query q0 + lrow, dims db*32 + 8g + 4*lhalf + (0..3)
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const int q = q0 + lrow;
  if (q >= tq) return;
  if constexpr (SPLIT) {
    const int64_t row = ((int64_t)blockIdx.y * (gridDim.x / qtiles) + bh) * tq + q;
    float* orow = split.o + row * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(orow + db * 32 + 8 * g + 4 * lhalf) =
            make_float4(o[db][4 * g + 0], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]);
    if (lhalf == 0) *reinterpret_cast<float2*>(split.ml + 2 * row) = make_float2(m_run * scale_log2, l_tot);
    return;
  }
  float scale_out = 1.0f / l_tot;
  if (gate) scale_out *= e2f<H>(gate[((int64_t)b * tq + q) * ld_gate + h]);
  store_o_row<H, DB>(O + ((int64_t)b * tq + q) * ldo + (int64_t)h * D, o, scale_out, lhalf);
}

// out = (sum_y 2^(m_y - M) O_y) / (sum_y 2^(m_y - M) l_y) * gate, M = max_y m_y: the slices of the
// split form merged (4 dims of one row per thread).
template <bool H, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part_o,
                                                           const float* __restrict__ part_ml, int splits,
                                                           int64_t rows, int tq, int heads,
                                                           uint16_t* __restrict__ O, int64_t ldo,
                                                           const uint16_t* __restrict__ gate, int64_t ld_gate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * (D / 4)) return;
  const int64_t row = idx / (D / 4);  // (b * heads + h) * tq + q
  const int d = (int)(idx - row * (D / 4)) * 4;
  float mx = -INFINITY;
  for (int y = 0; y < splits; ++y) mx = fmaxf(mx, part_ml[2 * (y * rows + row)]);
  float l = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int y = 0; y < splits; ++y) {
    const float2 ml = *reinterpret_cast<const float2*>(part_ml + 2 * (y * rows + row));
    const float w = __builtin_amdgcn_exp2f(ml.x - mx);
    const float4 p = *reinterpret_cast<const float4*>(part_o + (y * rows + row) * D + d);
    l += w * ml.y;
    acc.x += w * p.x;
    acc.y += w * p.y;
    acc.z += w * p.z;
    acc.w += w * p.w;
  }
  const int q = (int)(row % tq);
  const int64_t bh = row / tq;
  const int h = (int)(bh % heads), b = (int)(bh / heads);
  float scale_out = 1.0f / l;
  if (gate) scale_out *= e2f<H>(gate[((int64_t)b * tq + q) * ld_gate + h]);
  uint2 w2;
  w2.x = e_pack2<H>(acc.x * scale_out, acc.y * scale_out);
  w2.y = e_pack2<H>(acc.z * scale_out, acc.w * scale_out);
  *reinterpret_cast<uint2*>(O + ((int64_t)b * tq + q) * ldo + (int64_t)h * D + d) = w2;
}

template <bool H, int D, bool BIAS, bool SPLIT, bool RES = false>
void launch_attn_t(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, void* o,
                   int64_t ldo, int64_t tq, int64_t tk, int64_t heads, int64_t kv_heads, float scale,
                   const void* gate, int64_t ld_gate, ScoreBias bias, SplitOut split, dim3 grid, int qtiles,
                   hipStream_t s, int qpw = 1) {
  attn_fwd_kernel<H, D, BIAS, SPLIT, RES><<<grid, NWAVE * 64, 0, s>>>(
      (const uint16_t*)q, ldq, (const uint16_t*)k, ldk, (const uint16_t*)v, ldv, (uint16_t*)o, ldo, (int)tq,
      (int)tk, (int)heads, (int)(heads / kv_heads), scale * 1.4426950408889634f, (const uint16_t*)gate, ld_gate,
      qtiles, qpw, bias, split);
}

// Query tiles per workgroup for the resident-key form: the fewest workgroup rounds on the 256 CUs
// times the tiles each workgroup runs, ties to more tiles per workgroup (each keeps its keys).
int resident_qpw(int64_t qtiles, int64_t heads_total) {
  constexpr int64_t kCUs = 256;
  int best = 1;
  int64_t best_cost = -1;
  for (int qpw = 1; qpw <= 8 && qpw <= qtiles; ++qpw) {
    const int64_t groups = heads_total * ((qtiles + qpw - 1) / qpw);
    const int64_t cost = (groups + kCUs - 1) / kCUs * qpw;
    if (best_cost < 0 || cost <= best_cost) {
      best = qpw;
      best_cost = cost;
    }
  }
  return best;
}

template <bool H, int D>
int launch_attn(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                void* o, int64_t ldo, int64_t batch, int64_t tq, int64_t tk, int64_t heads,
                int64_t kv_heads, float scale, const void* gate, int64_t ld_gate, ScoreBias bias,
                SplitOut split, int splits, hipStream_t s) {
  const int qtiles = (int)((tq + BQ - 1) / BQ);
  const int64_t blocks = (int64_t)qtiles * heads * batch;
  const dim3 grid((unsigned)blocks, (unsigned)splits);
  if (splits > 1) {
    if (bias.ptr)
      launch_attn_t<H, D, true, true>(q, ldq, k, ldk, v, ldv, o, ldo, tq, tk, heads, kv_heads, scale, gate, ld_gate,
                                   bias, split, grid, qtiles, s);
    else
      launch_attn_t<H, D, false, true>(q, ldq, k, ldk, v, ldv, o, ldo, tq, tk, heads, kv_heads, scale, gate, ld_gate,
                                    bias, split, grid, qtiles, s);
    const int64_t rows = batch * heads * tq;
    attn_combine_kernel<H, D><<<(unsigned)((rows * (D / 4) + 255) / 256), 256, 0, s>>>(
        split.o, split.ml, splits, rows, (int)tq, (int)heads, (uint16_t*)o, ldo, (const uint16_t*)gate, ld_gate);
  } else if (bias.ptr) {
    launch_attn_t<H, D, true, false>(q, ldq, k, ldk, v, ldv, o, ldo, tq, tk, heads, kv_heads, scale, gate, ld_gate,
                                  bias, split, grid, qtiles, s);
  } else if (D == 128 && tk <= NSTAGE * BKV) {
    // few keys (a text context): they stay in LDS while a workgroup runs several query tiles
    const int qpw = resident_qpw(qtiles, heads * batch);
    const dim3 rgrid((unsigned)((qtiles + qpw - 1) / qpw * heads * batch));
    launch_attn_t<H, D, false, false, D == 128>(q, ldq, k, ldk, v, ldv, o, ldo, tq, tk, heads, kv_heads, scale, gate,
                                             ld_gate, bias, split, rgrid, qtiles, s, qpw);
  } else {
    launch_attn_t<H, D, false, false>(q, ldq, k, ldk, v, ldv, o, ldo, tq, tk, heads, kv_heads, scale, gate, ld_gate,
                                   bias, split, grid, qtiles, s);
  }
  return check_launch(ename<H>("kx_attention_fwd_bf16", "kx_attention_fwd_f16"));
}

}  // namespace
}  // namespace kx

using namespace kx;

namespace {
template <bool H>
int attention_entry(const char* name, const void* q, int64_t ldq, const void* k, int64_t ldk,
                    const void* v, int64_t ldv, void* o, int64_t ldo, int64_t batch, int64_t tq,
                    int64_t tk, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale,
                    const void* gate, int64_t ld_gate, kx_stream_t stream,
                    ScoreBias bias = ScoreBias{nullptr, 0, 0, 0, 0.0f},
                    SplitOut split = SplitOut{nullptr, nullptr, 0}, int splits = 1) {
  KX_REQUIRE(q && k && v && o, "%s: null tensor", name);
  KX_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim must be 64 or 128, got %lld", name,
             (long long)head_dim);
  KX_REQUIRE(batch >= 0 && tq >= 0 && tk > 0 && heads > 0 && tq < (1ll << 30) &&
                 tk < (1ll << 30),
             "%s: bad shape", name);
  KX_REQUIRE(kv_heads > 0 && heads % kv_heads == 0,
             "%s: %lld query heads do not group over %lld key/value heads", name, (long long)heads,
             (long long)kv_heads);
  const int64_t width = heads * head_dim, kv_width = kv_heads * head_dim;
  KX_REQUIRE(ldq >= width && ldk >= kv_width && ldv >= kv_width && ldo >= width,
             "%s: row strides must cover heads * head_dim", name);
  KX_REQUIRE(ldk < (1ll << 24) && ldv < (1ll << 24), "%s: key/value row strides must be below 2^24", name);
  KX_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 4 == 0 && aligned16(q) &&
                 aligned16(k) && aligned16(v) && aligned8(o),
             "%s: q/k/v rows must be 16-byte and o rows 8-byte aligned", name);
  KX_REQUIRE(!gate || ld_gate >= heads, "%s: gate stride must cover heads", name);
  KX_REQUIRE((int64_t)((tq + BQ - 1) / BQ) * heads * batch < (1ll << 31), "%s: too many tiles",
             name);
  if (tq == 0 || batch == 0) return KX_OK;
  if (head_dim == 128)
    return launch_attn<H, 128>(q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk, heads, kv_heads, scale,
                            gate, ld_gate, bias, split, splits, (hipStream_t)stream);
  return launch_attn<H, 64>(q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk, heads, kv_heads, scale,
                         gate, ld_gate, bias, split, splits, (hipStream_t)stream);
}
}  // namespace

#define KX_ATTN_ENTRY(SUFFIX, H)                                                                                \
extern "C" int kx_attention_gqa_fwd_##SUFFIX(const void* q, int64_t ldq, const void* k, int64_t ldk,                   \
                                         const void* v, int64_t ldv, void* o, int64_t ldo,                             \
                                         int64_t batch, int64_t tq, int64_t tk, int64_t heads,                         \
                                         int64_t kv_heads, int64_t head_dim, float scale,                              \
                                         const void* gate, int64_t ld_gate, kx_stream_t stream) {                      \
  return attention_entry<H>("kx_attention_gqa_fwd_" #SUFFIX, q, ldq, k, ldk, v, ldv, o, ldo, batch, tq,                \
                         tk, heads, kv_heads, head_dim, scale, gate, ld_gate, stream);                                 \
}                                                                                                                      \
                                                                                                                       \
extern "C" int kx_attention_fwd_##SUFFIX(const void* q, int64_t ldq, const void* k, int64_t ldk,                       \
                                     const void* v, int64_t ldv, void* o, int64_t ldo,                                 \
                                     int64_t batch, int64_t tq, int64_t tk, int64_t heads,                             \
                                     int64_t head_dim, float scale, const void* gate,                                  \
                                     int64_t ld_gate, kx_stream_t stream) {                                            \
  return attention_entry<H>("kx_attention_fwd_" #SUFFIX, q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk,                \
                         heads, heads, head_dim, scale, gate, ld_gate, stream);                                        \
}                                                                                                                      \
                                                                                                                       \
extern "C" int kx_attention_bias_fwd_##SUFFIX(const void* q, int64_t ldq, const void* k, int64_t ldk,                  \
                                          const void* v, int64_t ldv, void* o, int64_t ldo,                            \
                                          int64_t batch, int64_t tq, int64_t tk, int64_t heads,                        \
                                          int64_t kv_heads, int64_t head_dim, float scale,                             \
                                          const void* gate, int64_t ld_gate, const void* bias,                         \
                                          int64_t bias_bs, int64_t bias_hs, int64_t bias_qs,                           \
                                          kx_stream_t stream) {                                                        \
  KX_REQUIRE(bias, "kx_attention_bias_fwd_" #SUFFIX ": null bias");                                                    \
  KX_REQUIRE(aligned8(bias) && bias_bs >= 0 && bias_hs >= 0 && bias_qs >= 0 && bias_bs % 4 == 0 &&                     \
                 bias_hs % 4 == 0 && bias_qs % 4 == 0,                                                                 \
             "kx_attention_bias_fwd_" #SUFFIX ": bias must be 8-byte aligned with non-negative strides that "          \
             "are multiples of 4 elements");                                                                           \
  KX_REQUIRE(scale > 0.0f && isfinite(scale), "kx_attention_bias_fwd_" #SUFFIX ": scale must be positive");            \
  return attention_entry<H>("kx_attention_bias_fwd_" #SUFFIX, q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk,           \
                         heads, kv_heads, head_dim, scale, gate, ld_gate, stream,                                      \
                         ScoreBias{(const uint16_t*)bias, bias_bs, bias_hs, bias_qs, 1.0f / scale});                   \
}                                                                                                                      \
                                                                                                                       \
extern "C" int kx_attention_split_fwd_##SUFFIX(const void* q, int64_t ldq, const void* k, int64_t ldk,                 \
                                           const void* v, int64_t ldv, void* o, int64_t ldo, int64_t batch,            \
                                           int64_t tq, int64_t tk, int64_t heads, int64_t kv_heads,                    \
                                           int64_t head_dim, float scale, const void* gate, int64_t ld_gate,           \
                                           const void* bias, int64_t bias_bs, int64_t bias_hs, int64_t bias_qs,        \
                                           void* workspace, int64_t workspace_bytes, int splits,                       \
                                           kx_stream_t stream) {                                                       \
  const char* name = "kx_attention_split_fwd_" #SUFFIX;                                                                \
  KX_REQUIRE(workspace && aligned16(workspace), "%s: workspace must be a 16-byte aligned buffer", name);               \
  KX_REQUIRE(splits >= 2 && splits <= 256 && tk > 0, "%s: splits must be 2..256, got %d", name, splits);               \
  KX_REQUIRE(ldo % 4 == 0 && aligned8(o), "%s: output rows must be 8-byte aligned", name);                             \
  /* keys per slice: a whole number of 64-key tiles; the slices actually used cover tk exactly */                      \
  const int64_t chunk = ((tk + splits - 1) / splits + BKV - 1) / BKV * BKV;                                            \
  const int used = (int)((tk + chunk - 1) / chunk);                                                                    \
  const int64_t rows = batch * heads * tq;                                                                             \
  KX_REQUIRE(workspace_bytes >= (int64_t)used * rows * (head_dim + 2) * 4,                                             \
             "%s: workspace of %lld bytes is below splits * batch * heads * tq * (head_dim + 2) * 4", name,            \
             (long long)workspace_bytes);                                                                              \
  ScoreBias sb{nullptr, 0, 0, 0, 0.0f};                                                                                \
  if (bias) {                                                                                                          \
    KX_REQUIRE(aligned8(bias) && bias_bs >= 0 && bias_hs >= 0 && bias_qs >= 0 && bias_bs % 4 == 0 &&                   \
                   bias_hs % 4 == 0 && bias_qs % 4 == 0,                                                               \
               "%s: bias must be 8-byte aligned with non-negative strides that are multiples of 4", name);             \
    KX_REQUIRE(scale > 0.0f && isfinite(scale), "%s: scale must be positive", name);                                   \
    sb = ScoreBias{(const uint16_t*)bias, bias_bs, bias_hs, bias_qs, 1.0f / scale};                                    \
  }                                                                                                                    \
  float* ws = static_cast<float*>(workspace);                                                                          \
  const SplitOut split{ws, ws + (int64_t)used * rows * head_dim, (int)chunk};                                          \
  return attention_entry<H>(name, q, ldq, k, ldk, v, ldv, o, ldo, batch, tq, tk, heads, kv_heads, head_dim, scale,     \
                         gate, ld_gate, stream, sb, split, used);                                                      \
}                                                                                                                      \

KX_ATTN_ENTRY(bf16, false)
KX_ATTN_ENTRY(f16, true)
