// Non-causal flash attention forward for gfx950 (bf16 MFMA, fp32 softmax).
//
// Replaces the reference's splash kernel: kernels/splash.py:566-650
// (`attention`), its body _flash_attention_kernel :115-375 (online update
// :250-267, kv_len masking :216-218/:277-331, normalize :369-375) and the
// residual form :665-742.
//
// Two kernels:
//   * flash_fwd_d128_kernel (D = 128, every DiT workload): direct-to-LDS
//     tiles, transposing LDS reads, pipelined softmax with lazy rescaling;
//     described at its definition below.
//   * flash_fwd_kernel (generic, used for D = 64), described here:
//
// Generic kernel work decomposition
//   * One workgroup = NW wavefronts = one (batch, head, BQ-row query block);
//     each wavefront owns QB*32 query rows for the whole key sweep.
//   * Keys/values stream through LDS in BKV=64-row tiles, double buffered:
//     while tile j is consumed from LDS, tile j+1 is already in flight in
//     registers (global -> VGPR), and is written to the other LDS buffer
//     after the tile's math; one barrier per tile.
//   * Scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_bf16: A = K tile rows from LDS (16-byte reads),
//     B = Q^T straight from registers (Q is loaded once).  In the 32x32
//     accumulator layout lane l holds column l%32, i.e. ONE query row, and
//     32 of the tile's 64 keys; the other 32 keys of that row sit in lane
//     l^32.  Row statistics therefore need one cross-lane step (max), and
//     the row sum is kept per lane and folded once at the end.
//   * The output is accumulated transposed too, O^T = V^T P^T: the score
//     accumulator, converted to bf16, IS the B operand of the PV product
//     (same lane -> query-row mapping), so probabilities never leave
//     registers.  The A operand needs V^T: V is transposed while it is
//     staged into LDS (4 keys x 8 channels per thread, permuted in
//     registers, written as 8-byte runs), with the key order inside each
//     16-key group permuted to match the accumulator's key order so that
//     each lane's 8 keys are one 16-byte LDS read.
//   * Softmax runs in the exp2 domain: one FMA applies scale*log2(e) and
//     subtracts the running max, v_exp_f32 does the rest.
//   * Grid: 1-D, remapped so that consecutive query blocks of one head land
//     on the same XCD (workgroups are dealt round-robin to the 8 XCDs), so
//     the K/V tiles they sweep in step are shared in that XCD's L2.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "dt_common.h"

namespace dt {

constexpr float kLog2e = 1.4426950408889634f;

struct FlashParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* o32;
  float* m;
  float* l;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Skv;
  int kv_end;      // keys [0, kv_end) take part
  int n_qblk;      // query blocks per (b, h)
  int n_wg;        // workgroups in the grid
  float c;         // scale * log2(e)
};

template <int D, int NW, int QB>
struct FlashCfg {
  static constexpr int BKV = 64;
  static constexpr int BQ = NW * QB * 32;
  static constexpr int NT = NW * 64;
  static constexpr int KSTEPS = D / 16;   // QK^T contraction steps
  static constexpr int DBLK = D / 32;     // 32-channel blocks of O^T
  static constexpr int KSTR = D + 8;      // K tile row stride (bf16), padded
  static constexpr int VSTR = BKV + 8;    // V^T tile row stride (bf16), padded
  static constexpr int KTILE = BKV * KSTR;
  static constexpr int VTILE = D * VSTR;
  // global->LDS staging work items per tile
  static constexpr int K_ITEMS = BKV * D / 8;        // 16-byte pieces
  static constexpr int V_ITEMS = (BKV / 4) * (D / 8);  // 4 keys x 8 channels
  static constexpr int K_PER = (K_ITEMS + NT - 1) / NT;
  static constexpr int V_PER = (V_ITEMS + NT - 1) / NT;
  static constexpr int LDS_BYTES = 2 * (KTILE + VTILE) * 2;
};

// Position of key `kv` (0..63 within a tile) in the permuted V^T row: within
// each 16-key group the order is [0-3, 8-11, 4-7, 12-15], which is the order
// in which a lane half (l/32 = 0 or 1) holds keys in the score accumulator.
__device__ __forceinline__ int vperm(int kv) {
  const int g = kv & ~15, r = kv & 15;
  const int quad = r >> 2;  // 0..3
  const int nq = (quad == 1) ? 2 : (quad == 2) ? 1 : quad;
  return g + nq * 4 + (r & 3);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  // v_cvt_pk_bf16_f32 (round to nearest even)
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 r = {(__bf16)a, (__bf16)b};
  return *reinterpret_cast<uint32_t*>(&r);
}

template <int D, int NW, int QB>
__global__ __launch_bounds__(NW * 64) void flash_fwd_kernel(FlashParams p) {
  using C = FlashCfg<D, NW, QB>;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* ktile = lds;                      // [2][BKV][KSTR]
  uint16_t* vtile = lds + 2 * C::KTILE;       // [2][D][VSTR]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  // --- XCD-aware workgroup remap: XCD x (= blockIdx % 8) gets a contiguous
  // range of logical workgroups.
  int wg;
  {
    const int bid = blockIdx.x, n = p.n_wg;
    const int xcd = bid & 7, idx = bid >> 3;
    const int per = n >> 3, rem = n & 7;
    wg = (xcd < rem) ? xcd * (per + 1) + idx
                     : rem * (per + 1) + (xcd - rem) * per + idx;
  }
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);

  const uint16_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const int q0 = qblk * C::BQ + wave * (QB * 32);

  // --- Q^T operand, resident in registers: lane holds row q0+qb*32+l32,
  // channels [16t + 8hf, +8) for each contraction step t.
  bf16x8 qf[QB][C::KSTEPS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = q0 + qb * 32 + l32;
#pragma unroll
    for (int t = 0; t < C::KSTEPS; ++t) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row < p.Sq)
        raw = *(const u32x4*)(qbase + (int64_t)row * p.q_ss + 16 * t + 8 * hf);
      qf[qb][t] = *reinterpret_cast<bf16x8*>(&raw);
    }
  }

  // --- staging registers for the next K/V tile
  u32x4 kreg[C::K_PER];
  u32x4 vreg[C::V_PER][4];

  auto load_tile = [&](int j) {
    const int kv0 = j * C::BKV;
#pragma unroll
    for (int i = 0; i < C::K_PER; ++i) {
      const int it = tid + i * C::NT;
      const int row = it / (D / 8), piece = it % (D / 8);
      const int kv = kv0 + row;
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (it < C::K_ITEMS && kv < p.kv_end)
        raw = *(const u32x4*)(kbase + (int64_t)kv * p.k_ss + piece * 8);
      kreg[i] = raw;
    }
#pragma unroll
    for (int i = 0; i < C::V_PER; ++i) {
      const int it = tid + i * C::NT;
      const int kg = it / (D / 8), dg = it % (D / 8);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kv = kv0 + kg * 4 + r;
        u32x4 raw = {0u, 0u, 0u, 0u};
        if (it < C::V_ITEMS && kv < p.kv_end)
          raw = *(const u32x4*)(vbase + (int64_t)kv * p.v_ss + dg * 8);
        vreg[i][r] = raw;
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint16_t* kt = ktile + buf * C::KTILE;
    uint16_t* vt = vtile + buf * C::VTILE;
#pragma unroll
    for (int i = 0; i < C::K_PER; ++i) {
      const int it = tid + i * C::NT;
      if (it < C::K_ITEMS) {
        const int row = it / (D / 8), piece = it % (D / 8);
        *(u32x4*)(kt + row * C::KSTR + piece * 8) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < C::V_PER; ++i) {
      const int it = tid + i * C::NT;
      if (it < C::V_ITEMS) {
        const int kg = it / (D / 8), dg = it % (D / 8);
        const int col = vperm(kg * 4);
        // vreg[i][r] holds channels dg*8 .. +8 of key kg*4+r (2 per word).
        // Channel e of the 8 is half (e&1) of word e>>1.
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t a0 = vreg[i][0][w], a1 = vreg[i][1][w];
          const uint32_t a2 = vreg[i][2][w], a3 = vreg[i][3][w];
          // even channel 2w: low halves; odd channel 2w+1: high halves
          u32x2 ev, od;
          ev[0] = (a0 & 0xffffu) | (a1 << 16);
          ev[1] = (a2 & 0xffffu) | (a3 << 16);
          od[0] = (a0 >> 16) | (a1 & 0xffff0000u);
          od[1] = (a2 >> 16) | (a3 & 0xffff0000u);
          *(u32x2*)(vt + (dg * 8 + 2 * w) * C::VSTR + col) = ev;
          *(u32x2*)(vt + (dg * 8 + 2 * w + 1) * C::VSTR + col) = od;
        }
      }
    }
  };

  // --- accumulators
  f32x16 oacc[QB][C::DBLK];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int mb = 0; mb < C::DBLK; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][mb][r] = 0.f;
  float mrow[QB], lrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    mrow[qb] = -INFINITY;
    lrow[qb] = 0.f;
  }

  const int ntiles = (p.kv_end + C::BKV - 1) / C::BKV;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    if (j + 1 < ntiles) load_tile(j + 1);
    const uint16_t* kt = ktile + buf * C::KTILE;
    const uint16_t* vt = vtile + buf * C::VTILE;

    // ---- S^T = K Q^T : two 32-key blocks
    f32x16 sacc[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[qb][kb][r] = 0.f;
#pragma unroll
    for (int t = 0; t < C::KSTEPS; ++t) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 raw =
            *(const u32x4*)(kt + (kb * 32 + l32) * C::KSTR + 16 * t + 8 * hf);
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&raw);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sacc[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              kf, qf[qb][t], sacc[qb][kb], 0, 0, 0);
      }
    }

    // ---- mask keys at or past kv_end (only the last tile can hold them)
    const int kv0 = j * C::BKV;
    if (kv0 + C::BKV > p.kv_end) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kv0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (kv >= p.kv_end)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sacc[qb][kb][r] = -INFINITY;
        }
    }

    // ---- online softmax (exp2 domain), P^T in bf16
    uint32_t pw[QB][16];  // packed bf16 pairs: 4 k-steps x 4 words
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mx = sacc[qb][0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[qb][kb][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrow[qb], mx * p.c);
      const float alpha = __builtin_amdgcn_exp2f(mrow[qb] - mnew);
      mrow[qb] = mnew;
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float e0 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][kb][r], p.c, -mnew));
          const float e1 = __builtin_amdgcn_exp2f(
              __builtin_fmaf(sacc[qb][kb][r + 1], p.c, -mnew));
          sum += e0 + e1;
          pw[qb][kb * 8 + (r >> 1)] = pack_bf16x2(e0, e1);
        }
      lrow[qb] = lrow[qb] * alpha + sum;
#pragma unroll
      for (int mb = 0; mb < C::DBLK; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[qb][mb][r] *= alpha;
    }

    // ---- O^T += V^T P^T : 4 contraction steps of 16 keys
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int mb = 0; mb < C::DBLK; ++mb) {
        const u32x4 raw = *(const u32x4*)(vt + (mb * 32 + l32) * C::VSTR +
                                          16 * u + 8 * hf);
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&raw);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          u32x4 pr;
          pr[0] = pw[qb][u * 4 + 0];
          pr[1] = pw[qb][u * 4 + 1];
          pr[2] = pw[qb][u * 4 + 2];
          pr[3] = pw[qb][u * 4 + 3];
          const bf16x8 pf = *reinterpret_cast<const bf16x8*>(&pr);
          oacc[qb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              vf, pf, oacc[qb][mb], 0, 0, 0);
        }
      }
    }

    if (j + 1 < ntiles) {
      store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float ltot = lrow[qb] + __shfl_xor(lrow[qb], 32, 64);
    const int row = q0 + qb * 32 + l32;
    if (row >= p.Sq) continue;
    const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
    if (p.o32 != nullptr) {
      float* dst = p.o32 + bhrow * D;
#pragma unroll
      for (int mb = 0; mb < C::DBLK; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = oacc[qb][mb][g * 4 + e];
          *(f32x4*)(dst + mb * 32 + 8 * g + 4 * hf) = w;
        }
      if (hf == 0) {
        p.m[bhrow] = mrow[qb];
        p.l[bhrow] = ltot;
      }
    }
    if (p.o != nullptr) {
      const float inv = 1.0f / ltot;
      uint16_t* dst = p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
      for (int mb = 0; mb < C::DBLK; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 w;
          w[0] = pack_bf16x2(oacc[qb][mb][g * 4 + 0] * inv,
                             oacc[qb][mb][g * 4 + 1] * inv);
          w[1] = pack_bf16x2(oacc[qb][mb][g * 4 + 2] * inv,
                             oacc[qb][mb][g * 4 + 3] * inv);
          *(u32x2*)(dst + mb * 32 + 8 * g + 4 * hf) = w;
        }
    }
  }
}


// ===========================================================================
// D = 128 kernel: NW wavefronts x QB*32 query rows, software-pipelined.
//
//   * K/V tiles (64 keys) move global -> LDS with global_load_lds_dwordx4
//     (no VGPR staging) into a ring of NSTAGE (K, V) stages; a tile is
//     requested NSTAGE-2 iterations before it is consumed.  Rows are stored
//     unpadded (256 B) with 16-byte chunks XOR-swizzled per row so that the
//     operand reads below are bank-conflict free:
//       K chunk c of key r lives at chunk c ^ (r & 15)
//       V chunk c of key r lives at chunk c ^ (4 * (r & 3))
//   * K operand (A of S^T = K Q^T): one ds_read_b128 per 32x16 block.
//   * V^T operand (A of O^T = V^T P^T): ds_read_b64_tr_b16 reads V row-major
//     and transposes in flight: in each 16-lane group, source lane j names
//     4 channels of one key (key = kbase + j/4, channels dbase + 4*(j%4) ..
//     +3) and lane i receives channel dbase + i of keys kbase .. kbase+3.
//     Two such reads give the 8 keys a lane half holds in the score
//     accumulator (keys 16u + 4h + 0..3 and 16u + 8 + 4h + 0..3).
//   * Per iteration j a wavefront runs
//       phase A: S(j+1) = K(j+1) Q^T   interleaved with  softmax(j)
//       phase B: O += V(j)^T P(j)^T
//     and with two wavefronts per SIMD the hardware overlaps one wave's
//     phase B with the other's phase A.
//   * Lazy rescaling: probabilities are exp2(s*c - m) against the row's
//     current reference m; m only moves (with the O/l rescale) when a tile's
//     per-lane exp sum exceeds 2^12 or is not finite (first tile, a large new
//     maximum).  The result is the exact softmax; the common path has no row
//     max and no O rescale.
// ===========================================================================

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr float kTripSum = 4096.0f;

template <int NW, int QB, int NSTAGE>
struct Cfg128 {
  static constexpr int D = 128, BKV = 64, BQ = NW * QB * 32, NT = NW * 64;
  static constexpr int TILEB = BKV * D * 2;     // 16 KiB per K or V tile
  static constexpr int STAGEB = 2 * TILEB;
  static constexpr int LDSB = NSTAGE * STAGEB;
  static constexpr int ROWS_PER_WAVE = BKV / NW;  // tile rows each wave loads
  static constexpr int LOADS = ROWS_PER_WAVE / 4; // 1 KiB instructions / tensor
};

// exp2(s*c - m) for the 32 scores of one query block, packed to bf16 pairs;
// returns the per-lane sum.
__device__ __forceinline__ float softmax_exp(const f32x16 (&s)[2], float c,
                                             float m, uint32_t (&pw)[16]) {
  float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], c, -m));
      const float e1 =
          __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r + 1], c, -m));
      sum0 += e0;
      sum1 += e1;
      pw[kb * 8 + (r >> 1)] = pack_bf16x2(e0, e1);
    }
  return sum0 + sum1;
}

// Masks keys at or past kv_end (scores -> -inf) in one query block.
__device__ __forceinline__ void mask_scores(f32x16 (&s)[2], int kv0, int hf,
                                            int kv_end) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kv = kv0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (kv >= kv_end) s[kb][r] = -INFINITY;
    }
}

// Rare path: move the reference max of one query block to the true running
// max, recompute its probabilities and rescale l and the output accumulator.
__device__ __forceinline__ void softmax_fixup(const f32x16 (&s)[2], float c,
                                              float& m, float& l, float& sum,
                                              uint32_t (&pw)[16],
                                              f32x16 (&o)[4]) {
  float mx = s[0][0];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mnew = fmaxf(m, mx * c);
  const float alpha = __builtin_amdgcn_exp2f(m - mnew);
  m = mnew;
  sum = softmax_exp(s, c, mnew, pw);
  l = l * alpha;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] *= alpha;
}

__device__ __forceinline__ bool wave_any(bool x) {
  return __builtin_amdgcn_ballot_w64(x) != 0;
}

template <int NW, int QB, int NSTAGE>
__global__ __launch_bounds__(NW * 64) void flash_fwd_d128_kernel(FlashParams p) {
  using C = Cfg128<NW, QB, NSTAGE>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[];
  lds_u8* lds = (lds_u8*)lds_raw;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  int wg;
  {
    const int bid = blockIdx.x, n = p.n_wg;
    const int xcd = bid & 7, idx = bid >> 3;
    const int per = n >> 3, rem = n & 7;
    wg = (xcd < rem) ? xcd * (per + 1) + idx
                     : rem * (per + 1) + (xcd - rem) * per + idx;
  }
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);

  const uint16_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const int q0 = qblk * C::BQ + wave * (QB * 32);
  const float c = p.c;
  const int kv_end = p.kv_end;
  const int ntiles = (kv_end + C::BKV - 1) / C::BKV;

  // ---- Q^T operands (registers for the whole sweep)
  bf16x8 qf[QB][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = q0 + qb * 32 + l32;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row < p.Sq)
        raw = *(const u32x4*)(qbase + (int64_t)row * p.q_ss + 16 * t + 8 * hf);
      qf[qb][t] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  // ---- global -> LDS tile loads.  Wave w fills rows
  // [w*RPW, (w+1)*RPW) of the K and V tiles, 4 rows (1 KiB) per instruction.
  const int lrow = lane >> 4;         // row within the instruction's 4 rows
  const int pch = lane & 15;          // physical chunk written by this lane
  int kofs[C::LOADS], vofs[C::LOADS]; // element offsets within the tile
#pragma unroll
  for (int i = 0; i < C::LOADS; ++i) {
    const int row = wave * C::ROWS_PER_WAVE + i * 4 + lrow;
    kofs[i] = row * (int)p.k_ss + ((pch ^ (row & 15)) * 8);
    vofs[i] = row * (int)p.v_ss + ((pch ^ (4 * (row & 3))) * 8);
  }
  auto issue_tile = [&](int t) {
    const int kv0 = t * C::BKV;
    lds_u8* st = lds + (t % NSTAGE) * C::STAGEB;
    const uint16_t* kt = kbase + (int64_t)kv0 * p.k_ss;
    const uint16_t* vt = vbase + (int64_t)kv0 * p.v_ss;
    const bool tail = kv0 + C::BKV > kv_end;
#pragma unroll
    for (int i = 0; i < C::LOADS; ++i) {
      int ko = kofs[i], vo = vofs[i];
      if (tail) {
        // rows past kv_end re-read the last valid row (their scores are
        // masked; the data only has to be finite and in bounds)
        const int row = wave * C::ROWS_PER_WAVE + i * 4 + lrow;
        const int over = kv0 + row - (kv_end - 1);
        if (over > 0) {
          ko -= over * (int)p.k_ss;
          vo -= over * (int)p.v_ss;
        }
      }
      lds_u8* dk = st + (wave * C::ROWS_PER_WAVE + i * 4) * 256;
      __builtin_amdgcn_global_load_lds(
          (const void*)(kt + ko), (__attribute__((address_space(3))) void*)dk,
          16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const void*)(vt + vo),
          (__attribute__((address_space(3))) void*)(dk + C::TILEB), 16, 0, 0);
    }
  };

  // ---- per-lane LDS read offsets (bytes within a stage)
  // K operand for key block kb, step t: row kb*32 + l32, chunk 2t + hf;
  // row & 15 == l32 & 15 for both kb.
  int kread[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    kread[t] = l32 * 256 + (((2 * t + hf) ^ (l32 & 15)) * 16);
  // V^T operand for channel block mb, key step u, read half e: source lane
  // j = lane & 15 of group g = lane >> 4 names key 16u + 8e + 4(g>>1) + j/4
  // and channels 32mb + 16(g&1) + 4(j&3) .. +3.
  const int g = lane >> 4, j16 = lane & 15;
  const int vkey = 4 * (g >> 1) + (j16 >> 2);          // + 16u + 8e
  const int vd0 = 16 * (g & 1) + 4 * (j16 & 3);        // + 32mb
  const int vsw = 4 * (vkey & 3);  // (vkey + 16u + 8e) & 3 == vkey & 3
  int vread[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int d0 = 32 * mb + vd0;
    vread[mb] = vkey * 256 + (((d0 >> 3) ^ vsw) * 16) + (d0 & 7) * 2;
  }

  auto qk_tile = [&](int t, f32x16 (&s)[QB][2]) {
    const lds_u8* kt = lds + (t % NSTAGE) * C::STAGEB;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 raw = *(const __attribute__((address_space(3))) u32x4*)(
            kt + kread[st] + kb * 32 * 256);
        const bf16x8 kf = __builtin_bit_cast(bf16x8, raw);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (st == 0) {
            const f32x16 z = {};
            s[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][st],
                                                                z, 0, 0, 0);
          } else {
            s[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                kf, qf[qb][st], s[qb][kb], 0, 0, 0);
          }
        }
      }
    }
  };

  f32x16 o[QB][4];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qb][mb][r] = 0.f;

  auto pv_tile = [&](int t, const uint32_t (&pw)[QB][16]) {
    const lds_u8* vt = lds + (t % NSTAGE) * C::STAGEB + C::TILEB;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const lds_u8* a = vt + vread[mb] + (16 * u) * 256;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(a));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(a + 8 * 256));
        const v8i16 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        const bf16x8 vf = __builtin_bit_cast(bf16x8, both);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const u32x4 pr = {pw[qb][4 * u], pw[qb][4 * u + 1], pw[qb][4 * u + 2],
                            pw[qb][4 * u + 3]};
          o[qb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              vf, __builtin_bit_cast(bf16x8, pr), o[qb][mb], 0, 0, 0);
        }
      }
    }
  };

  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
  }

  // wait until at most `pending` tiles (C::LOADS*2 instructions each) of
  // this wave are still in flight, then make every wave's loads visible
  auto wait_tiles = [&](int pending) {
    constexpr int per = 2 * C::LOADS;
    if (pending >= 2)
      __builtin_amdgcn_s_waitcnt(((2 * per) & 15) | (((2 * per) >> 4) << 14) |
                                 (0x7 << 4) | (0xF << 8));
    else if (pending == 1)
      __builtin_amdgcn_s_waitcnt((per & 15) | ((per >> 4) << 14) | (0x7 << 4) |
                                 (0xF << 8));
    else
      __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
    __syncthreads();
  };

  auto softmax_tile = [&](f32x16 (&s)[QB][2], uint32_t (&pw)[QB][16],
                          float (&sum)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) sum[qb] = softmax_exp(s[qb], c, m[qb], pw[qb]);
  };
  auto softmax_finish = [&](f32x16 (&s)[QB][2], uint32_t (&pw)[QB][16],
                            float (&sum)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (wave_any(!(sum[qb] <= kTripSum)))
        softmax_fixup(s[qb], c, m[qb], l[qb], sum[qb], pw[qb], o[qb]);
      l[qb] += sum[qb];
    }
  };

  // ---- prologue: tiles 0 .. NSTAGE-2 requested, S(0), P(0)
#pragma unroll
  for (int t = 0; t < NSTAGE - 1; ++t)
    if (t < ntiles) issue_tile(t);
  {
    int pend = ntiles - 1 < NSTAGE - 2 ? ntiles - 1 : NSTAGE - 2;
    wait_tiles(pend);
  }

  f32x16 sA[QB][2], sB[QB][2];
  uint32_t pw[QB][16];
  float sum[QB];

  qk_tile(0, sA);
  if (kv_end < C::BKV) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) mask_scores(sA[qb], 0, hf, kv_end);
  }

  // Iteration jt: S(jt) is in `sc` (not yet exponentiated).
  auto iteration = [&](int jt, f32x16 (&sc)[QB][2], f32x16 (&sn)[QB][2]) {
    const bool has_next = jt + 1 < ntiles;
    // tile jt+1 must be resident; the stage that held tile jt-1 is free
    // once every wave has passed this barrier
    {
      int pend = ntiles - 1 - (jt + 1);
      if (pend > NSTAGE - 3) pend = NSTAGE - 3;
      if (pend < 0) pend = 0;
      wait_tiles(pend);
    }
    if (jt + NSTAGE - 1 < ntiles) issue_tile(jt + NSTAGE - 1);

    // phase A: S(j+1) || softmax(j)
    if (has_next) {
      qk_tile(jt + 1, sn);
      softmax_tile(sc, pw, sum);
#pragma unroll
      for (int i = 0; i < 16 * QB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        if (i % 2 == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    } else {
      softmax_tile(sc, pw, sum);
    }
    softmax_finish(sc, pw, sum);
    if (has_next && (jt + 2) * C::BKV > kv_end) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        mask_scores(sn[qb], (jt + 1) * C::BKV, hf, kv_end);
    }
    // phase B: O += V(j) P(j)
    pv_tile(jt, pw);
  };

  int jt = 0;
  for (; jt + 1 < ntiles; jt += 2) {
    iteration(jt, sA, sB);
    iteration(jt + 1, sB, sA);
  }
  if (jt < ntiles) iteration(jt, sA, sB);

  // ---- epilogue (same layout as the generic kernel)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float ltot = l[qb] + __shfl_xor(l[qb], 32, 64);
    const int row = q0 + qb * 32 + l32;
    if (row >= p.Sq) continue;
    const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
    if (p.o32 != nullptr) {
      float* dst = p.o32 + bhrow * 128;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          f32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = o[qb][mb][gq * 4 + e];
          *(f32x4*)(dst + mb * 32 + 8 * gq + 4 * hf) = w;
        }
      if (hf == 0) {
        p.m[bhrow] = m[qb];
        p.l[bhrow] = ltot;
      }
    }
    if (p.o != nullptr) {
      const float inv = 1.0f / ltot;
      uint16_t* dst = p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          u32x2 w;
          w[0] = pack_bf16x2(o[qb][mb][gq * 4 + 0] * inv,
                             o[qb][mb][gq * 4 + 1] * inv);
          w[1] = pack_bf16x2(o[qb][mb][gq * 4 + 2] * inv,
                             o[qb][mb][gq * 4 + 3] * inv);
          *(u32x2*)(dst + mb * 32 + 8 * gq + 4 * hf) = w;
        }
    }
  }
}

template <int NW, int QB, int NSTAGE>
static int launch128(const FlashParams& base, hipStream_t st) {
  using C = Cfg128<NW, QB, NSTAGE>;
  FlashParams p = base;
  p.n_qblk = (p.Sq + C::BQ - 1) / C::BQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  p.n_wg = (int)nwg;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)flash_fwd_d128_kernel<NW, QB, NSTAGE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              C::LDSB);
    attr_set = true;
  }
  hipLaunchKernelGGL((flash_fwd_d128_kernel<NW, QB, NSTAGE>), dim3(p.n_wg),
                     dim3(C::NT), C::LDSB, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

template <int D, int NW, int QB>
static int launch(const FlashParams& base, hipStream_t st) {
  using C = FlashCfg<D, NW, QB>;
  FlashParams p = base;
  p.n_qblk = (p.Sq + C::BQ - 1) / C::BQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  p.n_wg = (int)nwg;
  static bool attr_set = false;  // idempotent attribute; benign race
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)flash_fwd_kernel<D, NW, QB>,
                        hipFuncAttributeMaxDynamicSharedMemorySize,
                        C::LDS_BYTES);
    attr_set = true;
  }
  hipLaunchKernelGGL((flash_fwd_kernel<D, NW, QB>), dim3(p.n_wg),
                     dim3(C::NT), C::LDS_BYTES, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

static bool al16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace dt

extern "C" int dt_flash_fwd(const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, uint16_t* o, int B, int Hq,
                            int Hkv, int Sq, int Skv, int D,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides,
                            float scale, int kv_len, float* o32, float* m,
                            float* l, void* stream) {
  using namespace dt;
  const bool resid = (o32 != nullptr) || (m != nullptr) || (l != nullptr);
  if (!q || !k || !v || !q_strides || !k_strides || !v_strides)
    return set_error(DT_ERR_ARG, "dt_flash_fwd: null pointer argument");
  if (resid && !(o32 && m && l))
    return set_error(DT_ERR_ARG, "dt_flash_fwd: o32, m, l must all be given");
  if (!resid && !o)
    return set_error(DT_ERR_ARG, "dt_flash_fwd: null output");
  if (o && !o_strides)
    return set_error(DT_ERR_ARG, "dt_flash_fwd: null o_strides");
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Skv <= 0)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: B=%d Hq=%d Hkv=%d Sq=%d Skv=%d",
                     B, Hq, Hkv, Sq, Skv);
  if (Hq % Hkv)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: Hq %d not a multiple of Hkv %d",
                     Hq, Hkv);
  if (D != 64 && D != 128)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: head dim %d (supported: 64, 128)", D);
  if (kv_len > Skv)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: kv_len %d > Skv %d", kv_len, Skv);
  for (int i = 0; i < 3; ++i) {
    if (q_strides[i] % 8 || k_strides[i] % 8 || v_strides[i] % 8 ||
        (o && o_strides[i] % 4))
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_flash_fwd: strides must be multiples of 8 elements");
  }
  if (!al16(q) || !al16(k) || !al16(v) || (o && ((uintptr_t)o & 7u)) ||
      (o32 && !al16(o32)))
    return set_error(DT_ERR_UNSUPPORTED, "dt_flash_fwd: misaligned tensor");
  FlashParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.o32 = o32;
  p.m = m;
  p.l = l;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_ss = q_strides[2];
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  p.v_sb = v_strides[0];
  p.v_sh = v_strides[1];
  p.v_ss = v_strides[2];
  if (o) {
    p.o_sb = o_strides[0];
    p.o_sh = o_strides[1];
    p.o_ss = o_strides[2];
  } else {
    p.o_sb = p.o_sh = p.o_ss = 0;
  }
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.Sq = Sq;
  p.Skv = Skv;
  p.kv_end = (kv_len <= 0) ? Skv : kv_len;
  const float sc = (scale > 0.f) ? scale : 1.0f / sqrtf((float)D);
  p.c = sc * kLog2e;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) return launch128<8, 1, 4>(p, st);
  return launch<64, 4, 1>(p, st);
}
